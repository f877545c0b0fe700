"""GPU parity of the whole decode step (LlmModel / LlmDecoderLayer restated as the fused step
graph) against the oracle and against Hugging Face transformers logits."""
from __future__ import annotations

import numpy as np
import pytest

import l0llm_amd as l0
from oracle import pyoracle as orc
from tests.helpers import PROJECTIONS, load_hf, rel_err, rope_table_for

pytestmark = pytest.mark.gpu

STORAGE = {l0.PRECISION_FLOAT32: l0.F32, l0.PRECISION_FLOAT16: l0.F16, l0.PRECISION_BFLOAT16: l0.BF16,
           l0.PRECISION_INT8: l0.I8PC}


def hf_config(cfg: dict) -> l0.HfConfig:
    rp = cfg["rope"]
    scaling = None
    if rp.get("rope_type", "default") != "default":
        scaling = l0.RopeScaling(type=rp["rope_type"], factor=rp.get("factor", 1.0),
                                 original_max_position_embeddings=rp.get("original_max_position_embeddings"),
                                 low_freq_factor=rp.get("low_freq_factor", 1.0),
                                 high_freq_factor=rp.get("high_freq_factor", 4.0))
    return l0.HfConfig(hidden_size=cfg["hidden_size"], intermediate_size=cfg["intermediate_size"],
                       num_layers=cfg["num_layers"], num_attention_heads=cfg["num_attention_heads"],
                       num_key_value_heads=cfg["num_key_value_heads"], head_dim=cfg["head_dim"],
                       vocab_size=cfg["vocab_size"], max_position_embeddings=cfg["max_position_embeddings"],
                       rms_norm_eps=cfg["rms_norm_eps"], rope_theta=cfg["rope_theta"],
                       attention_bias=cfg["attention_bias"], tie_word_embeddings=cfg["tie_word_embeddings"],
                       rope_scaling=scaling)


def load_model(device, d, precision, cache, max_seq=64):
    m = l0.LlmModel(device, hf_config(d["cfg"]), precision=precision, cache_dtype=cache, max_seq_len=max_seq)
    for name, w in d["weights"].items():
        m.set_tensor(name, w)
    return m


def exported_weights(m: l0.LlmModel, cfg: dict) -> dict:
    """The weights exactly as the device stores them (read back through the ABI), HuggingFace names:
    projections as (storage, stored array, fp16 scales or None), vectors as fp32."""
    H, L = cfg["hidden_size"], cfg["num_layers"]
    w = {"model.embed_tokens.weight": m.export_vector("model.embed_tokens.weight", cfg["vocab_size"] * H),
         "model.norm.weight": m.export_vector("model.norm.weight", H)}
    st, lm, s = m.export_matrix("lm_head.weight")
    w["lm_head.weight"] = (st, lm, s)
    for i in range(L):
        p = f"model.layers.{i}."
        for n in PROJECTIONS:
            w[p + n] = m.export_matrix(p + n)
        w[p + "input_layernorm.weight"] = m.export_vector(p + "input_layernorm.weight", H)
        w[p + "post_attention_layernorm.weight"] = m.export_vector(p + "post_attention_layernorm.weight", H)
        if cfg.get("attention_bias"):
            for n, width in (("q", cfg["num_attention_heads"]), ("k", cfg["num_key_value_heads"]),
                             ("v", cfg["num_key_value_heads"])):
                w[p + f"self_attn.{n}_proj.bias"] = m.export_vector(p + f"self_attn.{n}_proj.bias", width * cfg["head_dim"])
    return w


def exported_oracle(m: l0.LlmModel, cfg: dict, cache: int, max_seq: int, copies: int = 1):
    """Oracle over the weights exactly as the device stores them; with copies > 1, that many
    oracles (own caches) sharing one host copy of the weights."""
    w = exported_weights(m, cfg)
    inv, att = rope_table_for(cfg)
    if copies > 1:
        return [orc.Model(cfg, w, inv, att, cache, max_seq) for _ in range(copies)]
    return orc.Model(cfg, w, inv, att, cache, max_seq)


@pytest.mark.parametrize("name", ["llama", "qwen2"])
def test_fp32_model_matches_transformers(device, name):
    """fp32 weights, fp32 cache: logits at every prompt position and the greedy continuation."""
    d = load_hf(name)
    with load_model(device, d, l0.PRECISION_FLOAT32, l0.F32) as m:
        for t, tok in enumerate(d["prompt"]):
            lg = m.compute_logits(tok, t)
            assert rel_err(lg, d["prompt_logits"][t]) < 1e-4, t
        out = m.generate_greedy(d["prompt"], len(d["generated"]))
        assert out == d["generated"]


@pytest.mark.parametrize("precision", [l0.PRECISION_INT8, l0.PRECISION_FLOAT16, l0.PRECISION_BFLOAT16])
@pytest.mark.parametrize("name", ["llama", "qwen2"])
def test_quantized_model_matches_oracle(device, name, precision):
    """Stored weights equal the oracle's conversion; logits match the oracle step by step."""
    d = load_hf(name)
    cfg = d["cfg"]
    with load_model(device, d, precision, l0.F16) as m:
        from tests.helpers import stored
        st, w, s = m.export_matrix("model.layers.1.self_attn.q_proj.weight")
        ost, ow, os_ = stored(STORAGE[precision], d["weights"]["model.layers.1.self_attn.q_proj.weight"])
        assert st == ost
        np.testing.assert_array_equal(w.view(np.uint8), np.ascontiguousarray(ow).view(np.uint8))
        if s is not None:
            np.testing.assert_array_equal(s, os_)
        om = exported_oracle(m, cfg, orc.F16, 64)
        seq = list(d["prompt"])
        for t in range(len(seq) + 6):
            tok = seq[t]
            lg = m.compute_logits(tok, t)
            onext, olg = om.step(tok, t)
            assert rel_err(lg, olg) < 2e-3, t
            if t >= len(d["prompt"]) - 1:
                nxt = int(np.argmax(lg))
                if nxt != onext:
                    assert orc.top2_margin(olg) < 1e-3, (t, nxt, onext)
                seq.append(onext)


def test_prefill_matches_sequential_decode(device):  # Qwen25PrefillTests.cs:41-75
    d = load_hf("qwen2")
    with load_model(device, d, l0.PRECISION_INT8, l0.F16) as m:
        prompt = d["prompt"][:7]
        seq = None
        for i, t in enumerate(prompt):
            seq = m.compute_logits(t, i)
        nxt = int(np.argmax(seq))
        seq_after = m.compute_logits(nxt, len(prompt))
        batched = m.prefill(prompt)
        assert m.position == len(prompt)
        after = m.decode(nxt)
        assert m.position == len(prompt) + 1
        assert int(np.argmax(batched)) == nxt
        assert np.max(np.abs(seq - batched)) < 2e-3
        assert np.max(np.abs(seq_after - after)) < 2e-3


# Chunked prefill against token-by-token decode on a random-init model whose head size takes the
# query-tiled prefill attention: 300 prompt tokens = a full 256-token chunk + a ragged one + the
# last token through the decode step. fp32 weights run multi-row GEMVs on fp32 activations (the
# decode arithmetic); int8 / fp16 / bf16 run the MFMA GEMM on activations rounded to fp16 / fp16 /
# bf16, hence their looser bounds (relative to max |logit|; measured on MI355X: int8 9.4e-4, fp16
# 6.6e-4, bf16 2.9e-3, so the bounds hold about 3x margin). The cache keys are bounded by key_tol
# relative to max(1, max |key|).
CHUNKED = [(l0.PRECISION_INT8, 3e-3, 4e-2), (l0.PRECISION_FLOAT32, 2e-3, 8e-3), (l0.PRECISION_FLOAT16, 3e-3, 4e-2),
           (l0.PRECISION_BFLOAT16, 1.5e-2, 2e-1)]


@pytest.mark.parametrize("precision,tol,key_tol", CHUNKED)
def test_chunked_prefill_matches_sequential_decode(device, precision, tol, key_tol, monkeypatch):
    monkeypatch.setenv("L0H_PREFILL_CHUNK", "256")  # read at model creation: 299 rows -> chunks of 256 and 43
    cfg = l0.HfConfig(hidden_size=256, intermediate_size=512, num_layers=3, num_attention_heads=4,
                      num_key_value_heads=2, head_dim=64, vocab_size=512, max_position_embeddings=4096,
                      rms_norm_eps=1e-5, rope_theta=500000.0, attention_bias=True)
    prompt = np.random.default_rng(11).integers(0, cfg.vocab_size, 300).tolist()
    with l0.LlmModel(device, cfg, precision=precision, cache_dtype=l0.F16, max_seq_len=320) as m:
        m.init_random(1234, 0.05)
        seq = None
        for i, t in enumerate(prompt):
            seq = m.compute_logits(t, i)
        kv_elems = len(prompt) * 2 * 64

        def keys(li):
            return l0.Buffer(device, kv_elems * 2, ptr=m.kv_cache(li)[0], owned=False).read(np.float16, kv_elems)

        k_seq = [keys(li) for li in range(3)]
        batched = m.prefill(prompt)
        assert m.position == len(prompt)
        scale = np.max(np.abs(seq))
        assert np.max(np.abs(seq - batched)) <= tol * scale, np.max(np.abs(seq - batched)) / scale
        if int(np.argmax(batched)) != int(np.argmax(seq)):
            assert orc.top2_margin(seq) < tol * scale
        for li in range(3):  # keys of every prompt position (the last one written by the decode step)
            a = k_seq[li].astype(np.float32)
            b = keys(li).astype(np.float32)
            assert np.max(np.abs(a - b)) <= key_tol * max(1.0, np.max(np.abs(a))), li


@pytest.mark.parametrize("precision,tol", [(l0.PRECISION_INT8, 1e-2), (l0.PRECISION_FLOAT16, 1e-2)])
def test_wide_prefill_split_k_epilogues_match_decode(device, precision, tol):
    """Hidden 4096 over 139 prefill rows: the q|k|v, O and gate|up GEMMs split K in two, so the
    split-K sums carry the store, residual and SwiGLU epilogues; down (K = 1024) does not split."""
    cfg = l0.HfConfig(hidden_size=4096, intermediate_size=1024, num_layers=2, num_attention_heads=32,
                      num_key_value_heads=8, head_dim=128, vocab_size=512, max_position_embeddings=4096,
                      rms_norm_eps=1e-5, rope_theta=500000.0)
    prompt = np.random.default_rng(12).integers(0, cfg.vocab_size, 140).tolist()
    with l0.LlmModel(device, cfg, precision=precision, cache_dtype=l0.F16, max_seq_len=160) as m:
        m.init_random(99, 0.02)
        seq = None
        for i, t in enumerate(prompt):
            seq = m.compute_logits(t, i)
        batched = m.prefill(prompt)
        scale = np.max(np.abs(seq))
        assert np.max(np.abs(seq - batched)) <= tol * scale, np.max(np.abs(seq - batched)) / scale


@pytest.mark.parametrize("tokens", [600, 2048])
@pytest.mark.parametrize("precision,tol", [(l0.PRECISION_INT8, 3e-3), (l0.PRECISION_BFLOAT16, 1.5e-2)])
def test_tall_prefill_eight_wave_tiles_match_decode(device, precision, tol, tokens):
    """599 prefill rows at hidden 4096, intermediate 8192: the int8 GEMMs take the eight-wave
    128-row tiles (gate|up one-step stages; down, K = 8192, two-step stages with K split in four).
    2047 rows: q|k|v (N = 6144) and gate|up (N = 16384, SwiGLU epilogue) take the 256 x 256 blocks
    with a ragged last row block, O and down the 128-row tiles. For bf16 weights all four GEMMs
    take the two-operand LDS-ring tiles: at 599 rows O and down with K split in two (the split-K
    sum carries the residual), at 2047 rows without a split, so the kernel's own LDS-staged
    epilogue stores q|k|v, adds O and down to the residual and applies SwiGLU to gate|up. Measured
    deviations on MI355X: int8 7.6e-4 / 7.0e-4, bf16 4.3e-3 / 4.9e-3 of max |logit| (600 / 2048
    tokens)."""
    cfg = l0.HfConfig(hidden_size=4096, intermediate_size=8192, num_layers=1, num_attention_heads=32,
                      num_key_value_heads=8, head_dim=128, vocab_size=256, max_position_embeddings=4096,
                      rms_norm_eps=1e-5, rope_theta=500000.0)
    prompt = np.random.default_rng(13).integers(0, cfg.vocab_size, tokens).tolist()
    with l0.LlmModel(device, cfg, precision=precision, cache_dtype=l0.F16, max_seq_len=tokens + 40) as m:
        m.init_random(77, 0.02)
        seq = None
        for i, t in enumerate(prompt):
            seq = m.compute_logits(t, i)
        batched = m.prefill(prompt)
        scale = np.max(np.abs(seq))
        assert np.max(np.abs(seq - batched)) <= tol * scale, np.max(np.abs(seq - batched)) / scale


def test_wide_hidden_prefill_residual_256_tiles_match_decode(device):
    """Hidden 8192 at 2047 prefill rows: O (8192 x 8192) and down (8192 x 2048) take the 256 x 256
    GEMM blocks with the residual epilogue (q|k|v and gate|up the 128-row tiles)."""
    cfg = l0.HfConfig(hidden_size=8192, intermediate_size=2048, num_layers=1, num_attention_heads=64,
                      num_key_value_heads=8, head_dim=128, vocab_size=256, max_position_embeddings=4096,
                      rms_norm_eps=1e-5, rope_theta=500000.0)
    prompt = np.random.default_rng(17).integers(0, cfg.vocab_size, 2048).tolist()
    with l0.LlmModel(device, cfg, precision=l0.PRECISION_INT8, cache_dtype=l0.F16, max_seq_len=2088) as m:
        m.init_random(91, 0.02)
        seq = None
        for i, t in enumerate(prompt):
            seq = m.compute_logits(t, i)
        batched = m.prefill(prompt)
        scale = np.max(np.abs(seq))
        assert np.max(np.abs(seq - batched)) <= 1e-2 * scale, np.max(np.abs(seq - batched)) / scale


@pytest.mark.parametrize("name,precision", [("qwen2", l0.PRECISION_INT8), ("llama", l0.PRECISION_BFLOAT16)])
def test_model_loads_from_safetensors(device, tmp_path, name, precision):
    """LlmModel.Load's weight pass from a sharded safetensors checkpoint (bf16 tensors, as HF
    checkpoints ship) stores exactly what set_tensor stores from the same values."""
    import json
    import torch
    from safetensors.torch import save_file
    d = load_hf(name)
    ws = {k: torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)).to(torch.bfloat16) for k, v in d["weights"].items()}
    if d["cfg"]["tie_word_embeddings"]:
        ws.pop("lm_head.weight", None)
    names = sorted(ws)
    half = len(names) // 2
    shards = {"model-00001-of-00002.safetensors": names[:half], "model-00002-of-00002.safetensors": names[half:]}
    for f, ns in shards.items():
        save_file({n: ws[n] for n in ns}, str(tmp_path / f))
    wm = {n: f for f, ns in shards.items() for n in ns}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    with load_model(device, {"cfg": d["cfg"], "weights": {}}, precision, l0.F16) as a, \
            load_model(device, {"cfg": d["cfg"], "weights": {}}, precision, l0.F16) as b:
        assert a.load_safetensors(tmp_path) == len(names)
        for n in names:
            b.set_tensor(n, ws[n].float().numpy(), sixteen_bit_source=True)
        for n in names:
            if n.endswith("proj.weight") or n == "lm_head.weight":
                sa, wa, sca = a.export_matrix(n)
                sb, wb, scb = b.export_matrix(n)
                assert sa == sb
                np.testing.assert_array_equal(wa.view(np.uint8), wb.view(np.uint8))
                if sca is not None:
                    np.testing.assert_array_equal(sca, scb)
        for t, tok in enumerate(d["prompt"][:5]):
            np.testing.assert_array_equal(a.compute_logits(tok, t), b.compute_logits(tok, t))


def test_model_load_rejects_missing_or_misshapen_tensors(device, tmp_path):
    from safetensors.numpy import save_file
    d = load_hf("llama")
    ws = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in d["weights"].items()}
    save_file({k: v for k, v in ws.items() if k != "model.norm.weight"}, str(tmp_path / "missing.safetensors"))
    bad = dict(ws)
    bad["model.layers.0.mlp.down_proj.weight"] = np.ascontiguousarray(bad["model.layers.0.mlp.down_proj.weight"].T)
    save_file(bad, str(tmp_path / "transposed.safetensors"))
    with load_model(device, {"cfg": d["cfg"], "weights": {}}, l0.PRECISION_INT8, l0.F16) as m:
        with pytest.raises(l0.InvalidDataError):
            m.load_safetensors(tmp_path / "missing.safetensors")
        with pytest.raises(l0.InvalidDataError):
            m.load_safetensors(tmp_path / "transposed.safetensors")


@pytest.mark.parametrize("name", ["llama", "qwen2"])
def test_probe_stages_match_oracle(device, name):
    """LlmDecoderLayer.Probe (LlmDecoderLayer.cs:113-119, :168-195, :315-317): every stage of every
    layer of one eager step, checked against the oracle's operators on the weights the device holds.
    At position 0 the attention over the one cached row returns that row's V, so attn_out is the
    output projection of the fp16-cached V of each q head's kv head. The step's own logits are the
    graph step's, bit for bit."""
    d = load_hf(name)
    cfg = d["cfg"]
    H, eps = cfg["hidden_size"], cfg["rms_norm_eps"]
    nh, nkv, hd = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    with load_model(device, d, l0.PRECISION_INT8, l0.F16) as m:
        tok = int(d["prompt"][0])
        logits, st = m.probe_step(tok, 0)
        np.testing.assert_array_equal(logits, m.compute_logits(tok, 0))
        assert len(st) == 8 * cfg["num_layers"]

        def proj(name_, x):
            wst, w, sc = m.export_matrix(name_)
            return orc.gemv_nk(wst, w, np.asarray(x, np.float32), sc)

        x = m.export_vector("model.embed_tokens.weight", cfg["vocab_size"] * H).reshape(-1, H)[tok]
        for li in range(cfg["num_layers"]):
            p = f"model.layers.{li}."
            _, want = orc.rmsnorm(x, m.export_vector(p + "input_layernorm.weight", H), eps)
            assert rel_err(st[(li, "input_norm")], want) < 1e-5, li
            for n, width in (("q", nh * hd), ("k", nkv * hd), ("v", nkv * hd)):
                want = proj(p + f"self_attn.{n}_proj.weight", st[(li, "input_norm")])
                if cfg.get("attention_bias"):
                    want = want + m.export_vector(p + f"self_attn.{n}_proj.bias", width)
                assert rel_err(st[(li, n)], want) < 1e-4, (li, n)
            v16 = st[(li, "v")].astype(np.float16).astype(np.float32).reshape(nkv, hd)
            attn = np.concatenate([v16[h // (nh // nkv)] for h in range(nh)])
            want = proj(p + "self_attn.o_proj.weight", attn.astype(np.float16).astype(np.float32))
            assert rel_err(st[(li, "attn_out")], want) < 1e-4, li
            resid = x + st[(li, "attn_out")]
            _, want = orc.rmsnorm(resid, m.export_vector(p + "post_attention_layernorm.weight", H), eps)
            assert rel_err(st[(li, "post_norm")], want) < 1e-4, li
            act = orc.swiglu(proj(p + "mlp.gate_proj.weight", st[(li, "post_norm")]),
                             proj(p + "mlp.up_proj.weight", st[(li, "post_norm")]))
            want = proj(p + "mlp.down_proj.weight", act)
            assert rel_err(st[(li, "mlp_out")], want) < 3e-3, li  # down reads the SwiGLU row in fp16
            np.testing.assert_allclose(st[(li, "output")], resid + st[(li, "mlp_out")], rtol=1e-5,
                                       atol=1e-5 * np.abs(st[(li, "output")]).max())
            x = st[(li, "output")]


def test_generate_greedy_matches_step_loop_and_stops(device):
    d = load_hf("llama")
    with load_model(device, d, l0.PRECISION_INT8, l0.F16) as m:
        gen = m.generate_greedy(d["prompt"], 10)
        assert len(gen) == 10
        logits = m.prefill(d["prompt"])
        loop = [int(np.argmax(logits))]
        while len(loop) < 10:
            loop.append(int(np.argmax(m.decode(loop[-1]))))
        assert gen == loop
        m.prefill(d["prompt"])
        dev_loop = m.decode_greedy_device(loop[0], 9)
        assert [loop[0]] + dev_loop.tolist() == loop
        stop = gen[3]
        cut = m.generate_greedy(d["prompt"], 10, stop_token_ids=[stop])
        assert cut == gen[: gen.index(stop) + 1]
        with pytest.raises(l0.InvalidArgumentError):
            m.generate_greedy(d["prompt"], 100)
        with pytest.raises(l0.InvalidArgumentError):
            m.compute_logits(d["cfg"]["vocab_size"], 0)


def _random_model(device, hf: l0.HfConfig, max_seq: int, seed: int) -> l0.LlmModel:
    m = l0.LlmModel(device, hf, precision=l0.PRECISION_INT8, cache_dtype=l0.F16, max_seq_len=max_seq)
    m.init_random(seed, 0.02)
    return m


def _as_cfg(hf: l0.HfConfig) -> dict:
    return dict(vocab_size=hf.vocab_size, hidden_size=hf.hidden_size, intermediate_size=hf.intermediate_size,
                num_layers=hf.num_layers, num_attention_heads=hf.num_attention_heads,
                num_key_value_heads=hf.num_key_value_heads, head_dim=hf.head_dim,
                max_position_embeddings=hf.max_position_embeddings, rms_norm_eps=hf.rms_norm_eps,
                rope_theta=hf.rope_theta, tie_word_embeddings=hf.tie_word_embeddings,
                attention_bias=hf.attention_bias, rope={"rope_type": "default", "rope_theta": hf.rope_theta})


QWEN05 = l0.HfConfig(hidden_size=896, intermediate_size=4864, num_layers=4, num_attention_heads=14,
                     num_key_value_heads=2, head_dim=64, vocab_size=151936, max_position_embeddings=32768,
                     rms_norm_eps=1e-6, rope_theta=1e6, attention_bias=True, tie_word_embeddings=True)
LLAMA8B = l0.HfConfig(hidden_size=4096, intermediate_size=14336, num_layers=32, num_attention_heads=32,
                      num_key_value_heads=8, head_dim=128, vocab_size=128256, max_position_embeddings=131072,
                      rms_norm_eps=1e-5, rope_theta=500000.0)


# Odd shapes: hidden 320 (20 int8 chunks per row), 5 q heads on 1 kv head, an odd vocabulary (a
# partial last row group), biases.
ODD = l0.HfConfig(hidden_size=320, intermediate_size=960, num_layers=2, num_attention_heads=5,
                  num_key_value_heads=1, head_dim=64, vocab_size=777, max_position_embeddings=4096,
                  rms_norm_eps=1e-6, rope_theta=10000.0, attention_bias=True)


@pytest.mark.parametrize("hf,steps", [(QWEN05, 6), (LLAMA8B, 4), (ODD, 8)],
                         ids=["qwen2.5-0.5b-4layers", "llama3.1-8b", "odd-320-5q1kv-777"])
def test_random_int8_model_matches_oracle(device, hf, steps):
    """Int8 per-channel random-init model at the real shapes: the device's weights are read
    back and the oracle runs the same steps; logits agree and greedy ids agree unless the
    oracle's own top-2 gap is below the accumulation noise."""
    max_seq = 16
    with _random_model(device, hf, max_seq, seed=599) as m:
        cfg = _as_cfg(hf)
        om = exported_oracle(m, cfg, orc.F16, max_seq)
        rng = np.random.default_rng(599)
        tok = int(rng.integers(0, hf.vocab_size))
        for t in range(steps):
            lg = m.compute_logits(tok, t)
            onext, olg = om.step(tok, t)
            assert rel_err(lg, olg) < 2e-3, t
            gnext = int(np.argmax(lg))
            if gnext != onext:
                assert orc.top2_margin(olg) < 1e-3 * np.max(np.abs(olg)), (t, gnext, onext)
            tok = onext


# hidden 256 (16 int8 chunks a row: 8-row groups), vocabulary 5003: the lm_head GEMV spreads the
# rows over ~600 waves, each keeping the greedy key of its own rows.
TIES = l0.HfConfig(hidden_size=256, intermediate_size=512, num_layers=1, num_attention_heads=4,
                   num_key_value_heads=2, head_dim=64, vocab_size=5003, max_position_embeddings=4096,
                   rms_norm_eps=1e-6, rope_theta=10000.0)


@pytest.mark.parametrize("negated", [0, 1700])
def test_greedy_ties_take_the_first_index(device, negated):
    """Exact ties across the waves of the lm_head GEMV: every lm_head row is the same vector (the
    first `negated` rows its negation), so thousands of logits are bit-for-bit equal. The device's
    greedy pick (per-wave keys reduced by one block) is the first index of the largest logit, as
    the reference's argmax (LlmAbstractions.cs:83-90) and numpy's."""
    rng = np.random.default_rng(7)
    row = rng.normal(0, 0.05, TIES.hidden_size).astype(np.float32)
    w = np.tile(row, (TIES.vocab_size, 1))
    w[:negated] = -row
    prompt = [5, 17, 300]
    with _random_model(device, TIES, 32, seed=3) as m:
        m.set_tensor("lm_head.weight", w)
        logits = m.prefill(prompt)
        first = int(np.argmax(logits))
        assert np.count_nonzero(logits == logits[first]) > 1000  # a tie over many waves
        assert first in (0, negated)
        assert m.generate_greedy(prompt, 1) == [first]
        m.prefill(prompt)
        dev = m.decode_greedy_device(first, 4).tolist()
        m.prefill(prompt)
        loop, tok = [], first
        for _ in range(4):
            tok = int(np.argmax(m.decode(tok)))
            loop.append(tok)
        assert dev == loop


def test_odd_shapes_chunked_prefill_matches_decode(device, monkeypatch):
    """The odd-shaped model in 64-token chunks (the MFMA GEMM at its smallest M, with the K = 320
    and 960 rows and the 448-row q|k|v, then a 21-token chunk on the multi-row GEMV)."""
    monkeypatch.setenv("L0H_PREFILL_CHUNK", "64")
    prompt = np.random.default_rng(21).integers(0, ODD.vocab_size, 150).tolist()
    with _random_model(device, ODD, 160, seed=5) as m:
        seq = None
        for i, t in enumerate(prompt):
            seq = m.compute_logits(t, i)
        batched = m.prefill(prompt)
        scale = np.max(np.abs(seq))
        assert np.max(np.abs(seq - batched)) <= 1e-2 * scale, np.max(np.abs(seq - batched)) / scale
