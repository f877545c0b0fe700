"""Pins the CPU oracle before anything is checked against it.

Each oracle function is checked against something independent of its own formula: the
reference's golden vectors and known answers (rope.golden.json, RopeLlama3Tests.cs:9-17,
LlmMatrixTests.cs:40-46 / :112-129, LlmLayerWeightsTests.cs:19-52, the Qwen2.5 layer golden),
library routines (numpy matmul and float16 casts, torch SDPA and silu, the transformers
rotary helper), closed forms, and the Hugging Face transformers decoders (the models the
reference's goldens come from) built from a config with seeded weights.

    oracle function          pinned by
    f16/bf16 conversions     numpy / torch casts over random, subnormal, tie and overflow values
    fits_in_half             LlmMatrixTests.cs:40-46 known answers
    transpose                LlmLayerWeightsTests.cs:19-52 cases
    quantize_i8pc            closed-form bounds (|q*s - w| <= s/2, max |q| = 127, zero rows)
    gemv_nk / gemv_kn        LlmMatrixTests.cs:112-129 known answer; numpy float64 matmul
    rmsnorm (+ residual)     closed form; Qwen2.5 layer golden (input->input_norm,
                             input+attn_out->post_norm across tokens)
    swiglu / add / bias_add  torch silu; numpy
    rope_frequencies         rope.golden.json (5 cases), llama3 table, linear/yarn identities
    rope_table / rope_theta  transformers apply_rotary_pos_emb; position-0 identity
    kv_store                 placement known answer
    attention decode/prefill torch SDPA in float64 (GQA expanded, causal mask); 1-slot closed form
    embedding / argmax       known answers; numpy.argmax first-maximum rule
    model step               transformers Llama (llama3 RoPE) and Qwen2 (bias, tied) logits and
                             greedy continuations
    device rounding          the step composed from the primitives above with numpy fp16 casts of
                             the attention and SwiGLU outputs (bit for bit)
"""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from oracle import pyoracle as orc
from tests.helpers import GOLDEN, bf16_bits, load_hf, oracle_model, rel_err, rope_table_for


# ---- conversions ------------------------------------------------------------------------------

def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.normal(0, 1, 2000), rng.normal(0, 1e-5, 500), rng.normal(0, 3e4, 500),
        [0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e6, -1e6, 2.0**-24, 2.0**-25, 3 * 2.0**-26, 2.0**-14,
         1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, np.inf, -np.inf],
    ]).astype(np.float32)
    got = np.array([orc.f32_to_f16_bits(float(v)) for v in vals], dtype=np.uint16)
    np.testing.assert_array_equal(got, vals.astype(np.float16).view(np.uint16))
    back = np.array([orc.f16_bits_to_f32(int(b)) for b in got], dtype=np.float32)
    np.testing.assert_array_equal(back, got.view(np.float16).astype(np.float32))


def test_bf16_conversion_matches_torch():
    rng = np.random.default_rng(2)
    vals = np.concatenate([rng.normal(0, 1, 2000), [1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8, -7.5e-39]]).astype(np.float32)
    got = np.array([orc.f32_to_bf16_bits(float(v)) for v in vals], dtype=np.uint16)
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(bf16_bits(vals), want)


# ---- weight handling --------------------------------------------------------------------------

def test_fits_in_half_known_answers():  # LlmMatrixTests.cs:40-46
    assert orc.fits_in_half([0.0, -1.0, 64000.0, 1e-9])
    assert not orc.fits_in_half([1.0, 70000.0])
    assert not orc.fits_in_half([1.0, float("nan")])
    assert not orc.fits_in_half([float("-inf")])


@pytest.mark.parametrize("rows,cols", [(1, 1), (2, 3), (33, 65), (64, 64), (70, 5)])
def test_transpose_moves_row_col_to_col_row(rows, cols):  # LlmLayerWeightsTests.cs:19-37
    src = np.arange(rows * cols, dtype=np.float32)
    out = orc.transpose(src, rows, cols)
    np.testing.assert_array_equal(out.reshape(cols, rows), src.reshape(rows, cols).T)


def test_transpose_twice_restores():  # LlmLayerWeightsTests.cs:40-48
    src = np.random.default_rng(3).random(37 * 91).astype(np.float32)
    np.testing.assert_array_equal(orc.transpose(orc.transpose(src, 37, 91), 91, 37), src)


def test_quantize_bounds_and_zero_rows():
    rng = np.random.default_rng(4)
    w = rng.normal(0, 0.02, (64, 96)).astype(np.float32)
    w[5] = 0.0
    q, s = orc.quantize_i8pc(w)
    sf = s.view(np.float16).astype(np.float32)
    assert sf[5] == 0 and np.all(q[5] == 0)
    live = np.arange(64) != 5
    assert np.all(np.abs(q) <= 127)
    assert np.all(np.abs(q[live]).max(axis=1) >= 126)
    err = np.abs(q[live].astype(np.float64) * sf[live, None] - w[live])
    assert np.all(err <= sf[live, None] * 0.5 * (1 + 1e-6) + 1e-12)
    # scale is half(max|w| / 127)
    np.testing.assert_array_equal(s[live], (np.abs(w[live]).max(axis=1) / np.float32(127)).astype(np.float16).view(np.uint16))


# ---- projections ------------------------------------------------------------------------------

HF = np.array([[1, 2], [3, 4], [5, 6], [7, 8]], dtype=np.float32)  # [out=4, in=2]


@pytest.mark.parametrize("storage", [orc.F32, orc.F16, orc.BF16])
def test_gemv_known_answer(storage):  # LlmMatrixTests.cs:112-129: y = [21, 43, 65, 87]
    from tests.helpers import stored
    dt, w, _ = stored(storage, HF)
    y = orc.gemv_nk(dt, w, np.array([1, 10], dtype=np.float32))
    np.testing.assert_array_equal(y[0], [21, 43, 65, 87])
    kn = HF.T.copy() if storage == orc.F32 else HF.T.astype(np.float16).view(np.uint16).copy()
    if storage != orc.BF16:
        np.testing.assert_array_equal(orc.gemv_kn(storage, kn, np.array([1, 10], np.float32))[0], [21, 43, 65, 87])


def test_gemv_int8_known_answer():
    q = HF.astype(np.int8)
    s = np.full(4, 0.5, dtype=np.float16)
    y = orc.gemv_nk(orc.I8PC, q, np.array([1, 10], dtype=np.float32), s)
    np.testing.assert_array_equal(y[0], [10.5, 21.5, 32.5, 43.5])


@pytest.mark.parametrize("storage", [orc.F32, orc.F16, orc.BF16, orc.I8PC])
@pytest.mark.parametrize("rows", [1, 3])
def test_gemv_matches_numpy(storage, rows):
    from tests.helpers import dequant, stored
    rng = np.random.default_rng(5 + rows)
    w = rng.normal(0, 0.1, (48, 80)).astype(np.float32)
    x = rng.normal(0, 1, (rows, 80)).astype(np.float32)
    dt, ws, s = stored(storage, w)
    y = orc.gemv_nk(dt, ws, x, s)
    want = x.astype(np.float64) @ dequant(dt, ws, s).T
    np.testing.assert_allclose(y, want, rtol=1e-6, atol=1e-6)


def test_gemv_kn_matches_numpy():
    rng = np.random.default_rng(6)
    w = rng.normal(0, 0.1, (30, 17)).astype(np.float32)  # [K, N]
    x = rng.normal(0, 1, (2, 30)).astype(np.float32)
    np.testing.assert_allclose(orc.gemv_kn(orc.F32, w, x), x.astype(np.float64) @ w, rtol=1e-6, atol=1e-6)


def test_int8_projection_within_reference_quantization_bar():
    # LlmMatrixInt8Tests.cs:80-119: relative RMSE < 0.02 against the fp64 product of the float weights.
    rng = np.random.default_rng(7)
    hf = rng.uniform(-0.2, 0.2, (96, 160)).astype(np.float32)
    x = rng.uniform(-1.5, 1.5, (5, 160)).astype(np.float32)
    q, s = orc.quantize_i8pc(hf)
    y = orc.gemv_nk(orc.I8PC, q, x, s)
    truth = x.astype(np.float64) @ hf.T.astype(np.float64)
    assert np.sqrt(np.sum((y - truth) ** 2) / np.sum(truth**2)) < 0.02


# ---- element-wise -----------------------------------------------------------------------------

def test_rmsnorm_closed_form():
    _, out = orc.rmsnorm([3.0, 4.0], [1.0, 2.0], 0.0)
    np.testing.assert_allclose(out, [3 / np.sqrt(12.5), 8 / np.sqrt(12.5)], rtol=1e-6)
    _, out = orc.rmsnorm([3.0, 4.0], [1.0, 1.0], 1.0)
    np.testing.assert_allclose(out, [3 / np.sqrt(13.5), 4 / np.sqrt(13.5)], rtol=1e-6)
    x, out = orc.rmsnorm([1.0, 2.0], [1.0, 1.0], 0.0, residual=[2.0, 2.0])
    np.testing.assert_array_equal(x, [3.0, 4.0])
    np.testing.assert_allclose(out, [3 / np.sqrt(12.5), 4 / np.sqrt(12.5)], rtol=1e-6)


def _recover_weight(x, y, eps):
    rms = np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps)
    return (y * rms / x).astype(np.float32)


@pytest.mark.parametrize("layer", ["0", "11"])
def test_rmsnorm_reproduces_qwen25_layer_golden(layer):
    # Qwen2.5-0.5B-Instruct layer golden (HF fp32): the norm weight is recovered from token 0,
    # then every other token's input_norm / post_norm must follow (|x| reaches 1.6e3 in layer 11).
    z = np.load(GOLDEN / "qwen25_layers_slice.npz")
    eps = float(z["eps"])
    x, inorm = z[f"l{layer}/input"], z[f"l{layer}/input_norm"]
    attn, pnorm = z[f"l{layer}/attn_out"], z[f"l{layer}/post_norm"]
    np.testing.assert_allclose(z[f"l{layer}/output"], x + attn + z[f"l{layer}/mlp_out"], atol=1e-4 * max(1, np.abs(x).max() / 100))
    for src, dst, resid in ((x, inorm, None), (x, pnorm, attn)):
        base = src[0] + (resid[0] if resid is not None else 0)
        w = _recover_weight(base, dst[0], eps)
        ok = np.abs(base) > 1e-3 * np.abs(base).max()
        for t in range(1, src.shape[0]):
            xs, out = orc.rmsnorm(src[t], np.where(ok, w, 0), eps, residual=None if resid is None else resid[t])
            if resid is not None:
                np.testing.assert_allclose(xs, src[t] + resid[t], rtol=1e-6)
            np.testing.assert_allclose(out[ok], dst[t][ok], rtol=2e-4, atol=2e-5 * np.abs(dst[t]).max())


def test_swiglu_add_bias_match_library():
    rng = np.random.default_rng(8)
    g, u = rng.normal(0, 3, 100).astype(np.float32), rng.normal(0, 1, 100).astype(np.float32)
    want = torch.nn.functional.silu(torch.from_numpy(g).double()) * torch.from_numpy(u).double()
    np.testing.assert_allclose(orc.swiglu(g, u), want.numpy(), rtol=1e-6, atol=1e-7)
    np.testing.assert_array_equal(orc.add(g, u), g + u)
    x = rng.normal(0, 1, (3, 10)).astype(np.float32)
    b = rng.normal(0, 1, 10).astype(np.float32)
    np.testing.assert_array_equal(orc.bias_add(x, b, 10, 3), x + b)


# ---- RoPE -------------------------------------------------------------------------------------

def _golden_rope():
    return json.loads((GOLDEN / "rope.golden.json").read_text())["cases"]


@pytest.mark.parametrize("name", ["default", "linear4", "yarn4_qwen3", "yarn8_small", "yarn2_explicit"])
def test_rope_tables_match_transformers_golden(name):  # RopeFrequenciesTests.cs:19-46
    c = _golden_rope()[name]
    s = c["scaling"] or {}
    inv, att = orc.rope_frequencies(
        c["head_dim"], c["theta"], c["max_position_embeddings"], s.get("rope_type", "default"),
        factor=s.get("factor", 1.0), original_max=s.get("original_max_position_embeddings", 0) or 0,
        beta_fast=s.get("beta_fast", 32.0), beta_slow=s.get("beta_slow", 1.0),
        attention_factor=s.get("attention_factor"))
    exp = np.array(c["inv_freq"])
    assert inv.shape == exp.shape
    assert np.all(np.abs(exp - inv) <= 1e-5 * np.abs(exp) + 1e-12)
    assert abs(att - c["attention_factor"]) < 1e-5


def test_rope_llama3_table_known_answer():  # RopeLlama3Tests.cs:9-37
    d = json.loads((GOLDEN / "llama3_table.json").read_text())
    p = d["params"]
    inv, att = orc.rope_frequencies(p["head_dim"], p["theta"], p["max_position_embeddings"], "llama3",
                                    factor=p["factor"], original_max=p["original_max_position_embeddings"],
                                    low_freq_factor=p["low_freq_factor"], high_freq_factor=p["high_freq_factor"])
    exp = np.array(d["expected"])
    assert att == 1.0
    assert np.all(np.abs(inv - exp) / exp <= 1e-5)


def test_rope_linear_and_yarn_identities():  # RopeFrequenciesTests.cs:48-69
    plain, _ = orc.rope_frequencies(16, 10000, 2048)
    lin, att = orc.rope_frequencies(16, 10000, 2048, "linear", factor=4)
    assert att == 1.0
    np.testing.assert_allclose(lin, plain / 4, rtol=1e-6)
    yarn, att = orc.rope_frequencies(16, 10000, 2048, "yarn", factor=1)
    assert att == 1.0
    np.testing.assert_array_equal(yarn, plain)
    with pytest.raises(ValueError):
        orc.rope_frequencies(15, 10000, 2048)


def _hf_rotate(q, k, positions, inv_freq, attn_scale, hd):
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    qt = torch.from_numpy(q).reshape(len(positions), -1, hd).transpose(0, 1).unsqueeze(0)
    kt = torch.from_numpy(k).reshape(len(positions), -1, hd).transpose(0, 1).unsqueeze(0)
    freqs = torch.from_numpy(np.asarray(positions, np.float32))[:, None] * torch.from_numpy(inv_freq)[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    cos, sin = (emb.cos() * attn_scale)[None], (emb.sin() * attn_scale)[None]
    qo, ko = apply_rotary_pos_emb(qt, kt, cos, sin)
    return (qo[0].transpose(0, 1).reshape(len(positions), -1).numpy(),
            ko[0].transpose(0, 1).reshape(len(positions), -1).numpy())


@pytest.mark.parametrize("hd,theta,positions", [(64, 1e6, [0, 1, 7, 300]), (128, 5e5, [2047, 2048, 4095, 32767])])
def test_rope_rotation_matches_transformers(hd, theta, positions):
    rng = np.random.default_rng(9)
    nh, nkv = 4, 2
    q = rng.normal(0, 1, (len(positions), nh * hd)).astype(np.float32)
    k = rng.normal(0, 1, (len(positions), nkv * hd)).astype(np.float32)
    inv, _ = orc.rope_frequencies(hd, theta, 131072)
    qo, ko = orc.rope_table(q, k, positions, inv, hd, nh, nkv, 0.75)
    hq, hk = _hf_rotate(q, k, positions, inv, 0.75, hd)
    np.testing.assert_allclose(qo, hq, rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(ko, hk, rtol=1e-5, atol=2e-6)
    qt, kt = orc.rope_theta(q, k, positions, hd, nh, nkv, theta)
    q1, k1 = orc.rope_table(q, k, positions, inv, hd, nh, nkv, 1.0)
    np.testing.assert_array_equal(qt, q1)
    np.testing.assert_array_equal(kt, k1)
    if positions[0] == 0:  # angle 0: identity
        q0, _ = orc.rope_table(q[:1], k[:1], [0], inv, hd, nh, nkv, 1.0)
        np.testing.assert_array_equal(q0, q[:1])


# ---- cache and attention ----------------------------------------------------------------------

def test_kv_store_places_rows_at_positions():
    kc = np.zeros(8 * 6, dtype=np.float32)
    vc = np.zeros(8 * 6, dtype=np.float32)
    k = np.arange(12, dtype=np.float32)
    orc.kv_store(k, -k, kc, vc, orc.F32, 3, 6, 2)
    np.testing.assert_array_equal(kc.reshape(8, 6)[3:5].reshape(-1), k)
    np.testing.assert_array_equal(vc.reshape(8, 6)[3:5].reshape(-1), -k)
    assert not kc.reshape(8, 6)[[0, 1, 2, 5, 6, 7]].any()
    kh = np.zeros(8 * 6, dtype=np.uint16)
    vh = np.zeros(8 * 6, dtype=np.uint16)
    orc.kv_store(k / 7, k, kh, vh, orc.F16, 0, 6, 2)
    np.testing.assert_array_equal(kh[:12], (k / 7).astype(np.float16).view(np.uint16))


def _sdpa(q, kc, vc, hd, nh, nkv, lengths):
    """torch float64 SDPA; query t attends to cache slots [0, lengths[t])."""
    T = len(lengths)
    L = max(lengths)
    qt = torch.from_numpy(q.astype(np.float64)).reshape(T, nh, hd).transpose(0, 1)  # [nh, T, hd]
    K = torch.from_numpy(kc[:L].astype(np.float64)).reshape(L, nkv, hd).transpose(0, 1)
    V = torch.from_numpy(vc[:L].astype(np.float64)).reshape(L, nkv, hd).transpose(0, 1)
    K = K.repeat_interleave(nh // nkv, dim=0)
    V = V.repeat_interleave(nh // nkv, dim=0)
    mask = torch.tensor([[j < lengths[t] for j in range(L)] for t in range(T)])
    out = torch.nn.functional.scaled_dot_product_attention(qt, K, V, attn_mask=mask)
    return out.transpose(0, 1).reshape(T, nh * hd).numpy()


@pytest.mark.parametrize("hd,nh,nkv,seq", [(64, 14, 2, 37), (128, 32, 8, 300), (128, 8, 8, 1)])
def test_attention_decode_matches_sdpa(hd, nh, nkv, seq):
    rng = np.random.default_rng(10 + seq)
    max_seq = seq + 5
    kc = rng.normal(0, 1, (max_seq, nkv * hd)).astype(np.float32)
    vc = rng.normal(0, 1, (max_seq, nkv * hd)).astype(np.float32)
    q = rng.normal(0, 1, nh * hd).astype(np.float32)
    out = orc.attention_decode(q, kc, vc, orc.F32, hd, nh, nkv, seq, max_seq)
    np.testing.assert_allclose(out, _sdpa(q[None], kc, vc, hd, nh, nkv, [seq])[0], rtol=1e-6, atol=1e-7)
    if seq == 1:  # softmax over one slot: the output is that slot's V row of the group
        for h in range(nh):
            g = h // (nh // nkv)
            np.testing.assert_allclose(out[h * hd:(h + 1) * hd], vc[0, g * hd:(g + 1) * hd], rtol=1e-6)
    kh, vh = kc.astype(np.float16), vc.astype(np.float16)
    out16 = orc.attention_decode(q, kh.view(np.uint16), vh.view(np.uint16), orc.F16, hd, nh, nkv, seq, max_seq)
    np.testing.assert_allclose(out16, _sdpa(q[None], kh.astype(np.float32), vh.astype(np.float32), hd, nh, nkv, [seq])[0],
                               rtol=1e-6, atol=1e-6)


def test_attention_prefill_is_causal_over_cache():
    rng = np.random.default_rng(11)
    hd, nh, nkv, pos0, T, max_seq = 64, 4, 2, 5, 4, 16
    kc = rng.normal(0, 1, (max_seq, nkv * hd)).astype(np.float32)
    vc = rng.normal(0, 1, (max_seq, nkv * hd)).astype(np.float32)
    q = rng.normal(0, 1, (T, nh * hd)).astype(np.float32)
    out = orc.attention_prefill(q, kc, vc, orc.F32, hd, nh, nkv, pos0, T, max_seq).reshape(T, -1)
    want = _sdpa(q, kc, vc, hd, nh, nkv, [pos0 + t + 1 for t in range(T)])
    np.testing.assert_allclose(out, want, rtol=1e-6, atol=1e-7)


# ---- embedding and greedy pick ----------------------------------------------------------------

def test_embedding_known_answer():
    table = np.arange(5 * 3, dtype=np.float32)
    np.testing.assert_array_equal(orc.embedding([4, 0], table, 3, 6), [12, 13, 14, 0, 1, 2])


def test_argmax_first_maximum():  # LlmAbstractions.cs:83-90
    assert orc.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert orc.argmax([-5.0, -5.0]) == 0
    rng = np.random.default_rng(12)
    for _ in range(20):
        v = rng.integers(0, 50, 1000).astype(np.float32)
        assert orc.argmax(v) == int(np.argmax(v))
    assert orc.top2_margin([1.0, 4.0, 2.5]) == 1.5


# ---- whole decoder ----------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["llama", "qwen2"])
def test_model_step_matches_transformers(name):
    d = load_hf(name)
    cfg, prompt = d["cfg"], d["prompt"]
    m = oracle_model(cfg, d["weights"], orc.F32, orc.F32, 64)
    for t, tok in enumerate(prompt):
        _, logits = m.step(tok, t)
        assert rel_err(logits, d["prompt_logits"][t]) < 2e-5, f"position {t}"
    nxt = orc.argmax(logits)
    seq = [nxt]
    pos = len(prompt)
    while len(seq) < len(d["generated"]):
        nxt, _ = m.step(nxt, pos)
        seq.append(nxt)
        pos += 1
    assert seq == d["generated"]


def test_model_rope_table_follows_config():
    d = load_hf("llama")
    inv, att = rope_table_for(d["cfg"])
    plain, _ = orc.rope_frequencies(16, 500000.0, 256)
    assert att == 1.0 and inv.shape == plain.shape and not np.allclose(inv, plain)


@pytest.mark.parametrize("wdtype", [orc.I8PC, orc.F16, orc.BF16, orc.F32])
def test_fp32_baseline_gemv_matches_fp64_restatement(wdtype):
    """The CPU-baseline form (fp32 accumulation, vectorised) computes the same GEMV as the fp64 check
    loop: within fp32 summation error, 1e-5 of the largest output."""
    from tests.helpers import stored
    rng = np.random.default_rng(77 + wdtype)
    w = rng.normal(0, 0.02, (300, 896)).astype(np.float32)
    dt, ws, s = stored(wdtype, w)
    x = rng.normal(0, 1, (3, 896)).astype(np.float32)
    want = orc.gemv_nk(dt, ws, x, s)
    got = orc.gemv_nk_f32acc(dt, ws, x, s)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
    # a wrong accumulation (one term dropped) would not pass
    bad = orc.gemv_nk_f32acc(dt, np.ascontiguousarray(ws[:, :-1]), x[:, :-1], s)
    assert np.max(np.abs(bad - want)) > 1e-5 * np.max(np.abs(want))


@pytest.mark.parametrize("wide_layer", [None, 1])
def test_device_rounding_rounds_attention_and_swiglu_outputs(wide_layer):
    """orc_set_device_rounding: a decode step with it on equals the step composed from the oracle's
    separately pinned primitives with numpy fp16 casts of the attention output and of the SwiGLU
    output (the latter only when every value is within fp16's range), bit for bit; off, the step
    differs. wide_layer: that layer's gate / up weights scaled so its SwiGLU output exceeds 65504
    (kept in fp32)."""
    from tests.helpers import stored
    rng = np.random.default_rng(4242)
    H, I, L, nh, nkv, hd, V, max_seq = 64, 128, 2, 4, 2, 16, 50, 8
    cfg = dict(vocab_size=V, hidden_size=H, intermediate_size=I, num_layers=L, num_attention_heads=nh,
               num_key_value_heads=nkv, head_dim=hd, rms_norm_eps=1e-5)
    shapes = {"self_attn.q_proj.weight": (nh * hd, H), "self_attn.k_proj.weight": (nkv * hd, H),
              "self_attn.v_proj.weight": (nkv * hd, H), "self_attn.o_proj.weight": (H, nh * hd),
              "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H), "mlp.down_proj.weight": (H, I)}
    w = {"model.embed_tokens.weight": rng.normal(0, 1, V * H).astype(np.float32),
         "model.norm.weight": rng.normal(1, 0.1, H).astype(np.float32),
         "lm_head.weight": stored(orc.I8PC, rng.normal(0, 0.05, (V, H)))}
    for i in range(L):
        p = f"model.layers.{i}."
        for n, shp in shapes.items():
            scale = 30.0 if (i == wide_layer and n.startswith("mlp.") and "down" not in n) else 0.1
            w[p + n] = stored(orc.I8PC, rng.normal(0, scale, shp))
        w[p + "input_layernorm.weight"] = rng.normal(1, 0.1, H).astype(np.float32)
        w[p + "post_attention_layernorm.weight"] = rng.normal(1, 0.1, H).astype(np.float32)
    inv, att = orc.rope_frequencies(hd, 10000.0, 4096)
    model = orc.Model(cfg, w, inv, att, orc.F16, max_seq)
    plain = orc.Model(cfg, w, inv, att, orc.F16, max_seq)
    kvd = nkv * hd
    kc = [np.zeros(max_seq * kvd * 2, np.uint8) for _ in range(L)]
    vc = [np.zeros(max_seq * kvd * 2, np.uint8) for _ in range(L)]

    def proj(name, x):
        dt, ws, s = w[name]
        return orc.gemv_nk(dt, ws, x, s)[0]

    def composed(tok, pos):
        hidden = orc.embedding([tok], w["model.embed_tokens.weight"], H, H)
        wide_seen = False
        for i in range(L):
            p = f"model.layers.{i}."
            _, normed = orc.rmsnorm(hidden, w[p + "input_layernorm.weight"], 1e-5)
            q = proj(p + "self_attn.q_proj.weight", normed)
            k = proj(p + "self_attn.k_proj.weight", normed)
            v = proj(p + "self_attn.v_proj.weight", normed)
            q, k = orc.rope_table(q, k, [pos], inv, hd, nh, nkv, att)
            orc.kv_store(k, v, kc[i], vc[i], orc.F16, pos, kvd, 1)
            a = orc.attention_decode(q, kc[i], vc[i], orc.F16, hd, nh, nkv, pos + 1, max_seq)
            a = a.astype(np.float16).astype(np.float32)
            hidden, normed = orc.rmsnorm(hidden, w[p + "post_attention_layernorm.weight"], 1e-5,
                                         residual=proj(p + "self_attn.o_proj.weight", a))
            act = orc.swiglu(proj(p + "mlp.gate_proj.weight", normed), proj(p + "mlp.up_proj.weight", normed))
            if np.all(np.abs(act) <= 65504.0):
                act = act.astype(np.float16).astype(np.float32)
            else:
                wide_seen = True
            hidden = orc.add(hidden, proj(p + "mlp.down_proj.weight", act))
        _, normed = orc.rmsnorm(hidden, w["model.norm.weight"], 1e-5)
        return proj("lm_head.weight", normed), wide_seen

    try:
        for pos, tok in enumerate([3, 17, 41, 9]):
            orc.set_device_rounding(True)
            _, got = model.step(tok, pos)
            orc.set_device_rounding(False)
            _, ref = plain.step(tok, pos)
            want, wide_seen = composed(tok, pos)
            np.testing.assert_array_equal(got, want)
            assert not np.array_equal(got, ref)  # the rounding is not a no-op
            assert wide_seen == (wide_layer is not None)
    finally:
        orc.set_device_rounding(False)
