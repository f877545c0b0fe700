"""GPU parity at the workload shapes the path is measured on, against the oracle on identical seeded
inputs: the Qwen2.5-0.5B decode linears in fp16 (fused O, gate|up + SwiGLU, lm_head), the eight
Llama-3.2-1B prefill GEMMs in bf16 at M = 128 and 512, GQA decode attention at batch 1 and 8 over 512,
4096 and 32768 positions, the Llama-3.1-8B int8 decode step at a 2048-token context (the split
attention the timed step runs), and int8 GEMV rows whose activations have a large mean or outlier
channels. Tolerances are written at each assertion."""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

import l0llm_amd as l0
from oracle import pyoracle as orc
from tests.helpers import bf16_bits, dequant, elementwise_excess, rel_err, stored
from tests.test_gpu_model import LLAMA8B, QWEN05, _as_cfg, exported_oracle

pytestmark = pytest.mark.gpu


def up(device, a):
    return device.alloc_shared(np.ascontiguousarray(a))


def normal16(rng, shape, dtype=np.float16) -> np.ndarray:
    """N(0, 1) samples rounded to fp16, generated in chunks (large caches)."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=dtype)
    step = 1 << 24
    for i in range(0, n, step):
        out[i:i + step] = rng.standard_normal(min(step, n - i), dtype=np.float32)
    return out.reshape(shape)


# ---- Qwen2.5-0.5B decode linears at M = 1 (fp16 and int8 weights) --------------------------------

# (N, K) of O 896 -> 896, fused gate|up 896 -> 2 x 4864 and lm_head 896 -> 151936 (q|k|v, up and down
# are in the kernel tests).
@pytest.mark.parametrize("n,k", [(896, 896), (9728, 896), (151936, 896)], ids=["o", "gate_up", "lm_head"])
@pytest.mark.parametrize("storage", [l0.F16, l0.I8PC, l0.BF16])
def test_qwen05_decode_linear_shapes(device, suite, storage, n, k):
    rng = np.random.default_rng(200 + n + storage)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    x = rng.normal(0, 1, k).astype(np.float32)
    dt, ws, s = stored(storage, w)
    want = orc.gemv_nk(dt, ws, x, s)[0]
    wb, xb, yb = up(device, ws), up(device, x), device.alloc(n * 4)
    sb = up(device, s) if s is not None else None
    suite.gemv_nk(storage, 1, n, k, xb, l0.F32, wb, sb, yb, l0.F32)
    assert rel_err(yb.read(np.float32, n), want) < 2e-5  # fp32 accumulation, different order
    # fp16 output: relative error at most 1e-2 per element (floor 1e-4 of max|y| near zero)
    y16 = device.alloc(n * 2)
    suite.gemv_nk(storage, 1, n, k, xb, l0.F32, wb, sb, y16, l0.F16)
    got = y16.read(np.float16, n).astype(np.float64)
    assert elementwise_excess(got, want) <= 1.0


@pytest.mark.parametrize("precision", [l0.PRECISION_FLOAT16, l0.PRECISION_BFLOAT16])
def test_qwen05_16bit_model_matches_oracle(device, precision):
    """The 4-layer Qwen2.5-0.5B-shaped model with fp16 (or bf16) weights, N(0, 0.02): the fused q|k|v
    (bias, RoPE, cache), O + residual, RMSNorm + gate|up + SwiGLU, down + residual and the tied
    lm_head 896 -> 151936 against the oracle on the weights the device holds."""
    max_seq, steps = 16, 6
    with l0.LlmModel(device, QWEN05, precision=precision, cache_dtype=l0.F16, max_seq_len=max_seq) as m:
        m.init_random(202, 0.02)
        om = exported_oracle(m, _as_cfg(QWEN05), orc.F16, max_seq)
        tok = int(np.random.default_rng(202).integers(0, QWEN05.vocab_size))
        for t in range(steps):
            lg = m.compute_logits(tok, t)
            onext, olg = om.step(tok, t)
            # the attention output is fp16 between kernels (within the fp16 cache's range), fp32 in
            # the oracle
            assert rel_err(lg, olg) < 2e-3, t
            if int(np.argmax(lg)) != onext:
                assert orc.top2_margin(olg) < 1e-3 * np.max(np.abs(olg)), t
            tok = onext


# ---- Llama-3.2-1B prefill GEMMs (bf16, M = 128 and 512) -----------------------------------------

LLAMA1B_GEMMS = [(3072, 2048), (2048, 2048), (16384, 2048), (2048, 8192)]


@pytest.mark.parametrize("m", [128, 512])
@pytest.mark.parametrize("n,k", LLAMA1B_GEMMS, ids=["qkv", "o", "gate_up", "down"])
def test_llama1b_prefill_gemm_bf16(device, suite, m, n, k):
    """bf16 W ~ N(0, 0.02), bf16 X ~ N(0, 1), fp32 accumulation on MFMA; fp32 and bf16 outputs. The
    fp64 oracle runs a seeded subset of 24 rows (every tile row group is represented)."""
    rng = np.random.default_rng(300 + m + n + k)
    xs = bf16_bits(rng.standard_normal((m, k), dtype=np.float32))
    ws = bf16_bits(rng.standard_normal((n, k), dtype=np.float32) * 0.02)
    rows = np.sort(np.concatenate([[0, m - 1], rng.choice(np.arange(1, m - 1), 22, replace=False)]))
    xf = dequant(l0.BF16, xs[rows], None).astype(np.float32)
    want = orc.gemv_nk(l0.BF16, ws, xf)
    xb, wb = up(device, xs), up(device, ws)
    yb = device.alloc(m * n * 4)
    suite.gemm_nk(l0.BF16, m, n, k, xb, wb, yb, l0.F32)
    got = yb.read(np.float32).reshape(m, n)[rows]
    assert rel_err(got, want) < 2e-5
    y16 = device.alloc(m * n * 2)
    suite.gemm_nk(l0.BF16, m, n, k, xb, wb, y16, l0.BF16)
    g16 = (y16.read(np.uint16).reshape(m, n)[rows].astype(np.uint32) << 16).view(np.float32)
    # bf16 output: relative error at most 1e-2 per element (floor 1e-4 of max|y| near zero)
    assert elementwise_excess(g16, want) <= 1.0
    for b in (xb, wb, yb, y16):
        b.free()


# ---- GQA decode attention (32 q / 8 kv heads, head_dim 128, fp16) -------------------------------

@pytest.mark.parametrize("batch,ctx", [(1, 512), (1, 4096), (8, 4096), (8, 32768)])
def test_gqa_decode_attention_config(device, suite, batch, ctx):
    """fp16 q / K / V ~ N(0, 1); q rotated by RoPE (theta 500000) at position ctx - 1, cached K taken as
    already rotated; causal over slots 0 .. ctx - 1, scale 1/sqrt(128), fp32 softmax, fp16 output.
    Batch 8 x 32768 takes two blocks per CU with 2048-position splits."""
    hd, nh, nkv = 128, 32, 8
    rng = np.random.default_rng(400 + batch * ctx)
    k = normal16(rng, (batch, ctx, nkv * hd))
    v = normal16(rng, (batch, ctx, nkv * hd))
    q = rng.standard_normal((batch, nh * hd), dtype=np.float32)
    kz = np.zeros(nkv * hd, np.float32)
    for b in range(batch):
        q[b], _ = orc.rope_theta(q[b], kz, [ctx - 1], hd, nh, nkv, 500000.0)
    q16 = q.astype(np.float16)
    ob = device.alloc(batch * nh * hd * 2)
    kb, vb, qb = up(device, k.view(np.uint16)), up(device, v.view(np.uint16)), up(device, q16.view(np.uint16))
    suite.attention_decode(qb, l0.F16, kb, vb, l0.F16, ob, l0.F16, batch, hd, nh, nkv, ctx, ctx)
    out = ob.read(np.float16).astype(np.float64).reshape(batch, -1)
    for b in range(batch):
        want = orc.attention_decode(q16[b].astype(np.float32), k[b].view(np.uint16), v[b].view(np.uint16), orc.F16,
                                    hd, nh, nkv, ctx, ctx)
        # fp16 output: relative error at most 1e-2 per element (floor 1e-4 of max|out| near zero)
        assert elementwise_excess(out[b], want) <= 1.0, b
    for buf in (kb, vb, qb, ob):
        buf.free()


# ---- Llama-3.1-8B int8 decode at a 2048-token context --------------------------------------------

def test_llama8b_int8_decode_after_2048_token_prefill(device):
    """Two layers at the 8B shapes (hidden 4096, intermediate 14336, 32/8 heads, vocab 128256), int8
    per-row weights, fp16 cache, the timed step's cache length (2078 slots: 17 attention splits).
    2048 seeded prompt tokens are prefilled on the device; the oracle is seeded with the device's KV
    cache and both run 4 greedy steps at positions 2048..2051: logits within 2e-3 of max|logit| and
    identical greedy ids (or a top-2 gap below the accumulation noise)."""
    hf = dataclasses.replace(LLAMA8B, num_layers=2)
    max_seq, ctx = 2078, 2048
    rng = np.random.default_rng(599)
    prompt = rng.integers(0, hf.vocab_size, ctx).tolist()
    with l0.LlmModel(device, hf, precision=l0.PRECISION_INT8, cache_dtype=l0.F16, max_seq_len=max_seq) as m:
        m.init_random(599, 0.02)
        om = exported_oracle(m, _as_cfg(hf), orc.F16, max_seq)
        m.prefill(prompt[:-1])  # slots 0 .. 2046; the last prompt token runs as the first decode step
        kv_bytes = (ctx - 1) * hf.num_key_value_heads * hf.head_dim * 2
        for layer in range(hf.num_layers):
            kp, vp = m.kv_cache(layer)
            kc = l0.Buffer(device, kv_bytes, ptr=kp, owned=False).read(np.uint8)
            vc = l0.Buffer(device, kv_bytes, ptr=vp, owned=False).read(np.uint8)
            om.load_cache(layer, kc, vc)
        tok = prompt[-1]
        for t in range(ctx - 1, ctx + 4):
            lg = m.compute_logits(tok, t)
            onext, olg = om.step(tok, t)
            assert rel_err(lg, olg) < 2e-3, t
            gnext = int(np.argmax(lg))
            if gnext != onext:
                assert orc.top2_margin(olg) < 1e-3 * np.max(np.abs(olg)), (t, gnext, onext)
            tok = onext


# ---- int8 GEMV rows with a large mean and outlier channels ---------------------------------------

@pytest.mark.parametrize("n,k", [(4096, 4096), (4096, 14336), (1152, 896)])
@pytest.mark.parametrize("x_dtype", [l0.F32, l0.F16])
def test_int8_gemv_large_mean_and_outlier_activations(device, suite, n, k, x_dtype):
    """Activations N(1000, 1) (a mean far above the spread) and N(0, 1) with 8 channels at +-1600 (the
    magnitude of the Qwen2.5 layer golden's outliers): the int8 bias is removed per 16-byte chunk, so
    no cancellation against sum(x) remains. fp32 accumulation: 2e-5 of the largest output."""
    rng = np.random.default_rng(n + k + x_dtype)
    q = rng.integers(-127, 128, (n, k), dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, n).astype(np.float16)
    xm = (1000.0 + rng.standard_normal(k)).astype(np.float32)
    xo = rng.standard_normal(k).astype(np.float32)
    xo[rng.choice(k, 8, replace=False)] = rng.choice([-1600.0, 1600.0], 8)
    qb, sb, yb = up(device, q), up(device, s.view(np.uint16)), device.alloc(n * 4)
    for x in (xm, xo):
        xr = x.astype(np.float16).astype(np.float32) if x_dtype == l0.F16 else x
        want = orc.gemv_nk(orc.I8PC, q, xr, s.view(np.uint16))[0]
        xb = up(device, x.astype(np.float16) if x_dtype == l0.F16 else x)
        suite.gemv_nk(l0.I8PC, 1, n, k, xb, x_dtype, qb, sb, yb, l0.F32)
        got = yb.read(np.float32, n)
        assert rel_err(got, want) < 2e-5, rel_err(got, want)
        # and row by row, against each row's own magnitude plus the rounding of its terms
        scale = np.abs(q).astype(np.float64) @ np.abs(xr).astype(np.float64) * s.astype(np.float64)
        assert np.all(np.abs(got - want) <= 1e-5 * scale + 1e-6)
        xb.free()


def test_swiglu_output_beyond_fp16_range_matches_oracle(device):
    """Gate / up weights scaled so that SwiGLU outputs exceed 65504 (fp16's largest value): the decode
    step keeps down's input in fp32, so the logits stay finite and match the oracle."""
    hf = l0.HfConfig(hidden_size=256, intermediate_size=512, num_layers=2, num_attention_heads=4,
                     num_key_value_heads=2, head_dim=64, vocab_size=1000, max_position_embeddings=4096,
                     rms_norm_eps=1e-5, rope_theta=500000.0)
    rng = np.random.default_rng(65504)
    H, I = hf.hidden_size, hf.intermediate_size
    for precision in (l0.PRECISION_INT8, l0.PRECISION_FLOAT16, l0.PRECISION_BFLOAT16):
        with l0.LlmModel(device, hf, precision=precision, cache_dtype=l0.F16, max_seq_len=8) as m:
            m.init_random(11, 0.02)
            for i in range(hf.num_layers):
                p = f"model.layers.{i}.mlp."
                m.set_tensor(p + "gate_proj.weight", rng.normal(0, 30.0, (I, H)).astype(np.float32))
                m.set_tensor(p + "up_proj.weight", rng.normal(0, 30.0, (I, H)).astype(np.float32))
            om = exported_oracle(m, _as_cfg(hf), orc.F16, 8)
            # the first layer's SwiGLU output, from the oracle's own arithmetic, is far above 65504
            for t, tok in enumerate([3, 14, 159]):
                lg = m.compute_logits(tok, t)
                _, olg = om.step(tok, t)
                assert np.all(np.isfinite(lg))
                assert rel_err(lg, olg) < 2e-3, (precision, t, rel_err(lg, olg))


@pytest.mark.parametrize("precision,tol", [(l0.PRECISION_INT8, 3e-3), (l0.PRECISION_FLOAT16, 3e-3),
                                           (l0.PRECISION_BFLOAT16, 1.5e-2)])
def test_swiglu_output_beyond_fp16_range_prefill_matches_oracle_and_decode(device, precision, tol):
    """The scaled gate / up weights of the test above through a 72-token prefill: 71 rows take the
    MFMA GEMMs, whose down operand rows are fp16 for int8 / fp16 weights. The gate|up GEMM flags the
    saturated SwiGLU values, so each such layer's down projection runs on fp32 rows (bf16 rows keep
    fp32's range and need no flag). The prefill's last logits match the oracle stepped token by token
    and the device's own token-by-token decode (bounds relative to max|logit|: the fp16 / bf16
    rounding of the GEMM operands, as the chunked-prefill tests); a saturated down input would be off
    by far more (the first layer's SwiGLU outputs reach well above 65504)."""
    hf = l0.HfConfig(hidden_size=256, intermediate_size=512, num_layers=2, num_attention_heads=4,
                     num_key_value_heads=2, head_dim=64, vocab_size=1000, max_position_embeddings=4096,
                     rms_norm_eps=1e-5, rope_theta=500000.0)
    rng = np.random.default_rng(65504)
    H, I = hf.hidden_size, hf.intermediate_size
    gates = [(rng.normal(0, 30.0, (I, H)).astype(np.float32), rng.normal(0, 30.0, (I, H)).astype(np.float32))
             for _ in range(hf.num_layers)]
    prompt = np.random.default_rng(72).integers(0, hf.vocab_size, 72).tolist()
    with l0.LlmModel(device, hf, precision=precision, cache_dtype=l0.F16, max_seq_len=80) as m:
        m.init_random(11, 0.02)
        for i, (g, u) in enumerate(gates):
            m.set_tensor(f"model.layers.{i}.mlp.gate_proj.weight", g)
            m.set_tensor(f"model.layers.{i}.mlp.up_proj.weight", u)
        om = exported_oracle(m, _as_cfg(hf), orc.F16, 80)
        olg = None
        for t, tok in enumerate(prompt):
            _, olg = om.step(tok, t)
        seq = None
        for t, tok in enumerate(prompt):
            seq = m.compute_logits(tok, t)
        batched = m.prefill(prompt)
        assert m.position == len(prompt)
        assert np.all(np.isfinite(batched))
        scale = np.max(np.abs(olg))
        assert np.max(np.abs(batched - olg)) <= tol * scale, (precision, np.max(np.abs(batched - olg)) / scale)
        assert np.max(np.abs(batched - seq)) <= tol * scale, (precision, np.max(np.abs(batched - seq)) / scale)
