"""GPU tests of the drop-in members an unchanged LlmMatrix / LlmModel call through a LevelZero-shaped
shim: the GemvQ8 members and scratch (LlmMatrix.cs:29-31, :89-94, :122-171, :231-251; LlmModel.cs:139-144),
the reference-layout [K, N] Gemv (LlmMatrix.cs:134-165), and the rules for memory that a recording
uses (workspace sizing before recording, replay after a free)."""
from __future__ import annotations

import numpy as np
import pytest

import l0llm_amd as l0
from oracle import pyoracle as orc
from tests.helpers import rel_err

pytestmark = pytest.mark.gpu


def up(device, a):
    return device.alloc_shared(np.ascontiguousarray(a))


# ---- GemvQ8 members (LlmMatrixInt8Tests.cs:80-149 pattern) -------------------------------------

def test_q8_members_project_like_llm_matrix(device, suite):
    """Quantize + Execute / ExecuteRows through the scratch, as LlmMatrix.Project(Rows) calls them, with
    the words and scales of l0h_quantize_i8pc (the shim's LlmQ8Quantizer.QuantizeOutIn)."""
    assert suite.q8_group_size() == 32
    rng = np.random.default_rng(81)
    n, k, rows = 1152, 896, 5
    hf = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    q, s = l0.quantize_i8pc(hf)
    words = q.view(np.int32)  # four int8 per 32-bit word, as the reference's int[] words
    assert words.shape == (n, k // 4)
    wb, sb = up(device, words), up(device, s)
    suite.ensure_q8_scratch(l0.lib.l0h_gemv_max_rows(), (k + 31) // 32 * 32)
    scratch = suite.q8_scratch
    assert scratch is not None and scratch.row_capacity == l0.lib.l0h_gemv_max_rows()
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    xb, yb = up(device, x), device.alloc(rows * n * 4)
    want = orc.gemv_nk(orc.I8PC, q, x, s)
    suite.gemv_q8_quantize(rows, k, xb, scratch)
    suite.gemv_q8_execute_rows(rows, n, k, scratch, wb, sb, yb)
    assert rel_err(yb.read(np.float32).reshape(rows, n), want) < 2e-5
    suite.gemv_q8_quantize(1, k, xb, scratch)
    suite.gemv_q8_execute(n, k, scratch, wb, sb, yb)
    assert rel_err(yb.read(np.float32, n), want[0]) < 2e-5
    # RequireScratch (LlmMatrix.cs:244-251): more rows than the scratch holds is an InvalidOperation.
    big = device.alloc((l0.lib.l0h_gemv_max_rows() + 1) * k * 4)
    with pytest.raises(l0.InvalidOperationError):
        suite.gemv_q8_quantize(l0.lib.l0h_gemv_max_rows() + 1, k, big, scratch)
    # Inside a recording the scratch is used as is; growing it there is refused (LlmModel.cs:141).
    yb.zero()
    device.begin_recording()
    suite.gemv_q8_quantize(rows, k, xb, scratch)
    suite.gemv_q8_execute_rows(rows, n, k, scratch, wb, sb, yb)
    with pytest.raises(l0.InvalidOperationError):
        suite.ensure_q8_scratch(64, 1 << 16)
    device.end_recording()
    assert rel_err(yb.read(np.float32).reshape(rows, n), want) < 2e-5


# ---- reference-layout [K, N] Gemv --------------------------------------------------------------

# Config 1 / config 2 shapes in the reference layout (K -> N): up 896 -> 4864, q|k|v 896 -> 1152,
# O 896 -> 896, gate|up 896 -> 9728, down 4864 -> 896, lm_head 896 -> 151936; MaxRows groups; a K that
# is no multiple of a slice; the any-shape path (N % 8 != 0).
KN_CASES = [(4864, 896, 1, l0.F16), (1152, 896, 1, l0.F16), (896, 896, 1, l0.F16), (9728, 896, 1, l0.F16),
            (896, 4864, 1, l0.F16), (151936, 896, 1, l0.F16), (4864, 896, 8, l0.F16), (4864, 896, 5, l0.F32),
            (1000, 300, 2, l0.F32), (2048, 1000, 3, l0.F16), (4100, 64, 1, l0.F16), (30, 17, 2, l0.F16),
            (4864, 896, 1, l0.F32), (1000, 1000, 1, l0.F16), (896, 14336, 1, l0.F16)]


@pytest.mark.parametrize("n,k,rows,wdt", KN_CASES)
def test_gemv_kn_tiled_matches_oracle(device, suite, n, k, rows, wdt):
    rng = np.random.default_rng(n * 3 + k + rows)
    w = rng.normal(0, 0.02, (k, n)).astype(np.float32)
    ws = w.astype(np.float16).view(np.uint16) if wdt == l0.F16 else w
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    want = orc.gemv_kn(wdt, ws, x)
    wb, xb, yb = up(device, ws), up(device, x), device.alloc(rows * n * 4)
    suite.gemv_execute_rows(rows, n, k, xb, wb, yb, w_dtype=wdt)
    got = yb.read(np.float32).reshape(rows, n)
    # fp32 accumulation in a different order: 2e-5 of the largest output (LlmMatrixTests.cs:71-80
    # asks 1e-4 absolute against fp64).
    assert rel_err(got, want) < 2e-5, rel_err(got, want)
    assert np.max(np.abs(got - want)) < 1e-4
    # Recorded: the workspace cannot grow, so fewer K slices run; same values within fp32 reordering.
    yb.zero()
    device.begin_recording()
    suite.gemv_execute_rows(rows, n, k, xb, wb, yb, w_dtype=wdt)
    device.end_recording()
    assert rel_err(yb.read(np.float32).reshape(rows, n), want) < 2e-5
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("n,k", [(896, 896), (896, 4864), (896, 14336)])
def test_gemv_kn_split_merge_repeats_bit_exact(device, suite, n, k):
    """One-row K-split launches (partials + a fixed-order slice sum): eager repeats and graph replays
    give the same bits as the first call."""
    rng = np.random.default_rng(n + 5 * k)
    w = rng.normal(0, 0.02, (k, n)).astype(np.float16).view(np.uint16)
    x = rng.normal(0, 1, k).astype(np.float32)
    wb, xb, yb = up(device, w), up(device, x), device.alloc(n * 4)
    suite.gemv_execute(n, k, xb, wb, yb, w_dtype=l0.F16)
    first = yb.read(np.float32, n)
    assert rel_err(first, orc.gemv_kn(l0.F16, w, x[None])[0]) < 2e-5
    for _ in range(3):
        yb.zero()
        suite.gemv_execute(n, k, xb, wb, yb, w_dtype=l0.F16)
        np.testing.assert_array_equal(yb.read(np.float32, n), first)
    device.begin_recording()
    suite.gemv_execute(n, k, xb, wb, yb, w_dtype=l0.F16)
    device.end_recording()
    for _ in range(3):
        yb.zero()
        device.replay_recording(2)
        np.testing.assert_array_equal(yb.read(np.float32, n), first)
    for b in (wb, xb, yb):
        b.free()


# ---- memory a recording uses ----------------------------------------------------------------------

def test_replay_refused_after_free_or_workspace_growth():
    """A kept recording may address freed memory: l0h_replay_recording refuses after l0h_free or a
    workspace reallocation, and works again after the next recording."""
    with l0.Device(0) as dev:
        suite = l0.LlmKernelSuite(dev)
        a, b = dev.alloc_shared(np.arange(256, dtype=np.float32)), dev.alloc(256 * 4)
        dev.begin_recording()
        suite.copy_execute(a, b, 0, 256)
        dev.end_recording()
        assert dev.replay_recording(2) >= 0
        spare = dev.alloc(1024)
        spare.free()
        with pytest.raises(l0.InvalidOperationError):
            dev.replay_recording(1)
        dev.begin_recording()
        suite.copy_execute(a, b, 0, 256)
        dev.end_recording()
        assert dev.replay_recording(1) >= 0
        # Workspace growth (attention at a long context) moves the workspace the recording may use.
        suite.attention_reserve(8, 32, 8, 128, 1 << 20)
        with pytest.raises(l0.InvalidOperationError):
            dev.replay_recording(1)
        np.testing.assert_array_equal(b.read(np.float32), np.arange(256, dtype=np.float32))


def test_attention_recorded_without_reserve_uses_the_workspace_it_has():
    """Decode attention at 131072 positions wants more split partials than the 1 MiB workspace a device
    starts with; recorded without l0h_attention_reserve it runs with fewer splits, with it at the default
    count. Both match the oracle."""
    nh, nkv, hd, max_seq, seq = 32, 8, 128, 131072, 777
    rng = np.random.default_rng(131)
    kv = nkv * hd
    k = rng.normal(0, 1, (seq, kv)).astype(np.float16)
    v = rng.normal(0, 1, (seq, kv)).astype(np.float16)
    q = rng.normal(0, 1, nh * hd).astype(np.float32)
    want = orc.attention_decode(q, k.view(np.uint16), v.view(np.uint16), orc.F16, hd, nh, nkv, seq, seq)
    with l0.Device(0) as dev:
        suite = l0.LlmKernelSuite(dev)
        kc, vc = dev.alloc(max_seq * kv * 2), dev.alloc(max_seq * kv * 2)
        kc.write(k)
        vc.write(v)
        qb, ob = up(dev, q), dev.alloc(nh * hd * 4)
        for reserve in (False, True):
            if reserve:
                suite.attention_reserve(1, nh, nkv, hd, max_seq)
            ob.zero()
            dev.begin_recording()
            suite.attention_execute(qb, kc, vc, ob, hd, nh, nkv, seq, max_seq, cache_dtype=l0.F16)
            dev.end_recording()
            assert rel_err(ob.read(np.float32), want) < 1e-4


# ---- the reference's decode step, operator by operator (the drop-in path) -----------------------

def test_reference_operator_sequence_matches_oracle_and_model(device):
    """LlmModel.Step over LlmDecoderLayer.Forward / MixFull as an unchanged C# host would issue them
    on this library (l0llm_amd.reference_step: 18 operators per layer, 5 per token, fp32 activations
    between them), on the 2-layer Llama-3.1-8B-shaped int8 model after a 300-token prefill by the
    model: recorded steps against the oracle seeded with the same cache rows (both keep fp32
    activations: 1e-4 of max|logit|) and against the model's fused step (fp16 attention and SwiGLU
    outputs between kernels: 2e-3), greedy ids equal unless the oracle's top-2 gap is within the
    bound, and eager steps equal to the recorded ones bit for bit. The recording holds 19 kernels per
    layer (the attention's split and merge) and the 5 of the head."""
    import dataclasses

    from l0llm_amd.reference_step import ReferenceStep
    from tests.test_gpu_model import LLAMA8B, _as_cfg, exported_oracle, exported_weights

    hf = dataclasses.replace(LLAMA8B, num_layers=2)
    n, max_seq = 300, 340
    prompt = np.random.default_rng(300).integers(0, hf.vocab_size, n).tolist()
    with l0.LlmModel(device, hf, precision=l0.PRECISION_INT8, cache_dtype=l0.F16, max_seq_len=max_seq) as m:
        m.init_random(301, 0.02)
        first = int(np.argmax(m.prefill(prompt)))
        w = exported_weights(m, _as_cfg(hf))
        om = exported_oracle(m, _as_cfg(hf), orc.F16, max_seq)
        kv_bytes = n * hf.num_key_value_heads * hf.head_dim * 2
        for layer in range(hf.num_layers):  # the prompt's rows 0 .. n - 1, as the device holds them
            kp, vp = m.kv_cache(layer)
            om.load_cache(layer, l0.Buffer(device, kv_bytes, ptr=kp, owned=False).read(np.uint8),
                          l0.Buffer(device, kv_bytes, ptr=vp, owned=False).read(np.uint8))
        ref = ReferenceStep(device, hf, w, max_seq, [m.kv_cache(i) for i in range(hf.num_layers)])
        try:
            tok = first
            for t in range(n, n + 4):
                ref.set_token(tok, t)
                ref.record_step(t)
                if t == n:
                    launches = device.recording_launches
                got, picked = ref.read_logits(), ref.read_sampled()
                ref.step(t)  # the same operators without a recording
                np.testing.assert_array_equal(ref.read_logits(), got)
                onext, olg = om.step(tok, t)
                assert rel_err(got, olg) < 1e-4, (t, rel_err(got, olg))
                assert rel_err(got, m.compute_logits(tok, t)) < 2e-3, t
                assert picked == int(np.argmax(got))
                if picked != onext:
                    assert orc.top2_margin(olg) < 2e-4 * np.max(np.abs(olg)), (t, picked, onext)
                tok = onext
            assert launches >= 19 * hf.num_layers + 5, launches
        finally:
            ref.close()
