"""Greedy-decode parity at the measured configuration, and two invariants of the reference's own
tests restated on the device.

- The full 32-layer Llama-3.1-8B-shaped int8 model with the timed run's weights (seed 500), prompt
  (2048 ids, seed 599) and cache length: the device prefills the prompt, two oracles are seeded with
  the device's cache rows and run the last prompt token and 10 teacher-forced steps next to the
  device, and the device-side greedy loop that the timed run replays gives exactly the step-by-step
  ids (Qwen25GenerationGoldenTests.cs:103-126 checks generation token for token with the
  reference's top-2 margins, gen_generation_golden.py:51-54). The oracles: the reference's fp32
  activations, and the same with the attention and SwiGLU outputs rounded to fp16 where the device
  stores them so between kernels (orc_set_device_rounding). Against the rounding oracle only the
  arithmetic differs (fp32 against fp64 sums, hardware exp2), and this random-init 32-layer network
  amplifies such differences: the rounding oracle's own fp32-sum form is 1.0-1.5e-3 of max|logit|
  from its fp64 form at these positions, and the device 1.0-1.5e-3 (measured on MI355X); against the
  fp32-activation oracle the device is 1.5-2.1e-3 away. So the device must stay within 3e-3 of the
  rounding oracle and within 3x that oracle's own fp32 spread at the same step (arithmetic noise, not
  a missing term), within 5e-3 of the fp32-activation oracle, and its greedy ids must be identical
  unless the oracle's top-2 gap is within twice the bound.
- Prefill restarts from position 0 each time: a prefill, a longer one, then the first again give the
  same logits and position (Qwen25PrefillTests.cs:76-89), on the MFMA GEMM path (>= 64 rows) and on
  the multi-row GEMV path (short prompts).
- Greedy generation is deterministic across runs (Qwen25GenerationGoldenTests.cs:180-191): two
  device-side greedy loops from the same prefill give the same ids and bitwise-equal logits.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

import l0llm_amd as l0
from oracle import pyoracle as orc
from tests.helpers import rel_err
from tests.test_gpu_model import LLAMA8B, _as_cfg, exported_oracle

pytestmark = pytest.mark.gpu

# bench.py's defaults: 2048 prompt tokens + 128 timed + 8 CPU-baseline + 8 spare cache slots
BENCH_CTX, BENCH_MAX_SEQ = 2048, 2048 + 128 + 8 + 8
# Logit bounds relative to max|logit| at the full depth: against the reference-semantics oracle and
# against the oracle that rounds where the device stores fp16.
TOL_REF, TOL_ROUNDED = 5e-3, 3e-3


def _flush(msg: str) -> None:
    print(f"[step] {msg}", flush=True)


def test_llama8b_full_depth_greedy_ids_at_2048_context(device):
    hf = LLAMA8B
    prompt = np.random.default_rng(599).integers(0, hf.vocab_size, BENCH_CTX).tolist()
    steps = 10
    with l0.LlmModel(device, hf, precision=l0.PRECISION_INT8, cache_dtype=l0.F16, max_seq_len=BENCH_MAX_SEQ) as m:
        m.init_random(500, 0.02)
        _flush("exporting the 32-layer model to the oracles")
        # the reference's fp32 activations, and rounded where the device stores fp16 (same weights)
        om, orr, o32 = exported_oracle(m, _as_cfg(hf), orc.F16, BENCH_MAX_SEQ, copies=3)
        _flush("prefilling 2048 tokens")
        last = m.prefill(prompt)
        assert m.position == BENCH_CTX
        # cache rows 0 .. 2046 (the prefill's chunk); row 2047 comes from the last token's decode step,
        # which the oracles run themselves
        rows = BENCH_CTX - 1
        kv_bytes = rows * hf.num_key_value_heads * hf.head_dim * 2
        for layer in range(hf.num_layers):
            kp, vp = m.kv_cache(layer)
            kb = l0.Buffer(device, kv_bytes, ptr=kp, owned=False).read(np.uint8)
            vb = l0.Buffer(device, kv_bytes, ptr=vp, owned=False).read(np.uint8)
            for o in (om, orr, o32):
                o.load_cache(layer, kb, vb)

        def both(tok, t):
            ref = om.step(tok, t)
            orc.set_device_rounding(True)
            try:
                rnd = orr.step(tok, t)
                orc.set_fast_projections(True)  # the same rounding with fp32 sums: the oracle's own spread
                r32 = o32.step(tok, t)
            finally:
                orc.set_device_rounding(False)
                orc.set_fast_projections(False)
            spread[t] = rel_err(r32[1], rnd[1])
            return ref, rnd

        spread = {}

        def check(lg, ref, rnd, t):
            e_ref, e_rnd = rel_err(lg, ref[1]), rel_err(lg, rnd[1])
            _flush(f"position {t}: {e_ref:.2e} of max|logit| against the fp32-activation oracle, {e_rnd:.2e} "
                   f"against the rounding one, whose fp32-sum form is {spread[t]:.2e} from it")
            assert e_rnd < TOL_ROUNDED, (t, e_rnd)
            assert e_rnd <= 3 * spread[t], (t, e_rnd, spread[t])
            assert e_ref < TOL_REF, (t, e_ref)
            g = int(np.argmax(lg))
            for (onext, olg), tol in ((ref, TOL_REF), (rnd, TOL_ROUNDED)):
                if g != onext:  # a tie-flip, not a bug: the oracle's own top-2 gap is within the bound
                    assert orc.top2_margin(olg) < 2 * tol * np.max(np.abs(olg)), (t, g, onext)
            return g, g != ref[0]

        _flush("oracles: last prompt token and teacher-forced steps")
        first, _ = check(last, *both(prompt[-1], rows), rows)
        tok, ids, flips = first, [], 0
        for t in range(BENCH_CTX, BENCH_CTX + steps):
            lg = m.compute_logits(tok, t)
            gnext, flipped = check(lg, *both(tok, t), t)
            flips += flipped
            ids.append(gnext)
            tok = gnext  # teacher-forced with the device's choice: all continue from the same sequence
        _flush(f"device greedy loop ({flips} tie-flips against the fp32-activation oracle)")
        m.prefill(prompt)
        looped = m.decode_greedy_device(first, steps)
        assert looped.tolist() == ids


@pytest.mark.parametrize("short,long", [(100, 300), (12, 20)], ids=["gemm-rows", "gemv-rows"])
def test_prefill_restarts_from_position_zero(device, short, long):
    hf = dataclasses.replace(LLAMA8B, num_layers=2)
    prompt = np.random.default_rng(76).integers(0, hf.vocab_size, long).tolist()
    with l0.LlmModel(device, hf, precision=l0.PRECISION_INT8, cache_dtype=l0.F16, max_seq_len=long + 8) as m:
        m.init_random(76, 0.02)
        first = m.prefill(prompt[:short])
        assert m.position == short
        m.prefill(prompt)
        assert m.position == long
        again = m.prefill(prompt[:short])
        assert m.position == short
        assert np.max(np.abs(first - again)) < 1e-4  # the reference's bound
        np.testing.assert_array_equal(first, again)  # fixed-order arithmetic: the same bits


def test_greedy_generation_is_deterministic_across_runs(device):
    hf = dataclasses.replace(LLAMA8B, num_layers=2)
    prompt = np.random.default_rng(180).integers(0, hf.vocab_size, 300).tolist()
    with l0.LlmModel(device, hf, precision=l0.PRECISION_INT8, cache_dtype=l0.F16, max_seq_len=340) as m:
        m.init_random(180, 0.02)
        runs = []
        for _ in range(2):
            first = int(np.argmax(m.prefill(prompt)))
            ids = m.decode_greedy_device(first, 16)
            runs.append((first, ids, m.last_logits(), m.position))
        assert runs[0][0] == runs[1][0]
        assert runs[0][1].tolist() == runs[1][1].tolist()
        assert runs[0][3] == runs[1][3] == len(prompt) + 16
        np.testing.assert_array_equal(runs[0][2], runs[1][2])
        # the same ids through LlmModel.GenerateGreedy (the prompt's last token picks the first one)
        assert m.generate_greedy(prompt, 17) == [runs[0][0]] + runs[0][1].tolist()

