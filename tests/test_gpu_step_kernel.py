"""GPU parity of the persistent decode step (one launch per token, L0H_STEP_KERNEL=1) against the
oracle on the weights the device holds, and against the graph-replayed step of the same model:
the int8 Llama-3.1-8B layer shapes at a 2048-token context, the Qwen2.5-0.5B shape (7 q heads per kv
head, biases, tied head) and odd shapes (5 q heads on 1 kv head, an odd vocabulary). Logits within
2e-3 of max|logit|, greedy ids equal unless the oracle's top-2 gap is below the accumulation noise,
and the device-side greedy loop equal to the step-by-step loop."""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

import l0llm_amd as l0
from oracle import pyoracle as orc
from tests.helpers import rel_err
from tests.test_gpu_model import LLAMA8B, ODD, QWEN05, _as_cfg, exported_oracle

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skip(reason="the persistent decode step faulted the GPU (illegal address) on its first run and its "
                            "cause is not established; the library refuses L0H_STEP_KERNEL=1 until it is"),
]


def _model(device, hf, max_seq, seed, monkeypatch, persistent=True):
    if persistent:
        monkeypatch.setenv("L0H_STEP_KERNEL", "1")
    else:
        monkeypatch.delenv("L0H_STEP_KERNEL", raising=False)
    m = l0.LlmModel(device, hf, precision=l0.PRECISION_INT8, cache_dtype=l0.F16, max_seq_len=max_seq)
    m.init_random(seed, 0.02)
    assert m.step_path == ("persistent" if persistent else "graph")
    return m


@pytest.mark.parametrize("hf,steps", [(ODD, 6), (QWEN05, 5), (dataclasses.replace(LLAMA8B, num_layers=2), 4)],
                         ids=["odd-320-5q1kv-777", "qwen2.5-0.5b-4layers", "llama3.1-8b-2layers"])
def test_persistent_step_matches_oracle(device, monkeypatch, hf, steps):
    max_seq = 24
    with _model(device, hf, max_seq, 77, monkeypatch) as m:
        om = exported_oracle(m, _as_cfg(hf), orc.F16, max_seq)
        tok = int(np.random.default_rng(77).integers(0, hf.vocab_size))
        for t in range(steps):
            lg = m.compute_logits(tok, t)
            onext, olg = om.step(tok, t)
            assert np.all(np.isfinite(lg)), t
            assert rel_err(lg, olg) < 2e-3, (t, rel_err(lg, olg))
            gnext = int(np.argmax(lg))
            if gnext != onext:
                assert orc.top2_margin(olg) < 1e-3 * np.max(np.abs(olg)), (t, gnext, onext)
            tok = onext


def test_persistent_step_at_2048_context_matches_oracle_and_graph(device, monkeypatch):
    """Two layers at the 8B shapes with the timed step's cache length (2078 slots): 2047 prompt tokens
    prefilled, then 5 steps of the persistent kernel against the oracle seeded with the device's cache,
    and the device-side greedy loop of the persistent kernel against the graph step's."""
    hf = dataclasses.replace(LLAMA8B, num_layers=2)
    max_seq, ctx = 2078, 2048
    prompt = np.random.default_rng(599).integers(0, hf.vocab_size, ctx).tolist()
    with _model(device, hf, max_seq, 599, monkeypatch) as m:
        om = exported_oracle(m, _as_cfg(hf), orc.F16, max_seq)
        m.prefill(prompt[:-1])
        kv_bytes = (ctx - 1) * hf.num_key_value_heads * hf.head_dim * 2
        for layer in range(hf.num_layers):
            kp, vp = m.kv_cache(layer)
            om.load_cache(layer, l0.Buffer(device, kv_bytes, ptr=kp, owned=False).read(np.uint8),
                          l0.Buffer(device, kv_bytes, ptr=vp, owned=False).read(np.uint8))
        tok = prompt[-1]
        for t in range(ctx - 1, ctx + 4):
            lg = m.compute_logits(tok, t)
            onext, olg = om.step(tok, t)
            assert rel_err(lg, olg) < 2e-3, (t, rel_err(lg, olg))
            gnext = int(np.argmax(lg))
            if gnext != onext:
                assert orc.top2_margin(olg) < 1e-3 * np.max(np.abs(olg)), (t, gnext, onext)
            tok = onext
        # device-side greedy loop (launches back to back, the token fed back on the device) against the
        # same kernel driven token by token from the host: identical ids
        m.prefill(prompt)
        first = int(np.argmax(m.compute_logits(prompt[-1], ctx - 1)))
        got = m.decode_greedy_device(first, 16).tolist()
        m.prefill(prompt)
        want, tok = [], first
        for _ in range(16):
            tok = int(np.argmax(m.decode(tok)))
            want.append(tok)
        assert got == want
    # the graph step of the same weights picks the same first token (or sits on a near-tie)
    with _model(device, hf, max_seq, 599, monkeypatch, persistent=False) as g:
        lg = g.prefill(prompt)
        if int(np.argmax(lg)) != first:
            assert orc.top2_margin(lg) < 1e-3 * np.max(np.abs(lg))


def test_persistent_generate_greedy_matches_step_loop(device, monkeypatch):
    prompt = np.random.default_rng(3).integers(0, QWEN05.vocab_size, 9).tolist()
    with _model(device, QWEN05, 40, 3, monkeypatch) as m:
        gen = m.generate_greedy(prompt, 12)
        m.reset_sequence()
        lg = m.prefill(prompt)
        seq = [int(np.argmax(lg))]
        for _ in range(11):
            seq.append(int(np.argmax(m.decode(seq[-1]))))
        assert gen == seq
