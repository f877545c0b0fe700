"""CPU tests of libl0hip: it loads, exports every entry point include/l0hip.h declares, and its
host-side helpers (quantizer, RoPE table, transpose, half-range check) agree with the oracle.
No compute call touches a GPU here."""
from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest

import l0llm_amd as l0
from l0llm_amd import _lib
from oracle import pyoracle as orc
from tests.helpers import GOLDEN


def test_every_declared_entry_point_is_exported():
    decl = l0.declared_functions()
    text = _lib.HEADER.read_text()
    names = set(re.findall(r"\b(l0h_\w+)\(", re.sub(r"/\*.*?\*/", "", text, flags=re.S)))
    assert set(decl) == names
    assert len(decl) >= 60
    for name in decl:
        assert hasattr(l0.lib, name), name


def test_header_and_oracle_share_dtype_codes():
    assert (l0.F32, l0.F16, l0.BF16, l0.I8PC) == (orc.F32, orc.F16, orc.BF16, orc.I8PC)


def test_static_support_queries():
    assert l0.lib.l0h_gemv_supports(4864) == 1 and l0.lib.l0h_gemv_supports(30) == 0
    assert l0.lib.l0h_gemv_q8_supports(64, 96) == 1
    assert l0.lib.l0h_gemv_q8_supports(30, 64) == 0 and l0.lib.l0h_gemv_q8_supports(64, 50) == 0
    assert l0.lib.l0h_gemv_max_rows() == 8


def test_quantizer_matches_oracle_bitwise():
    rng = np.random.default_rng(20)
    w = rng.normal(0, 0.02, (300, 896)).astype(np.float32)
    w[7] = 0
    w[8, 3] = 1e-8
    q, s = l0.quantize_i8pc(w)
    oq, os_ = orc.quantize_i8pc(w)
    np.testing.assert_array_equal(q, oq)
    np.testing.assert_array_equal(s.view(np.uint16), os_)


def test_quantizer_scale_stays_finite_and_nonzero():
    """Rows whose max|w| / 127 rounds to 0 in fp16 keep the smallest subnormal scale 2^-24, rows whose
    scale would overflow keep 65504, all-zero rows keep 0; library and oracle agree bit for bit, and
    every non-zero row dequantizes to finite values with |q * s - w| bounded."""
    rng = np.random.default_rng(21)
    w = rng.normal(0, 1, (6, 64)).astype(np.float32)
    w[0] *= 1e-8          # max|w| / 127 below half the smallest subnormal
    w[1] *= 1e-6          # subnormal scale
    w[2] *= 1e7           # max|w| / 127 above 65504
    w[3] = 0.0            # all-zero row
    w[4, :] = 0.0
    w[4, 5] = 3e-7        # one tiny value
    q, s = l0.quantize_i8pc(w)
    oq, os_ = orc.quantize_i8pc(w)
    np.testing.assert_array_equal(q, oq)
    np.testing.assert_array_equal(s.view(np.uint16), os_)
    bits = s.view(np.uint16)
    assert bits[0] == 0x0001 and bits[4] == 0x0001  # 2^-24
    assert bits[2] == 0x7BFF                        # 65504
    assert bits[3] == 0 and not q[3].any()
    deq = q.astype(np.float64) * s.astype(np.float64)[:, None]
    assert np.all(np.isfinite(deq))
    for r in (1, 5):  # normal and subnormal scales: rounding error at most half a step
        assert np.max(np.abs(deq[r] - w[r])) <= 0.5 * float(s[r]) * 1.0001
    assert np.all(np.abs(q) <= 127)


def test_rope_frequencies_match_oracle_and_golden():
    import json
    cases = json.loads((GOLDEN / "rope.golden.json").read_text())["cases"]
    for name, c in cases.items():
        sc = c["scaling"] or {}
        rs = l0.RopeScaling(type=sc.get("rope_type", "default"), factor=sc.get("factor", 1.0),
                            original_max_position_embeddings=sc.get("original_max_position_embeddings"),
                            beta_fast=sc.get("beta_fast", 32.0), beta_slow=sc.get("beta_slow", 1.0),
                            attention_factor=sc.get("attention_factor"))
        inv, att = l0.rope_frequencies(c["head_dim"], c["theta"], c["max_position_embeddings"], rs)
        exp = np.array(c["inv_freq"])
        assert np.all(np.abs(exp - inv) <= 1e-5 * np.abs(exp) + 1e-12), name
        assert abs(att - c["attention_factor"]) < 1e-5, name
        oinv, oatt = orc.rope_frequencies(c["head_dim"], c["theta"], c["max_position_embeddings"],
                                          sc.get("rope_type", "default"), factor=sc.get("factor", 1.0),
                                          original_max=sc.get("original_max_position_embeddings", 0) or 0,
                                          beta_fast=sc.get("beta_fast", 32.0), beta_slow=sc.get("beta_slow", 1.0),
                                          attention_factor=sc.get("attention_factor"))
        np.testing.assert_array_equal(inv, oinv)
        assert att == oatt
    with pytest.raises(l0.UnsupportedError):
        l0.rope_frequencies(16, 10000, 2048, l0.RopeScaling(type="longrope"))
    with pytest.raises(l0.InvalidArgumentError):
        l0.rope_frequencies(15, 10000, 2048)


def test_llama3_table_known_answer():
    import json
    d = json.loads((GOLDEN / "llama3_table.json").read_text())
    p = d["params"]
    inv, att = l0.rope_frequencies(p["head_dim"], p["theta"], p["max_position_embeddings"],
                                   l0.RopeScaling(type="llama3", factor=p["factor"],
                                                  original_max_position_embeddings=p["original_max_position_embeddings"],
                                                  low_freq_factor=p["low_freq_factor"],
                                                  high_freq_factor=p["high_freq_factor"]))
    assert att == 1.0
    assert np.all(np.abs(inv - np.array(d["expected"])) / np.array(d["expected"]) <= 1e-5)


def test_transpose_and_fits_in_half():
    src = np.arange(33 * 65, dtype=np.float32)
    np.testing.assert_array_equal(l0.transpose(src, 33, 65), orc.transpose(src, 33, 65))
    with pytest.raises(l0.InvalidArgumentError):
        l0.transpose(np.zeros(5, np.float32), 2, 3)  # LlmLayerWeightsTests.cs:51
    assert l0.fits_in_half(np.array([0, -1, 64000, 1e-9], np.float32))
    assert not l0.fits_in_half(np.array([1, 70000], np.float32))
    assert not l0.fits_in_half(np.array([1, np.nan], np.float32))


def test_errors_carry_status_and_message_without_a_device():
    # Null arguments are rejected before any device is touched (ArgumentNullException).
    with pytest.raises(l0.InvalidArgumentError) as e:
        _lib.check(l0.lib.l0h_device_open(0, None))
    assert e.value.code == _lib.ERR_INVALID_ARG and "null" in str(e.value)
    assert l0.lib.l0h_quantize_i8pc(None, 4, 4, None, None) == _lib.ERR_INVALID_ARG
    assert l0.lib.l0h_last_error().decode() == "null buffer"


def test_runtime_reports_no_device_here():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; this checks the CPU-only path")
    assert l0.runtime_is_available() is False
    h = ctypes.c_void_p()
    assert l0.lib.l0h_device_open(0, ctypes.byref(h)) == _lib.ERR_DEVICE
    assert h.value is None
