"""l0h_attention_decode_noalloc (split partials in the library's static scratch, no allocation)
against l0h_attention_decode on the same inputs, through the C ABI: two calls in a row, the second
smaller, each bit for bit equal to the allocating entry point (same kernels, same split count);
and a shape whose partials exceed the static scratch is refused before any launch."""
from __future__ import annotations

import numpy as np
import pytest

import l0llm_amd as l0

pytestmark = pytest.mark.gpu


def _case(device, suite, rng, batch, nh, nkv, hd, seq, max_seq):
    kv = nkv * hd
    k = rng.standard_normal((batch, max_seq, kv), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((batch, max_seq, kv), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((batch, nh * hd), dtype=np.float32).astype(np.float16)
    kb, vb, qb = (device.alloc_shared(a.view(np.uint16)) for a in (k, v, q))
    ref, got = device.alloc(batch * nh * hd * 4), device.alloc(batch * nh * hd * 4)
    ref.zero()
    got.zero()
    suite.attention_decode(qb, l0.F16, kb, vb, l0.F16, ref, l0.F32, batch, hd, nh, nkv, seq, max_seq)
    suite.attention_decode_noalloc(qb, l0.F16, kb, vb, l0.F16, got, l0.F32, batch, hd, nh, nkv, seq, max_seq)
    want = ref.read(np.float32)
    assert np.all(np.isfinite(want))
    np.testing.assert_array_equal(got.read(np.float32), want)
    for b in (kb, vb, qb, ref, got):
        b.free()


def test_noalloc_attention_matches_allocating_entry_point(device, suite):
    rng = np.random.default_rng(7)
    # batch 8 x 4096 positions (4 splits), then a smaller call: batch 1 x 1000 of 1100 slots (8 splits)
    _case(device, suite, rng, 8, 32, 8, 128, 4096, 4096)
    _case(device, suite, rng, 1, 32, 8, 128, 1000, 1100)
    # a third, smaller still, with 4 q heads per kv head at head_dim 64 (Qwen2.5-0.5B-like)
    _case(device, suite, rng, 1, 14, 2, 64, 300, 320)


def test_noalloc_attention_refuses_shapes_beyond_its_scratch(device, suite):
    """73 x 7 kv heads with 8 q heads each at 4096 slots: two splits per (batch, kv head), 1022 partials
    of 1040 floats = 4,251,520 bytes > 4 MiB. Refused with InvalidArgument; the caches are real
    allocations of the full shape, so nothing could read outside them even if a launch happened."""
    batch, nh, nkv, hd, max_seq = 73, 56, 7, 128, 4096
    kb = device.alloc(batch * max_seq * nkv * hd * 2)
    vb = device.alloc(batch * max_seq * nkv * hd * 2)
    qb = device.alloc(batch * nh * hd * 2)
    ob = device.alloc(batch * nh * hd * 4)
    with pytest.raises(l0.InvalidArgumentError):
        suite.attention_decode_noalloc(qb, l0.F16, kb, vb, l0.F16, ob, l0.F32, batch, hd, nh, nkv, max_seq, max_seq)
    for b in (kb, vb, qb, ob):
        b.free()
