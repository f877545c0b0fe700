"""The persistent decode step kernel (l0llm_amd/csrc/step_kernel.hip) run on the CPU: its own
source under a host emulation of the wave builtins (tests/step_emu), with AddressSanitizer on
exact-size buffers (the LDS tile included), against a float64 restatement of the decode step
(embedding, RMSNorm, int8 q|k|v + bias + RoPE + fp16 cache row, GQA attention, O, SwiGLU, down,
final norm, lm_head, greedy pick). The kernel is disabled in the library; this pins its indexing
and arithmetic independently of the GPU. Shapes: two layers of 320-wide rows with 5 q heads on 1
kv head and an odd vocabulary (the GPU test's odd shape), head_dim 128 with 4 q heads per kv
head at position 257 of 300, and one layer of the Qwen2.5-0.5B widths (7 q heads per kv head,
biases) with a 4000-token vocabulary, and one 320-wide layer at position 0; grids of 3 and 8 blocks
(512 threads each, one per lane)."""
from __future__ import annotations

import os
import subprocess

import pytest

from tests.step_emu import make_emu


@pytest.fixture(scope="module")
def step_emu(tmp_path_factory):
    if make_emu.clang() is None:
        pytest.skip("clang++ is not available")
    return make_emu.build(str(tmp_path_factory.mktemp("step_emu")))


def _run(exe, *args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0")
    r = subprocess.run([exe, *map(str, args)], capture_output=True, text=True, timeout=600, env=env)
    return r.returncode, r.stdout + r.stderr


def test_emulated_cross_lane_primitives(step_emu):
    """wave_sum, group_sum, slot_reduce, row_lane and lane_group_sum under the emulation's DPP and
    permlane semantics give the sums / maxima over the lanes they name."""
    rc, out = _run(step_emu, -1)
    assert rc == 0 and "0 mismatches" in out, out


@pytest.mark.parametrize("cfg", [0, 1, 2, 3], ids=["odd-2layers-5q1kv", "hd128-gqa4-pos257", "qwen-widths-1layer",
                                                  "odd-1layer-pos0"])
@pytest.mark.parametrize("blocks", [3, 8])
def test_persistent_step_emulated_matches_float64(step_emu, cfg, blocks):
    rc, out = _run(step_emu, cfg, blocks)
    assert rc == 0 and "-> OK" in out and "AddressSanitizer" not in out, out
