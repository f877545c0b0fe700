"""Builds the host emulation of the persistent decode step kernel (l0llm_amd/csrc/step_kernel.hip)
for the CPU test: the kernel's own source, with the device-only pieces it includes from
gemv_kernel.h, compiled by clang++ against the emulation headers in include/ with
AddressSanitizer. Three textual edits are made to the copy: the dynamic LDS array becomes the
emulated block's buffer, and two wave-synchronisation points are inserted where the kernel relies
on a wave executing in lockstep (LDS written by some lanes and read by others in stage_row; every
lane's stores issued before lane 0 arrives at a grid barrier)."""
from __future__ import annotations

import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(os.path.dirname(HERE)), "l0llm_amd", "csrc")


def clang() -> str | None:
    for c in ("/opt/rocm/llvm/bin/clang++", shutil.which("clang++")):
        if c and os.path.exists(c):
            return c
    return None


def generate(out_dir: str) -> str:
    os.makedirs(out_dir, exist_ok=True)
    lines = open(os.path.join(CSRC, "gemv_kernel.h")).read().split("\n")
    cut = next(i for i, l in enumerate(lines) if l.startswith("// XH (int8 weights, one fp16 activation row"))
    head = "\n".join(lines[:cut])
    # the fp16-row helpers (v_perm_b32 / v_dot2 builtins) are not used by the step kernel
    xh0 = head.index("typedef _Float16 half2_t")
    xh1 = head.index("// The 16 bytes of an activation chunk as fp32")
    head = head[:xh0] + head[xh1:]
    head = head.replace('asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");', "")
    head = head.replace('asm volatile("" ::: "memory");', "")
    head = head.replace('#include "dpp.h"', f'#include "{CSRC}/dpp.h"').replace('#include "kernels.h"', f'#include "{CSRC}/kernels.h"')
    with open(os.path.join(out_dir, "gemv_kernel.h"), "w") as f:
        f.write(head + "\n}  // namespace\n}  // namespace l0h\n")
    s = open(os.path.join(CSRC, "step_kernel.hip")).read()
    edits = [
        ("extern __shared__ float4 step_smem[];", "float4* step_smem = static_cast<float4*>(emu::t_block->smem);"),
        ("    if constexpr (WT == L0H_I8PC) {\n        for (int c = lane; c < padded / 16; c += 64) {",
         "    emu::wave_sync();\n    if constexpr (WT == L0H_I8PC) {\n        for (int c = lane; c < padded / 16; c += 64) {"),
        ("    ctl.nbar++;\n", "    emu::wave_sync();\n    ctl.nbar++;\n"),
    ]
    for old, new in edits:
        if s.count(old) != 1:
            raise RuntimeError(f"step_kernel.hip no longer has exactly one {old[:40]!r}")
        s = s.replace(old, new)
    src = os.path.join(out_dir, "step_emu.cpp")
    with open(src, "w") as f:
        f.write(s + f'\n#include "{HERE}/driver.inc"\n')
    return src


def build(out_dir: str) -> str:
    """Generates and compiles the emulation; returns the executable's path."""
    cxx = clang()
    if cxx is None:
        raise FileNotFoundError("clang++ not found")
    src = generate(out_dir)
    exe = os.path.join(out_dir, "step_emu")
    cmd = [cxx, "-std=c++20", "-O1", "-g", "-DL0H_WITH_STEP_KERNEL", "-fsanitize=address", "-fno-omit-frame-pointer",
           "-I", os.path.join(HERE, "include"), "-I", out_dir, "-I", CSRC, src,
           os.path.join(CSRC, "errors.cpp"), "-o", exe, "-lpthread"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe
