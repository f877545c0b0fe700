"""Builds libl0hip.so (gfx950) in-tree with hipcc: one object per source, compiled in
parallel, linked into l0llm_amd/libl0hip.so. Run as `python l0llm_amd/build.py` (this file does
not import the package, whose import loads the library being rebuilt)."""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libl0hip.so"
BUILD_DIR = PKG / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed-fp32 ops stay off: hipcc only emits them from ordinary float code, and some of their
# forms have been seen to give wrong results on this hardware.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall"]
# Per-source additions. attention.hip: MFMA accumulators in ordinary VGPRs rather than AGPRs, so the
# prefill kernel's per-tile softmax rescale of its output tile is a multiply per value, not a copy
# out of the accumulator registers, a multiply and a copy back (the 8B 2048-token prefill 0.0368-
# 0.0369 -> 0.0364 s, two interleaved pairs on one box).
FILE_FLAGS = {
    "attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    if src.suffix == ".hip":
        cmd = [HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    else:
        cmd = ["g++", *CXX_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found: the library is built for gfx950 with ROCm's hipcc")
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(p for p in CSRC.iterdir() if p.suffix in (".hip", ".cpp"))
    jobs = jobs or min(len(sources), max(1, min(16, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs), "-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(sources)} sources")
    return OUT


if __name__ == "__main__":
    build()
