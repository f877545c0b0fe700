"""The host-side C++ of libl0hip (errors.cpp, host.cpp, safetensors.cpp) built with g++'s address
and undefined-behaviour sanitizers and driven over well-formed and malformed checkpoints (the
header parser reads untrusted files) and edge-case quantizer / transpose / RoPE inputs. A
sanitizer report aborts the driver, so every run must exit 0 with the expected statuses. CPU only."""
from __future__ import annotations

import json
import os
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "l0llm_amd" / "csrc"
INVALID_DATA, UNSUPPORTED, INVALID_ARG = -4, -2, -1


@pytest.fixture(scope="module")
def driver(tmp_path_factory) -> Path:
    if shutil.which("g++") is None:
        pytest.skip("g++ is not installed")
    out = tmp_path_factory.mktemp("asan") / "host_sanitize_driver"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", str(ROOT / "tests" / "host_sanitize_driver.cpp"), str(CSRC / "errors.cpp"),
           str(CSRC / "host.cpp"), str(CSRC / "safetensors.cpp"), "-o", str(out), "-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    return out


def run(driver: Path, *args) -> list[str]:
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    res = subprocess.run([str(driver), *map(str, args)], capture_output=True, text=True, env=env, timeout=120)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    return res.stdout.splitlines()


def write(path: Path, header, data: bytes = b"", length: int | None = None) -> Path:
    raw = header if isinstance(header, bytes) else json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(raw) if length is None else length) + raw + data)
    return path


def open_status(lines: list[str]) -> int:
    return int(lines[0].split()[1])


def test_well_formed_checkpoints_read_cleanly(driver, tmp_path):
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    b = np.linspace(-2, 2, 6).astype(np.float16)
    c = np.array([1.5, -2.25], dtype=np.float64)
    data = a.tobytes() + b.tobytes() + c.tobytes()
    hdr = {"__metadata__": {"format": "pt"},
           "a": {"dtype": "F32", "shape": [3, 4], "data_offsets": [0, 48]},
           "b": {"dtype": "F16", "shape": [6], "data_offsets": [48, 60]},
           "c": {"dtype": "F64", "shape": [2], "data_offsets": [60, 76]},
           "e": {"dtype": "I32", "shape": [0], "data_offsets": [76, 76]},
           "s": {"dtype": "BF16", "shape": [], "data_offsets": [76, 78]}}
    lines = run(driver, "st", write(tmp_path / "ok.safetensors", hdr, data + b"\x80\x3f"))
    assert open_status(lines) == 0
    sums = {ln.split()[1]: ln for ln in lines if ln.startswith("tensor ")}
    assert "read 0 sum 66" in sums["a"] and "read 0 sum 1" in sums["s"]
    assert "read -2" in sums["e"]  # I32 does not convert to fp32
    assert any(ln.startswith("missing -1") for ln in lines)
    # a sharded directory with its index
    d = tmp_path / "sharded"
    d.mkdir()
    write(d / "s1.safetensors", {"x": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, b"\0" * 8)
    write(d / "s2.safetensors", {"y": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}, b"\0" * 4)
    (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"x": "s1.safetensors",
                                                                               "y": "s2.safetensors"}}))
    assert open_status(run(driver, "st", d)) == 0


MALFORMED = {
    "short_file": (b"{}", None, b"", "raw5"),
    "length_beyond_file": ({"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}, 1 << 20, b"\0" * 4, None),
    "length_over_limit": (b"{}", (1 << 63) + 5, b"", None),
    "bad_json": (b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]', None, b"", None),
    "not_object": (b"[1, 2, 3]", None, b"", None),
    "entry_not_object": ({"a": 5}, None, b"", None),
    "no_dtype": ({"a": {"shape": [1], "data_offsets": [0, 4]}}, None, b"\0" * 4, None),
    "negative_dim": ({"a": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}, None, b"\0" * 4, None),
    "fraction_dim": ({"a": {"dtype": "F32", "shape": [1.5], "data_offsets": [0, 4]}}, None, b"\0" * 4, None),
    "overflowing_shape": ({"a": {"dtype": "F64", "shape": [1 << 31, 1 << 31, 4], "data_offsets": [0, 8]}}, None,
                          b"\0" * 8, None),
    "offsets_outside": ({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, None, b"\0" * 8, None),
    "offsets_reversed": ({"a": {"dtype": "F32", "shape": [0], "data_offsets": [8, 4]}}, None, b"\0" * 8, None),
    "size_mismatch": ({"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, None, b"\0" * 8, None),
    "duplicate": (b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}, '
                  b'"a": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}', None, b"\0" * 8, None),
    "overlap": ({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
                 "b": {"dtype": "F32", "shape": [2], "data_offsets": [4, 12]}}, None, b"\0" * 12, None),
    "deep_nesting": (b"[" * 100000 + b"]" * 100000, None, b"", None),
    "bad_escape": (b'{"a\\u12": 1}', None, b"", None),
}


@pytest.mark.parametrize("case", sorted(MALFORMED))
def test_malformed_headers_are_refused_cleanly(driver, tmp_path, case):
    header, length, data, special = MALFORMED[case]
    path = tmp_path / f"{case}.safetensors"
    if special == "raw5":
        path.write_bytes(b"\x01\x02\x03\x04\x05")
    else:
        write(path, header, data, length)
    assert open_status(run(driver, "st", path)) == INVALID_DATA


def test_unknown_dtype_and_inconsistent_index(driver, tmp_path):
    p = write(tmp_path / "u.safetensors", {"a": {"dtype": "F8_E4M3", "shape": [1], "data_offsets": [0, 1]}}, b"\0")
    assert open_status(run(driver, "st", p)) == UNSUPPORTED
    d = tmp_path / "idx"
    d.mkdir()
    write(d / "s1.safetensors", {"x": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}, b"\0" * 4)
    (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"x": "s1.safetensors",
                                                                               "y": "s1.safetensors"}}))
    assert open_status(run(driver, "st", d)) == INVALID_DATA
    (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"x": "../s1.safetensors"}}))
    assert open_status(run(driver, "st", d)) == INVALID_DATA
    e = tmp_path / "empty_dir"
    e.mkdir()
    assert open_status(run(driver, "st", e)) == INVALID_ARG


def test_host_helpers_on_edge_inputs(driver):
    lines = run(driver, "host")
    quant = [ln for ln in lines if ln.startswith("quantize")]
    assert len(quant) == 3 and all(" 0 maxq " in ln for ln in quant)
    for ln in quant:
        s0, s1, s2 = (int(ln.split()[i]) for i in (6, 8, 10))
        assert s0 == 0 and s1 != 0 and s2 == 0x7BFF  # zero row, tiny row (non-zero scale), huge row
    assert all(ln.split()[-1] == "1" for ln in lines if ln.startswith("transpose ") and "x" in ln.split()[1])
    assert sum(ln.startswith("rope type") for ln in lines) == 12
