"""Checkpoint ingest on the host: the safetensors reader and checkpoint (the cases of the
reference's SafetensorsReaderTests.cs / SafetensorsCheckpointTests.cs, restated), plus files
written by the `safetensors` package itself. No GPU needed."""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest
import torch
from safetensors.numpy import save_file as save_np
from safetensors.torch import save_file as save_torch

import l0llm_amd as l0

def write(path, tensors, metadata=None, header_override=None, pad=0):
    """tensors: list of (name, dtype, shape, raw bytes). Offsets are assigned in order."""
    header, blobs, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, dtype, shape, raw in tensors:
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    text = header_override if header_override is not None else json.dumps(header)
    hb = text.encode() + b" " * pad
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for b in blobs:
            f.write(b)
    return str(path)


def raw16(*bits):
    return struct.pack(f"<{len(bits)}H", *bits)


def f32(*vals):
    return struct.pack(f"<{len(vals)}f", *vals)


def test_f32_round_trips_shape_and_values(tmp_path):  # SafetensorsReaderTests.cs:9-22
    p = write(tmp_path / "a.safetensors", [("w", "F32", [2, 3], f32(1, -2.5, 3, 4, 5.25, -6))])
    with l0.SafetensorsCheckpoint(p) as ck:
        assert len(ck) == 1 and ck.info(0) == ("w", "F32", (2, 3))
        np.testing.assert_array_equal(ck.read_float32("w"), np.array([[1, -2.5, 3], [4, 5.25, -6]], np.float32))


def test_bf16_shifts_into_the_float_high_bits(tmp_path):  # :25-35
    p = write(tmp_path / "b.safetensors", [("t", "BF16", [5], raw16(0x3F80, 0xC000, 0x3FC0, 0x0000, 0x7F80))])
    with l0.SafetensorsCheckpoint(p) as ck:
        np.testing.assert_array_equal(ck.read_float32("t"), np.array([1, -2, 1.5, 0, np.inf], np.float32))


def test_f16_and_f64_convert(tmp_path):  # :38-60
    p = write(tmp_path / "h.safetensors", [("t", "F16", [6], raw16(0x3C00, 0xC000, 0x3800, 0x7BFF, 0x0001, 0x8400)),
                                           ("d", "F64", [2], struct.pack("<2d", 0.1, -2.5e-50))])
    with l0.SafetensorsCheckpoint(p) as ck:
        want = np.array([1, -2, 0.5, 65504, 2.0 ** -24, -(2.0 ** -14)], np.float32)  # incl. a subnormal
        np.testing.assert_array_equal(ck.read_float32("t"), want)
        np.testing.assert_array_equal(ck.read_float32("d"), np.array([0.1, -2.5e-50], np.float64).astype(np.float32))


def test_scalar_empty_and_multiple_tensors(tmp_path):  # :63-88, :284-294
    p = write(tmp_path / "m.safetensors", [("s", "F32", [], f32(7)), ("e", "F32", [0], b""), ("a", "F32", [1], f32(3)),
                                           ("b", "F32", [2], f32(4, 5))], metadata={"format": "pt"})
    with l0.SafetensorsCheckpoint(p) as ck:
        assert ck.names == ["a", "b", "e", "s"]
        assert ck.read_float32("s").shape == () and float(ck.read_float32("s")) == 7
        assert ck.read_float32("e").size == 0
        np.testing.assert_array_equal(ck.read_float32("b"), [4, 5])
        assert "a" in ck and "nope" not in ck


def test_large_bf16_crosses_chunk_boundaries(tmp_path):  # :91-110 (1 MiB chunks: 524288 BF16 each)
    n = 700_001
    bits = (0x3F80 + (np.arange(n) % 0x400)).astype(np.uint16)
    p = write(tmp_path / "big.safetensors", [("t", "BF16", [n], bits.tobytes())])
    with l0.SafetensorsCheckpoint(p) as ck:
        want = (bits.astype(np.uint32) << 16).view(np.float32)
        np.testing.assert_array_equal(ck.read_float32("t"), want)


def test_files_written_by_the_safetensors_package(tmp_path):
    rng = np.random.default_rng(0)
    a = rng.normal(size=(17, 33)).astype(np.float32)
    h = rng.normal(size=(5, 8)).astype(np.float16)
    save_np({"a": a, "h": h}, str(tmp_path / "np.safetensors"), metadata={"k": "v"})
    t = torch.from_numpy(rng.normal(size=(9, 16)).astype(np.float32)).to(torch.bfloat16)
    save_torch({"t": t}, str(tmp_path / "pt.safetensors"))
    with l0.SafetensorsCheckpoint(tmp_path / "np.safetensors") as ck:
        np.testing.assert_array_equal(ck.read_float32("a"), a)
        np.testing.assert_array_equal(ck.read_float32("h"), h.astype(np.float32))
    with l0.SafetensorsCheckpoint(tmp_path / "pt.safetensors") as ck:
        np.testing.assert_array_equal(ck.read_float32("t"), t.float().numpy())


def test_integer_tensor_cannot_be_read_as_float(tmp_path):  # :139-148
    p = write(tmp_path / "i.safetensors", [("ids", "I32", [2], struct.pack("<2i", 1, 2))])
    with l0.SafetensorsCheckpoint(p) as ck:
        assert ck.info(0) == ("ids", "I32", (2,))
        with pytest.raises(l0.UnsupportedError):
            ck.read_float32("ids")


def test_missing_tensor_and_wrong_destination(tmp_path):  # :162-183
    p = write(tmp_path / "a.safetensors", [("a", "F32", [2], f32(1, 2))])
    with l0.SafetensorsCheckpoint(p) as ck:
        with pytest.raises(KeyError):
            ck.read_float32("nope")
        dst = np.empty(3, np.float32)
        with pytest.raises(l0.InvalidArgumentError):
            l0._lib.check(l0.lib.l0h_safetensors_read_f32(ck.handle, b"a", dst.ctypes.data, 3))
        with pytest.raises(l0.InvalidArgumentError):
            l0._lib.check(l0.lib.l0h_safetensors_read_f32(ck.handle, b"nope", dst.ctypes.data, 3))


@pytest.mark.parametrize("case", ["unknown_dtype", "offsets_beyond", "byte_length", "overlap", "duplicate",
                                  "header_too_long", "short_file", "not_json", "negative_dim", "not_object",
                                  "missing_dtype", "bad_offsets"])
def test_malformed_files_are_rejected(tmp_path, case):  # :152-158, :198-281
    p = tmp_path / f"{case}.safetensors"
    err = l0.InvalidDataError
    if case == "unknown_dtype":
        write(p, [("t", "F8_E4M3", [1], b"\0")])
        err = l0.UnsupportedError
    elif case == "offsets_beyond":
        write(p, [], header_override=json.dumps({"t": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}))
    elif case == "byte_length":
        write(p, [("t", "F32", [3], f32(1, 2))])
    elif case == "overlap":
        hdr = {"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
               "b": {"dtype": "F32", "shape": [2], "data_offsets": [4, 12]}}
        write(p, [("x", "U8", [12], b"\0" * 12)], header_override=json.dumps(hdr))
    elif case == "duplicate":
        text = ('{"t": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}, '
                '"t": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}')
        write(p, [("x", "U8", [8], b"\0" * 8)], header_override=text)
    elif case == "header_too_long":
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", 1000) + b"{}")
    elif case == "short_file":
        with open(p, "wb") as f:
            f.write(b"\1\2\3")
    elif case == "not_json":
        write(p, [], header_override="{not json")
    elif case == "negative_dim":
        write(p, [], header_override=json.dumps({"t": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 0]}}))
    elif case == "not_object":
        write(p, [], header_override="[1, 2]")
    elif case == "missing_dtype":
        write(p, [], header_override=json.dumps({"t": {"shape": [0], "data_offsets": [0, 0]}}))
    else:
        write(p, [], header_override=json.dumps({"t": {"dtype": "F32", "shape": [0], "data_offsets": [0]}}))
    with pytest.raises(err):
        l0.SafetensorsCheckpoint(p)


def test_header_padding_is_accepted(tmp_path):  # headers are padded to 8 bytes by writers
    p = write(tmp_path / "pad.safetensors", [("a", "F32", [1], f32(2))], pad=5)
    with l0.SafetensorsCheckpoint(p) as ck:
        np.testing.assert_array_equal(ck.read_float32("a"), [2])


def _shard_dir(tmp_path, weight_map, shards):
    for name, tensors in shards.items():
        write(tmp_path / name, tensors)
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    return tmp_path


def test_directory_single_file_and_file_path(tmp_path):  # SafetensorsCheckpointTests.cs:9-32
    write(tmp_path / "model.safetensors", [("a", "F32", [1], f32(1))])
    with l0.SafetensorsCheckpoint(tmp_path) as ck:
        assert ck.names == ["a"]
    with l0.SafetensorsCheckpoint(tmp_path / "model.safetensors") as ck:
        assert ck.names == ["a"]


def test_sharded_checkpoint_merges_shards(tmp_path):  # :34-57
    d = _shard_dir(tmp_path, {"a": "s1.safetensors", "b": "s2.safetensors", "c": "s2.safetensors"},
                   {"s1.safetensors": [("a", "F32", [1], f32(1))],
                    "s2.safetensors": [("b", "F32", [1], f32(2)), ("c", "F32", [2], f32(3, 4))]})
    with l0.SafetensorsCheckpoint(d) as ck:
        assert ck.names == ["a", "b", "c"]
        np.testing.assert_array_equal(ck.read_float32("c"), [3, 4])


@pytest.mark.parametrize("case", ["wrong_shard", "traversal", "two_shards"])
def test_inconsistent_index_is_rejected(tmp_path, case):  # :59-93
    if case == "wrong_shard":
        d = _shard_dir(tmp_path, {"a": "s2.safetensors"},
                       {"s1.safetensors": [("a", "F32", [1], f32(1))], "s2.safetensors": [("b", "F32", [1], f32(2))]})
    elif case == "traversal":
        d = _shard_dir(tmp_path, {"a": "../s1.safetensors"}, {"s1.safetensors": [("a", "F32", [1], f32(1))]})
    else:
        d = _shard_dir(tmp_path, {"a": "s1.safetensors", "b": "s2.safetensors"},
                       {"s1.safetensors": [("a", "F32", [1], f32(1))],
                        "s2.safetensors": [("a", "F32", [1], f32(1)), ("b", "F32", [1], f32(2))]})
    with pytest.raises(l0.InvalidDataError):
        l0.SafetensorsCheckpoint(d)


def test_missing_path_and_empty_directory(tmp_path):  # :96-109
    with pytest.raises(l0.InvalidArgumentError):
        l0.SafetensorsCheckpoint(tmp_path)
    with pytest.raises(l0.InvalidArgumentError):
        l0.SafetensorsCheckpoint(tmp_path / "nope.safetensors")
