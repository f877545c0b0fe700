"""Python mirror of the reference's operator interface over libl0hip's C ABI.

Names follow the reference: ``Device`` (ComputeDevice + LevelZeroRuntime), ``Buffer``
(SharedBuffer<T>), ``LlmKernelSuite`` (LevelZero.Kernels.LlmKernelSuite members),
``LlmMatrix`` (LlmMatrix.cs), ``LlmModel`` (LlmModel.cs). Buffers are device memory moved
with explicit ``write``/``read``; numpy arrays are the host side. Every call goes to the HIP
library; nothing here computes on the CPU."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, fields

import numpy as np

from . import _lib
from ._lib import BF16, F16, F32, I8PC, ModelConfig, check, lib

_NP = {F32: np.float32, F16: np.float16, BF16: np.uint16, I8PC: np.int8}


def _ptr(x) -> ctypes.c_void_p | None:
    if x is None:
        return None
    if isinstance(x, Buffer):
        return ctypes.c_void_p(x.ptr)
    if isinstance(x, int):
        return ctypes.c_void_p(x)
    raise TypeError(f"expected a device Buffer, got {type(x).__name__}")


def runtime_is_available() -> bool:
    """LevelZeroRuntime.IsAvailable: a gfx950 device is present."""
    return bool(lib.l0h_runtime_is_available())


class Buffer:
    """Device allocation (SharedBuffer<T>). ``ptr`` is the device address."""

    def __init__(self, device: "Device", nbytes: int, ptr: int | None = None, owned: bool = True):
        self.device = device
        self.nbytes = int(nbytes)
        self.owned = owned
        if ptr is None:
            p = ctypes.c_void_p()
            check(lib.l0h_alloc(device.handle, ctypes.c_size_t(self.nbytes), ctypes.byref(p)))
            ptr = p.value
        self.ptr = int(ptr)

    def write(self, array: np.ndarray, offset_bytes: int = 0) -> None:
        a = np.ascontiguousarray(array)
        if offset_bytes + a.nbytes > self.nbytes:
            raise ValueError(f"write of {a.nbytes} bytes at {offset_bytes} exceeds the {self.nbytes}-byte buffer")
        check(lib.l0h_write(self.device.handle, ctypes.c_void_p(self.ptr), offset_bytes,
                            a.ctypes.data_as(ctypes.c_void_p), a.nbytes))

    def read(self, dtype=np.float32, count: int | None = None, offset_bytes: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset_bytes) // dt.itemsize
        out = np.empty(count, dtype=dt)
        if offset_bytes + out.nbytes > self.nbytes:
            raise ValueError("read past the end of the buffer")
        check(lib.l0h_read(self.device.handle, ctypes.c_void_p(self.ptr), offset_bytes,
                           out.ctypes.data_as(ctypes.c_void_p), out.nbytes))
        return out

    def zero(self) -> None:
        check(lib.l0h_fill_zero(self.device.handle, ctypes.c_void_p(self.ptr), self.nbytes))

    def free(self) -> None:
        if self.owned and self.ptr and self.device.handle:
            check(lib.l0h_free(self.device.handle, ctypes.c_void_p(self.ptr)))
        self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()


class Device:
    """ComputeDevice: one HIP device with its stream (LevelZeroRuntime.GetDevice)."""

    def __init__(self, ordinal: int = 0):
        h = ctypes.c_void_p()
        check(lib.l0h_device_open(ordinal, ctypes.byref(h)))
        self.handle = h
        name = ctypes.create_string_buffer(256)
        cus = ctypes.c_int()
        check(lib.l0h_device_info(h, name, 256, ctypes.byref(cus)))
        self.name = name.value.decode()
        self.compute_units = cus.value

    @staticmethod
    def count() -> int:
        n = ctypes.c_int()
        check(lib.l0h_device_count(ctypes.byref(n)))
        return n.value

    def alloc(self, nbytes: int) -> Buffer:
        return Buffer(self, nbytes)

    def alloc_shared(self, data: np.ndarray) -> Buffer:
        """AllocShared(data): a buffer holding a copy of ``data``."""
        a = np.ascontiguousarray(data)
        b = Buffer(self, max(a.nbytes, 1))
        if a.nbytes:
            b.write(a)
        return b

    def begin_recording(self) -> None:
        check(lib.l0h_begin_recording(self.handle))

    def end_recording(self) -> None:
        check(lib.l0h_end_recording(self.handle))

    def abort_recording(self) -> None:
        check(lib.l0h_abort_recording(self.handle))

    def replay_recording(self, count: int = 1) -> float:
        """Launches the last recorded command list `count` more times back to back; returns the
        mean device time of one replay in milliseconds."""
        ms = ctypes.c_float()
        check(lib.l0h_replay_recording(self.handle, count, ctypes.byref(ms)))
        return ms.value

    @property
    def recording_launches(self) -> int:
        """Kernel launches (graph nodes) of the last recording."""
        n = ctypes.c_int()
        check(lib.l0h_recording_launches(self.handle, ctypes.byref(n)))
        return n.value

    @property
    def is_recording(self) -> bool:
        v = ctypes.c_int()
        check(lib.l0h_is_recording(self.handle, ctypes.byref(v)))
        return bool(v.value)

    def read_bandwidth(self, nbytes: int = 2 << 30, reps: int = 10) -> float:
        """HBM read rate (GB/s) of a streaming-read kernel over a fresh `nbytes` buffer."""
        g = ctypes.c_double()
        check(lib.l0h_device_read_bandwidth(self.handle, ctypes.c_size_t(nbytes), reps, ctypes.byref(g)))
        return g.value

    def synchronize(self) -> None:
        check(lib.l0h_synchronize(self.handle))

    def close(self) -> None:
        if self.handle:
            check(lib.l0h_device_close(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class LlmKernelSuite:
    """The LevelZero.Kernels.LlmKernelSuite members the reference calls, reference argument order."""

    def __init__(self, device: Device):
        self.device = device

    # Gemv.Execute / ExecuteRows (LlmMatrix.cs:134-165): W is [K, N], F32 or F16
    def gemv_execute(self, out_dim, in_dim, x, w, y, w_dtype=F16):
        check(lib.l0h_gemv_execute(self.device.handle, out_dim, in_dim, _ptr(x), _ptr(w), w_dtype, _ptr(y)))

    def gemv_execute_rows(self, rows, out_dim, in_dim, x, w, y, w_dtype=F16):
        check(lib.l0h_gemv_execute_rows(self.device.handle, rows, out_dim, in_dim, _ptr(x), _ptr(w), w_dtype, _ptr(y)))

    def gemm_execute(self, m, n, k, x, w, y):
        check(lib.l0h_gemm_execute(self.device.handle, m, n, k, _ptr(x), _ptr(w), _ptr(y)))

    # GemvQ8 in the weight-only int8 format (LlmMatrix.cs:29-31, :128-130, :155-157, :201, :235-251)
    @staticmethod
    def q8_group_size() -> int:
        """LlmGemvQ8Kernel.GroupSize."""
        return lib.l0h_gemv_q8_group_size()

    def ensure_q8_scratch(self, rows: int, cols: int) -> None:
        """LlmKernelSuite.EnsureQ8Scratch(device, rows, cols) (LlmModel.cs:139-144)."""
        check(lib.l0h_q8_scratch_ensure(self.device.handle, rows, cols))

    @property
    def q8_scratch(self) -> "Buffer | None":
        """LlmKernelSuite.Q8Scratch; its row_capacity attribute is RowCapacity."""
        ptr, rows, cols = ctypes.c_void_p(), ctypes.c_int(), ctypes.c_int()
        check(lib.l0h_q8_scratch(self.device.handle, ctypes.byref(ptr), ctypes.byref(rows), ctypes.byref(cols)))
        if not ptr.value:
            return None
        buf = Buffer(self.device, rows.value * cols.value * 4, ptr=ptr.value, owned=False)
        buf.row_capacity = rows.value
        buf.cols = cols.value
        return buf

    def gemv_q8_quantize(self, rows, in_dim, x, scratch):
        check(lib.l0h_gemv_q8_quantize(self.device.handle, rows, in_dim, _ptr(x), _ptr(scratch)))

    def gemv_q8_execute(self, out_dim, in_dim, scratch, words, scales, y):
        check(lib.l0h_gemv_q8_execute(self.device.handle, out_dim, in_dim, _ptr(scratch), _ptr(words), _ptr(scales),
                                      _ptr(y)))

    def gemv_q8_execute_rows(self, rows, out_dim, in_dim, scratch, words, scales, y):
        check(lib.l0h_gemv_q8_execute_rows(self.device.handle, rows, out_dim, in_dim, _ptr(scratch), _ptr(words),
                                           _ptr(scales), _ptr(y)))

    def attention_reserve(self, batch, n_heads, n_kv, head_dim, max_seq_len):
        check(lib.l0h_attention_reserve(self.device.handle, batch, n_heads, n_kv, head_dim, max_seq_len))

    def rmsnorm_execute(self, x, residual, w, out, eps, n, rows, add_residual):
        check(lib.l0h_rmsnorm_execute(self.device.handle, _ptr(x), _ptr(residual), _ptr(w), _ptr(out),
                                      ctypes.c_float(eps), n, rows, int(add_residual)))

    def swiglu_execute(self, gate, up, n):
        check(lib.l0h_swiglu_execute(self.device.handle, _ptr(gate), _ptr(up), n))

    def add_execute(self, a, b, n):
        check(lib.l0h_add_execute(self.device.handle, _ptr(a), _ptr(b), n))

    def bias_add_execute(self, x, bias, n, rows):
        check(lib.l0h_bias_add_execute(self.device.handle, _ptr(x), _ptr(bias), n, rows))

    def rope_execute(self, q, k, positions, head_dim, n_heads, n_kv, theta, tokens):
        check(lib.l0h_rope_execute(self.device.handle, _ptr(q), _ptr(k), _ptr(positions), head_dim, n_heads, n_kv,
                                   ctypes.c_float(theta), tokens))

    def rope_execute_with_frequencies(self, q, k, positions, inv_freq, head_dim, n_heads, n_kv, attn_scale, tokens,
                                      rotary_dim):
        check(lib.l0h_rope_execute_with_frequencies(self.device.handle, _ptr(q), _ptr(k), _ptr(positions),
                                                    _ptr(inv_freq), head_dim, n_heads, n_kv,
                                                    ctypes.c_float(attn_scale), tokens, rotary_dim))

    def kv_cache_store_execute(self, k, v, k_cache, v_cache, pos, kv_dim, cache_dtype=F32):
        check(lib.l0h_kv_cache_store_execute(self.device.handle, _ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache),
                                             cache_dtype, pos, kv_dim))

    def kv_cache_store_execute_rows(self, k, v, k_cache, v_cache, pos0, kv_dim, tokens, cache_dtype=F32):
        check(lib.l0h_kv_cache_store_execute_rows(self.device.handle, _ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache),
                                                  cache_dtype, pos0, kv_dim, tokens))

    def attention_execute(self, q, k_cache, v_cache, out, head_dim, n_heads, n_kv, seq_len, max_seq_len,
                          cache_dtype=F32):
        check(lib.l0h_attention_execute(self.device.handle, _ptr(q), _ptr(k_cache), _ptr(v_cache), cache_dtype,
                                        _ptr(out), head_dim, n_heads, n_kv, seq_len, max_seq_len))

    def attention_execute_prefill(self, q, k_cache, v_cache, out, head_dim, n_heads, n_kv, pos0, tokens, max_seq_len,
                                  cache_dtype=F32):
        check(lib.l0h_attention_execute_prefill(self.device.handle, _ptr(q), _ptr(k_cache), _ptr(v_cache),
                                                cache_dtype, _ptr(out), head_dim, n_heads, n_kv, pos0, tokens,
                                                max_seq_len))

    def embedding_execute(self, ids, table, out, h, n):
        check(lib.l0h_embedding_execute(self.device.handle, _ptr(ids), _ptr(table), _ptr(out), h, n))

    def copy_execute(self, src, dst, src_offset, n):
        check(lib.l0h_copy_execute(self.device.handle, _ptr(src), _ptr(dst), src_offset, n))

    def sampling_execute(self, logits, sampled, temperature, random_val, vocab):
        check(lib.l0h_sampling_execute(self.device.handle, _ptr(logits), _ptr(sampled), ctypes.c_float(temperature),
                                       ctypes.c_float(random_val), vocab))

    # [N, K] weight-format kernels (int8 weight-only per row, fp16, bf16, fp32)
    def gemv_nk(self, w_dtype, rows, out_dim, in_dim, x, x_dtype, w, scales, y, y_dtype):
        check(lib.l0h_gemv_nk(self.device.handle, w_dtype, rows, out_dim, in_dim, _ptr(x), x_dtype, _ptr(w),
                              _ptr(scales), _ptr(y), y_dtype))

    def gemm_nk(self, dtype, m, n, k, x, w, y, y_dtype):
        check(lib.l0h_gemm_nk(self.device.handle, dtype, m, n, k, _ptr(x), _ptr(w), _ptr(y), y_dtype))

    def gemm_nk_i8pc(self, m, n, k, x, w, scales, y, y_dtype):
        """x fp16 [m, k], w int8 [n, k], scales fp16 [n]."""
        check(lib.l0h_gemm_nk_i8pc(self.device.handle, m, n, k, _ptr(x), _ptr(w), _ptr(scales), _ptr(y), y_dtype))

    def attention_decode_noalloc(self, q, q_dtype, k_cache, v_cache, cache_dtype, out, out_dtype, batch, head_dim,
                                 n_heads, n_kv, seq_len, max_seq_len):
        """attention_decode with its split partials in the library's static scratch (no allocation)."""
        check(lib.l0h_attention_decode_noalloc(self.device.handle, _ptr(q), q_dtype, _ptr(k_cache), _ptr(v_cache),
                                               cache_dtype, _ptr(out), out_dtype, batch, head_dim, n_heads, n_kv,
                                               seq_len, max_seq_len))

    def attention_decode(self, q, q_dtype, k_cache, v_cache, cache_dtype, out, out_dtype, batch, head_dim, n_heads,
                         n_kv, seq_len, max_seq_len):
        check(lib.l0h_attention_decode(self.device.handle, _ptr(q), q_dtype, _ptr(k_cache), _ptr(v_cache),
                                       cache_dtype, _ptr(out), out_dtype, batch, head_dim, n_heads, n_kv, seq_len,
                                       max_seq_len))


def fits_in_half(values: np.ndarray) -> bool:
    a = np.ascontiguousarray(values, dtype=np.float32)
    return bool(lib.l0h_fits_in_half(a.ctypes.data_as(ctypes.c_void_p), a.size))


def transpose(src: np.ndarray, rows: int, cols: int) -> np.ndarray:
    a = np.ascontiguousarray(src, dtype=np.float32).reshape(-1)
    if a.size != rows * cols:
        raise _lib.InvalidArgumentError(_lib.ERR_INVALID_ARG, f"Expected {rows * cols} elements, got {a.size}.")
    out = np.empty(rows * cols, dtype=np.float32)
    check(lib.l0h_transpose(a.ctypes.data_as(ctypes.c_void_p), rows, cols, out.ctypes.data_as(ctypes.c_void_p)))
    return out


def quantize_i8pc(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-output-channel int8 quantization of an [N, K] matrix: (q int8 [N, K], fp16 scales [N])."""
    a = np.ascontiguousarray(w, dtype=np.float32)
    n, k = a.shape
    q = np.empty((n, k), dtype=np.int8)
    s = np.empty(n, dtype=np.uint16)
    check(lib.l0h_quantize_i8pc(a.ctypes.data_as(ctypes.c_void_p), n, k, q.ctypes.data_as(ctypes.c_void_p),
                                s.ctypes.data_as(ctypes.c_void_p)))
    return q, s.view(np.float16)


ROPE_TYPES = {None: 0, "default": 0, "linear": 1, "yarn": 2, "llama3": 3}


@dataclass
class RopeScaling:
    """HfRopeScaling (RopeFrequencies.cs:6-40)."""

    type: str = "default"
    factor: float = 1.0
    original_max_position_embeddings: int | None = None
    beta_fast: float = 32.0
    beta_slow: float = 1.0
    mscale: float | None = None
    mscale_all_dim: float | None = None
    attention_factor: float | None = None
    low_freq_factor: float = 1.0
    high_freq_factor: float = 4.0
    truncate: bool = True


def rope_frequencies(head_dim: int, theta: float, max_position_embeddings: int,
                     scaling: RopeScaling | None = None) -> tuple[np.ndarray, float]:
    """RopeFrequencies.Compute (RopeFrequencies.cs:60-183): (inv_freq fp32 [head_dim/2], attention factor)."""
    s = scaling or RopeScaling()
    if s.type not in ROPE_TYPES:
        raise _lib.UnsupportedError(_lib.ERR_UNSUPPORTED, f"rope_scaling '{s.type}' is not supported")
    inv = np.empty(max(head_dim // 2, 1), dtype=np.float32)
    att = ctypes.c_float()
    neg = lambda v: -1.0 if v is None else float(v)
    check(lib.l0h_rope_frequencies(head_dim, ctypes.c_double(theta), max_position_embeddings, ROPE_TYPES[s.type],
                                   ctypes.c_double(s.factor), s.original_max_position_embeddings or 0,
                                   ctypes.c_double(s.beta_fast), ctypes.c_double(s.beta_slow),
                                   ctypes.c_double(neg(s.mscale)), ctypes.c_double(neg(s.mscale_all_dim)),
                                   ctypes.c_double(neg(s.attention_factor)), ctypes.c_double(s.low_freq_factor),
                                   ctypes.c_double(s.high_freq_factor), int(s.truncate),
                                   inv.ctypes.data_as(ctypes.c_void_p), ctypes.byref(att)))
    return inv[: head_dim // 2], att.value


class LlmMatrix:
    """LlmMatrix (LlmMatrix.cs:7-260)."""

    def __init__(self, handle: ctypes.c_void_p):
        self.handle = handle
        i, o, st, sz = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_longlong()
        check(lib.l0h_matrix_info(handle, ctypes.byref(i), ctypes.byref(o), ctypes.byref(st), ctypes.byref(sz)))
        self.in_dim, self.out_dim, self.storage, self.size_in_bytes = i.value, o.value, st.value, sz.value

    @property
    def is_half(self) -> bool:
        return self.storage == F16

    @property
    def is_int8(self) -> bool:
        return self.storage == I8PC

    @classmethod
    def upload(cls, device: Device, data: np.ndarray, in_dim: int, out_dim: int, half: bool) -> "LlmMatrix":
        a = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
        if a.size != in_dim * out_dim:
            raise _lib.InvalidArgumentError(_lib.ERR_INVALID_ARG, f"Expected {in_dim * out_dim} elements, got {a.size}.")
        h = ctypes.c_void_p()
        check(lib.l0h_matrix_upload(device.handle, a.ctypes.data_as(ctypes.c_void_p), in_dim, out_dim, int(half),
                                    ctypes.byref(h)))
        return cls(h)

    @classmethod
    def from_hugging_face(cls, device: Device, hf: np.ndarray, sixteen_bit_source: bool, out_dim: int, in_dim: int,
                          precision: int) -> "LlmMatrix":
        a = np.ascontiguousarray(hf, dtype=np.float32).reshape(-1)
        if a.size != in_dim * out_dim:
            raise _lib.InvalidArgumentError(_lib.ERR_INVALID_ARG, f"Expected {in_dim * out_dim} elements, got {a.size}.")
        h = ctypes.c_void_p()
        check(lib.l0h_matrix_from_hf(device.handle, a.ctypes.data_as(ctypes.c_void_p), int(sixteen_bit_source),
                                     out_dim, in_dim, precision, ctypes.byref(h)))
        return cls(h)

    def data(self) -> tuple[int, int | None]:
        w, s = ctypes.c_void_p(), ctypes.c_void_p()
        check(lib.l0h_matrix_data(self.handle, ctypes.byref(w), ctypes.byref(s)))
        return w.value, s.value

    def project(self, device: Device, x: Buffer, y: Buffer) -> None:
        check(lib.l0h_matrix_project(device.handle, self.handle, _ptr(x), _ptr(y)))

    def project_rows(self, device: Device, rows: int, x: Buffer, y: Buffer) -> None:
        check(lib.l0h_matrix_project_rows(device.handle, self.handle, rows, _ptr(x), _ptr(y)))

    def project_any(self, device: Device, rows: int, x: Buffer, y: Buffer) -> None:
        check(lib.l0h_matrix_project_any(device.handle, self.handle, rows, _ptr(x), _ptr(y)))

    @staticmethod
    def project_shared(device: Device, rows: int, x: Buffer, pairs: list[tuple["LlmMatrix", Buffer]]) -> None:
        n = len(pairs)
        ms = (ctypes.c_void_p * n)(*[p[0].handle.value for p in pairs])
        ys = (ctypes.c_void_p * n)(*[p[1].ptr for p in pairs])
        check(lib.l0h_matrix_project_shared(device.handle, rows, _ptr(x), n, ms, ys))

    def dispose(self) -> None:
        if self.handle:
            check(lib.l0h_matrix_destroy(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()


@dataclass
class HfConfig:
    """The HfModelConfig fields the decoder uses (HfModelConfig.cs:10-120)."""

    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    vocab_size: int
    max_position_embeddings: int = 2048
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    attention_bias: bool = False
    tie_word_embeddings: bool = False
    rope_scaling: RopeScaling | None = None

    @property
    def query_dim(self) -> int:
        return self.num_attention_heads * self.head_dim

    @property
    def key_value_dim(self) -> int:
        return self.num_key_value_heads * self.head_dim

    def to_c(self) -> ModelConfig:
        s = self.rope_scaling or RopeScaling()
        neg = lambda v: -1.0 if v is None else float(v)
        return ModelConfig(self.hidden_size, self.intermediate_size, self.num_layers, self.num_attention_heads,
                           self.num_key_value_heads, self.head_dim, self.vocab_size, self.max_position_embeddings,
                           self.rms_norm_eps, self.rope_theta, int(self.attention_bias), int(self.tie_word_embeddings),
                           ROPE_TYPES[s.type], s.factor, s.original_max_position_embeddings or 0, s.beta_fast,
                           s.beta_slow, neg(s.mscale), neg(s.mscale_all_dim), neg(s.attention_factor),
                           s.low_freq_factor, s.high_freq_factor, int(s.truncate))


ST_DTYPES = ("BOOL", "U8", "I8", "I16", "U16", "F16", "BF16", "I32", "U32", "F32", "F64", "I64", "U64")


class SafetensorsCheckpoint:
    """SafetensorsCheckpoint (SafetensorsCheckpoint.cs): one .safetensors file, or a directory with
    model.safetensors.index.json and its shards, else model.safetensors. Host only."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(lib.l0h_safetensors_open(str(path).encode(), ctypes.byref(h)))
        self.handle = h

    def __len__(self) -> int:
        n = ctypes.c_int()
        check(lib.l0h_safetensors_count(self.handle, ctypes.byref(n)))
        return n.value

    def info(self, index: int) -> tuple[str, str, tuple[int, ...]]:
        """(name, dtype, shape) of tensor `index` in name order."""
        name = ctypes.create_string_buffer(1024)
        dt, rank = ctypes.c_int(), ctypes.c_int()
        shape = (ctypes.c_longlong * 16)()
        check(lib.l0h_safetensors_info(self.handle, index, name, 1024, ctypes.byref(dt), ctypes.byref(rank), shape, 16))
        return name.value.decode(), ST_DTYPES[dt.value], tuple(shape[i] for i in range(rank.value))

    @property
    def names(self) -> list[str]:
        return [self.info(i)[0] for i in range(len(self))]

    def __contains__(self, name: str) -> bool:
        i = ctypes.c_int()
        check(lib.l0h_safetensors_find(self.handle, name.encode(), ctypes.byref(i)))
        return i.value >= 0

    def read_float32(self, name: str) -> np.ndarray:
        """SafetensorsReader.ReadFloat32: F32 / F16 / BF16 / F64 as fp32, in the stored shape."""
        i = ctypes.c_int()
        check(lib.l0h_safetensors_find(self.handle, name.encode(), ctypes.byref(i)))
        if i.value < 0:
            raise KeyError(name)
        _, _, shape = self.info(i.value)
        out = np.empty(shape, dtype=np.float32)
        check(lib.l0h_safetensors_read_f32(self.handle, name.encode(), out.ctypes.data_as(ctypes.c_void_p), out.size))
        return out

    def close(self) -> None:
        if self.handle:
            check(lib.l0h_safetensors_close(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


KERNEL_KINDS = ("embedding", "qkv", "attention", "o_proj", "gate_up", "down", "lm_head", "argmax")


class KernelTiming(ctypes.Structure):
    """l0h_kernel_timing."""

    _fields_ = [("kind", ctypes.c_int), ("layer", ctypes.c_int), ("microseconds", ctypes.c_float),
                ("bytes", ctypes.c_double)]


class LlmModel:
    """LlmModel (LlmModel.cs): a decoder resident on the device, one sequence at a time."""

    def __init__(self, device: Device, config: HfConfig, precision: int = _lib.PRECISION_INT8,
                 cache_dtype: int = F16, max_seq_len: int = 2048):
        self.device = device
        self.config = config
        self.max_seq_len = max_seq_len
        self.cache_dtype = cache_dtype
        c = config.to_c()
        h = ctypes.c_void_p()
        check(lib.l0h_model_create(device.handle, ctypes.byref(c), precision, cache_dtype, max_seq_len,
                                   ctypes.byref(h)))
        self.handle = h

    def init_random(self, seed: int, std: float = 0.02) -> None:
        check(lib.l0h_model_init_random(self.handle, ctypes.c_uint64(seed), ctypes.c_float(std)))

    def set_tensor(self, name: str, data: np.ndarray, sixteen_bit_source: bool = False) -> None:
        a = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
        check(lib.l0h_model_set_tensor(self.handle, name.encode(), a.ctypes.data_as(ctypes.c_void_p), a.size,
                                       int(sixteen_bit_source)))

    def load_safetensors(self, checkpoint: "SafetensorsCheckpoint | str") -> int:
        """LlmModel.Load's weight pass from a safetensors checkpoint; returns the tensors read."""
        own = not isinstance(checkpoint, SafetensorsCheckpoint)
        ck = SafetensorsCheckpoint(checkpoint) if own else checkpoint
        try:
            n = ctypes.c_int()
            check(lib.l0h_model_load_safetensors(self.handle, ck.handle, ctypes.byref(n)))
            return n.value
        finally:
            if own:
                ck.close()

    def export_matrix(self, name: str) -> tuple[int, np.ndarray, np.ndarray | None]:
        st, n, k = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        check(lib.l0h_model_export_matrix(self.handle, name.encode(), ctypes.byref(st), ctypes.byref(n),
                                          ctypes.byref(k), None, None))
        w = np.empty((n.value, k.value), dtype=_NP[st.value])
        s = np.empty(n.value, dtype=np.uint16) if st.value == I8PC else None
        check(lib.l0h_model_export_matrix(self.handle, name.encode(), None, None, None,
                                          w.ctypes.data_as(ctypes.c_void_p),
                                          None if s is None else s.ctypes.data_as(ctypes.c_void_p)))
        return st.value, w, s

    def export_vector(self, name: str, count: int) -> np.ndarray:
        out = np.empty(count, dtype=np.float32)
        check(lib.l0h_model_export_vector(self.handle, name.encode(), out.ctypes.data_as(ctypes.c_void_p), count))
        return out

    def kv_cache(self, layer: int) -> tuple[int, int]:
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        check(lib.l0h_model_kv_cache(self.handle, layer, ctypes.byref(k), ctypes.byref(v)))
        return k.value, v.value

    def last_logits(self) -> np.ndarray:
        """The logits the last decode step left in device memory, read back."""
        p = ctypes.c_void_p()
        check(lib.l0h_model_logits(self.handle, ctypes.byref(p)))
        vocab = self.config.vocab_size
        return Buffer(self.device, 4 * vocab, ptr=p.value, owned=False).read(np.float32, vocab)

    @property
    def step_launches(self) -> int:
        """Kernel launches in one decode step (the nodes of the step's HIP graph)."""
        n = ctypes.c_int()
        check(lib.l0h_model_step_launches(self.handle, ctypes.byref(n)))
        return n.value

    @property
    def step_path(self) -> str:
        """'graph', 'eager' or 'persistent': how a decode step runs."""
        v = ctypes.c_int()
        check(lib.l0h_model_step_path(self.handle, ctypes.byref(v)))
        return ("graph", "eager", "persistent")[v.value]

    @property
    def projection_bytes(self) -> int:
        b = ctypes.c_longlong()
        check(lib.l0h_model_projection_bytes(self.handle, ctypes.byref(b)))
        return b.value

    @property
    def position(self) -> int:
        p = ctypes.c_int()
        check(lib.l0h_model_position(self.handle, ctypes.byref(p)))
        return p.value

    def reset_sequence(self) -> None:
        check(lib.l0h_model_reset_sequence(self.handle))

    def _logits_out(self):
        out = np.empty(self.config.vocab_size, dtype=np.float32)
        return out, out.ctypes.data_as(ctypes.c_void_p)

    def compute_logits(self, token: int, position: int) -> np.ndarray:
        out, p = self._logits_out()
        check(lib.l0h_model_compute_logits(self.handle, token, position, p))
        return out

    def prefill(self, prompt_ids) -> np.ndarray:
        ids = np.ascontiguousarray(prompt_ids, dtype=np.int32)
        out, p = self._logits_out()
        check(lib.l0h_model_prefill(self.handle, ids.ctypes.data_as(ctypes.c_void_p), ids.size, p))
        return out

    def decode(self, token: int) -> np.ndarray:
        out, p = self._logits_out()
        check(lib.l0h_model_decode(self.handle, token, p))
        return out

    def generate_greedy(self, prompt_ids, max_new_tokens: int, stop_token_ids=()) -> list[int]:
        ids = np.ascontiguousarray(prompt_ids, dtype=np.int32)
        stop = np.ascontiguousarray(list(stop_token_ids) or [0], dtype=np.int32)
        out = np.empty(max(max_new_tokens, 1), dtype=np.int32)
        n = ctypes.c_int()
        check(lib.l0h_model_generate_greedy(self.handle, ids.ctypes.data_as(ctypes.c_void_p), ids.size,
                                            max_new_tokens, stop.ctypes.data_as(ctypes.c_void_p),
                                            len(stop_token_ids), out.ctypes.data_as(ctypes.c_void_p), ctypes.byref(n)))
        return out[: n.value].tolist()

    def profile_step(self, token: int, position: int) -> list[dict]:
        """One eager decode step with a HIP-event pair around every launch: kind, layer, us, bytes."""
        cap = 8 * self.config.num_layers + 16
        buf = (KernelTiming * cap)()
        n = ctypes.c_int()
        check(lib.l0h_model_profile_step(self.handle, token, position, buf, cap, ctypes.byref(n)))
        return [dict(kind=KERNEL_KINDS[e.kind], layer=e.layer, us=e.microseconds, bytes=e.bytes)
                for e in buf[: n.value]]

    def probe_step(self, token: int, position: int) -> tuple[np.ndarray, dict[tuple[int, str], np.ndarray]]:
        """LlmDecoderLayer.Probe over every layer of one eager decode step: the logits and a copy of
        each stage's values, keyed (layer, stage) with the reference's stage names."""
        stages: dict[tuple[int, str], np.ndarray] = {}

        def on_stage(_user, layer, stage, values, count):
            stages[(layer, stage.decode())] = np.ctypeslib.as_array(values, shape=(count,)).copy()

        cb = _lib.PROBE_FN(on_stage)
        out, p = self._logits_out()
        check(lib.l0h_model_probe_step(self.handle, token, position, ctypes.cast(cb, ctypes.c_void_p), None, p))
        return out, stages

    def profile_kernel(self, kind: str, position: int, rounds: int = 4) -> dict:
        """Back-to-back launches of one kernel kind (every layer per round): avg us, bytes, launches/step."""
        us, b, n = ctypes.c_float(), ctypes.c_double(), ctypes.c_int()
        check(lib.l0h_model_profile_kernel(self.handle, KERNEL_KINDS.index(kind), position, rounds, ctypes.byref(us),
                                           ctypes.byref(b), ctypes.byref(n)))
        return dict(kind=kind, us=us.value, bytes=b.value, launches=n.value)

    def decode_greedy_device(self, token: int, steps: int) -> np.ndarray:
        out = np.empty(max(steps, 1), dtype=np.int32)
        check(lib.l0h_model_decode_greedy_device(self.handle, token, steps, out.ctypes.data_as(ctypes.c_void_p)))
        return out[:steps]

    def dispose(self) -> None:
        if self.handle:
            check(lib.l0h_model_destroy(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()


def _config_fields() -> list[str]:
    return [f.name for f in fields(HfConfig)]
