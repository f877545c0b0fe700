"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the cpu_baseline
leg of bench.py, as the checker. The product package (l0llm_amd) never imports it."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

F32, F16, BF16, I8PC = 0, 1, 2, 3


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def _load() -> ctypes.CDLL:
    if not LIB.exists():
        build()
    return ctypes.CDLL(str(LIB))


_lib = _load()
P = ctypes.c_void_p


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(P)


def _sig(name, args, res=None):
    f = getattr(_lib, name)
    f.argtypes = args
    f.restype = res
    return f


_sig("orc_f32_to_f16", [ctypes.c_float], ctypes.c_uint16)
_sig("orc_f16_to_f32", [ctypes.c_uint16], ctypes.c_float)
_sig("orc_f32_to_bf16", [ctypes.c_float], ctypes.c_uint16)
_sig("orc_bf16_to_f32", [ctypes.c_uint16], ctypes.c_float)
_sig("orc_fits_in_half", [P, ctypes.c_size_t], ctypes.c_int)
_sig("orc_transpose", [P, ctypes.c_int, ctypes.c_int, P])
_sig("orc_quantize_i8pc", [P, ctypes.c_int, ctypes.c_int, P, P])
_sig("orc_gemv_nk", [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P])
_sig("orc_gemv_kn", [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P])
_sig("orc_rmsnorm", [P, P, P, P, ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int])
_sig("orc_swiglu", [P, P, ctypes.c_int])
_sig("orc_add", [P, P, ctypes.c_int])
_sig("orc_bias_add", [P, P, ctypes.c_int, ctypes.c_int])
_sig("orc_rope_frequencies", [ctypes.c_int, ctypes.c_double, ctypes.c_int, ctypes.c_int, ctypes.c_double,
                              ctypes.c_int, ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_double,
                              ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_int, P, P], ctypes.c_int)
_sig("orc_rope_table", [P, P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int,
                        ctypes.c_int])
_sig("orc_rope_theta", [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int])
_sig("orc_kv_store", [P, P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int])
_sig("orc_attention_decode", [P, P, P, ctypes.c_int, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                              ctypes.c_int])
_sig("orc_attention_prefill", [P, P, P, ctypes.c_int, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                               ctypes.c_int, ctypes.c_int])
_sig("orc_embedding", [P, P, P, ctypes.c_int, ctypes.c_int])
_sig("orc_argmax", [P, ctypes.c_int], ctypes.c_int)
_sig("orc_top2_margin", [P, ctypes.c_int], ctypes.c_float)
_sig("orc_num_threads", [], ctypes.c_int)
_sig("orc_set_threads", [ctypes.c_int])
_sig("orc_set_fast_projections", [ctypes.c_int])
_sig("orc_set_device_rounding", [ctypes.c_int])
_sig("orc_gemv_nk_f32acc", [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P])


def gemv_nk_f32acc(wdtype: int, w: np.ndarray, x: np.ndarray, scales: np.ndarray | None = None) -> np.ndarray:
    """The CPU-baseline form of gemv_nk: fp32 accumulation, vectorised, OpenMP over output rows."""
    w = np.ascontiguousarray(w)
    n, k = w.shape
    xx = f32(x).reshape(-1, k)
    y = np.empty((xx.shape[0], n), dtype=np.float32)
    s = None if scales is None else np.ascontiguousarray(scales).view(np.uint16)
    _lib.orc_gemv_nk_f32acc(wdtype, xx.shape[0], n, k, _p(xx), _p(w), _p(s), _p(y))
    return y


def set_threads(n: int) -> None:
    _lib.orc_set_threads(int(n))


def set_fast_projections(on: bool) -> None:
    _lib.orc_set_fast_projections(int(bool(on)))


def set_device_rounding(on: bool) -> None:
    """Rounds the attention and SwiGLU outputs to fp16 inside the model step, where the HIP decode
    step stores them as fp16 (orc_set_device_rounding); off by default (the reference's fp32)."""
    _lib.orc_set_device_rounding(int(bool(on)))


def num_threads() -> int:
    return _lib.orc_num_threads()


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def f32_to_f16_bits(v: float) -> int:
    return _lib.orc_f32_to_f16(v)


def f16_bits_to_f32(h: int) -> float:
    return _lib.orc_f16_to_f32(h)


def f32_to_bf16_bits(v: float) -> int:
    return _lib.orc_f32_to_bf16(v)


def fits_in_half(v) -> bool:
    a = f32(v).reshape(-1)
    return bool(_lib.orc_fits_in_half(_p(a), a.size))


def transpose(src, rows: int, cols: int) -> np.ndarray:
    a = f32(src).reshape(-1)
    out = np.empty(rows * cols, dtype=np.float32)
    _lib.orc_transpose(_p(a), rows, cols, _p(out))
    return out


def quantize_i8pc(w) -> tuple[np.ndarray, np.ndarray]:
    a = f32(w)
    n, k = a.shape
    q = np.empty((n, k), dtype=np.int8)
    s = np.empty(n, dtype=np.uint16)
    _lib.orc_quantize_i8pc(_p(a), n, k, _p(q), _p(s))
    return q, s


def gemv_nk(wdtype: int, w: np.ndarray, x: np.ndarray, scales: np.ndarray | None = None) -> np.ndarray:
    """y[r, n] = sum_k x[r, k] W[n, k] (* s[n]); w is the stored array (int8 / fp16 bits / bf16 bits / fp32)."""
    w = np.ascontiguousarray(w)
    n, k = w.shape
    xx = f32(x).reshape(-1, k)
    y = np.empty((xx.shape[0], n), dtype=np.float32)
    s = None if scales is None else np.ascontiguousarray(scales).view(np.uint16)
    _lib.orc_gemv_nk(wdtype, xx.shape[0], n, k, _p(xx), _p(w), _p(s), _p(y))
    return y


def gemv_kn(wdtype: int, w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w)
    k, n = w.shape
    xx = f32(x).reshape(-1, k)
    y = np.empty((xx.shape[0], n), dtype=np.float32)
    _lib.orc_gemv_kn(wdtype, xx.shape[0], n, k, _p(xx), _p(w), _p(y))
    return y


def rmsnorm(x, w, eps: float, residual=None) -> tuple[np.ndarray, np.ndarray]:
    """Returns (x after the optional residual add, normalised output)."""
    xx = f32(x).copy()
    n = xx.shape[-1]
    rows = xx.size // n
    out = np.empty_like(xx)
    r = None if residual is None else f32(residual)
    _lib.orc_rmsnorm(_p(xx), _p(r), _p(f32(w)), _p(out), eps, n, rows, int(residual is not None))
    return xx, out


def swiglu(gate, up) -> np.ndarray:
    g = f32(gate).copy()
    _lib.orc_swiglu(_p(g), _p(f32(up)), g.size)
    return g


def add(a, b) -> np.ndarray:
    x = f32(a).copy()
    _lib.orc_add(_p(x), _p(f32(b)), x.size)
    return x


def bias_add(x, bias, n: int, rows: int) -> np.ndarray:
    xx = f32(x).copy()
    _lib.orc_bias_add(_p(xx), _p(f32(bias)), n, rows)
    return xx


ROPE = {"default": 0, "linear": 1, "yarn": 2, "llama3": 3}


def rope_frequencies(head_dim, theta, max_pos, type_="default", factor=1.0, original_max=0, beta_fast=32.0,
                     beta_slow=1.0, mscale=None, mscale_all_dim=None, attention_factor=None, low_freq_factor=1.0,
                     high_freq_factor=4.0, truncate=True) -> tuple[np.ndarray, float]:
    inv = np.empty(max(head_dim // 2, 1), dtype=np.float32)
    att = np.empty(1, dtype=np.float32)
    neg = lambda v: -1.0 if v is None else float(v)
    rc = _lib.orc_rope_frequencies(head_dim, theta, max_pos, ROPE[type_], factor, original_max or 0, beta_fast,
                                   beta_slow, neg(mscale), neg(mscale_all_dim), neg(attention_factor),
                                   low_freq_factor, high_freq_factor, int(truncate), _p(inv), _p(att))
    if rc != 0:
        raise ValueError("rope_frequencies rejected its arguments")
    return inv[: head_dim // 2], float(att[0])


def rope_table(q, k, positions, inv_freq, head_dim, nh, nkv, attn_scale=1.0, rotary_dim=None):
    qq, kk = f32(q).copy(), f32(k).copy()
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    _lib.orc_rope_table(_p(qq), _p(kk), _p(pos), _p(f32(inv_freq)), head_dim, nh, nkv, attn_scale, pos.size,
                        rotary_dim or head_dim)
    return qq, kk


def rope_theta(q, k, positions, head_dim, nh, nkv, theta):
    qq, kk = f32(q).copy(), f32(k).copy()
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    _lib.orc_rope_theta(_p(qq), _p(kk), _p(pos), head_dim, nh, nkv, theta, pos.size)
    return qq, kk


def kv_store(k, v, kc: np.ndarray, vc: np.ndarray, cache_dtype: int, pos0: int, kv_dim: int, tokens: int) -> None:
    _lib.orc_kv_store(_p(f32(k)), _p(f32(v)), _p(kc), _p(vc), cache_dtype, pos0, kv_dim, tokens)


def attention_decode(q, kc, vc, cache_dtype, head_dim, nh, nkv, seq_len, max_seq_len) -> np.ndarray:
    out = np.empty(nh * head_dim, dtype=np.float32)
    _lib.orc_attention_decode(_p(f32(q)), _p(np.ascontiguousarray(kc)), _p(np.ascontiguousarray(vc)), cache_dtype,
                              _p(out), head_dim, nh, nkv, seq_len, max_seq_len)
    return out


def attention_prefill(q, kc, vc, cache_dtype, head_dim, nh, nkv, pos0, tokens, max_seq_len) -> np.ndarray:
    out = np.empty(tokens * nh * head_dim, dtype=np.float32)
    _lib.orc_attention_prefill(_p(f32(q)), _p(np.ascontiguousarray(kc)), _p(np.ascontiguousarray(vc)), cache_dtype,
                               _p(out), head_dim, nh, nkv, pos0, tokens, max_seq_len)
    return out


def embedding(ids, table, h: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _lib.orc_embedding(_p(np.ascontiguousarray(ids, dtype=np.int32)), _p(f32(table)), _p(out), h, n)
    return out


def argmax(logits) -> int:
    a = f32(logits)
    return _lib.orc_argmax(_p(a), a.size)


def top2_margin(logits) -> float:
    a = f32(logits)
    return _lib.orc_top2_margin(_p(a), a.size)


# ---- whole-model oracle ---------------------------------------------------------------------

class _Config(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("intermediate", ctypes.c_int), ("n_layers", ctypes.c_int),
                ("n_heads", ctypes.c_int), ("n_kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("vocab", ctypes.c_int), ("eps", ctypes.c_float), ("attention_bias", ctypes.c_int),
                ("tie_embeddings", ctypes.c_int), ("rotary_dim", ctypes.c_int),
                ("rope_attention_scale", ctypes.c_float)]


class _Matrix(ctypes.Structure):
    _fields_ = [("wdtype", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int), ("w", P), ("scales", P)]


class _Layer(ctypes.Structure):
    _fields_ = [("input_norm", P), ("post_norm", P), ("q", _Matrix), ("k", _Matrix), ("v", _Matrix),
                ("o", _Matrix), ("gate", _Matrix), ("up", _Matrix), ("down", _Matrix), ("q_bias", P),
                ("k_bias", P), ("v_bias", P)]


class _Model(ctypes.Structure):
    _fields_ = [("cfg", _Config), ("embedding", P), ("final_norm", P), ("lm_head", _Matrix),
                ("layers", ctypes.POINTER(_Layer)), ("inv_freq", P), ("cache_dtype", ctypes.c_int),
                ("max_seq_len", ctypes.c_int), ("k_cache", ctypes.POINTER(P)), ("v_cache", ctypes.POINTER(P))]


_sig("orc_model_step", [ctypes.POINTER(_Model), ctypes.c_int, ctypes.c_int, P], ctypes.c_int)
_sig("orc_layer_forward", [ctypes.POINTER(_Model), ctypes.c_int, P, ctypes.c_int])


class Model:
    """Whole-decoder oracle (LlmModel.Step / LlmDecoderLayer.Forward restated).

    ``weights`` maps HuggingFace tensor names to arrays: projections as (storage dtype, stored
    array, fp16 scales or None), vectors as fp32 arrays."""

    def __init__(self, cfg: dict, weights: dict, inv_freq: np.ndarray, attn_scale: float, cache_dtype: int,
                 max_seq_len: int):
        self._keep = []
        c = cfg
        self.vocab = c["vocab_size"]
        self.hidden = c["hidden_size"]
        kv_dim = c["num_key_value_heads"] * c["head_dim"]
        conf = _Config(c["hidden_size"], c["intermediate_size"], c["num_layers"], c["num_attention_heads"],
                       c["num_key_value_heads"], c["head_dim"], c["vocab_size"], c["rms_norm_eps"],
                       int(c.get("attention_bias", False)), int(c.get("tie_word_embeddings", False)),
                       c["head_dim"], attn_scale)

        def keep(a):
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            return a.ctypes.data_as(P)

        def mat(name):
            dt, w, s = weights[name]
            w = np.ascontiguousarray(w)
            return _Matrix(dt, w.shape[0], w.shape[1], keep(w), None if s is None else keep(np.asarray(s).view(np.uint16)))

        layers = (_Layer * c["num_layers"])()
        for i in range(c["num_layers"]):
            p = f"model.layers.{i}."
            L = layers[i]
            L.input_norm = keep(f32(weights[p + "input_layernorm.weight"]))
            L.post_norm = keep(f32(weights[p + "post_attention_layernorm.weight"]))
            L.q, L.k, L.v = mat(p + "self_attn.q_proj.weight"), mat(p + "self_attn.k_proj.weight"), mat(p + "self_attn.v_proj.weight")
            L.o = mat(p + "self_attn.o_proj.weight")
            L.gate, L.up, L.down = mat(p + "mlp.gate_proj.weight"), mat(p + "mlp.up_proj.weight"), mat(p + "mlp.down_proj.weight")
            if c.get("attention_bias"):
                L.q_bias = keep(f32(weights[p + "self_attn.q_proj.bias"]))
                L.k_bias = keep(f32(weights[p + "self_attn.k_proj.bias"]))
                L.v_bias = keep(f32(weights[p + "self_attn.v_proj.bias"]))
        self._layers = layers
        cache_item = 2 if cache_dtype == F16 else 4
        self.k_caches = [np.zeros(max_seq_len * kv_dim * cache_item, dtype=np.uint8) for _ in range(c["num_layers"])]
        self.v_caches = [np.zeros(max_seq_len * kv_dim * cache_item, dtype=np.uint8) for _ in range(c["num_layers"])]
        kp = (P * c["num_layers"])(*[a.ctypes.data for a in self.k_caches])
        vp = (P * c["num_layers"])(*[a.ctypes.data for a in self.v_caches])
        self._keep += [kp, vp]
        self._m = _Model(conf, keep(f32(weights["model.embed_tokens.weight"])), keep(f32(weights["model.norm.weight"])),
                         mat("lm_head.weight"), ctypes.cast(layers, ctypes.POINTER(_Layer)), keep(f32(inv_freq)),
                         cache_dtype, max_seq_len, ctypes.cast(kp, ctypes.POINTER(P)), ctypes.cast(vp, ctypes.POINTER(P)))

    def load_cache(self, layer: int, k_bytes: np.ndarray, v_bytes: np.ndarray) -> None:
        """Seeds layer `layer`'s K and V caches with raw cache bytes ([max_seq_len, kv_dim] of the
        cache dtype; a shorter prefix fills the first slots)."""
        for dst, src in ((self.k_caches[layer], k_bytes), (self.v_caches[layer], v_bytes)):
            b = np.ascontiguousarray(src).view(np.uint8).reshape(-1)
            if b.size > dst.size:
                raise ValueError("cache bytes exceed the oracle's cache")
            dst[: b.size] = b

    def step(self, token: int, position: int) -> tuple[int, np.ndarray]:
        logits = np.empty(self.vocab, dtype=np.float32)
        nxt = _lib.orc_model_step(ctypes.byref(self._m), token, position, _p(logits))
        return nxt, logits
