"""Shared test helpers: fixtures of the tiny Hugging Face decoders and conversions between
stored weight formats."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from oracle import pyoracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden"


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns."""
    x = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    x = x + 0x7FFF + ((x >> 16) & 1)
    return (x >> 16).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def stored(storage: int, w: np.ndarray):
    """(storage, stored array, scales) of an fp32 [N, K] matrix, as the oracle consumes it."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    if storage == orc.F32:
        return orc.F32, w, None
    if storage == orc.F16:
        return orc.F16, w.astype(np.float16).view(np.uint16), None
    if storage == orc.BF16:
        return orc.BF16, bf16_bits(w), None
    q, s = orc.quantize_i8pc(w)
    return orc.I8PC, q, s


def dequant(storage: int, w: np.ndarray, s: np.ndarray | None) -> np.ndarray:
    if storage == orc.F32:
        return w.astype(np.float64)
    if storage == orc.F16:
        return w.view(np.float16).astype(np.float64)
    if storage == orc.BF16:
        return bf16_to_f32(w).astype(np.float64)
    return w.astype(np.float64) * s.view(np.float16).astype(np.float64)[:, None]


def load_hf(name: str) -> dict:
    z = np.load(GOLDEN / f"hf_tiny_{name}.npz", allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    weights = {k[2:]: z[k] for k in z.files if k.startswith("w/")}
    c = meta["config"]
    rp = c["rope_parameters"]
    cfg = dict(vocab_size=c["vocab_size"], hidden_size=c["hidden_size"], intermediate_size=c["intermediate_size"],
               num_layers=c["num_hidden_layers"], num_attention_heads=c["num_attention_heads"],
               num_key_value_heads=c["num_key_value_heads"],
               head_dim=c.get("head_dim", c["hidden_size"] // c["num_attention_heads"]),
               max_position_embeddings=c["max_position_embeddings"], rms_norm_eps=c["rms_norm_eps"],
               rope_theta=rp["rope_theta"], tie_word_embeddings=c["tie_word_embeddings"],
               attention_bias="q_proj.bias" in " ".join(weights), rope=rp)
    return dict(cfg=cfg, weights=weights, prompt=meta["prompt"], generated=meta["generated"],
                margins=meta["margins"], prompt_logits=z["prompt_logits"])


def rope_table_for(cfg: dict) -> tuple[np.ndarray, float]:
    rp = cfg["rope"]
    t = rp.get("rope_type", "default")
    return orc.rope_frequencies(cfg["head_dim"], rp["rope_theta"], cfg["max_position_embeddings"], t,
                                factor=rp.get("factor", 1.0),
                                original_max=rp.get("original_max_position_embeddings", 0) or 0,
                                low_freq_factor=rp.get("low_freq_factor", 1.0),
                                high_freq_factor=rp.get("high_freq_factor", 4.0))


PROJECTIONS = ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
               "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")


def oracle_weights(cfg: dict, weights: dict, storage: int) -> dict:
    """HF fp32 tensors -> the oracle's weight dict at a storage type (projections converted)."""
    out = {}
    for k, v in weights.items():
        if k.endswith(".weight") and v.ndim == 2 and k != "model.embed_tokens.weight":
            out[k] = stored(storage, v)
        else:
            out[k] = v
    if "lm_head.weight" not in weights:
        out["lm_head.weight"] = stored(storage, weights["model.embed_tokens.weight"])
    return out


def oracle_model(cfg: dict, weights: dict, storage: int, cache_dtype: int, max_seq_len: int) -> orc.Model:
    inv, att = rope_table_for(cfg)
    return orc.Model(cfg, oracle_weights(cfg, weights, storage), inv, att, cache_dtype, max_seq_len)


def rel_err(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def elementwise_excess(got, want, rtol: float = 1e-2, floor_frac: float = 1e-4) -> float:
    """Per-element relative bound for 16-bit outputs: |got - want| <= rtol * |want| + floor, where
    floor = floor_frac * max|want| stands in for the relative bound at values near zero (where a
    relative error is undefined). Returns the largest |got - want| / bound; at most 1 passes."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    bound = rtol * np.abs(want) + floor_frac * max(float(np.max(np.abs(want))), 1e-30)
    return float(np.max(np.abs(got - want) / bound))
