#!/usr/bin/env python3
"""Decode throughput of a Llama-3.1-8B-shaped int8 weight-only model on one MI355X.

Workload: 32 layers, hidden 4096, intermediate 14336, 32 q / 8 kv heads, head_dim 128, vocab
128256, RMSNorm eps 1e-5, RoPE theta 5e5; random-init weights N(0, 0.02) stored as int8 with one
fp16 scale per output row; fp16 KV cache. Batch 1: a 2048-token prompt of seeded random ids is
prefilled, then greedy decode. A step is one generated token (all 32 layers, lm_head, argmax);
the timed region is `--steps` back-to-back steps at positions 2048.. with every input resident
in HBM, bracketed by device synchronisation.

The JSON line also carries:
  roofline      the int8 weight-streaming GEMV (the dominant kernel: q|k|v, O, gate|up, down and
                lm_head launches): algorithmic bytes / HIP-event duration per launch, measured
                live on the model's stream (back-to-back launches over all layers), against 8 TB/s
  kernels       the same per kernel kind
  cpu_baseline  the CPU oracle (fp64-accumulating C) running the same model's decode steps on the
                host cores, for a bounded sample of `--cpu-tokens` tokens
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "int8 decode GEMV HBM GB/s (% of peak); 8B-shape decode tokens/s at 1 GPU"
GEMV_KINDS = ("qkv", "o_proj", "gate_up", "down", "lm_head")
PROJECTIONS = ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
               "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")


def llama8b():
    import l0llm_amd as l0
    return l0.HfConfig(hidden_size=4096, intermediate_size=14336, num_layers=32, num_attention_heads=32,
                       num_key_value_heads=8, head_dim=128, vocab_size=128256, max_position_embeddings=131072,
                       rms_norm_eps=1e-5, rope_theta=500000.0)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


KINDS = ("embedding", "qkv", "attention", "o_proj", "gate_up", "down", "lm_head", "argmax")


def kernel_table(model, position: int, rounds: int) -> dict:
    """Per kernel kind: HIP-event time of back-to-back launches on the model's stream (every
    layer once per round, so weights stream from HBM), divided per launch."""
    out = {}
    for kind in KINDS:
        r = model.profile_kernel(kind, position, rounds if kind in GEMV_KINDS + ("attention",) else 4 * rounds)
        gbs = r["bytes"] / (r["us"] * 1e-6) / 1e9 if r["us"] > 0 else 0.0
        out[kind] = dict(launches_per_step=r["launches"], avg_us=round(r["us"], 3), bytes_per_launch=round(r["bytes"]),
                         gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4))
    return out


def hbm_copy_probe(dev, mib: int = 1024, reps: int = 10) -> dict:
    """Achievable HBM rate on this box: Copy.Execute (a 16-byte grid-stride copy kernel) over two
    buffers of `mib` MiB, far larger than the 256 MB Infinity Cache; bytes = read + write."""
    import l0llm_amd as l0

    n = mib * (1 << 20) // 4
    suite = l0.LlmKernelSuite(dev)
    with dev.alloc(4 * n) as a, dev.alloc(4 * n) as b:
        a.zero()
        suite.copy_execute(a, b, 0, n)
        dev.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            suite.copy_execute(a, b, 0, n)
        dev.synchronize()
        dt = (time.perf_counter() - t0) / reps
    return dict(kernel="copy16_kernel", bytes_per_launch=8 * n, avg_us=round(dt * 1e6, 1),
                gbs=round(8 * n / dt / 1e9, 1))


def cpu_baseline(model, cfg, tokens: int, position: int) -> dict:
    from oracle import pyoracle as orc

    H = cfg.hidden_size
    w = {"model.embed_tokens.weight": model.export_vector("model.embed_tokens.weight", cfg.vocab_size * H),
         "model.norm.weight": model.export_vector("model.norm.weight", H),
         "lm_head.weight": model.export_matrix("lm_head.weight")}
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}."
        for n in PROJECTIONS:
            w[p + n] = model.export_matrix(p + n)
        for n in ("input_layernorm.weight", "post_attention_layernorm.weight"):
            w[p + n] = model.export_vector(p + n, H)
    inv, att = orc.rope_frequencies(cfg.head_dim, cfg.rope_theta, cfg.max_position_embeddings)
    c = dict(vocab_size=cfg.vocab_size, hidden_size=H, intermediate_size=cfg.intermediate_size,
             num_layers=cfg.num_layers, num_attention_heads=cfg.num_attention_heads,
             num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim, rms_norm_eps=cfg.rms_norm_eps)
    om = orc.Model(c, w, inv, att, orc.F16, position + tokens + 1)
    tok = 1
    om.step(tok, position)  # page in the weights once
    t0 = time.perf_counter()
    for i in range(tokens):
        tok, _ = om.step(tok, position + 1 + i)
    dt = time.perf_counter() - t0
    return dict(value=round(tokens / dt, 4), unit="tokens/s", cores=orc.num_threads(), kind="port",
                sample=f"{tokens} decode tokens of the same int8 model (all 32 layers + lm_head + argmax) at "
                       f"positions {position + 1}..{position + tokens}, fp64-accumulating C oracle, "
                       f"{orc.num_threads()} OpenMP threads")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="timed decode steps (generated tokens)")
    ap.add_argument("--warmup", type=int, default=8, help="untimed decode steps before the timed region")
    ap.add_argument("--ctx", type=int, default=2048, help="prefilled KV-cache length")
    ap.add_argument("--profile-rounds", type=int, default=4,
                    help="passes over all layers when timing each kernel kind for the roofline")
    ap.add_argument("--cpu-tokens", type=int, default=2, help="tokens in the CPU baseline sample (0: skip)")
    ap.add_argument("--eager-step", action="store_true",
                    help="enqueue the decode step's kernels one by one instead of replaying its HIP graph "
                         "(same kernels; for profilers that cannot trace graph launches)")
    args = ap.parse_args()
    if args.eager_step:
        os.environ["L0H_EAGER_STEP"] = "1"  # read by the library when the model is created
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the path runs on a single GPU (no sharding or collectives "
              "in this build); run it with --gpus 1.", file=sys.stderr)
        return 2

    import l0llm_amd as l0

    cfg = llama8b()
    dev = l0.Device(0)
    copy = hbm_copy_probe(dev)
    log(f"HBM copy probe: {copy['gbs']} GB/s ({copy['bytes_per_launch']} bytes in {copy['avg_us']} us)")
    max_seq = args.ctx + args.steps + args.cpu_tokens + 8
    log(f"device {dev.name}; building the model (max_seq {max_seq})")
    model = l0.LlmModel(dev, cfg, precision=l0.PRECISION_INT8, cache_dtype=l0.F16, max_seq_len=max_seq)
    model.init_random(500, 0.02)
    prompt = np.random.default_rng(599).integers(0, cfg.vocab_size, args.ctx).astype(np.int32)

    # Warm up the captured step graph on a short prompt, then prefill the full context.
    logits = model.prefill(prompt[:8])
    if args.warmup:
        model.decode_greedy_device(int(np.argmax(logits)), args.warmup)
    t0 = time.perf_counter()
    logits = model.prefill(prompt)
    log(f"prefilled {args.ctx} tokens in {time.perf_counter() - t0:.2f} s")
    first = int(np.argmax(logits))

    dev.synchronize()
    t0 = time.perf_counter()
    toks = model.decode_greedy_device(first, args.steps)
    dev.synchronize()
    dt = time.perf_counter() - t0
    tps = args.steps / dt
    log(f"decoded {args.steps} tokens in {dt * 1e3:.2f} ms: {tps:.1f} tokens/s; first ids {toks[:8].tolist()}")

    pos = model.position
    table = kernel_table(model, pos, args.profile_rounds)
    gemv_us = sum(table[k]["avg_us"] * table[k]["launches_per_step"] for k in GEMV_KINDS)
    gemv_bytes = sum(table[k]["bytes_per_launch"] * table[k]["launches_per_step"] for k in GEMV_KINDS)
    launches = sum(table[k]["launches_per_step"] for k in GEMV_KINDS)
    achieved = gemv_bytes / (gemv_us * 1e-6) / 1e9
    step_bytes = sum(t["bytes_per_launch"] * t["launches_per_step"] for t in table.values())
    traffic = None
    tf = ROOT / "profiles" / "gemv_i8_traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("hbm_bytes_per_launch")
    log(f"int8 GEMV: {achieved:.0f} GB/s over {launches} launches/step ({gemv_us:.0f} us/step)")

    cpu = None
    if args.cpu_tokens > 0:
        log("CPU baseline: exporting the model and running the oracle")
        cpu = cpu_baseline(model, cfg, args.cpu_tokens, pos)
        log(f"CPU baseline {cpu['value']} tokens/s on {cpu['cores']} threads")

    line = {
        "metric": METRIC,
        "value": round(tps, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: random-init N(0,0.02) weights quantized to int8 per output row, seeded random prompt ids",
        "config": {"workload": f"llama3.1-8b-shaped int8 weight-only greedy decode, batch 1, "
                               f"{args.ctx}-token prefilled KV cache (fp16), {args.steps} generated tokens",
                   "layers": 32, "hidden": 4096, "intermediate": 14336, "heads": 32, "kv_heads": 8,
                   "head_dim": 128, "vocab": 128256, "batch": 1, "ctx": args.ctx,
                   "step": "eager launches" if args.eager_step else "HIP graph replay"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "gemv_nk_kernel<I8PC> (q|k|v, O, gate|up, down, lm_head)",
                     "bytes_per_launch": round(gemv_bytes / launches), "avg_us_per_launch": round(gemv_us / launches, 3)},
        "step_roofline": {"bytes_per_step": round(step_bytes), "ideal_tokens_per_s": round(HBM_PEAK_GBS * 1e9 / step_bytes, 1),
                          "frac": round(tps * step_bytes / (HBM_PEAK_GBS * 1e9), 4)},
        "kernels": table,
        "hbm_copy_probe": copy,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    model.dispose()
    dev.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
