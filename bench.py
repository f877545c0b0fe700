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
  cpu_baseline  the CPU restatements (fp32-accumulating vectorised C, and the fp64 check loop)
                running the same model's decode steps and the int8 GEMV 896 -> 4864 on the host
                cores, all cores and one core, for a bounded sample
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


COLD_BYTES = 640 << 20  # replicas per timed pass: well past the 256 MB Infinity Cache
MFMA_BF16_PEAK_TFLOPS = 2500.0


def _replicated(dev, block: np.ndarray, nbytes_each: int, count: int):
    """One device buffer holding `count` replicas of a `nbytes_each`-byte operand, filled by
    tiling `block` (the data only has to be finite; distinct addresses keep the cache cold)."""
    import l0llm_amd as l0

    raw = np.ascontiguousarray(block).view(np.uint8).reshape(-1)
    one = np.resize(raw, nbytes_each)
    buf = dev.alloc(nbytes_each * count)
    buf.write(one)
    suite = l0.LlmKernelSuite(dev)
    done = 1
    while done < count:  # doubling device copies
        n = min(done, count - done)
        suite.copy_execute(buf.ptr, buf.ptr + done * nbytes_each, 0, n * nbytes_each // 4)
        done += n
    dev.synchronize()
    return buf


def _replay_us(dev, enqueue, launches: int, reps: int = 5) -> float:
    """Records `enqueue` (which issues `launches` kernels) as one command list, runs it once, then
    replays it back to back: mean device microseconds per launch. With --eager-step (profiler
    runs, whose kernel trace faults inside hipGraphLaunch) the launches are issued directly and
    timed on the host clock; the profiler's own kernel durations are the figures then."""
    if os.environ.get("L0H_EAGER_STEP") == "1":
        enqueue()
        dev.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            enqueue()
        dev.synchronize()
        return (time.perf_counter() - t0) * 1e6 / (reps * launches)
    dev.begin_recording()
    try:
        enqueue()
    except Exception:
        dev.abort_recording()
        raise
    dev.end_recording()
    return dev.replay_recording(reps) * 1e3 / launches


def measure_configs(dev) -> dict:
    """The other workloads of the path, timed on the device (cold weights / KV, graph replay of
    back-to-back launches): int8 GEMV 896->4864 with fp16 I/O; the Qwen2.5-0.5B decode linears
    in int8 and fp16; the Llama-3.2-1B prefill GEMMs in bf16 on MFMA; GQA decode attention."""
    import l0llm_amd as l0

    suite = l0.LlmKernelSuite(dev)
    rng = np.random.default_rng(7)
    out = {}

    def gemv_case(name, wdt, n, k, x_dt=l0.F16, y_dt=l0.F16):
        wsize = 1 if wdt == l0.I8PC else 2
        wbytes = n * k * wsize
        reps = max(2, min(512, -(-COLD_BYTES // wbytes)))
        if wdt == l0.I8PC:
            wblock = rng.integers(-127, 128, size=min(n * k, 1 << 22), dtype=np.int8)
        else:
            wblock = (rng.standard_normal(min(n * k, 1 << 22), dtype=np.float32) * 0.02).astype(np.float16)
        w = _replicated(dev, wblock, wbytes, reps)
        sblock = rng.uniform(1e-3, 1e-2, n).astype(np.float16)
        sc = _replicated(dev, sblock, 2 * n, reps) if wdt == l0.I8PC else None
        x = dev.alloc_shared(rng.standard_normal(k).astype(np.float16 if x_dt == l0.F16 else np.float32))
        y = dev.alloc(n * 4)

        def run(count, cold=True):
            for i in range(count):
                j = i % reps if cold else 0
                suite.gemv_nk(wdt, 1, n, k, x, x_dt, w.ptr + j * wbytes, None if sc is None else sc.ptr + j * 2 * n,
                              y, y_dt)

        cold_us = _replay_us(dev, lambda: run(reps), reps)
        hot_us = _replay_us(dev, lambda: run(64, cold=False), 64)
        xb = 2 if x_dt == l0.F16 else 4
        nbytes = wbytes + (2 * n if wdt == l0.I8PC else 0) + k * xb + n * (2 if y_dt == l0.F16 else 4)
        for b in (w, sc, x, y):
            if b is not None:
                b.free()
        out[name] = dict(n=n, k=k, w="int8-per-row" if wdt == l0.I8PC else "fp16", bytes=nbytes,
                         us=round(cold_us, 3), gbs=round(nbytes / cold_us / 1e3, 1),
                         frac=round(nbytes / cold_us / 1e3 / HBM_PEAK_GBS, 4), hot_us=round(hot_us, 3))

    # int8 GEMV 896 -> 4864, fp16 activations in and out (Qwen2.5-0.5B up-proj shape)
    gemv_case("int8_gemv_896x4864_fp16io", l0.I8PC, 4864, 896)
    # Qwen2.5-0.5B decode linears, M = 1 (gate|up measured as one 896 -> 9728 GEMV)
    for wdt, tag in ((l0.I8PC, "int8"), (l0.F16, "fp16")):
        for name, n, k in (("qkv", 1152, 896), ("o", 896, 896), ("gate_up", 9728, 896), ("down", 896, 4864),
                           ("lm_head", 151936, 896)):
            gemv_case(f"qwen05b_{tag}_{name}", wdt, n, k)

    # The reference-layout fp16 GEMV (Gemv.Execute, W as [K, N], fp32 x and y), which an unchanged
    # LlmMatrix.Project reaches for fp16 storage: the int8 GEMV's 896 -> 4864 shape and the
    # Qwen2.5-0.5B linears, next to the [N, K] kernel at the same shapes (vs_nk = kn / nk time).
    def kn_case(name, n, k):
        wbytes = n * k * 2
        reps = max(2, min(512, -(-COLD_BYTES // wbytes)))
        wblock = (rng.standard_normal(min(n * k, 1 << 22), dtype=np.float32) * 0.02).astype(np.float16)
        w = _replicated(dev, wblock, wbytes, reps)
        x = dev.alloc_shared(rng.standard_normal(k).astype(np.float32))
        y = dev.alloc(n * 4)
        suite.gemv_execute(n, k, x, w, y)  # sizes the K-slice workspace before recording

        def run(count, cold=True):
            for i in range(count):
                suite.gemv_execute(n, k, x, w.ptr + (i % reps if cold else 0) * wbytes, y)

        cold_us = _replay_us(dev, lambda: run(reps), reps)
        hot_us = _replay_us(dev, lambda: run(64, cold=False), 64)
        nbytes = wbytes + k * 4 + n * 4
        for b in (w, x, y):
            b.free()
        nk = out.get(f"qwen05b_fp16_{name}") if name != "up_896x4864" else None
        out[f"fp16_gemv_kn_{name}"] = dict(
            n=n, k=k, w="fp16 [K,N]", bytes=nbytes, us=round(cold_us, 3), gbs=round(nbytes / cold_us / 1e3, 1),
            frac=round(nbytes / cold_us / 1e3 / HBM_PEAK_GBS, 4), hot_us=round(hot_us, 3),
            vs_nk=round(cold_us / nk["us"], 3) if nk else None)

    gemv_case("fp16_gemv_nk_up_896x4864", l0.F16, 4864, 896, x_dt=l0.F32, y_dt=l0.F32)
    kn_case("up_896x4864", 4864, 896)
    out["fp16_gemv_kn_up_896x4864"]["vs_nk"] = round(
        out["fp16_gemv_kn_up_896x4864"]["us"] / out["fp16_gemv_nk_up_896x4864"]["us"], 3)
    for name, n, k in (("qkv", 1152, 896), ("o", 896, 896), ("gate_up", 9728, 896), ("down", 896, 4864),
                       ("lm_head", 151936, 896)):
        kn_case(name, n, k)

    # Llama-3.2-1B prefill GEMMs, bf16 operands, fp32 accumulation on MFMA, bf16 out
    for m in (128, 512):
        for name, n, k in (("qkv", 3072, 2048), ("o", 2048, 2048), ("gate_up", 16384, 2048), ("down", 2048, 8192)):
            wbytes = 2 * n * k
            reps = max(2, min(64, -(-COLD_BYTES // wbytes)))
            wblock = (rng.standard_normal(1 << 22, dtype=np.float32) * 0.02).astype(np.float16)
            w = _replicated(dev, wblock, wbytes, reps)  # bf16 bits from fp16 bits: finite values suffice
            x = dev.alloc_shared(rng.standard_normal(m * k).astype(np.float16))
            y = dev.alloc(2 * m * n)
            suite.gemm_nk(l0.BF16, m, n, k, x, w, y, l0.BF16)  # sizes the split-K workspace before recording
            us = _replay_us(dev, lambda: [suite.gemm_nk(l0.BF16, m, n, k, x, w.ptr + i * wbytes, y, l0.BF16)
                                          for i in range(reps)], reps)
            flops = 2.0 * m * n * k
            nbytes = 2 * (k * n + m * k + m * n)
            tf = flops / us / 1e6
            out[f"llama1b_prefill_bf16_m{m}_{name}"] = dict(
                m=m, n=n, k=k, us=round(us, 3), tflops=round(tf, 2), mfma_frac=round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                gbs=round(nbytes / us / 1e3, 1), hbm_frac=round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4))
            for b in (w, x, y):
                b.free()

    # GQA decode attention 32 q / 8 kv heads, head_dim 128, fp16 q/K/V/out, fp32 softmax
    hd, nh, nkv = 128, 32, 8
    kvblock = rng.standard_normal(1 << 22).astype(np.float16)
    for ctx in (512, 4096, 32768):
        for batch in (1, 8):
            cbytes = batch * ctx * nkv * hd * 2
            reps = max(1, min(128, -(-COLD_BYTES // (2 * cbytes))))
            kc = _replicated(dev, kvblock, cbytes, reps)
            vc = _replicated(dev, kvblock, cbytes, reps)
            q = dev.alloc_shared(rng.standard_normal(batch * nh * hd).astype(np.float16))
            o = dev.alloc(batch * nh * hd * 2)

            def attn(i):
                suite.attention_decode(q, l0.F16, kc.ptr + i * cbytes, vc.ptr + i * cbytes, l0.F16, o, l0.F16, batch,
                                       hd, nh, nkv, ctx, ctx)

            attn(0)  # sizes the split workspace before recording
            launches = max(reps, 4)
            us = _replay_us(dev, lambda: [attn(i % reps) for i in range(launches)], launches)
            nbytes = 2 * cbytes + 2 * 2 * batch * nh * hd
            out[f"gqa_attention_ctx{ctx}_b{batch}"] = dict(
                ctx=ctx, batch=batch, bytes=nbytes, us=round(us, 3), gbs=round(nbytes / us / 1e3, 1),
                frac=round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4))
            for b in (kc, vc, q, o):
                b.free()
    return out


def _median_s(fn, runs: int) -> float:
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def greedy_ids_check(model, om, cfg, ctx: int, first: int, ids, count: int) -> dict:
    """The timed run's first `count` greedy ids against the oracle: the oracle's caches are seeded
    with the device's rows 0 .. ctx - 1 (the prefilled prompt), then it runs the same tokens at the
    same positions (teacher-forced with the device's ids). An id may differ only where the oracle's
    own top-2 gap is below 1e-2 of max|logit|: twice the 5e-3 that the device's fp16 storage of the
    attention and SwiGLU outputs is allowed to move the logits over 32 layers (a tie, not a bug)."""
    import l0llm_amd as l0
    from oracle import pyoracle as orc

    kv_bytes = ctx * cfg.num_key_value_heads * cfg.head_dim * 2
    for layer in range(cfg.num_layers):
        kp, vp = model.kv_cache(layer)
        om.load_cache(layer, l0.Buffer(model.device, kv_bytes, ptr=kp, owned=False).read(np.uint8),
                      l0.Buffer(model.device, kv_bytes, ptr=vp, owned=False).read(np.uint8))
    tok, equal, flips = first, 0, 0
    for i in range(count):
        onext, olg = om.step(tok, ctx + i)
        got = int(ids[i])
        if got == onext:
            equal += 1
        elif orc.top2_margin(olg) < 1e-2 * float(np.max(np.abs(olg))):
            flips += 1
        tok = got
    return dict(checked=count, equal=equal, tie_flips=flips, match=equal + flips == count,
                oracle="fp64 C restatement, caches seeded with the device's prefill rows, teacher-forced")


def export_weights(model, cfg) -> dict:
    """The model's weights as the device holds them, in HuggingFace names and order: projections as
    (storage, int8 [N, K], fp16 scales), vectors as fp32 (read back through the ABI)."""
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
    return w


def dropin_path(dev, model, cfg, w: dict, ctx: int, first: int, next_id: int, reps: int = 20, tokens: int = 5) -> dict:
    """The reference's own decode step on this library's operator entry points (the drop-in path:
    an unchanged LlmModel.Step over LlmDecoderLayer.Forward / MixFull, l0llm_amd.reference_step),
    with the same weights (separate q, k, v, gate and up matrices in the int8 weight-only format),
    a copy of the model's prefilled caches and fp32 activations between operators. Timed as one
    recorded token replayed back to back (replay), recorded afresh per token as Step does
    (record_per_token, host clock, the sampled id read back each token), and issued without
    recording (eager, host clock); checked against the model's greedy id at position ctx."""
    from l0llm_amd.reference_step import ReferenceStep

    ref = ReferenceStep(dev, cfg, w, model.max_seq_len, [model.kv_cache(i) for i in range(cfg.num_layers)])
    try:
        ref.set_token(first, ctx)
        ref.record_step(ctx)  # runs it once
        launches = dev.recording_launches
        picked, dl = ref.read_sampled(), ref.read_logits()
        replay_ms = dev.replay_recording(reps)
        t0 = time.perf_counter()
        for i in range(tokens):
            ref.set_token(first, ctx + i)
            ref.record_step(ctx + i)
            ref.read_sampled()
        rec_s = (time.perf_counter() - t0) / tokens
        t0 = time.perf_counter()
        for i in range(tokens):
            ref.set_token(first, ctx + i)
            ref.step(ctx + i)
            ref.read_sampled()
        eager_s = (time.perf_counter() - t0) / tokens
    finally:
        ref.close()
    ml = model.compute_logits(first, ctx)  # the model's own step at the same position and token
    rel = float(np.max(np.abs(dl - ml)) / np.max(np.abs(ml)))
    return dict(
        launches_per_step=launches, operators_per_step=18 * cfg.num_layers + 5,
        replay=dict(ms_per_token=round(replay_ms, 4), tokens_per_s=round(1000.0 / replay_ms, 1), reps=reps),
        record_per_token=dict(ms_per_token=round(rec_s * 1e3, 3), tokens_per_s=round(1.0 / rec_s, 1), tokens=tokens),
        eager=dict(ms_per_token=round(eager_s * 1e3, 3), tokens_per_s=round(1.0 / eager_s, 1), tokens=tokens),
        greedy_id=picked, greedy_id_match=picked == next_id, logits_rel_to_model=round(rel, 6),
        path="reference operator sequence (LlmDecoderLayer.Forward / MixFull, LlmModel.Step) on l0h_*_execute entry "
             "points: int8 weight-only GemvQ8 with fp32 activations, fp16 KV cache, split-K attention")


def cpu_baseline(model, cfg, tokens: int, position: int, ids_check=None, w: dict | None = None) -> dict:
    """The CPU restatements timed on this host's cores: the fp64 check loop (the reference's own CPU
    matmul semantics, LlmMatrixTests.cs:71-80) and an fp32-accumulating, vectorised, OpenMP form of the
    same operations; all cores and one core. The int8 GEMV 896 -> 4864 is the median of 21 runs per
    form; the 8B decode steps are the median over `tokens` steps per form and core count (at least 8),
    so the whole leg stays around a minute. ids_check = (ctx, first, ids, count): before timing, the
    same model's oracle checks the timed run's first greedy ids (greedy_ids_check)."""
    from oracle import pyoracle as orc

    all_cores = orc.num_threads()
    # int8 GEMV 896 -> 4864: int8 weights uniform in [-127, 127], fp16 scales U[1e-3, 1e-2], x ~ N(0, 1)
    rng = np.random.default_rng(101)
    q = rng.integers(-127, 128, (4864, 896), dtype=np.int8)
    sc = rng.uniform(1e-3, 1e-2, 4864).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(896).astype(np.float16).astype(np.float32)
    gemv = {}
    for label, fn in (("fp64_check_loop", orc.gemv_nk), ("fp32_vectorised", orc.gemv_nk_f32acc)):
        for cores in (all_cores, 1):
            orc.set_threads(cores)
            fn(orc.I8PC, q, x, sc)
            t = _median_s(lambda: fn(orc.I8PC, q, x, sc), 21)
            gemv[f"{label}_{cores}_cores"] = dict(us=round(t * 1e6, 1), gbs=round(4379392 / t / 1e9, 2))
    orc.set_threads(all_cores)

    H = cfg.hidden_size
    if w is None:
        w = export_weights(model, cfg)
    inv, att = orc.rope_frequencies(cfg.head_dim, cfg.rope_theta, cfg.max_position_embeddings)
    c = dict(vocab_size=cfg.vocab_size, hidden_size=H, intermediate_size=cfg.intermediate_size,
             num_layers=cfg.num_layers, num_attention_heads=cfg.num_attention_heads,
             num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim, rms_norm_eps=cfg.rms_norm_eps)
    om = orc.Model(c, w, inv, att, orc.F16, position + 3 * tokens + 8)
    ids = greedy_ids_check(model, om, cfg, *ids_check) if ids_check else None
    pos = [position]

    def step():
        om.step(1, pos[0])
        pos[0] += 1

    steps = {}
    orc.set_fast_projections(True)
    step()  # pages the weights in
    for cores in (all_cores, 1):
        orc.set_threads(cores)
        t = _median_s(step, tokens)
        steps[f"fp32_vectorised_{cores}_cores"] = dict(tokens_per_s=round(1 / t, 4), tokens=tokens)
    orc.set_threads(all_cores)
    orc.set_fast_projections(False)
    t = _median_s(step, tokens)
    steps[f"fp64_check_loop_{all_cores}_cores"] = dict(tokens_per_s=round(1 / t, 4), tokens=tokens)
    value = steps[f"fp32_vectorised_{all_cores}_cores"]["tokens_per_s"]
    return dict(value=value, unit="tokens/s", cores=all_cores, kind="port",
                sample=f"median decode step of the same int8 Llama-3.1-8B-shaped model (32 layers + lm_head + "
                       f"argmax, positions from {position}) over {tokens} steps: the fp32-accumulating vectorised "
                       f"C restatement on {all_cores} OpenMP threads; the other forms and core counts below",
                step=steps, gemv_int8_896x4864=gemv, cpu_model=host_cpu_model(),
                host_cpus=len(os.sched_getaffinity(0)), nproc=os.cpu_count(), greedy_ids=ids)


def host_cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="timed decode steps (generated tokens)")
    ap.add_argument("--warmup", type=int, default=8, help="untimed decode steps before the timed region")
    ap.add_argument("--ctx", type=int, default=2048, help="prefilled KV-cache length")
    ap.add_argument("--profile-rounds", type=int, default=4,
                    help="passes over all layers when timing each kernel kind for the roofline")
    ap.add_argument("--cpu-tokens", type=int, default=8,
                    help="decode steps per form and core count in the CPU baseline (its median; 0: skip the CPU "
                         "baseline and the greedy-id check)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-configuration kernel measurements (GEMV, prefill GEMM, attention)")
    ap.add_argument("--no-dropin", action="store_true",
                    help="skip the reference operator sequence on the operator entry points (the drop-in path)")
    ap.add_argument("--eager-step", action="store_true",
                    help="enqueue the decode step's kernels one by one instead of replaying its HIP graph "
                         "(same kernels; for profilers that cannot trace graph launches)")
    args = ap.parse_args()
    if args.eager_step:
        os.environ["L0H_EAGER_STEP"] = "1"  # read by the library when the model is created
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the path runs on a single GPU (no sharding or collectives "
              "are implemented); run it with --gpus 1.", file=sys.stderr)
        return 2

    import l0llm_amd as l0

    cfg = llama8b()
    dev = l0.Device(0)
    copy = hbm_copy_probe(dev)
    read_gbs = dev.read_bandwidth(2 << 30, 10)
    copy["read_stream_gbs"] = round(read_gbs, 1)
    copy["read_stream_kernel"] = "read_stream_kernel (16-byte non-temporal loads over 2 GiB, best of 3 launch shapes)"
    log(f"HBM probes: streaming read {read_gbs:.0f} GB/s; copy {copy['gbs']} GB/s ({copy['bytes_per_launch']} bytes "
        f"read + written in {copy['avg_us']} us)")
    max_seq = args.ctx + args.steps + args.cpu_tokens + 8
    log(f"device {dev.name}; building the model (max_seq {max_seq})")
    model = l0.LlmModel(dev, cfg, precision=l0.PRECISION_INT8, cache_dtype=l0.F16, max_seq_len=max_seq)
    model.init_random(500, 0.02)
    prompt = np.random.default_rng(599).integers(0, cfg.vocab_size, args.ctx).astype(np.int32)

    # Warm up the captured step graph on a short prompt and the prefill kernels on one full prefill
    # (their first launches load code objects), then time three prefills of the full context (each
    # starts a new sequence); the cache holds the prompt afterwards.
    logits = model.prefill(prompt[:8])
    if args.warmup:
        model.decode_greedy_device(int(np.argmax(logits)), args.warmup)
    model.prefill(prompt)
    runs = []
    for _ in range(3):
        t0 = time.perf_counter()
        logits = model.prefill(prompt)  # returns after the logits are read back
        runs.append(time.perf_counter() - t0)
    pf_s = min(runs)
    log(f"prefilled {args.ctx} tokens in {pf_s:.3f} s ({args.ctx / pf_s:.0f} tokens/s; runs "
        + ", ".join(f"{r:.4f}" for r in runs) + " s)")
    prefill = {"tokens": args.ctx, "s": round(pf_s, 4), "tokens_per_s": round(args.ctx / pf_s, 1),
               "runs_s": [round(r, 4) for r in runs],
               "path": "chunks of 2048 tokens: int8 weights dequantized to fp16 on MFMA, query-tiled causal "
                       "attention; the last token through the decode step; host clock around the call, best "
                       "of 3 after a warm-up prefill"}
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
    for t in table.values():  # the same rates against the read ceiling measured on this box
        t["frac_of_read_ceiling"] = round(t["gbs"] / read_gbs, 4) if read_gbs > 0 else None
    step_bytes = sum(t["bytes_per_launch"] * t["launches_per_step"] for t in table.values())
    # HBM bytes per int8 GEMV launch from the rocprofv3 FETCH_SIZE / WRITE_SIZE runs (calibrated
    # against the copy kernel of known size), summarised in profiles/.
    traffic = None
    tf = ROOT / "profiles" / "gemv_int8_hbm_traffic.txt"
    if tf.exists():
        for line in tf.read_text().splitlines():
            if line.startswith("hbm_bytes_per_launch:"):
                traffic = int(line.split(":", 1)[1])
    log(f"int8 GEMV: {achieved:.0f} GB/s over {launches} launches/step ({gemv_us:.0f} us/step)")

    configs = None
    if not args.no_configs:
        log("timing the per-configuration kernels")
        configs = measure_configs(dev)

    weights = export_weights(model, cfg) if (args.cpu_tokens > 0 or not args.no_dropin) else None
    dropin = None
    if not args.no_dropin:
        log("drop-in path: the reference's operator sequence on the operator entry points")
        dropin = dropin_path(dev, model, cfg, weights, args.ctx, first, int(toks[0]))
        log(f"drop-in path: {dropin['replay']['tokens_per_s']} tokens/s replayed, {dropin['launches_per_step']} launches "
            f"per token; greedy id match {dropin['greedy_id_match']}")

    cpu = None
    if args.cpu_tokens > 0:
        log("CPU baseline: running the oracle")
        cpu = cpu_baseline(model, cfg, args.cpu_tokens, pos,
                           ids_check=(args.ctx, first, toks, min(8, args.steps)), w=weights)
        log(f"CPU baseline {cpu['value']} tokens/s on {cpu['cores']} threads; greedy ids {cpu['greedy_ids']}")

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
                   "step": {"graph": "HIP graph replay", "eager": "eager launches"}[model.step_path]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "gemv_nk_kernel<I8PC> (q|k|v, O, gate|up, down, lm_head)",
                     "bytes_per_launch": round(gemv_bytes / launches), "avg_us_per_launch": round(gemv_us / launches, 3),
                     "frac_of_read_ceiling": round(achieved / read_gbs, 4) if read_gbs > 0 else None,
                     "read_ceiling_gbs": round(read_gbs, 1)},
        "step_roofline": {"bytes_per_step": round(step_bytes), "ideal_tokens_per_s": round(HBM_PEAK_GBS * 1e9 / step_bytes, 1),
                          "frac": round(tps * step_bytes / (HBM_PEAK_GBS * 1e9), 4)},
        "kernels": table,
        "hbm_probe": copy,
        "prefill": prefill,
        "configs": configs,
        "cpu_baseline": cpu,
        "greedy_ids_match": cpu["greedy_ids"]["match"] if cpu else None,
        "dropin": dropin,
        "step_launches": model.step_launches,
    }
    print(json.dumps(line), flush=True)
    model.dispose()
    dev.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
