"""Benchmark: Qwen3-30B-A3B-shaped Q4_K_M batch-1 decode on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]
    python bench.py --only 0|1|3|4 [--steps K] one of the other configs alone (profiling)
    python bench.py --only cache [--cache-frac F] configs[2]'s decode through the expert cache
    python bench.py --only prompt                 a 4096-token prompt through configs[2]'s model
    python bench.py --only prompt-abi             the same prompt layer by layer through the ABI (model.c's path)

Workload: a full 48-layer Qwen3-30B-A3B-shaped model
with seeded random weights (Q4_K gate/up/q/k/o, Q6_K down/v/LM head, Q4_K
embedding, F32 router), a float32 key-value cache prefilled with N(0,1) at
positions 0..2047, and one new token at position 2048 per step. A step is one
whole device-resident decode step: embedding, 48 layers (attention, router and
top-k on the device, 8 experts), LM head; logits left in HBM. All weights and
the cache are resident in HBM before the timed region.

Prints one JSON line. Besides the step throughput it carries:
  roofline: the dominant kernel (the experts' gate/up GEMV) timed with HIP
            events on the model's stream, its algorithmic bytes per launch, the
            achieved GB/s against the 8 TB/s HBM peak;
  copy_probe_GBps: a plain device copy, what streaming reaches on this box;
  cpu_baseline: the CPU checker's decode step (the reference's CPU arithmetic
            restated, oracle/) on this host, single-threaded, over a bounded
            number of tokens; cpu_baseline_mt the same with each matrix's rows
            split over up to 16 host threads;
  configs:  the other BASELINE workloads measured on the same device (unless
            --no-extra): configs[3], 32 sequences of one new token each at
            key-value lengths drawn from U{128..8192}, one rows step (device
            routing, experts grouped so each chosen expert is read once a
            layer); configs[4], a prefill of 4096 rows through one
            Qwen3-shaped MoE layer with Q8_0 experts (bf16 MFMA grouped GEMM),
            with the matrix cores' yardstick (back-to-back MFMAs) beside it;
            configs[0] and [1], one MoE layer of one token; prompt, a
            4096-token prompt through configs[2]'s whole model in passes
            of 1024 rows, exact and --precision fast; expert_cache,
            configs[2]'s model decoded a layer at a time through the
            reference's ABI with every expert resident and with a cache
            holding half of them (copied in from host memory).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "vitna-anchor_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "Qwen3-30B-A3B Q4_K_M decode tok/s @1 GPU; expert GEMV HBM GB/s (% of peak)"
# The committed rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE passes, each scaled by its factor calibrated on
# copy_probe_kernel) that roofline.traffic is read from.
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_step_qwen3_hbm_traffic.md")
KERNELS = {0: "experts_in (gate/up + SiLU)", 1: "experts_down (+ weighted sum)", 2: "route (norm + router + top-k)",
           3: "q/k/v projections", 4: "attention (+ merge and o-projection)", 5: "o-projection alone (GEMV)", 6: "LM head",
           7: "route without top-k", 8: "routing rule alone (1 block)", 9: "tiny launch (floor)"}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--no-extra", action="store_true", help="measure configs[2] only")
    ap.add_argument("--only", choices=["0", "1", "3", "4", "4k", "cache", "prompt", "prompt-abi"],
                    help="run one of the other configs alone (profiling), or the expert cache's decode, and print its object")
    ap.add_argument("--cache-frac", type=float, default=0.5, help="--only cache: the share of the experts the cache holds")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every GPU box here has one GPU). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import vitna_amd as va

    if args.only:
        if args.only in ("0", "1"):
            res = bench_layer(va, int(args.only), reps=args.steps)
        elif args.only == "4k":
            res = bench_prefill_kquant(va, reps=args.steps)
        elif args.only == "4":
            res = bench_prefill(va, reps=args.steps)
        elif args.only == "cache":
            res = bench_cache(va, args.steps, args.warmup, args.cache_frac, args.layers)
        elif args.only in ("prompt", "prompt-abi"):
            model = va.Model(va.shape(n_layers=args.layers, ctx=4096, seqs=1, kv_host=0), 20260101, threads=16)
            res = bench_prompt(va, model) if args.only == "prompt" else bench_prompt_abi(va, model)
            model.free()
        else:
            model = va.Model(va.shape(n_layers=args.layers, ctx=8193, seqs=32, kv_host=0), 20260101, threads=16)
            dev = va.Device(model)
            res = bench_ragged(va, model, dev, args.steps, reps=args.steps)
            dev.close()
            model.free()
        print(json.dumps({"configs": {args.only: res}}), flush=True)
        return

    pos, token = 2048, 1234
    t0 = time.time()
    # 32 sequences of up to 8193 positions serve configs[3]; configs[2] uses sequence 0 (the host cache is
    # allocated lazily: only what is written is committed)
    shp = va.shape(n_layers=args.layers, ctx=8193, seqs=32, kv_host=1)
    model = va.Model(shp, 20260101, threads=16)
    cfg = model.cfg
    kd = cfg.n_kv_heads * cfg.head_dim
    L = cfg.n_layers
    kc = np.ctypeslib.as_array(model.m.k_cache, shape=(L, model.m.ctx, kd))  # sequence 0
    vc = np.ctypeslib.as_array(model.m.v_cache, shape=(L, model.m.ctx, kd))
    for l in range(L):
        kc[l, :pos] = va.normal(7, 2 * l, pos * kd).reshape(pos, kd)
        vc[l, :pos] = va.normal(7, 2 * l + 1, pos * kd).reshape(pos, kd)
    log("synthetic model generated in %.1f s" % (time.time() - t0))
    t0 = time.time()
    # configs[2]'s device model holds one sequence of pos + 1 positions (the attention grid is sized by the
    # cache); the host model keeps its layout for the CPU baseline
    saved = (model.m.ctx, model.m.seqs)
    model.m.ctx, model.m.seqs = pos + 1, 1
    try:
        dev = va.Device(model)
    finally:
        model.m.ctx, model.m.seqs = saved
    for l in range(L):
        dev.kv(0, l, 0, pos, kc[l, :pos], vc[l, :pos])
    log("uploaded to %s in %.1f s" % (dev.device_name(), time.time() - t0))

    # The library links the image's HIP runtime; torch bundles another, so torch is not loaded in this process.
    # dev.sync() is the barrier (hipStreamSynchronize on the only stream the model uses).
    for _ in range(args.warmup):
        dev.step_async(0, token, pos)
    dev.sync()
    t_wall = time.perf_counter()
    ms = dev.time_steps(0, token, pos, args.steps)  # HIP events on the model's stream around the K steps
    dev.sync()
    wall_ms = (time.perf_counter() - t_wall) * 1000.0 / args.steps
    tok_s = 1000.0 / ms
    log("step: %.3f ms (events), %.3f ms (wall), %.1f tok/s" % (ms, wall_ms, tok_s))

    # algorithmic bytes of one step (weights and cache read once, logits written)
    per_kernel = {}
    for which in range(10):
        us, b = dev.time_kernel(which, reps=4 * L if which != 6 else 20, warmup=L)
        if which == 4:
            b = 2.0 * (pos + 1) * kd * 4 + cfg.n_heads * cfg.head_dim * 8.0
        per_kernel[which] = (us, b)
        log("  %-32s %9.2f us  %10.0f B  %7.1f GB/s" % (KERNELS[which], us, b, b / us / 1e3))
    us0, b0 = per_kernel[0]
    achieved = b0 / us0 / 1e3
    step_bytes = L * sum(per_kernel[w][1] for w in range(6)) + per_kernel[6][1]
    log("algorithmic bytes a step: %.3f GB -> %.1f GB/s over the whole step" % (step_bytes / 1e9, step_bytes / ms / 1e6))

    # the yardstick: a plain device copy of 256 MiB (reads + writes), what streaming reaches on this box
    copy_bytes = 256 << 20
    copy_us = va.copy_probe(copy_bytes, reps=10)
    copy_gbs = 2.0 * copy_bytes / copy_us / 1e3
    log("copy probe: %d MiB in %.1f us -> %.1f GB/s (read + write)" % (copy_bytes >> 20, copy_us, copy_gbs))

    cpu = cpu_mt = None
    if not args.no_cpu:
        import oracle
        n, t_cpu = 0, 0.0
        while t_cpu < args.cpu_seconds and n < 20:
            t1 = time.perf_counter()
            oracle.step(model, 0, token, pos, threads=1, trace=False)
            t_cpu += time.perf_counter() - t1
            n += 1
        host = host_info()
        cpu = {"value": round(n / t_cpu, 4), "unit": "tok/s", "cores": 1, "kind": "port",
               "sample": "%d whole decode steps of the same model and position (48 layers + head), single thread, "
                         "the reference's CPU arithmetic (AVX2 order) restated in oracle/vitna_oracle.c" % n,
               "host": host}
        log("cpu baseline: %d steps in %.1f s -> %.3f tok/s" % (n, t_cpu, n / t_cpu))
        # the same arithmetic with each matrix's rows split over the host's cores (the reference's pool pattern),
        # as many as this process may use up to 16, the CPU share a GPU box grants one GPU
        threads = max(1, min(16, host["cores_usable"]))
        n2, t2 = 0, 0.0
        while t2 < args.cpu_seconds / 2 and n2 < 40:
            t1 = time.perf_counter()
            oracle.step(model, 0, token, pos, threads=threads, trace=False)
            t2 += time.perf_counter() - t1
            n2 += 1
        cpu_mt = {"value": round(n2 / t2, 4), "unit": "tok/s", "cores": threads, "kind": "port",
                  "sample": "%d whole decode steps, rows of each matrix split over %d threads (same sums in the same "
                            "order per row); threads = the cores this process may use, capped at 16, the host share of one GPU"
                            % (n2, threads), "host": host}
        log("cpu baseline, %d threads: %d steps in %.1f s -> %.3f tok/s" % (threads, n2, t2, n2 / t2))

    dev.close()
    extra = None
    if not args.no_extra:
        t0 = time.time()
        dev = va.Device(model)
        log("uploaded for 32 sequences of 8193 positions in %.1f s" % (time.time() - t0))
        extra = {"3": bench_ragged(va, model, dev, args.steps)}
        dev.close()
        extra["prompt"] = bench_prompt(va, model)
        extra["4"] = bench_prefill(va)
        extra["4_kquant"] = bench_prefill_kquant(va)
        extra["0"] = bench_layer(va, 0)
        extra["1"] = bench_layer(va, 1)
        extra["expert_cache"] = bench_cache(va, 8, 2, 0.5, L, model, kc, vc)

    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 (Q4_K/Q6_K weights widened, fp32 accumulate)", "data": "synthetic",
        "config": {"workload": "BASELINE configs[2]: Qwen3-30B-A3B-shaped full decode step, batch 1, Q4_K_M, "
                               "48 layers, KV 2048 positions fp32, LM head Q6_K 151936x2048",
                   "layers": L, "position": pos, "global_batch": 1},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profile_traffic(TRAFFIC_PROFILE, "experts_in_kernel<17,"),
                     "kernel": "experts_in_kernel<Q4_K> (8 experts x (gate + up) 768 x 2048)",
                     "bytes_per_launch": b0, "avg_us": round(us0, 3)},
        "kernels_us": {KERNELS[w]: round(per_kernel[w][0], 3) for w in per_kernel},
        "step_algorithmic_GBps": round(step_bytes / ms / 1e6, 1),
        "copy_probe_GBps": round(copy_gbs, 1),
        "cpu_baseline": cpu,
        "cpu_baseline_mt": cpu_mt,
        "configs": extra,
    }
    print(json.dumps(out), flush=True)
    model.free()


def profile_traffic(path, kernel):
    """HBM bytes a launch of the kernel whose name contains `kernel` moves, from a committed --pmc summary: the
    table row's scaled bytes read plus bytes written (columns 'bytes read (scaled)', 'bytes written (scaled)').
    None when the file or the row is missing."""
    try:
        with open(path) as f:
            lines = f.read().splitlines()
    except OSError:
        return None
    head = None
    for ln in lines:
        if not ln.startswith("|"):
            continue
        cells = [c.strip() for c in ln.strip().strip("|").split("|")]
        if head is None and "bytes read (scaled)" in cells:
            head = cells
            continue
        if head and cells and kernel in cells[0].replace(" ", ""):
            try:
                return int(cells[head.index("bytes read (scaled)")]) + int(cells[head.index("bytes written (scaled)")])
            except (ValueError, IndexError):
                return None
    return None


def host_info():
    """The host the CPU baseline ran on: CPU model, cores, compiler and C library."""
    import platform
    import subprocess
    info = {"cpu_model": "unknown", "cores_online": os.cpu_count(), "cores_usable": len(os.sched_getaffinity(0)),
            "gcc": "unknown", "glibc": "-".join(platform.libc_ver()), "oracle_flags": "-O3 -mavx2 -mfma -ffp-contract=off"}
    try:
        with open("/proc/cpuinfo") as f:
            lines = f.read().splitlines()
        pick = lambda key: next((l.split(":", 1)[1].strip() for l in lines if l.split(":")[0].strip() == key), None)
        info["cpu_model"] = pick("model name") or "unknown"
        info["cpu_family_model_stepping"] = "%s/%s/%s" % (pick("cpu family"), pick("model"), pick("stepping"))
        info["cpu_mhz"] = pick("cpu MHz")
    except OSError:
        pass
    try:
        info["gcc"] = subprocess.run(["gcc", "--version"], capture_output=True, text=True, timeout=10).stdout.splitlines()[0]
    except (OSError, IndexError, subprocess.SubprocessError):
        pass
    return info


def bench_ragged(va, model, dev, steps, reps=None):
    """32 sequences, one new token each, key-value lengths U{128..8192} (seeded), values N(0,1).
    Times max(steps / 5, 5) rows steps, or reps of them."""
    cfg = model.cfg
    rng = np.random.RandomState(20260103)
    lengths = rng.randint(128, 8193, size=32)
    t0 = time.time()
    dev.kv_fill(3, [int(n) for n in lengths])
    rows = [(int(rng.randint(0, cfg.vocab)), int(lengths[s]), s) for s in range(32)]
    ms = dev.time_rows(rows, reps if reps else max(steps // 5, 5))
    L, kd = cfg.n_layers, cfg.n_kv_heads * cfg.head_dim
    kv_bytes = float(np.sum(lengths + 1)) * kd * 4 * 2 * L
    # the distinct experts each layer reads: the same rows walked layer by layer through the reference's ABI
    # (vitna_cuda_moe_rows_route / _rows_experts), each row routed by the device's rule (vitna_hip_route_check)
    E, K = cfg.n_experts, cfg.n_experts_used
    distinct = []
    for l in range(L):
        lg = dev.rows_route(rows, l)
        ids = np.empty((len(rows), K), np.int32)
        wts = np.empty((len(rows), K), np.float32)
        for i in range(len(rows)):
            _, ids[i], wts[i] = va.route_check(lg[i], K, bool(cfg.renormalize))
        dev.rows_experts(l, ids, wts)
        distinct.append(len(np.unique(ids)))
    uniq = float(np.mean(distinct))
    expert_bytes = float(np.sum(distinct)) * (2 * 884736 + 1290240)
    log("configs[3]: %d rows, %.3f ms a step, %.1f tok/s (cache filled in %.1f s)" % (len(rows), ms, 32e3 / ms, time.time() - t0))
    return {"workload": "BASELINE configs[3]: 32 sequences, one new token each, key-value lengths U{128..8192}, "
                        "Qwen3-30B-A3B-shaped Q4_K_M, 48 layers",
            "value": round(32e3 / ms, 1), "unit": "tok/s", "ms_per_step": round(ms, 4),
            "kv_positions": int(np.sum(lengths)),
            "est_GBps": round((kv_bytes + expert_bytes + 5.2258e8 + 5.0332e7 + 2.5525e8) / ms / 1e6, 1),
            "distinct_experts": {"mean": round(uniq, 2), "min": int(min(distinct)), "max": int(max(distinct))},
            "est_note": "key-value bytes exact; expert bytes for the distinct experts each layer reads, counted "
                        "(%.1f a layer on average)" % uniq}


def bench_prompt(va, model, tokens=4096, chunk=1024):
    """A prompt of `tokens` tokens through configs[2]'s whole model (48 layers and the head), in passes of `chunk`
    rows of one sequence at consecutive positions, in a cache of `tokens` positions (model.c's default context is the
    model's, at most 4096), as model.c feeds a prompt in chunks of vitna_cuda_moe_rows_max
    (the rows step: each row's attention over the keys of the positions before it and its own, device routing,
    experts grouped), with the exact kernels and with --precision fast (a gpu_fast model: the passes' experts as
    the bf16 grouped GEMM). The last position's logits come back, as model.c asks of a prompt. Wall-clock of the
    second prompt (the first captures the graphs and makes the tiled copies)."""
    cfg = model.cfg
    out = {"workload": "a %d-token prompt through BASELINE configs[2]'s model (Qwen3-30B-A3B-shaped Q4_K_M, 48 layers), "
                       "passes of %d rows of one sequence" % (tokens, chunk),
           "context": "the reference publishes 349 (exact fp32) and 1,014 (--precision fast) tok/s for a 4,096-token "
                      "Qwen3-30B-A3B Q4_K_M prompt on an RTX 3070 with most experts in host memory (README.md:714); "
                      "other hardware, not a baseline"}
    for name, fast in (("exact", False), ("fast", True)):
        # a device model of one sequence and the context model.c gives by default (at most 4096 positions)
        saved = (model.m.ctx, model.m.seqs)
        model.m.ctx, model.m.seqs = tokens, 1
        try:
            dev = va.Device(model, fast=fast)
        finally:
            model.m.ctx, model.m.seqs = saved
        try:
            def prompt():
                for c in range(tokens // chunk):
                    rows = [((7 * (c * chunk + i) + 3) % cfg.vocab, c * chunk + i, 0) for i in range(chunk)]
                    # the last position's logits, as model.c asks of a prompt
                    dev.rows_step(rows, logits=(c == tokens // chunk - 1), only=[chunk - 1])
                dev.sync()
            prompt()
            t = time.perf_counter()
            prompt()
            sec = time.perf_counter() - t
        finally:
            dev.close()
        out[name] = {"value": round(tokens / sec, 1), "unit": "tok/s", "ms": round(sec * 1e3, 1)}
        log("prompt of %d tokens, %s: %.1f ms, %.0f tok/s" % (tokens, name, sec * 1e3, tokens / sec))
    return out


def bench_prompt_abi(va, model, tokens=4096, chunk=1024):
    """The same prompt as bench_prompt, fed as model.c feeds it: layer by layer through the ABI
    (vitna_cuda_moe_rows_route, then the host's routing of every row, then vitna_cuda_moe_rows_experts;
    vitna_cuda_moe_rows_head for the last position), engine/src/model.c:1006-1030 and moe_rows_on_gpu
    :1052-1190. The host routing here is a vectorized top-k of the device's logits (largest first, ties to the
    lower index) with the softmax over the chosen (Qwen3 renormalizes), so the time is the device's and the ABI's,
    not a Python loop's. No graph is replayed, so this is the form the prompt is profiled in."""
    cfg = model.cfg
    K, L = cfg.n_experts_used, cfg.n_layers
    out = {"workload": "a %d-token prompt through BASELINE configs[2]'s model, passes of %d rows, layer by layer "
                       "through the ABI with host routing" % (tokens, chunk)}
    for name, fast in (("exact", False), ("fast", True)):
        saved = (model.m.ctx, model.m.seqs)
        model.m.ctx, model.m.seqs = tokens, 1
        try:
            dev = va.Device(model, fast=fast)
        finally:
            model.m.ctx, model.m.seqs = saved
        try:
            def prompt():
                for c in range(tokens // chunk):
                    rows = [((7 * (c * chunk + i) + 3) % cfg.vocab, c * chunk + i, 0) for i in range(chunk)]
                    for l in range(L):
                        lg = dev.rows_route(rows, l)
                        ids = np.argsort(-lg, axis=1, kind="stable")[:, :K].astype(np.int32)
                        top = np.take_along_axis(lg, ids, axis=1).astype(np.float64)
                        w = np.exp(top - top[:, :1])
                        w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
                        order = np.argsort(ids, axis=1)
                        dev.rows_experts(l, np.take_along_axis(ids, order, axis=1), np.take_along_axis(w, order, axis=1))
                    if c == tokens // chunk - 1:
                        dev.rows_head(chunk, only=[chunk - 1])
                dev.sync()
            prompt()
            t = time.perf_counter()
            prompt()
            sec = time.perf_counter() - t
        finally:
            dev.close()
        out[name] = {"value": round(tokens / sec, 1), "unit": "tok/s", "ms": round(sec * 1e3, 1)}
        log("prompt of %d tokens through the ABI, %s: %.1f ms, %.0f tok/s" % (tokens, name, sec * 1e3, tokens / sec))
    return out


def bench_cache(va, tokens, warmup, frac, layers, model=None, kc=None, vc=None):
    """configs[2]'s model decoded a layer at a time through the reference's ABI (vitna_cuda_moe_route, the host's
    routing, vitna_cuda_moe_experts with the next layer's guess, vitna_cuda_moe_head), once with every expert
    resident and once with an expert cache holding `frac` of them, copied in from page-locked host memory as the
    layers ask. Wall-clock per token (the ABI waits for the device every layer). model, kc, vc: the main bench's
    model and its sequence 0's cache (positions 0..2047 filled), or None to make them."""
    pos0 = 2048
    own = model is None
    if own:
        model = va.Model(va.shape(n_layers=layers, ctx=pos0 + warmup + tokens + 1, seqs=1, kv_host=1), 20260101, threads=16)
    cfg = model.cfg
    L, K, E = cfg.n_layers, cfg.n_experts_used, cfg.n_experts
    kd = cfg.n_kv_heads * cfg.head_dim
    if own:
        kc = np.ctypeslib.as_array(model.m.k_cache, shape=(L, model.m.ctx, kd))
        vc = np.ctypeslib.as_array(model.m.v_cache, shape=(L, model.m.ctx, kd))
        for l in range(L):
            kc[l, :pos0] = va.normal(7, 2 * l, pos0 * kd).reshape(pos0, kd)
            vc[l, :pos0] = va.normal(7, 2 * l + 1, pos0 * kd).reshape(pos0, kd)
    e0 = model.m.layers[0].experts[0]
    expert_bytes = sum(va.row_bytes(m.dtype, m.cols) * m.rows for m in (e0.gate, e0.up, e0.down))
    renorm = bool(cfg.renormalize)
    out = {}
    for name, cache in (("resident", 0), ("cached", int(frac * L * E * expert_bytes * 1.02))):
        t0 = time.time()
        # the device holds one sequence of the positions decoded here
        saved = (model.m.ctx, model.m.seqs)
        model.m.ctx, model.m.seqs = pos0 + warmup + tokens + 1, 1
        try:
            dev = va.Device(model, expert_cache_bytes=cache)
        finally:
            model.m.ctx, model.m.seqs = saved
        for l in range(L):
            dev.kv(0, l, 0, pos0, kc[l, :pos0], vc[l, :pos0])
        log("%s: uploaded in %.1f s" % (name, time.time() - t0))
        try:
            def token(t):
                pos = pos0 + t
                tok = (1234 + 7919 * t) % cfg.vocab
                for l in range(L):
                    lg, nx = dev.moe_route(0, tok, pos, l, want_next=True)
                    _, order, w = va.host_route(lg, K, renorm)
                    guess = va.host_route(nx, K, renorm)[0] if l + 1 < L else None
                    dev.moe_experts(l, order, w, guess)
                dev.moe_head()
            for t in range(warmup):
                token(t)
            c0 = dev.expert_cache_state()[1] if cache else None
            t1 = time.perf_counter()
            for t in range(warmup, warmup + tokens):
                token(t)
            ms = (time.perf_counter() - t1) * 1000.0 / tokens
            res = {"ms_per_token": round(ms, 3), "tok_s": round(1000.0 / ms, 2)}
            if cache:
                c1 = dev.expert_cache_state()[1]
                d = {k: c1[k] - c0[k] for k in c1 if k not in ("slots", "slot_bytes")}
                res.update({"slots": c1["slots"], "slot_bytes": c1["slot_bytes"],
                            "misses_per_token": round(d["misses"] / tokens, 2),
                            "present_per_token": round((d["hits"] + d["in_flight"]) / tokens, 2),
                            "guess_copies_per_token": round(d["prefetched"] / tokens, 2),
                            "guesses_used_per_token": round(d["prefetch_used"] / tokens, 2),
                            "MB_copied_per_token": round(d["bytes_copied"] / tokens / 1e6, 2)})
                res["report"] = dev.moe_report()
            out[name] = res
            log("%s: %.3f ms a token" % (name, ms))
        finally:
            dev.close()
    if own:
        model.free()
    r, c = out["resident"], out["cached"]
    extra_ms = c["ms_per_token"] - r["ms_per_token"]
    c["copy_GBps_est"] = round(c["MB_copied_per_token"] / extra_ms, 2) if extra_ms > 0 else None
    return {"workload": "BASELINE configs[2]'s model (Qwen3-30B-A3B-shaped Q4_K_M, 48 layers), batch 1 from position %d, "
                        "decoded a layer at a time through the reference's ABI with the host routing; the expert cache "
                        "holding %.0f%% of the %d experts" % (pos0, 100 * frac, L * E),
            "tokens": tokens, "warmup_tokens": warmup, "expert_bytes": expert_bytes, "resident": r, "cached": c,
            "note": "synthetic routing spreads over every expert, so hits follow the cache's share; copy_GBps_est is "
                    "the bytes copied a token over the extra time a token takes"}


def bench_layer(va, c, reps=20):
    """configs[0] / [1]: one MoE layer of one token (norm, router, top-k, experts, weighted sum), batch 1. The
    model holds `copies` distinct layers, more weight than the 256 MB MALL, timed one after another in one graph,
    so each layer's experts stream from HBM as in a real step."""
    copies = 8 if c == 0 else 12
    model = va.Model(va.shape(**dict(va.CONFIGS[c], n_layers=copies)), 20260100 + c, threads=16)
    dev = va.Device(model)
    try:
        cfg = model.cfg
        x = va.normal(7, 1, cfg.hidden).astype(np.float32)
        dev.set_residual(x)
        us = dev.time_ffn(reps)
        e0 = model.m.layers[0].experts[0]
        expert_bytes = sum(va.row_bytes(m.dtype, m.cols) * m.rows for m in (e0.gate, e0.up, e0.down))
        b = cfg.n_experts_used * expert_bytes + cfg.n_experts * cfg.hidden * 4
        gbs = b / us / 1e3
        log("configs[%d]: one MoE layer %.2f us (%d layers cycled), %d bytes -> %.1f GB/s" % (c, us, copies, b, gbs))
        name = ("BASELINE configs[0]: OLMoE-1B-7B-shaped MoE layer, batch 1, Q8_0, 64 experts top-8" if c == 0 else
                "BASELINE configs[1]: Qwen3-30B-A3B-shaped MoE layer, batch 1, Q4_K gate/up, Q6_K down, 128 experts top-8")
        return {"workload": name, "value": round(1e6 / us, 1), "unit": "MoE layers/s (one token)", "us": round(us, 3),
                "layers_cycled": copies, "bytes_per_layer": b,
                "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(gbs / HBM_PEAK_GBS, 4),
                             "note": "the 8 chosen experts' gate, up and down plus the fp32 router, over the whole "
                                     "layer (norm, router, top-k, experts, sum: three launches)"}}
    finally:
        dev.close()
        model.free()


def bench_prefill(va, reps=10):
    """4096 rows N(0,1) through one Qwen3-shaped MoE layer, Q8_0 experts, top-8 of 128."""
    model = va.Model(va.shape(**va.CONFIGS[4]), 20260104, threads=16)
    dev = va.Device(model)
    try:
        n = 4096
        tot, ph = dev.time_prefill(0, n, seed=11, reps=reps)
        cfg = model.cfg
        flops = 2.0 * n * cfg.n_experts_used * 3 * cfg.intermediate * cfg.hidden
        gemm_us = ph[2] + ph[3]
        log("configs[4]: prefill of %d rows %.1f us (norm+router %.1f, routing %.1f, gate/up %.1f, down %.1f, sum %.1f)"
            % (n, tot, *ph))
        # the yardstick: what back-to-back MFMAs sustain on this box, as the copy probe is for streaming
        probe = va.mfma_probe()
        log("MFMA probe: %.1f TFLOP/s dense bf16" % probe)
        return {"workload": "BASELINE configs[4]: prefill of 4096 rows through one Qwen3-shaped MoE layer, Q8_0 experts, "
                            "bf16 MFMA grouped GEMM", "value": round(n / tot * 1e6, 1), "unit": "tok/s",
                "us": round(tot, 1), "phases_us": {k: round(v, 1) for k, v in zip(
                    ["norm+router", "routing+grouping", "gate/up GEMM", "down GEMM", "ordered sum"], ph)},
                "roofline": {"bound": "mfma", "achieved": round(flops / gemm_us / 1e6, 1), "peak": 2500.0,
                             "unit": "TFLOP/s", "frac": round(flops / gemm_us / 1e6 / 2500.0, 4),
                             "note": "both GEMMs: 2 n K (3 I H) flops over their summed duration"},
                "tflops_whole": round(flops / tot / 1e6, 1),
                "mfma_probe_TFLOPs": round(probe, 1), "frac_of_probe": round(flops / gemm_us / 1e6 / probe, 4)}
    finally:
        dev.close()
        model.free()


def bench_prefill_kquant(va, reps=10):
    """The same prefill (4096 rows, top-8 of 128, hidden 2048, expert width 768) with Q4_K gate/up and Q6_K down, the
    Q4_K_M convention: the grouped GEMM's K-quant form, which also serves the reference's fast passes of 64 to 1024
    rows (gpu_fast). Not a BASELINE config; reported beside configs[4]."""
    spec = dict(va.CONFIGS[4], dt_gate_up=va.Q4_K, dt_down=va.Q6_K)
    model = va.Model(va.shape(**spec), 20260105, threads=16)
    dev = va.Device(model)
    try:
        n = 4096
        tot, ph = dev.time_prefill(0, n, seed=12, reps=reps)
        cfg = model.cfg
        flops = 2.0 * n * cfg.n_experts_used * 3 * cfg.intermediate * cfg.hidden
        gemm_us = ph[2] + ph[3]
        log("Q4_K/Q6_K prefill of %d rows %.1f us (norm+router %.1f, routing %.1f, gate/up %.1f, down %.1f, sum %.1f)"
            % (n, tot, *ph))
        return {"workload": "prefill of 4096 rows through one Qwen3-shaped MoE layer, Q4_K gate/up + Q6_K down experts "
                            "(the grouped GEMM's K-quant form; not a BASELINE config)", "value": round(n / tot * 1e6, 1),
                "unit": "tok/s", "us": round(tot, 1), "phases_us": {k: round(v, 1) for k, v in zip(
                    ["norm+router", "routing+grouping", "gate/up GEMM", "down GEMM", "ordered sum"], ph)},
                "roofline": {"bound": "mfma", "achieved": round(flops / gemm_us / 1e6, 1), "peak": 2500.0,
                             "unit": "TFLOP/s", "frac": round(flops / gemm_us / 1e6 / 2500.0, 4)}}
    finally:
        dev.close()
        model.free()


if __name__ == "__main__":
    main()
