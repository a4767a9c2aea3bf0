"""Benchmark: Qwen3-30B-A3B-shaped Q4_K_M batch-1 decode on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

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
  cpu_baseline: the CPU checker's decode step (the reference's CPU arithmetic
            restated, oracle/) on this host, single-threaded, over a bounded
            number of tokens.
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
KERNELS = {0: "experts_in (gate/up + SiLU)", 1: "experts_down (+ weighted sum)", 2: "route (norm + router + top-k)",
           3: "q/k/v projections", 4: "attention (+ merge)", 5: "o-projection", 6: "LM head",
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
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every GPU box here has one GPU). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import vitna_amd as va

    pos, token = 2048, 1234
    t0 = time.time()
    shp = va.shape(n_layers=args.layers, ctx=pos + 1, seqs=1, kv_host=1)
    model = va.Model(shp, 20260101, threads=16)
    cfg = model.cfg
    kd = cfg.n_kv_heads * cfg.head_dim
    L = cfg.n_layers
    kc = np.ctypeslib.as_array(model.m.k_cache, shape=(L, model.m.ctx, kd))
    vc = np.ctypeslib.as_array(model.m.v_cache, shape=(L, model.m.ctx, kd))
    for l in range(L):
        kc[l, :pos] = va.normal(7, 2 * l, pos * kd).reshape(pos, kd)
        vc[l, :pos] = va.normal(7, 2 * l + 1, pos * kd).reshape(pos, kd)
    log("synthetic model generated in %.1f s" % (time.time() - t0))
    t0 = time.time()
    dev = va.Device(model)
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

    cpu = None
    if not args.no_cpu:
        import oracle
        n, t_cpu = 0, 0.0
        while t_cpu < args.cpu_seconds and n < 20:
            t1 = time.perf_counter()
            oracle.step(model, 0, token, pos, threads=1, trace=False)
            t_cpu += time.perf_counter() - t1
            n += 1
        cpu = {"value": round(n / t_cpu, 4), "unit": "tok/s", "cores": 1, "kind": "port",
               "sample": "%d whole decode steps of the same model and position (48 layers + head), single thread, "
                         "the reference's CPU arithmetic (AVX2 order) restated in oracle/vitna_oracle.c" % n}
        log("cpu baseline: %d steps in %.1f s -> %.3f tok/s" % (n, t_cpu, n / t_cpu))

    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 (Q4_K/Q6_K weights widened, fp32 accumulate)", "data": "synthetic",
        "config": {"workload": "BASELINE configs[2]: Qwen3-30B-A3B-shaped full decode step, batch 1, Q4_K_M, "
                               "48 layers, KV 2048 positions fp32, LM head Q6_K 151936x2048",
                   "layers": L, "position": pos, "global_batch": 1},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "experts_in_kernel<Q4_K> (8 experts x (gate + up) 768 x 2048)",
                     "bytes_per_launch": b0, "avg_us": round(us0, 3)},
        "kernels_us": {KERNELS[w]: round(per_kernel[w][0], 3) for w in per_kernel},
        "step_algorithmic_GBps": round(step_bytes / ms / 1e6, 1),
        "copy_probe_GBps": round(copy_gbs, 1),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    dev.close()
    model.free()


if __name__ == "__main__":
    main()
