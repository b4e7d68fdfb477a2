#!/usr/bin/env python3
"""Benchmark of the MI355X decode-path kernels (one GPU).

Prints ONE JSON line.  Workload: the Q8_0 GEMV /
small-batch GEMM sweep over the shapes [6144 x 2048], [2048 x 6144] and
[151936 x 2048] with batch M in {1, 4, 16, 32}.  One "step" is one pass over
the 12 (shape, M) points; `value` is the whole sweep's algorithmic bytes per
second (weights + activations in + outputs), with inputs resident in HBM.

Weights are rotated over enough distinct copies (> 512 MiB per shape) that the
256 MiB MALL cannot serve repeated reads.  Timing uses HIP events recorded on
the library's own stream (anehip_timer_start/stop), around exactly `--steps`
steps after `--warmup` untimed steps, with a stream synchronisation on both
sides.

The `roofline` object is for the dominant kernel (the lm_head GEMV, M = 1):
achieved = its algorithmic bytes per launch / its average launch duration
(HIP events over a run of back-to-back launches).  `cpu_baseline` times the
oracle's row-parallel restatement of the reference's rayon q8_gemv on this
host over a bounded sample (same byte formula).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ane-infer_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

HBM_PEAK_GBS = 8000.0
SHAPES = [(6144, 2048), (2048, 6144), (151936, 2048)]
BATCHES = [1, 4, 16, 32]
MALL_DEFEAT_BYTES = 512 << 20
Q8 = 8


def algo_bytes(m: int, n: int, batch: int) -> int:
    """Weights once + fp32 activations in + fp32 outputs."""
    return m * (n // 32) * 34 + 4 * batch * (n + m)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    return ap.parse_args()


class Shape:
    def __init__(self, ctx, oracle, m, n, seed):
        self.m, self.n = m, n
        self.w_host = oracle.gen_quant(Q8, seed, m, m, n, std=0.02)
        self.wbytes = self.w_host.nbytes
        self.copies = max(2, -(-MALL_DEFEAT_BYTES // self.wbytes))
        self.w = ctx.alloc(self.wbytes * self.copies)
        for c in range(self.copies):
            self.w.upload(self.w_host, offset=c * self.wbytes)
        self.x_host = oracle.normal(seed, 7, 32 * n).reshape(32, n)
        self.x = ctx.to_device(self.x_host)
        self.y = ctx.alloc(32 * m * 4)
        self.next = 0

    def wptr(self):
        p = self.w.ptr + self.next * self.wbytes
        self.next = (self.next + 1) % self.copies
        return p


def run_sweep(ctx, shapes):
    for s in shapes:
        for b in BATCHES:
            ctx.quant_gemm(Q8, s.wptr(), s.m, s.n, s.x, b, s.y)


def time_kernel(ctx, s, batch, launches):
    for _ in range(3):
        ctx.quant_gemm(Q8, s.wptr(), s.m, s.n, s.x, batch, s.y)
    ctx.sync()
    ctx.timer_start()
    for _ in range(launches):
        ctx.quant_gemm(Q8, s.wptr(), s.m, s.n, s.x, batch, s.y)
    return ctx.timer_stop() / launches


def cpu_baseline(oracle, shapes, budget_s):
    """Row-parallel CPU GEMV (the reference's rayon path restated) on the config-1
    shapes at M = 1, repeated until the time budget is used."""
    threads = oracle.max_threads()
    total_bytes, total_t, reps = 0, 0.0, 0
    t_end = time.perf_counter() + budget_s
    ys = [np.empty(s.m, np.float32) for s in shapes]
    for s, y in zip(shapes, ys):  # warm up
        oracle.lib().ao_quant_gemv_mt(Q8, s.w_host, s.m, s.n, s.x_host[0], y, threads)
    while time.perf_counter() < t_end:
        for s, y in zip(shapes, ys):
            t0 = time.perf_counter()
            oracle.lib().ao_quant_gemv_mt(Q8, s.w_host, s.m, s.n, s.x_host[0], y, threads)
            total_t += time.perf_counter() - t0
            total_bytes += algo_bytes(s.m, s.n, 1)
        reps += 1
    return {
        "value": round(total_bytes / total_t / 1e9, 2),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} passes of the three config-1 shapes at M=1 (row-parallel q8_gemv restatement, "
                  f"{total_t:.1f} s of GEMV time)",
    }


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)
    import anehip
    import oracle

    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    rc = anehip.lib().anehip_init()
    if rc != 0:
        raise SystemExit(f"no gfx950 device: {anehip.lib().anehip_last_error(None).decode()}")
    ctx = anehip.Context(0)
    shapes = [Shape(ctx, oracle, m, n, 100 + i) for i, (m, n) in enumerate(SHAPES)]
    ctx.sync()

    for _ in range(args.warmup):
        run_sweep(ctx, shapes)
    ctx.sync()
    ctx.timer_start()
    for _ in range(args.steps):
        run_sweep(ctx, shapes)
    ms_total = ctx.timer_stop()
    ms_per_step = ms_total / args.steps
    sweep_bytes = sum(algo_bytes(s.m, s.n, b) for s in shapes for b in BATCHES)
    value = sweep_bytes / (ms_per_step * 1e-3) / 1e9

    # per-point kernel times (HIP events over back-to-back launches)
    points = {}
    for s in shapes:
        for b in BATCHES:
            launches = 20 if s.m > 100000 else 200
            t = time_kernel(ctx, s, b, launches)
            gbs = algo_bytes(s.m, s.n, b) / (t * 1e-3) / 1e9
            points[f"{s.m}x{s.n}_M{b}"] = {"us": round(t * 1e3, 2), "GB/s": round(gbs, 1)}
    lm = shapes[2]
    t_lm = time_kernel(ctx, lm, 1, 50)
    lm_bytes = algo_bytes(lm.m, lm.n, 1)
    achieved = lm_bytes / (t_lm * 1e-3) / 1e9
    c0 = points["6144x2048_M1"]

    out = {
        "metric": "Q8_0 GEMV HBM GB/s (% peak); decode tok/s Qwen3.5-2B-shape at B=1 and B=32",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 weights, fp32 activations/accumulate",
        "data": "synthetic: seeded N(0,0.02) weights quantised absmax/127, N(0,1) activations",
        "config": {
            "workload": "configs[1]: Q8_0 GEMV/GEMM sweep, shapes 6144x2048, 2048x6144, 151936x2048, "
                        "M in {1,4,16,32}, weights rotated over >512 MiB of copies",
            "step": "one pass over the 12 (shape, M) points",
            "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "quant_gemm_rows64<Q8_0,1> lm_head 151936x2048 M=1",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "algorithmic_bytes": lm_bytes,
            "avg_launch_us": round(t_lm * 1e3, 2),
        },
        "c0_gemv_6144x2048": {"us": c0["us"], "GB/s": c0["GB/s"],
                               "pct_of_hbm_peak": round(100 * c0["GB/s"] / HBM_PEAK_GBS, 1)},
        "sweep_points": points,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(oracle, shapes, args.cpu_seconds)
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
