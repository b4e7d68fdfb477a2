#!/usr/bin/env python3
"""Benchmark of the MI355X decode path (one GPU).  Prints ONE JSON line.

Workload for `value`: the Q8_0 GEMV / small-batch
GEMM sweep over the shapes [6144 x 2048], [2048 x 6144], [151936 x 2048] with
batch M in {1, 4, 16, 32}.  One "step" is one pass over the 12 (shape, M)
points; `value` is the sweep's algorithmic bytes (weights once + fp32
activations in + fp32 outputs) per second, inputs resident in HBM.  M = 1
runs the batch-1 GEMV and M > 1 the MFMA GEMM over the panel copy of the
weights (the layout the decode step keeps resident: same bytes, permuted once
at upload); `gguf_layout_points` times the same points through the entry
point that reads the GGUF blocks directly (anehip_quant_gemm).  Weights are rotated over enough distinct
copies (> 512 MiB per shape) that the 256 MiB MALL cannot serve repeated
reads.  Each sweep pass is one captured hipGraph (anehip_capture_*), so the
host's launch rate does not enter the figure.

`configs2_q4` times configs[2], the same three shapes in Q4_0 at M = 1
(panel and GGUF layouts, weights rotated past the MALL as above).
`configs3_deltanet` times configs[3]: 256 Gated DeltaNet decode steps
(anehip_deltanet_step: conv + SiLU, L2 norms, beta / decay, recurrence) at
batch 1 / 8 / 32, once on one resident state (the configuration as stated:
B MiB of state, which the 256 MiB MALL holds) and once with the steps rotated
over > 512 MiB of distinct states (the HBM-bound figure, as in the decode
step where 18 layers' states stream).

`decode` reports configs[4]: the full random-init Qwen3.5-2B-shape Q8_0 decode
step (24 layers, fp16 KV cache) at batch 1 and 32 and context 1k / 8k / 32k,
as tokens/s of greedy decoding with on-device token feedback (one captured
hipGraph per step); the `_cap32768` points run a 32k-position cache at a live
length of 1k / 8k (the attention work follows the live length).  `decode_q4`
is the same model shape with Q4_0 weights on every linear layer (configs[2]'s
quantisation) at batch 1 and 32, context 1k.

Timing: HIP events recorded on the library's own stream (anehip_timer_*),
around exactly `--steps` steps after `--warmup` untimed steps, with a stream
synchronisation on both sides.  All GPU inputs are generated on the device
(seeded fill + on-device quantiser); the CPU oracle is used only by the
`cpu_baseline` leg, which times the row-parallel restatement of the
reference's rayon q8_gemv and CPU decode on this host.
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

HBM_PEAK_GBS = 8000.0
SHAPES = [(6144, 2048), (2048, 6144), (151936, 2048)]
BATCHES = [1, 4, 16, 32]
MALL_DEFEAT_BYTES = 512 << 20
Q8 = 8
Q4 = 2
BLOCK_BYTES = {Q8: 34, Q4: 18}
# (batch, live context, cache capacity)
DECODE_POINTS = [(1, 1024, 1024), (1, 8192, 8192), (1, 32768, 32768), (32, 1024, 1024), (32, 8192, 8192),
                 (32, 32768, 32768), (1, 1024, 32768), (1, 8192, 32768), (32, 1024, 32768), (32, 8192, 32768)]
DECODE_Q4_POINTS = [(1, 1024, 1024), (32, 1024, 1024)]
# algorithmic bytes of one decode step: every weight once, KV rows read, DeltaNet
# state read + written (S and the 4-wide conv window), per sequence
DECODE_WEIGHT_BYTES = 18 * 62_459_904 + 6 * 55_705_600 + 330_612_736
KV_BYTES_PER_POS = 6 * 2 * 2 * 256 * 2
DN_STATE_BYTES = 18 * (2 * 16 * 128 * 128 * 4 + 2 * 6144 * 4 * 4)
# H = 16 heads of dk = dv = 128, 6144 conv channels (q, k, v)
DN_HEADS, DN_CH = 16, 6144
DN_STEPS = 256


def dn_step_bytes(batch: int) -> int:
    """Algorithmic bytes of one DeltaNet decode step: per sequence the state S
    read and written (2 x 1 MiB), the window's three kept columns read and its
    new column written (3 + 1 x 6144 fp32), qkv in (6144 fp32), o out
    (16 x 128 fp32), beta and alpha in (2 x 16 fp32); once per step the conv
    weights (6144 x 4 fp32)."""
    per_seq = 2 * DN_HEADS * 128 * 128 * 4 + 3 * DN_CH * 4 + DN_CH * 4 + DN_CH * 4 + DN_HEADS * 128 * 4 + 2 * DN_HEADS * 4
    return batch * per_seq + DN_CH * 4 * 4


def profiled_value(key: str):
    """A `key: value` line of the committed rocprofv3 summary of the roofline
    kernel (HBM bytes per launch from FETCH_SIZE / WRITE_SIZE scaled by a copy
    of known size; rocprof's average launch duration), or None."""
    path = os.path.join(ROOT, "profiles", "gemv_packed_lm_head_m1.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return float(line.split(":")[1])
    except OSError:
        pass
    return None


def profiled_traffic():
    v = profiled_value("traffic_bytes_per_launch")
    return None if v is None else int(v)


def algo_bytes(m: int, n: int, batch: int, t: int = Q8) -> int:
    return m * (n // 32) * BLOCK_BYTES[t] + 4 * batch * (n + m)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--decode-steps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of each CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--profile-kernel", action="store_true",
                    help="only run the roofline kernel (lm_head GEMV, M=1) back to back, for rocprofv3")
    ap.add_argument("--decode-only", default=None,
                    help="only run decode points, e.g. '1:1024,32:1024:32768' (batch:ctx[:capacity]), and print "
                         "their line")
    ap.add_argument("--deltanet-only", action="store_true", help="only run the configs[3] DeltaNet leg")
    ap.add_argument("--q4", action="store_true", help="with --decode-only: Q4_0 weights")
    ap.add_argument("--profile-c0", action="store_true",
                    help="only run the configs[0] GEMV, the streaming-read floor and the empty kernel (for rocprofv3)")
    ap.add_argument("--profile-b1-floors", action="store_true",
                    help="only run the floors (streaming read, empty kernel) under the batch-1 decode GEMVs")
    ap.add_argument("--profile-points", default=None,
                    help="only run these sweep points back to back, e.g. '151936x2048:32,6144x2048:4' (for rocprofv3)")
    ap.add_argument("--prefill-only", type=int, default=0,
                    help="only run the batch-1 prefill of this many tokens (twice, the second timed)")
    return ap.parse_args()


class Shape:
    """One sweep shape: Q8_0 (or Q4_0) weights generated and quantised on the
    device, replicated into `copies` distinct GGUF buffers, each with its
    panel copy."""

    def __init__(self, anehip, ctx, m, n, seed, t=Q8):
        self.m, self.n, self.t = m, n, t
        self.wbytes = m * (n // 32) * BLOCK_BYTES[t]
        self.pbytes = int(anehip.lib().anehip_quant_packed_bytes(t, m, n))
        self.copies = max(2, -(-MALL_DEFEAT_BYTES // self.wbytes))
        self.w = ctx.alloc(self.wbytes * self.copies)
        self.p = ctx.alloc(self.pbytes * self.copies)
        tmp = ctx.alloc(m * n * 4)
        ctx.fill_random(tmp, m * n, 0, seed, 0.0, 0.02)
        ctx.quantize(t, tmp, m, n, self.w.ptr)
        for c in range(1, self.copies):
            ctx.d2d(self.w.ptr + c * self.wbytes, self.w.ptr, self.wbytes)
        for c in range(self.copies):
            ctx.call("quant_pack", t, self.wptr(c), m, n, self.pptr(c))
        ctx.sync()
        tmp.free()
        self.x = ctx.alloc(32 * n * 4)
        ctx.fill_random(self.x, 32 * n, 0, seed + 1, 0.0, 1.0)
        self.y = ctx.alloc(32 * m * 4)

    def wptr(self, c):
        return self.w.ptr + (c % self.copies) * self.wbytes

    def pptr(self, c):
        return self.p.ptr + (c % self.copies) * self.pbytes

    def free(self):
        for b in (self.w, self.p, self.x, self.y):
            b.free()


def launch_point(ctx, s, batch, c, gguf=False):
    """One GEMV (M = 1) or MFMA GEMM (M > 1) on copy c: over the panel copy
    (the decode step's layout), or with gguf=True over the GGUF blocks."""
    if gguf:
        ctx.quant_gemm(s.t, s.wptr(c), s.m, s.n, s.x, batch, s.y)
    else:
        ctx.call("quant_gemm_packed", s.t, s.pptr(c), s.m, s.n, s.x.ptr, batch, s.y.ptr)


def capture(ctx, enqueue):
    """A hipGraph of the kernel-level calls `enqueue` makes (run once eagerly
    first, so no workspace grows during capture)."""
    enqueue()
    ctx.sync()
    ctx.capture_begin()
    try:
        enqueue()
    finally:
        g = ctx.capture_end()
    return g


def time_graphs(ctx, graphs, launches, warmup=2):
    for i in range(warmup):
        ctx.graph_launch(graphs[i % len(graphs)])
    ctx.sync()
    ctx.timer_start()
    for i in range(launches):
        ctx.graph_launch(graphs[i % len(graphs)])
    return ctx.timer_stop()


def time_point(ctx, s, batch, launches, gguf=False):
    """Average time of one launch, `launches` back to back in one graph (copies rotated)."""
    g = capture(ctx, lambda: [launch_point(ctx, s, batch, c, gguf) for c in range(launches)])
    ms = time_graphs(ctx, [g], 3) / 3
    ctx.graph_destroy(g)
    return ms / launches


def decode_weight_bytes(anehip, spec, ggml_type):
    """Bytes of every quantised weight of the model (read once per step)."""
    per_block = BLOCK_BYTES[ggml_type]
    return sum(rows * cols // 32 * per_block for layer in [-1] + list(range(spec.n_layers))
               for rows, cols, quant in spec.shapes(layer).values() if quant)


def bench_decode(anehip, steps, warmup, points=DECODE_POINTS, prefill_tokens=0, ggml_type=Q8):
    """Greedy decode tok/s of the random-init Qwen3.5-2B shape at each
    (batch, live context, cache capacity), Q8_0 (or Q4_0) weights."""
    spec = anehip.Spec()
    gm = anehip.Model(spec)
    gm.randomize(seed=1, ggml_type=ggml_type)
    weight_bytes = decode_weight_bytes(anehip, spec, ggml_type)
    assert ggml_type != Q8 or weight_bytes == DECODE_WEIGHT_BYTES
    out = {}
    for batch, ctx_len, cap in points:
        gm.alloc_state(batch, cap)
        for l in range(spec.n_layers):
            if spec.layer_types[l] == anehip.LAYER_DELTANET:
                p, n = gm.state_ptr(l, 0)
                gm.fill_random(p, n // 4, 0, 100 + l, 0.0, 1.0)
                p, n = gm.state_ptr(l, 1)
                gm.fill_random(p, n // 4, 0, 200 + l, 0.0, 0.01)
            else:
                for which in (2, 3):
                    p, n = gm.state_ptr(l, which)
                    gm.fill_random(p, n // 2, 0, 300 + 10 * l + which, 0.0, 1.0, f16=True)
        start = ctx_len - 1 - (steps + warmup)
        for b in range(batch):
            gm.set_pos(b, start)
        toks = (np.arange(batch, dtype=np.uint32) * 7919) % spec.vocab_size
        gm.generate(toks, warmup)
        gm.sync()
        gm.timer_start()
        gm.generate(toks, steps)
        ms = gm.timer_stop()
        step_ms = ms / steps
        step_bytes = weight_bytes + batch * (ctx_len * KV_BYTES_PER_POS + DN_STATE_BYTES)
        key = f"B{batch}_ctx{ctx_len}" + (f"_cap{cap}" if cap != ctx_len else "")
        out[key] = {
            "tok_s": round(batch * steps / (ms * 1e-3), 1),
            "ms_per_step": round(step_ms, 3),
            "algorithmic_GB_per_step": round(step_bytes / 1e9, 3),
            "effective_GB_s": round(step_bytes / (step_ms * 1e-3) / 1e9, 1),
        }
    lengths = [prefill_tokens] if isinstance(prefill_tokens, int) else list(prefill_tokens)
    lengths = [n for n in lengths if n]
    if lengths:
        # anehip_prefill of one sequence from position 0 (chunks of 256 tokens),
        # synchronous, timed on the host clock; one untimed run first
        gm.alloc_state(1, max([1024] + lengths))
        for n_tok in lengths:
            prompt = (np.arange(n_tok, dtype=np.uint32) * 7919) % spec.vocab_size
            gm.set_pos(0, 0)
            gm.prefill(0, prompt, want_logits=False)
            gm.set_pos(0, 0)
            t0 = time.perf_counter()
            gm.prefill(0, prompt, want_logits=True)
            dt = time.perf_counter() - t0
            out[f"prefill_B1_tokens{n_tok}"] = {"tok_s": round(n_tok / dt, 1), "ms": round(dt * 1e3, 2)}
    gm.close()
    return out


_probe = None


def probe_lib():
    """libanehip_probe.so: the measurement-only roofline probes (built beside
    libanehip.so; not part of the product library)."""
    global _probe
    if _probe is None:
        import ctypes as C

        path = os.path.join(ROOT, "ane-infer_amd", "libanehip_probe.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} not built; run python ane-infer_amd/build.py")
        L = C.CDLL(path)
        vp, u32 = C.c_void_p, C.c_uint32
        L.anehip_probe_read.argtypes = [vp, vp, C.c_size_t, u32, u32, u32, vp]
        L.anehip_probe_read.restype = C.c_int
        L.anehip_probe_empty.argtypes = [vp, u32, u32]
        L.anehip_probe_empty.restype = C.c_int
        _probe = L
    return _probe


def probe_read(ctx, src, nbytes, wgs, threads, depth, sink):
    ctx._check(probe_lib().anehip_probe_read(ctx.h, src, nbytes, wgs, threads, depth, sink.ptr))


def probe_empty(ctx, wgs, threads):
    ctx._check(probe_lib().anehip_probe_empty(ctx.h, wgs, threads))


FLOOR_GRIDS = [(96, 1024), (192, 1024), (256, 256), (256, 512), (384, 512), (512, 256), (512, 512), (1024, 256), (1024, 512),
               (2048, 256)]
FLOOR_DEPTHS = [2, 4, 8]


def c0_floor(ctx, s, launches=40):
    """The floor under the configs[0] GEMV: a 16-byte streaming read of the
    same bytes (one panel copy, rotated as the GEMV's weights are) on each grid
    of FLOOR_GRIDS x FLOOR_DEPTHS, and an empty kernel, each timed as
    `launches` back-to-back nodes of one graph (per-launch time)."""
    sink = ctx.alloc(max(w * t for w, t in FLOOR_GRIDS) * 4)
    res = {}
    for wgs, threads in FLOOR_GRIDS:
        for depth in FLOOR_DEPTHS:
            g = capture(ctx, lambda: [probe_read(ctx, s.pptr(c), s.pbytes, wgs, threads, depth, sink)
                                      for c in range(launches)])
            ms = time_graphs(ctx, [g], 3) / 3 / launches
            ctx.graph_destroy(g)
            res[f"{wgs}x{threads}_d{depth}"] = round(ms * 1e3, 3)
    empty = {}
    for wgs, threads in ((256, 512), (288, 512)):
        g = capture(ctx, lambda: [probe_empty(ctx, wgs, threads) for _ in range(launches)])
        empty[f"{wgs}x{threads}"] = round(time_graphs(ctx, [g], 3) / 3 / launches * 1e3, 3)
        ctx.graph_destroy(g)
    sink.free()
    best = min(res, key=res.get)
    gbs = algo_bytes(s.m, s.n, 1) / (res[best] * 1e-6) / 1e9
    return {"read_us": res, "best": best, "best_us": res[best], "best_GB/s": round(gbs, 1),
            "best_pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1), "empty_kernel_us": empty,
            "bytes": s.pbytes}


# The batch-1 decode step's GEMVs at the 2B shape: role, m x n, and the
# workgroups of the step's kernel (its K-split grid, as the kernel trace of
# `--decode-only 1:1024` shows it).
B1_GEMVS = [("ffn gate/up", 12288, 2048, 192), ("DeltaNet in-proj", 8224, 2048, 129),
            ("ffn down", 2048, 6144, 192), ("attention qkv", 5120, 2048, 160), ("ssm_out", 2048, 2048, 256),
            ("o_proj", 2048, 2048, 256), ("lm_head", 151936, 2048, 2374)]


def b1_floors(anehip, ctx, launches=40):
    """Floors under each batch-1 decode GEMV: a 16-byte streaming read of its
    panel bytes (rotated past the MALL) on the step kernel's own grid
    (workgroups x 512 threads, the best of depths 2 / 4 / 8), and an empty
    kernel on that grid, each timed as `launches` back-to-back graph nodes."""
    out = {}
    for i, (role, m, n, wgs) in enumerate(B1_GEMVS):
        s = Shape(anehip, ctx, m, n, 500 + i)
        sink = ctx.alloc(wgs * 512 * 4)
        reads = {}
        for depth in FLOOR_DEPTHS:
            g = capture(ctx, lambda: [probe_read(ctx, s.pptr(c), s.pbytes, wgs, 512, depth, sink)
                                      for c in range(launches)])
            reads[depth] = time_graphs(ctx, [g], 3) / 3 / launches * 1e3
            ctx.graph_destroy(g)
        g = capture(ctx, lambda: [probe_empty(ctx, wgs, 512) for _ in range(launches)])
        empty = time_graphs(ctx, [g], 3) / 3 / launches * 1e3
        ctx.graph_destroy(g)
        best = min(reads, key=reads.get)
        out[role] = {"m": m, "n": n, "workgroups": wgs, "algorithmic_bytes": algo_bytes(m, n, 1),
                     "read_us": round(reads[best], 2), "read_depth": best,
                     "read_GB/s": round(algo_bytes(m, n, 1) / (reads[best] * 1e-6) / 1e9, 1),
                     "empty_us": round(empty, 2)}
        sink.free()
        s.free()
    return out


def bench_q4(anehip, ctx):
    """Q4_0 GEMV at M = 1 on the three shapes (panel layout, and
    the GGUF blocks through anehip_quant_gemm), weights rotated past the MALL."""
    out = {}
    for i, (m, n) in enumerate(SHAPES):
        s = Shape(anehip, ctx, m, n, 400 + i, t=Q4)
        for gguf in (False, True):
            t = time_point(ctx, s, 1, max(s.copies, 20), gguf)
            gbs = algo_bytes(m, n, 1, Q4) / (t * 1e-3) / 1e9
            out[f"{m}x{n}_M1" + ("_gguf_layout" if gguf else "")] = {
                "us": round(t * 1e3, 2), "GB/s": round(gbs, 1), "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1)}
        s.free()
    return out


def bench_deltanet(anehip, ctx):
    """DN_STEPS anehip_deltanet_step calls at batch 1 / 8 / 32
    (16 heads, dk = dv = 128, S0 ~ N(0, 0.01), fresh N(0, 1) qkv / beta /
    alpha per step from 8 rotating input sets, ssm_a = -U(0, 1)), captured as
    one graph: on one resident state, and rotated over > 512 MiB of states."""
    out = {}
    per_state = DN_HEADS * 128 * 128 * 4
    cw, sa, dt = ctx.alloc(DN_CH * 4 * 4), ctx.alloc(DN_HEADS * 4), ctx.alloc(DN_HEADS * 4)
    ctx.fill_random(cw, DN_CH * 4, 0, 31, 0.0, 0.5)
    ctx.fill_random(sa, DN_HEADS, 1, 32, -1.0, 0.0)
    ctx.fill_random(dt, DN_HEADS, 0, 33, 0.0, 1.0)
    for batch in (1, 8, 32):
        ins = []
        for i in range(8):
            q, b, a = ctx.alloc(batch * DN_CH * 4), ctx.alloc(batch * DN_HEADS * 4), ctx.alloc(batch * DN_HEADS * 4)
            ctx.fill_random(q, batch * DN_CH, 0, 1000 + i, 0.0, 1.0)
            ctx.fill_random(b, batch * DN_HEADS, 0, 2000 + i, 0.0, 1.0)
            ctx.fill_random(a, batch * DN_HEADS, 0, 3000 + i, 0.0, 1.0)
            ins.append((q, b, a))
        o = ctx.alloc(batch * DN_HEADS * 128 * 4)
        res = {}
        for mode, copies in (("resident", 1), ("rotated", max(2, -(-MALL_DEFEAT_BYTES // (batch * per_state))))):
            S = ctx.alloc(copies * batch * per_state)
            W = ctx.alloc(copies * batch * DN_CH * 4 * 4)
            ctx.fill_random(S, copies * batch * per_state // 4, 0, 40 + batch, 0.0, 0.01)
            ctx.fill_random(W, copies * batch * DN_CH * 4, 0, 50 + batch, 0.0, 1.0)

            def enqueue():
                for step in range(DN_STEPS):
                    c = step % copies
                    q, b, a = ins[step % 8]
                    ctx.call("deltanet_step", batch, DN_HEADS, q, b, a, cw, sa, dt,
                             W.ptr + c * batch * DN_CH * 16, S.ptr + c * batch * per_state, o)

            g = capture(ctx, enqueue)
            ms = time_graphs(ctx, [g], 3, warmup=1) / 3
            ctx.graph_destroy(g)
            us = ms * 1e3 / DN_STEPS
            res[mode] = {"us_per_step": round(us, 2), "ms_256_steps": round(ms, 3),
                         "GB/s": round(dn_step_bytes(batch) / (us * 1e-6) / 1e9, 1),
                         "states": copies}
            S.free()
            W.free()
        res["algorithmic_bytes_per_step"] = dn_step_bytes(batch)
        out[f"B{batch}"] = res
        o.free()
        for t in ins:
            for buf in t:
                buf.free()
    for buf in (cw, sa, dt):
        buf.free()
    return out


def host_info():
    """nproc and the CPU model of this host (for the CPU baseline)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return {"nproc": usable, "cpu_count": os.cpu_count(), "cpu_model": model}


def time_cpu(fn, budget_s, min_runs=20):
    """Median wall time (s) of fn() over at least `min_runs` runs or `budget_s`, after one warm-up run."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < min_runs:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times), float(sum(times))


def cpu_baseline(anehip, ctx, shapes, budget_s, decode):
    """Oracle (restated reference CPU path) on this host: row-parallel q8_gemv
    over the config-1 shapes at M = 1, q4_gemv_cpu, the DeltaNet step at B = 1
    / 8 / 32 (B independent sequences), and, if `decode`,
    qwen35_forward_token tok/s at B = 1 and B = 32 (32 independent sequences)
    on the same random-init 2B-shape weights."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    threads = oracle.max_threads()
    hosts = []
    for s in shapes:
        w = np.empty(s.wbytes, np.uint8)
        ctx._check(anehip.lib().anehip_d2h(ctx.h, w.ctypes.data, anehip.C.c_void_p(s.w.ptr), s.wbytes))
        x = s.x.download(np.float32, s.n)
        hosts.append((s, w, x, np.empty(s.m, np.float32)))
    for s, w, x, y in hosts:
        oracle.lib().ao_quant_gemv_mt(Q8, w, s.m, s.n, x, y, threads)
    total_bytes, total_t, reps = 0, 0.0, 0
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end:
        for s, w, x, y in hosts:
            t0 = time.perf_counter()
            oracle.lib().ao_quant_gemv_mt(Q8, w, s.m, s.n, x, y, threads)
            total_t += time.perf_counter() - t0
            total_bytes += algo_bytes(s.m, s.n, 1)
        reps += 1
    res = {
        "value": round(total_bytes / total_t / 1e9, 2),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} passes of the three config-1 shapes at M=1 (row-parallel q8_gemv restatement, "
                  f"{total_t:.1f} s of GEMV time)",
    }
    res.update(host_info())
    # Q4_0 GEMV (row-parallel q4_gemv_cpu restatement), M = 1, host-side quantisation
    q4 = {}
    for i, (m, n) in enumerate(SHAPES):
        w = oracle.gen_quant(Q4, 400 + i, 1, m, n, std=0.02)
        x = oracle.normal(401 + i, 2, n)
        y = np.empty(m, np.float32)
        med, runs, _ = time_cpu(lambda: oracle.lib().ao_quant_gemv_mt(Q4, w, m, n, x, y, threads), budget_s / 6)
        q4[f"{m}x{n}_M1"] = {"us_median": round(med * 1e6, 1),
                             "GB/s": round(algo_bytes(m, n, 1, Q4) / med / 1e9, 2), "runs": runs}
    res["q4_gemv"] = q4
    res["q4_sample"] = f"median of >= 20 runs per shape, {threads} threads"
    # one sequence's DeltaNet step (deltanet_decode_step's mixer core, single thread)
    conv_w = oracle.normal(31, 1, DN_CH * 4, std=0.5)
    ssm_a = -oracle.uniform(32, 2, DN_HEADS)
    dt_bias = oracle.normal(33, 3, DN_HEADS)
    S = oracle.normal(34, 4, DN_HEADS * 128 * 128, std=0.01)
    win = oracle.normal(35, 5, DN_CH * 4)
    steps_in = [(oracle.normal(36, 10 + i, DN_CH), oracle.normal(36, 20 + i, DN_HEADS),
                 oracle.normal(36, 30 + i, DN_HEADS)) for i in range(8)]
    k = [0]

    def dn_step():
        q, b, a = steps_in[k[0] % 8]
        k[0] += 1
        oracle.deltanet_core(q, b, a, conv_w, ssm_a, dt_bias, win, S, DN_HEADS, 128)

    med, runs, _ = time_cpu(dn_step, budget_s / 4)
    res["deltanet_B1"] = {"us_per_step_median": round(med * 1e6, 1),
                          "GB/s": round(dn_step_bytes(1) / med / 1e9, 2), "runs": runs, "cores": 1,
                          "sample": "deltanet_decode_step's conv + norms + gates + recurrence (restated), "
                                    "one sequence, single thread (the reference's loop is serial)"}
    # configs[3] at B = 8 / 32: the reference has no batch, so a batched step
    # is B independent sequences' steps, each on its own state and window
    for batch in (8, 32):
        Ss = [S.copy() for _ in range(batch)]
        wins = [win.copy() for _ in range(batch)]

        def dn_batch(batch=batch, Ss=Ss, wins=wins):
            q, b, a = steps_in[k[0] % 8]
            k[0] += 1
            for i in range(batch):
                oracle.deltanet_core(q, b, a, conv_w, ssm_a, dt_bias, wins[i], Ss[i], DN_HEADS, 128)

        med, runs, _ = time_cpu(dn_batch, budget_s / 8, min_runs=5)
        res[f"deltanet_B{batch}"] = {"us_per_step_median": round(med * 1e6, 1),
                                     "GB/s": round(dn_step_bytes(batch) / med / 1e9, 2), "runs": runs, "cores": 1,
                                     "sample": f"{batch} sequences' deltanet_decode_step in turn per step "
                                               "(restated), single thread"}
    if decode:
        spec = anehip.Spec()
        gm = anehip.Model(spec)
        gm.randomize(seed=1)
        om = oracle.OracleModel(spec.dim, spec.hidden_dim, spec.n_layers, spec.n_heads, spec.n_kv_heads,
                                spec.head_dim, spec.vocab_size, spec.ssm_state_size, spec.ssm_conv_kernel,
                                spec.ssm_group_count, spec.rope_freq_base, spec.rms_norm_eps, spec.layer_types)
        for layer in [-1] + list(range(spec.n_layers)):
            for kind, (rows, cols, quant) in spec.shapes(layer).items():
                arr = gm.download_tensor(layer, kind)
                if quant:
                    om.set_quant(layer, kind, arr, rows, cols, Q8)
                else:
                    om.set_f32(layer, kind, arr)
        gm.close()
        # attention at ctx ~1k: the sequence starts at position 1023 (the cache
        # below it zero; attention's cost does not depend on the values)
        start, cap = 1023, 1024 + 512
        seq = oracle.OracleSeq(om, cap)
        seq.pos = start
        seq.forward(1, threads)
        n_tok, t_dec = 0, 0.0
        t_end = time.perf_counter() + budget_s
        tok = 1
        while (time.perf_counter() < t_end or n_tok < 2) and seq.pos < cap - 1:
            t0 = time.perf_counter()
            tok = oracle.argmax(seq.forward(tok, threads))
            t_dec += time.perf_counter() - t0
            n_tok += 1
        res["decode_tok_s_B1_ctx1k"] = round(n_tok / t_dec, 2)
        res["decode_sample"] = (f"{n_tok} greedy tokens of qwen35_forward_token (restated) at positions "
                                f"{start + 1}..{start + n_tok}, 2B shape, Q8_0, {threads} threads for the GEMVs")
        seq.close()
        # B = 32 as 32 independent sequences (the reference decodes one
        # sequence at a time): each round gives every sequence one token
        seqs = []
        for i in range(32):
            q = oracle.OracleSeq(om, cap)
            q.pos = start
            seqs.append(q)
        toks = [1 + i for i in range(32)]
        rounds, t32 = 0, 0.0
        t_end = time.perf_counter() + budget_s
        while (time.perf_counter() < t_end or rounds < 1) and seqs[0].pos < cap - 1:
            t0 = time.perf_counter()
            for i, q in enumerate(seqs):
                toks[i] = oracle.argmax(q.forward(toks[i], threads))
            t32 += time.perf_counter() - t0
            rounds += 1
        res["decode_tok_s_B32_ctx1k"] = round(32 * rounds / t32, 2)
        res["decode_B32_sample"] = (f"{rounds} rounds of one greedy token for each of 32 independent sequences "
                                    f"(qwen35_forward_token restated, positions from {start + 1}), "
                                    f"{threads} threads for the GEMVs")
        for q in seqs:
            q.close()
        om.close()
    return res


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)
    import anehip

    rc = anehip.lib().anehip_init()
    if rc != 0:
        raise SystemExit(f"no gfx950 device: {anehip.lib().anehip_last_error(None).decode()}")
    if args.decode_only:
        pts = []
        for p in args.decode_only.split(","):
            v = [int(t) for t in p.split(":")]
            pts.append((v[0], v[1], v[2] if len(v) > 2 else v[1]))
        qt = Q4 if args.q4 else Q8
        print(json.dumps({"decode_q4" if args.q4 else "decode": bench_decode(anehip, args.decode_steps, 3, pts,
                                                                             ggml_type=qt)}), flush=True)
        return
    if args.prefill_only:
        print(json.dumps({"decode": bench_decode(anehip, args.decode_steps, 3, [],
                                                 prefill_tokens=args.prefill_only)}), flush=True)
        return
    ctx = anehip.Context(0)
    if args.deltanet_only:
        print(json.dumps({"configs3_deltanet": bench_deltanet(anehip, ctx)}), flush=True)
        ctx.close()
        return
    if args.profile_c0:
        c0 = Shape(anehip, ctx, 6144, 2048, 100)
        t = time_point(ctx, c0, 1, 40)
        print(json.dumps({"c0_us": round(t * 1e3, 3), "floor": c0_floor(ctx, c0)}), flush=True)
        ctx.close()
        return
    if args.profile_b1_floors:
        print(json.dumps({"b1_floors": b1_floors(anehip, ctx)}), flush=True)
        ctx.close()
        return
    if args.profile_points:
        res = {}
        for p in args.profile_points.split(","):
            shape, batch = p.split(":")
            m, n = (int(v) for v in shape.split("x"))
            s = Shape(anehip, ctx, m, n, 100)
            t = time_point(ctx, s, int(batch), max(s.copies, 20))
            res[p] = {"us": round(t * 1e3, 2), "GB/s": round(algo_bytes(m, n, int(batch)) / (t * 1e-3) / 1e9, 1)}
            s.free()
        print(json.dumps(res), flush=True)
        ctx.close()
        return
    if args.profile_kernel:
        lm = Shape(anehip, ctx, 151936, 2048, 102)
        t = time_point(ctx, lm, 1, args.steps)
        # reference for the HBM byte counters: plain device copies of known size
        cp = 256 << 20
        a, b = ctx.alloc(cp), ctx.alloc(cp)
        for _ in range(5):
            ctx.d2d(b.ptr, a.ptr, cp)
        ctx.sync()
        print(json.dumps({"kernel": "gemv_packed<Q8_0, PLAIN> lm_head 151936x2048, M=1",
                          "avg_launch_us": round(t * 1e3, 2),
                          "GB/s": round(algo_bytes(lm.m, lm.n, 1) / (t * 1e-3) / 1e9, 1),
                          "copy_reference_bytes": cp}), flush=True)
        ctx.close()
        return
    shapes = [Shape(anehip, ctx, m, n, 100 + i) for i, (m, n) in enumerate(SHAPES)]

    # one graph per rotation phase r; every launch of a shape reads the next
    # copy of its weights (point j of phase r: copy r * len(BATCHES) + j), so
    # between two reads of one copy every other copy of the shape (> 512 MiB)
    # has been read and the MALL cannot serve it
    phases = max(s.copies for s in shapes)
    sweeps = [capture(ctx, lambda r=r: [launch_point(ctx, s, b, r * len(BATCHES) + j) for s in shapes
                                        for j, b in enumerate(BATCHES)])
              for r in range(phases)]
    for i in range(args.warmup):
        ctx.graph_launch(sweeps[i % phases])
    ctx.sync()
    ctx.timer_start()
    for i in range(args.steps):
        ctx.graph_launch(sweeps[i % phases])
    ms_total = ctx.timer_stop()
    for g in sweeps:
        ctx.graph_destroy(g)
    ms_per_step = ms_total / args.steps
    sweep_bytes = sum(algo_bytes(s.m, s.n, b) for s in shapes for b in BATCHES)
    value = sweep_bytes / (ms_per_step * 1e-3) / 1e9

    points, gguf_points = {}, {}
    for s in shapes:
        for b in BATCHES:
            for gguf, dst in ((False, points), (True, gguf_points)):
                t = time_point(ctx, s, b, max(s.copies, 20), gguf)
                dst[f"{s.m}x{s.n}_M{b}"] = {"us": round(t * 1e3, 2),
                                            "GB/s": round(algo_bytes(s.m, s.n, b) / (t * 1e-3) / 1e9, 1)}
    lm = shapes[2]
    t_lm = time_point(ctx, lm, 1, 50)
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
        "dtype": "q8_0 weights, fp32 activations and accumulation",
        "data": "synthetic: seeded N(0,0.02) weights quantised absmax/127 on device, N(0,1) activations",
        "config": {
            "workload": "configs[1]: Q8_0 GEMV/GEMM sweep, shapes 6144x2048, 2048x6144, 151936x2048, "
                        "M in {1,4,16,32}, weights rotated over >512 MiB of copies",
            "step": "one pass over the 12 (shape, M) points",
            "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "gemv_packed<Q8_0, PLAIN> (lm_head 151936x2048, M=1, panel layout)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic(),
            "traffic_source": "profiles/gemv_packed_lm_head_m1.md (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-scaled)",
            "algorithmic_bytes": lm_bytes,
            "avg_launch_us": round(t_lm * 1e3, 2),
            "timing": "HIP events on the library stream around a graph of back-to-back launches, this run",
        },
        "c0_gemv_6144x2048": {"us": c0["us"], "GB/s": c0["GB/s"],
                               "pct_of_hbm_peak": round(100 * c0["GB/s"] / HBM_PEAK_GBS, 1)},
        "sweep_points": points,
        "gguf_layout_points": gguf_points,
    }
    rp_us = profiled_value("rocprof_avg_us")
    if rp_us:
        # the committed rocprofv3 kernel-trace average of the same kernel and
        # workload, and the fraction it gives (beside the live event figure)
        out["roofline"]["rocprof_avg_us"] = rp_us
        out["roofline"]["frac_rocprof"] = round(lm_bytes / (rp_us * 1e3) / HBM_PEAK_GBS, 4)
    out["c0_gemv_6144x2048"]["floor"] = c0_floor(ctx, shapes[0])
    out["c0_gemv_6144x2048"]["pct_of_floor"] = round(100 * out["c0_gemv_6144x2048"]["floor"]["best_us"] / c0["us"], 1)
    out["configs2_q4"] = bench_q4(anehip, ctx)
    out["configs3_deltanet"] = bench_deltanet(anehip, ctx)
    if not args.no_decode:
        out["decode"] = bench_decode(anehip, args.decode_steps, 3, prefill_tokens=(512, 2048))
        # the same model shape with Q4_0 weights (configs[2]'s quantisation on every linear layer)
        out["decode_q4"] = bench_decode(anehip, args.decode_steps, 3, DECODE_Q4_POINTS, ggml_type=Q4)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(anehip, ctx, shapes, args.cpu_seconds, decode=not args.no_decode)
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
