#!/usr/bin/env python3
"""Benchmark of the Q8 matvec hot path on one MI355X.

A step is one activation vector through config 2's three Q8_0 products
(4096x4096, 14336x4096, 4096x14336): for each, the input is quantized and
multiplied, as num.MatVecQ8 does (internal/num/quant.go:167-180). Weights are
synthetic (codes uniform in [-127, 127], scales U(1e-3, 1e-2)), resident in
HBM before timing, and rotated over several copies totalling more than the
256 MB Infinity Cache, so every step streams its weights from HBM.

value = algorithmic bytes of a step / step time (GB/s), where a product's
bytes are rows*cols (codes) + rows*cols/32*4 (scales) + 4*cols (x) +
4*rows (out). roofline = the matvec_q8 kernel's bytes per launch over its
average duration, timed with HIP events on its own stream (the library's
profile). cpu_baseline = the C restatement of the reference CPU path (AVX2
block sums, rows over threads) on this host, on a bounded sample.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "rakkan-mesh_amd"))
sys.path.insert(0, ROOT)

SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336)]
HBM_PEAK_GBS = 8000.0


def q8_bytes(rows, cols):
    return rows * cols + rows * (cols // 32) * 4 + 4 * cols + 4 * rows


def cpu_baseline(q_all, s_all, xs, threads, budget_s):
    """Times the oracle's AVX2 restatement (internal/num/dot_amd64.s block
    sums, quant.go qrow, rows split as matvec.go:90-104) on the same shapes
    for about budget_s seconds, and returns GB/s plus its outputs."""
    from oracle import oracle

    outs = [oracle.matvec_q8_avx2(q, s, x, r, c, threads) for (r, c), q, s, x in zip(SHAPES, q_all, s_all, xs)]
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        for (r, c), q, s, x in zip(SHAPES, q_all, s_all, xs):
            oracle.matvec_q8_avx2(q, s, x, r, c, threads)
        reps += 1
    el = time.perf_counter() - t0
    gbs = reps * sum(q8_bytes(r, c) for r, c in SHAPES) / el / 1e9
    return gbs, reps, el, outs


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--sets", type=int, default=4, help="weight copies rotated per step (>256 MB total)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py runs on one GPU only: this build has no multi-GPU path (row-sharding is described in "
              "DESIGN.md, not built). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import ctypes

    import rkhip

    dev = rkhip.Device(0)
    info = rkhip.device_info(0)
    rng = np.random.default_rng(1)
    q_all, s_all = [], []
    for r, c in SHAPES:
        q_all.append(rng.integers(-127, 128, r * c, dtype=np.int8))
        s_all.append(rng.uniform(1e-3, 1e-2, r * c // 32).astype(np.float32))
    xs = [rng.normal(0, 1, c).astype(np.float32) for _, c in SHAPES]
    sets = [[dev.upload_q8(q, s, r, c) for (r, c), q, s in zip(SHAPES, q_all, s_all)] for _ in range(args.sets)]
    # inputs and outputs in one arena (HBM)
    x_off, out_off, at = [], [], 0
    for _, c in SHAPES:
        x_off.append(at)
        at += c
    for r, _ in SHAPES:
        out_off.append(at)
        at += r
    arena = dev.arena(at, at)
    b = arena.begin()
    for o, x in zip(x_off, xs):
        b.write(o, x)
    b.submit()

    def sync():
        arena.begin().submit()

    L = rkhip.lib()
    P = ctypes.c_void_p
    calls = []
    for k in range(args.sets):
        for i, (r, c) in enumerate(SHAPES):
            calls.append(((P * 1)(sets[k][i].h), (P * 1)(arena.device_ptr(out_off[i])), P(arena.device_ptr(x_off[i])),
                          c))
    per_step = len(SHAPES)

    def run(steps, start):
        for st in range(start, start + steps):
            base = (st % args.sets) * per_step
            for j in range(per_step):
                hs, ops, xp, c = calls[base + j]
                rc = L.rk_matvecs_device(dev.h, 1, hs, ops, xp, c, None)
                if rc:
                    raise rkhip.RKError(rc, L.rk_last_error(dev.h).decode())

    # The timed steps run as HIP graph replays (one graph = one step per
    # weight copy), so the host's per-call cost does not pace the GPU.
    run(1, 0)
    sync()
    dev.graph_begin()
    run(args.sets, 0)
    g_full = dev.graph_end()
    rem = args.steps % args.sets
    g_rem = None
    if rem:
        dev.graph_begin()
        run(rem, 0)
        g_rem = dev.graph_end()
    g_full.launch(max(1, args.warmup // args.sets))
    t0 = time.perf_counter()
    g_full.launch(args.steps // args.sets)
    if g_rem:
        g_rem.launch(1)
    t1 = time.perf_counter()
    # The same steps again, eagerly, with each kernel's dispatch stamped by
    # HIP events on its own stream (the library's profile): per-kernel times.
    dev.profile_start()
    run(args.steps, args.warmup)
    sync()
    prof = dev.profile_stop()
    ms_per_step = (t1 - t0) / args.steps * 1e3
    step_bytes = sum(q8_bytes(r, c) for r, c in SHAPES)
    value = step_bytes / (ms_per_step / 1e3) / 1e9

    calls_mv, ms_mv = prof.get("matvec_q8", (0, 0.0))
    avg_launch_ms = ms_mv / max(calls_mv, 1)
    bytes_per_launch = step_bytes / per_step  # average over the three shapes
    achieved = bytes_per_launch / (avg_launch_ms / 1e3) / 1e9

    # per-shape kernel times in a second, profiled pass (one shape at a time)
    per_shape = {}
    for i, (r, c) in enumerate(SHAPES):
        dev.profile_start()
        for st in range(50):
            hs, ops, xp, cc = calls[(st % args.sets) * per_step + i]
            L.rk_matvecs_device(dev.h, 1, hs, ops, xp, cc, None)
        sync()
        p = dev.profile_stop()
        n, ms = p["matvec_q8"]
        us = ms / n * 1e3
        per_shape[f"{r}x{c}"] = {"kernel_us": round(us, 3), "GB/s": round(q8_bytes(r, c) / (us / 1e6) / 1e9, 1),
                                 "frac": round(q8_bytes(r, c) / (us / 1e6) / 1e9 / HBM_PEAK_GBS, 4)}

    result = {
        "metric": "Q8 matvec HBM GB/s (% of peak) + decode tok/s, 8B-shape batch 1",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: Q8_0 codes U[-127,127], scales U(1e-3,1e-2), x N(0,1); weights rotated over "
                f"{args.sets} HBM copies ({args.sets * step_bytes / 1e6:.0f} MB)",
        "config": {"workload": "config 2: Q8_0 group-32 matvec, batch 1, shapes 4096x4096 + 14336x4096 + "
                               "4096x14336 per step (quantize + product each)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "matvec_q8", "avg_launch_us": round(avg_launch_ms * 1e3, 3),
                     "bytes_per_launch": bytes_per_launch},
        "per_shape": per_shape,
        "kernels_ms": {k: [v[0], round(v[1], 4)] for k, v in prof.items()},
        "decode_tok_s": None,
        "device": {"name": info.name.decode(), "arch": info.arch.decode(), "cu": info.compute_units},
    }
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        gbs, reps, el, outs = cpu_baseline(q_all, s_all, xs, threads, args.cpu_seconds)
        gpu_outs = []
        ms0 = sets[0]
        for i, (r, c) in enumerate(SHAPES):
            gpu_outs.append(dev.matvec(ms0[i], xs[i]))
        exact = all(np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(outs, gpu_outs))
        result["cpu_baseline"] = {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
                                  "sample": f"{reps} passes over the three config-2 products in {el:.1f} s "
                                            "(C restatement of the reference CPU path, AVX2, rows over threads)",
                                  "bit_exact_vs_gpu": bool(exact)}
    g_full.free()
    if g_rem:
        g_rem.free()
    arena.free()
    for st in sets:
        for m in st:
            m.free()
    dev.close()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
