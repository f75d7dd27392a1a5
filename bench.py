#!/usr/bin/env python3
"""Benchmark of the Q8 matvec hot path on one MI355X.

Two measurements, one JSON line:

* value (GB/s): config 2. A step is one activation vector through the three
  Q8_0 products 4096x4096, 14336x4096 and 4096x14336; each product
  quantizes its input and multiplies, as num.MatVecQ8 does
  (internal/num/quant.go:167-180). Weights are synthetic (codes uniform in
  [-127, 127], scales U(1e-3, 1e-2)), resident in HBM before timing and
  rotated over copies totalling more than the 256 MB Infinity Cache, so every
  step streams its weights from HBM. value = algorithmic bytes of a step /
  step time, a product's bytes being rows*cols (codes) + rows*cols/32*4
  (scales) + 4*cols (x) + 4*rows (out). The timed steps are HIP graph
  replays. roofline = the product kernel's bytes per launch over its
  average duration, each launch stamped with HIP events on its own stream.
* prefill_tok_s / decode_q4_tok_s: config 4, a Qwen-7B-shape decoder with
  Q4_0 layers: a 512-token prompt through the batched prefill (int8 MFMA
  block sums, the per-token f32 steps on the vector ALUs), then batch-1
  decode. The products' int8 multiply-accumulate rate is reported against
  the MFMA peak and against the ceiling the f32 steps set.
* decode_tok_s: config 3, an 8B-shape llama decoder with random Q8 weights
  (dim 4096, 32 layers, 32 q / 8 kv heads of 128, SwiGLU 14336, vocab
  128256, RoPE theta 5e5, f32 KV cache): greedy decode of 256 tokens after
  a 512-token seeded prompt, entirely on the device (one recorded graph per
  token). decode_tok_s = decoded tokens / decode wall time.

cpu_baseline: the C restatement of the reference CPU path (AVX2 block sums,
rows over threads; test infrastructure under oracle/) on this host, on a
bounded sample of config 2, bit-compared with the GPU's outputs.
"""
import argparse
import ctypes
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
METRIC = "Q8 matvec HBM GB/s (% of peak) + decode tok/s, 8B-shape batch 1"


def q8_bytes(rows, cols):
    return rows * cols + rows * (cols // 32) * 4 + 4 * cols + 4 * rows


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def code_pool(rng, n):
    """n random Q8 codes in [-127, 127] (uniform bytes from the generator's
    raw words, -128 moved to -127: fast at model sizes)."""
    q = rng.bit_generator.random_raw((n + 7) // 8).view(np.int8)[:n].copy()
    q[q == -128] = -127
    return q


def cpu_baseline(q_all, s_all, xs, threads, budget_s):
    """Times the oracle's AVX2 restatement (internal/num/dot_amd64.s block
    sums, quant.go qrow, rows split as matvec.go:90-104) on the config-2
    shapes for about budget_s seconds; returns GB/s, passes, seconds and the
    first pass's outputs."""
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


def matvec_bench(dev, rkhip, args):
    rng = np.random.default_rng(1)
    q_all, s_all = [], []
    for r, c in SHAPES:
        q_all.append(code_pool(rng, r * c))
        s_all.append(rng.uniform(1e-3, 1e-2, r * c // 32).astype(np.float32))
    xs = [rng.normal(0, 1, c).astype(np.float32) for _, c in SHAPES]
    sets = [[dev.upload_q8(q, s, r, c) for (r, c), q, s in zip(SHAPES, q_all, s_all)] for _ in range(args.sets)]
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

    # Timed steps: the warmup steps, then exactly `steps` steps, each recorded
    # as one HIP graph (the weight copies rotating from step to step). The
    # timed graph is one replay bracketed by two events on the device
    # stream, after a synchronisation and before another: ms_per_step is
    # device time. The host clock around the same call is reported beside it.
    run(1, 0)
    sync()
    g_warm = None
    if args.warmup > 0:
        dev.graph_begin()
        run(args.warmup, 0)
        g_warm = dev.graph_end()
    dev.graph_begin()
    run(args.steps, args.warmup)
    g_timed = dev.graph_end()
    if g_warm:
        g_warm.launch(1)
    t0 = time.perf_counter()
    dev_ms = g_timed.launch_timed(1)
    t1 = time.perf_counter()
    ms_per_step = dev_ms / args.steps
    host_ms_per_step = (t1 - t0) / args.steps * 1e3
    step_bytes = sum(q8_bytes(r, c) for r, c in SHAPES)
    value = step_bytes / (ms_per_step / 1e3) / 1e9

    # The same steps eagerly, each launch stamped by HIP events on its stream.
    dev.profile_start()
    run(args.steps, args.warmup)
    sync()
    prof = dev.profile_stop()
    calls_mv, ms_mv = prof.get("matvec_q8", (0, 0.0))
    avg_launch_ms = ms_mv / max(calls_mv, 1)
    bytes_per_launch = step_bytes / per_step  # the three shapes, equally often
    achieved = bytes_per_launch / (avg_launch_ms / 1e3) / 1e9

    per_shape = {}
    for i, (r, c) in enumerate(SHAPES):
        dev.profile_start()
        for st in range(100):
            hs, ops, xp, cc = calls[(st % args.sets) * per_step + i]
            L.rk_matvecs_device(dev.h, 1, hs, ops, xp, cc, None)
        sync()
        p = dev.profile_stop()
        entry = {}
        for k, (n, ms) in p.items():
            entry[k + "_us"] = round(ms / n * 1e3, 3)
        us = p["matvec_q8"][1] / p["matvec_q8"][0] * 1e3
        entry["GB/s"] = round(q8_bytes(r, c) / (us / 1e6) / 1e9, 1)
        entry["frac"] = round(q8_bytes(r, c) / (us / 1e6) / 1e9 / HBM_PEAK_GBS, 4)
        # the floor under a launch that reads these bytes: back-to-back plain
        # reads of the same size (rotated past the MALL) and empty launches
        nb16 = q8_bytes(r, c) // 16 * 16
        empty_us, read_us = dev.launch_floor(nb16, copies=max(2, -(-600_000_000 // nb16)), launches=200)
        entry["plain_read_us"] = round(read_us, 3)
        entry["empty_launch_us"] = round(empty_us, 3)
        entry["plain_read_frac"] = round(q8_bytes(r, c) / (read_us / 1e6) / 1e9 / HBM_PEAK_GBS, 4)
        entry["frac_of_plain_read"] = round(read_us / us, 4)
        per_shape[f"{r}x{c}"] = entry

    out = {
        "value": round(value, 2), "ms_per_step": round(ms_per_step, 5),
        "host_ms_per_step": round(host_ms_per_step, 5),
        "data": "synthetic: Q8_0 codes U[-127,127], scales U(1e-3,1e-2), x N(0,1); weights rotated over "
                f"{args.sets} HBM copies ({args.sets * step_bytes / 1e6:.0f} MB)",
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": pmc_traffic(), "kernel": "matvec_q8",
                     "avg_launch_us": round(avg_launch_ms * 1e3, 3), "bytes_per_launch": bytes_per_launch},
        "per_shape": per_shape,
        "kernels_ms": {k: [v[0], round(v[1], 4)] for k, v in prof.items()},
    }
    gpu_outs = [dev.matvec(sets[0][i], xs[i]) for i in range(len(SHAPES))]
    g_timed.free()
    if g_warm:
        g_warm.free()
    arena.free()
    for st in sets:
        for m in st:
            m.free()
    return out, (q_all, s_all, xs, gpu_outs)


def measure_speed_weights(rows, cols):
    """MeasureSpeed's weights (internal/llm/speed.go:20-25): an LCG seed
    s = s·1664525 + 1013904223 per element, w = ToBF16(float32(int32(s>>8) -
    2^23) / 2^30), computed in closed form (s_k = a^k·s_0 + c·(1 + a + ... +
    a^(k-1)) mod 2^32); x_i = float32(i mod 17) / 17."""
    n = rows * cols
    a = np.full(n, 1664525, np.uint64)
    ak = np.cumprod(a)                                    # a^k, k = 1..n (mod 2^64)
    geo = np.cumsum(np.concatenate(([np.uint64(1)], ak[:-1])))  # 1 + a + ... + a^(k-1)
    seed = ((ak * np.uint64(1) + np.uint64(1013904223) * geo) & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    v = ((seed >> 8).astype(np.int32) - (1 << 23)).astype(np.float32) / np.float32(1 << 30)
    b = v.view(np.uint32).astype(np.uint64)
    w16 = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    x = (np.arange(cols) % 17).astype(np.float32) / np.float32(17)
    return w16, x


def dense_bench(dev, rkhip, args):
    """The planner's speed probe (internal/llm/speed.go:16-47 MeasureSpeed):
    products with a 4096x4096 bfloat16 matrix, reported as GB of weights per
    second. Device-resident products rotated over copies past the MALL
    (graph replays; roofline_frac is a product's bytes over its share of the
    replay time, launch gaps included), and the reference's own measure
    (median of 7 host round trips, input and output copies included). A
    float32 matrix of the same shape beside it."""
    rows = cols = 4096
    w16, x = measure_speed_weights(rows, cols)
    w32 = (w16.astype(np.uint32) << 16).view(np.float32)
    out = {}
    L = rkhip.lib()
    P = ctypes.c_void_p
    for name, kind, w, es in (("bf16", rkhip.BF16, w16, 2), ("f32", rkhip.F32, w32, 4)):
        wbytes = rows * cols * es
        copies = max(2, int(600e6 // wbytes) + 1)
        ms = [dev.upload(kind, rows, cols, w) for _ in range(copies)]
        arena = dev.arena(cols + rows, cols)
        b = arena.begin()
        b.write(0, x)
        b.submit()
        xp, op = P(arena.device_ptr(0)), (P * 1)(arena.device_ptr(cols))
        hs = [(P * 1)(m.h) for m in ms]

        def run(n, start=0):
            for k in range(start, start + n):
                rc = L.rk_matvecs_device(dev.h, 1, hs[k % copies], op, xp, cols, None)
                if rc:
                    raise rkhip.RKError(rc, L.rk_last_error(dev.h).decode())

        run(copies)
        arena.begin().submit()
        dev.graph_begin()
        run(copies)
        g = dev.graph_end()
        g.launch(2)
        reps = max(1, 400 // copies)
        t0 = time.perf_counter()
        g.launch(reps)
        t1 = time.perf_counter()
        per = (t1 - t0) / (reps * copies)
        alg = wbytes + 4 * cols + 4 * rows
        rt = []
        for _ in range(8):
            s0 = time.perf_counter()
            dev.matvec(ms[0], x)
            rt.append(time.perf_counter() - s0)
        rt = sorted(rt[1:])
        got = dev.matvec(ms[0], x)
        g.free()
        arena.free()
        for m in ms:
            m.free()
        out[name] = {"weights_GB_s": round(wbytes / per / 1e9, 1), "us_per_product": round(per * 1e6, 3),
                     "roofline_frac": round(alg / per / 1e9 / HBM_PEAK_GBS, 4),
                     "round_trip_GB_s": round(2 * rows * cols / rt[len(rt) // 2] / 1e9, 1),
                     "copies": copies}
        if name == "bf16" and not args.no_cpu:
            from oracle import oracle

            want = oracle.matvec_bf16(w16, x, rows, cols)
            n, c0 = 0, time.perf_counter()
            while time.perf_counter() - c0 < min(3.0, args.cpu_seconds):
                oracle.matvec_bf16(w16, x, rows, cols)
                n += 1
            el = time.perf_counter() - c0
            out[name]["bit_exact_vs_cpu"] = bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))
            out[name]["cpu_baseline"] = {"weights_GB_s": round(n * 2 * rows * cols / el / 1e9, 2), "cores": 1,
                                         "kind": "port", "sample": f"{n} products in {el:.1f} s (scalar C "
                                         "restatement of MatVecBF16, one thread)"}
    return {"measure_speed": {"config": "MeasureSpeed: 4096x4096 bfloat16 (LCG weights as speed.go), f32 input "
                              "i%17/17; float32 matrix of the same values beside it", **out}}


MX_SHAPES = [  # DeepSeek-V4.1's decode products (dim 5120, q_lora 1280, 64x512 heads, 2304-wide experts)
    ("fp8", 32768, 1280, "wq_b: q_lora 1280 -> 64 heads x 512"),
    ("fp8", 5120, 8192, "wo_b: 8 x 1024 -> dim"),
    ("fp4", 13824, 5120, "6 routed experts' gate rows stacked (6 x 2304)"),
    ("fp4", 5120, 2304, "one expert's down projection"),
]


def mx_bench(dev, rkhip, args):
    """DeepSeek-V4.1 block-scaled products (internal/num/mx.go MatVecFP8 /
    MatVecFP4 through internal/gpu): E4M3 / E2M1 weights with E8M0 scales,
    the input quantized on the device each call. Device-resident products
    rotated over copies past the MALL (graph replays); roofline_frac is a
    product's bytes (weights + scales + input codes and scales + output)
    over its share of the replay time, the input's quantize and launch gaps
    included. One product per format checked bit for bit against the CPU
    oracle, which is also timed (one thread)."""
    L = rkhip.lib()
    P = ctypes.c_void_p
    rng = np.random.default_rng(41)
    out = []
    for kind, rows, cols, what in MX_SHAPES:
        x = rng.normal(0, 1, cols).astype(np.float32)
        nb = cols // 32
        if kind == "fp8":
            w = rng.integers(0, 0x7E, rows * cols, dtype=np.uint8) | (rng.integers(0, 2, rows * cols, dtype=np.uint8) << 7)
            sc = rng.integers(118, 128, (rows + 31) // 32 * nb).astype(np.uint8)
            fmt, wbytes = rkhip.FP8, rows * cols
        else:
            w = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
            sc = rng.integers(118, 128, rows * nb).astype(np.uint8)
            fmt, wbytes = rkhip.FP4, rows * cols // 2
        alg = wbytes + sc.size + cols + 4 * nb + 4 * rows
        copies = max(2, int(600e6 // wbytes) + 1)
        ms = [dev.upload_mx(fmt, rows, cols, w, sc) for _ in range(copies)]
        arena = dev.arena(cols + rows, cols)
        b = arena.begin()
        b.write(0, x)
        b.submit()
        xp, op = P(arena.device_ptr(0)), (P * 1)(arena.device_ptr(cols))
        hs = [(P * 1)(m.h) for m in ms]

        def run(n):
            for k in range(n):
                rc = L.rk_matvecs_device(dev.h, 1, hs[k % copies], op, xp, cols, None)
                if rc:
                    raise rkhip.RKError(rc, L.rk_last_error(dev.h).decode())

        run(copies)
        arena.begin().submit()
        dev.graph_begin()
        run(copies)
        g = dev.graph_end()
        g.launch(2)
        reps = max(1, 400 // copies)
        t0 = time.perf_counter()
        g.launch(reps)
        per = (time.perf_counter() - t0) / (reps * copies)
        got = dev.matvecs([ms[0]], x)[0]
        g.free()
        arena.free()
        for m in ms:
            m.free()
        r = {"format": kind, "shape": f"{rows}x{cols}", "matrix": what, "weights_MB": round((wbytes + sc.size) / 1e6, 1),
             "us_per_product": round(per * 1e6, 3), "weights_GB_s": round((wbytes + sc.size) / per / 1e9, 1),
             "roofline_frac": round(alg / per / 1e9 / HBM_PEAK_GBS, 4), "copies": copies}
        if not args.no_cpu and (rows, cols) in ((5120, 8192), (5120, 2304)):
            from oracle import oracle

            mv = oracle.matvec_fp8 if kind == "fp8" else oracle.matvec_fp4
            want = mv(w, sc, x, rows, cols)
            n, c0 = 0, time.perf_counter()
            while time.perf_counter() - c0 < min(3.0, args.cpu_seconds):
                mv(w, sc, x, rows, cols)
                n += 1
            el = time.perf_counter() - c0
            r["bit_exact_vs_cpu"] = bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))
            r["cpu_baseline"] = {"weights_GB_s": round(n * (wbytes + sc.size) / el / 1e9, 3), "cores": 1,
                                 "kind": "port", "sample": f"{n} products in {el:.1f} s (scalar C restatement of "
                                 f"MatVec{kind.upper()}, one thread)"}
        log(f"  {kind} {rows}x{cols}: {r['us_per_product']} us/product, {r['weights_GB_s']} GB/s "
            f"(frac {r['roofline_frac']})")
        out.append(r)
    # selected experts (ExpertMatVecs): 6 of 64 E2M1 experts of 2304 rows a
    # call, the ids rotated over 10 sets (60 experts, past the MALL)
    E, P, cols, slots = 64, 2304, 5120, 6
    nb = cols // 32
    w = rng.integers(0, 256, E * P * cols // 2, dtype=np.uint8)
    sc = rng.integers(118, 128, E * P * nb).astype(np.uint8)
    x = rng.normal(0, 1, cols).astype(np.float32)
    m = dev.upload_mx(rkhip.FP4, E * P, cols, w, sc)
    sets = [np.arange(slots, dtype=np.uint32) * 10 + k for k in range(10)]
    idw, outw = cols, cols + 64
    qx = outw + slots * P
    arena = dev.arena(qx + 2 * cols, 2 * cols + slots * P)
    arena.set_quant_scratch(qx, qx + cols // 4)
    b = arena.begin()
    b.write(0, x)
    for k, ids in enumerate(sets):
        b.write(idw + 6 * k, ids.view(np.float32))
    b.submit()

    def call(k):
        bb = arena.begin()
        bb.expert_matvecs(m, P, idw + 6 * (k % 10), slots, 0, cols, 0, outw, P)
        bb.submit()

    for k in range(10):
        call(k)
    t0 = time.perf_counter()
    for k in range(200):
        call(k)
    call_us = (time.perf_counter() - t0) / 200 * 1e6
    ebytes = slots * (P * cols // 2 + P * nb)
    b = arena.begin()
    b.expert_matvecs(m, P, idw, slots, 0, cols, 0, outw, P)
    got = np.asarray(b.read(outw, slots * P)).reshape(slots, P)
    b.submit()
    r = {"format": "fp4", "shape": f"{slots} of {E} experts, {P}x{cols} each", "matrix": "ExpertMatVecs: one token's "
         "routed experts' gate rows", "weights_MB": round(ebytes / 1e6, 1),
         "us_per_batch_call": round(call_us, 3),
         "timing": "wall time of a Batch (begin, input quantize, products, submit and wait) per call; the "
                   "kernel's own duration is in the kernel trace"}
    if not args.no_cpu:
        from oracle import oracle

        e = int(sets[0][2])
        want = oracle.matvec_fp4(w[e * P * cols // 2:(e + 1) * P * cols // 2], sc[e * P * nb:(e + 1) * P * nb], x, P,
                                 cols)
        r["bit_exact_vs_cpu"] = bool(np.array_equal(got[2].view(np.uint32), want.view(np.uint32)))
    log(f"  fp4 experts {slots}x{P}x{cols}: {r['us_per_batch_call']} us a batch call")
    out.append(r)
    arena.free()
    m.free()
    return {"deepseek_mx": out}


PMC_COPY_WORDS = 1 << 26  # the calibration copy: 256 MiB read, 256 MiB written
PMC_SUMMARY = os.path.join(ROOT, "profiles", "q8_matvec_config2_pmc.md")


def pmc_pass(dev, rkhip, args):
    """What the PMC runs count (rocprofv3 --pmc FETCH_SIZE, then
    WRITE_SIZE): each config-2 product as rk_matvecs_device runs it,
    `steps` times over the rotated weight copies, then one copy kernel of
    PMC_COPY_WORDS words, whose counters against its known bytes give the
    scale of each counter."""
    rng = np.random.default_rng(1)
    sets = []
    for _ in range(args.sets):
        sets.append([dev.upload_q8(rng.integers(-127, 128, r * c, dtype=np.int8),
                                   rng.uniform(1e-3, 1e-2, r * c // 32).astype(np.float32), r, c) for r, c in SHAPES])
    at, offs = 0, []
    for r, c in SHAPES:
        offs.append((at, at + c))
        at += r + c
    arena = dev.arena(max(at, 2 * PMC_COPY_WORDS), sum(c for _, c in SHAPES))
    b = arena.begin()
    for (xo, _), (r, c) in zip(offs, SHAPES):
        b.write(xo, rng.normal(0, 1, c).astype(np.float32))
    b.submit()
    for st in range(args.steps):
        for i, (r, c) in enumerate(SHAPES):
            xo, oo = offs[i]
            dev.matvecs_device([sets[st % args.sets][i]], [arena.device_ptr(oo)], arena.device_ptr(xo), c)
    arena.begin().submit()
    b = arena.begin()
    b.copy(0, PMC_COPY_WORDS, PMC_COPY_WORDS)
    b.submit()
    arena.free()
    for st in sets:
        for m in st:
            m.free()
    log(f"pmc pass: {args.steps} x {len(SHAPES)} products, one copy of {PMC_COPY_WORDS} words")


def pmc_traffic():
    """HBM bytes per matvec_q8 launch from the committed PMC summary (the
    `traffic_bytes_per_launch` line), or None."""
    try:
        for line in open(PMC_SUMMARY):
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def rope_table(theta, hs, n):
    """Rotary table [n][hs/2] (NewRope's formula, internal/llm/model.go:
    428-441) in numpy float64: a synthetic input here, timing only."""
    half = hs // 2
    p = np.arange(half, dtype=np.float64)
    freq = np.exp(-np.log(theta) * (2 * p) / hs)
    ang = np.arange(n, dtype=np.float64)[:, None] * freq[None, :]
    return np.cos(ang).astype(np.float32).ravel(), np.sin(ang).astype(np.float32).ravel()


def decode_bench(dev, rkhip, args):
    """Config 3: 8B-shape Q8 decoder, greedy, entirely on the device."""
    dim, hidden, heads, kv_heads, hs, vocab = 4096, 14336, 32, 8, 128, 128256
    layers, prompt_len, steps = args.layers, args.prompt, args.decode
    ctx = prompt_len + steps
    kvdim = kv_heads * hs
    rng = np.random.default_rng(3)
    # Codes come from one random pool at per-matrix offsets (distinct
    # matrices without generating 8 GB on the host); scales keep the
    # activations finite through the layers.
    pool = code_pool(rng, vocab * dim + (1 << 20))
    spool = rng.uniform(2e-5, 2e-4, vocab * dim // 32 + (1 << 16)).astype(np.float32)
    mats = []

    def mat(rows, cols):
        n = rows * cols
        o = int(rng.integers(0, pool.size - n + 1))
        so = int(rng.integers(0, spool.size - n // 32 + 1))
        m = dev.upload_q8(pool[o:o + n], spool[so:so + n // 32], rows, cols)
        mats.append(m)
        return m

    t0 = time.perf_counter()
    lay = []
    for li in range(layers):
        lay.append({"wq": mat(dim, dim), "wk": mat(kvdim, dim), "wv": mat(kvdim, dim), "wo": mat(dim, dim),
                    "w1": mat(hidden, dim), "w2": mat(dim, hidden), "w3": mat(hidden, dim),
                    "rms_att": rng.normal(1, 0.1, dim).astype(np.float32),
                    "rms_ffn": rng.normal(1, 0.1, dim).astype(np.float32)})
    embed, wcls = mat(vocab, dim), mat(vocab, dim)
    log(f"decode bench: {layers} layers uploaded in {time.perf_counter() - t0:.1f} s")
    cos, sin = rope_table(500000.0, hs, ctx)
    st = rkhip.Stage(dev, dim, hidden, heads, kv_heads, ctx, lay, cos, sin, head_dim=hs, norm_eps=1e-5)
    st.set_head(embed, wcls, rng.normal(1, 0.1, dim).astype(np.float32))
    prompt = rng.integers(0, vocab, prompt_len).astype(np.int32)

    if args.eager:  # one launch at a time (for tools that cannot follow graph replays)
        dev.profile_start()
    # warm-up: records the graph, touches every weight once
    st.generate_start(prompt)
    st.generate_run(4)
    st.generate_start(prompt)
    t0 = time.perf_counter()
    st.generate_run(prompt_len)  # positions 0..prompt-1; the last yields the first new token
    t1 = time.perf_counter()
    st.generate_run(steps - 1)   # each position: layers + logits + argmax -> the next token
    t2 = time.perf_counter()
    if args.eager:
        dev.profile_stop()
    toks = st.tokens(prompt_len, steps)
    decode_s = t2 - t1
    tok_s = (steps - 1) / decode_s
    # per-kernel times over 8 decode positions after the prompt (launched one
    # by one while profiling, each launch stamped by HIP events)
    if args.eager:
        dev.profile_start()
    st.generate_start(prompt)
    st.generate_run(prompt_len)
    if args.eager:
        dev.profile_stop()
    dev.profile_start()
    st.generate_run(8)
    prof = dev.profile_stop()
    # The same loop drawing from softmax(logits / 0.8) with a seeded
    # xorshift64* state on the device (sample.go:26-43): the step ends with
    # the sampler's launches instead of the argmax's.
    st.sampler(0.8, 1234)
    if args.eager:
        dev.profile_start()
    st.generate_start(prompt)
    st.generate_run(prompt_len)
    t3 = time.perf_counter()
    st.generate_run(steps - 9)
    t4 = time.perf_counter()
    if args.eager:
        dev.profile_stop()
    dev.profile_start()
    st.generate_run(8)
    prof_s = dev.profile_stop()
    toks_s = st.tokens(prompt_len, 8)
    weight_bytes = sum(m.bytes for m in mats) - embed.bytes
    kv_bytes = layers * 2 * kvdim * 4 * (prompt_len + steps / 2)  # average positions read per decode step
    per_token = weight_bytes + kv_bytes + 4 * vocab
    ms_tok = decode_s / (steps - 1) * 1e3
    out = {
        "decode_tok_s": round(tok_s, 2),
        "decode": {"config": f"config 3: dim {dim}, {layers} layers, {heads} q / {kv_heads} kv heads of {hs}, "
                             f"ffn {hidden}, vocab {vocab}, RoPE theta 5e5, f32 KV; greedy {steps} tokens after a "
                             f"{prompt_len}-token seeded prompt; random Q8 codes, scales U(2e-5, 2e-4)",
                   "ms_per_token": round(ms_tok, 4), "prefill_s": round(t1 - t0, 4),
                   "prefill_tok_s": round(prompt_len / (t1 - t0), 2),
                   "bytes_per_token": int(per_token),
                   "effective_GB/s": round(per_token / (ms_tok / 1e3) / 1e9, 1),
                   "frac_of_hbm_peak": round(per_token / (ms_tok / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                   "first_tokens": [int(t) for t in toks[:8]],
                   "kernels_us_per_token": {k: round(v[1] / 8 * 1e3, 2) for k, v in prof.items()},
                   "kernel_launches_per_token": {k: v[0] // 8 for k, v in prof.items()}},
        "decode_sampled": {"temperature": 0.8, "seed": 1234,
                           "tok_s": round((steps - 9) / (t4 - t3), 2),
                           "ms_per_token": round((t4 - t3) / (steps - 9) * 1e3, 4),
                           "sample_us_per_token": round(prof_s.get("sample", (0, 0.0))[1] / 8 * 1e3, 2),
                           "first_tokens": [int(t) for t in toks_s]},
    }
    st.free()
    for m in mats:
        m.free()
    return out


INT8_MFMA_PEAK_TMACS = 2500.0   # MI355X dense int8: 5.0 POPS = 2.5 P multiply-accumulates/s
VALU_PEAK_TOPS = 39.32          # 256 CUs x 4 SIMD x 16 lanes x 2.4 GHz, non-packed f32 lane-ops/s


def prefill_bench(dev, rkhip, args):
    """Config 4: Qwen-7B-shape decoder with Q4_0 layers (Q8 embedding and
    classifier): the 512-token prompt through the batched prefill (int8 MFMA
    block sums, per-token f32 epilogue), then batch-1 greedy decode."""
    dim, hidden, heads, kv_heads, hs, vocab = 3584, 18944, 28, 4, 128, 152064
    layers, prompt_len, steps = args.prefill_layers, args.prefill_prompt, args.prefill_decode
    ctx = prompt_len + steps
    qdim, kvdim = heads * hs, kv_heads * hs
    rng = np.random.default_rng(4)
    pool = rng.integers(0, 256, hidden * dim // 2 + (1 << 20), dtype=np.uint8)
    pool8 = code_pool(rng, vocab * dim + (1 << 20))
    spool = rng.uniform(2e-5, 2e-4, vocab * dim // 32 + (1 << 16)).astype(np.float32)
    mats = []

    def mat(rows, cols, q4=True):
        n = rows * cols
        src = pool if q4 else pool8
        nbytes = n // 2 if q4 else n
        o = int(rng.integers(0, src.size - nbytes + 1))
        so = int(rng.integers(0, spool.size - n // 32 + 1))
        m = (dev.upload_q4 if q4 else dev.upload_q8)(src[o:o + nbytes], spool[so:so + n // 32], rows, cols)
        mats.append(m)
        return m

    t0 = time.perf_counter()
    lay = []
    for _ in range(layers):
        lay.append({"wq": mat(qdim, dim), "wk": mat(kvdim, dim), "wv": mat(kvdim, dim), "wo": mat(dim, qdim),
                    "w1": mat(hidden, dim), "w2": mat(dim, hidden), "w3": mat(hidden, dim),
                    "rms_att": rng.normal(1, 0.1, dim).astype(np.float32),
                    "rms_ffn": rng.normal(1, 0.1, dim).astype(np.float32),
                    "bq": rng.normal(0, 0.5, qdim).astype(np.float32),
                    "bk": rng.normal(0, 0.5, kvdim).astype(np.float32),
                    "bv": rng.normal(0, 0.5, kvdim).astype(np.float32)})
    embed, wcls = mat(vocab, dim, False), mat(vocab, dim, False)
    log(f"prefill bench: {layers} layers uploaded in {time.perf_counter() - t0:.1f} s")
    cos, sin = rope_table(1000000.0, hs, ctx)
    st = rkhip.Stage(dev, dim, hidden, heads, kv_heads, ctx, lay, cos, sin, head_dim=hs, norm_eps=1e-6,
                     qkv_bias=True)
    st.set_head(embed, wcls, rng.normal(1, 0.1, dim).astype(np.float32))
    prompt = rng.integers(0, vocab, prompt_len).astype(np.int32)
    # warm-up (batch buffers, graphs), then the timed prompt and decode
    if args.eager:  # one launch at a time (for tools that cannot follow graph replays)
        dev.profile_start()
    st.generate_start(prompt)
    st.generate_run(prompt_len)
    st.generate_start(prompt)
    t0 = time.perf_counter()
    st.generate_run(prompt_len - 1)  # positions 0..prompt-2: the batched path
    t1 = time.perf_counter()
    st.generate_run(1)               # the last prompt position: the first new token
    t2 = time.perf_counter()
    st.generate_run(steps - 1)
    t3 = time.perf_counter()
    if args.eager:
        dev.profile_stop()
    # per-kernel times of the batched prompt, launches stamped one by one
    st.generate_start(prompt)
    dev.profile_start()
    st.generate_run(prompt_len - 1)
    prof = dev.profile_stop()
    n_pre = prompt_len - 1
    layer_weights = qdim * dim + 2 * kvdim * dim + dim * qdim + 3 * hidden * dim
    macs = float(n_pre) * layers * layer_weights
    mm_ms = sum(prof.get(k, (0, 0.0))[1] for k in ("qkv", "wo", "w13", "w2"))
    mm_tmacs = macs / (mm_ms / 1e3) / 1e12 if mm_ms else None
    pre_s = t1 - t0
    dec_s = t3 - t2
    out = {
        "prefill_tok_s": round(n_pre / pre_s, 1),
        "prefill": {
            "config": f"config 4: Qwen-7B shape, dim {dim}, {layers} layers, {heads} q / {kv_heads} kv heads of "
                      f"{hs}, ffn {hidden}, vocab {vocab}, QKV bias, RoPE theta 1e6; Q4_0 layers, Q8_0 embedding "
                      f"and classifier; random codes, scales U(2e-5, 2e-4); {prompt_len}-token seeded prompt",
            "tokens": n_pre, "seconds": round(pre_s, 4), "ms_per_layer": round(pre_s / layers * 1e3, 3),
            "products_int8_macs": macs,
            "products_ms": round(mm_ms, 3),
            "products_TMAC_s": round(mm_tmacs, 1) if mm_tmacs else None,
            "mfma_frac_of_int8_peak": round(mm_tmacs / INT8_MFMA_PEAK_TMACS, 4) if mm_tmacs else None,
            # each (row, token, block) needs cvt, mul, mul, add on the vector ALUs in a fixed order:
            # 4 lane-ops per 32 MACs cap the products at VALU_PEAK * 8 MACs
            "f32_step_ceiling_TMAC_s": round(VALU_PEAK_TOPS * 8, 1),
            "frac_of_f32_step_ceiling": round(mm_tmacs / (VALU_PEAK_TOPS * 8), 4) if mm_tmacs else None,
            "kernels_ms": {k: round(v[1], 3) for k, v in prof.items()},
        },
        "decode_q4_tok_s": round((steps - 1) / dec_s, 2),
        "decode_q4": {"config": "config 4, batch-1 greedy decode after the prompt",
                      "steps": steps - 1, "ms_per_token": round(dec_s / (steps - 1) * 1e3, 4)},
    }
    st.free()
    for m in mats:
        m.free()
    return out


def moe_bench(dev, rkhip, args):
    """Config 5: a Qwen3-MoE-shape decoder, 48 layers (dim 2048, 32 q / 4 kv
    heads of 128 with QK-norm, 128 Q8 experts of ffn 768, Q8 router, top 8,
    vocab 151936), greedy decode entirely on the device: batch 1 (one
    sequence, one recorded graph per token) and batch 16 (16 independent
    sequences, each with its own prompt, position and caches; one recorded
    graph per step, each selected expert's rows read once per step for all
    the sequences that chose it). Every layer's matrices are distinct device
    copies (codes from one random pool at per-matrix offsets)."""
    dim, heads, kv_heads, hs, experts, ehidden, topk, vocab = 2048, 32, 4, 128, 128, 768, 8, 151936
    nl, prompt_len, steps = args.moe_layers, args.moe_prompt, args.moe_decode
    ctx = prompt_len + steps
    qdim, kvdim = heads * hs, kv_heads * hs
    rng = np.random.default_rng(5)
    pool = code_pool(rng, vocab * dim + (1 << 20))
    spool = rng.uniform(2e-5, 2e-4, vocab * dim // 32 + (1 << 16)).astype(np.float32)
    mats = []

    def mat(rows, cols, lo=1.0):
        n = rows * cols
        o = int(rng.integers(0, pool.size - n + 1))
        so = int(rng.integers(0, spool.size - n // 32 + 1))
        m = dev.upload_q8(pool[o:o + n], spool[so:so + n // 32] * np.float32(lo), rows, cols)
        mats.append(m)
        return m

    t0 = time.perf_counter()
    lay, moes = [], []
    for _ in range(nl):
        moe = rkhip.Moe(dev, mat(experts, dim, 10.0), [mat(ehidden, dim) for _ in range(experts)],
                        [mat(dim, ehidden) for _ in range(experts)], [mat(ehidden, dim) for _ in range(experts)], topk)
        moes.append(moe)
        lay.append({"wq": mat(qdim, dim), "wk": mat(kvdim, dim), "wv": mat(kvdim, dim), "wo": mat(dim, qdim),
                    "moe": moe, "rms_att": rng.normal(1, 0.1, dim).astype(np.float32),
                    "rms_ffn": rng.normal(1, 0.1, dim).astype(np.float32),
                    "q_norm": rng.normal(1, 0.1, hs).astype(np.float32),
                    "k_norm": rng.normal(1, 0.1, hs).astype(np.float32)})
    embed = mat(vocab, dim)
    rms_final = rng.normal(1, 0.1, dim).astype(np.float32)
    log(f"moe bench: {nl} layers ({len(mats)} matrices) uploaded in {time.perf_counter() - t0:.1f} s")
    cos, sin = rope_table(1000000.0, hs, ctx)
    q8 = lambda r, c: r * c + r * (c // 32) * 4  # noqa: E731
    attn_bytes = q8(qdim + 2 * kvdim, dim) + q8(dim, qdim)
    expert_bytes = 2 * q8(ehidden, dim) + q8(dim, ehidden)
    router_bytes = q8(experts, dim)
    cls_bytes = q8(vocab, dim)
    kv_read = 2 * kvdim * 4 * (prompt_len + steps / 2)  # one sequence's cache reads per layer, average position
    out = {}
    for batch in (1, 16):
        st = rkhip.Stage(dev, dim, ehidden, heads, kv_heads, ctx, lay, cos, sin, head_dim=hs, norm_eps=1e-6,
                         qk_norm=True, seqs=batch)
        st.set_head(embed, embed, rms_final)
        prompts = [[int(t) for t in rng.integers(0, vocab, prompt_len)] for _ in range(batch)]
        if batch == 1:
            def start():
                st.generate_start(prompts[0])
                st.generate_run(prompt_len)  # the prompt (batched) and its last position's token

            def run(n):
                st.generate_run(n)
        else:
            def start():
                st.seqs_start(prompts)

            def run(n):
                st.seqs_run(n)
        if args.eager:  # one launch at a time (for tools that cannot follow graph replays)
            dev.profile_start()
        start()
        run(2)  # records the graph, touches every weight
        start()
        st.moe_stats()  # the device's grouping counters restart here
        t0 = time.perf_counter()
        run(steps - 1)
        el = time.perf_counter() - t0
        selected, groupings = st.moe_stats()
        if args.eager:
            dev.profile_stop()
        ms_step = el / (steps - 1) * 1e3

        def start_outside_profile():  # (batch 1's start runs the prompt: eager too under --eager)
            if args.eager:
                dev.profile_start()
            start()
            if args.eager:
                dev.profile_stop()

        # per-kernel times: eager launches stamped one by one, after one
        # unstamped eager step (the first eager launches pay one-time host
        # work between a kernel's start event and its dispatch)
        start_outside_profile()
        dev.profile_start()
        run(1)
        dev.profile_stop()
        start_outside_profile()
        dev.profile_start()
        run(4)
        prof = dev.profile_stop()
        # distinct experts a step streams per layer: the 8 selected at batch
        # 1; at batch 16 the device's own count, each layer's grouping of the
        # step's (token, slot) pairs summed over the timed steps
        if batch == 1:
            distinct = topk
        else:
            if groupings != nl * (steps - 1):
                raise RuntimeError(f"moe bench: {groupings} groupings for {nl} layers x {steps - 1} steps")
            distinct = selected / groupings
        step_bytes = nl * (attn_bytes + router_bytes + distinct * expert_bytes + batch * kv_read) + cls_bytes
        out[f"batch{batch}"] = {
            "tok_s": round(batch / (ms_step / 1e3), 1),
            "ms_per_step": round(ms_step, 4),
            "tokens_per_step": batch,
            "distinct_experts_per_layer": round(distinct, 2),
            "distinct_experts_source": "top-k" if batch == 1 else "device grouping count",
            "bytes_per_step": int(step_bytes),
            "effective_GB/s": round(step_bytes / (ms_step / 1e3) / 1e9, 1),
            "frac_of_hbm_peak": round(step_bytes / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "kernels_us_per_step": {k: round(v[1] / 4 * 1e3, 2) for k, v in prof.items()},
            "kernel_launches_per_step": {k: v[0] // 4 for k, v in prof.items()},
        }
        log(f"  batch {batch}: {out[f'batch{batch}']['tok_s']} tok/s, {ms_step:.3f} ms a step")
        st.free()
    for m in moes:
        m.free()
    for m in mats:
        m.free()
    return {"moe_decode_tok_s": out["batch1"]["tok_s"], "moe_decode_b16_tok_s": out["batch16"]["tok_s"],
            "moe": {"config": f"config 5: dim {dim}, {nl} layers, {heads} q / {kv_heads} kv heads of {hs} with "
                              f"QK-norm, {experts} Q8 experts of ffn {ehidden}, Q8 router, top {topk}, vocab {vocab}, "
                              f"RoPE theta 1e6, f32 KV; greedy {steps} tokens after {prompt_len}-token seeded "
                              f"prompts, batch 1 and 16 independent sequences; random Q8 codes, scales U(2e-5, "
                              f"2e-4) (router x10)", **out}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--sets", type=int, default=8, help="weight copies rotated per step (1.2 GB: far past the 256 MB MALL)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--decode", type=int, default=256)
    ap.add_argument("--eager", action="store_true", help="decode without graph replays (for profilers)")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="only the launches the PMC runs count (config-2 products and a calibration copy)")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--no-dense", action="store_true")
    ap.add_argument("--no-mx", action="store_true")
    ap.add_argument("--moe-layers", type=int, default=48)
    ap.add_argument("--moe-prompt", type=int, default=64)
    ap.add_argument("--moe-decode", type=int, default=64)
    ap.add_argument("--prefill-layers", type=int, default=28)
    ap.add_argument("--prefill-prompt", type=int, default=512)
    ap.add_argument("--prefill-decode", type=int, default=64)
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py runs on one GPU: this build has no multi-GPU path (the products' sharding is a "
              "design, not built). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import rkhip

    dev = rkhip.Device(0)
    info = rkhip.device_info(0)
    if args.pmc_pass:
        pmc_pass(dev, rkhip, args)
        dev.close()
        return
    log("matvec bench (config 2)")
    mv, (q_all, s_all, xs, gpu_outs) = matvec_bench(dev, rkhip, args)
    result = {
        "metric": METRIC,
        "value": mv.pop("value"),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": mv.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": mv.pop("data"),
        "config": {"workload": "config 2: Q8_0 group-32 matvec, batch 1, shapes 4096x4096 + 14336x4096 + "
                               "4096x14336 per step (quantize + product each)"},
    }
    result.update(mv)
    result["decode_tok_s"] = None
    if not args.no_decode:
        log("decode bench (config 3)")
        result.update(decode_bench(dev, rkhip, args))
    if not args.no_prefill:
        log("prefill bench (config 4)")
        result.update(prefill_bench(dev, rkhip, args))
    if not args.no_moe:
        log("moe bench (config 5)")
        result.update(moe_bench(dev, rkhip, args))
    if not args.no_dense:
        log("dense bench (MeasureSpeed)")
        result.update(dense_bench(dev, rkhip, args))
    if not args.no_mx:
        log("DeepSeek-V4.1 block-scaled products")
        result.update(mx_bench(dev, rkhip, args))
    result["device"] = {"name": info.name.decode(), "arch": info.arch.decode(), "cu": info.compute_units}
    if not args.no_cpu:
        log("cpu baseline")
        # every CPU this process may run on, up to the 16 threads a one-GPU
        # job is allotted on the GPU hosts (nproc and the affinity set are
        # reported beside it)
        nproc = os.cpu_count() or 1
        try:
            avail = len(os.sched_getaffinity(0))
        except (AttributeError, OSError):
            avail = nproc
        threads = max(1, min(16, avail))
        gbs, reps, el, outs = cpu_baseline(q_all, s_all, xs, threads, args.cpu_seconds)
        exact = all(np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(outs, gpu_outs))
        gbs1, reps1, el1, _ = cpu_baseline(q_all, s_all, xs, 1, min(4.0, args.cpu_seconds))
        result["cpu_baseline"] = {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
                                  "sample": f"{reps} passes over the three config-2 products in {el:.1f} s "
                                            "(C restatement of the reference CPU path: AVX2 block sums, rows "
                                            "over threads)",
                                  "host_nproc": nproc, "cpus_available": avail,
                                  "threads_rule": "all CPUs available to the process, at most the 16 threads a "
                                                  "one-GPU job is allotted on the GPU host",
                                  "one_thread": {"value": round(gbs1, 2), "unit": "GB/s", "cores": 1,
                                                 "sample": f"{reps1} passes in {el1:.1f} s"},
                                  "bit_exact_vs_gpu": bool(exact)}
    dev.close()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
