#!/usr/bin/env python3
"""Benchmark of the MI355X contraction / permutation hot path.

Prints ONE compact JSON line last on stdout (under 4000 bytes). The headline (`value`) is
fp32 contraction TFLOP/s on the north-star workload, C[4096,4096] = A[4096,4096] .
B[4096,4096] row-major (a "step" is one such contraction over resident HBM inputs). The same
line carries the permutation headline (GB/s on the 1 GiB-traffic [512,1024,256] perm (2,0,1)
materialization) and a [value, unit, roofline frac] summary of every benchmark configuration;
each workload's full record (plan, kernels, median/best, CPU baselines) goes to the --detail
file. Rooflines:
  contraction: achieved = 2*B*M*N*K / mean kernel time, peak = 157.3 TFLOP/s fp32 MFMA
  permutation: achieved = 2*numel*4 B / mean kernel time,  peak = 8000 GB/s HBM
Kernel time is measured with HIP events recorded on the stream the kernels are launched on,
around `steps` back-to-back launches after `warmup` untimed ones (and at least `--warmup-ms`
of untimed launches, so short kernels reach the steady clock), with the stream synchronized
on both sides. The CPU baseline times the C restatement of crates/cpu on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME] [--no-cpu]
                       [--detail FILE]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "pipeline-parallelism-deep-learning-library_amd"))
sys.path.insert(0, str(REPO))

METRIC = "contraction TFLOP/s (% fp32 MFMA peak); permute GB/s (% HBM peak)"
PEAK_TFLOPS = 157.3     # MI355X dense fp32 MFMA
PEAK_GBS = 8000.0       # MI355X HBM3E
PEAK_F64_TFLOPS = 78.6  # MI355X dense fp64 MFMA
# MI355X published fp32 vector peak. The 16-bit Backend gemm spends two f32 operations (one
# multiply, one add, never fused) per term; it is priced against this figure.
PEAK_VECTOR_TFLOPS = 157.3


class HipEvents:
    """hipEvent timing on a given stream (the library's own stream)."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        vp, pvp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
        self.hip.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
        self.hip.hipStreamEndCapture.argtypes = [vp, pvp]
        self.hip.hipGraphInstantiate.argtypes = [pvp, vp, vp, ctypes.c_char_p, ctypes.c_size_t]
        self.hip.hipGraphLaunch.argtypes = [vp, vp]
        self.hip.hipGraphExecDestroy.argtypes = [vp]
        self.hip.hipGraphDestroy.argtypes = [vp]

    def new(self):
        ev = ctypes.c_void_p()
        assert self.hip.hipEventCreate(ctypes.byref(ev)) == 0
        return ev

    def destroy(self, *evs):
        for ev in evs:
            assert self.hip.hipEventDestroy(ev) == 0

    def record(self, ev, stream):
        assert self.hip.hipEventRecord(ev, stream) == 0

    def elapsed_ms(self, a, b) -> float:
        assert self.hip.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return float(ms.value)


HOST_MS = {}  # host ms per enqueue call of the last timed() loop, by launch closure
WARMUP_MS = 30.0  # least wall time of untimed launches per workload (--warmup-ms)


def warm_up(ctx, launch, warmup):
    """`warmup` untimed launches, then as many more as fill WARMUP_MS of wall time. The shader
    clock settles over ~10-20 ms of a new load: 50 launches of a 90 us product (4.5 ms) time
    config 4 at 90 us, 200 or more at 80-82 us, so short kernels get a time floor."""
    t0 = time.perf_counter()
    for _ in range(warmup):
        launch()
    ctx.sync()
    spent = time.perf_counter() - t0
    if WARMUP_MS > 0 and warmup > 0 and spent * 1e3 < WARMUP_MS:
        per = spent / warmup
        for _ in range(int((WARMUP_MS / 1e3 - spent) / max(per, 1e-6)) + 1):
            launch()
        ctx.sync()


def timed(ctx, events, launch, steps, warmup):
    """Mean ms per launch over `steps` launches, bracketed by stream syncs. The host time of
    the enqueue loop is kept in HOST_MS: when it approaches the device time, the launches are
    bound by the caller's enqueue rate rather than by the kernels."""
    warm_up(ctx, launch, warmup)
    s = ctx.queue.handle
    e0, e1 = events.new(), events.new()
    events.record(e0, s)
    t0 = time.perf_counter()
    for _ in range(steps):
        launch()
    HOST_MS[launch] = (time.perf_counter() - t0) * 1e3 / steps
    events.record(e1, s)
    total = events.elapsed_ms(e0, e1)
    ctx.sync()
    events.destroy(e0, e1)
    return total / steps


def native_lib():
    from linalg_hip import _native
    return _native.lib()


GRAPH_BELOW_MS = 0.1  # workloads faster than this per step also get a graph-replay figure
GRAPH_REPLAYS = 5


def graph_rate(ctx, events, launch, steps):
    """Device ms per step when `steps` enqueues are captured once into a HIP graph and the
    graph is replayed: the caller's enqueue rate drops out. Through ctypes each enqueue costs
    ~7 us of host time, which bounds the back-to-back rate of the smallest products; a
    compiled caller spends ~3.4 us (2.7 of them in the HIP launch itself). None if the
    capture fails."""
    hip, s = events.hip, ctx.queue.handle
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipStreamBeginCapture(s, 1) != 0:  # hipStreamCaptureModeThreadLocal
        return None
    try:
        for _ in range(steps):
            launch()
    finally:
        ended = hip.hipStreamEndCapture(s, ctypes.byref(graph))
    try:
        if ended != 0 or hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) != 0:
            return None
        assert hip.hipGraphLaunch(exe, s) == 0  # untimed
        ctx.sync()
        e0, e1 = events.new(), events.new()
        events.record(e0, s)
        for _ in range(GRAPH_REPLAYS):
            assert hip.hipGraphLaunch(exe, s) == 0
        events.record(e1, s)
        total = events.elapsed_ms(e0, e1)
        ctx.sync()
        events.destroy(e0, e1)
        return total / (GRAPH_REPLAYS * steps)
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)


def per_launch(ctx, events, launch, n):
    """(median, best) ms of `n` launches each bracketed by its own event pair, taken after the
    timed loop (the way tests/contraction_test.rs:1199-1217 reports best and median)."""
    s = ctx.queue.handle
    pairs = [(events.new(), events.new()) for _ in range(n)]
    for a, b in pairs:
        events.record(a, s)
        launch()
        events.record(b, s)
    ms = sorted(events.elapsed_ms(a, b) for a, b in pairs)
    ctx.sync()
    for a, b in pairs:
        events.destroy(a, b)
    return ms[len(ms) // 2], ms[0]


def abi_call(fn, *args):
    """A launch closure over the C ABI entry point `fn` with its descriptors built once, the
    way a compiled caller holds its lg_view structs: the timed loop measures the library's
    own per-call cost (planning, validation, launch), not Python's struct building."""
    refs = [ctypes.byref(a) if isinstance(a, ctypes.Structure) else a for a in args]
    keep = args  # the structs outlive the closure's byrefs

    def launch():
        st = fn(*refs)
        if st != 0:
            raise RuntimeError(f"{fn.__name__} returned {st} ({keep[0]!r})")
    return launch


def upload(pool, L, data: np.ndarray):
    buf = pool.alloc("f32", data.size)
    buf.write(data)
    return buf


def kernels_of(ctx, call):
    """Run `call` once and return the names of the kernels it launched (the launch log)."""
    lib = native_lib()
    before = lib.lg_debug_launch_count(ctx.handle)
    call()
    after = lib.lg_debug_launch_count(ctx.handle)
    names = (lib.lg_debug_launch_name(ctx.handle, i) for i in range(max(before, after - 256), after))
    return sorted(set(n.decode() for n in names if n))


def bench_gemm(ctx, events, pool, L, C, name, m, n, k, args, a_t=False, b_t=False, batch=1,
               seed=(12, 13), sigma=None, beta=0.0):
    g = np.random.Generator(np.random.PCG64(seed[0]))
    h = np.random.Generator(np.random.PCG64(seed[1]))
    if sigma is None:
        a = g.uniform(-1, 1, batch * m * k).astype(np.float32)
        b = h.uniform(-1, 1, batch * k * n).astype(np.float32)
    else:
        a = (g.standard_normal(batch * m * k) * sigma).astype(np.float32)
        b = (h.standard_normal(batch * k * n) * sigma).astype(np.float32)
    A, B = upload(pool, L, a), upload(pool, L, b)
    Cb = pool.alloc("f32", batch * m * n)
    bs = [] if batch == 1 else [batch]
    av = (L.TensorView(A, 0, bs + [m, k], ([m * k] if bs else []) + [1, m]) if a_t
          else L.TensorView.row_major(A, 0, bs + [m, k]))
    bv = (L.TensorView(B, 0, bs + [k, n], ([k * n] if bs else []) + [1, k]) if b_t
          else L.TensorView.row_major(B, 0, bs + [k, n]))
    cv = L.TensorView.row_major(Cb, 0, bs + [m, n])
    plan = C.plan_gemm(1.0, av, bv, beta, cv)
    # Validated once through Python.
    kernels = kernels_of(ctx, lambda: C.encode_gemm(ctx, ctx.queue, 1.0, av, bv, beta, cv))
    launch = abi_call(native_lib().lg_encode_gemm_f32, ctx.handle, ctx.queue.handle,
                      ctypes.c_float(1.0), av.to_c(), bv.to_c(), ctypes.c_float(beta), cv.to_c())
    ms = timed(ctx, events, launch, args.steps, args.warmup)
    med, best = per_launch(ctx, events, launch, args.steps)
    flops = 2.0 * batch * m * n * k
    tflops = flops / (ms * 1e-3) / 1e12
    extra = {}
    if ms < GRAPH_BELOW_MS:
        g = graph_rate(ctx, events, launch, args.steps)
        if g:
            extra = {"ms_graph": g, "tflops_graph": flops / (g * 1e-3) / 1e12}
    return {"name": name, "ms": ms, "ms_median": med, "ms_best": best,
            "host_ms": HOST_MS[launch], "tflops": tflops, **extra,
            "frac": tflops / PEAK_TFLOPS,
            "plan": {k_: plan[k_] for k_ in ("kind", "kernel", "tile", "a_mode", "b_mode",
                                              "splits", "workgroups")},
            "kernels": kernels, "_host": (a, b), "_geom": (m, n, k, a_t, b_t, batch, beta)}


def bench_perm(ctx, events, pool, L, P, name, shape, perm, seed, args):
    n = int(np.prod(shape))
    x = np.random.Generator(np.random.PCG64(seed)).uniform(-1, 1, n).astype(np.float32)
    src_buf = upload(pool, L, x)
    dst_buf = pool.alloc("f32", n)
    src = P.permute_view(L.TensorView.row_major(src_buf, 0, shape), perm)
    dst = L.TensorView.row_major(dst_buf, 0, src.shape)
    plan = P.plan("materialize", src, dst)
    kernels = kernels_of(ctx, lambda: P.encode_materialize(ctx, ctx.queue, src, dst))
    launch = abi_call(native_lib().lg_encode_materialize, ctx.handle, ctx.queue.handle, src.elem,
                      src.to_c(), dst.to_c())
    ms = timed(ctx, events, launch, args.steps, args.warmup)
    med, best = per_launch(ctx, events, launch, args.steps)
    gbs = 2.0 * n * 4 / (ms * 1e-3) / 1e9
    return {"name": name, "ms": ms, "ms_median": med, "ms_best": best,
            "host_ms": HOST_MS[launch], "gbs": gbs, "frac": gbs / PEAK_GBS,
            "plan": {k_: plan[k_] for k_ in ("kind", "vector", "workgroups", "shape")},
            "kernels": kernels, "_host": x, "_geom": (list(shape), list(perm))}


def bench_copy(ctx, events, pool, L, P, n, args):
    """A plain 128-bit copy through the same library (contiguous materialize)."""
    src_buf = pool.alloc("f32", n)
    dst_buf = pool.alloc("f32", n)
    src = L.TensorView.row_major(src_buf, 0, [n])
    dst = L.TensorView.row_major(dst_buf, 0, [n])
    launch = abi_call(native_lib().lg_encode_materialize, ctx.handle, ctx.queue.handle, src.elem,
                      src.to_c(), dst.to_c())
    ms = timed(ctx, events, launch, args.steps, args.warmup)
    return 2.0 * n * 4 / (ms * 1e-3) / 1e9


def bench_contract(ctx, events, pool, L, C, name, a_spec, b_spec, c_spec, args, seed=42):
    """One contraction of the reference's own benchmark list (tests/contraction_test.rs:
    1293-1395, bench_other_paths): each spec is (shape, strides, labels), inputs uniform in
    [-1, 1), beta = 0. FLOP = 2 * product of every label's extent; algorithmic bytes = A and B
    read once plus C written once. The roofline is whichever of the fp32 MFMA peak and the HBM
    peak binds at that intensity."""
    g = np.random.Generator(np.random.PCG64(seed))
    bufs, views, host = [], [], []
    for i, (shape, strides, labels) in enumerate((a_spec, b_spec, c_spec)):
        span = 1 + sum((e - 1) * st for e, st in zip(shape, strides))
        buf = pool.alloc("f32", span)
        if i < 2:
            x = g.uniform(-1, 1, span).astype(np.float32)
            buf.write(x)
            host.append(x)
        views.append((L.TensorView(buf, 0, shape, strides), labels))
    extents = {}
    for (v, labels) in views:
        extents.update(zip(labels, v.shape))
    flops = 2.0 * float(np.prod([float(e) for e in extents.values()]))
    nbytes = 4.0 * sum(float(np.prod(v.shape)) for v, _ in views)
    plan = C.plan_contract(1.0, views[0], views[1], 0.0, views[2])
    kernels = kernels_of(ctx, lambda: C.encode_contract(ctx, ctx.queue, 1.0, views[0], views[1],
                                                        0.0, views[2]))
    (av, la), (bv, lb), (cv, lc) = views
    launch = abi_call(native_lib().lg_encode_contract_f32, ctx.handle, ctx.queue.handle,
                      ctypes.c_float(1.0), av.to_c(), la.encode(), bv.to_c(), lb.encode(),
                      ctypes.c_float(0.0), cv.to_c(), lc.encode())
    ms = timed(ctx, events, launch, args.steps, args.warmup)
    med, best = per_launch(ctx, events, launch, args.steps)
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = nbytes / (ms * 1e-3) / 1e9
    extra = {}
    if ms < GRAPH_BELOW_MS:
        g = graph_rate(ctx, events, launch, args.steps)
        if g:
            extra = {"ms_graph": g, "tflops_graph": flops / (g * 1e-3) / 1e12,
                     "gbs_graph": nbytes / (g * 1e-3) / 1e9}
    mfma_bound = flops / (PEAK_TFLOPS * 1e12) >= nbytes / (PEAK_GBS * 1e9)
    roof = ({"bound": "mfma", "achieved": tflops, "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
             "frac": tflops / PEAK_TFLOPS} if mfma_bound else
            {"bound": "hbm", "achieved": gbs, "peak": PEAK_GBS, "unit": "GB/s",
             "frac": gbs / PEAK_GBS})
    return {"name": name, "ms": ms, "ms_median": med, "ms_best": best, "host_ms": HOST_MS[launch],
            "tflops": tflops, "gbs": gbs, **extra, "flop": flops, "bytes": nbytes, "roofline": roof,
            "plan": {k_: plan[k_] for k_ in ("kind", "kernel", "tile", "a_mode", "b_mode",
                                              "splits", "workgroups", "swapped")},
            "kernels": kernels, "_other": (host, [(v.shape, v.strides, l) for v, l in views])}


def other_paths_specs():
    """(key, name, a, b, c) of the reference's bench_other_paths (tests/contraction_test.rs:
    1293-1395); shapes with their strides and labels."""
    def dense(shape):
        st, p = [], 1
        for e in reversed(shape):
            st.append(p)
            p *= e
        return list(shape), st[::-1]

    def cm(r, c):  # Layout::transposed(rows, cols): column-major
        return [r, c], [1, r]
    n2, k16, k1 = 2048, 1 << 24, 1 << 20
    return [
        ("o_t2048", "transposed 2048 (A, B, C column-major)", (*cm(n2, n2), "mk"),
         (*cm(n2, n2), "kn"), (*cm(n2, n2), "mn")),
        ("o_batched", "batched 4096 x 32^3", (*dense([4096, 32, 32]), "bmk"),
         (*dense([4096, 32, 32]), "bkn"), (*dense([4096, 32, 32]), "bmn")),
        ("o_dot", "dot K=16M", (*dense([1, k16]), "mk"), (*dense([k16, 1]), "kn"),
         (*dense([1, 1]), "mn")),
        ("o_32k1m", "32x32 K=1M (B column-major)", (*dense([32, k1]), "mk"), (*cm(k1, 32), "kn"),
         (*dense([32, 32]), "mn")),
        ("o_rank1", "rank-1 4096^2", (*dense([4096, 1]), "mk"), (*dense([1, 4096]), "kn"),
         (*dense([4096, 4096]), "mn")),
        ("o_rank4", "rank-4 ijkl,klmn->ijmn 48^6", (*dense([48] * 4), "ijkl"),
         (*dense([48] * 4), "klmn"), (*dense([48] * 4), "ijmn")),
    ]


def cpu_other_rate(host, specs):
    """The literal crates/cpu loop (oracle.gemm_seq, one core) on a bounded sample of one
    bench_other_paths workload, on its own inputs: (FLOP, seconds, runs, what). Batched and
    merged-axis workloads run as the 2-D products crates/cpu would be called with."""
    import oracle
    (a_shape, a_st, la), (b_shape, b_st, lb), (c_shape, c_st, lc) = specs
    x, y = host
    if la == "bmk":  # one 32x32x32 product per batch: a sample of 256 batches
        bm, m, k = a_shape
        n = b_shape[2]
        c = np.zeros(m * n, np.float32)
        nb = 256

        def run():
            for i in range(nb):
                oracle.gemm_seq(m, n, k, 1.0, 0.0, x, i * m * k, (k, 1), y, i * k * n, (n, 1), c, 0,
                                (n, 1))
        what, flop = f"{nb} of {bm} batches", 2.0 * nb * m * n * k
    else:
        if la == "ijkl":
            e = a_shape[0] * a_shape[1]
            m = n = k = e
            sa, sb, sc = (e, 1), (e, 1), (e, 1)
        else:
            m, k = a_shape
            n = b_shape[1]
            sa, sb, sc = tuple(a_st), tuple(b_st), tuple(c_st)
        rows = max(1, min(m, int(2e8 // max(1, 2 * n * k))))  # about 0.2 GFLOP
        c = np.zeros(max(m * n, 1), np.float32)

        def run():
            for r in range(rows):
                oracle.gemm_seq(1, n, k, 1.0, 0.0, x, r * sa[0], sa, y, 0, sb, c, r * sc[0], sc)
        what, flop = f"{rows} of {m} output rows", 2.0 * rows * n * k
    runs, dt = repeat_for(run)
    return flop * runs, dt, runs, what


def bench_gemm_f16(ctx, events, pool, L, C, m, n, k, args):
    """f16 contraction (each output rounded once from an f64 dot on the f64 matrix cores):
    TFLOP/s against the 78.6 TFLOP/s f64 MFMA peak the kernel runs on."""
    g = np.random.Generator(np.random.PCG64(31))
    a = pool.alloc("f16", m * k)
    b = pool.alloc("f16", k * n)
    c = pool.alloc("f16", m * n)
    a.write(g.uniform(-1, 1, m * k).astype(np.float16))
    b.write(g.uniform(-1, 1, k * n).astype(np.float16))
    av = L.TensorView.row_major(a, 0, [m, k], "f16")
    bv = L.TensorView.row_major(b, 0, [k, n], "f16")
    cv = L.TensorView.row_major(c, 0, [m, n], "f16")
    plan = C.plan_gemm(1.0, av, bv, 0.0, cv)
    ms = timed(ctx, events, lambda: C.encode_gemm(ctx, ctx.queue, 1.0, av, bv, 0.0, cv),
               args.steps, args.warmup)
    tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    res = {"name": f"f16 gemm {m}x{n}x{k} (f64 accumulation, one f16 rounding)", "ms": ms,
           "ms_median": per_launch(ctx, events, lambda: C.encode_gemm(ctx, ctx.queue, 1.0, av, bv,
                                                                     0.0, cv), args.steps)[0],
           "tflops": tf, "frac_f64_mfma": tf / PEAK_F64_TFLOPS,
           "plan": {k_: plan[k_] for k_ in ("kind", "workgroups")}}
    if not args.no_cpu:
        # The f64 reference of tests/contraction_test.rs:200-268 (oracle/oracle.c), one
        # thread, on 16 output rows: the reference has no CPU f16 contraction of its own.
        import oracle
        ah = a.read(np.float16, 0, m * k).astype(np.float32)
        bh = b.read(np.float16, 0, k * n).astype(np.float32)
        rows = 16
        t0 = time.perf_counter()
        oracle.contract_f64(1.0, ah[: rows * k], (0, [rows, k], [k, 1]), "mk", bh, (0, [k, n], [n, 1]),
                            "kn", 0.0, np.zeros(rows * n, np.float32), (0, [rows, n], [n, 1]), "mn")
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": round(2.0 * rows * n * k / dt / 1e12, 6), "unit": "TFLOP/s",
                               "cores": 1, "kind": "port",
                               "sample": f"{rows} of {m} output rows, f64 reference loop ({dt:.2f} s)"}
    return res


def bench_backend_gemm16(events, args, timed_fn, m=4096, n=4096, k=4096):
    """Backend::gemm on F16 tensors, bit-exact with CpuBackend (one lane per output runs the
    reference's serial f32 chain): 10^12 terms (multiply-add pairs) per second, and the two f32
    operations per term against the published 157.3 TFLOP/s fp32 vector peak (which counts
    packed FMA; the chain can use neither packing nor fusion)."""
    import oracle
    from linalg_hip import backend as B
    hb = B.HipBackend(0)
    g = np.random.Generator(np.random.PCG64(37))
    a16 = oracle.f32_to_f16(g.uniform(-1, 1, m * k).astype(np.float32))
    b16 = oracle.f32_to_f16(g.uniform(-1, 1, k * n).astype(np.float32))
    ta = hb.upload(B.DType.F16, [m, k], a16.tobytes())
    tb = hb.upload(B.DType.F16, [k, n], b16.tobytes())
    tc = hb.alloc(B.DType.F16, [m, n])
    ms = timed_fn(hb.ctx, events, lambda: hb.gemm(ta, tb, tc, 1.0, 0.0), args.steps, args.warmup)
    terms = m * n * k / (ms * 1e-3) / 1e12
    res = {"name": f"Backend::gemm f16 {m}x{n}x{k} (CpuBackend's f32 chain, bit-exact)", "ms": ms,
           "tterms": terms, "tflops_vector": 2 * terms, "frac_vector": 2 * terms / PEAK_VECTOR_TFLOPS,
           "kernel": "gemm16_seq<0, 8>"}
    hb.close()
    if not args.no_cpu:
        rows = 4
        out = np.zeros((rows, n), np.uint16)
        t0 = time.perf_counter()
        oracle.gemm_seq_16("f16", 1.0, 0.0, a16.reshape(m, k)[:rows], b16.reshape(k, n), out)
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": round(rows * n * k / dt / 1e12, 6), "unit": "10^12 terms/s",
                               "cores": 1, "kind": "port",
                               "sample": f"{rows} of {m} output rows, CpuBackend's loop ({dt:.2f} s)"}
    return res


def bench_train_ops(events, args, timed_fn):
    """The Backend activation and training ops at the config-5 layer shape [4096, 16384]
    (Y = X.W of the 1F1B linear step): each op's algorithmic bytes / mean kernel time."""
    from linalg_hip import backend as B
    hb = B.HipBackend(0)
    rows, cols = 4096, 16384
    n = rows * cols
    g = np.random.Generator(np.random.PCG64(21))
    a = (g.standard_normal(n) * 0.5).astype(np.float32)
    b = (g.standard_normal(n) * 0.5).astype(np.float32)
    x = hb.upload_f32([rows, cols], a)
    t = hb.upload_f32([rows, cols], b)
    y = hb.alloc(B.DType.F32, [rows, cols])
    z = hb.alloc(B.DType.F32, [rows, cols])
    bias = hb.upload_f32([cols], a[:cols])
    db = hb.alloc(B.DType.F32, [cols])
    h = hb.alloc(B.DType.BF16, [rows, cols])
    f4, f2 = 4 * n, 2 * n
    ops = [
        ("gelu", lambda: hb.gelu(x, y), 2 * f4, "gelu_f32<true>"),
        ("gelu_backward", lambda: hb.gelu_backward(x, t, y), 3 * f4, "gelu_backward_f32<true>"),
        ("add_bias", lambda: hb.add_bias(x, bias, y), 2 * f4 + 4 * cols, "add_bias_f32<true>"),
        ("bias_grad", lambda: hb.bias_grad(x, db), f4 + 8 * cols, "bias_grad_f32"),
        ("mse_grad", lambda: hb.mse_grad(x, t, z), 3 * f4, "mse_grad_f32 (synchronous)"),
        ("sgd_step", lambda: hb.sgd_step(y, z, 1e-3), 4 * f4, "sgd_step_f32<true>"),
        ("convert_f32_bf16", lambda: hb.convert(x, h), f4 + f2, "convert_f32_bf16<true>"),
        ("convert_bf16_f32", lambda: hb.convert(h, y), f2 + f4, "convert_bf16_f32<true>"),
    ]
    out = {}
    for name, fn, nbytes, kernel in ops:
        ms = timed_fn(hb.ctx, events, fn, args.steps, args.warmup)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"ms": ms, "gbs": gbs, "frac": gbs / PEAK_GBS, "bytes": nbytes,
                     "kernel": kernel}
    hb.close()
    if not args.no_cpu:
        cpu_train_ops(out, a, b, rows, cols)
    out["_shape"] = [rows, cols]
    return out


def cpu_train_ops(out, a, b, rows, cols):
    """The crates/cpu loops (oracle/oracle.c, one thread) on a [1024, cols] slab of the same
    data, the same bytes-per-element accounting as the GPU figures."""
    import oracle
    r = 1024
    x = a[: r * cols].reshape(r, cols)
    t = b[: r * cols].reshape(r, cols)
    n = r * cols
    f4, f2 = 4 * n, 2 * n
    bias = a[:cols].copy()
    db = np.zeros(cols, np.float32)
    h = oracle.f32_to_bf16(x)
    jobs = [
        ("gelu", lambda: oracle.gelu(x), 2 * f4),
        ("gelu_backward", lambda: oracle.gelu_backward(x, t), 3 * f4),
        ("add_bias", lambda: oracle.add_bias(x, bias), 2 * f4),
        ("bias_grad", lambda: oracle.bias_grad(x, db), f4),
        ("mse_grad", lambda: oracle.mse_grad(x, t), 3 * f4),
        ("sgd_step", lambda: oracle.sgd_step(x, t, 1e-3), 4 * f4),
        ("convert_f32_bf16", lambda: oracle.f32_to_bf16(x), f4 + f2),
        ("convert_bf16_f32", lambda: oracle.bf16_to_f32(h), f2 + f4),
    ]
    for name, fn, nbytes in jobs:
        t0 = time.perf_counter()
        fn()
        dt = time.perf_counter() - t0
        out[name]["cpu_baseline"] = {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s",
                                     "cores": 1, "kind": "port",
                                     "sample": f"[{r}, {cols}] slab, crates/cpu loop ({dt:.2f} s)"}


def traffic_from_profile(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/traffic_<name>.txt)."""
    p = REPO / "profiles" / f"traffic_{name}.txt"
    if not p.exists():
        return None
    vals = {}
    for line in p.read_text().splitlines():
        if "=" in line and not line.startswith("#"):
            key, val = line.split("=", 1)
            vals[key.strip()] = val.strip()
    try:
        return float(vals["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


# Bounded CPU samples per GEMM workload: (literal rows, rows for the threaded variant or None
# for all, batches for the threaded variant). About 20 s of CPU work for the whole set.
CPU_GEMM_SAMPLES = {"gemm4096": (48, None, 1), "sq1024": (256, None, 1), "sq2048": (64, None, 1),
                    "c1": (512, None, 1), "c3": (32, None, 4),
                    "c4": (4, None, 1), "c5": (4, 256, 1)}


def host_cpu():
    """The host the CPU baselines ran on: model name, logical CPUs, the threads used."""
    model = "unknown"
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"model": model, "logical_cpus": os.cpu_count(),
            "threads_used": min(os.cpu_count() or 1, 16)}


def repeat_for(fn, min_s=0.25):
    """Runs fn until at least min_s seconds have passed (at least once): (runs, seconds), so
    the short samples are not timer noise."""
    runs, t0 = 0, time.perf_counter()
    while True:
        fn()
        runs += 1
        dt = time.perf_counter() - t0
        if dt >= min_s:
            return runs, dt


VENDOR_SHAPES = {"gemm4096": (1, 4096, 4096, 4096, False), "sq1024": (1, 1024, 1024, 1024, False),
                 "sq2048": (1, 2048, 2048, 2048, False), "c3": (32, 1024, 1024, 1024, True)}


def attach_vendor(results, args):
    """The vendor library on the same shapes (the reference times MPSMatrixMultiplication beside
    its own kernel): torch.matmul in fp32 with TF32 off, which runs hipBLASLt, timed with torch's
    events on torch's stream after the same warm-up. `ratio` = this library's TFLOP/s over
    the vendor's."""
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    dev = torch.device("cuda", 0)
    for name, (batch, m, n, k, b_t) in VENDOR_SHAPES.items():
        r = results.get(name)
        if not isinstance(r, dict) or "tflops" not in r:
            continue
        g = torch.Generator(device=dev).manual_seed(7)
        a = torch.rand((batch, m, k), device=dev, generator=g) * 2 - 1
        b = torch.rand((batch, n, k) if b_t else (batch, k, n), device=dev, generator=g) * 2 - 1
        # Config 3's B is a permuted view for this library; the vendor gets it contiguous.
        bb = b.transpose(1, 2).contiguous() if b_t else b
        c = torch.empty((batch, m, n), device=dev)
        step = (lambda: torch.matmul(a[0], bb[0], out=c[0])) if batch == 1 else \
            (lambda: torch.matmul(a, bb, out=c))
        t0 = time.perf_counter()
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        while time.perf_counter() - t0 < WARMUP_MS / 1e3:
            step()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        tf = 2.0 * batch * m * n * k / (ms * 1e-3) / 1e12
        r["vendor"] = {"tflops": tf, "ms": ms, "ratio": r["tflops"] / tf,
                       "library": "hipBLASLt through torch.matmul, fp32, TF32 off" +
                                  (", B contiguous" if b_t else "")}
        del a, b, c


def cpu_gemm_rates(host, geom, seq_rows, fast_rows, fast_batches, threads):
    """crates/cpu's gemm restated (oracle/): the literal single-thread k-order loop on the
    first `seq_rows` output rows, and the bit-identical loop-interchanged variant on `threads`
    threads, on the workload's own host inputs; FLOP and seconds of each sample."""
    import oracle
    a, b = host
    m, n, k, a_t, b_t, batch, beta = geom
    seq_rows, fast_batches = min(seq_rows, m), min(fast_batches, batch)
    fast_rows = None if fast_rows is None or fast_rows >= m else fast_rows
    a_st = (1, m) if a_t else (k, 1)
    b_st = (1, k) if b_t else (n, 1)
    c = np.zeros(m * n, np.float32)

    def literal():
        for r in range(seq_rows):
            oracle.gemm_seq(1, n, k, 1.0, beta, a, r * a_st[0], a_st, b, 0, b_st, c, r * n,
                            (n, 1))
    rows = None if fast_rows is None else np.arange(fast_rows, dtype=np.uint64)
    nr = (m if fast_rows is None else fast_rows) * fast_batches

    def threaded():
        for bi in range(fast_batches):
            oracle.gemm_fast(m, n, k, 1.0, beta, a, bi * m * k, a_st, b, bi * k * n, b_st, c, 0,
                             (n, 1), rows=rows, threads=threads)
    runs, dt = repeat_for(literal)
    seq = (2.0 * seq_rows * n * k * runs, dt, runs)
    runs, dt = repeat_for(threaded)
    fast = (2.0 * nr * n * k * runs, dt, runs)
    return seq, fast, (seq_rows, nr, batch * m)


def cpu_perm_rates(x, geom, threads):
    """gather_words restated (oracle/) over the whole permuted view, one thread and
    `threads` threads: bytes moved (one read + one write per word) and seconds."""
    import oracle
    shape, perm = geom
    words = x.view(np.uint32)
    st = [int(np.prod(shape[d + 1:], dtype=np.int64)) for d in range(len(shape))]
    pshape, pst = [shape[p] for p in perm], [st[p] for p in perm]
    nbytes = 2.0 * words.size * 4
    runs, dt = repeat_for(lambda: oracle.gather_words(words, 1, 0, pshape, pst))
    one = (nbytes * runs, dt, runs)
    runs, dt = repeat_for(lambda: oracle.gather_words_mt(words, 1, 0, pshape, pst,
                                                         threads=threads))
    par = (nbytes * runs, dt, runs)
    return one, par


def attach_cpu_baselines(results, threads):
    """Adds cpu_baseline (one core, the literal restatement) and cpu_baseline_parallel
    (`threads` cores, bit-identical) to every GEMM and permutation workload, timed on bounded
    samples of the workload's own inputs after all GPU timing is done."""
    def note(what, dt, runs):
        return f"{what} ({runs} runs, {dt:.2f} s)" if runs > 1 else f"{what} ({dt:.2f} s)"

    def tf(work, what, cores):
        flop, dt, runs = work
        return {"value": flop / dt / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
                "sample": note(what, dt, runs)}

    def gb(work, what, cores):
        nbytes, dt, runs = work
        return {"value": nbytes / dt / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
                "sample": note(what, dt, runs)}

    for name, r in results.items():
        if not isinstance(r, dict):
            continue
        if "_other" in r:
            flop, dt, runs, what = cpu_other_rate(*r.pop("_other"))
            r["cpu_baseline"] = tf((flop, dt, runs), f"{what}, literal k-order loop", 1)
            continue
        parts = r.get("parts") or [r]
        if all("_geom" in p and isinstance(p["_host"], tuple) for p in parts):
            spec = CPU_GEMM_SAMPLES.get(name)
            if spec is None:
                continue
            tot = [[0.0, 0.0, 1], [0.0, 0.0, 1]]
            for p in parts:
                seq, fast, (sr, fr, total_rows) = cpu_gemm_rates(p.pop("_host"), p.pop("_geom"),
                                                                 *spec, threads)
                p["cpu_baseline"] = tf(seq, f"{sr} of {total_rows} output rows, literal "
                                            "k-order loop", 1)
                p["cpu_baseline_parallel"] = tf(fast, f"{fr} of {total_rows} output rows, "
                                                      "bit-identical loop-interchanged variant "
                                                      f"on {threads} threads", threads)
                for i, w in enumerate((seq, fast)):
                    tot[i][0] += w[0]
                    tot[i][1] += w[1]
            if len(parts) > 1:
                r["cpu_baseline"] = tf(tot[0], "the three products' literal samples", 1)
                r["cpu_baseline_parallel"] = tf(tot[1], "the three products' threaded samples",
                                                threads)
        elif "_geom" in r:
            one, par = cpu_perm_rates(r.pop("_host"), r.pop("_geom"), threads)
            r["cpu_baseline"] = gb(one, "gather_words over the whole permuted view", 1)
            r["cpu_baseline_parallel"] = gb(par, "gather_words_mt over the whole permuted view, "
                                                 f"{threads} contiguous output ranges", threads)


LINE_LIMIT = 4000  # bytes of the final stdout line: the driver keeps only the tail of stdout

# Workloads summarised on the final line, in this order: {name: [value, unit, roofline frac]}.
SUMMARY_ORDER = ("gemm4096", "sq1024", "sq2048", "c1", "c3", "c4", "c5", "c2a", "c2b", "c2b_1g",
                 "copy", "t8191", "floor", "f16", "o_t2048", "o_batched", "o_dot", "o_32k1m",
                 "o_rank1", "o_rank4", "o_f16_2048")


def _r(x, nd=4):
    return round(x, nd) if isinstance(x, float) else x


def summary_entry(r):
    """[value, unit, frac] of one workload's result: the figure its roofline is priced in."""
    if "roofline" in r:
        roof = r["roofline"]
        return [_r(roof["achieved"], 2), roof["unit"], _r(roof["frac"])]
    if "frac_f64_mfma" in r:
        return [_r(r["tflops"], 2), "TFLOP/s f64-MFMA", _r(r["frac_f64_mfma"])]
    if "tflops" in r:
        return [_r(r["tflops"], 2), "TFLOP/s", _r(r["frac"])]
    if "gbs" in r:
        return [_r(r["gbs"], 1), "GB/s", _r(r.get("frac", r["gbs"] / PEAK_GBS))]
    if "ms" in r:
        return [_r(r["ms"] * 1e3, 2), "us", None]
    return None


def short_cpu(cb):
    return None if not cb else {k: _r(v, 6) for k, v in cb.items()}


def detail_record(results, args, train, bgemm16):
    """Every workload's full result (plan, kernels, per-launch median and best, graph-replay
    figures, CPU baselines): written to the --detail file, not to stdout."""
    rec = {"metric": METRIC, "steps": args.steps, "warmup": args.warmup,
           "warmup_min_ms": args.warmup_ms}
    rec["configs"] = {k_: {kk: _r(v) for kk, v in r.items()} for k_, r in results.items()}
    if train:
        rec["train_ops"] = {k_: ({kk: _r(v) for kk, v in r.items()} if isinstance(r, dict) else r)
                            for k_, r in train.items()}
    if bgemm16:
        rec["backend_gemm16"] = {k_: _r(v) for k_, v in bgemm16.items()}
    if not args.no_cpu:
        rec["cpu_host"] = host_cpu()
    return rec


def headline_line(results, args, train, bgemm16, detail_path):
    """The one JSON line printed last on stdout (under LINE_LIMIT bytes): the 4096^3 headline
    with its roofline and CPU baselines, the permutation headline, and a [value, unit, frac]
    summary of every other workload."""
    head = results.get("gemm4096")
    perm = results.get("c2b")
    line = {"metric": METRIC, "value": round(head["tflops"], 3) if head else None,
            "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(head["ms"], 4) if head else None, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "fp32 contraction C[4096,4096] = A.B row-major (4096^3)",
                       "m": 4096, "n": 4096, "k": 4096, "parallelism": "single-gpu"}}
    if head:
        line["roofline"] = {"bound": "mfma", "achieved": round(head["tflops"], 3),
                            "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                            "frac": round(head["frac"], 4),
                            "traffic": traffic_from_profile("gemm4096"),
                            "kernel": ", ".join(head.get("kernels", [])),
                            "algorithmic": "2*4096^3 FLOP per launch"}
        line["cpu_baseline"] = short_cpu(head.get("cpu_baseline"))
        line["cpu_baseline_parallel"] = short_cpu(head.get("cpu_baseline_parallel"))
    if perm:
        line["permute"] = {"value": round(perm["gbs"], 1), "unit": "GB/s",
                           "workload": "[512,1024,256] perm (2,0,1) materialize",
                           "ms_per_step": round(perm["ms"], 4),
                           "roofline": {"bound": "hbm", "achieved": round(perm["gbs"], 1),
                                        "peak": PEAK_GBS, "unit": "GB/s",
                                        "frac": round(perm["frac"], 4),
                                        "traffic": traffic_from_profile("c2b"),
                                        "kernel": ", ".join(perm.get("kernels", []))},
                           "cpu_baseline": short_cpu(perm.get("cpu_baseline")),
                           "cpu_baseline_parallel": short_cpu(perm.get("cpu_baseline_parallel"))}
    summ = {}
    for name in SUMMARY_ORDER:
        r = results.get(name)
        e = summary_entry(r) if isinstance(r, dict) else None
        if e is not None:
            summ[name] = e
    if bgemm16:
        summ["bgemm16"] = [_r(2 * bgemm16["tterms"], 2), "TFLOP/s f32 vector",
                           _r(2 * bgemm16["tterms"] / PEAK_VECTOR_TFLOPS)]
    if train:
        for op, r in train.items():
            if isinstance(r, dict) and "gbs" in r:
                summ[op] = [_r(r["gbs"], 1), "GB/s", _r(r["frac"])]
    line["configs_summary"] = summ
    if detail_path:
        line["detail"] = str(detail_path)
    # Dropping optional parts keeps the line parseable whatever the workload set.
    for key in ("detail", "cpu_baseline_parallel", "configs_summary"):
        if len(json.dumps(line)) <= LINE_LIMIT:
            break
        line.pop(key, None)
    return line


def main() -> int:
    global WARMUP_MS
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=50,
                    help="untimed launches before the timed ones; the MI355X needs tens of ms "
                         "of sustained MFMA load to reach its steady clock (5 launches of the "
                         "4096^3 GEMM measure ~7%% below steady state)")
    ap.add_argument("--warmup-ms", type=float, default=WARMUP_MS,
                    help="least wall time of untimed launches per workload after the --warmup "
                         "ones (short kernels need more than 50 launches to reach the steady "
                         "clock); 0 turns it off")
    ap.add_argument("--only", default=None,
                    help="run only these workloads (comma-separated): gemm4096, sq1024, sq2048, c1, c3, c4, c5, c2a, c2b, c2b_1g, copy, t8191, floor, "
                         "train, bgemm16, f16, o_t2048, o_batched, o_dot, o_32k1m, o_rank1, "
                         "o_rank4, o_f16_2048")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--vendor", action="store_true",
                    help="also time the vendor library on the square GEMMs and config 3, as the "
                         "reference's spec benchmark does against MPS: torch.matmul in fp32 with "
                         "TF32 off (hipBLASLt); imports torch")
    ap.add_argument("--prewarm", type=float, default=0.0,
                    help="seconds of 4096^3 GEMMs to run before any timing, so workloads timed "
                         "alone start at the steady shader clock")
    ap.add_argument("--detail", default=str(Path("gpurun_out") / "bench_detail.json"),
                    help="file for every workload's full result (the stdout line carries the "
                         "headline and a summary); empty to skip")
    args = ap.parse_args()
    WARMUP_MS = args.warmup_ms
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus above 1 is not supported",
                          "n_gpus": args.gpus}))
        return 2

    import linalg_hip as L
    from linalg_hip import contraction as C
    from linalg_hip import permutation as P
    sys.path.insert(0, str(REPO / "tests"))

    ctx = L.Context.new(0)
    events = HipEvents()

    class Pool:
        def __init__(self):
            self.b = []

        def alloc(self, dt, n):
            buf = L.alloc_shared(ctx, dt, n)
            self.b.append(buf)
            return buf

        def free(self):
            for x in self.b:
                x.free()
            self.b = []

    pool = Pool()
    only = args.only
    results = {}

    wanted = None if only is None else set(only.split(","))
    if args.prewarm > 0:
        pool_warm = [L.alloc_shared(ctx, "f32", 4096 * 4096) for _ in range(3)]
        vs = [L.TensorView.row_major(b, 0, [4096, 4096]) for b in pool_warm]
        t_end = time.perf_counter() + args.prewarm
        while time.perf_counter() < t_end:
            for _ in range(20):
                C.encode_gemm(ctx, ctx.queue, 1.0, vs[0], vs[1], 0.0, vs[2])
            ctx.sync()
        for b in pool_warm:
            b.free()

    def run(name, fn):
        if wanted is None or name in wanted:
            print(f"[bench] {name} ...", file=sys.stderr, flush=True)
            results[name] = fn()
            pool.free()
            r = results[name]
            e = summary_entry(r) if isinstance(r, dict) else None
            if e is not None:
                print(f"[bench] {name}: {e[0]} {e[1]} (frac {e[2]})", file=sys.stderr, flush=True)

    run("gemm4096", lambda: bench_gemm(ctx, events, pool, L, C, "gemm 4096^3", 4096, 4096, 4096, args))
    # The reference's spec benchmark squares (tests/contraction_test.rs:1246-1291).
    run("sq1024", lambda: bench_gemm(ctx, events, pool, L, C, "square gemm 1024^3", 1024, 1024, 1024,
                                     args, seed=(1024, 1025)))
    run("sq2048", lambda: bench_gemm(ctx, events, pool, L, C, "square gemm 2048^3", 2048, 2048, 2048,
                                     args, seed=(2048, 2049)))
    run("c1", lambda: bench_gemm(ctx, events, pool, L, C, "C1 gemm 512^3", 512, 512, 512, args, seed=(1, 2)))
    run("c3", lambda: bench_gemm(ctx, events, pool, L, C, "C3 bik,bkj->bij B=32 1024^3, B permuted",
                                 1024, 1024, 1024, args, b_t=True, batch=32, seed=(5, 6)))
    run("c4", lambda: bench_gemm(ctx, events, pool, L, C, "C4 split-K 256x256x65536", 256, 256, 65536,
                                 args, seed=(7, 8), sigma=1.0 / 256))

    def c5():
        M, K, N = 4096, 4096, 16384
        y = bench_gemm(ctx, events, pool, L, C, "C5 Y=X.W", M, N, K, args, seed=(9, 10), sigma=0.02)
        pool.free()
        dx = bench_gemm(ctx, events, pool, L, C, "C5 dX=dY.W^T", M, K, N, args, b_t=True,
                        seed=(11, 10), sigma=0.02)
        pool.free()
        dw = bench_gemm(ctx, events, pool, L, C, "C5 dW=X^T.dY", K, N, M, args, a_t=True,
                        seed=(9, 11), sigma=0.02, beta=1.0)
        ms = y["ms"] + dx["ms"] + dw["ms"]
        tf = 3 * 2.0 * M * N * K / (ms * 1e-3) / 1e12
        return {"name": "C5 linear-layer step (3 gemms)", "ms": ms, "tflops": tf,
                "frac": tf / PEAK_TFLOPS, "parts": [y, dx, dw]}
    run("c5", c5)
    run("c2a", lambda: bench_perm(ctx, events, pool, L, P, "C2a [64,128,64,32] perm (0,2,3,1)",
                                  [64, 128, 64, 32], [0, 2, 3, 1], 3, args))
    run("c2b", lambda: bench_perm(ctx, events, pool, L, P, "C2b [512,1024,256] perm (2,0,1)",
                                  [512, 1024, 256], [2, 0, 1], 4, args))
    # The other reading of the "1 GiB" permutation target: a 1 GiB tensor (2 GiB moved).
    run("c2b_1g", lambda: bench_perm(ctx, events, pool, L, P, "[1024,1024,256] perm (2,0,1), 1 GiB tensor",
                                     [1024, 1024, 256], [2, 0, 1], 5, args))
    run("copy", lambda: {"name": "plain 128-bit copy 512 MiB", "gbs": bench_copy(ctx, events, pool,
                                                                                 L, P, 1 << 27, args)})
    def t8191():
        # The reference's transpose benchmark (tests/permutation_test.rs:741-792): an
        # 8191x4099 f32 transpose against a plain copy of the same bytes; it asserts >= 70 %.
        r = bench_perm(ctx, events, pool, L, P, "transpose [8191,4099] perm (1,0)", [8191, 4099],
                       [1, 0], 3000, args)
        r.pop("_host")
        r.pop("_geom")
        r["copy_gbs"] = bench_copy(ctx, events, pool, L, P, 8191 * 4099, args)
        r["ratio_vs_copy"] = r["gbs"] / r["copy_gbs"]
        r["reference_gate"] = {"min_ratio_vs_copy": 0.70, "passed": r["ratio_vs_copy"] >= 0.70,
                               "source": "tests/permutation_test.rs:741-792"}
        return r
    run("t8191", t8191)

    def floor():
        # The launch floor of the small-product paths: C[32,32] = 0 (K = 0, one fill kernel)
        # through the same entry point, back to back and one at a time between events.
        a, b, c = pool.alloc("f32", 1), pool.alloc("f32", 1), pool.alloc("f32", 32 * 32)
        av = L.TensorView(a, 0, [32, 0], [1, 1])
        bv = L.TensorView(b, 0, [0, 32], [32, 1])
        cv = L.TensorView.row_major(c, 0, [32, 32])
        kernels = kernels_of(ctx, lambda: C.encode_gemm(ctx, ctx.queue, 1.0, av, bv, 0.0, cv))
        launch = abi_call(native_lib().lg_encode_gemm_f32, ctx.handle, ctx.queue.handle,
                          ctypes.c_float(1.0), av.to_c(), bv.to_c(), ctypes.c_float(0.0), cv.to_c())
        ms = timed(ctx, events, launch, args.steps, args.warmup)
        med, best = per_launch(ctx, events, launch, args.steps)
        return {"name": "launch floor: C[32,32] = 0 (K = 0)", "ms": ms, "ms_median": med,
                "ms_best": best, "host_ms": HOST_MS[launch],
                "ms_graph": graph_rate(ctx, events, launch, args.steps), "kernels": kernels}
    run("floor", floor)
    run("train", lambda: bench_train_ops(events, args, timed))
    run("bgemm16", lambda: bench_backend_gemm16(events, args, timed))
    run("f16", lambda: bench_gemm_f16(ctx, events, pool, L, C, 4096, 4096, 4096, args))
    # The reference's own benchmark list (tests/contraction_test.rs:1293-1395).
    for key, name, a_spec, b_spec, c_spec in other_paths_specs():
        run(key, lambda: bench_contract(ctx, events, pool, L, C, name, a_spec, b_spec, c_spec, args))
    run("o_f16_2048", lambda: bench_gemm_f16(ctx, events, pool, L, C, 2048, 2048, 2048, args))

    if args.vendor:
        print("[bench] vendor ...", file=sys.stderr, flush=True)
        attach_vendor(results, args)
    train = results.pop("train", None)
    bgemm16 = results.pop("bgemm16", None)
    if not args.no_cpu:
        print("[bench] cpu baselines ...", file=sys.stderr, flush=True)
        attach_cpu_baselines(results, min(os.cpu_count() or 1, 16))
    for r in results.values():
        for p in ([r] + list(r.get("parts", []))) if isinstance(r, dict) else []:
            p.pop("_host", None)
            p.pop("_geom", None)
            p.pop("_other", None)

    detail = detail_record(results, args, train, bgemm16)
    line = headline_line(results, args, train, bgemm16, args.detail)
    if args.detail:
        path = Path(args.detail)
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(json.dumps(detail, indent=1) + "\n")
    print(json.dumps(line), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
