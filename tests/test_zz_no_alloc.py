"""lg_encode_gemm_f32_noalloc against lg_encode_gemm_f32, through the C ABI.

The entry point allocates nothing: split-K, split-dot and stream-K partials (and stream-K's
ticket counters) live in a static device
array. Its results must be the existing entry point's (the same plans, so bit for bit) and
pass the north-star bound against the crates/cpu restatement, over calls in a row whose later
inputs are smaller (the array keeps the last call's contents, so stale partials would
show), on the context stream and on a caller's stream. An invalid call returns its
status and launches nothing.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import linalg_hip as L
import oracle
from helpers import rng
from linalg_hip import _native as N

pytestmark = pytest.mark.gpu

SHAPES = [
    (384, 384, 65536),  # split-K on 128x128 tiles, 56 splits: 31.5 MiB of partials
    (256, 256, 65536),  # split-K on 64x64 K-split-wave tiles, 16 splits
    (64, 48, 30000),    # one 64x64 register-staged tile, split 209 ways along K
    (1, 1, 1 << 20),    # split dot
    (1, 1, 100003),     # a smaller split dot
    (300, 200, 100),    # one tiled launch, no scratch
    (256, 128, 9000),   # split-K again on 64x64 tiles, fewer and smaller partials
    (2304, 2304, 1152), # stream-K: 324 tiles over 256 runs, tile sums and tickets in the array
]


def _views(pool, m, n, k, seed):
    # N(0, 1/sqrt(K)) as in config 4: the k-order f32 sums of crates/cpu then stay far inside
    # the north-star bound even at K = 2^20.
    g = rng(seed)
    x = (g.standard_normal(m * k) / np.sqrt(k)).astype(np.float32)
    y = (g.standard_normal(k * n) / np.sqrt(k)).astype(np.float32)
    a, b = pool.alloc("f32", m * k), pool.alloc("f32", k * n)
    a.write(x)
    b.write(y)
    return x, y, L.TensorView.row_major(a, 0, [m, k]), L.TensorView.row_major(b, 0, [k, n])


def _out(pool, m, n, fill):
    c = pool.alloc("f32", m * n)
    c.write(fill)
    return c, L.TensorView.row_major(c, 0, [m, n])


@pytest.mark.parametrize("on_user_stream", [False, True])
def test_noalloc_matches_the_allocating_entry_point(ctx, pool, on_user_stream):
    lib = N.lib()
    q = ctx.new_stream() if on_user_stream else None
    stream = q.handle if q else None
    try:
        for i, (m, n, k) in enumerate(SHAPES):
            x, y, av, bv = _views(pool, m, n, k, 500 + i)
            beta = 0.0 if i % 2 == 0 else -0.5
            c0 = rng(600 + i).uniform(-1, 1, m * n).astype(np.float32)
            fill = np.full(m * n, np.nan, np.float32) if beta == 0.0 else c0
            c_ref, cv_ref = _out(pool, m, n, fill)
            c_na, cv_na = _out(pool, m, n, fill)
            args = (ctypes.c_float(1.0), ctypes.byref(av.to_c()), ctypes.byref(bv.to_c()),
                    ctypes.c_float(beta))
            assert lib.lg_encode_gemm_f32(ctx.handle, stream, *args, ctypes.byref(cv_ref.to_c())) == 0
            assert lib.lg_encode_gemm_f32_noalloc(ctx.handle, stream, *args,
                                                  ctypes.byref(cv_na.to_c())) == 0
            if q:
                q.wait_until_completed()
            got = c_na.read(np.float32, count=m * n)
            want = c_ref.read(np.float32, count=m * n)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, n, k)
            tol = 1e-5 * np.sqrt(k) * float(np.abs(x).max()) * float(np.abs(y).max())
            if beta == 0.0:
                # The crates/cpu restatement (k-order f32 sums).
                ref = np.zeros(m * n, np.float32)
                oracle.gemm_fast(m, n, k, 1.0, 0.0, x, 0, (k, 1), y, 0, (n, 1), ref, 0, (n, 1))
            else:
                # crates/cpu starts from beta*C (~0.5 here) and adds K products of ~1/K, each
                # rounded at that magnitude: its own error (~8e-6 at K = 30000) exceeds the
                # bound, so the comparand is the exact value, plus C's one rounding.
                ref = beta * c0.astype(np.float64) + (
                    x.reshape(m, k).astype(np.float64) @ y.reshape(k, n).astype(np.float64)).ravel()
                tol += 2.0 ** -24 * abs(beta) * float(np.abs(c0).max())
            err = float(np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64))))
            assert np.all(np.isfinite(got)) and err <= tol, (m, n, k, err, tol)
    finally:
        if q:
            q.close()


def test_noalloc_rejects_an_invalid_call_and_launches_nothing(ctx, pool):
    lib = N.lib()
    x, y, av, bv = _views(pool, 64, 64, 64, 700)
    count = lambda: N.lib().lg_debug_launch_count(ctx.handle)
    before = count()
    # C overlapping A: LG_OVERLAP, nothing written.
    st = lib.lg_encode_gemm_f32_noalloc(ctx.handle, None, ctypes.c_float(1.0),
                                        ctypes.byref(av.to_c()), ctypes.byref(bv.to_c()),
                                        ctypes.c_float(0.0), ctypes.byref(av.to_c()))
    assert st == N.LG_OVERLAP
    ctx.sync()
    a_now = av.buffer.read(np.float32, count=64 * 64)
    assert np.array_equal(a_now.view(np.uint32), x.view(np.uint32))
    assert count() == before
    # Shape mismatch: LG_INVALID_ARGUMENT.
    c, cv = _out(pool, 63, 64, np.zeros(63 * 64, np.float32))
    st = lib.lg_encode_gemm_f32_noalloc(ctx.handle, None, ctypes.c_float(1.0),
                                        ctypes.byref(av.to_c()), ctypes.byref(bv.to_c()),
                                        ctypes.c_float(0.0), ctypes.byref(cv.to_c()))
    assert st == N.LG_INVALID_ARGUMENT
    assert count() == before


def test_noalloc_split_calls_capture_and_replay_like_eager_calls(ctx, pool):
    """A split-K, a split-dot and a stream-K noalloc call recorded under stream capture: the
    static array's address was looked up when the context was made, so capture records kernels
    only (the stream-K tickets are left at zero by every launch). Three
    replays on new inputs, each bit for bit equal to the eager noalloc call on the same
    inputs, with eager work and synchronizations between the replays."""
    import test_graph_gpu as G
    hip = G.Hip()
    lib = N.lib()
    q = ctx.new_stream()
    g = rng(7300)
    shapes = [(256, 256, 65536), (1, 1, 1 << 20), (2304, 2304, 1152)]
    calls = []
    for m, n, k in shapes:
        a, b, c = pool.alloc("f32", m * k), pool.alloc("f32", k * n), pool.alloc("f32", m * n)
        av = L.TensorView.row_major(a, 0, [m, k])
        bv = L.TensorView.row_major(b, 0, [k, n])
        cv = L.TensorView.row_major(c, 0, [m, n])
        from linalg_hip import contraction as C
        plan = C.plan_gemm(1.0, av, bv, 0.0, cv)
        assert plan["scratch_bytes"] > 0, plan  # split-K, split dot, stream-K
        calls.append((m, n, k, a, b, c, (ctypes.c_float(1.0), ctypes.byref(av.to_c()),
                                        ctypes.byref(bv.to_c()), ctypes.c_float(0.0),
                                        ctypes.byref(cv.to_c()))))

    def step(stream):
        for *_, args in calls:
            assert lib.lg_encode_gemm_f32_noalloc(ctx.handle, stream, *args) == 0

    graph, exe = hip.capture(q.handle, lambda: step(q.handle))
    try:
        for replay in range(3):
            for m, n, k, a, b, c, _ in calls:
                a.write((g.standard_normal(m * k) / np.sqrt(k)).astype(np.float32))
                b.write((g.standard_normal(k * n) / np.sqrt(k)).astype(np.float32))
                c.write(np.full(m * n, np.nan, np.float32))
            assert hip.h.hipGraphLaunch(exe, q.handle) == 0
            q.wait_until_completed()
            got = [c.read(np.uint32, count=m * n).copy() for m, n, k, a, b, c, _ in calls]
            for m, n, k, a, b, c, _ in calls:
                c.write(np.full(m * n, np.nan, np.float32))
            step(None)
            ctx.sync()
            for (m, n, k, a, b, c, _), x in zip(calls, got):
                assert np.array_equal(x, c.read(np.uint32, count=m * n)), (replay, m, n, k)
                assert np.all(np.isfinite(x.view(np.float32))), (replay, m, n, k)
    finally:
        hip.h.hipGraphExecDestroy(exe)
        hip.h.hipGraphDestroy(graph)
        q.close()
