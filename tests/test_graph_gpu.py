"""The enqueue entry points under HIP graph capture.

A caller that replays a fixed step (a pipeline stage's forward products and the transposes
around them) can capture the library's encode calls on its own stream into a hipGraph and
launch that graph instead. Every GEMM path and the permutation paths enqueue kernels only (no
allocation, no memset, no synchronization): the split-K, split-small and split-dot paths use
the context's scratch, made with the context, so they capture too. Each replay is checked against the eager
result of the same step on inputs changed between replays, with eager work and
synchronizations in between, as the graph must see the buffers' current contents.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import linalg_hip as L
from helpers import rng
from linalg_hip import contraction as C
from linalg_hip import permutation as P

pytestmark = pytest.mark.gpu

CAPTURE_THREAD_LOCAL = 1  # hipStreamCaptureModeThreadLocal


class Hip:
    def __init__(self):
        h = ctypes.CDLL("libamdhip64.so")
        vp, pvp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
        h.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
        h.hipStreamEndCapture.argtypes = [vp, pvp]
        h.hipGraphInstantiate.argtypes = [pvp, vp, vp, ctypes.c_char_p, ctypes.c_size_t]
        h.hipGraphLaunch.argtypes = [vp, vp]
        h.hipGraphExecDestroy.argtypes = [vp]
        h.hipGraphDestroy.argtypes = [vp]
        self.h = h

    def capture(self, stream, enqueue):
        assert self.h.hipStreamBeginCapture(stream, CAPTURE_THREAD_LOCAL) == 0
        try:
            enqueue()
        finally:
            graph = ctypes.c_void_p()
            end = self.h.hipStreamEndCapture(stream, ctypes.byref(graph))
        assert end == 0
        exe = ctypes.c_void_p()
        assert self.h.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        return graph, exe


def test_captured_gemm_and_transpose_replay_like_eager_work(ctx, pool):
    hip = Hip()
    q = ctx.new_stream()
    g = rng(7100)
    # (m, n, k): the single-launch small kernel and the 128x128 kernel without split-K.
    shapes = [(256, 192, 320), (2048, 2048, 256)]
    views = []
    for m, n, k in shapes:
        a = pool.alloc("f32", m * k)
        b = pool.alloc("f32", k * n)
        c = pool.alloc("f32", m * n)
        d = pool.alloc("f32", m * n)
        av = L.TensorView.row_major(a, 0, [m, k])
        bv = L.TensorView.row_major(b, 0, [k, n])
        cv = L.TensorView.row_major(c, 0, [m, n])
        dv = L.TensorView.row_major(d, 0, [n, m])
        plan = C.plan_gemm(1.0, av, bv, 0.0, cv)
        assert plan["kind"] == "tiled", plan
        views.append((m, n, k, a, b, c, d, av, bv, cv, dv))

    def step(stream):
        for m, n, k, a, b, c, d, av, bv, cv, dv in views:
            C.encode_gemm(ctx, stream, 1.0, av, bv, 0.0, cv)
            P.encode_materialize(ctx, stream, P.permute_view(cv, [1, 0]), dv)

    graph, exe = hip.capture(q.handle, lambda: step(q))
    try:
        for replay in range(3):
            inputs = []
            for m, n, k, a, b, c, d, *_ in views:
                x = g.uniform(-1, 1, m * k).astype(np.float32)
                y = g.uniform(-1, 1, k * n).astype(np.float32)
                a.write(x)
                b.write(y)
                d.write(np.full(m * n, np.nan, np.float32))
                inputs.append((x, y))
            assert hip.h.hipGraphLaunch(exe, q.handle) == 0
            q.wait_until_completed()
            graph_out = [d.read(np.uint32, count=m * n).copy()
                         for m, n, k, a, b, c, d, *_ in views]
            # The same step eagerly on the same inputs gives the same bits.
            for (m, n, k, a, b, c, d, *_), _ in zip(views, inputs):
                d.write(np.full(m * n, np.nan, np.float32))
            step(ctx.queue)
            ctx.sync()
            for (m, n, k, a, b, c, d, *_), (x, y), got in zip(views, inputs, graph_out):
                eager = d.read(np.uint32, count=m * n)
                assert np.array_equal(got, eager), (replay, m, n, k)
                ref = (x.reshape(m, k).astype(np.float64) @ y.reshape(k, n).astype(np.float64)).T
                val = got.view(np.float32).reshape(n, m)
                assert np.max(np.abs(val - ref)) <= 1e-5 * np.sqrt(k), (replay, m, n, k)
    finally:
        hip.h.hipGraphExecDestroy(exe)
        hip.h.hipGraphDestroy(graph)
        q.close()


def test_captured_split_products_replay_like_eager_work(ctx, pool):
    """Split-K (128x128 tiles), split 32x32 tiles and a split dot under capture: the partials live
    in the context's scratch, so capture needs no allocation; three replays on new
    inputs, eager runs of the same products between them, all bit for bit equal."""
    hip = Hip()
    q = ctx.new_stream()
    g = rng(7200)
    shapes = [(256, 256, 16384), (32, 40, 100000), (1, 1, 1 << 20)]
    views = []
    for m, n, k in shapes:
        a, b, c = pool.alloc("f32", m * k), pool.alloc("f32", k * n), pool.alloc("f32", m * n)
        av = L.TensorView.row_major(a, 0, [m, k])
        bv = L.TensorView.row_major(b, 0, [k, n])
        cv = L.TensorView.row_major(c, 0, [m, n])
        plan = C.plan_gemm(1.0, av, bv, 0.0, cv)
        assert plan["kind"] in ("split", "dot") and plan["splits"] > 1, plan
        views.append((m, n, k, a, b, c, av, bv, cv))

    def step(stream):
        for m, n, k, a, b, c, av, bv, cv in views:
            C.encode_gemm(ctx, stream, 1.0, av, bv, 0.0, cv)

    graph, exe = hip.capture(q.handle, lambda: step(q))
    try:
        for replay in range(3):
            inputs = []
            for m, n, k, a, b, c, *_ in views:
                x = g.uniform(-1, 1, m * k).astype(np.float32)
                y = g.uniform(-1, 1, k * n).astype(np.float32)
                a.write(x)
                b.write(y)
                c.write(np.full(m * n, np.nan, np.float32))
                inputs.append((x, y))
            assert hip.h.hipGraphLaunch(exe, q.handle) == 0
            q.wait_until_completed()
            graph_out = [c.read(np.uint32, count=m * n).copy() for m, n, k, a, b, c, *_ in views]
            for m, n, k, a, b, c, *_ in views:
                c.write(np.full(m * n, np.nan, np.float32))
            step(ctx.queue)
            ctx.sync()
            for (m, n, k, a, b, c, *_), (x, y), got in zip(views, inputs, graph_out):
                assert np.array_equal(got, c.read(np.uint32, count=m * n)), (replay, m, n, k)
                ref = x.reshape(m, k).astype(np.float64) @ y.reshape(k, n).astype(np.float64)
                val = got.view(np.float32).reshape(m, n)
                assert np.max(np.abs(val - ref)) <= 1e-5 * np.sqrt(k), (replay, m, n, k)
    finally:
        hip.h.hipGraphExecDestroy(exe)
        hip.h.hipGraphDestroy(graph)
        q.close()
