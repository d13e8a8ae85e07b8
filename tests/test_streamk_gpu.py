"""Stream-K GEMM (gemm_f32_sk) parity on the GPU.

Products of full 128x128 tiles that a plain grid would spread unevenly over the 256 compute
units (the busiest one holding more than 10/9 of the mean) run as 256 equal runs of pipeline
steps; a tile two runs share is summed by whichever run finishes second, from the two sums
the runs leave in the context's scratch, and a ticket counter per run boundary that each
launch leaves at zero. Checked here, through the C ABI:
  * every output element against the crates/cpu restatement (oracle.gemm_fast, bit-identical
    to the literal loop) with the north-star bound max|err| <= 1e-5 sqrt(K) max|a| max|b|,
    on the rank-4 48^6 product of tests/contraction_test.rs:1293-1395 and on transposed,
    batched, column-major-C and scaled (alpha, beta) variants;
  * run-to-run determinism: repeated launches (which also re-use the ticket counters the
    previous launch cleared) give the same bits;
  * a shape whose runs hold whole tiles only (K of one step) and the plan's geometry.
"""
from __future__ import annotations

import numpy as np
import pytest

import linalg_hip as L
import oracle
from helpers import rng
from linalg_hip import contraction as C

pytestmark = pytest.mark.gpu


def _dense(shape):
    st, p = [], 1
    for e in reversed(shape):
        st.append(p)
        p *= e
    return list(shape), st[::-1]


def _upload(pool, x):
    buf = pool.alloc("f32", x.size)
    buf.write(x)
    return buf


def _run(ctx, pool, m, n, k, seed, a_t=False, b_t=False, c_t=False, batch=1, alpha=1.0,
         beta=0.0, repeats=3):
    """One product through lg_gemm_f32 `repeats` times; returns (host A, B, C0, C result)."""
    g = rng(seed)
    a = g.uniform(-1, 1, batch * m * k).astype(np.float32)
    b = g.uniform(-1, 1, batch * k * n).astype(np.float32)
    c0 = g.uniform(-1, 1, batch * m * n).astype(np.float32)
    A, B = _upload(pool, a), _upload(pool, b)
    Cb = _upload(pool, c0 if beta != 0.0 else np.full(batch * m * n, np.nan, np.float32))
    bs = [batch] if batch > 1 else []

    def view(buf, rows, cols, trans, plane):
        st = [1, rows] if trans else [cols, 1]
        return L.TensorView(buf, 0, bs + [rows, cols], ([plane] if bs else []) + st)
    av = view(A, m, k, a_t, m * k)
    bv = view(B, k, n, b_t, k * n)
    cv = view(Cb, m, n, c_t, m * n)
    plan = C.plan_gemm(alpha, av, bv, beta, cv)
    assert plan["kernel"] == "streamk" and plan["workgroups"] == 256, plan
    assert plan["scratch_bytes"] == 2 * 256 * 128 * 128 * 4, plan
    outs = []
    for _ in range(repeats):
        if beta != 0.0:
            Cb.write(c0)
        C.gemm(ctx, alpha, av, bv, beta, cv)
        outs.append(Cb.read(np.float32, count=batch * m * n).copy())
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), "not deterministic"
    return a, b, c0, outs[0]


def _check(a, b, c0, got, m, n, k, a_t=False, b_t=False, c_t=False, batch=1, alpha=1.0,
           beta=0.0):
    """Every element against crates/cpu (the threaded, bit-identical restatement)."""
    tol = 1e-5 * np.sqrt(k) * abs(alpha) * float(np.abs(a).max()) * float(np.abs(b).max())
    if beta != 0.0:
        tol += 1e-5 * abs(beta) * float(np.abs(c0).max())
    for bi in range(batch):
        ref = c0[bi * m * n:(bi + 1) * m * n].copy()
        oracle.gemm_fast(m, n, k, alpha, beta, a, bi * m * k, (1, m) if a_t else (k, 1), b,
                         bi * k * n, (1, k) if b_t else (n, 1), ref, 0, (1, m) if c_t else (n, 1))
        out = got[bi * m * n:(bi + 1) * m * n]
        err = np.abs(out.astype(np.float64) - ref.astype(np.float64))
        worst = int(np.argmax(err))
        assert np.all(np.isfinite(out)) and err[worst] <= tol, (
            f"batch {bi}: max|err| {err[worst]:e} > {tol:e} at element {worst}")


def test_rank4_48_pow6_through_contract(ctx, pool):
    """The reference's rank-4 benchmark, ijkl,klmn->ijmn at 48^6: axes merge to 2304^3, 324
    tiles over 256 runs (every run shares a tile with each neighbour)."""
    g = rng(4848)
    shape = [48] * 4
    x = g.uniform(-1, 1, 48 ** 4).astype(np.float32)
    y = g.uniform(-1, 1, 48 ** 4).astype(np.float32)
    X, Y = _upload(pool, x), _upload(pool, y)
    Z = _upload(pool, np.full(48 ** 4, np.nan, np.float32))
    sh, st = _dense(shape)
    xv, yv, zv = (L.TensorView(buf, 0, sh, st) for buf in (X, Y, Z))
    plan = C.plan_contract(1.0, (xv, "ijkl"), (yv, "klmn"), 0.0, (zv, "ijmn"))
    assert (plan["kernel"], plan["m"], plan["n"], plan["k"]) == ("streamk", 2304, 2304, 2304), plan
    outs = []
    for _ in range(3):
        C.contract(ctx, 1.0, (xv, "ijkl"), (yv, "klmn"), 0.0, (zv, "ijmn"))
        outs.append(Z.read(np.float32, count=48 ** 4).copy())
    assert all(np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)) for o in outs[1:])
    _check(x, y, np.zeros(48 ** 4, np.float32), outs[0], 2304, 2304, 2304)


@pytest.mark.parametrize("m,n,k,a_t,b_t,c_t,batch,alpha,beta", [
    (2304, 2304, 2304, False, False, False, 1, 1.0, 0.0),     # row-major, 324 tiles
    (2560, 2560, 1024, True, False, False, 1, -1.5, 0.5),     # A column-major, scaled, beta
    (2304, 2560, 768, False, True, False, 1, 1.0, 1.0),      # B transposed view, beta = 1
    (2304, 2304, 1152, False, False, True, 1, 0.75, 0.0),    # C column-major: C^T = B^T.A^T
    (1280, 1280, 512, False, False, False, 3, 1.0, -0.25),   # batched, 300 tiles across planes
    (3072, 3072, 640, True, True, False, 1, 2.0, 0.0),       # 576 tiles, both operands transposed
])
def test_streamk_matches_crates_cpu(ctx, pool, m, n, k, a_t, b_t, c_t, batch, alpha, beta):
    a, b, c0, got = _run(ctx, pool, m, n, k, 9000 + m + k, a_t, b_t, c_t, batch, alpha, beta)
    _check(a, b, c0, got, m, n, k, a_t, b_t, c_t, batch, alpha, beta)


def test_streamk_with_whole_tile_runs(ctx, pool):
    """K of one pipeline step: runs hold whole tiles only, nothing is shared."""
    a, b, c0, got = _run(ctx, pool, 2304, 2304, 128, 9100)
    _check(a, b, c0, got, 2304, 2304, 128)


def test_streamk_and_split_k_calls_interleaved(ctx, pool):
    """Stream-K and split-K products alternate on one stream (both use the context's scratch):
    every result stays equal to its own first run."""
    m = n = 2304
    g = rng(9200)
    x = g.uniform(-1, 1, m * m).astype(np.float32)
    X = _upload(pool, x)
    Y1 = _upload(pool, np.zeros(m * n, np.float32))
    xs = g.uniform(-1, 1, 256 * 65536).astype(np.float32)
    Xs, Ys = _upload(pool, xs), _upload(pool, xs[::-1].copy())
    Z = _upload(pool, np.zeros(256 * 256, np.float32))
    big = L.TensorView.row_major(X, 0, [m, m])
    out = L.TensorView.row_major(Y1, 0, [m, n])
    sa = L.TensorView.row_major(Xs, 0, [256, 65536])
    sb = L.TensorView.row_major(Ys, 0, [65536, 256])
    sc = L.TensorView.row_major(Z, 0, [256, 256])
    assert C.plan_gemm(1.0, big, big, 0.0, out)["kernel"] == "streamk"
    assert C.plan_gemm(1.0, sa, sb, 0.0, sc)["kind"] == "split"
    first = None
    for i in range(3):
        C.encode_gemm(ctx, ctx.queue, 1.0, big, big, 0.0, out)
        C.encode_gemm(ctx, ctx.queue, 1.0, sa, sb, 0.0, sc)
        ctx.sync()
        now = (Y1.read(np.uint32, count=m * n).copy(), Z.read(np.uint32, count=256 * 256).copy())
        if first is None:
            first = now
        else:
            assert np.array_equal(now[0], first[0]) and np.array_equal(now[1], first[1]), i
