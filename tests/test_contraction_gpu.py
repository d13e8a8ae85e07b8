"""Contraction parity on the GPU.

Every result is gated componentwise against the f64 reference of
tests/contraction_test.rs:200-268 with its tolerance
  |C_gpu - C_ref| <= (K+2)u(|alpha| sum|a||b| + |beta||C0|) + u|C_ref| + tiny,  u = 2^-24,
and, for 2-D gemm cases, against the crates/cpu restatement with the north-star bound
  max|err| <= 1e-5 * sqrt(K) * max|a| * max|b|.
Every buffer element outside C's view must keep its bits; with beta = 0, C starts as NaN.
The case list restates tests/contraction_test.rs (the 20 typed cases for f32 and the 96-case
random sweep); the benchmark configurations run at full size with every output element checked
against the oracle (config 5's two gradient products: one whole row in every 128-row tile band)
and size-independent properties (determinism, linearity) on the whole output.
"""
from __future__ import annotations

import numpy as np
import pytest

import linalg_hip as L
import oracle
from helpers import Case, Layout, Tensor, assert_untouched, rng
from linalg_hip import contraction as C
from linalg_hip import permutation as P

pytestmark = pytest.mark.gpu


def test_square(ctx, pool):
    for seed, n in enumerate([1, 8, 64, 96, 100, 256, 384]):
        Case.matmul(n, n, n).run(ctx, pool, seed)
    Case.matmul(192, 192, 192).scalars(-1.25, 0.75).run(ctx, pool, 7)


def test_unit_extents(ctx, pool):
    shapes = [(1, 37, 29), (41, 1, 29), (41, 37, 1), (1, 1, 1), (1, 1, 500), (1, 300, 1),
              (300, 1, 1), (1, 64, 64), (64, 1, 64), (64, 64, 1)]
    for seed, (m, n, k) in enumerate(shapes):
        Case.matmul(m, n, k).run(ctx, pool, 100 + seed)
        Case.matmul(m, n, k).scalars(1.5, -0.5).run(ctx, pool, 200 + seed)


def test_zero_k(ctx, pool):
    for seed, beta in enumerate([0.0, 1.0, -0.5]):
        Case.matmul(17, 9, 0).scalars(1.0, beta).run(ctx, pool, 300 + seed)
        batched = Case("batched K=0", (Layout.dense([3, 5, 0, 2]), "bmkl"),
                       (Layout.dense([3, 0, 2, 4]), "bkln"), (Layout.dense([3, 5, 4]), "bmn"))
        batched.scalars(2.0, beta).run(ctx, pool, 310 + seed)


def test_empty_output(ctx, pool):
    for seed, (m, n, k) in enumerate([(0, 5, 3), (5, 0, 3), (0, 0, 0), (0, 4, 0)]):
        Case.matmul(m, n, k).scalars(1.0, -0.5).run(ctx, pool, 400 + seed)
    Case("empty batch", (Layout.dense([0, 4, 3]), "bmk"), (Layout.dense([0, 3, 5]), "bkn"),
         (Layout.dense([0, 4, 5]), "bmn")).run(ctx, pool, 410)


def test_prime_sizes(ctx, pool):
    Case.matmul(127, 251, 63).run(ctx, pool, 500)
    Case.matmul(127, 251, 63).scalars(-0.75, 1.0).run(ctx, pool, 501)
    Case.matmul(251, 127, 67).scalars(0.5, -0.5).run(ctx, pool, 502)
    Case.matmul(257, 131, 129).scalars(1.0, 0.0).run(ctx, pool, 503)


def test_transposed_views(ctx, pool):
    for (m, n, k) in [(45, 70, 33), (48, 72, 32), (130, 260, 96)]:
        pick = lambda t, r, c: Layout.transposed(r, c) if t else Layout.dense([r, c])
        for mask in range(8):
            ta, tb, tc = bool(mask & 1), bool(mask & 2), bool(mask & 4)
            case = Case(f"transposed a={ta} b={tb} c={tc} {m}x{n}x{k}", (pick(ta, m, k), "mk"),
                        (pick(tb, k, n), "kn"), (pick(tc, m, n), "mn"))
            case.scalars(1.0, 0.0 if mask % 2 == 0 else -0.5).run(ctx, pool, 600 + mask)
    via = Case.matmul(45, 70, 33)
    via.a = (Layout.transposed(45, 33), "mk")
    via.c = (Layout.transposed(45, 70), "mn")
    via.run(ctx, pool, 610)


def test_strided_views(ctx, pool):
    m, n, k = 37, 41, 19
    layouts = [
        (Layout.with_([m, k], [0, 1], [2, 3], 5), Layout.with_([k, n], [0, 1], [3, 1], 11),
         Layout.with_([m, n], [0, 1], [2, 2], 3)),
        (Layout.with_([m, k], [1, 0], [1, 2], 1), Layout.with_([k, n], [1, 0], [2, 2], 9),
         Layout.with_([m, n], [1, 0], [3, 1], 17)),
        (Layout.with_([m, k], [0, 1], [1, 1], 64), Layout.with_([k, n], [0, 1], [1, 1], 1),
         Layout.with_([m, n], [0, 1], [1, 1], 77)),
    ]
    for seed, (a, b, c) in enumerate(layouts):
        for alpha, beta in [(1.0, 0.0), (-2.0, 1.0), (0.5, -0.5)]:
            Case(f"strided #{seed}", (a, "mk"), (b, "kn"), (c, "mn")).scalars(alpha, beta).run(
                ctx, pool, 700 + seed)
    via = Case.matmul(70, 70, 70)
    via.a = (Layout.with_([70, 70], [0, 1], [1, 2], 3), "mk")
    via.b = (Layout.with_([70, 70], [1, 0], [2, 1], 6), "kn")
    via.c = (Layout.with_([70, 70], [0, 1], [3, 1], 9), "mn")
    via.scalars(1.0, -0.5).run(ctx, pool, 710)


def test_batched(ctx, pool):
    for seed, batch in enumerate([[3], [2, 3], [1, 1, 5], [70]]):
        m, n, k = 33, 20, 17
        labels = "xyz"[: len(batch)]
        case = Case(f"batched gemm {batch}", (Layout.dense(batch + [m, k]), labels + "mk"),
                    (Layout.dense(batch + [k, n]), labels + "kn"),
                    (Layout.dense(batch + [m, n]), labels + "mn"), via_gemm=True)
        case.scalars(1.0, 0.0 if seed % 2 == 0 else -0.5).run(ctx, pool, 800 + seed)
    Case("batch axis in the middle", (Layout.with_([19, 6, 23], [1, 0, 2], [1, 1, 1], 2), "mbk"),
         (Layout.with_([23, 31, 6], [0, 2, 1], [1, 1, 2], 0), "knb"),
         (Layout.with_([31, 6, 19], [1, 2, 0], [1, 1, 1], 4), "nbm")).scalars(0.5, -0.5).run(ctx, pool, 810)
    Case("many small matrices", (Layout.dense([500, 4, 3]), "bmk"), (Layout.dense([500, 3, 5]), "bkn"),
         (Layout.dense([500, 4, 5]), "bmn")).run(ctx, pool, 811)
    Case("one B for every A", (Layout.dense([7, 21, 40]), "bmk"), (Layout.dense([40, 13]), "kn"),
         (Layout.dense([7, 21, 13]), "bmn")).scalars(1.0, 1.0).run(ctx, pool, 812)


def test_rank4_two_axes(ctx, pool):
    i, j, k, l, m, n = 5, 7, 6, 9, 4, 11
    Case("ijkl,klmn->ijmn dense", (Layout.dense([i, j, k, l]), "ijkl"),
         (Layout.dense([k, l, m, n]), "klmn"), (Layout.dense([i, j, m, n]), "ijmn")).run(ctx, pool, 900)
    Case("ijkl,lkmn->imjn scrambled",
         (Layout.with_([i, j, k, l], [2, 0, 3, 1], [1, 1, 1, 1], 3), "ijkl"),
         (Layout.with_([l, k, m, n], [3, 0, 2, 1], [1, 2, 1, 1], 0), "lkmn"),
         (Layout.with_([i, m, j, n], [1, 3, 0, 2], [1, 1, 2, 1], 8), "imjn")).scalars(-1.5, -0.5).run(ctx, pool, 901)
    i, j, k, l, m, n = 9, 10, 12, 11, 8, 13
    Case("ijkl,mlkn->njim larger", (Layout.dense([i, j, k, l]), "ijkl"),
         (Layout.dense([m, l, k, n]), "mlkn"), (Layout.dense([n, j, i, m]), "njim")).scalars(1.0, 1.0).run(ctx, pool, 902)


def test_collapsible_axes(ctx, pool):
    Case("six collapsible M axes", (Layout.dense([2, 3, 2, 3, 2, 3, 5]), "abcdefk"),
         (Layout.dense([5, 7]), "kn"), (Layout.dense([2, 3, 2, 3, 2, 3, 7]), "abcdefn")).scalars(1.0, -0.5).run(ctx, pool, 1000)
    Case("unit axes everywhere",
         (Layout.with_([1, 6, 1, 1, 9, 1], [5, 3, 1, 0, 2, 4], [1, 2, 1, 3, 1, 1], 1), "pmqrks"),
         (Layout.with_([1, 9, 1, 1, 8, 1], [0, 4, 2, 1, 3, 5], [2, 1, 1, 1, 1, 4], 0), "skrtnq"),
         (Layout.with_([1, 1, 6, 8, 1, 1], [3, 2, 0, 1, 4, 5], [1, 1, 1, 1, 1, 1], 2), "tpmnsq")).run(ctx, pool, 1001)


def test_beta_variants(ctx, pool):
    seed = 1100
    for m, n, k in [(70, 50, 40), (33, 65, 1), (5, 6, 20000)]:
        for beta in [0.0, 1.0, -0.5]:
            for alpha in [1.0, -2.5]:
                Case.matmul(m, n, k).scalars(alpha, beta).run(ctx, pool, seed)
                seed += 1


def test_split_k(ctx, pool):
    shapes = [(1, 1, 1000003), (8, 8, 65536), (3, 5, 200001), (40, 24, 30000), (1, 70, 9973),
              (130, 200, 20000)]
    for seed, (m, n, k) in enumerate(shapes):
        Case.matmul(m, n, k).run(ctx, pool, 1200 + seed)
        Case.matmul(m, n, k).scalars(0.5, -0.5).run(ctx, pool, 1210 + seed)
    Case("batched long K", (Layout.with_([3, 2, 50000], [2, 0, 1], [1, 1, 1], 1), "bmk"),
         (Layout.dense([3, 50000, 4]), "bkn"), (Layout.dense([3, 2, 4]), "bmn")).scalars(-1.0, 1.0).run(ctx, pool, 1220)


def test_deterministic(ctx, pool):
    for seed, (m, n, k) in enumerate([(4, 4, 300000), (130, 70, 90), (9, 1, 1), (256, 256, 65536)]):
        g = rng(1300 + seed)
        a = Tensor.random(pool, Layout.dense([m, k]), g)
        b = Tensor.random(pool, Layout.dense([k, n]), g)
        runs = []
        for _ in range(3):
            c = Tensor(pool, Layout.dense([m, n]))
            C.gemm(ctx, 1.0, a.view(), b.view(), 0.0, c.view())
            runs.append(c.read().view(np.uint32).copy())
        assert np.array_equal(runs[0], runs[1]) and np.array_equal(runs[1], runs[2]), (m, n, k)


def test_non_finite_inputs(ctx, pool):
    for seed, (m, n, k) in enumerate([(70, 45, 50), (3, 2, 40000), (9, 11, 1), (200, 150, 300)]):
        g = rng(1400 + seed)
        a = Tensor.random(pool, Layout.dense([m, k]), g)
        b = Tensor.random(pool, Layout.dense([k, n]), g)
        c = Tensor(pool, Layout.dense([m, n]))
        nan_row, inf_col = m - 1, n - 2
        a.host[nan_row * k + (k - 1)] = np.nan
        b.host[(k // 2) * n + inf_col] = np.inf
        a.upload()
        b.upload()
        c0 = c.host.copy()
        e = oracle.contract_f64(1.0, a.host, a.layout.tup(), "mk", b.host, b.layout.tup(), "kn",
                                0.0, c0, c.layout.tup(), "mn")
        C.gemm(ctx, 1.0, a.view(), b.view(), 0.0, c.view())
        got = c.read()
        name = f"non-finite {m}x{n}x{k}"
        oracle.gate(got, e, name)
        out = got[: m * n].reshape(m, n)
        poisoned = np.zeros((m, n), bool)
        poisoned[nan_row, :] = True
        poisoned[:, inf_col] = True
        assert np.array_equal(np.isfinite(out), ~poisoned), name


def test_alpha_zero(ctx, pool):
    for seed, (m, n, k) in enumerate([(20, 30, 40), (2, 2, 50000), (7, 5, 1)]):
        for beta in [0.0, 1.0, -0.5]:
            g = rng(1500 + seed)
            a = Tensor(pool, Layout.dense([m, k]), np.full(m * k + 13, np.nan, np.float32))
            b = Tensor(pool, Layout.dense([k, n]), np.full(k * n + 13, np.nan, np.float32))
            c = Tensor.random(pool, Layout.dense([m, n]), g)
            c0 = c.host.copy()
            C.gemm(ctx, 0.0, a.view(), b.view(), beta, c.view())
            got = c.read()[: m * n]
            if beta == 0.0:
                # crates/cpu starts the accumulator at +0 and never reads C (lib.rs:680-681).
                assert np.all(got.view(np.uint32) == 0), (m, n, k, beta)
            else:
                want = (np.float32(beta) * c0[: m * n]).astype(np.float32)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, n, k, beta)


def test_lu_trailing_update(ctx, pool):
    for seed, (n, done, panel) in enumerate([(96, 0, 32), (131, 17, 40), (64, 5, 1)]):
        g = rng(1600 + seed)
        mat = Tensor.random(pool, Layout.dense([n, n]), g)
        split = done + panel
        rest = n - split
        l_ = Layout(split * n + done, [rest, panel], [n, 1])
        u_ = Layout(done * n + split, [panel, rest], [n, 1])
        c_ = Layout(split * n + split, [rest, rest], [n, 1])
        before = mat.host.copy()
        e = oracle.contract_f64(-1.0, before, l_.tup(), "mk", before, u_.tup(), "kn", 1.0, before,
                                c_.tup(), "mn")
        mk = lambda lay: L.TensorView(mat.buffer, lay.offset, lay.shape, lay.strides)
        C.gemm(ctx, -1.0, mk(l_), mk(u_), 1.0, mk(c_))
        got = mat.read()
        name = f"LU trailing update n={n} panel={panel}"
        assert_untouched(name, before, got, e.index)
        oracle.gate(got, e, name)


def test_in_place_scale(ctx, pool):
    n, col, top = 50, 7, 8
    g = rng(1700)
    mat = Tensor.random(pool, Layout.dense([n, n]), g)
    piv = Tensor.random(pool, Layout.dense([1, 1]), g)
    column = Layout(top * n + col, [n - top, 1], [n, 1])
    before = mat.host.copy()
    e = oracle.contract_f64(1.0, before, column.tup(), "mk", piv.host, piv.layout.tup(), "kn", 0.0,
                            before, column.tup(), "mn")
    v = L.TensorView(mat.buffer, column.offset, column.shape, column.strides)
    C.gemm(ctx, 1.0, v, piv.view(), 0.0, v)
    got = mat.read()
    assert_untouched("in-place column scale", before, got, e.index)
    oracle.gate(got, e, "in-place column scale")
    row = Layout(3 * n + 2, [1, n - 5], [n, 1])
    before = got.copy()
    mat.host[:] = before
    e = oracle.contract_f64(-0.5, piv.host, piv.layout.tup(), "mk", before, row.tup(), "kn", 1.0,
                            before, row.tup(), "mn")
    v = L.TensorView(mat.buffer, row.offset, row.shape, row.strides)
    C.gemm(ctx, -0.5, piv.view(), v, 1.0, v)
    got = mat.read()
    assert_untouched("in-place row scale", before, got, e.index)
    oracle.gate(got, e, "in-place row scale")


def test_repeated_calls_plan_again_on_any_change(ctx, pool):
    """The library keeps the plans of a thread's last few gemm calls, keyed on the views,
    alpha and beta. A repeat gives the same bits; the same shapes on other buffers, another
    beta, a shifted offset or an overlapping destination are planned again (the overlap still
    rejected, nothing launched), and the first call afterwards still holds."""
    m, n, k = 256, 192, 320
    g = rng(1750)
    A1, A2 = (Tensor.random(pool, Layout.dense([m, k]), g) for _ in range(2))
    B1, B2 = (Tensor.random(pool, Layout.dense([k, n]), g) for _ in range(2))
    C1, C2 = (Tensor.random(pool, Layout.dense([m, n]), g) for _ in range(2))
    c1_0, c2_0 = C1.host.copy(), C2.host.copy()

    def check(name, Cc, c0, A, B, alpha, beta, la=Layout.dense([m, k])):
        _gemm_fast_check(name, Cc.read(), A.host, la, B.host, Layout.dense([k, n]), c0,
                         Layout.dense([m, n]), m, n, k, alpha, beta)

    C.gemm(ctx, 1.0, A1.view(), B1.view(), 0.0, C1.view())
    first = C1.read().copy()
    check("first call", C1, c1_0, A1, B1, 1.0, 0.0)
    C.gemm(ctx, 1.0, A1.view(), B1.view(), 0.0, C1.view())
    assert np.array_equal(first.view(np.uint32), C1.read().view(np.uint32))
    # Same shapes, other buffers: C2 written, C1 untouched.
    C.gemm(ctx, 1.0, A2.view(), B2.view(), 0.0, C2.view())
    check("other buffers", C2, c2_0, A2, B2, 1.0, 0.0)
    assert np.array_equal(first.view(np.uint32), C1.read().view(np.uint32))
    # Same views, another beta (C2 now holds A2.B2).
    c2_1 = C2.read().copy()
    C.gemm(ctx, 1.0, A1.view(), B1.view(), 0.5, C2.view())
    check("beta 0.5", C2, c2_1, A1, B1, 1.0, 0.5)
    # A view shifted by one element (the last row of A2's buffer, its spare tail, unread before).
    shifted = L.TensorView(A2.buffer, 1, [m, k], [k, 1])
    c2_2 = C2.read().copy()
    C.gemm(ctx, -0.75, shifted, B1.view(), 0.0, C2.view())
    check("shifted A", C2, c2_2, A2, B1, -0.75, 0.0, la=Layout(1, [m, k], [k, 1]))
    # A destination overlapping A, shapes unchanged: rejected before any launch.
    n0 = ctx.launches()
    over = L.TensorView(A1.buffer, 0, [m, n], [n, 1])
    with pytest.raises(L.Overlap):
        C.gemm(ctx, 1.0, A1.view(), B1.view(), 0.0, over)
    assert ctx.launches() == n0
    assert np.array_equal(A1.read().view(np.uint32), A1.host.view(np.uint32))
    C.gemm(ctx, 1.0, A1.view(), B1.view(), 0.0, C1.view())
    assert np.array_equal(first.view(np.uint32), C1.read().view(np.uint32))


def test_overlap_rejected_without_launch(ctx, pool):
    n = 24
    g = rng(1800)
    mat = Tensor.random(pool, Layout.dense([2 * n, 2 * n]), g)
    other = Tensor.random(pool, Layout.dense([n, n]), g)
    block = lambda r, c_, rows, cols: L.TensorView(mat.buffer, r * 2 * n + c_, [rows, cols], [2 * n, 1])
    whole, shifted, apart = block(0, 0, n, n), block(n - 1, n - 1, n, n), block(n, n, n, n)
    n0 = ctx.launches()
    for A, B, Cv in [(whole, other.view(), whole), (other.view(), whole, whole),
                     (whole, other.view(), shifted), (other.view(), shifted, whole)]:
        with pytest.raises(L.Overlap):
            C.gemm(ctx, 1.0, A, B, 0.0, Cv)
    src = block(0, 0, 4, 4)
    for bad in ([0, 1], [1, 1]):
        with pytest.raises(L.Overlap):
            C.gemm(ctx, 1.0, src, src, 0.0, L.TensorView(other.buffer, 0, [4, 4], bad))
    assert ctx.launches() == n0
    assert np.array_equal(mat.read().view(np.uint32), mat.host.view(np.uint32))
    assert np.array_equal(other.read().view(np.uint32), other.host.view(np.uint32))
    C.gemm(ctx, 1.0, whole, whole, 0.0, apart)  # A may alias B
    got = mat.read()
    e = oracle.contract_f64(1.0, mat.host, (0, [n, n], [2 * n, 1]), "mk", mat.host,
                            (0, [n, n], [2 * n, 1]), "kn", 0.0, mat.host,
                            (n * 2 * n + n, [n, n], [2 * n, 1]), "mn")
    oracle.gate(got, e, "A aliases B")


def test_invalid_metadata_without_launch(ctx, pool):
    g = rng(1900)
    a = Tensor.random(pool, Layout.dense([4, 6]), g)
    b = Tensor.random(pool, Layout.dense([6, 5]), g)
    c = Tensor.random(pool, Layout.dense([4, 5]), g)
    av, bv, cv = a.view(), b.view(), c.view()
    C.contract(ctx, 1.0, (av, "mk"), (bv, "kn"), 0.0, (cv, "mn"))
    c1 = c.read()
    assert not np.array_equal(c1, c.host)
    n0 = ctx.launches()
    for la, lb, lc in [("mk", "kn", "m"), ("mkx", "kn", "mn"), ("mk", "jn", "mn"),
                       ("kk", "kn", "mn"), ("mk", "kn", "nm"), ("mk", "nk", "mn")]:
        with pytest.raises(L.InvalidArgument):
            C.contract(ctx, 1.0, (av, la), (bv, lb), 0.0, (cv, lc))
    with pytest.raises(L.InvalidArgument):
        C.gemm(ctx, 1.0, L.TensorView.row_major(a.buffer, 0, [4, 7]), bv, 0.0, cv)
    with pytest.raises(L.InvalidArgument):
        C.encode_gemm(ctx, ctx.queue, 1.0, L.TensorView.row_major(a.buffer, 0, [4, 7]), bv, 0.0, cv)
    with pytest.raises(L.InvalidArgument):
        C.encode_contract(ctx, ctx.queue, 1.0, (av, "mk"), (bv, "kn"), 0.0, (cv, "m"))
    ctx.sync()
    assert ctx.launches() == n0
    assert np.array_equal(c.read().view(np.uint32), c1.view(np.uint32))


def test_shared_stream_orders_dependent_work(ctx, pool):
    m, k, n, p = 37, 29, 43, 3
    g = rng(2000)
    a = Tensor.random(pool, Layout.dense([m, k]), g)
    b = Tensor.random(pool, Layout.dense([k, n]), g)
    d = Tensor.random(pool, Layout.transposed(n, p), g)
    long = Tensor.random(pool, Layout.dense([2, 40000]), g)
    ab = Tensor.random(pool, Layout.dense([m, n]), g)
    abd = Tensor.random(pool, Layout.dense([m, p]), g)
    gram = Tensor.random(pool, Layout.dense([2, 2]), g)
    ab0, abd0, gram0 = ab.host.copy(), abd.host.copy(), gram.host.copy()
    s = ctx.new_stream()
    try:
        C.encode_gemm(ctx, s, 1.0, a.view(), b.view(), 0.0, ab.view())
        C.encode_contract(ctx, s, 0.5, (ab.view(), "mn"), (d.view(), "np"), -0.5, (abd.view(), "mp"))
        C.encode_contract(ctx, s, 1.0, (long.view(), "ik"), (long.view(), "jk"), 1.0, (gram.view(), "ij"))
        s.wait_until_completed()
    finally:
        s.close()
    ab1 = ab.read()
    oracle.gate(ab1, oracle.contract_f64(1.0, a.host, a.layout.tup(), "mk", b.host, b.layout.tup(), "kn",
                                         0.0, ab0, ab.layout.tup(), "mn"), "A.B")
    oracle.gate(abd.read(), oracle.contract_f64(0.5, ab1, ab.layout.tup(), "mn", d.host, d.layout.tup(),
                                                "np", -0.5, abd0, abd.layout.tup(), "mp"), "(A.B).D")
    oracle.gate(gram.read(), oracle.contract_f64(1.0, long.host, long.layout.tup(), "ik", long.host,
                                                 long.layout.tup(), "jk", 1.0, gram0, gram.layout.tup(),
                                                 "ij"), "Gram")


def test_split_partials_shared_across_streams():
    """A context's split-K partial buffer serves calls on its own stream and on two caller
    streams, enqueued back to back with no host wait and growing three times on the way;
    every result matches the oracle. The context is then destroyed after a last use on a
    caller stream."""
    import linalg_hip as L
    from helpers import Pool
    ctx2 = L.Context.new(0)
    p2 = Pool(ctx2)
    s1, s2 = ctx2.new_stream(), ctx2.new_stream()
    try:
        shapes = [(8, 8, 65536), (40, 24, 30000), (130, 200, 20000), (192, 128, 40000),
                  (3, 5, 200001)]
        streams = [s1, ctx2.queue, s2, s1, ctx2.queue]
        jobs, last = [], 0
        for i, (m, n, k) in enumerate(shapes):
            g = rng(2100 + i)
            a = Tensor.random(p2, Layout.dense([m, k]), g)
            b = Tensor.random(p2, Layout.dense([k, n]), g)
            c = Tensor(p2, Layout.dense([m, n]))
            plan = C.plan_gemm(1.0, a.view(), b.view(), 0.0, c.view())
            assert plan["kind"] == "split", (m, n, k, plan)
            jobs.append((a, b, c, plan["scratch_bytes"] > last))
            last = max(last, plan["scratch_bytes"])
        assert sum(grow for *_, grow in jobs) >= 4  # the first call allocates, three grow it
        for (a, b, c, _), s in zip(jobs, streams):
            C.encode_gemm(ctx2, s, 1.0, a.view(), b.view(), 0.0, c.view())
        s1.wait_until_completed()
        s2.wait_until_completed()
        ctx2.sync()
        for (a, b, c, _), (m, n, k) in zip(jobs, shapes):
            want = oracle.contract_f64(1.0, a.host, a.layout.tup(), "mk", b.host, b.layout.tup(),
                                       "kn", 0.0, c.host, c.layout.tup(), "mn")
            oracle.gate(c.read(), want, f"gemm {m}x{n}x{k} across streams")
        a, b, c, _ = jobs[0]
        C.encode_gemm(ctx2, s2, 1.0, a.view(), b.view(), 0.0, c.view())
        s2.wait_until_completed()
    finally:
        s1.close()
        s2.close()
        p2.free_all()
        ctx2.close()


def test_split_partials_under_concurrent_threads(ctx, pool):
    """Four host threads, each with its own stream on one context, enqueue split-K GEMMs of
    different sizes in a loop with no host waits between calls; the shared partial buffer is
    handed out under the context's lock and ordered across streams, so every result matches
    the single-threaded one bit for bit."""
    import threading
    shapes = [(8, 8, 65536), (40, 24, 30000), (130, 200, 20000), (64, 64, 50000)]
    jobs = []
    for i, (m, n, k) in enumerate(shapes):
        g = rng(2200 + i)
        a = Tensor.random(pool, Layout.dense([m, k]), g)
        b = Tensor.random(pool, Layout.dense([k, n]), g)
        ref = Tensor(pool, Layout.dense([m, n]))
        assert C.plan_gemm(1.0, a.view(), b.view(), 0.0, ref.view())["kind"] == "split"
        C.gemm(ctx, 1.0, a.view(), b.view(), 0.0, ref.view())
        outs = [Tensor(pool, Layout.dense([m, n])) for _ in range(6)]
        jobs.append((a, b, ref.read(), outs))
    errors = []

    def worker(job):
        a, b, _, outs = job
        s = ctx.new_stream()
        try:
            for c in outs:
                C.encode_gemm(ctx, s, 1.0, a.view(), b.view(), 0.0, c.view())
            s.wait_until_completed()
        except BaseException as e:  # reported below
            errors.append(e)
        finally:
            s.close()

    threads = [threading.Thread(target=worker, args=(j,)) for j in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not errors and not any(t.is_alive() for t in threads)
    for _, _, want, outs in jobs:
        for c in outs:
            assert np.array_equal(c.read().view(np.uint32), want.view(np.uint32))


# --------------------------------------------------------------------------------------
# Random einsum sweep (tests/contraction_test.rs:1008-1096), own seeded generator.
# --------------------------------------------------------------------------------------
def random_operand(labels, g):
    logical = list(labels)
    order = list(range(len(logical)))
    for i in range(len(logical) - 1, 0, -1):
        j = int(g.integers(0, i + 1))
        logical[i], logical[j] = logical[j], logical[i]
        j = int(g.integers(0, i + 1))
        order[i], order[j] = order[j], order[i]
    shape = [n for _, n in logical]
    steps = [int(g.integers(1, 3)) for _ in shape]
    return Layout.with_(shape, order, steps, int(g.integers(0, 8))), "".join(l for l, _ in logical)


def test_random_contractions(ctx, pool):
    g = rng(0xC0FFEE)
    for case_no in range(96):
        def extent():
            r = g.integers(0, 12)
            if r == 0:
                return 0
            if r <= 2:
                return 1
            if r <= 10:
                return int(g.integers(2, 7))
            return int(g.integers(17, 41))
        groups = [[extent() for _ in range(int(g.integers(0, 3)))] for _ in range(4)]
        while np.prod([max(n, 1) for grp in groups for n in grp]) > 400000:
            flat = [(n, gi, i) for gi, grp in enumerate(groups) for i, n in enumerate(grp)]
            n, gi, i = max(flat)
            groups[gi][i] = (n + 1) // 2
        names = iter("abcdefgh")
        lab = [[(next(names), n) for n in grp] for grp in groups]
        batch, m, n, k = lab
        lg = rng(int(g.integers(0, 2 ** 63)))
        a, la = random_operand(batch + m + k, lg)
        b, lb = random_operand(batch + n + k, lg)
        c, lc = random_operand(batch + m + n, lg)
        alpha = [1.0, -0.75, 0.0][int(g.integers(0, 3))]
        beta = [0.0, 1.0, -0.5][int(g.integers(0, 3))]
        Case(f"random #{case_no} {la},{lb}->{lc} {groups}", (a, la), (b, lb), (c, lc)).scalars(
            alpha, beta).run(ctx, pool, int(lg.integers(0, 2 ** 31)))


def test_tile_edge_sweep(ctx, pool):
    """Ragged M/N/K around the 128x128x32 tile and the 64-row wave tile."""
    seed = 5000
    for m in [1, 31, 32, 33, 63, 64, 65, 127, 128, 129]:
        for n in [1, 33, 64, 127, 129]:
            for k in [1, 7, 31, 32, 33, 64, 100]:
                if (m * n * k) % 3:
                    continue
                alpha, beta = [(1.0, 0.0), (-0.75, 1.0), (0.5, -0.5), (2.0, 0.0)][seed % 4]
                Case.matmul(m, n, k).scalars(alpha, beta).run(ctx, pool, seed)
                seed += 1


def test_both_output_tiles_on_ragged_edges(ctx, pool):
    """Grids of at least 256 128x128 tiles take 128x128 tiles, smaller ones with short K
    64x64 (with split-K on top when K allows): ragged M/N/K at each, against both oracles."""
    seed = 6100
    for m, n, k in [(2100, 2050, 37), (2047, 2177, 129), (1900, 1950, 45), (130, 250, 300),
                    (200, 190, 2000)]:
        alpha, beta = [(1.0, 0.0), (-0.75, 1.0), (0.5, -0.5)][seed % 3]
        Case.matmul(m, n, k).scalars(alpha, beta).run(ctx, pool, seed)
        seed += 1


def test_transposed_a_direct_load_pipeline(ctx, pool):
    """A read along M (transpose_matrix(X), the weight-gradient operand) through the 128x128
    direct-load kernel's three-stage pipeline: K shorter than the pipeline, full slices followed
    by a partial last slice loaded through registers, exact slices, ragged M/N edge tiles (loaded
    through registers), split-K chunks, and both B layouts, against both oracles."""
    seed = 6200
    cases = [((3000, 2050, 37), (False,)), ((3000, 2060, 147), (False, True)),
             ((2048, 2048, 96), (False,)), ((400, 300, 8192), (False, True))]
    for (m, n, k), b_layouts in cases:
        for tb in b_layouts:
            alpha, beta = [(1.0, 0.0), (-0.75, 1.0), (0.5, -0.5)][seed % 3]
            case = Case(f"A^T tb={tb} {m}x{n}x{k}", (Layout.transposed(m, k), "mk"),
                        (Layout.transposed(k, n) if tb else Layout.dense([k, n]), "kn"),
                        (Layout.dense([m, n]), "mn"), via_gemm=True)
            plan = C.plan_gemm(alpha, _dummy_view(pool, case.a[0]), _dummy_view(pool, case.b[0]),
                               beta, _dummy_view(pool, case.c[0]))
            assert plan["tile"] == (128, 128) and plan["a_mode"] == "mn", plan
            # A B row pitch off a multiple of four elements has no 16-byte aligned unit-stride
            # axis: the register-staged kernel; every other case loads slices straight into LDS.
            assert plan["kernel"] == ("tile" if plan["b_mode"] == "strided" else "direct"), plan
            case.scalars(alpha, beta).run(ctx, pool, seed)
            pool.free_all()
            seed += 1


def test_transposed_a_pipeline_batched(ctx, pool):
    """Batched products whose A is read along M take the same direct-load kernel per batch
    plane: four 1024x1024x256 planes (256 tiles of 128x128, no split-K)."""
    b, m, n, k = 4, 1024, 1024, 256
    case = Case("batched A^T", (Layout.with_([b, m, k], [0, 2, 1], [1, 1, 1], 0), "bmk"),
                (Layout.dense([b, k, n]), "bkn"), (Layout.dense([b, m, n]), "bmn"))
    plan = C.plan_contract(0.5, (_dummy_view(pool, case.a[0]), "bmk"),
                           (_dummy_view(pool, case.b[0]), "bkn"), 1.0,
                           (_dummy_view(pool, case.c[0]), "bmn"))
    assert plan["tile"] == (128, 128) and plan["a_mode"] == "mn" and plan["splits"] == 1, plan
    pool.free_all()
    case.scalars(0.5, 1.0).run(ctx, pool, 6400)


def test_transposed_a_pipeline_is_deterministic(ctx, pool):
    """The direct-load pipeline with split-K chunks (A read along M) gives the same bits on
    three runs, with beta = 1 accumulating into the same starting C each time."""
    m, n, k = 400, 300, 8192
    g = rng(6300)
    a = Tensor.random(pool, Layout.transposed(m, k), g)
    b = Tensor.random(pool, Layout.dense([k, n]), g)
    c = Tensor.random(pool, Layout.dense([m, n]), g)
    c0 = c.host.copy()
    plan = C.plan_gemm(0.5, a.view(), b.view(), 1.0, c.view())
    assert plan["tile"] == (128, 128) and plan["a_mode"] == "mn" and plan["splits"] > 1, plan
    outs = []
    for _ in range(3):
        c.host[:] = c0
        c.upload()
        C.gemm(ctx, 0.5, a.view(), b.view(), 1.0, c.view())
        outs.append(c.read().view(np.uint32).copy())
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def _dummy_view(pool, layout):
    buf = pool.alloc("f32", layout.span() + 64)
    return L.TensorView(buf, layout.offset, layout.shape, layout.strides, "f32")


# --------------------------------------------------------------------------------------
# benchmark configurations at full size
# --------------------------------------------------------------------------------------
def _rows_check(name, got_rows, want_rows, k, amax, bmax):
    """The north-star bound on every element given: max|err| <= 1e-5*sqrt(K)*max|a|*max|b|."""
    tol = 1e-5 * np.sqrt(k) * amax * bmax
    err = np.abs(got_rows.astype(np.float64) - want_rows.astype(np.float64))
    worst = int(np.argmax(err))
    assert err[worst] <= tol and np.all(np.isfinite(got_rows)), (
        f"{name}: max|err| {err[worst]:e} > {tol:e} at element {worst}")
    return float(err[worst])


def test_config1_gemm_512_full_oracle(ctx, pool):
    m = n = k = 512
    g = rng(1)
    a = g.uniform(-1, 1, m * k).astype(np.float32)
    b = rng(2).uniform(-1, 1, k * n).astype(np.float32)
    A, B, Cc = (Tensor(pool, Layout.dense(s), d) for s, d in
                (([m, k], a), ([k, n], b), ([m, n], np.zeros(m * n, np.float32))))
    C.gemm(ctx, 1.0, A.view(), B.view(), 0.0, Cc.view())
    got = Cc.read()[: m * n]
    ref = np.zeros(m * n, np.float32)
    oracle.gemm_fast(m, n, k, 1.0, 0.0, a, 0, (k, 1), b, 0, (n, 1), ref, 0, (n, 1))
    _rows_check("config 1", got, ref, k, 1.0, 1.0)
    e = oracle.contract_f64(1.0, a, (0, [m, k], [k, 1]), "mk", b, (0, [k, n], [n, 1]), "kn", 0.0,
                            ref, (0, [m, n], [n, 1]), "mn")
    oracle.gate(got, e, "config 1")


def test_config3_batched_with_permuted_b(ctx, pool):
    bsz, m = 32, 1024
    g = rng(5)
    a = g.uniform(-1, 1, bsz * m * m).astype(np.float32)
    bstore = rng(6).uniform(-1, 1, bsz * m * m).astype(np.float32)  # [b, j, k]
    A = Tensor(pool, Layout.dense([bsz, m, m]), a)
    Bs = Tensor(pool, Layout.dense([bsz, m, m]), bstore)
    Cc = Tensor(pool, Layout.dense([bsz, m, m]))
    bview = P.permute_view(Bs.view(), [0, 2, 1])  # "bkj": strides [2^20, 1, 1024]
    assert bview.strides == [m * m, 1, m]
    plan = C.plan_contract(1.0, (A.view(), "bik"), (bview, "bkj"), 0.0, (Cc.view(), "bij"))
    assert plan["kind"] == "tiled" and plan["b_mode"] == "k"
    C.contract(ctx, 1.0, (A.view(), "bik"), (bview, "bkj"), 0.0, (Cc.view(), "bij"))
    got = Cc.read()[: bsz * m * m]
    # Every output of every batch against crates/cpu's layout (RM, Transposed, RM):
    # B[k][j] = Bstore[j][k], strides [1, K].
    for bi in range(bsz):
        ref = np.zeros(m * m, np.float32)
        oracle.gemm_fast(m, m, m, 1.0, 0.0, a, bi * m * m, (m, 1), bstore, bi * m * m, (1, m),
                         ref, 0, (m, 1))
        _rows_check(f"config 3 batch {bi}", got[bi * m * m:(bi + 1) * m * m], ref, m, 1.0, 1.0)


def test_config4_split_k_full_oracle_and_deterministic(ctx, pool):
    m = n = 256
    k = 65536
    sigma = 1.0 / np.sqrt(k)
    a = (rng(7).standard_normal(m * k) * sigma).astype(np.float32)
    b = (rng(8).standard_normal(k * n) * sigma).astype(np.float32)
    A = Tensor(pool, Layout.dense([m, k]), a)
    B = Tensor(pool, Layout.dense([k, n]), b)
    plan = C.plan_gemm(1.0, A.view(), B.view(), 0.0, Tensor(pool, Layout.dense([m, n])).view())
    assert plan["kind"] == "split"
    outs = []
    for _ in range(3):
        Cc = Tensor(pool, Layout.dense([m, n]))
        C.gemm(ctx, 1.0, A.view(), B.view(), 0.0, Cc.view())
        outs.append(Cc.read()[: m * n].copy())
    assert all(np.array_equal(outs[0].view(np.uint32), o.view(np.uint32)) for o in outs[1:])
    ref = np.zeros(m * n, np.float32)
    oracle.gemm_fast(m, n, k, 1.0, 0.0, a, 0, (k, 1), b, 0, (n, 1), ref, 0, (n, 1))
    _rows_check("config 4", outs[0], ref, k, float(np.abs(a).max()), float(np.abs(b).max()))


def test_config5_linear_layer_step(ctx, pool):
    """One 1F1B stage's linear step: Y = X.W, dX = dY.W^T, dW += X^T.dY (transposed views)."""
    M, K, N = 4096, 4096, 16384
    x = (rng(9).standard_normal(M * K) * 0.02).astype(np.float32)
    w = (rng(10).standard_normal(K * N) * 0.02).astype(np.float32)
    dy = (rng(11).standard_normal(M * N) * 0.02).astype(np.float32)
    X = Tensor(pool, Layout.dense([M, K]), x)
    W = Tensor(pool, Layout.dense([K, N]), w)
    DY = Tensor(pool, Layout.dense([M, N]), dy)
    Y = Tensor(pool, Layout.dense([M, N]))
    DX = Tensor(pool, Layout.dense([M, K]))
    DW = Tensor(pool, Layout.dense([K, N]))
    Wt = L.TensorView(W.buffer, 0, [N, K], [1, N])   # transpose_matrix(W)
    Xt = L.TensorView(X.buffer, 0, [K, M], [1, K])   # transpose_matrix(X)
    C.gemm(ctx, 1.0, X.view(), W.view(), 0.0, Y.view())
    C.gemm(ctx, 1.0, DY.view(), Wt, 0.0, DX.view())
    C.gemm(ctx, 1.0, Xt, DY.view(), 1.0, DW.view())   # dW starts at zero, beta = 1 accumulates
    y, dx, dw = Y.read()[: M * N], DX.read()[: M * K], DW.read()[: K * N]
    ax, aw, ady = (float(np.abs(t).max()) for t in (x, w, dy))
    # Y = X.W: every element.
    ref = np.zeros(M * N, np.float32)
    oracle.gemm_fast(M, N, K, 1.0, 0.0, x, 0, (K, 1), w, 0, (N, 1), ref, 0, (N, 1))
    _rows_check("Y", y, ref, K, ax, aw)
    # dX = dY.W^T and dW = X^T.dY: every element too (about 20 s of the threaded oracle).
    ref = np.zeros(M * K, np.float32)
    oracle.gemm_fast(M, K, N, 1.0, 0.0, dy, 0, (N, 1), w, 0, (1, N), ref, 0, (K, 1))
    _rows_check("dX", dx, ref, N, ady, aw)
    ref = np.zeros(K * N, np.float32)
    oracle.gemm_fast(K, N, M, 1.0, 1.0, x, 0, (1, K), dy, 0, (N, 1), ref, 0, (N, 1))
    _rows_check("dW", dw, ref, M, ax, ady)


def test_gemm_4096_cubed_full_oracle_and_linearity(ctx, pool):
    n = 4096
    a = rng(12).uniform(-1, 1, n * n).astype(np.float32)
    b = rng(13).uniform(-1, 1, n * n).astype(np.float32)
    A, B = Tensor(pool, Layout.dense([n, n]), a), Tensor(pool, Layout.dense([n, n]), b)
    C1, C2 = Tensor(pool, Layout.dense([n, n])), Tensor(pool, Layout.dense([n, n]))
    C.gemm(ctx, 1.0, A.view(), B.view(), 0.0, C1.view())
    # Linearity: C2 = 2*A.B computed as alpha = 2 must be exactly twice C1 (power-of-two scale).
    C.gemm(ctx, 2.0, A.view(), B.view(), 0.0, C2.view())
    c1, c2 = C1.read()[: n * n], C2.read()[: n * n]
    assert np.array_equal((c1 * np.float32(2)).view(np.uint32), c2.view(np.uint32))
    # Every output element against the crates/cpu restatement.
    ref = np.zeros(n * n, np.float32)
    oracle.gemm_fast(n, n, n, 1.0, 0.0, a, 0, (n, 1), b, 0, (n, 1), ref, 0, (n, 1))
    _rows_check("4096^3", c1, ref, n, 1.0, 1.0)


@pytest.mark.parametrize("m,n,k", [(300, 200, 100), (256, 256, 8192)])
def test_gemm_nowait_is_ordered_before_a_download(ctx, pool, m, n, k):
    """gemm_nowait (src/ops/contraction.rs:1116-1130) enqueues on the context stream and returns
    before the device finishes; a download (ordered after it on that stream) sees the result,
    bit for bit what the synchronous gemm stores. A second gemm_nowait that reads the first one's
    output, with no wait between them, sees the finished values. (256x256x8192 is split-K.)"""
    g = rng(m + n + k)
    a = g.uniform(-1, 1, m * k).astype(np.float32)
    b = g.uniform(-1, 1, k * n).astype(np.float32)
    sq = g.uniform(-1, 1, n * n).astype(np.float32)
    A = Tensor(pool, Layout.dense([m, k]), a)
    B = Tensor(pool, Layout.dense([k, n]), b)
    SQ = Tensor(pool, Layout.dense([n, n]), sq)
    nan = np.full(m * n, np.nan, np.float32)
    C1, C2, D = (Tensor(pool, Layout.dense([m, n]), nan) for _ in range(3))
    C.gemm(ctx, 1.0, A.view(), B.view(), 0.0, C1.view())
    assert C.gemm_nowait(ctx, 1.0, A.view(), B.view(), 0.0, C2.view()) is ctx.queue
    C.gemm_nowait(ctx, 1.0, C2.view(), SQ.view(), 0.0, D.view())
    c1, c2, d = C1.read()[: m * n], C2.read()[: m * n], D.read()[: m * n]
    assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32))
    ref = np.zeros(m * n, np.float32)
    oracle.gemm_fast(m, n, k, 1.0, 0.0, a, 0, (k, 1), b, 0, (n, 1), ref, 0, (n, 1))
    _rows_check("gemm_nowait C", c2, ref, k, 1.0, 1.0)
    ref2 = np.zeros(m * n, np.float32)
    oracle.gemm_fast(m, n, n, 1.0, 0.0, c2, 0, (n, 1), sq, 0, (n, 1), ref2, 0, (n, 1))
    _rows_check("gemm_nowait D", d, ref2, n, float(np.abs(c2).max()), 1.0)


def _gemm_fast_check(name, got_buf, a, la, b, lb, c0, lc, m, n, k, alpha, beta):
    """Every element of C (layout lc inside got_buf) against the crates/cpu restatement."""
    ref = c0.copy()
    oracle.gemm_fast(m, n, k, alpha, beta, a, la.offset, la.strides, b, lb.offset, lb.strides,
                     ref, lc.offset, lc.strides)
    idx = (lc.offset + np.arange(m)[:, None] * lc.strides[0] +
           np.arange(n)[None, :] * lc.strides[1]).ravel()
    tol = 1e-5 * np.sqrt(k) * abs(alpha) + (1e-5 * abs(beta) if beta != 0.0 else 0.0)
    err = np.abs(got_buf[idx].astype(np.float64) - ref[idx].astype(np.float64))
    assert np.all(np.isfinite(got_buf[idx])) and float(err.max()) <= tol, (name, float(err.max()), tol)


@pytest.mark.parametrize("ta,tb,tc", [(False, False, False), (True, False, False), (False, True, False),
                                      (True, True, False), (False, False, True)])
def test_wide_direct_load_tiles_with_ragged_edges(ctx, pool, ta, tb, tc):
    """128x256 direct-load tiles (grids of at least 512 of them): ragged M and N edge tiles and a
    partial last K-slice (both loaded through registers), every operand layout pair, and C
    stored column-major (computed transposed), against crates/cpu on every element."""
    m, n, k = 4100, 4100, 1000
    pick = lambda t, r, c: Layout.transposed(r, c) if t else Layout.dense([r, c])
    la, lb, lc = pick(ta, m, k), pick(tb, k, n), pick(tc, m, n)
    g = rng(7300 + 4 * ta + 2 * tb + tc)
    alpha, beta = (1.0, 0.0) if not (ta or tb) else (-0.75, 0.5)
    A, B = Tensor.random(pool, la, g), Tensor.random(pool, lb, g)
    Cc = Tensor.random(pool, lc, g)
    plan = C.plan_gemm(alpha, A.view(), B.view(), beta, Cc.view())
    assert (plan["kernel"], plan["tile"]) == ("direct", (128, 256)), plan
    c0 = Cc.host.copy()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    _gemm_fast_check(f"wide ta={ta} tb={tb} tc={tc}", Cc.read(), A.host, la, B.host, lb, c0, lc,
                     m, n, k, alpha, beta)


def test_wide_direct_load_batched_with_permuted_b(ctx, pool):
    """Eight 1100x2100x300 planes with B a permuted view (unit stride along K), beta = 1: 648
    wide tiles, ragged in M and N."""
    bsz, m, n, k = 8, 1100, 2100, 300
    g = rng(7400)
    a = g.uniform(-1, 1, bsz * m * k).astype(np.float32)
    bstore = g.uniform(-1, 1, bsz * n * k).astype(np.float32)  # [b, n, k]
    c0 = g.uniform(-1, 1, bsz * m * n).astype(np.float32)
    A = Tensor(pool, Layout.dense([bsz, m, k]), a)
    Bs = Tensor(pool, Layout.dense([bsz, n, k]), bstore)
    Cc = Tensor(pool, Layout.dense([bsz, m, n]), c0)
    bview = P.permute_view(Bs.view(), [0, 2, 1])
    plan = C.plan_contract(0.5, (A.view(), "bik"), (bview, "bkj"), 1.0, (Cc.view(), "bij"))
    assert (plan["kernel"], plan["tile"], plan["b_mode"]) == ("direct", (128, 256), "k"), plan
    C.contract(ctx, 0.5, (A.view(), "bik"), (bview, "bkj"), 1.0, (Cc.view(), "bij"))
    got = Cc.read()
    for bi in range(bsz):
        ref = c0[bi * m * n:(bi + 1) * m * n].copy()
        oracle.gemm_fast(m, n, k, 0.5, 1.0, a, bi * m * k, (k, 1), bstore, bi * n * k, (1, k),
                         ref, 0, (n, 1))
        err = np.abs(got[bi * m * n:(bi + 1) * m * n].astype(np.float64) - ref.astype(np.float64))
        assert float(err.max()) <= 1e-5 * np.sqrt(k) * 0.5 + 1e-5, (bi, float(err.max()))


@pytest.mark.parametrize("m,n,k,ta,tb,tc", [(2048, 2048, 1936, False, False, False),
                                            (1952, 2040, 1004, True, False, False),
                                            (2040, 1932, 300, False, True, True),
                                            (2048, 1924, 260, True, True, False)])
def test_two_wave_groups_per_workgroup(ctx, pool, m, n, k, ta, tb, tc):
    """Grids of exactly 256 128x128 direct-load tiles (one workgroup per compute unit) run two
    wave groups per workgroup, each on half of the K slices, their sums added in group order:
    ragged M and N edges, K not in whole steps of the pipelined kernel (K = 1936), odd slice
    counts (the second group one slice short: K = 1004, 63 slices; K = 260, 17), partial last
    slices (K = 1004, 300, 260), every operand layout, and C
    column-major, against crates/cpu on every element; the same bits over two runs."""
    pick = lambda t, r, c: Layout.transposed(r, c) if t else Layout.dense([r, c])
    la, lb, lc = pick(ta, m, k), pick(tb, k, n), pick(tc, m, n)
    g = rng(7500 + m + n + k)
    alpha, beta = (1.0, 0.0) if not (ta or tb) else (0.75, -0.5)
    A, B = Tensor.random(pool, la, g), Tensor.random(pool, lb, g)
    Cc = Tensor.random(pool, lc, g)
    plan = C.plan_gemm(alpha, A.view(), B.view(), beta, Cc.view())
    assert (plan["kernel"], plan["tile"], plan["kgroups"], plan["workgroups"]) == \
        ("direct", (128, 128), 2, 256), plan
    c0 = Cc.host.copy()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    first = Cc.read().copy()
    Cc.host[:] = c0
    Cc.upload()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    assert np.array_equal(first.view(np.uint32), Cc.read().view(np.uint32))
    _gemm_fast_check(f"two groups {m}x{n}x{k} ta={ta} tb={tb} tc={tc}", first, A.host, la,
                     B.host, lb, c0, lc, m, n, k, alpha, beta)


@pytest.mark.parametrize("m,n,k,ta,tb,tc", [(1024, 1024, 1000, False, False, False),
                                            (1000, 1020, 900, True, False, False),
                                            (1020, 968, 1000, False, True, True),
                                            (964, 1024, 516, True, True, False)])
def test_four_wave_groups_on_64x64_tiles(ctx, pool, m, n, k, ta, tb, tc):
    """Grids of exactly 256 64x64 tiles (a 128x128 grid would need split-K) on the direct-load
    kernel with four wave groups of 32-deep slices: ragged edges, K not in whole steps of the
    K-split kernel (K = 1000), groups with fewer slices than the others (K = 900: 8, 8, 8, 5
    slices; K = 516: 5, 5, 5, 2), partial last slices,
    every operand layout and C column-major, against crates/cpu on every element; the same
    bits over two runs."""
    pick = lambda t, r, c: Layout.transposed(r, c) if t else Layout.dense([r, c])
    la, lb, lc = pick(ta, m, k), pick(tb, k, n), pick(tc, m, n)
    g = rng(7600 + m + n + k)
    alpha, beta = (1.0, 0.0) if not (ta or tb) else (-1.25, 0.5)
    A, B = Tensor.random(pool, la, g), Tensor.random(pool, lb, g)
    Cc = Tensor.random(pool, lc, g)
    plan = C.plan_gemm(alpha, A.view(), B.view(), beta, Cc.view())
    assert (plan["kernel"], plan["tile"], plan["kgroups"], plan["workgroups"]) == \
        ("direct", (64, 64), 4, 256), plan
    c0 = Cc.host.copy()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    first = Cc.read().copy()
    Cc.host[:] = c0
    Cc.upload()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    assert np.array_equal(first.view(np.uint32), Cc.read().view(np.uint32))
    _gemm_fast_check(f"four groups {m}x{n}x{k} ta={ta} tb={tb} tc={tc}", first, A.host, la,
                     B.host, lb, c0, lc, m, n, k, alpha, beta)


@pytest.mark.parametrize("m,n,k,ta,tb,tc", [(1024, 1024, 1024, False, False, False),
                                            (1024, 1024, 512, True, False, False),
                                            (1024, 1024, 768, False, True, True),
                                            (1024, 1024, 1536, True, True, False)])
def test_k_split_waves_on_64x64_tiles(ctx, pool, m, n, k, ta, tb, tc):
    """Grids of 256 full 64x64 tiles on the kernel whose four waves each take a quarter of K
    through their own stages (K = 512: eight 16-deep slices per wave, one loop pass of four
    stages twice): every operand layout, with C column-major the swapped product, alpha != 1
    with beta != 0, against crates/cpu on every element; the same bits over two runs (the four
    quarter sums are added in a fixed order)."""
    pick = lambda t, r, c: Layout.transposed(r, c) if t else Layout.dense([r, c])
    la, lb, lc = pick(ta, m, k), pick(tb, k, n), pick(tc, m, n)
    g = rng(7800 + m + n + k)
    alpha, beta = (1.0, 0.0) if not (ta or tc) else (-0.75, 0.5)
    A, B = Tensor.random(pool, la, g), Tensor.random(pool, lb, g)
    Cc = Tensor.random(pool, lc, g)
    plan = C.plan_gemm(alpha, A.view(), B.view(), beta, Cc.view())
    assert (plan["kernel"], plan["tile"], plan["kgroups"], plan["workgroups"]) == \
        ("pipelined", (64, 64), 4, 256), plan
    c0 = Cc.host.copy()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    first = Cc.read().copy()
    Cc.host[:] = c0
    Cc.upload()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    assert np.array_equal(first.view(np.uint32), Cc.read().view(np.uint32))
    _gemm_fast_check(f"k-split waves {m}x{n}x{k} ta={ta} tb={tb} tc={tc}", first, A.host, la,
                     B.host, lb, c0, lc, m, n, k, alpha, beta)


@pytest.mark.parametrize("m,n,k,ta,tb,tc,splits", [(512, 512, 16384, True, False, False, 4),
                                                   (256, 512, 8192, False, True, True, 8),
                                                   (256, 256, 16384, True, True, False, 16)])
def test_k_split_waves_split_along_k(ctx, pool, m, n, k, ta, tb, tc, splits):
    """Short outputs with long K: 64x64 tiles of the K-split-wave kernel, split along K to about
    one workgroup per compute unit, partials added in split order by the reduction: (MN, MN),
    the swapped (K, K) product with C column-major, (MN, K) with 16 splits of 1024; alpha != 1,
    beta != 0; against crates/cpu on every element, the same bits over two runs. (With inputs
    uniform on [-1, 1], K stays at most 16384: both sides accumulate in f32, and for longer K
    their rounding alone approaches the bound.)"""
    pick = lambda t, r, c: Layout.transposed(r, c) if t else Layout.dense([r, c])
    la, lb, lc = pick(ta, m, k), pick(tb, k, n), pick(tc, m, n)
    g = rng(7900 + m + n + k)
    alpha, beta = 0.75, -0.5
    A, B = Tensor.random(pool, la, g), Tensor.random(pool, lb, g)
    Cc = Tensor.random(pool, lc, g)
    plan = C.plan_gemm(alpha, A.view(), B.view(), beta, Cc.view())
    assert (plan["kind"], plan["kernel"], plan["tile"], plan["splits"], plan["workgroups"]) == \
        ("split", "pipelined", (64, 64), splits, 256), plan
    c0 = Cc.host.copy()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    first = Cc.read().copy()
    Cc.host[:] = c0
    Cc.upload()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    assert np.array_equal(first.view(np.uint32), Cc.read().view(np.uint32))
    _gemm_fast_check(f"k-split waves, split {m}x{n}x{k} ta={ta} tb={tb} tc={tc}", first, A.host, la,
                     B.host, lb, c0, lc, m, n, k, alpha, beta)


@pytest.mark.parametrize("m,n,k,ta,tb,tc,splits", [(1024, 1024, 16384, False, True, False, 8),
                                                   (1024, 2048, 8192, True, False, True, 4)])
def test_pipelined_kernel_split_along_k(ctx, pool, m, n, k, ta, tb, tc, splits):
    """Split-K on the pipelined 128x128 kernel (outputs too large for the 64x64 K-split
    waves): raw partials in chunks of 2048, added in split order by the reduction; (K, K) and,
    with C column-major, the swapped product; against crates/cpu on every element, the same
    bits over two runs."""
    pick = lambda t, r, c: Layout.transposed(r, c) if t else Layout.dense([r, c])
    la, lb, lc = pick(ta, m, k), pick(tb, k, n), pick(tc, m, n)
    g = rng(8100 + m + n + k)
    alpha, beta = (1.0, 0.0) if not tc else (0.75, -0.5)
    A, B = Tensor.random(pool, la, g), Tensor.random(pool, lb, g)
    Cc = Tensor.random(pool, lc, g)
    plan = C.plan_gemm(alpha, A.view(), B.view(), beta, Cc.view())
    assert (plan["kind"], plan["kernel"], plan["tile"], plan["splits"], plan["workgroups"]) == \
        ("split", "pipelined", (128, 128), splits, 512), plan
    c0 = Cc.host.copy()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    first = Cc.read().copy()
    Cc.host[:] = c0
    Cc.upload()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    assert np.array_equal(first.view(np.uint32), Cc.read().view(np.uint32))
    _gemm_fast_check(f"pipelined split {m}x{n}x{k} ta={ta} tb={tb} tc={tc}", first, A.host, la,
                     B.host, lb, c0, lc, m, n, k, alpha, beta)


@pytest.mark.parametrize("m,n,k,ta,tb,tc", [(2304, 2240, 256, False, False, False),
                                            (2048, 2880, 128, True, False, False),
                                            (2880, 2048, 192, False, True, True),
                                            (2304, 2240, 64, True, True, False)])
def test_pipelined_128x64_tiles(ctx, pool, m, n, k, ta, tb, tc):
    """Grids of 512-768 full 128x64 tiles whose N is not a multiple of 128 (full 128x128 grids
    of that size take stream-K): three pipelined workgroups per compute unit in one round.
    (K, MN), (MN, MN), the swapped (K, K) product with C column-major, (MN, K) with K of one
    pipeline step; alpha != 1 with beta != 0; against crates/cpu on every element, the same
    bits over two runs."""
    pick = lambda t, r, c: Layout.transposed(r, c) if t else Layout.dense([r, c])
    la, lb, lc = pick(ta, m, k), pick(tb, k, n), pick(tc, m, n)
    g = rng(8000 + m + n + k)
    alpha, beta = (1.0, 0.0) if not (ta or tc) else (0.75, -0.5)
    A, B = Tensor.random(pool, la, g), Tensor.random(pool, lb, g)
    Cc = Tensor.random(pool, lc, g)
    plan = C.plan_gemm(alpha, A.view(), B.view(), beta, Cc.view())
    assert (plan["kernel"], plan["tile"], plan["workgroups"]) == \
        ("pipelined", (128, 64), m * n // (128 * 64)), plan
    c0 = Cc.host.copy()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    first = Cc.read().copy()
    Cc.host[:] = c0
    Cc.upload()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    assert np.array_equal(first.view(np.uint32), Cc.read().view(np.uint32))
    _gemm_fast_check(f"pipelined 128x64 {m}x{n}x{k} ta={ta} tb={tb} tc={tc}", first, A.host, la,
                     B.host, lb, c0, lc, m, n, k, alpha, beta)


@pytest.mark.parametrize("m,n,k,ta,tb,tc,tile_m", [(4096, 2048, 192, False, False, False, 256),
                                                   (4096, 2048, 128, True, False, False, 128),
                                                   (2048, 4096, 256, False, True, True, 256),
                                                   (4096, 2048, 64, True, True, False, 128),
                                                   (4096, 2048, 4224, False, True, False, 128),
                                                   (2048, 2048, 2048, False, False, False, 128),
                                                   (2048, 2048, 1152, True, True, True, 128)])
def test_pipelined_kernel(ctx, pool, m, n, k, ta, tb, tc, tile_m):
    """Full tiles on the software-pipelined kernel. Grids of 512 128x128 tiles (16-deep
    slices): every operand layout ((K, MN), (MN, MN), (MN, K) and, with C column-major, the
    swapped product), alpha != 1 (fragments scaled as they are read) with beta != 0, K of one
    pipeline step (64) and of several; those whose A-role operand is contiguous along K run as
    256 tiles of 256x128 with eight waves (gemm_f32_pl256). (K, K) operands with K >= 4096
    (32-deep slices, K = 4224: 132 slices). Grids of 256 tiles (one workgroup per compute
    unit, 32-deep slices), also swapped. Against crates/cpu on every element; the same bits
    over two runs."""
    pick = lambda t, r, c: Layout.transposed(r, c) if t else Layout.dense([r, c])
    la, lb, lc = pick(ta, m, k), pick(tb, k, n), pick(tc, m, n)
    g = rng(7700 + m + n + k)
    alpha, beta = (1.0, 0.0) if not (ta or tc) else (0.75, -0.5)
    A, B = Tensor.random(pool, la, g), Tensor.random(pool, lb, g)
    Cc = Tensor.random(pool, lc, g)
    plan = C.plan_gemm(alpha, A.view(), B.view(), beta, Cc.view())
    assert (plan["kernel"], plan["tile"], plan["kgroups"], plan["workgroups"]) == \
        ("pipelined", (tile_m, 128), 1, m * n // (tile_m * 128)), plan
    c0 = Cc.host.copy()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    first = Cc.read().copy()
    Cc.host[:] = c0
    Cc.upload()
    C.gemm(ctx, alpha, A.view(), B.view(), beta, Cc.view())
    assert np.array_equal(first.view(np.uint32), Cc.read().view(np.uint32))
    _gemm_fast_check(f"pipelined {m}x{n}x{k} ta={ta} tb={tb} tc={tc}", first, A.host, la,
                     B.host, lb, c0, lc, m, n, k, alpha, beta)


@pytest.mark.parametrize("m,n,k,tc,batch,bk,ab", [(4096, 4096, 512, False, 1, True, False),
                                                  (4096, 4096, 1088, True, 1, True, True),
                                                  (1024, 1024, 256, False, 16, True, False),
                                                  (4096, 4096, 4160, False, 1, True, False),
                                                  (4096, 4096, 320, False, 1, False, False),
                                                  (4096, 4096, 1088, False, 1, False, True),
                                                  (1024, 1024, 256, False, 16, False, True)])
def test_pipelined_256x256_tiles(ctx, pool, m, n, k, tc, batch, bk, ab):
    """A row-major with B transposed (K, K) or row-major (K, MN, whose B loads go out apart from
    the A loads), 256x256 tiles numbering at least one per compute unit: gemm_f32_pl2x (eight
    waves of 4x2 blocks). 256 tiles; with C column-major (the swapped product, K = 1088: 17
    pipeline steps); 16 batches of 16 tiles; K = 4160 (65 steps), which 128x128 tiles would take
    on 32-deep slices; alpha != 1 with beta != 0 where marked, else C filled with NaN (beta = 0
    never reads it). Against crates/cpu on every element of every batch; the same bits over
    two runs."""
    la = Layout(0, [batch, m, k], [m * k, k, 1])
    lb = Layout(0, [batch, k, n], [k * n, 1, k] if bk else [k * n, n, 1])
    lc = Layout(0, [batch, m, n], [m * n, 1, m] if tc else [m * n, n, 1])
    g = rng(7750 + m + k + batch + 2 * bk)
    alpha, beta = (0.75, -0.5) if ab else (1.0, 0.0)
    A, B, Cc = Tensor.random(pool, la, g), Tensor.random(pool, lb, g), Tensor.random(pool, lc, g)
    if beta == 0.0:  # C must never be read: NaN there would reach the result
        Cc.host[:] = np.nan
        Cc.upload()
    if batch == 1:  # plain matrices: the same buffers as rank-2 views
        mat = lambda t_: L.TensorView(t_.buffer, 0, t_.layout.shape[1:], t_.layout.strides[1:])
        av, bv, cv = mat(A), mat(B), mat(Cc)
    else:
        av, bv, cv = A.view(), B.view(), Cc.view()
    plan = C.plan_gemm(alpha, av, bv, beta, cv)
    assert (plan["kernel"], plan["tile"], plan["kgroups"], plan["workgroups"], plan["b_mode"]) == \
        ("pipelined", (256, 256), 1, batch * m * n // 65536, "k" if bk else "mn"), plan
    c0 = Cc.host.copy()
    C.gemm(ctx, alpha, av, bv, beta, cv)
    first = Cc.read().copy()
    Cc.host[:] = c0
    Cc.upload()
    C.gemm(ctx, alpha, av, bv, beta, cv)
    assert np.array_equal(first.view(np.uint32), Cc.read().view(np.uint32))
    for i in range(batch):
        at = lambda lay: Layout(i * lay.strides[0], lay.shape[1:], lay.strides[1:])
        _gemm_fast_check(f"256x256 {m}x{n}x{k} tc={tc} bk={bk} batch {i}", first, A.host, at(la),
                         B.host, at(lb), c0, at(lc), m, n, k, alpha, beta)


@pytest.mark.parametrize("bk", [True, False])
def test_pipelined_256x256_tiles_offset_padded_views(ctx, pool, bk):
    """The 256x256 tiles read and write through view offsets and padded row pitches (each a
    multiple of four elements, so 128-bit loads stay aligned): A at offset 8 with rows of
    K + 4, B (transposed, or row-major) at offset 4 with a pitch of 4 more, C at offset 12 with
    rows of N + 8, alpha != 1 and beta != 0; every element against crates/cpu, the padding
    left untouched."""
    m, n, k = 4096, 4096, 256
    la = Layout(8, [m, k], [k + 4, 1])
    lb = Layout(4, [k, n], [1, k + 4]) if bk else Layout(4, [k, n], [n + 4, 1])
    lc = Layout(12, [m, n], [n + 8, 1])
    g = rng(7990 + bk)
    A, B, Cc = Tensor.random(pool, la, g), Tensor.random(pool, lb, g), Tensor.random(pool, lc, g)
    plan = C.plan_gemm(0.75, A.view(), B.view(), -0.5, Cc.view())
    assert (plan["kernel"], plan["tile"], plan["workgroups"], plan["b_mode"]) == \
        ("pipelined", (256, 256), 256, "k" if bk else "mn"), plan
    c0 = Cc.host.copy()
    C.gemm(ctx, 0.75, A.view(), B.view(), -0.5, Cc.view())
    got = Cc.read()
    written = (lc.offset + np.arange(m)[:, None] * lc.strides[0] + np.arange(n)[None, :]).ravel()
    assert_untouched("256x256 padded C", c0, got, written)
    _gemm_fast_check(f"256x256 offset views bk={bk}", got, A.host, la, B.host, lb, c0, lc, m, n, k,
                     0.75, -0.5)
