"""Contraction parity on the GPU for the paths that serve small and skinny outputs.

* one 32x32 tile per wave (batches of small products),
* sixteen waves per 32x32 tile with the K range split over workgroups (small outputs with
  long K), partials added in a fixed order,
* dot products on the VALU (M = N = 1), split along K, the partials added in order by a
  second launch,
* C stored contiguous along M, computed as C^T = B^T.A^T (alpha still scales A's elements),
* K <= 8 on the VALU in the reference's own order, bit for bit against crates/cpu.

Small cases run through helpers.Case (the f64 reference of tests/contraction_test.rs:200-268
with its gate, the crates/cpu restatement with the north-star bound for 2-D gemm, and every
element outside C bit-untouched). The shapes of the reference's own benchmark,
tests/contraction_test.rs:1293-1395 (bench_other_paths), run at full size with every output
checked, and the split paths three times with bitwise equal results.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from helpers import Case, Layout, Tensor, rng
from linalg_hip import contraction as C

pytestmark = pytest.mark.gpu


def dense(shape):
    return Layout.dense(shape)


def plan_of(case: Case, pool):
    views = [Tensor(pool, lay) for lay, _ in (case.a, case.b, case.c)]
    return C.plan_contract(case.alpha, (views[0].view(), case.a[1]), (views[1].view(), case.b[1]),
                           case.beta, (views[2].view(), case.c[1]))


# --------------------------------------------------------------------------------------
# one tile per wave
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("bsz,m,n,k", [(1024, 32, 32, 32), (1100, 17, 31, 9), (1030, 33, 20, 45),
                                       (600, 40, 50, 12), (2048, 8, 8, 100)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (-1.25, 0.5)])
def test_batched_small_products_one_tile_per_wave(ctx, pool, bsz, m, n, k, alpha, beta):
    case = Case(f"batched {bsz}x{m}x{n}x{k}", (dense([bsz, m, k]), "bmk"), (dense([bsz, k, n]), "bkn"),
                (dense([bsz, m, n]), "bmn")).scalars(alpha, beta)
    p = plan_of(case, pool)
    assert (p["kind"], p["kernel"], p["tile"]) == ("tiled", "wave", (32, 32)), p
    case.run(ctx, pool, bsz + m + n + k)


def test_wave_kernel_strided_and_transposed_operands(ctx, pool):
    bsz, m, n, k = 1024, 24, 28, 20
    for mask in range(8):
        ta, tb, tc = bool(mask & 1), bool(mask & 2), bool(mask & 4)
        lay = lambda t, r, c: (Layout.with_([bsz, r, c], [0, 2, 1], [1, 1, 1], 0) if t
                               else dense([bsz, r, c]))
        case = Case(f"wave a={ta} b={tb} c={tc}", (lay(ta, m, k), "bmk"), (lay(tb, k, n), "bkn"),
                    (lay(tc, m, n), "bmn")).scalars(0.75, -0.5 if mask % 2 else 0.0)
        p = plan_of(case, pool)
        assert p["kernel"] == "wave" and p["swapped"] == tc, (mask, p)
        case.run(ctx, pool, 9000 + mask)
    # Odd strides: predicated 32-bit loads.
    case = Case("wave strided", (Layout.with_([bsz, m, k], [0, 1, 2], [1, 2, 3], 5), "bmk"),
                (Layout.with_([bsz, k, n], [0, 1, 2], [1, 3, 1], 7), "bkn"),
                (Layout.with_([bsz, m, n], [0, 1, 2], [1, 1, 2], 3), "bmn")).scalars(1.5, 0.25)
    p = plan_of(case, pool)
    assert p["kernel"] == "wave" and (p["a_mode"], p["b_mode"]) == ("strided", "strided"), p
    case.run(ctx, pool, 9100)


# --------------------------------------------------------------------------------------
# sixteen waves per tile, split along K
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("m,n,k", [(32, 32, 20000), (5, 70, 33333), (64, 16, 4096), (1, 40, 9000),
                                   (100, 3, 7777)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.5, -1.5)])
def test_small_outputs_with_long_k_split_over_workgroups(ctx, pool, m, n, k, alpha, beta):
    case = Case.matmul(m, n, k).scalars(alpha, beta)
    p = plan_of(case, pool)
    assert (p["kind"], p["kernel"], p["tile"]) == ("split", "small", (32, 32)), p
    case.run(ctx, pool, m * 7 + n + k)


def test_small_split_is_bitwise_deterministic_and_transposed_c(ctx, pool):
    m, n, k = 40, 24, 50000
    g = rng(31)
    a = Tensor(pool, dense([m, k]), g.uniform(-1, 1, m * k).astype(np.float32))
    b = Tensor(pool, Layout.transposed(k, n), g.uniform(-1, 1, k * n).astype(np.float32))
    outs = []
    for _ in range(3):
        c = Tensor(pool, Layout.transposed(m, n))
        C.gemm(ctx, 1.0, a.view(), b.view(), 0.0, c.view())
        outs.append(c.read()[: m * n].copy())
    assert all(np.array_equal(outs[0].view(np.uint32), o.view(np.uint32)) for o in outs[1:])
    # Against the oracles at K = 20000: at K = 50000 the sequential f32 sum of crates/cpu is
    # itself ~1.6e-3 from the exact value on these uniform inputs, above the north-star bound
    # (1.1e-3 at alpha = -0.5), whatever the GPU computes.
    k = 20000
    Case("small split, C column-major", (dense([m, k]), "mk"), (Layout.transposed(k, n), "kn"),
         (Layout.transposed(m, n), "mn"), via_gemm=True).scalars(-0.5, 2.0).run(ctx, pool, 32)


# --------------------------------------------------------------------------------------
# one-wave 32x32 direct-load tiles, split along long K
# --------------------------------------------------------------------------------------
def _matrix(rows, cols, cm):
    return Layout.transposed(rows, cols) if cm else dense([rows, cols])


@pytest.mark.parametrize("a_cm,b_cm,c_cm", [(False, True, False), (False, False, False),
                                            (True, False, False), (True, True, True),
                                            (False, False, True)])
def test_skinny_direct_load_tiles(ctx, pool, a_cm, b_cm, c_cm):
    """Three whole 32x32 tiles with K = 70012: 244 splits of 288 (the last 28 deep, through the
    register path), every pair of operand layouts (K- or M/N-contiguous, so both [row][k] and
    the 32-row [k][row] stage layouts), C row- or column-major (the swapped roles). Checked
    against the exact f64 product under the north-star bound and against the reference's gate,
    and bitwise equal over two runs."""
    m, n, k = 32, 96, 70012
    alpha, beta = 1.25, -0.5
    g = rng(700 + 4 * a_cm + 2 * b_cm + c_cm)
    x = g.uniform(-1, 1, m * k).astype(np.float32)
    y = g.uniform(-1, 1, k * n).astype(np.float32)
    c0 = g.uniform(-1, 1, m * n).astype(np.float32)
    la, lb, lc = _matrix(m, k, a_cm), _matrix(k, n, b_cm), _matrix(m, n, c_cm)
    a, b = Tensor(pool, la, x), Tensor(pool, lb, y)
    p = C.plan_gemm(alpha, a.view(), b.view(), beta, Tensor(pool, lc).view())
    assert (p["kind"], p["kernel"], p["tile"], p["splits"], p["k_chunk"]) == \
        ("split", "direct", (32, 32), 244, 288), p
    assert p["swapped"] == c_cm
    outs = []
    for _ in range(2):
        c = Tensor(pool, lc, c0)
        C.gemm(ctx, alpha, a.view(), b.view(), beta, c.view())
        outs.append(c.read()[: m * n].copy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    # Logical matrices from the stored words.
    A = (x.reshape(k, m).T if a_cm else x.reshape(m, k)).astype(np.float64)
    B = (y.reshape(n, k).T if b_cm else y.reshape(k, n)).astype(np.float64)
    C0 = (c0.reshape(n, m).T if c_cm else c0.reshape(m, n)).astype(np.float64)
    got = outs[0].reshape(n, m).T if c_cm else outs[0].reshape(m, n)
    exact = alpha * (A @ B) + beta * C0
    _gate_north_star("skinny direct vs exact", got.ravel(), exact.ravel(), k, alpha, 1.0)
    e = oracle.contract_f64(alpha, x, (0, la.shape, la.strides), "mk", y, (0, lb.shape, lb.strides),
                            "kn", beta, c0.copy(), (0, lc.shape, lc.strides), "mn")
    oracle.gate(outs[0], e, "skinny direct")


def test_skinny_direct_load_batched_with_permuted_b(ctx, pool):
    """Three batches of 32x32 with K = 40000 and B a permuted view ("bnk" storage read as
    bkn): 139 splits per batch, 417 workgroups."""
    bsz, m, n, k = 3, 32, 32, 40000
    case = Case("skinny batched", (dense([bsz, m, k]), "bmk"),
                (Layout.with_([bsz, k, n], [0, 2, 1], [1, 1, 1], 0), "bkn"),
                (dense([bsz, m, n]), "bmn")).scalars(0.5, 0.0)
    p = plan_of(case, pool)
    assert (p["kind"], p["kernel"], p["tile"], p["splits"]) == ("split", "direct", (32, 32), 139), p
    case.run(ctx, pool, 4242)


# --------------------------------------------------------------------------------------
# dot products
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("k", [1, 3, 4, 1000, 1023, 8192, 8195, 100000, 262147])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (-0.75, 0.5)])
def test_dot_products(ctx, pool, k, alpha, beta):
    case = Case.matmul(1, 1, k).scalars(alpha, beta)
    p = plan_of(case, pool)
    assert p["kind"] == "dot", p
    case.run(ctx, pool, k + 11)


def test_dot_batched_offset_and_strided(ctx, pool):
    # A batch of dots with a padded batch stride (128-bit loads), then unit-less strides along K
    # (32-bit loads), and an offset that breaks 16-byte alignment.
    cases = [
        Case("batched dots", (Layout(0, [7, 1, 30001], [30004, 30004, 1]), "bmk"),
             (Layout(0, [7, 30001, 1], [30004, 1, 1]), "bkn"), (dense([7, 1, 1]), "bmn")),
        Case("strided dot", (Layout.with_([1, 20000], [0, 1], [1, 3], 2), "mk"),
             (Layout.with_([20000, 1], [0, 1], [2, 1], 1), "kn"), (dense([1, 1]), "mn"),
             via_gemm=True),
        Case("misaligned dot", (Layout.with_([1, 50000], [0, 1], [1, 1], 1), "mk"),
             (dense([50000, 1]), "kn"), (dense([1, 1]), "mn"), via_gemm=True),
        Case("many dots", (dense([5000, 1, 64]), "bmk"), (dense([5000, 64, 1]), "bkn"),
             (dense([5000, 1, 1]), "bmn")),
    ]
    for i, case in enumerate(cases):
        p = plan_of(case, pool)
        assert p["kind"] == "dot", (case.name, p)
        case.scalars(1.25, -0.5).run(ctx, pool, 300 + i)


def test_dot_split_partials_stay_consistent_across_calls(ctx, pool):
    """The split dot's partials share the context's buffer: a run of calls of different split
    counts and batches gives each one's own bits, also when repeated."""
    shapes = [(1, 1 << 20), (3, 200000), (1, 70000), (2, 1 << 19)]
    outs = {}
    for rep in range(2):
        for bsz, k in shapes:
            a = Tensor(pool, dense([bsz, 1, k]), rng(bsz * k).uniform(-1, 1, bsz * k).astype(np.float32))
            b = Tensor(pool, dense([bsz, k, 1]), rng(bsz + k).uniform(-1, 1, bsz * k).astype(np.float32))
            c = Tensor(pool, dense([bsz, 1, 1]))
            C.contract(ctx, 1.0, (a.view(), "bmk"), (b.view(), "bkn"), 0.0, (c.view(), "bmn"))
            got = c.read()[:bsz].copy()
            if rep == 0:
                outs[(bsz, k)] = got
                ref = [np.dot(a.host[i * k:(i + 1) * k].astype(np.float64),
                              b.host[i * k:(i + 1) * k].astype(np.float64)) for i in range(bsz)]
                assert np.max(np.abs(got - np.array(ref))) <= 1e-5 * np.sqrt(k), (bsz, k)
            else:
                assert np.array_equal(got.view(np.uint32), outs[(bsz, k)].view(np.uint32)), (bsz, k)


# --------------------------------------------------------------------------------------
# K <= 8: the VALU in crates/cpu's own order, bit for bit
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("k", [1, 2, 5, 8])
@pytest.mark.parametrize("m,n", [(1, 7), (33, 64), (130, 257), (4, 1000)])
@pytest.mark.parametrize("layout", ["rm", "c_cm", "b_strided"])
def test_low_rank_updates_equal_crates_cpu_bit_for_bit(ctx, pool, k, m, n, layout):
    """acc = beta == 0 ? +0 : beta*C, then acc += (alpha*a)*b in k order: the reference's loop
    (crates/cpu/src/lib.rs:664-691), so every output equals oracle.gemm_seq's bits."""
    g = rng(k * 1000 + m + n)
    la = Layout.dense([m, k])
    lb = Layout.with_([k, n], [0, 1], [1, 3], 1) if layout == "b_strided" else Layout.dense([k, n])
    lc = Layout.transposed(m, n) if layout == "c_cm" else Layout.dense([m, n])
    for alpha, beta in [(1.0, 0.0), (-1.5, 0.75), (0.3, 1.0)]:
        a, b, c = (Tensor.random(pool, lay, g) for lay in (la, lb, lc))
        if beta == 0.0:
            c.host[:] = np.nan
            c.upload()
        a0, b0, c0 = a.host.copy(), b.host.copy(), c.host.copy()
        plan = C.plan_gemm(alpha, a.view(), b.view(), beta, c.view())
        assert (plan["kind"], plan["kernel"]) == ("tiled", "outer"), plan
        C.gemm(ctx, alpha, a.view(), b.view(), beta, c.view())
        ref = c0.copy()
        oracle.gemm_seq(m, n, k, alpha, beta, a0, la.offset, la.strides, b0, lb.offset, lb.strides,
                        ref, lc.offset, lc.strides)
        got = c.read()
        assert np.array_equal(got[: ref.size].view(np.uint32), ref.view(np.uint32)), (k, m, n, layout,
                                                                                     alpha, beta)


# --------------------------------------------------------------------------------------
# C contiguous along M
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("m,n,k", [(300, 200, 100), (512, 512, 512), (256, 256, 20000),
                                   (2000, 130, 64)])
def test_c_column_major_is_computed_transposed(ctx, pool, m, n, k):
    for j, (alpha, beta) in enumerate([(1.0, 0.0), (-1.5, 0.75)]):
        case = Case(f"C column-major {m}x{n}x{k}", (dense([m, k]), "mk"), (dense([k, n]), "kn"),
                    (Layout.transposed(m, n), "mn"), via_gemm=True).scalars(alpha, beta)
        assert plan_of(case, pool)["swapped"]
        case.run(ctx, pool, m + n + k + j)


def test_association_known_answer_with_swapped_operands(ctx, pool):
    """crates/cpu/src/invariants.rs:182-187: (alpha*a)*b, not alpha*(a*b). With C column-major the
    caller's A is the kernel's B-role operand; alpha must still scale A's element."""
    a = Tensor(pool, dense([2, 1]), np.array([1e20, 1e20], np.float32))
    b = Tensor(pool, dense([1, 2]), np.array([1e-20, 1e-20], np.float32))
    c = Tensor(pool, Layout.transposed(2, 2))
    C.gemm(ctx, 1e-20, a.view(), b.view(), 0.0, c.view())
    want = np.float32(np.float32(np.float32(1e-20) * np.float32(1e20)) * np.float32(1e-20))
    assert plan_of(Case("kat", (dense([2, 1]), "mk"), (dense([1, 2]), "kn"),
                        (Layout.transposed(2, 2), "mn")), pool)["swapped"]
    assert np.array_equal(c.read()[:4].view(np.uint32), np.full(4, want).view(np.uint32))


# --------------------------------------------------------------------------------------
# the reference's benchmark shapes at full size (tests/contraction_test.rs:1293-1395)
# --------------------------------------------------------------------------------------
def _gate_north_star(name, got, ref, k, amax, bmax):
    tol = 1e-5 * np.sqrt(k) * amax * bmax
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    worst = int(np.argmax(err))
    assert np.all(np.isfinite(got)) and err[worst] <= tol, f"{name}: {err[worst]:e} > {tol:e} at {worst}"


def test_bench_transposed_2048(ctx, pool):
    n = 2048
    g = rng(42)
    x = g.uniform(-1, 1, n * n).astype(np.float32)
    y = g.uniform(-1, 1, n * n).astype(np.float32)
    a = Tensor(pool, Layout.transposed(n, n), x)
    b = Tensor(pool, Layout.transposed(n, n), y)
    c = Tensor(pool, Layout.transposed(n, n))
    C.contract(ctx, 1.0, (a.view(), "mk"), (b.view(), "kn"), 0.0, (c.view(), "mn"))
    got = c.read()[: n * n]
    ref = np.zeros(n * n, np.float32)
    oracle.gemm_fast(n, n, n, 1.0, 0.0, x, 0, (1, n), y, 0, (1, n), ref, 0, (1, n))
    _gate_north_star("transposed 2048", got, ref, n, 1.0, 1.0)


def test_bench_batched_4096_x_32_cubed(ctx, pool):
    case = Case("batched 4096 x 32^3", (dense([4096, 32, 32]), "bmk"), (dense([4096, 32, 32]), "bkn"),
                (dense([4096, 32, 32]), "bmn"))
    assert plan_of(case, pool)["kernel"] == "wave"
    case.run(ctx, pool, 42)


def test_bench_dot_16m_oracle_and_determinism(ctx, pool):
    k = 1 << 24
    g = rng(42)
    x = g.uniform(-1, 1, k).astype(np.float32)
    y = g.uniform(-1, 1, k).astype(np.float32)
    a = Tensor(pool, dense([1, k]), x)
    b = Tensor(pool, dense([k, 1]), y)
    outs = []
    for _ in range(3):
        c = Tensor(pool, dense([1, 1]), np.array([np.nan], np.float32))
        C.contract(ctx, 1.0, (a.view(), "mk"), (b.view(), "kn"), 0.0, (c.view(), "mn"))
        outs.append(c.read()[:1].copy())
    assert all(np.array_equal(outs[0].view(np.uint32), o.view(np.uint32)) for o in outs[1:])
    # The f64 reference with the reference's gate, and the north-star bound against the exact
    # value: at K = 2^24 on uniform inputs the k-order f32 sum of crates/cpu is itself ~0.15 from
    # the exact value, 3.7 times the bound (0.041), so it cannot serve as the comparand; it must
    # still pass the reference's gate, as the GPU result must.
    e = oracle.contract_f64(1.0, x, (0, [1, k], [k, 1]), "mk", y, (0, [k, 1], [1, 1]), "kn", 0.0,
                            np.zeros(1, np.float32), (0, [1, 1], [1, 1]), "mn")
    oracle.gate(outs[0], e, "dot 16M")
    exact = np.array([np.dot(x.astype(np.float64), y.astype(np.float64))])
    _gate_north_star("dot 16M vs exact", outs[0], exact, k, 1.0, 1.0)
    seq = np.zeros(1, np.float32)
    oracle.gemm_seq(1, 1, k, 1.0, 0.0, x, 0, (k, 1), y, 0, (1, 1), seq, 0, (1, 1))
    oracle.gate(seq, e, "dot 16M, crates/cpu")


def test_bench_32x32_k_1m_oracle_and_determinism(ctx, pool):
    m = n = 32
    k = 1 << 20
    g = rng(43)
    x = g.uniform(-1, 1, m * k).astype(np.float32)
    y = g.uniform(-1, 1, k * n).astype(np.float32)  # B column-major: y[j*k + kk] = B[kk][j]
    a = Tensor(pool, dense([m, k]), x)
    b = Tensor(pool, Layout.transposed(k, n), y)
    outs = []
    for _ in range(3):
        c = Tensor(pool, dense([m, n]))
        C.contract(ctx, 1.0, (a.view(), "mk"), (b.view(), "kn"), 0.0, (c.view(), "mn"))
        outs.append(c.read()[: m * n].copy())
    assert all(np.array_equal(outs[0].view(np.uint32), o.view(np.uint32)) for o in outs[1:])
    # As for the dot: at K = 2^20 the k-order f32 sums of crates/cpu are ~0.02 from the exact
    # values, twice the north-star bound, so the bound is taken against the exact (f64) product,
    # and the reference's gate against its f64 reference.
    e = oracle.contract_f64(1.0, x, (0, [m, k], [k, 1]), "mk", y, (0, [k, n], [1, k]), "kn", 0.0,
                            np.zeros(m * n, np.float32), (0, [m, n], [n, 1]), "mn")
    oracle.gate(outs[0], e, "32x32 K=1M")
    exact = (x.reshape(m, k).astype(np.float64) @ y.reshape(n, k).T.astype(np.float64)).ravel()
    _gate_north_star("32x32 K=1M vs exact", outs[0], exact, k, 1.0, 1.0)


def test_bench_rank1_4096(ctx, pool):
    n = 4096
    g = rng(44)
    x = g.uniform(-1, 1, n).astype(np.float32)
    y = g.uniform(-1, 1, n).astype(np.float32)
    a = Tensor(pool, dense([n, 1]), x)
    b = Tensor(pool, dense([1, n]), y)
    c = Tensor(pool, dense([n, n]))
    C.contract(ctx, 1.0, (a.view(), "mk"), (b.view(), "kn"), 0.0, (c.view(), "mn"))
    got = c.read()[: n * n]
    # K = 1 runs crates/cpu's loop: +0 + (alpha*a)*b, exactly the f32 product (+0 for a zero
    # product of either sign).
    want = np.float32(0.0) + np.outer(x, y).astype(np.float32).ravel()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_bench_rank4_48_pow6(ctx, pool):
    e = 48
    g = rng(45)
    x = g.uniform(-1, 1, e ** 4).astype(np.float32)
    y = g.uniform(-1, 1, e ** 4).astype(np.float32)
    a = Tensor(pool, dense([e] * 4), x)
    b = Tensor(pool, dense([e] * 4), y)
    c = Tensor(pool, dense([e] * 4))
    C.contract(ctx, 1.0, (a.view(), "ijkl"), (b.view(), "klmn"), 0.0, (c.view(), "ijmn"))
    got = c.read()[: e ** 4]
    # ij, kl and mn each merge to one 2304-long axis: a dense 2304^3 product.
    n = e * e
    ref = np.zeros(n * n, np.float32)
    oracle.gemm_fast(n, n, n, 1.0, 0.0, x, 0, (n, 1), y, 0, (n, 1), ref, 0, (n, 1))
    _gate_north_star("rank-4 48^6", got, ref, n, 1.0, 1.0)
