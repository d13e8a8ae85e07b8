"""f16 contraction on the GPU (the `_f16` entry points).

The reference rounds each f16 output once from a double-float sum of exact products
(shaders/contraction.metal:444-678). Two bars:
* exact-input cases -- halves on a 2^-10 grid, short alpha and beta -- where the exact result
  fits in 53 bits: the output must be the exact value rounded once to f16, bit for bit
  (oracle.contract_exact_f16, Python rationals), which is also the reference's result;
* random halves: the reference's own gate (tests/contraction_test.rs:280-313 with f16's
  U_OUT = 2^-11 and TINY = 2^-24) against the f64 reference.
Every element outside C keeps its bits.
"""
from __future__ import annotations

import numpy as np
import pytest

import linalg_hip as L
import oracle
from helpers import Layout, rng
from linalg_hip import contraction as C

pytestmark = pytest.mark.gpu

U_OUT = 2.0 ** -11
TINY = 2.0 ** -24
TAIL = 13


class Half:
    """A device buffer of f16 holding one view (plus spare elements) and its host image."""

    def __init__(self, pool, layout: Layout, data: np.ndarray):
        self.layout = layout
        self.cap = layout.span() + TAIL
        self.buffer = pool.alloc("f16", self.cap)
        self.host = np.zeros(self.buffer.nbytes // 2, dtype=np.float16)
        self.host[: min(data.size, self.host.size)] = data[: self.host.size]
        self.buffer.write(self.host)

    def view(self) -> L.TensorView:
        lay = self.layout
        return L.TensorView(self.buffer, lay.offset, lay.shape, lay.strides, "f16")

    def read(self) -> np.ndarray:
        return self.buffer.read(np.float16)

    def logical(self) -> np.ndarray:
        """The view's elements as a dense array."""
        lay = self.layout
        idx = np.full(lay.shape, lay.offset, dtype=np.int64)
        for d, (n, st) in enumerate(zip(lay.shape, lay.strides)):
            sh = [1] * len(lay.shape)
            sh[d] = n
            idx = idx + (np.arange(n) * st).reshape(sh)
        return self.host[idx]


def grid_halves(g, n):
    """Halves on the 2^-10 grid in [-2, 2): products are exact multiples of 2^-20."""
    return (g.integers(-2048, 2048, n).astype(np.float64) / 1024.0).astype(np.float16)


def random_halves(g, n):
    return g.uniform(-1.0, 1.0, n).astype(np.float16)


def f16_bits_equal(got, want_bits):
    got_bits = np.asarray(got, np.float16).view(np.uint16)
    zero = (got_bits & 0x7FFF) == 0
    return np.array_equal(np.where(zero, 0, got_bits), np.where((want_bits & 0x7FFF) == 0, 0, want_bits))


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (64, 64, 64), (100, 70, 37), (65, 129, 16),
                                   (130, 65, 300), (3, 200, 17)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (-0.5, 0.25), (2.0, 1.0), (0.75, -1.5)])
def test_exact_inputs_round_once_bit_for_bit(ctx, pool, m, n, k, alpha, beta):
    g = rng(m * 7 + n * 3 + k)
    a = Half(pool, Layout.dense([m, k]), grid_halves(g, m * k))
    b = Half(pool, Layout.dense([k, n]), grid_halves(g, k * n))
    c0 = grid_halves(g, m * n)
    if beta == 0.0:
        c0[:] = np.nan
    c = Half(pool, Layout.dense([m, n]), c0)
    before = c.read()
    C.gemm(ctx, alpha, a.view(), b.view(), beta, c.view())
    got = c.read()
    want = oracle.contract_exact_f16(alpha, a.logical(), b.logical(), beta,
                                     np.nan_to_num(c.logical()) if beta == 0 else c.logical())
    assert f16_bits_equal(got[: m * n].reshape(m, n), want)
    assert np.array_equal(got[m * n:].view(np.uint16), before[m * n:].view(np.uint16))


@pytest.mark.parametrize("at,bt", [(True, False), (False, True), (True, True)])
def test_transposed_operands_are_read_in_place(ctx, pool, at, bt):
    m, n, k = 70, 90, 45
    g = rng(5 + at + 2 * bt)
    la = Layout.transposed(m, k) if at else Layout.dense([m, k])
    lb = Layout.transposed(k, n) if bt else Layout.dense([k, n])
    a = Half(pool, la, grid_halves(g, la.span()))
    b = Half(pool, lb, grid_halves(g, lb.span()))
    c = Half(pool, Layout.dense([m, n]), np.zeros(m * n, np.float16))
    plan = C.plan_gemm(1.0, a.view(), b.view(), 0.0, c.view())
    assert plan["kind"] == "tiled"
    C.gemm(ctx, 1.0, a.view(), b.view(), 0.0, c.view())
    want = oracle.contract_exact_f16(1.0, a.logical(), b.logical(), 0.0, np.zeros((m, n), np.float16))
    assert f16_bits_equal(c.read()[: m * n].reshape(m, n), want)


def _mode_layout(operand, mode, rows, cols):
    """A [rows, cols] view of A (rows = M, cols = K) or B (rows = K, cols = N) whose plan
    takes `mode`: "k" or "mn" unit stride along that axis with 16-byte alignment, "strided"
    the same storage shifted by one element (misaligned for 128-bit loads)."""
    contiguous_cols = (operand == "a") == (mode != "mn")
    lay = Layout.dense([rows, cols]) if contiguous_cols else Layout.transposed(rows, cols)
    if mode == "strided":
        lay = Layout(1, lay.shape, lay.strides)
    return lay


@pytest.mark.parametrize("amode", ["k", "mn", "strided"])
@pytest.mark.parametrize("bmode", ["k", "mn", "strided"])
def test_every_load_mode_pair_rounds_once(ctx, pool, amode, bmode):
    """Each operand layout the tile kernel loads differently (128-bit loads along K, along M/N,
    or predicated 16-bit loads) on a ragged 72x136x40 product. Halves on the 2^-10 grid keep
    every partial sum exact in f64 (|sum| < 2^8 in steps of 2^-20), and alpha = -1/2,
    beta = 1/4 keep alpha*sum + beta*c exact, so numpy's correctly rounded f64 -> f16
    conversion of the f64 result is the exact value rounded once: bit for bit."""
    m, n, k = 72, 136, 40
    g = rng(11 + 3 * ["k", "mn", "strided"].index(amode) + ["k", "mn", "strided"].index(bmode))
    la, lb = _mode_layout("a", amode, m, k), _mode_layout("b", bmode, k, n)
    a = Half(pool, la, grid_halves(g, la.span()))
    b = Half(pool, lb, grid_halves(g, lb.span()))
    c = Half(pool, Layout.dense([m, n]), grid_halves(g, m * n))
    before = c.read()
    plan = C.plan_gemm(-0.5, a.view(), b.view(), 0.25, c.view())
    assert (plan["kind"], plan["a_mode"], plan["b_mode"]) == ("tiled", amode, bmode), plan
    C.gemm(ctx, -0.5, a.view(), b.view(), 0.25, c.view())
    exact = (-0.5 * (a.logical().astype(np.float64) @ b.logical().astype(np.float64))
             + 0.25 * c.logical().astype(np.float64))
    want = exact.astype(np.float16).view(np.uint16)
    got = c.read()
    assert f16_bits_equal(got[: m * n].reshape(m, n), want)
    assert np.array_equal(got[m * n:].view(np.uint16), before[m * n:].view(np.uint16))


def gate_check(name, got, exact, magnitude, k):
    rounded = exact.astype(np.float16).astype(np.float64)
    fin = np.isfinite(rounded)
    got = got.astype(np.float64)
    assert np.array_equal(np.isnan(got[~fin]), np.isnan(rounded[~fin])), name
    err = np.abs(got[fin] - rounded[fin])
    tol = (k + 2) * 2.0 ** -24 * magnitude[fin] + U_OUT * np.abs(rounded[fin]) + TINY
    assert np.all(err <= tol), f"{name}: worst {np.max(err / tol):.3f} of the gate"


@pytest.mark.parametrize("case", ["gemm", "batched_permuted_b", "general", "edges"])
def test_random_halves_pass_the_reference_gate(ctx, pool, case):
    g = rng(hash(case) % 1000)
    if case == "gemm":
        specs = [((Layout.dense([256, 512]), "mk"), (Layout.dense([512, 192]), "kn"),
                  (Layout.dense([256, 192]), "mn"), 1.0, 0.0)]
    elif case == "batched_permuted_b":
        # C3's shape at small size: B given as "bkj" storage viewed as "bkj" -> k unit stride.
        bs = Layout.dense([4, 96, 80])  # [b][j][k]
        bview = Layout(0, [4, 80, 96], [96 * 80, 1, 80])  # "bkj"
        specs = [((Layout.dense([4, 64, 80]), "bik"), (bview, "bkj"),
                  (Layout.dense([4, 64, 96]), "bij"), -1.25, 0.5)]
        del bs
    elif case == "general":
        specs = [((Layout.with_([5, 7, 6, 9], [2, 0, 3, 1], [1] * 4, 3), "ijkl"),
                  (Layout.with_([9, 6, 4, 11], [3, 0, 2, 1], [1, 2, 1, 1], 0), "lkmn"),
                  (Layout.with_([5, 4, 7, 11], [1, 3, 0, 2], [1, 1, 2, 1], 8), "imjn"), 0.5, -0.5)]
    else:
        specs = []
        for m in (1, 63, 64, 65, 127):
            for n in (1, 64, 65):
                for k in (1, 15, 16, 17, 33):
                    specs.append(((Layout.dense([m, k]), "mk"), (Layout.dense([k, n]), "kn"),
                                  (Layout.dense([m, n]), "mn"), 1.0, 0.5))
    for (la, sa), (lb, sb), (lc, sc), alpha, beta in specs:
        a = Half(pool, la, random_halves(g, la.span()))
        b = Half(pool, lb, random_halves(g, lb.span()))
        c = Half(pool, lc, random_halves(g, lc.span() + TAIL))
        before = c.read()
        a32, b32, c32 = (x.host.astype(np.float32) for x in (a, b, c))
        exp = oracle.contract_f64(alpha, a32, la.tup(), sa, b32, lb.tup(), sb, beta, c32, lc.tup(), sc)
        C.contract(ctx, alpha, (a.view(), sa), (b.view(), sb), beta, (c.view(), sc))
        got = c.read()
        gate_check(f"{case} {la.shape}x{lb.shape}", got[exp.index], exp.exact, exp.magnitude, exp.k)
        mask = np.ones(got.size, bool)
        mask[exp.index] = False
        assert np.array_equal(got[mask].view(np.uint16), before[mask].view(np.uint16))


def test_scale_zero_and_nan_rules(ctx, pool):
    from fractions import Fraction
    # beta*C alone is the exact product rounded once: the reference's 0x0DDC example.
    cvals = np.array([np.uint16(0x0DDC).view(np.float16), 1.0, -3.5, 65504.0, 6e-8], np.float16)
    c = Half(pool, Layout.dense([1, 5]), cvals)
    a = Half(pool, Layout.dense([1, 0]), np.zeros(0, np.float16))
    b = Half(pool, Layout.dense([0, 5]), np.zeros(0, np.float16))
    beta = np.float32(-0.999)
    assert C.plan_gemm(1.0, a.view(), b.view(), float(beta), c.view())["kind"] == "scale"
    C.gemm(ctx, 1.0, a.view(), b.view(), float(beta), c.view())
    got = c.read()[:5].view(np.uint16)
    want = [oracle.f16_round_exact(Fraction(float(beta)) * Fraction(float(v))) for v in cvals]
    assert got.tolist() == want and got[0] == 0x8DDB
    # beta = 0 never reads C (NaN cannot survive); alpha = 0 never reads A or B.
    g = rng(3)
    a = Half(pool, Layout.dense([8, 8]), np.full(64, np.nan, np.float16))
    b = Half(pool, Layout.dense([8, 8]), np.full(64, np.nan, np.float16))
    c = Half(pool, Layout.dense([8, 8]), np.full(64, np.nan, np.float16))
    C.gemm(ctx, 0.0, a.view(), b.view(), 0.0, c.view())
    assert not c.read()[:64].view(np.uint16).any()
    a = Half(pool, Layout.dense([8, 8]), grid_halves(g, 64))
    b = Half(pool, Layout.dense([8, 8]), grid_halves(g, 64))
    C.gemm(ctx, 1.0, a.view(), b.view(), 0.0, c.view())  # C holds zeros, beta = 0
    want = oracle.contract_exact_f16(1.0, a.logical(), b.logical(), 0.0, np.zeros((8, 8), np.float16))
    assert f16_bits_equal(c.read()[:64].reshape(8, 8), want)


def test_overflow_and_specials(ctx, pool):
    a = Half(pool, Layout.dense([2, 2]), np.array([60000, 60000, np.inf, 1], np.float16))
    b = Half(pool, Layout.dense([2, 2]), np.array([2, 0, 1, 1], np.float16))
    c = Half(pool, Layout.dense([2, 2]), np.zeros(4, np.float16))
    C.gemm(ctx, 1.0, a.view(), b.view(), 0.0, c.view())
    got = c.read()[:4].astype(np.float64)
    # Row 0: 60000*2 + 60000*1 overflows to +inf; 60000*0 + 60000*1 = 60000 (exact in f16? no:
    # 60000 rounds to 60000 exactly as it is an f16). Row 1: inf*2 + 1 = inf; inf*0 + 1 = NaN.
    assert got[0] == np.inf and got[1] == 60000.0 and got[2] == np.inf and np.isnan(got[3])


def test_repeated_f16_gemm_is_bitwise_stable(ctx, pool):
    g = rng(4)
    a = Half(pool, Layout.dense([200, 300]), random_halves(g, 60000))
    b = Half(pool, Layout.dense([300, 150]), random_halves(g, 45000))
    outs = []
    for _ in range(3):
        c = Half(pool, Layout.dense([200, 150]), np.zeros(30000, np.float16))
        C.gemm(ctx, 1.0, a.view(), b.view(), 0.0, c.view())
        outs.append(c.read().view(np.uint16).copy())
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1], outs[2])


def test_gemm_nowait_f16_is_ordered_before_a_download(ctx, pool):
    """gemm_nowait (src/ops/contraction.rs:1116-1130) enqueues on the context stream and
    returns; a download, ordered after it on that stream, sees the exact result. A second
    gemm_nowait reading the first one's output, with no wait between them, sees it too."""
    g = rng(41)
    m, n, k = 96, 80, 64
    a = Half(pool, Layout.dense([m, k]), grid_halves(g, m * k))
    b = Half(pool, Layout.dense([k, n]), grid_halves(g, k * n))
    c = Half(pool, Layout.dense([m, n]), np.full(m * n, np.nan, np.float16))
    sq = Half(pool, Layout.dense([n, n]), grid_halves(g, n * n))
    d = Half(pool, Layout.dense([m, n]), np.full(m * n, np.nan, np.float16))
    C.gemm_nowait(ctx, 0.5, a.view(), b.view(), 0.0, c.view())
    C.gemm_nowait(ctx, 1.0, c.view(), sq.view(), 0.0, d.view())
    got_c, got_d = c.read(), d.read()
    want_c = oracle.contract_exact_f16(0.5, a.logical(), b.logical(), 0.0, np.zeros((m, n)))
    assert f16_bits_equal(got_c[: m * n].reshape(m, n), want_c)
    c_exact = got_c[: m * n].reshape(m, n)
    want_d = oracle.contract_exact_f16(1.0, c_exact, sq.logical(), 0.0, np.zeros((m, n)))
    assert f16_bits_equal(got_d[: m * n].reshape(m, n), want_d)


def test_square_2048_exact_inputs_round_once_bit_for_bit(ctx, pool):
    """The reference's f16 benchmark shape (tests/contraction_test.rs:1345-1352) at full size on
    halves of the 2^-10 grid: every partial sum is a multiple of 2^-20 below 2^13 in magnitude,
    so an f64 matmul in any order is exact, and each output must be that value rounded once to
    f16 (round to nearest even)."""
    n = 2048
    g = rng(2048)
    x = grid_halves(g, n * n)
    y = grid_halves(g, n * n)
    a = Half(pool, Layout.dense([n, n]), x)
    b = Half(pool, Layout.dense([n, n]), y)
    c = Half(pool, Layout.dense([n, n]), np.full(n * n, np.nan, np.float16))
    C.gemm(ctx, 1.0, a.view(), b.view(), 0.0, c.view())
    exact = x.astype(np.float64).reshape(n, n) @ y.astype(np.float64).reshape(n, n)
    want = exact.astype(np.float16).view(np.uint16)
    assert f16_bits_equal(c.read()[: n * n].reshape(n, n), want)
