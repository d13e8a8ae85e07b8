"""lg_backend_gemm on the GPU: the Backend::gemm contract through the C ABI.

Restates crates/cpu/src/invariants.rs:133-308 and crates/cuda/src/invariants.rs:133-284 for
the HIP backend. Where the reference's known answers are exact in f32 (small integer data,
single products, fills), the device must return the same bits: every product is formed as
(alpha*a)*b, exactly as in the reference's loop. Where the summation order matters, results
are gated against the f64 reference and the crates/cpu restatement with the north-star
bound. The general kernel (the path for non-finite alpha and unmergeable axes) runs the
reference's loop itself and must match the oracle bit for bit. On F16 / BF16 tensors every
output must have the bits of the oracle's restatement of CpuBackend's f32 loop (NaN for NaN).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from helpers import Layout, Tensor, rng
from linalg_hip import backend as B
from linalg_hip import contraction as C

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hb():
    backend = B.HipBackend(0)
    assert backend.kind() == "Hip"
    yield backend
    backend.close()


def f32(values) -> np.ndarray:
    return np.asarray(values, dtype=np.float32)


def bits(x) -> np.ndarray:
    return f32(x).view(np.uint32)


def transposed(hb, rows, cols, logical) -> B.Tensor:
    """Upload the row-major [cols, rows] transpose and view it back as [rows, cols]."""
    physical = f32(logical).reshape(rows, cols).T.copy()
    t = B.transpose_matrix(hb.upload_f32([cols, rows], physical.ravel()))
    assert t.shape == [rows, cols] and t.strides == [1, rows] and t.offset == 0
    return t


def sequential(m, n, k, a, b, c, alpha, beta) -> np.ndarray:
    """crates/cpu accumulation (the oracle's restatement) on dense row-major data."""
    out = f32(c).copy()
    oracle.gemm_seq(m, n, k, alpha, beta, f32(a).copy(), 0, [k, 1], f32(b).copy(), 0, [n, 1],
                    out, 0, [n, 1])
    return out


def gemm_layouts(hb, a, b, c0, m, k, n, alpha, beta, check):
    """Runs the three supported layouts (invariants.rs:99-131) and hands each result to
    `check`."""
    layouts = [
        (hb.upload_f32([m, k], a), hb.upload_f32([k, n], b)),
        (transposed(hb, m, k, a), hb.upload_f32([k, n], b)),
        (hb.upload_f32([m, k], a), transposed(hb, k, n, b)),
    ]
    for name, (ta, tb) in zip(["rm", "a^T", "b^T"], layouts):
        c = hb.upload_f32([m, n], c0)
        hb.gemm(ta, tb, c, alpha, beta)
        check(name, hb.download_f32(c))


def test_exact_known_answers_in_every_layout(hb):
    a, b = [1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0]

    def exact(expected):
        def check(name, got):
            assert np.array_equal(bits(got), bits(expected)), f"{name}: {got} != {expected}"
        return check

    expected = sequential(2, 2, 2, a, b, [0.0] * 4, 1.0, 0.0)
    assert expected.tolist() == [19.0, 22.0, 43.0, 50.0]
    gemm_layouts(hb, a, b, [0.0] * 4, 2, 2, 2, 1.0, 0.0, exact(expected))
    c0 = [1.0, -2.0, 0.5, 4.0]
    expected = sequential(2, 2, 2, a, b, c0, -0.5, 0.25)
    acc = np.float32(0.25) * np.float32(c0[0])
    acc += np.float32(-0.5) * np.float32(a[0]) * np.float32(b[0])
    acc += np.float32(-0.5) * np.float32(a[1]) * np.float32(b[2])
    assert bits(expected[0]) == bits(acc)
    gemm_layouts(hb, a, b, c0, 2, 2, 2, -0.5, 0.25, exact(expected))
    # alpha*A*B associates left: (1e20 * 1e-20) * 1e-20, not 1e20 * (1e-20 * 1e-20).
    alpha = np.float32(1e20)
    left = (alpha * np.float32(1e-20)) * np.float32(1e-20)
    right = alpha * (np.float32(1e-20) * np.float32(1e-20))
    assert bits(left) != bits(right)
    gemm_layouts(hb, [1e-20], [1e-20], [0.0], 1, 1, 1, float(alpha), 0.0, exact([left]))
    # beta*C + alpha*a*b with one product is one rounding of each step, in any order.
    gemm_layouts(hb, [3.0], [5.0], [1.5], 1, 1, 1, 4.0, 2.0,
                 exact([np.float32(2.0) * np.float32(1.5) + np.float32(4.0 * 3.0) * np.float32(5.0)]))


def test_cancellation_known_answer_is_one_of_the_two_orders(hb):
    # 2^25 has f32 ulp 4: k order loses the 1 (crates/cpu gives 0), any order that cancels
    # the large terms first keeps it. The backend's fixed order may be either; nothing else.
    big = 33554432.0
    expected = sequential(1, 1, 3, [big, 1.0, -big], [1.0, 1.0, 1.0], [0.0], 1.0, 0.0)
    assert bits(expected) == bits([0.0])

    def check(name, got):
        assert got[0] in (0.0, 1.0), f"{name}: {got[0]}"
        assert abs(got[0] - expected[0]) <= oracle.north_star_tol(3, f32([big]), f32([1.0]))
    gemm_layouts(hb, [big, 1.0, -big], [1.0, 1.0, 1.0], [0.0], 1, 3, 1, 1.0, 0.0, check)


def test_beta_zero_ignores_nan_in_c_and_alpha_zero_ignores_nan_operands(hb):
    nan = np.uint32(0x7FC01234).view(np.float32)
    c = hb.upload_f32([1, 1], [nan])
    hb.gemm(hb.upload_f32([1, 2], [2.0, 3.0]), hb.upload_f32([2, 1], [4.0, 5.0]), c, 1.0, 0.0)
    assert bits(hb.download_f32(c)) == bits([23.0])
    snan = np.uint32(0x7F800011).view(np.float32)
    c = hb.upload_f32([1, 2], [3.0, -4.0])
    hb.gemm(hb.upload_f32([1, 2], [nan, snan]), hb.upload_f32([2, 2], [nan] * 4), c, 0.0, 2.0)
    assert np.array_equal(bits(hb.download_f32(c)), bits([6.0, -8.0]))
    c = hb.upload_f32([2, 2], [nan] * 4)
    hb.gemm(hb.upload_f32([2, 2], [nan] * 4), hb.upload_f32([2, 2], [nan] * 4), c, 0.0, 0.0)
    assert np.array_equal(bits(hb.download_f32(c)), bits([0.0] * 4))
    # crates/cuda/src/invariants.rs:261-270.
    c = hb.upload_f32([2, 2], [np.nan] * 4)
    hb.gemm(hb.upload_f32([2, 2], [1.0, 0.0, 0.0, 1.0]), hb.upload_f32([2, 2], [2.0, 3.0, 4.0, 5.0]),
            c, 1.0, 0.0)
    assert hb.download_f32(c).tolist() == [2.0, 3.0, 4.0, 5.0]


def test_k_zero(hb):
    a, b = hb.alloc(B.DType.F32, [2, 0]), hb.alloc(B.DType.F32, [0, 3])
    assert a.storage.storage_id() != b.storage.storage_id()
    assert a.shape == [2, 0] and a.strides == B.row_major_strides([2, 0])
    assert hb.download(a) == b""
    nan = np.uint32(0x7FA000AB).view(np.float32)
    c = hb.upload_f32([2, 3], [nan] * 6)
    before = len(hb.debug_launches())
    hb.gemm(a, b, c, 1.5, 0.0)
    assert hb.download(c) == bytes(24)
    launches = hb.debug_launches()
    assert len(launches) == before + 1 and launches[-1] == "zero_f32"
    # K = 0 with a non-zero beta scales C and does not invent zeros.
    a, b = hb.alloc(B.DType.F32, [1, 0]), hb.alloc(B.DType.F32, [0, 2])
    c = hb.upload_f32([1, 2], [1.5, -3.0])
    hb.gemm(a, b, c, 4.0, 2.0)
    assert np.array_equal(bits(hb.download_f32(c)), bits([3.0, -6.0]))
    # crates/cuda/src/invariants.rs:273-282 (an empty upload).
    c = hb.upload_f32([3, 4], [1.0] * 12)
    hb.gemm(hb.upload_f32([3, 0], []), hb.upload_f32([0, 4], []), c, 1.0, 0.0)
    assert hb.download_f32(c).tolist() == [0.0] * 12


def test_empty_storage_ids_are_distinct(hb):
    a, b = hb.alloc(B.DType.F32, [0]), hb.alloc(B.DType.F32, [0])
    assert a.storage.storage_id() != 0 and b.storage.storage_id() != 0
    assert a.storage.storage_id() != b.storage.storage_id()


def test_errors_leave_c_unchanged_and_launch_nothing(hb):
    sentinel = [1.25, -2.5, 3.5, -4.5]
    c = hb.upload_f32([2, 2], sentinel)
    a = hb.upload_f32([2, 2], [1.0, 0.0, 0.0, 1.0])
    b = hb.upload_f32([2, 2], [9.0, 8.0, 7.0, 6.0])
    a_bad = hb.upload_f32([2, 2], [1.0, 2.0, 3.0, 4.0])
    a_bad.strides = [1, 1]
    shifted = hb.upload_f32([2, 2], [1.0, 2.0, 3.0, 4.0])
    shifted.offset = 1
    alias = B.Tensor(c.storage, B.DType.F32, [2, 2], [2, 1])
    shared = hb.upload_f32([2, 2], [4.0, 3.0, 2.0, 1.0])
    alias_ab = B.Tensor(shared.storage, B.DType.F32, [2, 2], [2, 1])
    cases = [
        (a_bad, b, c, "UnsupportedLayout"),
        (transposed(hb, 2, 2, [1.0, 2.0, 3.0, 4.0]), transposed(hb, 2, 2, [5.0, 6.0, 7.0, 8.0]),
         c, "UnsupportedLayout"),
        (a, b, B.transpose_matrix(c), "UnsupportedLayout"),
        (shifted, b, c, "UnsupportedLayout"),
        (alias, b, c, "Alias"),
        (a, alias, c, "Alias"),
        (shared, alias_ab, c, "Alias"),
        (a, a, c, "Alias"),
        (hb.upload(B.DType.F16, [2, 2], bytes(8)), b, c, "Dtype"),
    ]
    launches = hb.debug_launches()
    for ta, tb, tc, kind in cases:
        with pytest.raises(B.BackendError) as e:
            hb.gemm(ta, tb, tc, 1.0, 1.0)
        assert e.value.kind == kind
        assert np.array_equal(bits(hb.download_f32(c)), bits(sentinel))
    assert hb.debug_launches() == launches


def metal_fixture(rows, cols) -> np.ndarray:
    """crates/cuda/src/invariants.rs:31-40."""
    i, j = np.meshgrid(np.arange(rows), np.arange(cols), indexing="ij")
    return f32((((i * 17 + j * 3) % 100).astype(np.float32) / np.float32(100.0)) - np.float32(0.5)).ravel()


def test_fixture_gemm_against_f64_and_crates_cpu(hb):
    m = k = n = 32
    a, b, c0 = metal_fixture(m, k), metal_fixture(k, n), metal_fixture(m, n)
    ref64 = a.astype(np.float64).reshape(m, k) @ b.astype(np.float64).reshape(k, n)
    cpu = sequential(m, n, k, a, b, c0, 1.0, 0.0)
    tol = oracle.north_star_tol(k, a, b)

    def check(name, got):
        assert np.max(np.abs(got - ref64.ravel())) <= 1e-3, name  # the CUDA backend's bound
        assert np.max(np.abs(got.astype(np.float64) - cpu)) <= tol, name
    gemm_layouts(hb, a, b, c0, m, k, n, 1.0, 0.0, check)


def test_repeated_gemm_is_bitwise_stable_and_transposes_are_read_in_place(hb):
    for m, n, k in [(16, 16, 16), (96, 80, 24576)]:  # the second takes the split-K path
        g = rng(m + k)
        a = g.uniform(-1, 1, m * k).astype(np.float32)
        b = g.uniform(-1, 1, k * n).astype(np.float32)
        ta, tb = hb.upload_f32([m, k], a), transposed(hb, k, n, b)
        outs = []
        for _ in range(2):
            c = hb.upload_f32([m, n], np.zeros(m * n, np.float32))
            before = len(hb.debug_launches())
            hb.gemm(ta, tb, c, 1.0, 0.0)
            new = hb.debug_launches()[before:]
            # One MFMA launch (plus the ordered reduction when split): no packed copy.
            assert [x for x in new if not x.startswith("gemm_f32_")] in ([], ["reduce_f32"]), new
            assert sum(x.startswith("gemm_f32_") for x in new) == 1, new
            outs.append(hb.download(c))
        assert outs[0] == outs[1], f"{m}x{n}x{k}: repeated gemm must be bitwise stable"
        got = np.frombuffer(outs[0], np.float32).astype(np.float64)
        cpu = sequential(m, n, k, a, b, np.zeros(m * n), 1.0, 0.0)
        assert np.max(np.abs(got - cpu)) <= oracle.north_star_tol(k, a, b)


def test_pipeline_stage_linear_step(hb):
    """One 1F1B stage's linear layer through the backend: Y = X.W, dX = dY.W^T, dW = X^T.dY
    (the fifth benchmark configuration at reduced size; the operands are transpose_matrix
    views of the stored row-major tensors, read in place)."""
    mb, d, h = 256, 384, 640
    g = rng(5)
    x = (g.standard_normal(mb * d) * 0.02).astype(np.float32)
    w = (g.standard_normal(d * h) * 0.02).astype(np.float32)
    dy = (g.standard_normal(mb * h) * 0.02).astype(np.float32)
    tx, tw, tdy = hb.upload_f32([mb, d], x), hb.upload_f32([d, h], w), hb.upload_f32([mb, h], dy)
    ty, tdx, tdw = hb.alloc(B.DType.F32, [mb, h]), hb.alloc(B.DType.F32, [mb, d]), \
        hb.alloc(B.DType.F32, [d, h])
    hb.gemm(tx, tw, ty, 1.0, 0.0)
    hb.gemm(tdy, B.transpose_matrix(tw), tdx, 1.0, 0.0)
    hb.gemm(B.transpose_matrix(tx), tdy, tdw, 1.0, 0.0)
    X, W, DY = (v.reshape(s) for v, s in ((x, (mb, d)), (w, (d, h)), (dy, (mb, h))))
    for name, t, (m, n, k, am, bm) in [
        ("Y", ty, (mb, h, d, X, W)),
        ("dX", tdx, (mb, d, h, DY, W.T)),
        ("dW", tdw, (d, h, mb, X.T, DY)),
    ]:
        got = hb.download_f32(t).astype(np.float64)
        a64, b64 = np.ascontiguousarray(am), np.ascontiguousarray(bm)
        cpu = sequential(m, n, k, a64.ravel(), b64.ravel(), np.zeros(m * n), 1.0, 0.0)
        exact = a64.astype(np.float64) @ b64.astype(np.float64)
        tol = oracle.north_star_tol(k, a64, b64)
        assert np.max(np.abs(got - cpu)) <= tol, name
        mag = np.abs(a64.astype(np.float64)) @ np.abs(b64.astype(np.float64))
        gate = (k + 2) * 2.0 ** -24 * mag.ravel() + 2.0 ** -24 * np.abs(exact.ravel()) + 1.4e-45
        assert np.all(np.abs(got - exact.ravel()) <= gate), name


def test_general_kernel_is_the_sequential_loop_bit_for_bit(ctx, pool):
    # K split over two axes whose strides cannot merge in A: the general kernel, which walks
    # k in the same order as the reference's loop and must return identical bits.
    m, k1, k2, n = 37, 6, 7, 29
    g = rng(11)
    la = Layout(3, [m, k1, k2], [k1 * (k2 + 1), k2 + 1, 1])  # a padded row: x, y unmergeable
    lb = Layout.dense([k1, k2, n])
    lc = Layout.dense([m, n])
    for alpha, beta in [(1.0, 0.0), (-1.5, 0.75), (0.3, -2.0)]:
        a, b, c = Tensor.random(pool, la, g), Tensor.random(pool, lb, g), Tensor.random(pool, lc, g)
        plan = C.plan_contract(alpha, (a.view(), "mxy"), (b.view(), "xyn"), beta, (c.view(), "mn"))
        assert plan["kind"] == "general"
        c0 = c.host.copy()
        C.contract(ctx, alpha, (a.view(), "mxy"), (b.view(), "xyn"), beta, (c.view(), "mn"))
        got = c.read()[: m * n]
        idx = la.offset + (np.arange(m)[:, None, None] * la.strides[0]
                           + np.arange(k1)[None, :, None] * la.strides[1]
                           + np.arange(k2)[None, None, :] * la.strides[2])
        am = a.host[idx].reshape(m, k1 * k2).copy()
        ref = c0[: m * n].copy()
        oracle.gemm_seq(m, n, k1 * k2, alpha, beta, am, 0, [k1 * k2, 1], b.host[: k1 * k2 * n].copy(),
                        0, [n, 1], ref, 0, [n, 1])
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (alpha, beta)


def test_non_finite_alpha_matches_the_sequential_loop(ctx, pool):
    # Non-finite alpha takes the general kernel: inf/NaN appear exactly where the reference
    # loop puts them (zero padding of the tiled kernel would otherwise inject NaN).
    m, n, k = 40, 33, 20
    g = rng(12)
    la, lb, lc = Layout.dense([m, k]), Layout.dense([k, n]), Layout.dense([m, n])
    for alpha in (math.inf, -math.inf):
        a, b, c = Tensor.random(pool, la, g), Tensor.random(pool, lb, g), Tensor.random(pool, lc, g)
        a.host[5 * k: 6 * k] = 0.0  # row 5 of A is zero: inf*0 = NaN in every product
        a.upload()
        c0 = c.host.copy()
        C.gemm(ctx, alpha, a.view(), b.view(), 0.0, c.view())
        got = c.read()[: m * n]
        ref = c0[: m * n].copy()
        oracle.gemm_seq(m, n, k, alpha, 0.0, a.host[: m * k].copy(), 0, [k, 1],
                        b.host[: k * n].copy(), 0, [n, 1], ref, 0, [n, 1])
        assert np.array_equal(np.isnan(got), np.isnan(ref))
        fin = ~np.isnan(ref)
        assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))


# ---- Backend::gemm on F16 / BF16 tensors (crates/cpu/src/lib.rs:270-291) --------------------
from test_oracle import GEMM_16_KATS, GEMM_16_ORDER_KATS, to_16  # noqa: E402

DT16 = {"f16": B.DType.F16, "bf16": B.DType.BF16}


def up16(hb, kind, bits16, shape, transpose=False):
    """Upload uint16 bits as a [rows, cols] tensor; with `transpose`, as the transpose_matrix
    view of the row-major [cols, rows] storage."""
    bits16 = np.ascontiguousarray(np.asarray(bits16, np.uint16).reshape(shape))
    if not transpose:
        return hb.upload(DT16[kind], list(shape), bits16.tobytes())
    t = hb.upload(DT16[kind], [shape[1], shape[0]], np.ascontiguousarray(bits16.T).tobytes())
    return B.transpose_matrix(t)


def down16(hb, t) -> np.ndarray:
    return np.frombuffer(hb.download(t), dtype=np.uint16).copy()


def widen16(kind, bits16) -> np.ndarray:
    bits16 = np.asarray(bits16, np.uint16)
    if kind == "f16":
        return bits16.view(np.float16).astype(np.float64)
    return oracle.bf16_to_f32(bits16).astype(np.float64)


@pytest.mark.parametrize("case", GEMM_16_KATS + GEMM_16_ORDER_KATS)
def test_16_bit_gemm_known_answers(hb, case):
    kind, a, b, c, alpha, beta, want = case
    k = len(a)
    ta = up16(hb, kind, to_16(kind, a), (1, k))
    tb = up16(hb, kind, to_16(kind, b), (k, 1))
    tc = up16(hb, kind, to_16(kind, c), (1, 1))
    n0 = len(hb.debug_launches())
    hb.gemm(ta, tb, tc, alpha, beta)
    assert int(down16(hb, tc)[0]) == want
    assert len(hb.debug_launches()) == n0 + 1


def test_16_bit_gemm_reads_no_operand_when_alpha_is_zero(hb):
    nan = np.array([0x7E00], np.uint16)
    two = to_16("f16", [2.0])
    tc = up16(hb, "f16", two, (1, 1))
    hb.gemm(up16(hb, "f16", nan, (1, 1)), up16(hb, "f16", nan, (1, 1)), tc, 0.0, 1.0)
    assert int(down16(hb, tc)[0]) == int(two[0])


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("layout", ["rm", "at", "bt"])
def test_16_bit_gemm_rounds_exact_sums_once(hb, kind, layout):
    """Inputs on a grid the 16-bit type holds exactly with |sum| < 2^9 in steps of 2^-14 (exact
    in f32 and f64): the stored value is the exact sum rounded once, as the reference's f32
    accumulation also gives there, bit for bit, in all three layouts and over ragged tiles."""
    m, k, n = 75, 70, 131
    g = rng(hash((kind, layout)) % 1000)
    step = 2.0 ** -7
    av = (g.integers(-256, 256, (m, k)) * step).astype(np.float32)
    bv = (g.integers(-256, 256, (k, n)) * step).astype(np.float32)
    cv = (g.integers(-256, 256, (m, n)) * step).astype(np.float32)
    a16, b16, c16 = to_16(kind, av.ravel()), to_16(kind, bv.ravel()), to_16(kind, cv.ravel())
    ta = up16(hb, kind, a16, (m, k), transpose=layout == "at")
    tb = up16(hb, kind, b16, (k, n), transpose=layout == "bt")
    tc = up16(hb, kind, c16, (m, n))
    hb.gemm(ta, tb, tc, -0.5, 0.25)
    exact = -0.5 * (av.astype(np.float64) @ bv.astype(np.float64)) + 0.25 * cv.astype(np.float64)
    e32 = exact.astype(np.float32).ravel()
    assert np.array_equal(e32.astype(np.float64), exact.ravel())  # exact in f32, so one rounding:
    want = e32.astype(np.float16).view(np.uint16) if kind == "f16" else oracle.f32_to_bf16(e32)
    assert np.array_equal(down16(hb, tc), want)
    cpu = oracle.gemm_seq_16(kind, -0.5, 0.25, a16.reshape(m, k), b16.reshape(k, n),
                             c16.reshape(m, n))
    assert np.array_equal(cpu.ravel(), want)


def same16(kind, got, want) -> bool:
    """Bit equality of 16-bit results, NaN against NaN of any sign and payload (x86 and the
    GPU propagate different NaN payloads through f32 arithmetic; the reference fixes none)."""
    got, want = np.asarray(got, np.uint16).ravel(), np.asarray(want, np.uint16).ravel()
    gn, wn = np.isnan(widen16(kind, got)), np.isnan(widen16(kind, want))
    return bool(np.array_equal(gn, wn) and np.array_equal(got[~wn], want[~wn]))


def run16(hb, kind, layout, a16, b16, c16, m, k, n, alpha, beta) -> np.ndarray:
    ta = up16(hb, kind, a16, (m, k), transpose=layout == "at")
    tb = up16(hb, kind, b16, (k, n), transpose=layout == "bt")
    tc = up16(hb, kind, c16, (m, n))
    n0 = len(hb.debug_launches())
    hb.gemm(ta, tb, tc, alpha, beta)
    assert len(hb.debug_launches()) == n0 + 1
    return down16(hb, tc)


def rand16(g, kind, count, lo=-1.0, hi=1.0) -> np.ndarray:
    x = g.uniform(lo, hi, count).astype(np.float32)
    return oracle.f32_to_f16(x) if kind == "f16" else oracle.f32_to_bf16(x)


ALPHA_THIRD = float(np.float32(1.0 / 3.0))


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("layout", ["rm", "at", "bt"])
@pytest.mark.parametrize("m,k,n,alpha,beta", [(64, 64, 64, 1.0, 0.0), (130, 300, 70, 0.75, -0.5),
                                              (256, 512, 192, ALPHA_THIRD, 0.7), (3, 1000, 5, -2.0, 0.0),
                                              (129, 17, 257, ALPHA_THIRD, 1.0), (1, 1, 1, 1.5, 0.5),
                                              (4096, 24, 2000, ALPHA_THIRD, 0.7)])
def test_16_bit_gemm_is_bit_exact_with_the_cpu_restatement(hb, kind, layout, m, k, n, alpha, beta):
    """Random data, every supported layout, ragged tiles and K slices, on 64x64 tiles (grids
    of fewer than 512 128x128 tiles) and 128x128 ones (the 4096 x 2000 output): the device repeats
    CpuBackend's f32 arithmetic per output (beta*C, then (alpha*a)*b added in k order, each
    step rounded, one 16-bit rounding at the end), so every output has the oracle's bits."""
    g = rng(m * 31 + k * 7 + n + (kind == "bf16") + 3 * len(layout))
    a16, b16, c16 = rand16(g, kind, m * k), rand16(g, kind, k * n), rand16(g, kind, m * n)
    got = run16(hb, kind, layout, a16, b16, c16, m, k, n, alpha, beta)
    want = oracle.gemm_seq_16(kind, alpha, beta, a16.reshape(m, k), b16.reshape(k, n),
                              c16.reshape(m, n))
    assert same16(kind, got, want)


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_16_bit_gemm_bits_at_the_edges_of_the_range(hb, kind):
    """Magnitudes from the 16-bit subnormals to overflow, subnormal operands and results,
    infinities and NaNs in A, B and C: the same bits as the oracle (NaN for NaN)."""
    m, k, n = 70, 90, 66
    g = rng(1600 + (kind == "bf16"))
    top = 15.0 if kind == "f16" else 120.0
    bottom = -24.0 if kind == "f16" else -133.0

    def wide(count):
        x = g.uniform(-1, 1, count) * 2.0 ** g.uniform(bottom, top / 2, count)
        return oracle.f32_to_f16(x.astype(np.float32)) if kind == "f16" else \
            oracle.f32_to_bf16(x.astype(np.float32))
    a16, b16, c16 = wide(m * k), wide(k * n), wide(m * n)
    inf, nan = (0x7C00, 0x7E00) if kind == "f16" else (0x7F80, 0x7FC0)
    a16[g.choice(m * k, 6, replace=False)] = [inf, inf | 0x8000, nan, 0, 0x8000, 1]
    b16[g.choice(k * n, 4, replace=False)] = [inf | 0x8000, nan | 0x8000, 0x8001, 0]
    c16[g.choice(m * n, 4, replace=False)] = [nan, inf, 0x8000, 3]
    for alpha, beta in ((1.0, 0.0), (ALPHA_THIRD, -1.25), (1e-3, 3.0)):
        for layout in ("rm", "at", "bt"):
            got = run16(hb, kind, layout, a16, b16, c16, m, k, n, alpha, beta)
            want = oracle.gemm_seq_16(kind, alpha, beta, a16.reshape(m, k), b16.reshape(k, n),
                                      c16.reshape(m, n))
            assert same16(kind, got, want), (alpha, beta, layout)


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("k,alpha", [(0, 1.0), (40, 0.0)])
def test_16_bit_gemm_beta_scaling_rounds_through_f32(hb, kind, k, alpha):
    """K = 0 or alpha = 0: C = narrow(beta * widen(C)) with the product rounded to f32 first,
    as the reference's loop does (a single f64 rounding can differ), and A, B unread when
    alpha is 0 (they hold NaN)."""
    m, n = 150, 140
    g = rng(1700 + k + (kind == "bf16"))
    c16 = rand16(g, kind, m * n, -100.0, 100.0)
    nan = 0x7E00 if kind == "f16" else 0x7FC0
    a16, b16 = np.full(m * k, nan, np.uint16), np.full(k * n, nan, np.uint16)
    for beta in (0.0, float(np.float32(0.3)), float(np.float32(-1.0 / 7.0))):
        got = run16(hb, kind, "rm", a16, b16, c16, m, k, n, alpha, beta)
        want = oracle.gemm_seq_16(kind, alpha, beta, a16.reshape(m, k), b16.reshape(k, n),
                                  c16.reshape(m, n))
        assert np.array_equal(got, want.ravel()), beta


def test_download_into_and_upload_into(hb):
    """Backend::download_into / upload_into (crates/core/src/lib.rs:118-133): row-major bytes
    out into caller memory and back over an existing tensor, in call order; a failed check
    changes nothing."""
    x = hb.upload_f32([3, 5], np.arange(15, dtype=np.float32))
    out = np.zeros(15, np.float32)
    hb.download_into(x, out)
    assert np.array_equal(out, np.arange(15, dtype=np.float32))
    # In order with earlier work: the gelu enqueued before is in the bytes.
    y = hb.alloc(B.DType.F32, [3, 5])
    hb.gelu(x, y)
    got = bytearray(60)
    hb.download_into(y, got)
    assert np.array_equal(np.frombuffer(bytes(got), np.float32), hb.download_f32(y))
    # upload_into overwrites every element; the source may be reused right away.
    src = np.linspace(-1, 1, 15, dtype=np.float32)
    hb.upload_into(src, y)
    src[:] = 7.0
    assert np.array_equal(hb.download_f32(y), np.linspace(-1, 1, 15, dtype=np.float32))
    # bf16 bytes travel unchanged.
    h = hb.alloc(B.DType.BF16, [4])
    hb.upload_into(np.array([0x3F80, 0xBF81, 0x7FC0, 0x0001], np.uint16), h)
    back = np.zeros(4, np.uint16)
    hb.download_into(h, back)
    assert back.tolist() == [0x3F80, 0xBF81, 0x7FC0, 0x0001]
    # Failed checks: nothing written either way.
    before = hb.download_f32(y)
    for bad, kind in [(np.zeros(14, np.float32), "Shape"), (np.zeros(16, np.float32), "Shape")]:
        with pytest.raises(B.BackendError) as e:
            hb.upload_into(bad, y)
        assert e.value.kind == kind
        sentinel = np.full(bad.size, 3.0, np.float32)
        with pytest.raises(B.BackendError) as e:
            hb.download_into(y, sentinel)
        assert e.value.kind == kind and np.all(sentinel == 3.0)
    with pytest.raises(B.BackendError) as e:
        hb.upload_into(np.zeros(15, np.float32), B.transpose_matrix(y))
    assert e.value.kind == "UnsupportedLayout"
    assert np.array_equal(hb.download_f32(y), before)
    # Zero elements: nothing to move.
    z = hb.alloc(B.DType.F32, [0, 4])
    hb.download_into(z, bytearray())
    hb.upload_into(b"", z)
