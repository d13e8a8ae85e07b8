"""Element offsets and strides past 2^31 (64-bit address arithmetic in every kernel).

The reference limits indices to 2^31 (src/ops/permutation.rs:11-24); this library takes
64-bit element offsets and strides and limits only the extents one kernel handles. Small
operands placed more than 2^31 elements into an 8.6 GB allocation, and a batch stride past
2^31, exercise the 64-bit paths of the GEMM (128-bit and strided loads, split-K), the f16
tile kernel and the transpose, each checked against the oracle on the small regions."""
from __future__ import annotations

import numpy as np
import pytest

import linalg_hip as L
import oracle
from helpers import rng
from linalg_hip import contraction as C
from linalg_hip import permutation as P

pytestmark = pytest.mark.gpu

FAR = 2 ** 31 + 4096  # elements: every operand below starts past 2^31


@pytest.fixture(scope="module")
def big(ctx):
    buf = L.alloc_shared(ctx, "f32", FAR + 2 ** 23)
    yield buf
    buf.free()


def place(buf, offset, data, itemsize=4):
    buf.write(np.ascontiguousarray(data), byte_offset=offset * itemsize)


def fetch(buf, offset, count, dtype=np.float32):
    return buf.read(dtype, byte_offset=offset * np.dtype(dtype).itemsize, count=count)


@pytest.mark.parametrize("a_off,k", [(FAR, 512), (FAR + 17, 300), (FAR, 40000)])
def test_gemm_operands_past_2_to_the_31(ctx, pool, big, a_off, k):
    """Aligned (128-bit loads), misaligned (strided loads) and tall-K (split-K) GEMMs whose
    A and B live past element 2^31 of one allocation; C in another."""
    m, n = 70, 96
    g = rng(a_off + k)
    a = g.uniform(-1, 1, m * k).astype(np.float32)
    b = g.uniform(-1, 1, k * n).astype(np.float32)
    b_off = a_off + m * k + 1024 - (a_off + m * k) % 4
    place(big, a_off, a)
    place(big, b_off, b)
    cbuf = pool.alloc("f32", m * n)
    av = L.TensorView(big, a_off, [m, k], [k, 1])
    bv = L.TensorView(big, b_off, [k, n], [n, 1])
    cv = L.TensorView.row_major(cbuf, 0, [m, n])
    C.gemm(ctx, 1.0, av, bv, 0.0, cv)
    got = cbuf.read(np.float32, count=m * n)
    want = np.zeros(m * n, np.float32)
    oracle.gemm_fast(m, n, k, 1.0, 0.0, a, 0, (k, 1), b, 0, (n, 1), want, 0, (n, 1))
    tol = 1e-5 * np.sqrt(k)
    assert np.max(np.abs(got.astype(np.float64) - want)) <= tol


def test_batched_gemm_with_a_batch_stride_past_2_to_the_31(ctx, pool, big):
    m, k, n = 33, 64, 48
    g = rng(5)
    a0 = g.uniform(-1, 1, m * k).astype(np.float32)
    a1 = g.uniform(-1, 1, m * k).astype(np.float32)
    b = g.uniform(-1, 1, 2 * k * n).astype(np.float32)
    place(big, 0, a0)
    place(big, FAR, a1)
    bbuf, cbuf = pool.alloc("f32", 2 * k * n), pool.alloc("f32", 2 * m * n)
    bbuf.write(b)
    av = L.TensorView(big, 0, [2, m, k], [FAR, k, 1])
    bv = L.TensorView.row_major(bbuf, 0, [2, k, n])
    cv = L.TensorView.row_major(cbuf, 0, [2, m, n])
    C.contract(ctx, 1.0, (av, "bmk"), (bv, "bkn"), 0.0, (cv, "bmn"))
    got = cbuf.read(np.float32, count=2 * m * n).reshape(2, m, n)
    for i, a in enumerate((a0, a1)):
        want = a.reshape(m, k).astype(np.float64) @ b.reshape(2, k, n)[i].astype(np.float64)
        assert np.max(np.abs(got[i] - want)) <= 1e-5 * np.sqrt(k)


def test_f16_gemm_operands_past_2_to_the_31(ctx, pool, big):
    """Halves addressed past element 2^31 (byte offsets past 4 GiB) in the f16 tile kernel."""
    m, k, n = 80, 96, 72
    g = rng(9)
    a = (g.integers(-2048, 2048, m * k) / 1024.0).astype(np.float16)
    b = (g.integers(-2048, 2048, k * n) / 1024.0).astype(np.float16)
    hbuf = L.Buffer(ctx, big.base, big.nbytes)  # the same allocation viewed as halves
    a_off, b_off = FAR, FAR + m * k + 64
    hbuf.write(a, byte_offset=2 * a_off)
    hbuf.write(b, byte_offset=2 * b_off)
    cbuf = pool.alloc("f16", m * n)
    C.gemm(ctx, 1.0, L.TensorView(hbuf, a_off, [m, k], [k, 1], "f16"),
           L.TensorView(hbuf, b_off, [k, n], [n, 1], "f16"), 0.0,
           L.TensorView.row_major(cbuf, 0, [m, n], "f16"))
    got = cbuf.read(np.float16, count=m * n)
    exact = a.reshape(m, k).astype(np.float64) @ b.reshape(k, n).astype(np.float64)
    assert np.array_equal(got.view(np.uint16), exact.astype(np.float16).ravel().view(np.uint16))


@pytest.mark.parametrize("shift", [0, 3])
def test_transpose_past_2_to_the_31(ctx, pool, big, shift):
    """Source and destination both past element 2^31; aligned (128-bit tiles) and shifted by
    three words (32-bit path)."""
    rows, cols = 130, 200
    src_off, dst_off = FAR + shift, FAR + 2 ** 20 + shift
    words = rng(21 + shift).integers(0, 2 ** 32, rows * cols, dtype=np.uint64).astype(np.uint32)
    place(big, src_off, words)
    src = L.TensorView(big, src_off, [rows, cols], [cols, 1])
    dst = L.TensorView(big, dst_off, [cols, rows], [rows, 1])
    P.materialize(ctx, P.permute_view(src, [1, 0]), dst)
    got = fetch(big, dst_off, rows * cols, np.uint32)
    assert np.array_equal(got, words.reshape(rows, cols).T.ravel())
