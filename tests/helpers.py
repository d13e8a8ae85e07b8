"""Test helpers: layouts, seeded inputs, device buffers, and the reference's case runner.

Restates the fixtures of tests/contraction_test.rs (Layout :87-128, Tensor :130-166,
Case::run :330-401) and tests/permutation_test.rs (SENTINEL, SPECIALS, fills, span,
check_materialize :18-171) over the C ABI. Inputs come from numpy's PCG64 with the seeds
the reference uses (its ChaCha8 streams need Rust; the values differ, the cases do not).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

import linalg_hip as L
import oracle
from linalg_hip import contraction as C
from linalg_hip import permutation as P

GOLDEN = Path(__file__).resolve().parent / "golden"
TAIL = 13                  # spare elements past every contraction view (contraction_test.rs:37)
SENTINEL = 0xDEADBEEF      # permutation_test.rs:18
SPECIALS = np.array(json.loads((GOLDEN / "permutation_kats.json").read_text())["specials"],
                    dtype=np.uint32)
WORDS = {"f32": 1, "u32": 1, "i32": 1, "c64": 2}


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


class Pool:
    """Device buffers allocated by one test, freed at teardown."""

    def __init__(self, ctx):
        self.ctx = ctx
        self.buffers = []

    def alloc(self, dtype: str, length: int) -> L.Buffer:
        b = L.alloc_shared(self.ctx, dtype, length)
        self.buffers.append(b)
        return b

    def free_all(self):
        for b in self.buffers:
            b.free()
        self.buffers = []


# ---------------------------------------------------------------------------------------
# Contraction fixtures
# ---------------------------------------------------------------------------------------
class Layout:
    """Offset, shape and strides of a view, in elements (contraction_test.rs:87-128)."""

    def __init__(self, offset, shape, strides):
        self.offset, self.shape, self.strides = int(offset), list(shape), list(strides)

    @classmethod
    def dense(cls, shape):
        return cls.with_(shape, list(range(len(shape))), [1] * len(shape), 0)

    @classmethod
    def with_(cls, shape, order, steps, offset):
        """Memory nests axes in `order` (outermost first), axis d spaced by steps[d] times
        its natural pitch."""
        strides = [0] * len(shape)
        pitch = 1
        for axis in reversed(order):
            strides[axis] = pitch * steps[axis]
            pitch *= max(shape[axis], 1) * steps[axis]
        return cls(offset, shape, strides)

    @classmethod
    def transposed(cls, rows, cols):
        return cls.with_([rows, cols], [1, 0], [1, 1], 0)

    def span(self) -> int:
        if 0 in self.shape:
            return self.offset
        return self.offset + sum((n - 1) * s for n, s in zip(self.shape, self.strides)) + 1

    def tup(self):
        return (self.offset, self.shape, self.strides)


class Tensor:
    """A device buffer holding one view plus TAIL spare elements, with its host image."""

    def __init__(self, pool: Pool, layout: Layout, data: np.ndarray = None):
        self.layout = layout
        self.cap = layout.span() + TAIL
        self.buffer = pool.alloc("f32", self.cap)
        self.host = np.zeros(self.buffer.nbytes // 4, dtype=np.float32)
        if data is not None:
            self.host[: data.size] = data
        self.buffer.write(self.host)

    @classmethod
    def random(cls, pool, layout, g: np.random.Generator):
        t = cls.__new__(cls)
        cap = layout.span() + TAIL
        data = g.uniform(-1.0, 1.0, cap).astype(np.float32)
        cls.__init__(t, pool, layout, data)
        return t

    def upload(self):
        self.buffer.write(self.host)

    def view(self) -> L.TensorView:
        lay = self.layout
        return L.TensorView(self.buffer, lay.offset, lay.shape, lay.strides, "f32")

    def read(self) -> np.ndarray:
        return self.buffer.read(np.float32)


def assert_untouched(name, before: np.ndarray, after: np.ndarray, written) -> None:
    """Every element outside `written` kept its exact bit pattern (contraction_test.rs:316-328)."""
    mask = np.ones(before.size, dtype=bool)
    if len(written):
        mask[np.asarray(written, dtype=np.int64)] = False
    b, a = before.view(np.uint32), after.view(np.uint32)
    diff = np.flatnonzero(mask & (b != a))
    assert diff.size == 0, f"{name}: element {diff[0]} outside the destination changed"


class Case:
    """One labelled contraction on fresh random tensors (contraction_test.rs:330-401)."""

    def __init__(self, name, a, b, c, alpha=1.0, beta=0.0, via_gemm=False):
        self.name, self.a, self.b, self.c = name, a, b, c
        self.alpha, self.beta, self.via_gemm = alpha, beta, via_gemm

    @classmethod
    def matmul(cls, m, n, k):
        return cls(f"gemm {m}x{n}x{k}", (Layout.dense([m, k]), "mk"), (Layout.dense([k, n]), "kn"),
                   (Layout.dense([m, n]), "mn"), via_gemm=True)

    def scalars(self, alpha, beta):
        self.alpha, self.beta = alpha, beta
        self.name = f"{self.name} alpha={alpha} beta={beta}"
        return self

    def run(self, ctx, pool: Pool, seed: int) -> dict:
        g = rng(seed)
        a = Tensor.random(pool, self.a[0], g)
        b = Tensor.random(pool, self.b[0], g)
        c = Tensor.random(pool, self.c[0], g)
        if self.beta == 0.0:
            c.host[: c.cap] = np.nan
            c.upload()
        a0, b0, c0 = a.host.copy(), b.host.copy(), c.host.copy()
        expected = oracle.contract_f64(self.alpha, a0, self.a[0].tup(), self.a[1], b0,
                                       self.b[0].tup(), self.b[1], self.beta, c0,
                                       self.c[0].tup(), self.c[1])
        if self.via_gemm:
            C.gemm(ctx, self.alpha, a.view(), b.view(), self.beta, c.view())
        else:
            C.contract(ctx, self.alpha, (a.view(), self.a[1]), (b.view(), self.b[1]), self.beta,
                       (c.view(), self.c[1]))
        got = c.read()
        assert_untouched(self.name, a0, a.read(), [])
        assert_untouched(self.name, b0, b.read(), [])
        assert_untouched(self.name, c0, got, expected.index)
        stats = oracle.gate(got, expected, self.name)
        if self.via_gemm and len(self.a[0].shape) == 2:
            check_cpu_oracle(self, a0, b0, c0, got)
        return stats


def check_cpu_oracle(case: Case, a0, b0, c0, got) -> None:
    """North-star gate against the crates/cpu restatement (2-D gemm only)."""
    la, lb, lc = case.a[0], case.b[0], case.c[0]
    m, k = la.shape
    n = lb.shape[1]
    ref = c0.copy()
    oracle.gemm_seq(m, n, k, case.alpha, case.beta, a0, la.offset, la.strides, b0, lb.offset,
                    lb.strides, ref, lc.offset, lc.strides)
    if m == 0 or n == 0:
        return
    rows = np.arange(m)[:, None] * lc.strides[0] + np.arange(n)[None, :] * lc.strides[1] + lc.offset
    r, g = ref[rows].astype(np.float64), got[rows].astype(np.float64)
    fin = np.isfinite(r)
    assert np.array_equal(np.isnan(r), np.isnan(g)), f"{case.name}: NaN pattern differs from crates/cpu"
    assert np.array_equal(r[~fin & ~np.isnan(r)], g[~fin & ~np.isnan(r)]), f"{case.name}: inf mismatch"
    if case.alpha == 0.0 or k == 0:
        assert np.array_equal(r[fin].view(np.uint64), g[fin].view(np.uint64)), \
            f"{case.name}: fill must equal crates/cpu bit for bit"
        return
    am = a0[la.offset + np.arange(m)[:, None] * la.strides[0] + np.arange(k)[None, :] * la.strides[1]]
    bm = b0[lb.offset + np.arange(k)[:, None] * lb.strides[0] + np.arange(n)[None, :] * lb.strides[1]]
    tol = oracle.north_star_tol(k, am * abs(case.alpha), bm)
    if case.beta != 0.0:
        cm = c0[rows]
        tol += 1e-5 * np.max(np.abs(cm)) * abs(case.beta)
    err = np.max(np.abs(r[fin] - g[fin])) if fin.any() else 0.0
    assert err <= tol, f"{case.name}: max|err| {err:e} vs crates/cpu exceeds {tol:e}"


# ---------------------------------------------------------------------------------------
# Permutation fixtures
# ---------------------------------------------------------------------------------------
def span(offset, shape, strides) -> int:
    if 0 in shape:
        return offset
    return offset + 1 + sum((n - 1) * s for n, s in zip(shape, strides))


def random_words(g, n) -> np.ndarray:
    return g.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)


def special_words(g, n) -> np.ndarray:
    coin = g.integers(0, 2, n)
    pick = SPECIALS[g.integers(0, SPECIALS.size, n)]
    return np.where(coin == 0, pick, random_words(g, n)).astype(np.uint32)


def word_buffer(pool, dtype, length, words_fn=None, g=None, fill=None):
    """A buffer of `length` elements whose every word is random/special/`fill`."""
    buf = pool.alloc(dtype, length)
    nw = buf.nbytes // 4
    if words_fn is not None:
        host = words_fn(g, nw)
    else:
        host = np.full(nw, SENTINEL if fill is None else fill, dtype=np.uint32)
    buf.write(host)
    return buf, host


def assert_dst(label, dst: L.Buffer, dtype, dst_offset, expected: np.ndarray) -> None:
    """dst holds `expected` at dst_offset and SENTINEL in every other word."""
    w = WORDS[dtype]
    got = dst.words()
    want = np.full(got.size, SENTINEL, dtype=np.uint32)
    want[dst_offset * w: dst_offset * w + expected.size] = expected
    diff = np.flatnonzero(got != want)
    assert diff.size == 0, (f"{label}: word {diff[0]}: got {got[diff[0]]:#010x}, "
                            f"want {want[diff[0]]:#010x}")


def gather(host_words, view: L.TensorView, conj=False) -> np.ndarray:
    w = WORDS[view.dtype]
    return oracle.gather_words(host_words, w, view.offset, view.shape, view.strides, conj,
                               view.dtype == "c64")


def check_materialize(ctx, pool, dtype, base, perm, src_offset, src_strides, dst_offset, seed):
    """tests/permutation_test.rs:134-159."""
    strides = src_strides if src_strides is not None else L.row_major_strides(base)
    src_buf, src_host = word_buffer(pool, dtype, span(src_offset, base, strides), random_words,
                                    rng(seed))
    src = L.TensorView(src_buf, src_offset, base, strides, dtype)
    view = P.permute_view(src, perm)
    want = gather(src_host, view)
    dst_buf, _ = word_buffer(pool, dtype, dst_offset + view.len() + 17)
    dst = L.TensorView.row_major(dst_buf, dst_offset, view.shape, dtype)
    label = f"{dtype} base={base} perm={perm}"
    P.materialize(ctx, view, dst)
    assert_dst(label, dst_buf, dtype, dst_offset, want)


def permutations(n):
    """All permutations of 0..n in the reference's insertion order (permutation_test.rs:119-132)."""
    if n == 0:
        return [[]]
    out = []
    for tail in permutations(n - 1):
        for pos in range(n):
            p = list(tail)
            p.insert(pos, n - 1)
            out.append(p)
    return out
