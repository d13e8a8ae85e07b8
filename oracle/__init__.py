"""CPU oracle for the contraction / permutation hot path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker or the timed CPU baseline. The product
(liblinalg_hip.so) never routes through it.

Functions (C implementations in oracle.c, each citing the reference code it restates):
  gemm_seq        CpuBackend::gemm accumulation, literal single-thread form
                  (crates/cpu/src/lib.rs:203-295, 606-691)
  gemm_fast       the same arithmetic, loop-interchanged and multi-threaded; bit-identical
  gather_words    tests/permutation_test.rs:84-116 (gather_words_mt: same words, threaded)
  contract_f64    tests/contraction_test.rs:200-268 (f64 accumulation, error magnitude)
  gate            tests/contraction_test.rs:280-313 accuracy gate
  north_star_tol  max|err| <= 1e-5 * sqrt(K) * max|a| * max|b|
  gemm_seq_16     CpuBackend::gemm on F16 / BF16 tensors: f32 accumulation, one 16-bit
                  rounding per output (crates/cpu/src/lib.rs:270-291, 700-720)
  f32_to_f16, f16_to_f32
                  the half crate's (2.7.1) f16 conversions crates/cpu stores and loads with
  gelu, gelu_backward, add_bias, bias_grad, mse_grad, sgd_step, f32_to_bf16, bf16_to_f32
                  the CpuBackend activation and training ops (crates/cpu/src/lib.rs:297-533,
                  722-729, 809-842), sequential, one rounding per operation
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

U = 2.0 ** -24          # unit roundoff of f32 (tests/contraction_test.rs:35-36)
TINY_F32 = 1.401298464324817e-45

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            from . import build as _build
            _build.build()
        L = ctypes.CDLL(str(LIB_PATH))
        f32p = ctypes.POINTER(ctypes.c_float)
        i64, u64 = ctypes.c_int64, ctypes.c_uint64
        L.oracle_gemm_seq_f32.argtypes = [u64, u64, u64, ctypes.c_float, ctypes.c_float,
                                          f32p, i64, i64, f32p, i64, i64, f32p, i64, i64]
        L.oracle_gemm_seq_f32.restype = None
        L.oracle_gemm_fast_f32.argtypes = [u64, u64, u64, ctypes.c_float, ctypes.c_float,
                                           f32p, i64, i64, f32p, i64, i64, f32p, i64, i64,
                                           ctypes.POINTER(u64), u64, ctypes.c_int]
        L.oracle_gemm_fast_f32.restype = ctypes.c_int
        L.oracle_gather_words.argtypes = [ctypes.POINTER(ctypes.c_uint32), ctypes.c_uint32, u64,
                                          ctypes.c_uint32, ctypes.POINTER(u64),
                                          ctypes.POINTER(u64), ctypes.c_int, ctypes.c_int,
                                          ctypes.POINTER(ctypes.c_uint32)]
        L.oracle_gather_words.restype = u64
        L.oracle_gather_words_mt.argtypes = L.oracle_gather_words.argtypes + [
            ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
        L.oracle_gather_words_mt.restype = u64
        dp = ctypes.POINTER(ctypes.c_double)
        i64p = ctypes.POINTER(i64)
        u64p = ctypes.POINTER(u64)
        L.oracle_contract_f64.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_uint32, u64p,
                                          i64p, i64p, i64p, ctypes.c_uint32, u64p, i64p, i64p,
                                          f32p, u64, f32p, u64, f32p, u64, dp, dp, u64p]
        L.oracle_contract_f64.restype = None
        vp = ctypes.c_void_p
        L.oracle_erf_constants.argtypes = [vp]
        L.oracle_erf_constants.restype = None
        for name, args in [("oracle_gelu_f32", [vp, vp, u64]),
                           ("oracle_gelu_backward_f32", [vp, vp, vp, u64]),
                           ("oracle_add_bias_f32", [vp, vp, vp, u64, u64]),
                           ("oracle_bias_grad_f32", [vp, vp, u64, u64]),
                           ("oracle_sgd_step_f32", [vp, vp, ctypes.c_float, u64]),
                           ("oracle_f32_to_bf16", [vp, vp, u64]),
                           ("oracle_bf16_to_f32", [vp, vp, u64]),
                           ("oracle_f32_to_f16", [vp, vp, u64]),
                           ("oracle_f16_to_f32", [vp, vp, u64])]:
            getattr(L, name).argtypes = args
            getattr(L, name).restype = None
        L.oracle_gemm_seq_16.argtypes = [ctypes.c_int, u64, u64, u64, ctypes.c_float,
                                         ctypes.c_float, vp, i64, i64, vp, i64, i64, vp, i64, i64]
        L.oracle_gemm_seq_16.restype = None
        L.oracle_mse_grad_f32.argtypes = [vp, vp, vp, u64]
        L.oracle_mse_grad_f32.restype = ctypes.c_float
        _lib = L
    return _lib


def _fp(arr: np.ndarray, offset: int = 0):
    assert arr.dtype == np.float32
    return ctypes.cast(arr.ctypes.data + 4 * offset, ctypes.POINTER(ctypes.c_float))


def gemm_seq(m, n, k, alpha, beta, a, a_off, a_strides, b, b_off, b_strides, c, c_off, c_strides):
    """Literal crates/cpu accumulation on flat float32 buffers (updated in place: c)."""
    lib().oracle_gemm_seq_f32(m, n, k, alpha, beta, _fp(a, a_off), a_strides[0], a_strides[1],
                              _fp(b, b_off), b_strides[0], b_strides[1], _fp(c, c_off),
                              c_strides[0], c_strides[1])


def default_threads() -> int:
    """Threads for the threaded forms: the CPUs this process may run on, at most 16 (the
    CPU share of one GPU on the GPU hosts, whatever their total count)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def gemm_fast(m, n, k, alpha, beta, a, a_off, a_strides, b, b_off, b_strides, c, c_off,
              c_strides, rows=None, threads=None):
    """Bit-identical multi-threaded form; `rows` restricts the computed rows."""
    if threads is None:
        threads = default_threads()
    rp = None
    nrows = 0
    if rows is not None:
        rows = np.ascontiguousarray(rows, dtype=np.uint64)
        rp = rows.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))
        nrows = rows.size
    rc = lib().oracle_gemm_fast_f32(m, n, k, alpha, beta, _fp(a, a_off), a_strides[0],
                                    a_strides[1], _fp(b, b_off), b_strides[0], b_strides[1],
                                    _fp(c, c_off), c_strides[0], c_strides[1], rp, nrows,
                                    int(threads))
    if rc != 0:
        raise RuntimeError(f"oracle_gemm_fast_f32 failed ({rc})")


def gather_words(words: np.ndarray, w: int, offset: int, shape, strides, conj=False,
                 complex_elem=False) -> np.ndarray:
    """Raw words of a view in row-major logical order (tests/permutation_test.rs:84-116)."""
    words = np.ascontiguousarray(words, dtype=np.uint32)
    n = int(np.prod(shape, dtype=np.uint64)) if len(shape) else 1
    out = np.zeros(max(n * w, 1), dtype=np.uint32)
    sh = (ctypes.c_uint64 * max(len(shape), 1))(*shape)
    st = (ctypes.c_uint64 * max(len(strides), 1))(*strides)
    got = lib().oracle_gather_words(words.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), w,
                                    offset, len(shape), sh, st, int(conj), int(complex_elem),
                                    out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
    return out[:got]


def gather_words_mt(words: np.ndarray, w: int, offset: int, shape, strides, conj=False,
                    complex_elem=False, threads=None) -> np.ndarray:
    """gather_words with the logical elements split into `threads` contiguous ranges."""
    if threads is None:
        threads = default_threads()
    words = np.ascontiguousarray(words, dtype=np.uint32)
    n = int(np.prod(shape, dtype=np.uint64)) if len(shape) else 1
    out = np.zeros(max(n * w, 1), dtype=np.uint32)
    sh = (ctypes.c_uint64 * max(len(shape), 1))(*shape)
    st = (ctypes.c_uint64 * max(len(strides), 1))(*strides)
    failed = ctypes.c_int(0)
    got = lib().oracle_gather_words_mt(words.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), w,
                                       offset, len(shape), sh, st, int(conj), int(complex_elem),
                                       out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                       int(threads), ctypes.byref(failed))
    if failed.value:
        raise RuntimeError("oracle_gather_words_mt could not start its threads")
    return out[:got]


class Expected:
    """exact / magnitude / index per logical element of C, and K (contraction_test.rs:186-197)."""

    def __init__(self, exact, magnitude, index, k):
        self.exact, self.magnitude, self.index, self.k = exact, magnitude, index, k


def contract_f64(alpha, a, a_layout, a_labels, b, b_layout, b_labels, beta, c, c_layout,
                 c_labels) -> Expected:
    """f64 reference over labelled operands. Layouts are (offset, shape, strides)."""
    extent = {}
    for labels, (_, shape, _) in ((a_labels, a_layout), (b_labels, b_layout), (c_labels, c_layout)):
        for l, n in zip(labels, shape):
            assert extent.setdefault(l, n) == n, "test bug: extent mismatch"
    free = list(c_labels)
    summed = [l for l in a_labels if l in b_labels and l not in c_labels]

    def strides_for(labels, layout, over):
        _, _, st = layout
        return [st[labels.index(l)] if l in labels else 0 for l in over]

    u64a = lambda v: np.ascontiguousarray(v, dtype=np.uint64)
    i64a = lambda v: np.ascontiguousarray(v, dtype=np.int64)
    fe = u64a([extent[l] for l in free] or [1])
    se = u64a([extent[l] for l in summed] or [1])
    af, bf, cf = (i64a(strides_for(lbl, lay, free) or [0]) for lbl, lay in
                  ((a_labels, a_layout), (b_labels, b_layout), (c_labels, c_layout)))
    as_, bs_ = (i64a(strides_for(lbl, lay, summed) or [0]) for lbl, lay in
                ((a_labels, a_layout), (b_labels, b_layout)))
    nf = int(np.prod([extent[l] for l in free], dtype=np.int64)) if free else 1
    k = int(np.prod([extent[l] for l in summed], dtype=np.int64)) if summed else 1
    exact = np.zeros(nf, dtype=np.float64)
    mag = np.zeros(nf, dtype=np.float64)
    index = np.zeros(nf, dtype=np.uint64)
    P = lambda arr, t: arr.ctypes.data_as(ctypes.POINTER(t))
    lib().oracle_contract_f64(alpha, beta, len(free), P(fe, ctypes.c_uint64), P(af, ctypes.c_int64),
                              P(bf, ctypes.c_int64), P(cf, ctypes.c_int64), len(summed),
                              P(se, ctypes.c_uint64), P(as_, ctypes.c_int64), P(bs_, ctypes.c_int64),
                              _fp(a), a_layout[0], _fp(b), b_layout[0], _fp(c), c_layout[0],
                              P(exact, ctypes.c_double), P(mag, ctypes.c_double),
                              P(index, ctypes.c_uint64))
    if nf == 0:
        k = k
    return Expected(exact, mag, index.astype(np.int64), k)


def gate(got_buffer: np.ndarray, expected: Expected, name: str = "") -> dict:
    """tests/contraction_test.rs:280-313: |got - ref| <= (K+2)u*mag + u*|ref| + tiny, where ref
    is the f64 result rounded once to f32; non-finite refs must match exactly (NaN ~ NaN).
    Returns statistics; raises AssertionError on the first violation."""
    k = float(expected.k)
    if expected.index.size == 0:
        return {"normalized": 0.0, "gate": 0.0, "max_err": 0.0}
    value = got_buffer[expected.index].astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        rounded = expected.exact.astype(np.float32).astype(np.float64)
    finite = np.isfinite(rounded)
    bad_nf = ~finite & ~((value == rounded) | (np.isnan(value) & np.isnan(rounded)))
    if bad_nf.any():
        i = int(np.flatnonzero(bad_nf)[0])
        raise AssertionError(f"{name}: element {i} is {value[i]}, expected {rounded[i]}")
    with np.errstate(invalid="ignore"):
        err = np.where(finite, np.abs(value - rounded), 0.0)
    tol = (k + 2.0) * U * expected.magnitude + U * np.abs(np.where(finite, rounded, 0.0)) + TINY_F32
    viol = finite & ~(err <= tol)
    if viol.any():
        i = int(np.flatnonzero(viol)[0])
        raise AssertionError(f"{name}: element {i} is {value[i]}, expected {rounded[i]} "
                             f"(exact {expected.exact[i]}); error {err[i]:e} exceeds {tol[i]:e}, K={k}")
    max_err = float(err.max()) if err.size else 0.0
    return {"normalized": max_err / (max(k, 1.0) ** 0.5 * U),
            "gate": float((err / tol).max()) if err.size else 0.0,
            "max_err": max_err}


def north_star_tol(k: int, a: np.ndarray, b: np.ndarray) -> float:
    """max|err| <= 1e-5 * sqrt(K) * max|a| * max|b| (the fp32 north-star bound)."""
    ma = float(np.max(np.abs(a))) if a.size else 0.0
    mb = float(np.max(np.abs(b))) if b.size else 0.0
    return 1e-5 * max(k, 1) ** 0.5 * ma * mb


# ---- Backend activation and training ops --------------------------------------------------
def _f32(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


def erf_constants() -> list:
    out = np.zeros(6, dtype=np.uint32)
    lib().oracle_erf_constants(out.ctypes.data)
    return [int(v) for v in out]


def gelu(x) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    lib().oracle_gelu_f32(x.ctypes.data, y.ctypes.data, x.size)
    return y


def gelu_backward(pre, dy) -> np.ndarray:
    pre, dy = _f32(pre), _f32(dy)
    dx = np.empty_like(pre)
    lib().oracle_gelu_backward_f32(pre.ctypes.data, dy.ctypes.data, dx.ctypes.data, pre.size)
    return dx


def add_bias(x, b) -> np.ndarray:
    x, b = _f32(x), _f32(b)
    y = np.empty_like(x)
    rows, cols = x.shape
    lib().oracle_add_bias_f32(x.ctypes.data, b.ctypes.data, y.ctypes.data, rows, cols)
    return y


def bias_grad(dpre, db) -> np.ndarray:
    dpre = _f32(dpre)
    out = _f32(db).copy()
    rows, cols = dpre.shape
    lib().oracle_bias_grad_f32(dpre.ctypes.data, out.ctypes.data, rows, cols)
    return out


def mse_grad(y, t):
    """(dy, loss) of CpuBackend::mse_grad."""
    y, t = _f32(y), _f32(t)
    dy = np.empty_like(y)
    loss = lib().oracle_mse_grad_f32(y.ctypes.data, t.ctypes.data, dy.ctypes.data, y.size)
    return dy, np.float32(loss)


def sgd_step(w, dw, lr):
    """(w', dw') of CpuBackend::sgd_step."""
    w, dw = _f32(w).copy(), _f32(dw).copy()
    lib().oracle_sgd_step_f32(w.ctypes.data, dw.ctypes.data, float(lr), w.size)
    return w, dw


def f32_to_bf16(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32).view(np.uint32))
    y = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16(x.ctypes.data, y.ctypes.data, x.size)
    return y


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.uint32)
    lib().oracle_bf16_to_f32(h.ctypes.data, y.ctypes.data, h.size)
    return y.view(np.float32)


# ---- f16 contraction: the exact result rounded once ----------------------------------------
def f32_to_f16(x) -> np.ndarray:
    """f16::from_f32_const of the half crate 2.7.1 (crates/cpu/src/lib.rs:700-703): the f32
    bits rounded to nearest even, NaN quiet with its top payload bits; uint16 bits."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32).view(np.uint32))
    y = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16(x.ctypes.data, y.ctypes.data, x.size)
    return y


def f16_to_f32(h) -> np.ndarray:
    """f16::to_f32_const (crates/cpu/src/lib.rs:694-697): exact widening of uint16 bits."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().oracle_f16_to_f32(h.ctypes.data, y.ctypes.data, h.size)
    return y


def gemm_seq_16(kind: str, alpha: float, beta: float, a, b, c) -> np.ndarray:
    """CpuBackend::gemm on F16 or BF16 tensors (crates/cpu/src/lib.rs:270-291 with
    `accumulate`, :664-691): every element widened exactly to f32, acc = beta*C (0 when beta is
    0, C unread), then acc += (alpha*a)*b over k in order in f32 unless alpha is 0, stored
    rounded to the nearest 16-bit value, ties to even (`from_f32_const`, :700-720). a, b, c
    are uint16 bit arrays [m, k], [k, n], [m, n] of any strides; returns the uint16 bits of
    C (a new dense array; c is not changed)."""
    if kind not in ("f16", "bf16"):
        raise ValueError(kind)
    a = np.asarray(a, dtype=np.uint16)
    b = np.asarray(b, dtype=np.uint16)
    out = np.array(c, dtype=np.uint16, order="C", copy=True)
    m, k = a.shape
    n = b.shape[1]
    assert b.shape[0] == k and out.shape == (m, n)
    lib().oracle_gemm_seq_16(0 if kind == "f16" else 1, m, n, k, alpha, beta,
                             a.ctypes.data, a.strides[0] // 2, a.strides[1] // 2,
                             b.ctypes.data, b.strides[0] // 2, b.strides[1] // 2,
                             out.ctypes.data, n, 1)
    return out


def f16_round_exact(x) -> int:
    """Bits of the f16 nearest the exact rational `x` (fractions.Fraction or int), ties to
    even, overflow to infinity, subnormals kept: the single rounding the reference's f16 path
    performs from its double-float dot (shaders/contraction.metal:575-607)."""
    from fractions import Fraction
    x = Fraction(x)
    if x == 0:
        return 0
    sign = 0x8000 if x < 0 else 0
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    elif Fraction(2) ** (e + 1) <= a:
        e += 1
    quantum = Fraction(2) ** (max(e, -14) - 10)
    q = a / quantum
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    value = n * quantum
    if value >= 65536:
        return sign | 0x7C00
    return sign | int(np.float16(float(value)).view(np.uint16))


def contract_exact_f16(alpha, a, b, beta, c) -> np.ndarray:
    """Exact C = alpha*A.B + beta*C for dense 2-D f16 arrays, each element rounded once to
    f16 (returned as uint16 bits). Test sizes only: Python rationals."""
    from fractions import Fraction
    a = np.asarray(a, np.float16)
    b = np.asarray(b, np.float16)
    c = np.asarray(c, np.float16)
    m, k = a.shape
    n = b.shape[1]
    fa = [[Fraction(float(v)) for v in row] for row in a]
    fb = [[Fraction(float(v)) for v in row] for row in b]
    al, be = Fraction(float(np.float32(alpha))), Fraction(float(np.float32(beta)))
    out = np.zeros((m, n), np.uint16)
    for i in range(m):
        for j in range(n):
            s = sum((fa[i][t] * fb[t][j] for t in range(k)), Fraction(0)) if alpha != 0 else 0
            v = al * s
            if beta != 0:
                v += be * Fraction(float(c[i, j]))
            out[i, j] = f16_round_exact(v)
    return out
