"""Pins the CPU oracle before it is trusted as the checker (CPU only).

Each oracle function is checked against the reference's own known-answer vectors
(tests/golden/, transcribed from crates/cpu/src/invariants.rs and
tests/permutation_test.rs), closed forms, an independent library routine, and each
other. Planted mistakes (wrong association, f64 accumulation, reversed k order, a
transposed operand, a dropped conjugation) are shown to fail these checks.
"""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest

import oracle
from helpers import GOLDEN, Layout, permutations, rng

KATS = json.loads((GOLDEN / "cpu_gemm_kats.json").read_text())
PKATS = json.loads((GOLDEN / "permutation_kats.json").read_text())


def f32_from_bits(words):
    return np.array(words, dtype=np.uint32).view(np.float32)


def layouts(m, k, n, a, b):
    """The three crates/cpu layouts (crates/cpu/src/lib.rs:236-241) of the same logical A, B:
    yields (A storage, A offset/strides, B storage, B strides)."""
    A = np.asarray(a, np.float32).reshape(m, k) if m * k else np.zeros((m, k), np.float32)
    B = np.asarray(b, np.float32).reshape(k, n) if k * n else np.zeros((k, n), np.float32)
    yield "rm,rm", A.ravel().copy(), (k, 1), B.ravel().copy(), (n, 1)
    # transpose_matrix of a row-major [k, m] matrix: strides [1, m].
    yield "t,rm", A.T.ravel().copy(), (1, m), B.ravel().copy(), (n, 1)
    yield "rm,t", A.ravel().copy(), (k, 1), B.T.ravel().copy(), (1, k)


@pytest.mark.parametrize("kat", KATS, ids=[k["name"] for k in KATS])
@pytest.mark.parametrize("fn", ["seq", "fast"])
def test_gemm_known_answers_all_layouts(kat, fn):
    m, k, n = kat["m"], kat["k"], kat["n"]
    a, b = f32_from_bits(kat["a"]), f32_from_bits(kat["b"])
    for name, As, ast, Bs, bst in layouts(m, k, n, a, b):
        c = f32_from_bits(kat["c0"]).copy()
        As = np.ascontiguousarray(As if As.size else np.zeros(1, np.float32))
        Bs = np.ascontiguousarray(Bs if Bs.size else np.zeros(1, np.float32))
        if fn == "seq":
            oracle.gemm_seq(m, n, k, kat["alpha"], kat["beta"], As, 0, ast, Bs, 0, bst, c, 0, (n, 1))
        else:
            oracle.gemm_fast(m, n, k, kat["alpha"], kat["beta"], As, 0, ast, Bs, 0, bst, c, 0,
                             (n, 1), threads=2)
        got = c.view(np.uint32).tolist()
        assert got == kat["expected"], f"{kat['name']} [{name}]: {got} != {kat['expected']}"
        if "not_expected" in kat:
            assert got != kat["not_expected"]


def _wrong_right_assoc(m, n, k, alpha, beta, a, b, c):
    out = c.copy()
    for i in range(m):
        for j in range(n):
            acc = np.float32(0) if beta == 0 else np.float32(beta) * c[i * n + j]
            if alpha != 0:
                for p in range(k):
                    acc = np.float32(acc + np.float32(alpha) * np.float32(a[i * k + p] * b[p * n + j]))
            out[i * n + j] = acc
    return out


def _wrong_f64(m, n, k, alpha, beta, a, b, c):
    A, B = a.reshape(m, k).astype(np.float64), b.reshape(k, n).astype(np.float64)
    base = np.zeros((m, n)) if beta == 0 else beta * c.reshape(m, n).astype(np.float64)
    return (base + alpha * (A @ B)).astype(np.float32).ravel() if alpha != 0 else base.astype(np.float32).ravel()


def _wrong_reversed_k(m, n, k, alpha, beta, a, b, c):
    out = c.copy()
    for i in range(m):
        for j in range(n):
            acc = np.float32(0) if beta == 0 else np.float32(beta) * c[i * n + j]
            if alpha != 0:
                for p in reversed(range(k)):
                    acc = np.float32(acc + np.float32(np.float32(alpha) * a[i * k + p]) * b[p * n + j])
            out[i * n + j] = acc
    return out


# Closed form of the k-order rule that the reference's 2^25 vector leaves open: with
# a = [1, 2^25, -2^25], b = 1, ascending k gives (0 + 1) + 2^25 -> 2^25 (ties to even), then
# + (-2^25) -> +0; descending k gives (-2^25 + 2^25) + 1 = 1.
ORDER_KAT = {"name": "ascending k order", "m": 1, "k": 3, "n": 1, "alpha": 1.0, "beta": 0.0,
             "a": np.array([1.0, 2.0 ** 25, -2.0 ** 25], np.float32).view(np.uint32).tolist(),
             "b": np.array([1.0, 1.0, 1.0], np.float32).view(np.uint32).tolist(),
             "c0": [0], "expected": [0]}


@pytest.mark.parametrize("fn", ["seq", "fast"])
def test_gemm_ascending_k_order(fn):
    kat = ORDER_KAT
    a, b = f32_from_bits(kat["a"]), f32_from_bits(kat["b"])
    for name, As, ast, Bs, bst in layouts(1, 3, 1, a, b):
        c = np.zeros(1, np.float32)
        f = oracle.gemm_seq if fn == "seq" else oracle.gemm_fast
        f(1, 1, 3, 1.0, 0.0, As, 0, ast, Bs, 0, bst, c, 0, (1, 1))
        assert c.view(np.uint32).tolist() == [0], name


@pytest.mark.parametrize("wrong", [_wrong_right_assoc, _wrong_f64, _wrong_reversed_k])
def test_known_answers_reject_planted_mistakes(wrong):
    """At least one known answer fails for each plausible restatement mistake."""
    caught = False
    with np.errstate(all="ignore"):
        for kat in KATS + [ORDER_KAT]:
            m, k, n = kat["m"], kat["k"], kat["n"]
            a, b = f32_from_bits(kat["a"]), f32_from_bits(kat["b"])
            c0 = f32_from_bits(kat["c0"]).copy()
            got = wrong(m, n, k, kat["alpha"], kat["beta"], a, b, c0).view(np.uint32).tolist()
            caught |= got != kat["expected"]
    assert caught


def test_seq_and_fast_are_bit_identical_on_random_and_edge_cases():
    g = rng(42)
    cases = [(1, 1, 1), (3, 5, 7), (17, 33, 65), (64, 130, 257), (5, 600, 3), (40, 24, 3000),
             (2, 1100, 16)]
    for (m, n, k) in cases:
        for alpha, beta in [(1.0, 0.0), (-0.75, 1.0), (0.5, -0.5), (0.0, 2.0)]:
            for lay in ("rm", "ta", "tb"):
                a = g.uniform(-1, 1, m * k).astype(np.float32)
                b = g.uniform(-1, 1, k * n).astype(np.float32)
                c = g.uniform(-1, 1, m * n).astype(np.float32)
                ast, bst = (k, 1), (n, 1)
                if lay == "ta":
                    ast = (1, m)
                if lay == "tb":
                    bst = (1, k)
                c1, c2 = c.copy(), c.copy()
                oracle.gemm_seq(m, n, k, alpha, beta, a, 0, ast, b, 0, bst, c1, 0, (n, 1))
                oracle.gemm_fast(m, n, k, alpha, beta, a, 0, ast, b, 0, bst, c2, 0, (n, 1), threads=3)
                assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32)), (m, n, k, alpha, beta, lay)
    # Row subset mode computes exactly the listed rows and leaves the others alone.
    m, n, k = 50, 40, 30
    a = g.uniform(-1, 1, m * k).astype(np.float32)
    b = g.uniform(-1, 1, k * n).astype(np.float32)
    full = np.zeros(m * n, np.float32)
    oracle.gemm_seq(m, n, k, 1.0, 0.0, a, 0, (k, 1), b, 0, (n, 1), full, 0, (n, 1))
    part = np.full(m * n, 7.0, np.float32)
    rows = [0, 13, 49]
    oracle.gemm_fast(m, n, k, 1.0, 0.0, a, 0, (k, 1), b, 0, (n, 1), part, 0, (n, 1), rows=rows)
    for r in range(m):
        seg = slice(r * n, (r + 1) * n)
        if r in rows:
            assert np.array_equal(part[seg], full[seg])
        else:
            assert np.all(part[seg] == 7.0)


def test_gemm_closed_forms():
    g = rng(7)
    n = 37
    x = g.uniform(-1, 1, n * n).astype(np.float32)
    eye = np.eye(n, dtype=np.float32).ravel()
    out = np.zeros(n * n, np.float32)
    oracle.gemm_seq(n, n, n, 1.0, 0.0, x, 0, (n, 1), eye, 0, (n, 1), out, 0, (n, 1))
    assert np.array_equal(out, x), "X.I must equal X bit for bit"
    perm = g.permutation(n)
    pm = np.zeros((n, n), np.float32)
    pm[np.arange(n), perm] = 1.0
    oracle.gemm_seq(n, n, n, 1.0, 0.0, pm.ravel().copy(), 0, (n, 1), x, 0, (n, 1), out, 0, (n, 1))
    assert np.array_equal(out.reshape(n, n), x.reshape(n, n)[perm]), "P.X permutes rows exactly"
    # Integer-valued inputs: every partial sum is an integer below 2^24, so the result is exact
    # and must equal an int64 matrix product; a transposed operand would not.
    m, k, nn = 23, 41, 19
    ai = g.integers(-20, 21, (m, k))
    bi = g.integers(-20, 21, (k, nn))
    out = np.zeros(m * nn, np.float32)
    oracle.gemm_seq(m, nn, k, 1.0, 0.0, ai.astype(np.float32).ravel(), 0, (k, 1),
                    bi.astype(np.float32).ravel(), 0, (nn, 1), out, 0, (nn, 1))
    assert np.array_equal(out.reshape(m, nn).astype(np.int64), ai @ bi)
    # Rank one: a column times a row is one rounding per element.
    col = g.uniform(-1, 1, m).astype(np.float32)
    row = g.uniform(-1, 1, nn).astype(np.float32)
    out = np.zeros(m * nn, np.float32)
    oracle.gemm_seq(m, nn, 1, 1.0, 0.0, col, 0, (1, 1), row, 0, (nn, 1), out, 0, (nn, 1))
    assert np.array_equal(out.reshape(m, nn), np.outer(col, row).astype(np.float32))
    # 2-D strides are honoured: C^T = B^T A^T with transposed views of the same storage.
    a = g.uniform(-1, 1, m * k).astype(np.float32)
    b = g.uniform(-1, 1, k * nn).astype(np.float32)
    c1 = np.zeros(m * nn, np.float32)
    oracle.gemm_seq(m, nn, k, 1.0, 0.0, a, 0, (k, 1), b, 0, (nn, 1), c1, 0, (nn, 1))
    c2 = np.zeros(m * nn, np.float32)
    oracle.gemm_seq(nn, m, k, 1.0, 0.0, b, 0, (1, nn), a, 0, (1, k), c2, 0, (1, nn))
    # Same products, same k order, only the roles of a and b swap inside each product.
    assert np.allclose(c1, c2, rtol=0, atol=1e-5)


def _einsum_f64(alpha, a, la, al, b, lb, bl, beta, c, lc, cl):
    def dense(buf, lay):
        off, shape, st = lay
        idx = np.full(shape, off, dtype=np.int64)
        for d, (n, s) in enumerate(zip(shape, st)):
            sh = [1] * len(shape)
            sh[d] = n
            idx = idx + (np.arange(n) * s).reshape(sh)
        return buf[idx].astype(np.float64)
    A, B, C0 = dense(a, la), dense(b, lb), dense(c, lc)
    out = alpha * np.einsum(f"{al},{bl}->{cl}", A, B) if alpha != 0 else np.zeros(C0.shape)
    if beta != 0:
        out = out + beta * C0
    return out


def test_contract_f64_matches_numpy_einsum_and_exact_integers():
    g = rng(11)
    cases = [
        ("mk", "kn", "mn", Layout.dense([7, 5]), Layout.dense([5, 9]), Layout.dense([7, 9])),
        ("bmk", "bkn", "bmn", Layout.dense([3, 4, 6]), Layout.dense([3, 6, 5]), Layout.dense([3, 4, 5])),
        ("ijkl", "lkmn", "imjn", Layout.with_([5, 7, 6, 9], [2, 0, 3, 1], [1, 1, 1, 1], 3),
         Layout.with_([9, 6, 4, 11], [3, 0, 2, 1], [1, 2, 1, 1], 0),
         Layout.with_([5, 4, 7, 11], [1, 3, 0, 2], [1, 1, 2, 1], 8)),
        ("mbk", "knb", "nbm", Layout.with_([19, 6, 23], [1, 0, 2], [1, 1, 1], 2),
         Layout.with_([23, 31, 6], [0, 2, 1], [1, 1, 2], 0),
         Layout.with_([31, 6, 19], [1, 2, 0], [1, 1, 1], 4)),
    ]
    for la, lb, lc, A, B, Cl in cases:
        for alpha, beta in [(1.0, 0.0), (-1.5, -0.5), (0.0, 2.0)]:
            a = g.uniform(-1, 1, A.span() + 3).astype(np.float32)
            b = g.uniform(-1, 1, B.span() + 3).astype(np.float32)
            c = g.uniform(-1, 1, Cl.span() + 3).astype(np.float32)
            e = oracle.contract_f64(alpha, a, A.tup(), la, b, B.tup(), lb, beta, c, Cl.tup(), lc)
            want = _einsum_f64(alpha, a, A.tup(), la, b, B.tup(), lb, beta, c, Cl.tup(), lc)
            assert np.allclose(e.exact, want.ravel(), rtol=1e-12, atol=1e-12)
            got_c = np.zeros(c.size)
            got_c[e.index] = 1
            # C's element indices enumerate C's view exactly once, in row-major order.
            off, shape, st = Cl.tup()
            first = off + sum(0 for _ in shape)
            assert e.index[0] == first and len(set(e.index.tolist())) == e.index.size
    # Integer data: exact results, and a planted transposed operand disagrees.
    ai = g.integers(-9, 10, 6 * 4).astype(np.float32)
    bi = g.integers(-9, 10, 4 * 5).astype(np.float32)
    ci = np.zeros(6 * 5, np.float32)
    e = oracle.contract_f64(1.0, ai, (0, [6, 4], [4, 1]), "mk", bi, (0, [4, 5], [5, 1]), "kn",
                            0.0, ci, (0, [6, 5], [5, 1]), "mn")
    assert np.array_equal(e.exact, (ai.reshape(6, 4).astype(np.int64) @
                                    bi.reshape(4, 5).astype(np.int64)).ravel())
    assert e.k == 4 and np.all(e.magnitude >= np.abs(e.exact))


def test_gate_accepts_rounding_and_rejects_a_dropped_term():
    g = rng(5)
    m, n, k = 20, 30, 400
    a = g.uniform(-1, 1, m * k).astype(np.float32)
    b = g.uniform(-1, 1, k * n).astype(np.float32)
    c = np.zeros(m * n, np.float32)
    e = oracle.contract_f64(1.0, a, (0, [m, k], [k, 1]), "mk", b, (0, [k, n], [n, 1]), "kn", 0.0,
                            c, (0, [m, n], [n, 1]), "mn")
    seq = c.copy()
    oracle.gemm_seq(m, n, k, 1.0, 0.0, a, 0, (k, 1), b, 0, (n, 1), seq, 0, (n, 1))
    stats = oracle.gate(seq, e, "seq")  # the sequential f32 sum passes the f64 gate
    assert stats["gate"] <= 1.0
    dropped = c.copy()  # one missing product term is far outside the gate
    oracle.gemm_seq(m, n, k - 1, 1.0, 0.0, a, 0, (k, 1), b, 0, (n, 1), dropped, 0, (n, 1))
    with pytest.raises(AssertionError):
        oracle.gate(dropped, e, "dropped term")
    flipped = (-seq).copy()
    with pytest.raises(AssertionError):
        oracle.gate(flipped, e, "wrong sign")
    nan = seq.copy()
    nan[3] = np.nan
    with pytest.raises(AssertionError):
        oracle.gate(nan, e, "nan")


def test_gather_matches_numpy_transpose_for_every_rank_5_permutation():
    base = [3, 5, 7, 11, 13]
    g = rng(3)
    words = g.integers(0, 2 ** 32, int(np.prod(base)), dtype=np.uint64).astype(np.uint32)
    x = words.reshape(base)
    strides = [int(s // 4) for s in x.strides]
    for perm in permutations(5):
        got = oracle.gather_words(words, 1, 0, [base[p] for p in perm], [strides[p] for p in perm])
        assert np.array_equal(got, np.transpose(x, perm).ravel())


def test_gather_offsets_strides_and_complex_words():
    g = rng(4)
    words = g.integers(0, 2 ** 32, 2 * 400, dtype=np.uint64).astype(np.uint32)
    # complex [f32;2] view, offset 5, padded rows (strides in elements of two words)
    shape, strides, off = [4, 9], [20, 1], 5
    got = oracle.gather_words(words, 2, off, shape, strides)
    cw = words.view(np.uint64)
    want = cw[off + np.arange(4)[:, None] * 20 + np.arange(9)[None, :]].ravel().view(np.uint32)
    assert np.array_equal(got, want)
    conj = oracle.gather_words(words, 2, off, shape, strides, conj=True, complex_elem=True)
    assert np.array_equal(conj[0::2], want[0::2])
    assert np.array_equal(conj[1::2], want[1::2] ^ np.uint32(0x80000000))
    # conj on a real type is a plain copy; a dropped conjugation is caught by the table below.
    real = oracle.gather_words(words, 1, 0, [10, 10], [10, 1], conj=True, complex_elem=False)
    assert np.array_equal(real, words[:100])
    # Zero strides broadcast.
    bc = oracle.gather_words(words, 1, 7, [3, 4], [0, 1])
    assert np.array_equal(bc, np.tile(words[7:11], 3))
    # Rank 0 is one element; an empty view is no words.
    assert oracle.gather_words(words, 1, 9, [], []).tolist() == [int(words[9])]
    assert oracle.gather_words(words, 1, 0, [3, 0], [1, 1]).size == 0


def test_threaded_gather_writes_the_same_words():
    """gather_words_mt (the all-core CPU baseline) against numpy and the one-thread form,
    with range splits falling mid-row, more threads than elements, rank 0 and empty views."""
    g = rng(5)
    words = g.integers(0, 2 ** 32, 2 * 7 * 11 * 13, dtype=np.uint64).astype(np.uint32)
    x = words[: 7 * 11 * 13].reshape(7, 11, 13)
    for threads in (1, 2, 3, 7, 16, 2000):
        got = oracle.gather_words_mt(words, 1, 0, [13, 7, 11], [1, 143, 13], threads=threads)
        assert np.array_equal(got, np.transpose(x, (2, 0, 1)).ravel()), threads
        cj = oracle.gather_words_mt(words, 2, 3, [5, 9], [1, 5], conj=True, complex_elem=True,
                                    threads=threads)
        assert np.array_equal(cj, oracle.gather_words(words, 2, 3, [5, 9], [1, 5], conj=True,
                                                      complex_elem=True)), threads
    assert oracle.gather_words_mt(words, 1, 9, [], [], threads=4).tolist() == [int(words[9])]
    assert oracle.gather_words_mt(words, 1, 0, [3, 0], [1, 1], threads=4).size == 0


def test_gather_reproduces_the_complex_adjoint_word_table():
    t = PKATS["complex_adjoint"]
    m, n = t["m"], t["n"]
    words = np.array(t["input_words"], dtype=np.uint32)
    # adjoint = swap the last two axes of row-major [m, n] (strides [n, 1]) and conjugate.
    got = oracle.gather_words(words, 2, 0, [n, m], [1, n], conj=True, complex_elem=True)
    assert got.tolist() == t["adjoint_words"]
    no_conj = oracle.gather_words(words, 2, 0, [n, m], [1, n], conj=False, complex_elem=True)
    assert no_conj.tolist() != t["adjoint_words"]


def test_north_star_tolerance_formula():
    a = np.array([0.5, -2.0], np.float32)
    b = np.array([4.0, -1.0], np.float32)
    assert oracle.north_star_tol(100, a, b) == pytest.approx(1e-5 * 10 * 2.0 * 4.0)
    assert struct.pack("<f", 1.0) == np.float32(1.0).tobytes()


# ---- f16: the single-rounding reference ----------------------------------------------------
def test_f16_round_exact_agrees_with_numpy_on_doubles():
    from fractions import Fraction
    g = np.random.Generator(np.random.PCG64(16))
    vals = list(g.standard_normal(3000) * np.exp2(g.integers(-30, 18, 3000)))
    # Ties, the overflow threshold, subnormal boundaries.
    vals += [1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 65504.0, 65519.99, 65520.0, 2.0 ** -24,
             2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -25 + 2.0 ** -40, 2.0 ** -14 - 2.0 ** -25, -0.5]
    for v in vals:
        with np.errstate(over="ignore"):
            want = int(np.float16(v).view(np.uint16))
        assert oracle.f16_round_exact(Fraction(v)) == want, v


def test_f16_scale_known_answer_from_the_reference():
    # shaders/contraction.metal:730-733: beta = -0.999 times C = 0x0DDC rounds once to 0x8DDB
    # (rounding the f32 product first gives 0x8DDA).
    from fractions import Fraction
    c = np.uint16(0x0DDC).view(np.float16)
    beta = np.float32(-0.999)
    exact = Fraction(float(beta)) * Fraction(float(c))
    assert oracle.f16_round_exact(exact) == 0x8DDB
    twice = int(np.float16(np.float32(beta) * np.float32(c)).view(np.uint16))
    assert twice == 0x8DDA  # the double rounding the reference avoids


def test_contract_exact_f16_small_closed_forms():
    a = np.array([[1, 2], [3, 4]], np.float16)
    b = np.array([[5, 6], [7, 8]], np.float16)
    got = oracle.contract_exact_f16(1.0, a, b, 0.0, np.zeros((2, 2), np.float16))
    assert got.view(np.float16).tolist() == [[19, 22], [43, 50]]
    # 2048 + 1 is a tie in f16 (spacing 2 above 2048): rounds to even 2048; + 3 rounds to 2052.
    a = np.array([[2048, 1]], np.float16)
    b = np.array([[1], [1]], np.float16)
    assert oracle.contract_exact_f16(1.0, a, b, 0.0, np.zeros((1, 1), np.float16)).view(np.float16)[0, 0] == 2048
    a = np.array([[2048, 3]], np.float16)
    assert oracle.contract_exact_f16(1.0, a, b, 0.0, np.zeros((1, 1), np.float16)).view(np.float16)[0, 0] == 2052


# ---- CpuBackend::gemm on F16 / BF16 (crates/cpu/src/invariants.rs:556-720) ------------------
TIE_DOWN = 1.0 / 256.0          # the exact halfway step at 1.0 for bf16 (ulp 2^-7)
ONE_PLUS_ULP = 1.0 + 1.0 / 128.0
GEMM_16_KATS = [  # (dtype, a, b, c, alpha, beta, expected bits), the reference's case list
    ("f16", [2048.0, 1.0], [1.0, 1.0], [0.0], 1.0, 0.0, 0x6800),
    ("f16", [2050.0, 1.0], [1.0, 1.0], [0.0], 1.0, 0.0, 0x6802),
    ("f16", [2048.0, 1.0, 1.0], [1.0, 1.0, 1.0], [0.0], 1.0, 0.0, 0x6801),
    ("f16", [2048.0, 1.0, 0.5], [1.0, 1.0, 1.0], [0.0], 1.0, 0.0, 0x6801),
    ("f16", [-2048.0, -1.0], [1.0, 1.0], [0.0], 1.0, 0.0, 0xE800),
    ("f16", [2048.0, 1.0], [1.0, 1.0], [1.0], 1.0, 1.0, 0x6801),
    ("bf16", [1.0, TIE_DOWN], [1.0, 1.0], [0.0], 1.0, 0.0, 0x3F80),
    ("bf16", [ONE_PLUS_ULP, TIE_DOWN], [1.0, 1.0], [0.0], 1.0, 0.0, 0x3F82),
    ("bf16", [1.0, TIE_DOWN, TIE_DOWN], [1.0, 1.0, 1.0], [0.0], 1.0, 0.0, 0x3F81),
    ("bf16", [-1.0, -TIE_DOWN], [1.0, 1.0], [0.0], 1.0, 0.0, 0xBF80),
    ("bf16", [1.0, TIE_DOWN], [1.0, 1.0], [TIE_DOWN], 1.0, 1.0, 0x3F81),
]


def to_16(kind, values):
    v = np.asarray(values, np.float32)
    bits = v.astype(np.float16).view(np.uint16) if kind == "f16" else oracle.f32_to_bf16(v)
    back = (bits.view(np.float16).astype(np.float32) if kind == "f16" else oracle.bf16_to_f32(bits))
    assert np.array_equal(back, v), "fixture value not exact in the 16-bit type"
    return bits


@pytest.mark.parametrize("case", GEMM_16_KATS)
def test_gemm_seq_16_on_the_reference_known_answers(case):
    kind, a, b, c, alpha, beta, want = case
    k = len(a)
    got = oracle.gemm_seq_16(kind, alpha, beta, to_16(kind, a).reshape(1, k),
                             to_16(kind, b).reshape(k, 1), to_16(kind, c).reshape(1, 1))
    assert int(got[0, 0]) == want


def test_gemm_seq_16_reads_nothing_unread_and_sums_in_f32():
    nan = np.array([[0x7E00]], np.uint16)
    two = to_16("f16", [2.0]).reshape(1, 1)
    assert int(oracle.gemm_seq_16("f16", 0.0, 1.0, nan, nan, two)[0, 0]) == int(two[0, 0])
    # f32 accumulation, not f16: 2048 + 1 + 1 in f16 steps would stay at 2048.
    ones = to_16("f16", [2048.0, 1.0, 1.0]).reshape(1, 3)
    assert int(oracle.gemm_seq_16("f16", 1.0, 0.0, ones, to_16("f16", [1.0] * 3).reshape(3, 1),
                                  nan)[0, 0]) == 0x6801
    # and f32, not f64: 1 + 2^-8 + 2^-30 is just above the bf16 tie at 1 + 2^-8 (0x3F81),
    # but its f32 sum drops the 2^-30 and lands on the tie, which rounds to even: 0x3F80.
    ops = to_16("bf16", [1.0, 2.0 ** -8, 2.0 ** -30]).reshape(1, 3)
    got = oracle.gemm_seq_16("bf16", 1.0, 0.0, ops, to_16("bf16", [1.0] * 3).reshape(3, 1), nan)
    assert int(got[0, 0]) == 0x3F80


def test_f32_to_f16_matches_numpy_rounding_on_every_rounding_position():
    """The half crate's f32 -> f16 (oracle.f32_to_f16) against numpy's IEEE conversion on
    every finite f32 whose low 13 mantissa bits are a rounding-critical pattern (exact, just
    below, at and just above the halfway point, all kept-bit parities), for every exponent
    from far below the f16 subnormals to past the overflow threshold, both signs, every value
    of the top ten mantissa bits; plus random bit patterns. Covers the subnormal positions,
    where the round bit moves into the top ten bits, and the carry into the exponent."""
    low = np.array([0, 1, 0x7FF, 0x800, 0x801, 0xFFF, 0x1000, 0x1001, 0x17FF, 0x1800, 0x1FFF],
                   np.uint32)
    top = np.arange(1024, dtype=np.uint32) << 13
    exps = np.arange(90, 148, dtype=np.uint32) << 23
    bits = (exps[:, None, None] | top[None, :, None] | low[None, None, :]).ravel()
    bits = np.concatenate([bits, bits | 0x80000000, np.array([0, 0x80000000, 1, 0x807FFFFF,
                                                             0x7F800000, 0xFF800000,
                                                             0x7F7FFFFF, 0x477FF000,
                                                             0x477FEFFF, 0x33000000,
                                                             0x33000001], np.uint32)])
    rnd = np.random.default_rng(16).integers(0, 2 ** 32, 1 << 21, dtype=np.uint64).astype(np.uint32)
    bits = np.concatenate([bits, rnd[(rnd & 0x7F800000) != 0x7F800000]])
    got = oracle.f32_to_f16(bits.view(np.float32))
    with np.errstate(over="ignore"):
        want = bits.view(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    # The reference's own asserted bits (crates/cpu/src/invariants.rs:560-564).
    assert list(oracle.f32_to_f16(np.array([2048, 2050, 2052, 2049, 2051], np.float32))) == \
        [0x6800, 0x6801, 0x6802, 0x6800, 0x6802]
    # 65520 is the tie between 65504 and 2^16: ties to even overflow to infinity.
    assert list(oracle.f32_to_f16(np.array([65504, 65519.996, 65520, -1e9], np.float32))) == \
        [0x7BFF, 0x7BFF, 0x7C00, 0xFC00]


def test_f16_nan_conversions_keep_sign_and_payload_quietly():
    """The crate's NaN rule, both directions: f32 NaN -> sign | 0x7C00 | 0x0200 | top ten
    payload bits; f16 NaN -> sign | 0x7FC00000 | payload << 13; infinities stay exact."""
    f = np.array([0x7F800001, 0x7FC00000, 0xFFFFFFFF, 0x7F802000, 0xFF800000], np.uint32)
    assert [hex(v) for v in oracle.f32_to_f16(f.view(np.float32))] == \
        ["0x7e00", "0x7e00", "0xffff", "0x7e01", "0xfc00"]
    h = np.array([0x7C01, 0x7E00, 0xFFFF, 0x7C00, 0xFC00], np.uint16)
    assert [hex(v) for v in oracle.f16_to_f32(h).view(np.uint32)] == \
        ["0x7fc02000", "0x7fc00000", "0xffffe000", "0x7f800000", "0xff800000"]


def test_f16_to_f32_is_exact_on_every_finite_half():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (h & 0x7C00) != 0x7C00
    got = oracle.f16_to_f32(h[finite])
    assert np.array_equal(got.view(np.uint32), h[finite].view(np.float16).astype(np.float32).view(np.uint32))


# Closed forms where the evaluation order decides the bits (same layout as GEMM_16_KATS).
# k order: 2^-14 + 2048 - 2048 + 2^-14 in f32 loses the first 2^-14 against 2048 (f32 ulp
# there is 2^-12) and keeps the last: 2^-14 = f16 0x0400. A pairwise sum
# (2^-14 + 2048) + (-2048 + 2^-14) would give +0.
# No fused multiply-add: alpha = 1 + 2^-23, a = b = 1 + 2^-10 (f16) / 1 + 2^-7 (bf16).
# t = alpha*a rounds to 1 + 2^-10 + 2^-23 (the 2^-33 term drops), t*b rounds again, so the
# second term -t*b cancels the first exactly: +0. A fused acc + t*(-b) would keep the
# dropped -2^-33 (f16: -0, 0x8000) or -2^-30 (bf16: 0xB080).
ALPHA_1ULP = float(np.float32(1.0 + 2.0 ** -23))
GEMM_16_ORDER_KATS = [
    ("f16", [2.0 ** -14, 2048.0, -2048.0, 2.0 ** -14], [1.0] * 4, [0.0], 1.0, 0.0, 0x0400),
    ("f16", [1.0 + 2.0 ** -10] * 2, [1.0 + 2.0 ** -10, -1.0 - 2.0 ** -10], [0.0], ALPHA_1ULP, 0.0,
     0x0000),
    ("bf16", [1.0 + 2.0 ** -7] * 2, [1.0 + 2.0 ** -7, -1.0 - 2.0 ** -7], [0.0], ALPHA_1ULP, 0.0,
     0x0000),
]


@pytest.mark.parametrize("case", GEMM_16_ORDER_KATS)
def test_gemm_seq_16_keeps_k_order_and_rounds_each_multiply(case):
    test_gemm_seq_16_on_the_reference_known_answers(case)


def test_the_fused_results_the_order_cases_rule_out():
    from fractions import Fraction as F
    for e, want in ((2.0 ** -10, -(F(2) ** -33)), (2.0 ** -7, -(F(2) ** -30))):
        t = np.float32(ALPHA_1ULP) * np.float32(1.0 + e)
        p = t * np.float32(1.0 + e)
        assert F(float(p)) - F(float(t)) * F(1.0 + e) == want
    assert int(oracle.f32_to_f16(np.array([-(2.0 ** -33)], np.float32))[0]) == 0x8000
    assert int(oracle.f32_to_bf16(np.array([-(2.0 ** -30)], np.float32))[0]) == 0xB080


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_gemm_seq_16_matches_a_numpy_restatement_on_strided_views(kind):
    """The C loop against an independent numpy evaluation of the same arithmetic (f32
    elementwise products and sums, k ascending) on random data with transposed A and B,
    bit for bit."""
    g = np.random.default_rng(7 + (kind == "bf16"))
    m, k, n = 23, 41, 19
    alpha, beta = float(np.float32(1.0 / 3.0)), float(np.float32(-0.7))

    def rand16(shape):
        x = g.uniform(-2, 2, shape).astype(np.float32)
        return oracle.f32_to_f16(x) if kind == "f16" else oracle.f32_to_bf16(x)
    a = rand16((k, m)).T          # strides (1, m)
    b = rand16((n, k)).T          # strides (1, k)
    c = rand16((m, n))
    got = oracle.gemm_seq_16(kind, alpha, beta, a, b, c)
    widen = (lambda h: h.view(np.float16).astype(np.float32)) if kind == "f16" else oracle.bf16_to_f32
    a32, b32 = widen(np.ascontiguousarray(a)), widen(np.ascontiguousarray(b))
    acc = np.float32(beta) * widen(c)
    for t in range(k):
        acc = acc + (np.float32(alpha) * a32[:, t:t + 1]) * b32[t:t + 1, :]
    want = acc.astype(np.float16).view(np.uint16) if kind == "f16" else oracle.f32_to_bf16(acc)
    assert np.array_equal(got, want)
