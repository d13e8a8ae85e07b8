"""Pins the oracle's restatement of the CpuBackend activation and training ops (CPU only).

Each check is one the reference itself makes, or one the mathematics fixes:
* the A&S 7.1.26 constants carry the bit patterns crates/cpu/src/lib.rs:846-853 asserts;
* GELU and its derivative lie within 1e-6 of the normal-cdf definition on the reference's
  sample list (crates/cpu/src/invariants.rs:462-500), here against math.erf in f64;
* add_bias / bias_grad / mse_grad / sgd_step equal the sequential f32 loops and lie within
  1e-6 of f64 (crates/cpu/src/training.rs:93-217), including the known answers of
  `every_v2_method_is_implemented_on_cpu` (:72-91);
* f32 -> bf16 is the nearest bf16 by f64 distance, ties to even, on the reference's case list
  (:219-270), NaN stays a quiet NaN of the same sign, and bf16 -> f32 is exact on all 65536
  patterns.
Planted mistakes (a dropped erf term, f64 accumulation, truncating conversion) fail them.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle

SAMPLES = [i * 0.25 for i in range(-24, 25)] + [4.75, -4.75, 8.0, -8.0, 1.0e-4, -1.0e-3]


def f32(v):
    return np.asarray(v, dtype=np.float32)


def pattern(count: int, seed: int) -> np.ndarray:
    """crates/cpu/src/training.rs:32-34."""
    i = np.arange(count)
    return f32(((i * 17 + seed * 31 + 3) % 101).astype(np.float32) / np.float32(101.0) - np.float32(0.5))


def gelu_ref(x: float) -> float:
    return 0.5 * x * (1.0 + math.erf(x / math.sqrt(2.0)))


def gelu_prime_ref(x: float) -> float:
    phi = 0.5 * (1.0 + math.erf(x / math.sqrt(2.0)))
    return phi + x * math.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)


def test_erf_constants_have_the_asserted_bits():
    assert oracle.erf_constants() == [0x3E827906, 0x3E91A98E, 0x3FB5F0E3, 0x3FBA00E3,
                                      0x3F87DC22, 0x3ECC422A]


def test_gelu_and_backward_match_the_normal_cdf_definition_within_1e_6():
    x = f32(SAMPLES)
    y = oracle.gelu(x)
    for got, s in zip(y, x):
        assert abs(float(got) - gelu_ref(float(s))) <= 1e-6, (s, got)
    dy = f32([s * 0.5 - 0.25 for s in SAMPLES])
    dx = oracle.gelu_backward(x, dy)
    for got, s, g in zip(dx, x, dy):
        assert abs(float(got) - float(g) * gelu_prime_ref(float(s))) <= 1e-6, (s, got)
    # Closed forms: GELU(0) = 0, GELU(-0) = -0 * 0.5 * (1 + erf(-0)) keeps the sign of zero,
    # GELU'(0) = 1/2.
    assert oracle.gelu(f32([0.0]))[0] == 0.0
    assert oracle.gelu_backward(f32([0.0]), f32([1.0]))[0] == np.float32(0.5)


def test_a_planted_erf_mistake_fails_the_definition_check():
    # The same series with the a5 term dropped misses the definition by far more than 1e-6.
    def bad_erf(z):
        a = abs(z)
        t = 1.0 / (1.0 + 0.3275911 * a)
        poly = ((((-1.4531521) * t + 1.4214138) * t - 0.28449672) * t + 0.2548296) * t
        return math.copysign(1.0 - poly * math.exp(-a * a), z)

    worst = max(abs(0.5 * s * (1.0 + bad_erf(s / math.sqrt(2.0))) - gelu_ref(s)) for s in SAMPLES)
    assert worst > 1e-3


def test_every_v2_method_known_answers():
    # crates/cpu/src/training.rs:72-91, in the same order.
    x = f32([[1, 2, 3], [4, 5, 6]])
    b = f32([0.5, -0.5, 1.0])
    y = oracle.add_bias(x, b)
    db = oracle.bias_grad(y, np.zeros(3, np.float32))
    dy, loss = oracle.mse_grad(y, np.zeros((2, 3), np.float32))
    w, db2 = oracle.sgd_step(f32([1, 1, 1]), db, 0.5)
    h = oracle.f32_to_bf16(y)
    back = oracle.bf16_to_f32(h)
    assert back.ravel().tolist() == [1.5, 1.5, 4.0, 4.5, 4.5, 7.0]
    assert db2.tolist() == [0.0, 0.0, 0.0]
    assert w.tolist() == [1.0 - 0.5 * 6.0, 1.0 - 0.5 * 6.0, 1.0 - 0.5 * 11.0]
    assert loss > 0.0


def test_add_bias_and_bias_grad_are_the_sequential_loops():
    rows, cols = 7, 33
    xs, bs = pattern(rows * cols, 1).reshape(rows, cols), pattern(cols, 2)
    y = oracle.add_bias(xs, bs)
    assert np.array_equal(y, xs + bs[None, :])
    assert np.max(np.abs(y.astype(np.float64) - (xs.astype(np.float64) + bs))) <= 1e-6
    rows, cols = 64, 37
    ds, seed = pattern(rows * cols, 3).reshape(rows, cols), pattern(cols, 4)
    got = oracle.bias_grad(ds, seed)
    s = np.zeros(cols, np.float32)
    for i in range(rows):
        s = s + ds[i]  # f32, rows in order
    assert np.array_equal(got, seed + s)
    want = seed.astype(np.float64) + ds.astype(np.float64).sum(axis=0)
    assert np.max(np.abs(got - want)) <= 1e-6
    # B = 0 leaves db unchanged.
    assert np.array_equal(oracle.bias_grad(np.zeros((0, cols), np.float32), got), got)
    # f64 accumulation (a planted mistake) differs in the bits somewhere.
    wide = (seed.astype(np.float64) + ds.astype(np.float64).sum(axis=0)).astype(np.float32)
    assert not np.array_equal(wide, got) or rows < 2


def test_mse_grad_is_the_sequential_loop():
    rows, cols = 8, 65
    n = rows * cols
    ys, ts = pattern(n, 5).reshape(rows, cols), pattern(n, 6).reshape(rows, cols)
    dy, loss = oracle.mse_grad(ys, ts)
    d = ys.astype(np.float64) - ts.astype(np.float64)
    assert np.max(np.abs(dy - 2.0 * d / n)) <= 1e-6
    assert abs(float(loss) - float((d * d).sum() / n)) <= 1e-6
    total = np.float32(0.0)
    for a, b in zip(ys.ravel(), ts.ravel()):
        total = np.float32(total + (a - b) * (a - b))
    assert loss == np.float32(total / np.float32(n))
    dd = (ys - ts)
    assert np.array_equal(dy, (np.float32(2.0) * dd) / np.float32(n))
    dz, lz = oracle.mse_grad(ts, ts)
    assert lz == 0.0 and not dz.any()


def test_sgd_step_updates_and_zeroes():
    ws, gs = pattern(300, 7).reshape(10, 30), pattern(300, 8).reshape(10, 30)
    lr = np.float32(1e-3)
    w, dw = oracle.sgd_step(ws, gs, lr)
    assert np.array_equal(w, ws - lr * gs)
    assert np.max(np.abs(w.astype(np.float64) - (ws.astype(np.float64) - float(lr) * gs.astype(np.float64)))) <= 1e-6
    assert not dw.view(np.uint32).any()


def bf16_nearest_f64(x: np.float32) -> int:
    """crates/cpu/src/training.rs:54-71, restated."""
    bits = int(np.float32(x).view(np.uint32))
    low = bits >> 16
    high = (low + 1) & 0xFFFF

    def value(h):
        if h & 0x7FFF == 0x7F80:
            return (-1.0 if h & 0x8000 else 1.0) * 2.0 ** 128
        return float(np.uint32(h << 16).view(np.float32))
    xv = float(x)
    dl, dh = abs(xv - value(low)), abs(value(high) - xv)
    if bits & 0xFFFF == 0 or dl < dh or (dl == dh and low & 1 == 0):
        return low
    return high


def test_f32_to_bf16_rounds_to_nearest_even_and_keeps_specials():
    bits = [0x00000000, 0x80000000, 0x3F800000, 0x3F808000, 0x3F818000, 0x3F808001, 0x3F807FFF,
            0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F7FFF, 0x7F800000, 0xFF800000, 0x00010000, 0x80018000,
            0x00000001]
    cases = np.concatenate([np.asarray(bits, np.uint32).view(np.float32), pattern(1000, 9) * np.float32(1e3)])
    got = oracle.f32_to_bf16(cases)
    for v, g in zip(cases, got):
        want = int(v.view(np.uint32)) >> 16 if np.isinf(v) else bf16_nearest_f64(v)
        assert int(g) == want, hex(int(v.view(np.uint32)))
    assert got[7] == 0x7F80 and got[8] == 0xFF80 and got[12] == 0x0001
    nans = np.asarray([0x7F800001, 0xFF800001, 0x7FC00000, 0xFFFFFFFF, 0x7F812345], np.uint32)
    for b, g in zip(nans, oracle.f32_to_bf16(nans.view(np.float32))):
        g = int(g)
        assert g & 0x7F80 == 0x7F80 and g & 0x007F and g & 0x0040
        assert g & 0x8000 == (int(b) >> 16) & 0x8000
    # Truncation (a planted mistake) disagrees on the tie-above case.
    assert (0x3F818000 >> 16) != int(got[4])


def test_bf16_to_f32_is_exact_on_every_pattern():
    h = np.arange(65536, dtype=np.uint16)
    f = oracle.bf16_to_f32(h)
    assert np.array_equal(f.view(np.uint32), h.astype(np.uint32) << 16)
