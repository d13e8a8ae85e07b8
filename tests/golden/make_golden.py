"""Writes the golden fixtures of the contraction / permutation oracle.

Nothing here runs or imports the reference. Every vector is transcribed from a
known-answer test the reference's own test suite states explicitly:

cpu_gemm_kats.json  <- crates/cpu/src/invariants.rs:137-243 (f32 gemm, three layouts)
  * [1,2;3,4].[5,6;7,8] = [19,22;43,50]                                    (:137-147)
  * alpha=-0.5, beta=0.25, C0=[1,-2;0.5,4]; C[0,0] is written out there as
    0.25*1 + (-0.5*1)*5 + (-0.5*2)*7; the other three entries are the same dyadic
    arithmetic by hand (every intermediate is exact in f32)                (:149-158)
  * [2^25, 1, -2^25].[1,1,1] = +0 in k order (f64 or cancel-first gives 1)  (:160-180)
  * alpha=1e20, A=[1e-20], B=[1e-20]: (alpha*a)*b, left association       (:182-187)
  * beta=0 ignores NaN in C: [2,3].[4;5] = 23                               (:190-200)
  * alpha=0, beta=2 ignores NaN operands: C=[3,-4] -> [6,-8]                (:202-208)
  * alpha=0, beta=0 with NaN everywhere -> zeros                           (:210-217)
  * K=0, beta=0, alpha=1.5, NaN C -> zeros; K=0, alpha=4, beta=2 -> [3,-6] (:219-243)
permutation_kats.json <- tests/permutation_test.rs
  * SPECIALS bit patterns                                                  (:20-34)
  * view-path metadata of permute_view                                    (:229-245)
  * rejected non-permutations                                             (:263-282)
  * complex adjoint word table, m=2, n=3                                   (:464-492)
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def f32(x: float) -> float:
    return float(np.float32(x))


def gemm_kats() -> list:
    nan = 0x7fc01234
    snan = 0x7f800011
    kats = []
    kats.append({"name": "2x2 sequential", "m": 2, "k": 2, "n": 2, "alpha": 1.0, "beta": 0.0,
                 "a": [bits(v) for v in [1, 2, 3, 4]], "b": [bits(v) for v in [5, 6, 7, 8]],
                 "c0": [bits(0.0)] * 4, "expected": [bits(v) for v in [19, 22, 43, 50]],
                 "source": "crates/cpu/src/invariants.rs:137-147"})
    # The written-out C[0,0] of invariants.rs:153-157, evaluated with one f32 rounding per op.
    a32 = np.float32
    acc = a32(0.25) * a32(1.0)
    acc = a32(acc + (a32(-0.5) * a32(1.0)) * a32(5.0))
    acc = a32(acc + (a32(-0.5) * a32(2.0)) * a32(7.0))
    assert float(acc) == -9.25
    kats.append({"name": "alpha beta", "m": 2, "k": 2, "n": 2, "alpha": -0.5, "beta": 0.25,
                 "a": [bits(v) for v in [1, 2, 3, 4]], "b": [bits(v) for v in [5, 6, 7, 8]],
                 "c0": [bits(v) for v in [1, -2, 0.5, 4]],
                 "expected": [bits(v) for v in [-9.25, -11.5, -21.375, -24.0]],
                 "source": "crates/cpu/src/invariants.rs:149-158"})
    big = 33554432.0
    kats.append({"name": "2^25 cancellation in k order", "m": 1, "k": 3, "n": 1, "alpha": 1.0,
                 "beta": 0.0, "a": [bits(big), bits(1.0), bits(-big)],
                 "b": [bits(1.0)] * 3, "c0": [0], "expected": [0],
                 "source": "crates/cpu/src/invariants.rs:160-180"})
    left = (a32(1e20) * a32(1e-20)) * a32(1e-20)
    right = a32(1e20) * (a32(1e-20) * a32(1e-20))
    assert bits(float(left)) != bits(float(right))
    kats.append({"name": "left association", "m": 1, "k": 1, "n": 1, "alpha": f32(1e20),
                 "beta": 0.0, "a": [bits(1e-20)], "b": [bits(1e-20)], "c0": [0],
                 "expected": [bits(float(left))], "not_expected": [bits(float(right))],
                 "source": "crates/cpu/src/invariants.rs:182-187"})
    kats.append({"name": "beta 0 ignores NaN in C", "m": 1, "k": 2, "n": 1, "alpha": 1.0,
                 "beta": 0.0, "a": [bits(2.0), bits(3.0)], "b": [bits(4.0), bits(5.0)],
                 "c0": [nan], "expected": [bits(23.0)],
                 "source": "crates/cpu/src/invariants.rs:190-200"})
    kats.append({"name": "alpha 0 ignores NaN operands", "m": 1, "k": 2, "n": 2, "alpha": 0.0,
                 "beta": 2.0, "a": [nan, snan], "b": [nan] * 4, "c0": [bits(3.0), bits(-4.0)],
                 "expected": [bits(6.0), bits(-8.0)],
                 "source": "crates/cpu/src/invariants.rs:202-208"})
    kats.append({"name": "alpha 0 beta 0 never reads", "m": 2, "k": 2, "n": 2, "alpha": 0.0,
                 "beta": 0.0, "a": [nan] * 4, "b": [nan] * 4, "c0": [nan] * 4,
                 "expected": [0] * 4, "source": "crates/cpu/src/invariants.rs:210-217"})
    kats.append({"name": "K 0 beta 0 stores zeros", "m": 2, "k": 0, "n": 3, "alpha": 1.5,
                 "beta": 0.0, "a": [], "b": [], "c0": [0x7fa000ab] * 6, "expected": [0] * 6,
                 "source": "crates/cpu/src/invariants.rs:219-233"})
    kats.append({"name": "K 0 beta 2 scales", "m": 1, "k": 0, "n": 2, "alpha": 4.0, "beta": 2.0,
                 "a": [], "b": [], "c0": [bits(1.5), bits(-3.0)],
                 "expected": [bits(3.0), bits(-6.0)],
                 "source": "crates/cpu/src/invariants.rs:235-243"})
    return kats


def permutation_kats() -> dict:
    specials = [0x00000000, 0x80000000, 0x7f800000, 0xff800000, 0x7fc00000, 0xffc00000,
                0x7fc00001, 0xffc12345, 0x7f800001, 0xff800007, 0x00000001, 0x80000001]
    rejects = [[0, 0, 1], [0, 1], [0, 1, 2, 3], [0, 1, 3], [3, 1, 0], [2 ** 64 - 1, 0, 1], [],
               [1, 1, 1]]
    words = [[0x00000000, 0x00000000], [0x80000000, 0x80000000], [0x7fc00001, 0x7fc00001],
             [0x7f800000, 0xff800000], [0x3f800000, 0x00000001], [0xffc12345, 0x7f800001]]
    m, n = 2, 3
    adj = [0] * (2 * m * n)
    for i in range(m):
        for j in range(n):
            re, im = words[i * n + j]
            at = 2 * (j * m + i)
            adj[at] = re
            adj[at + 1] = im ^ 0x80000000
    return {
        "specials": specials,
        "view_path": {"offset": 5, "shape": [2, 3, 4], "strides": [12, 4, 1], "perm": [2, 0, 1],
                      "want_shape": [4, 2, 3], "want_strides": [1, 12, 4],
                      "index_of": [3, 1, 2], "equals_source_index_of": [1, 2, 3],
                      "source": "tests/permutation_test.rs:229-245"},
        "rejected_perms": {"shape": [2, 3, 4], "perms": rejects,
                           "source": "tests/permutation_test.rs:263-282"},
        "complex_adjoint": {"m": m, "n": n, "input_words": [w for p in words for w in p],
                            "adjoint_words": adj, "source": "tests/permutation_test.rs:464-492"},
    }


def main() -> None:
    (HERE / "cpu_gemm_kats.json").write_text(json.dumps(gemm_kats(), indent=1) + "\n")
    (HERE / "permutation_kats.json").write_text(json.dumps(permutation_kats(), indent=1) + "\n")


if __name__ == "__main__":
    main()
