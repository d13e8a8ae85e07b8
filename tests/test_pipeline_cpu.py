"""The pipeline driver's host logic, restated for the tests (tests/pipeline_restated.py):
the 1F1B order against the case list of crates/schedule/src/lib.rs:40-180 and the contiguous
placement against crates/pipeline/tests/pipeline.rs:485-515. No GPU."""
from __future__ import annotations

import pytest

from linalg_hip import backend as B
from pipeline_restated import contiguous_placement, local_order


def f(i):
    return ("F", i)


def b(i):
    return ("B", i)


@pytest.mark.parametrize("stages,rank,m,want", [
    (1, 0, 3, [f(0), b(0), f(1), b(1), f(2), b(2)]),
    (2, 0, 4, [f(0), f(1), b(0), f(2), b(1), f(3), b(2), b(3)]),
    (2, 1, 4, [f(0), b(0), f(1), b(1), f(2), b(2), f(3), b(3)]),
    (3, 0, 4, [f(0), f(1), f(2), b(0), f(3), b(1), b(2), b(3)]),
    (3, 1, 4, [f(0), f(1), b(0), f(2), b(1), f(3), b(2), b(3)]),
    (3, 2, 4, [f(0), b(0), f(1), b(1), f(2), b(2), f(3), b(3)]),
    (3, 0, 1, [f(0), b(0)]),
    (4, 0, 2, [f(0), f(1), b(0), b(1)]),
])
def test_local_order_matches_the_reference_cases(stages, rank, m, want):
    assert local_order(stages, rank, m) == want


def test_local_order_rejections():
    for args in [(0, 0, 1), (2, 2, 1), (2, 3, 1), (3, 0, 0), (1, 0, 2 ** 32)]:
        with pytest.raises(B.BackendError) as e:
            local_order(*args)
        assert e.value.kind == "Schedule"


def test_local_order_counts_relative_order_and_interleaving():
    for stages in range(1, 6):
        for rank in range(stages):
            for m in range(1, 9):
                order = local_order(stages, rank, m)
                assert [i for k, i in order if k == "F"] == list(range(m))
                assert [i for k, i in order if k == "B"] == list(range(m))
                for mb in range(m):
                    assert order.index(f(mb)) < order.index(b(mb))
                # An F follows the first B exactly when the steady phase has two pairs.
                first_b = next(i for i, op in enumerate(order) if op[0] == "B")
                w = stages - rank - 1
                assert any(op[0] == "F" for op in order[first_b + 1:]) == (m > w + 1)


def test_placement_examples_and_rejections():
    assert contiguous_placement(5, 3) == [0, 0, 1, 1, 2]
    assert contiguous_placement(3, 3) == [0, 1, 2]
    assert contiguous_placement(3, 1) == [0, 0, 0]
    assert contiguous_placement(3, 2) == [0, 0, 1]
    assert contiguous_placement(7, 3) == [0, 0, 0, 1, 1, 2, 2]
    assert contiguous_placement(4, 2) == [0, 0, 1, 1]
    for layers, stages in [(0, 1), (1, 0), (0, 0), (2, 3)]:
        with pytest.raises(B.BackendError) as e:
            contiguous_placement(layers, stages)
        assert e.value.kind == "Schedule"
    for stages in range(1, 7):
        for layers in range(stages, 13):
            o = contiguous_placement(layers, stages)
            assert len(o) == layers
            assert all(0 <= y - x <= 1 for x, y in zip(o, o[1:]))
            for r in range(stages):
                assert o.count(r) == layers // stages + (1 if r < layers % stages else 0)
