"""Pipelined training steps through the HIP backend: several ranks, each a thread with its
own backend context on the one GPU, exchange boundary tensors as LNGL wire messages written
from and read into device memory (crates/pipeline/tests/pipeline.rs:296-640, restated).

The math of a layer does not depend on where the pipeline is cut, so every split must give
the single-rank result bit for bit; the boundary messages must have the activation's wire
size; every rank must launch exactly 3 GEMMs, one GELU and one GELU backward per owned layer
and microbatch; weights are left untouched."""
from __future__ import annotations

import threading

import numpy as np
import pytest

from linalg_hip import backend as B
from pipeline_restated import Loopback, contiguous_placement, train
from test_training_gpu import DY0, DY1, WIDTHS, X0, X1, up, weight

pytestmark = pytest.mark.gpu

BATCH = 2
LAYERS = 3


def run_rank(hub: Loopback, rank: int, stages: int, order, out: dict) -> None:
    hb = B.HipBackend(0)
    try:
        ep = hub.endpoint(rank)
        owners = contiguous_placement(LAYERS, stages)
        layers = [l for l in range(LAYERS) if owners[l] == rank]
        weights = [up(hb, weight(l)) for l in layers]
        xs = [np.array(X0 if i == 0 else X1, np.float32).reshape(BATCH, WIDTHS[0]) for i in order]
        dys = [np.array(DY0 if i == 0 else DY1, np.float32).reshape(BATCH, WIDTHS[LAYERS])
               for i in order]
        inputs = [up(hb, x) for x in xs] if rank == 0 else []
        dy = [up(hb, g) for g in dys] if rank + 1 == stages else []
        start = len(hb.debug_launches())
        y, dw = train(hb, ep, owners, len(order), weights, inputs, dy)
        out[rank] = {
            "y": [hb.download_f32(t).tobytes() for t in y],
            "dw": [hb.download_f32(t).tobytes() for t in dw],
            "launches": hb.debug_launches()[start:],
            "sent": list(ep.sent),
            "layers": layers,
            "weights_after": [hb.download_f32(w).tobytes() for w in weights],
        }
    except BaseException as e:  # reported by the caller
        out[rank] = e
    finally:
        hb.close()


def run(stages: int, order=(0, 1)):
    hub = Loopback(stages)
    out: dict = {}
    threads = [threading.Thread(target=run_rank, args=(hub, r, stages, list(order), out))
               for r in range(stages)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a rank did not finish"
    for r in range(stages):
        if isinstance(out[r], BaseException):
            raise out[r]
    return [out[r] for r in range(stages)]


def gather(ranks):
    return ranks[-1]["y"], [d for r in ranks for d in r["dw"]]


def assert_full_shape(y, dw, m):
    assert len(y) == m and all(len(b) == BATCH * WIDTHS[LAYERS] * 4 for b in y)
    assert len(dw) == LAYERS
    for l, b in enumerate(dw):
        assert len(b) == WIDTHS[l] * WIDTHS[l + 1] * 4


@pytest.mark.parametrize("stages", [2, 3])
def test_ranks_on_loopback_equal_a_single_rank_bit_for_bit(stages):
    sy, sdw = gather(run(1))
    assert_full_shape(sy, sdw, 2)
    y, dw = gather(run(stages))
    assert_full_shape(y, dw, 2)
    assert y == sy and dw == sdw


def test_longer_schedule_with_repeated_microbatches():
    order = (0, 1, 1, 0, 1)
    sy, sdw = gather(run(1, order))
    y, dw = gather(run(3, order))
    assert y == sy and dw == sdw


def test_launch_counts_and_boundary_sizes():
    m = 2

    def wire_len(width):
        return 16 + 4 * 2 + BATCH * width * 4

    for stages in (1, 2, 3):
        ranks = run(stages)
        assert sum(len(r["layers"]) for r in ranks) == LAYERS
        for rank, r in enumerate(ranks):
            l = len(r["layers"])
            names = r["launches"]
            gemms = sum(1 for n in names if n.startswith("gemm_f32"))
            assert gemms == 3 * l * m, (stages, rank, names)
            assert names.count("gelu_f32") == l * m
            assert names.count("gelu_backward_f32") == l * m
            assert len(names) == 5 * l * m, (stages, rank, names)
            links = (rank > 0) + (rank + 1 < stages)
            assert len(r["sent"]) == links * m
            for i, lay in enumerate(r["layers"]):
                assert r["weights_after"][i] == weight(lay).tobytes()
    # Placement [0, 1, 2]: forward boundaries carry widths 4 and 2, backward ones the input
    # widths of layers 1 and 2 (4 and 2).
    ranks = run(3)
    want = [[wire_len(WIDTHS[1])] * m,
            sorted([wire_len(WIDTHS[2])] * m + [wire_len(WIDTHS[1])] * m),
            [wire_len(WIDTHS[2])] * m]
    assert [sorted(r["sent"]) for r in ranks] == want

