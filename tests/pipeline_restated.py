"""Test restatement of the reference's pipeline driver over the HIP backend.

crates/pipeline/src/lib.rs evaluates no math: every product and activation goes through a
`Backend`, every stage boundary through a `Transport`. This module restates, for the tests,
that driver (`train`, `contiguous_placement`, `send_tensor`, `recv_tensor`), the 1F1B op order
of crates/schedule/src/lib.rs (`local_order`) and the in-process loopback transport, so several
ranks -- each a thread with its own HipBackend context on the one GPU -- can run a pipelined
step whose boundary tensors cross as LNGL wire messages written straight from device memory
(`lg_wire_encode_tensor`) and read straight back into it (`lg_wire_decode_into`).
"""
from __future__ import annotations

import queue
from typing import List, Optional, Sequence

from linalg_hip import backend as B
from linalg_hip import wire

RECV_TIMEOUT = 5.0  # seconds (crates/pipeline/src/lib.rs:19)


def schedule_error(msg: str) -> B.BackendError:
    return B.BackendError("Schedule", msg)


def local_order(stages: int, rank: int, microbatches: int) -> List[tuple]:
    """1F1B order for one rank (crates/schedule/src/lib.rs:15-35): min(stages - rank - 1, M)
    warm-up forwards, then forward/backward pairs, then the remaining backwards."""
    if stages == 0 or rank >= stages or microbatches == 0 or microbatches > 0xFFFFFFFF:
        raise schedule_error("bad stages, rank or microbatch count")
    m = microbatches
    warmup = min(stages - rank - 1, m)
    steady = m - warmup
    out = [("F", i) for i in range(warmup)]
    for i in range(steady):
        out += [("F", warmup + i), ("B", i)]
    out += [("B", i) for i in range(steady, m)]
    return out


def contiguous_placement(layers: int, stages: int) -> List[int]:
    """owners[layer] = rank; rank r owns floor(L/S) + 1 layers when r < L mod S
    (crates/pipeline/src/lib.rs:28-40)."""
    if stages == 0 or layers == 0 or stages > layers:
        raise schedule_error("bad layer or stage count")
    base, extra = divmod(layers, stages)
    owners: List[int] = []
    for rank in range(stages):
        owners += [rank] * (base + (1 if rank < extra else 0))
    return owners


class Loopback:
    """In-process transport: one FIFO per ordered rank pair, byte messages."""

    def __init__(self, world: int):
        self.world = world
        self.queues = {(s, d): queue.Queue() for s in range(world) for d in range(world) if s != d}

    def endpoint(self, rank: int) -> "Endpoint":
        return Endpoint(self, rank)


class Endpoint:
    def __init__(self, hub: Loopback, rank: int):
        self.hub, self.rank = hub, rank
        self.sent: List[int] = []  # byte length of each message sent

    def send(self, dest: int, message: bytes) -> None:
        self.sent.append(len(message))
        self.hub.queues[(self.rank, dest)].put(bytes(message))

    def recv_timeout(self, src: int, timeout: float) -> bytes:
        try:
            return self.hub.queues[(src, self.rank)].get(timeout=timeout)
        except queue.Empty:
            raise B.BackendError("Transport", f"rank {self.rank}: nothing from {src}") from None


def check_matrix(t: B.Tensor) -> None:
    if t.dtype != B.DType.F32:
        raise B.BackendError("Dtype", "boundary tensors are f32")
    if len(t.shape) != 2 or t.offset != 0 or list(t.strides) != B.row_major_strides(t.shape):
        raise B.BackendError("Shape", "not a row-major matrix at offset 0")


def send_tensor(hb: B.HipBackend, transport: Endpoint, dest: int, t: B.Tensor) -> None:
    """download + encode_wire (crates/pipeline/src/lib.rs:71-80), one device-to-host copy."""
    transport.send(dest, wire.encode_tensor(hb, t))


def recv_tensor(hb: B.HipBackend, transport: Endpoint, src: int, rows: Optional[int],
                cols: int) -> B.Tensor:
    """decode_wire + upload (crates/pipeline/src/lib.rs:82-98), one host-to-device copy."""
    message = transport.recv_timeout(src, RECV_TIMEOUT)
    dtype, shape, _ = wire.parse_header(message)
    if dtype != B.DType.F32:
        raise B.BackendError("Dtype", "boundary tensors are f32")
    if len(shape) != 2 or shape[1] != cols or (rows is not None and rows != shape[0]):
        raise B.BackendError("Shape", "boundary shape differs")
    t = hb.alloc(B.DType.F32, shape)
    wire.decode_into(hb, message, t)
    return t


def train(hb: B.HipBackend, transport: Endpoint, owners: Sequence[int], microbatches: int,
          weights: Sequence[B.Tensor], inputs: Sequence[B.Tensor], dy: Sequence[B.Tensor]):
    """pipeline::train (crates/pipeline/src/lib.rs:100-230) on this rank: returns (y, dw)."""
    if not owners or owners[0] != 0 or any(b not in (a, a + 1) for a, b in zip(owners, owners[1:])):
        raise schedule_error("owners must be contiguous from rank 0")
    stages = owners[-1] + 1
    rank = transport.rank
    if transport.hub.world != stages or rank >= stages:
        raise schedule_error("transport world differs from the placement")
    order = local_order(stages, rank, microbatches)
    count = sum(1 for o in owners if o == rank)
    if len(weights) != count or count == 0:
        raise schedule_error("weights differ from the owned layers")
    is_first, is_last = rank == 0, rank + 1 == stages
    if len(inputs) != (microbatches if is_first else 0) or len(dy) != (microbatches if is_last else 0):
        raise schedule_error("inputs or dy on the wrong rank")
    for w in weights:
        check_matrix(w)
    if any(a.shape[1] != b.shape[0] for a, b in zip(weights, weights[1:])):
        raise B.BackendError("Shape", "layer widths do not chain")
    n_in, n_out = weights[0].shape[0], weights[-1].shape[1]
    for x in inputs:
        check_matrix(x)
        if x.shape[1] != n_in:
            raise B.BackendError("Shape", "input width")
    for g in dy:
        check_matrix(g)
        if g.shape[1] != n_out:
            raise B.BackendError("Shape", "dy width")

    dw = [hb.alloc(B.DType.F32, w.shape) for w in weights]  # zeroed; accumulated with beta = 1
    y: List[B.Tensor] = []
    saved = [None] * microbatches
    for kind, m in order:
        if kind == "F":
            received = None if is_first else recv_tensor(hb, transport, rank - 1, None, n_in)
            x0 = received if received is not None else inputs[m]
            batch = x0.shape[0]
            if is_last and dy[m].shape[0] != batch:
                raise B.BackendError("Shape", "dy batch")
            pre_all, act_all = [], []
            for l, w in enumerate(weights):
                x = act_all[-1] if act_all else x0
                n = w.shape[1]
                pre = hb.alloc(B.DType.F32, [batch, n])
                hb.gemm(x, w, pre, 1.0, 0.0)
                act = hb.alloc(B.DType.F32, [batch, n])
                hb.gelu(pre, act)
                pre_all.append(pre)
                if l + 1 < count:
                    act_all.append(act)
                elif is_last:
                    y.append(act)
                else:
                    send_tensor(hb, transport, rank + 1, act)
            saved[m] = (received, pre_all, act_all)
        else:
            if saved[m] is None:
                raise schedule_error("backward before forward")
            received, pre_all, act_all = saved[m]
            saved[m] = None
            batch = pre_all[0].shape[0]
            owned = None if is_last else recv_tensor(hb, transport, rank + 1, batch, n_out)
            for l in range(count - 1, -1, -1):
                g = owned if owned is not None else dy[m]
                k, n = weights[l].shape
                dpre = hb.alloc(B.DType.F32, [batch, n])
                hb.gelu_backward(pre_all[l], g, dpre)
                x = (received if received is not None else inputs[m]) if l == 0 else act_all[l - 1]
                hb.gemm(B.transpose_matrix(x), dpre, dw[l], 1.0, 1.0)
                dx = hb.alloc(B.DType.F32, [batch, k])
                hb.gemm(dpre, B.transpose_matrix(weights[l]), dx, 1.0, 0.0)
                if l == 0 and not is_first:
                    send_tensor(hb, transport, rank - 1, dx)
                owned = dx
    return y, dw
