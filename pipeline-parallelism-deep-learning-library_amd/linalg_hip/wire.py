"""The "LNGL" wire format of stage boundaries (crates/core/src/lib.rs:298-412).

`write_header`, `parse_header`, `encode`, `decode` mirror write_wire_header,
parse_wire_header, encode_wire and decode_wire; `encode_tensor` and `decode_into` are the
device-buffer ends of a boundary (send_tensor / recv_tensor, crates/pipeline/src/lib.rs:71-98),
each one direct copy between a HipBackend tensor and the wire bytes. Errors raise
`backend.BackendError` with the reference's `Wire` / `Shape` / `Dtype` kinds.
"""
from __future__ import annotations

import ctypes
from typing import List, Sequence, Tuple

from . import _native as N
from .backend import BackendError, DType, HipBackend, Tensor, _raise

WIRE_MAGIC = b"LNGL"
WIRE_VERSION = 1
WIRE_HEADER_MAX = N.LG_WIRE_HEADER_MAX


def _shape(shape: Sequence[int]):
    if any(int(e) < 0 or int(e) >= 2 ** 64 for e in shape):
        raise BackendError("Shape", "extent does not fit 64 bits")
    return (ctypes.c_uint64 * max(len(shape), 1))(*[int(e) for e in shape])


def write_header(dtype: int, shape: Sequence[int]) -> bytes:
    out = (ctypes.c_uint8 * WIRE_HEADER_MAX)()
    n = ctypes.c_uint64()
    _raise(N.lib().lg_wire_write_header(int(dtype), _shape(shape), len(shape), out,
                                        ctypes.byref(n)))
    return bytes(out[: n.value])


def parse_header(message: bytes) -> Tuple[DType, List[int], int]:
    buf = ctypes.create_string_buffer(bytes(message), max(len(message), 1))
    dt, rank, off = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
    shape = (ctypes.c_uint64 * 8)()
    _raise(N.lib().lg_wire_parse_header(buf, len(message), ctypes.byref(dt), shape,
                                        ctypes.byref(rank), ctypes.byref(off)))
    return DType(dt.value), [int(shape[i]) for i in range(rank.value)], off.value


def encode(dtype: int, shape: Sequence[int], payload: bytes) -> bytes:
    payload = bytes(payload)
    cap = WIRE_HEADER_MAX + len(payload)
    out = ctypes.create_string_buffer(cap)
    n = ctypes.c_uint64()
    src = ctypes.create_string_buffer(payload, max(len(payload), 1))
    _raise(N.lib().lg_wire_encode(int(dtype), _shape(shape), len(shape), src, len(payload), out,
                                  cap, ctypes.byref(n)))
    return out.raw[: n.value]


def decode(message: bytes) -> Tuple[DType, List[int], bytes]:
    dtype, shape, off = parse_header(message)
    return dtype, shape, bytes(message[off:])


def encode_tensor(hb: HipBackend, t: Tensor) -> bytes:
    """download + encode_wire in one device-to-host copy into the message buffer."""
    cap = WIRE_HEADER_MAX + t.numel() * t.dtype.size_of()
    out = ctypes.create_string_buffer(max(cap, 1))
    n = ctypes.c_uint64()
    _raise(N.lib().lg_wire_encode_tensor(hb.ctx.handle, ctypes.byref(t.to_c()), out, cap,
                                         ctypes.byref(n)))
    return out.raw[: n.value]


def decode_into(hb: HipBackend, message: bytes, t: Tensor) -> None:
    """decode_wire + upload_into an existing tensor in one host-to-device copy."""
    buf = ctypes.create_string_buffer(bytes(message), max(len(message), 1))
    _raise(N.lib().lg_wire_decode_into(hb.ctx.handle, buf, len(message), ctypes.byref(t.to_c())))
