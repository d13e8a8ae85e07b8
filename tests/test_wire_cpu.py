"""The "LNGL" wire format on the host: restates crates/core/tests/invariants.rs:111-240 and
crates/core/tests/additions.rs:15-110 (golden bytes, round trips, every rejection and which
error it is)."""
from __future__ import annotations

import struct

import pytest

from linalg_hip import wire as W
from linalg_hip.backend import BackendError, DType

F32_SCALAR = b"LNGL" + bytes([1, 0, 0, 0, 1, 0, 0, 0, 1, 0, 0, 0, 1, 0, 0, 0, 0x11, 0x22, 0x33, 0x44])
F16_MATRIX = (b"LNGL" + bytes([1, 0, 0, 0, 2, 0, 0, 0, 2, 0, 0, 0, 2, 0, 0, 0, 1, 0, 0, 0])
              + bytes([0xAB, 0xCD, 0x11, 0x22]))
BF16_SCALAR = b"LNGL" + bytes([1, 0, 0, 0, 3, 0, 0, 0, 0, 0, 0, 0, 0xEE, 0xFF])
F32_ZERO_EXTENT = b"LNGL" + bytes([1, 0, 0, 0, 1, 0, 0, 0, 2, 0, 0, 0, 0, 0, 0, 0, 5, 0, 0, 0])

CASES = [
    (DType.F32, [1], bytes([0x11, 0x22, 0x33, 0x44])),
    (DType.F32, [], bytes([1, 2, 3, 4])),
    (DType.F32, [2, 3], bytes(range(24))),
    (DType.F32, [0, 5], b""),
    (DType.F16, [2, 1], bytes([0xAB, 0xCD, 0x11, 0x22])),
    (DType.F16, [2, 1, 1, 1, 1, 1, 1, 1], bytes([9, 8, 7, 6])),
    (DType.F16, [2, 1, 2], bytes([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE])),
    (DType.BF16, [], bytes([0xEE, 0xFF])),
    (DType.BF16, [3], bytes([1, 2, 3, 4, 5, 6])),
    (DType.BF16, [4, 0, 7], b""),
]


def message(tag, extents, payload):
    out = b"LNGL" + struct.pack("<III", 1, tag, len(extents))
    for e in extents:
        out += struct.pack("<I", e)
    return out + bytes(payload)


def kind(fn, *args):
    with pytest.raises(BackendError) as e:
        fn(*args)
    return e.value.kind


def test_golden_messages_round_trip():
    assert W.WIRE_MAGIC == b"LNGL" and W.WIRE_VERSION == 1 and W.WIRE_HEADER_MAX == 48
    assert W.encode(DType.F32, [1], [0x11, 0x22, 0x33, 0x44]) == F32_SCALAR
    assert W.decode(F32_SCALAR) == (DType.F32, [1], bytes([0x11, 0x22, 0x33, 0x44]))
    assert W.encode(DType.F16, [2, 1], [0xAB, 0xCD, 0x11, 0x22]) == F16_MATRIX
    assert W.decode(F16_MATRIX) == (DType.F16, [2, 1], bytes([0xAB, 0xCD, 0x11, 0x22]))
    assert W.encode(DType.BF16, [], [0xEE, 0xFF]) == BF16_SCALAR
    assert W.decode(BF16_SCALAR) == (DType.BF16, [], bytes([0xEE, 0xFF]))
    assert W.encode(DType.F32, [0, 5], b"") == F32_ZERO_EXTENT
    assert W.decode(F32_ZERO_EXTENT) == (DType.F32, [0, 5], b"")
    payload = bytes([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE])
    assert W.decode(W.encode(DType.F16, [2, 1, 2], payload)) == (DType.F16, [2, 1, 2], payload)
    for dt, shape, p in [(DType.F32, [1], [0x11, 0x22]), (DType.F32, [1], [1, 2, 3, 4, 5]),
                         (DType.F16, [], [0xEE, 0xFF, 0, 0]), (DType.BF16, [2], [0xEE, 0xFF]),
                         (DType.F32, [0, 5], [0])]:
        assert kind(W.encode, dt, shape, p) == "Wire"


def test_lengths():
    s = W.encode(DType.F32, [], [1, 2, 3, 4])
    assert len(s) == 20 and s[:4] == b"LNGL" and s[-4:] == bytes([1, 2, 3, 4])
    m = W.encode(DType.F32, [2, 3], bytes([0xAB] * 24))
    assert len(m) == 48 and m[-24:] == bytes([0xAB] * 24)
    r8 = W.encode(DType.F16, [2, 1, 1, 1, 1, 1, 1, 1], [9, 8, 7, 6])
    assert len(r8) == 52 and struct.unpack("<I", r8[12:16])[0] == 8 and r8[-4:] == bytes([9, 8, 7, 6])


def test_rejections_and_their_errors():
    bad = bytearray(F32_SCALAR)
    bad[0] = ord("X")
    assert kind(W.decode, bytes(bad)) == "Wire"
    for version in (2, 0):
        v = bytearray(F32_SCALAR)
        v[4:8] = struct.pack("<I", version)
        assert kind(W.decode, bytes(v)) == "Wire"
    for short in (b"", bytes(15), F32_SCALAR[:16], F32_SCALAR[:-1], F32_SCALAR + b"\xff"):
        assert kind(W.decode, short) == "Wire"
    assert kind(W.decode, message(1, [1] * 9, [0, 0, 0, 0])) == "Wire"
    assert kind(W.encode, DType.F32, [1] * 9, [0, 0, 0, 0]) == "Wire"
    assert kind(W.decode, message(0, [1], [0, 0, 0, 0])) == "Wire"
    assert kind(W.decode, message(4, [1], [0, 0, 0, 0])) == "Wire"
    mid = message(1, [1, 1], [0, 0, 0, 0])[:18]
    assert kind(W.decode, mid) == "Wire"
    above = 2 ** 32
    assert kind(W.encode, DType.F32, [above], b"") == "Shape"
    assert kind(W.encode, DType.F16, [above + 5], b"") == "Shape"
    assert kind(W.encode, DType.BF16, [1, above + 5, 2], [0, 0]) == "Shape"
    assert kind(W.encode, DType.F32, [2 ** 32 - 1], b"") == "Wire"
    assert kind(W.encode, DType.F32, [1 << 16] * 4, b"") == "Shape"
    assert kind(W.encode, DType.F32, [1 << 31, 1 << 31], b"") == "Shape"
    assert kind(W.encode, DType.F16, [1 << 31, 1 << 31, 2], b"") == "Shape"
    assert kind(W.encode, DType.BF16, [1 << 31, 1 << 31, 2], b"") == "Shape"
    assert kind(W.decode, message(1, [65536] * 4, b"")) == "Shape"
    assert kind(W.decode, message(1, [1 << 31, 1 << 31], b"")) == "Shape"
    assert kind(W.decode, message(2, [1 << 31, 1 << 31, 2], b"")) == "Shape"


def test_written_header_plus_payload_equals_encode_and_parses_back():
    for dt, shape, payload in CASES:
        h = W.write_header(dt, shape)
        assert len(h) == 16 + 4 * len(shape)
        assert h + payload == W.encode(dt, shape, payload)
        assert W.parse_header(h + payload) == (dt, shape, len(h))
        assert W.decode(h + payload) == (dt, shape, payload)
    for shape, err in [([1] * 9, "Wire"), ([1] * 12, "Wire"), ([2 ** 32], "Shape"),
                       ([1 << 16] * 4, "Shape"), ([1 << 31, 1 << 31], "Shape")]:
        assert kind(W.write_header, DType.F32, shape) == err


def test_corrupted_and_random_messages_never_misparse():
    """Every truncation, every single-byte change and a few thousand random strings around
    the header: decode either raises BackendError or returns a message that re-encodes to the
    same bytes (the parser reads nothing outside the message; a host sanitizer build runs this
    same suite)."""
    import numpy as np
    g = np.random.Generator(np.random.PCG64(77))
    seeds = [W.encode(dt, shape, payload) for dt, shape, payload in CASES]
    trials = []
    for m in seeds:
        trials += [m[:i] for i in range(len(m))]
        for i in range(len(m)):
            for v in (0, 1, 2, 3, 4, 8, 9, 0x7F, 0xFF):
                b = bytearray(m)
                b[i] = v
                trials.append(bytes(b))
        trials.append(m + bytes(g.integers(0, 256, int(g.integers(1, 9)), dtype=np.uint8)))
    for _ in range(3000):
        n = int(g.integers(0, 64))
        head = b"LNGL" + struct.pack("<I", 1) if g.random() < 0.7 else b""
        body = bytes(g.integers(0, 256, n, dtype=np.uint8))
        if g.random() < 0.5 and len(body) >= 8:
            # plausible tag and rank, random extents
            body = struct.pack("<II", int(g.integers(0, 5)), int(g.integers(0, 10))) + body[8:]
        trials.append(head + body)
    ok = 0
    for t in trials:
        try:
            dt, shape, payload = W.decode(t)
        except BackendError:
            continue
        assert W.encode(dt, shape, payload) == t
        h = W.parse_header(t)
        assert h[0] == dt and h[1] == shape and h[2] == len(t) - len(payload)
        ok += 1
    assert ok >= len(seeds)


def encode_tensor_kind(t, out_cap=None) -> str:
    """lg_wire_encode_tensor with no context: the first failing check, or UnsupportedDevice
    ("null context") when every check passes. Storage bases are never dereferenced."""
    import ctypes
    from linalg_hip import _native as N
    from linalg_hip.backend import _raise
    cap = out_cap if out_cap is not None else W.WIRE_HEADER_MAX + t.numel() * t.dtype.size_of()
    out = ctypes.create_string_buffer(max(cap, 1))
    n = ctypes.c_uint64()
    code = N.lib().lg_wire_encode_tensor(None, ctypes.byref(t.to_c()), out, cap, ctypes.byref(n))
    with pytest.raises(BackendError) as e:
        _raise(code)
    return e.value.kind


def test_encode_tensor_checks_in_download_then_encode_wire_order():
    """send_tensor = download (crates/cpu/src/lib.rs:183-194) then encode_wire
    (crates/core/src/lib.rs:309-322): layout, then the storage range, then the header."""
    from linalg_hip.backend import Storage, Tensor, row_major_strides

    def tensor(shape, nbytes, offset=0, strides=None, dtype=DType.F32):
        st = Storage(0x50000000, nbytes)
        return Tensor(st, dtype, list(shape), strides or row_major_strides(shape), offset)

    # Row-major at a nonzero offset inside the storage passes every check.
    assert encode_tensor_kind(tensor([5, 7], 4 * 38, offset=3)) == "UnsupportedDevice"
    assert encode_tensor_kind(tensor([5, 7], 4 * 38, offset=4)) == "Shape"
    # Not row-major: UnsupportedLayout, before the storage range.
    assert encode_tensor_kind(tensor([5, 7], 4, strides=[1, 5])) == "UnsupportedLayout"
    # Rank 9: the storage range (Shape) comes before encode_wire's rank check (Wire).
    nine = [1] * 8 + [2]
    assert encode_tensor_kind(tensor(nine, 4)) == "Shape"
    assert encode_tensor_kind(tensor(nine, 8)) == "Wire"
    # An extent above u32::MAX is the header's Shape once the range is in the storage.
    assert encode_tensor_kind(tensor([1 << 32], 4 << 32)) == "Shape"
    # An undecodable dtype tag is Wire before anything else.
    assert encode_tensor_kind(tensor([5, 7], 4, strides=[1, 5], dtype=7), out_cap=200) == "Wire"
    # An output buffer shorter than the message.
    assert encode_tensor_kind(tensor([5, 7], 4 * 35), out_cap=16 + 8 + 139) == "Shape"
    assert encode_tensor_kind(tensor([5, 7], 4 * 35), out_cap=16 + 8 + 140) == "UnsupportedDevice"
