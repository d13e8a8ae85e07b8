"""The device-buffer ends of a stage boundary: a HipBackend tensor straight to wire bytes and
back (send_tensor / recv_tensor, crates/pipeline/src/lib.rs:71-98)."""
from __future__ import annotations

import numpy as np
import pytest

from linalg_hip import backend as B
from linalg_hip import wire as W
from helpers import rng

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hb():
    backend = B.HipBackend(0)
    yield backend
    backend.close()


@pytest.mark.parametrize("dtype,shape", [(B.DType.F32, [64, 33]), (B.DType.F32, []),
                                         (B.DType.F32, [0, 5]), (B.DType.F16, [2, 1, 2]),
                                         (B.DType.BF16, [4096, 16]), (B.DType.F32, [2, 1, 1, 1, 1, 1, 1, 3])])
def test_tensor_to_wire_and_back_is_bit_exact(hb, dtype, shape):
    n = int(np.prod(shape)) if shape else 1
    raw = rng(n + 1).integers(0, 256, n * dtype.size_of(), dtype=np.uint8).tobytes()
    t = hb.upload(dtype, shape, raw)
    msg = W.encode_tensor(hb, t)
    assert msg == W.encode(dtype, shape, raw)  # the same bytes encode_wire(download) makes
    fresh = hb.alloc(dtype, shape)
    W.decode_into(hb, msg, fresh)
    assert hb.download(fresh) == raw


@pytest.mark.parametrize("dtype,offset,shape", [(B.DType.F32, 3, [5, 7]), (B.DType.BF16, 1, [33, 9]),
                                                (B.DType.F16, 1000, [2, 1, 3]), (B.DType.F32, 41, [])])
def test_tensor_at_an_offset_encodes_its_own_bytes(hb, dtype, offset, shape):
    # download accepts row-major strides at any in-bounds offset (crates/cpu/src/lib.rs:183-194).
    n = int(np.prod(shape)) if shape else 1
    size = dtype.size_of()
    total = offset + n + 5
    raw = rng(offset).integers(0, 256, total * size, dtype=np.uint8).tobytes()
    whole = hb.upload(dtype, [total], raw)
    t = B.Tensor(whole.storage, dtype, list(shape), B.row_major_strides(shape), offset)
    msg = W.encode_tensor(hb, t)
    assert msg == W.encode(dtype, shape, raw[offset * size:(offset + n) * size])


def test_boundary_activation_after_device_work(hb):
    # A boundary activation produced by the device: the message carries its final bytes.
    x = hb.upload_f32([256, 384], rng(2).standard_normal(256 * 384).astype(np.float32))
    y = hb.alloc(B.DType.F32, [256, 384])
    hb.gelu(x, y)
    msg = W.encode_tensor(hb, y)
    assert len(msg) == 16 + 4 * 2 + 256 * 384 * 4  # pipeline.rs wire_len
    assert W.decode(msg)[2] == hb.download(y)


def test_decode_into_errors_leave_the_tensor_unchanged(hb):
    seed = rng(3).standard_normal(12).astype(np.float32)
    t = hb.upload_f32([3, 4], seed)
    good = W.encode(B.DType.F32, [3, 4], seed.tobytes())
    cases = [
        (W.encode(B.DType.F32, [4, 3], seed.tobytes()), t, "Shape"),
        (W.encode(B.DType.F32, [12], seed.tobytes()), t, "Shape"),
        (W.encode(B.DType.BF16, [3, 4], bytes(24)), t, "Dtype"),
        (good[:-1], t, "Wire"),
        (b"XNGL" + good[4:], t, "Wire"),
        (W.encode(B.DType.F32, [4, 3], seed.tobytes()), B.transpose_matrix(t), "UnsupportedLayout"),
    ]
    for msg, dst, k in cases:
        with pytest.raises(B.BackendError) as e:
            W.decode_into(hb, msg, dst)
        assert e.value.kind == k
    assert hb.download_f32(t).tolist() == seed.tolist()
    with pytest.raises(B.BackendError) as e:
        W.encode_tensor(hb, B.transpose_matrix(t))
    assert e.value.kind == "UnsupportedLayout"
