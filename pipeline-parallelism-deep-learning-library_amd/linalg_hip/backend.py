"""The pipeline's tensor-backend surface on a HIP device.

Mirrors `linalg_core` (crates/core/src/lib.rs): `DType` (:10-32), `Error` (:42-53), `Tensor`
(:55-61), the `Backend` trait (:103-255: alloc / upload / download / sync, gemm, gelu,
gelu_backward, add_bias, bias_grad, mse_grad, sgd_step, convert), `row_major_strides`
(:275-283) and `transpose_matrix` (:285-296). Every op calls its `lg_backend_*` entry point,
which checks operands in `CpuBackend`'s order (crates/cpu/src/lib.rs:203-533) and runs a HIP
kernel; nothing is computed on the host. A tensor's storage id is its device allocation's base
address.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

from . import _native as N
from .abi import Buffer, Context, NoDevice, alloc_shared


class DType(enum.IntEnum):
    """Wire tags of crates/core/src/lib.rs:10-32."""
    F32 = N.LG_DTYPE_F32
    F16 = N.LG_DTYPE_F16
    BF16 = N.LG_DTYPE_BF16

    def size_of(self) -> int:
        return 4 if self is DType.F32 else 2


class BackendError(Exception):
    """`linalg_core::Error`; `kind` is the variant name ("Shape", "Dtype", "Alias", ...)."""

    def __init__(self, kind: str, message: str = ""):
        super().__init__(f"{kind}: {message}" if message else kind)
        self.kind = kind
        self.message = message


def _raise(code: int) -> None:
    if code != 0:
        kind = N.CORE_ERRORS[code] if 0 <= code < len(N.CORE_ERRORS) else f"code {code}"
        raise BackendError(kind, N.lib().lg_last_error().decode(errors="replace"))


@dataclass
class Storage:
    """One allocation: `base` is its device address (the storage id), `nbytes` its length."""
    base: int
    nbytes: int
    buffer: Optional[Buffer] = None

    def storage_id(self) -> int:
        return self.base


@dataclass
class Tensor:
    """`linalg_core::Tensor`: storage plus dtype, shape, strides and offset in elements."""
    storage: Storage
    dtype: DType
    shape: List[int]
    strides: List[int]
    offset: int = 0

    def numel(self) -> int:
        return int(np.prod(self.shape, dtype=object)) if self.shape else 1

    def to_c(self) -> N.lg_tensor:
        if len(self.shape) > N.LG_MAX_RANK or len(self.strides) > N.LG_MAX_RANK:
            raise BackendError("Shape", "rank above LG_MAX_RANK")
        t = N.lg_tensor()
        t.base = self.storage.base
        t.bytes = self.storage.nbytes
        t.dtype = int(self.dtype)
        t.rank = len(self.shape)
        t.nstrides = len(self.strides)
        t.offset = self.offset
        for i, v in enumerate(self.shape):
            t.shape[i] = v
        for i, v in enumerate(self.strides):
            t.strides[i] = v
        return t


def row_major_strides(shape: Sequence[int]) -> List[int]:
    """crates/core/src/lib.rs:275-283 (the stride of an axis is the product of later extents)."""
    strides, stride = [0] * len(shape), 1
    for i in range(len(shape) - 1, -1, -1):
        strides[i] = stride
        stride *= shape[i]
    return strides


def transpose_matrix(t: Tensor) -> Tensor:
    """A view of a rank-2 tensor with its axes swapped (crates/core/src/lib.rs:285-296)."""
    if len(t.shape) != 2 or len(t.strides) != 2:
        raise BackendError("Shape", "transpose_matrix needs rank 2")
    return Tensor(t.storage, t.dtype, [t.shape[1], t.shape[0]], [t.strides[1], t.strides[0]],
                  t.offset)


def _refs(*tensors):
    return [ctypes.byref(t.to_c()) for t in tensors]


def gemm_checks(a: Tensor, b: Tensor, c: Tensor, alpha: float, beta: float) -> None:
    """Runs `lg_backend_gemm`'s operand checks with no context: raises the first check that
    fails, or `UnsupportedDevice` ("null context") when every check passes. Host only."""
    _raise(N.lib().lg_backend_gemm(None, None, *_refs(a, b, c), alpha, beta))


def op_checks(op: str, *args) -> None:
    """The same for the activation and training ops: `op` is "gelu", "gelu_backward",
    "add_bias", "bias_grad", "mse_grad", "sgd_step" or "convert"; `args` are the op's tensors
    followed by its scalar (`lr` for sgd_step). Host only."""
    fn = getattr(N.lib(), f"lg_backend_{op}")
    tensors = [a for a in args if isinstance(a, Tensor)]
    scalars = [a for a in args if not isinstance(a, Tensor)]
    if op == "mse_grad":
        scalars = [ctypes.byref(ctypes.c_float(0.0))]
    _raise(fn(None, None, *_refs(*tensors), *scalars))


def _nbytes(dtype: DType, shape: Sequence[int]) -> int:
    n = dtype.size_of()
    for d in shape:
        n *= d
    return n


class HipBackend:
    """`Backend` for one HIP device (the role `CudaBackend`, crates/cuda/src/device.rs,
    plays on CUDA). Launch order is execution order on the backend's stream; `gemm` returns
    before the device finishes, `download` and `sync` wait for every earlier call."""

    def __init__(self, device: int = 0):
        try:
            self.ctx = Context.new(device)
        except NoDevice as e:
            raise BackendError("UnsupportedDevice", str(e)) from e
        self._live: List[Buffer] = []

    def kind(self) -> str:
        return "Hip"

    def _storage(self, nbytes: int) -> Storage:
        buf = alloc_shared(self.ctx, "u32", (nbytes + 3) // 4)
        self._live.append(buf)
        return Storage(buf.base, nbytes, buf)

    def alloc(self, dtype: DType, shape: Sequence[int]) -> Tensor:
        """Zero-filled row-major tensor; every call gets its own storage, empty ones too."""
        dtype = DType(dtype)
        return Tensor(self._storage(_nbytes(dtype, shape)), dtype, list(shape),
                      row_major_strides(shape))

    def upload(self, dtype: DType, shape: Sequence[int], row_major: bytes) -> Tensor:
        """crates/cpu/src/lib.rs:170-183: a byte count other than the shape's is `Dtype`."""
        dtype = DType(dtype)
        if len(row_major) != _nbytes(dtype, shape):
            raise BackendError("Dtype", "byte count does not match dtype and shape")
        t = self.alloc(dtype, shape)
        if row_major:
            t.storage.buffer.write(np.frombuffer(bytes(row_major), dtype=np.uint8))
        return t

    def upload_f32(self, shape: Sequence[int], values) -> Tensor:
        return self.upload(DType.F32, shape, np.asarray(values, dtype=np.float32).tobytes())

    def download(self, t: Tensor) -> bytes:
        """Row-major bytes of a row-major tensor (crates/cpu/src/lib.rs:185-201)."""
        if list(t.strides) != row_major_strides(t.shape):
            raise BackendError("UnsupportedLayout", "download needs a row-major tensor")
        size = t.dtype.size_of()
        start, length = t.offset * size, t.numel() * size
        if start + length > t.storage.nbytes:
            raise BackendError("Shape", "tensor reaches past its storage")
        self.sync()
        if length == 0:
            return b""
        return t.storage.buffer.read(np.uint8, start, length).tobytes()

    def download_f32(self, t: Tensor) -> np.ndarray:
        return np.frombuffer(self.download(t), dtype=np.float32).copy()

    def download_into(self, t: Tensor, out) -> None:
        """`Backend::download_into` (crates/cpu/src/lib.rs:328-346): the tensor's row-major
        bytes into `out` (a writable buffer: bytearray or contiguous numpy array), no host
        allocation; returns after every earlier call has completed."""
        view = memoryview(out).cast("B")
        if view.readonly:
            raise BackendError("Shape", "output buffer is read-only")
        buf = (ctypes.c_uint8 * len(view)).from_buffer(view) if len(view) else None
        _raise(N.lib().lg_backend_download_into(self.ctx.handle, None, ctypes.byref(t.to_c()),
                                                buf, len(view)))

    def upload_into(self, data, t: Tensor) -> None:
        """`Backend::upload_into` (crates/cpu/src/lib.rs:348-370): overwrites every element of
        the existing row-major tensor with `data`'s bytes; `data` may be reused at once."""
        raw = bytes(memoryview(data).cast("B"))
        _raise(N.lib().lg_backend_upload_into(self.ctx.handle, None, raw, len(raw),
                                              ctypes.byref(t.to_c())))

    def gemm(self, a: Tensor, b: Tensor, c: Tensor, alpha: float, beta: float) -> None:
        """`Backend::gemm` (crates/core/src/lib.rs:143-164); raises `BackendError`."""
        _raise(N.lib().lg_backend_gemm(self.ctx.handle, None, ctypes.byref(a.to_c()),
                                       ctypes.byref(b.to_c()), ctypes.byref(c.to_c()), alpha,
                                       beta))

    def _op(self, op: str, *args) -> None:
        _raise(getattr(N.lib(), f"lg_backend_{op}")(self.ctx.handle, None, *args))

    def gelu(self, x: Tensor, y: Tensor) -> None:
        """`Backend::gelu` (crates/core/src/lib.rs:165-168)."""
        self._op("gelu", *_refs(x, y))

    def gelu_backward(self, pre: Tensor, dy: Tensor, dx: Tensor) -> None:
        """`Backend::gelu_backward` (crates/core/src/lib.rs:170-180)."""
        self._op("gelu_backward", *_refs(pre, dy, dx))

    def add_bias(self, x: Tensor, b: Tensor, y: Tensor) -> None:
        """`Backend::add_bias` (crates/core/src/lib.rs:182-191); `y` may be `x`."""
        self._op("add_bias", *_refs(x, b, y))

    def bias_grad(self, dpre: Tensor, db: Tensor) -> None:
        """`Backend::bias_grad` (crates/core/src/lib.rs:193-201)."""
        self._op("bias_grad", *_refs(dpre, db))

    def mse_grad(self, y: Tensor, target: Tensor, dy: Tensor) -> float:
        """`Backend::mse_grad` (crates/core/src/lib.rs:203-217): returns the loss once every
        earlier call and this one have completed."""
        loss = ctypes.c_float(0.0)
        self._op("mse_grad", *_refs(y, target, dy), ctypes.byref(loss))
        return loss.value

    def sgd_step(self, w: Tensor, dw: Tensor, lr: float) -> None:
        """`Backend::sgd_step` (crates/core/src/lib.rs:219-227)."""
        self._op("sgd_step", *_refs(w, dw), lr)

    def convert(self, x: Tensor, y: Tensor) -> None:
        """`Backend::convert` (crates/core/src/lib.rs:229-236): F32 <-> BF16."""
        self._op("convert", *_refs(x, y))

    def sync(self) -> None:
        try:
            self.ctx.sync()
        except Exception as e:  # a device fault reported at the wait
            raise BackendError("UnsupportedDevice", str(e)) from e

    def debug_launches(self) -> list:
        return self.ctx.launches()

    def close(self) -> None:
        if self.ctx.handle:
            self.sync()
            for buf in self._live:
                buf.free()
            self._live.clear()
            self.ctx.close()
