"""Data model: errors, context, device buffers and strided views.

Mirrors the reference's frozen data model (src/abi.rs): `LinalgError` and its variants
(:20-33), `MetalContext::new` (:51-62, here `Context.new` on a HIP device), `TensorView`
(:64-211), `row_major_strides` (:213-220), `ALLOC_GRANULE` / `alloc_shared` (:221-243).
MI355X memory is not host-visible, so a `Buffer` carries explicit `write`/`read` copies in
place of the reference's `contents()` pointer arithmetic.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import numpy as np

from . import _native as N

ALLOC_GRANULE = N.LG_ALLOC_GRANULE

# dtype name -> (lg_elem, element bytes, numpy dtype of one word-group)
DTYPES = {
    "f32": (N.LG_ELEM_F32, 4, np.float32),
    "u32": (N.LG_ELEM_U32, 4, np.uint32),
    "i32": (N.LG_ELEM_I32, 4, np.int32),
    "c64": (N.LG_ELEM_C32, 8, np.complex64),  # [f32; 2] (re, im)
    "f16": (None, 2, np.float16),             # contraction only (not a permutation element)
}


class LinalgError(Exception):
    """Errors of every fallible operation (LinalgError, src/abi.rs:20-33)."""


class NoDevice(LinalgError):
    pass


class InvalidArgument(LinalgError):
    pass


class Overlap(LinalgError):
    pass


class ShaderCompile(LinalgError):
    """Kernel load, launch or runtime failure (the reference's ShaderCompile slot)."""


_ERRORS = {N.LG_NO_DEVICE: NoDevice, N.LG_INVALID_ARGUMENT: InvalidArgument,
           N.LG_OVERLAP: Overlap, N.LG_KERNEL: ShaderCompile}


def check(status: int) -> None:
    if status != N.LG_OK:
        msg = N.lib().lg_last_error().decode(errors="replace")
        raise _ERRORS.get(status, LinalgError)(msg)


class Stream:
    """A HIP stream: what the reference's command buffer is to `encode_*` calls."""

    def __init__(self, ctx: "Context", handle: int, owned: bool):
        self.ctx, self.handle, self.owned = ctx, handle, owned

    def wait_until_completed(self) -> None:
        check(N.lib().lg_stream_sync(self.ctx.handle, self.handle))

    def close(self) -> None:
        if self.owned and self.handle:
            check(N.lib().lg_stream_destroy(self.ctx.handle, self.handle))
            self.handle = None


class Context:
    """One HIP device and its stream (MetalContext, src/abi.rs:51-62)."""

    def __init__(self, handle: int):
        self.handle = handle
        self.queue = Stream(self, N.lib().lg_ctx_stream(handle), owned=False)

    @classmethod
    def new(cls, device: int = 0) -> "Context":
        h = ctypes.c_void_p()
        check(N.lib().lg_ctx_create(device, ctypes.byref(h)))
        return cls(h.value)

    def new_stream(self) -> Stream:
        h = ctypes.c_void_p()
        check(N.lib().lg_stream_create(self.handle, ctypes.byref(h)))
        return Stream(self, h.value, owned=True)

    def sync(self) -> None:
        check(N.lib().lg_ctx_sync(self.handle))

    def launches(self) -> list:
        """Names of the kernels launched so far (last 256)."""
        L = N.lib()
        n = L.lg_debug_launch_count(self.handle)
        out = []
        for i in range(max(0, n - 256), n):
            s = L.lg_debug_launch_name(self.handle, i)
            out.append(s.decode() if s else None)
        return out

    def close(self) -> None:
        if self.handle:
            N.lib().lg_ctx_destroy(self.handle)
            self.handle = None


class Buffer:
    """A zero-filled device allocation rounded up to ALLOC_GRANULE bytes."""

    def __init__(self, ctx: Context, base: int, nbytes: int):
        self.ctx, self.base, self.nbytes = ctx, base, nbytes

    def length(self) -> int:
        return self.nbytes

    def contents(self) -> int:
        return self.base

    def write(self, data: np.ndarray, byte_offset: int = 0) -> None:
        data = np.ascontiguousarray(data)
        if byte_offset + data.nbytes > self.nbytes:
            raise ValueError("write beyond the buffer")
        check(N.lib().lg_upload(self.ctx.handle, self.base, byte_offset,
                                data.ctypes.data, data.nbytes))

    def read(self, dtype=np.uint32, byte_offset: int = 0, count: Optional[int] = None) -> np.ndarray:
        dt = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - byte_offset) // dt.itemsize
        out = np.empty(count, dtype=dt)
        check(N.lib().lg_download(self.ctx.handle, self.base, byte_offset, out.ctypes.data,
                                  out.nbytes))
        return out

    def words(self) -> np.ndarray:
        return self.read(np.uint32)

    def free(self) -> None:
        if self.base:
            check(N.lib().lg_free(self.ctx.handle, self.base))
            self.base = None


def alloc_shared(ctx: Context, dtype: str, length: int) -> Buffer:
    """Zeroed allocation of at least `length` elements (alloc_shared, src/abi.rs:225-243)."""
    _, size, _ = DTYPES[dtype]
    base = ctypes.c_void_p()
    nbytes = ctypes.c_uint64()
    check(N.lib().lg_alloc(ctx.handle, size, length, ctypes.byref(base), ctypes.byref(nbytes)))
    return Buffer(ctx, base.value, nbytes.value)


def row_major_strides(shape: Sequence[int]) -> list:
    strides = [1] * len(shape)
    for d in range(len(shape) - 2, -1, -1):
        strides[d] = strides[d + 1] * shape[d + 1]
    return strides


class TensorView:
    """A strided window of `dtype` elements inside one buffer (TensorView, src/abi.rs:64-76).

    The element at multi-index idx lives at element `offset + sum(idx[d] * strides[d])`
    of the buffer. No validation happens at construction; operations validate."""

    def __init__(self, buffer: Buffer, offset: int, shape: Sequence[int], strides: Sequence[int],
                 dtype: str = "f32"):
        self.buffer = buffer
        self.offset = int(offset)
        self.shape = [int(x) for x in shape]
        self.strides = [int(x) for x in strides]
        self.dtype = dtype

    @classmethod
    def row_major(cls, buffer: Buffer, offset: int, shape: Sequence[int], dtype: str = "f32"):
        return cls(buffer, offset, shape, row_major_strides(shape), dtype)

    @property
    def elem_bytes(self) -> int:
        return DTYPES[self.dtype][1]

    @property
    def elem(self) -> int:
        return DTYPES[self.dtype][0]

    def rank(self) -> int:
        return len(self.shape)

    def len(self) -> int:
        n = 1
        for e in self.shape:
            n *= e
        return n

    def is_empty(self) -> bool:
        return 0 in self.shape

    def element_index(self, idx: Sequence[int]) -> int:
        return self.offset + sum(i * s for i, s in zip(idx, self.strides))

    def to_c(self) -> N.lg_view:
        v = N.lg_view()
        v.base = self.buffer.base
        v.bytes = self.buffer.nbytes
        v.offset = self.offset
        if len(self.shape) > N.LG_MAX_RANK or len(self.strides) > N.LG_MAX_RANK:
            raise InvalidArgument("rank exceeds LG_MAX_RANK")
        v.rank = len(self.shape)
        v.nstrides = len(self.strides)
        for i, x in enumerate(self.shape):
            v.shape[i] = x
        for i, x in enumerate(self.strides):
            v.strides[i] = x & 0xFFFFFFFFFFFFFFFF
        return v

    @classmethod
    def from_c(cls, v: N.lg_view, buffer: Buffer, dtype: str) -> "TensorView":
        return cls(buffer, v.offset, list(v.shape[:v.rank]), list(v.strides[:v.nstrides]), dtype)

    def validate(self) -> None:
        check(N.lib().lg_view_validate(ctypes.byref(self.to_c()), self.elem_bytes))

    def element_range(self):
        if self.is_empty():
            return None
        last = self.offset + sum((n - 1) * s for n, s in zip(self.shape, self.strides))
        return range(self.offset, last + 1)

    def byte_range(self):
        r = self.element_range()
        if r is None:
            return None
        return range(r.start * self.elem_bytes, r.stop * self.elem_bytes)

    def may_overlap(self, other: "TensorView") -> bool:
        return bool(N.lib().lg_view_may_overlap(ctypes.byref(self.to_c()), self.elem_bytes,
                                                ctypes.byref(other.to_c()), other.elem_bytes))

    def __repr__(self) -> str:
        return (f"TensorView(dtype={self.dtype}, offset={self.offset}, shape={self.shape}, "
                f"strides={self.strides})")
