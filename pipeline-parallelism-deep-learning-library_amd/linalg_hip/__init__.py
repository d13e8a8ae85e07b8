"""linalg_hip: MI355X-native tensor contraction and permutation.

Host-side mirror of the reference's L0/L1 surface (`linalg::abi`,
`linalg::ops::contraction`, `linalg::ops::permutation`) over the C ABI of
liblinalg_hip.so (include/linalg_hip.h). All compute runs in hand-written gfx950 HIP
kernels; there is no CPU fallback.
"""
from . import backend, contraction, permutation, wire
from ._native import LIB_PATH, lib
from .abi import (ALLOC_GRANULE, DTYPES, Buffer, Context, InvalidArgument, LinalgError,
                  NoDevice, Overlap, ShaderCompile, Stream, TensorView, alloc_shared,
                  row_major_strides)

__all__ = [
    "ALLOC_GRANULE", "DTYPES", "Buffer", "Context", "InvalidArgument", "LinalgError", "NoDevice",
    "Overlap", "ShaderCompile", "Stream", "TensorView", "alloc_shared", "row_major_strides",
    "backend", "contraction", "permutation", "wire", "lib", "LIB_PATH",
]
