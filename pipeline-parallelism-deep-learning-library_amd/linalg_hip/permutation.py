"""Axis permutation views, contiguous materialization, conjugate and adjoint.

Mirrors `linalg::ops::permutation` (src/ops/permutation.rs:272-387): `permute_view`,
`materialize` / `encode_materialize`, `conjugate` / `encode_conjugate`, `adjoint` /
`encode_adjoint`. Elements move as raw bits; f32, u32, i32 and complex f32 ("c64").
"""
from __future__ import annotations

import ctypes
from typing import Sequence

from . import _native as N
from .abi import Context, InvalidArgument, Stream, TensorView, check


def permute_view(view: TensorView, perm: Sequence[int]) -> TensorView:
    """Axis i of the result is axis perm[i] of `view`; metadata only (:295-320)."""
    n = len(perm)
    arr = (ctypes.c_uint64 * max(n, 1))(*[p & 0xFFFFFFFFFFFFFFFF if p >= 0 else
                                          0xFFFFFFFFFFFFFFFF for p in perm])
    out = N.lg_view()
    check(N.lib().lg_permute_view(ctypes.byref(view.to_c()), arr, n, ctypes.byref(out)))
    return TensorView.from_c(out, view.buffer, view.dtype)


def _same_dtype(src: TensorView, dst: TensorView) -> int:
    if src.dtype != dst.dtype:
        raise InvalidArgument(f"source {src.dtype} and destination {dst.dtype} differ")
    if src.elem is None:
        raise InvalidArgument(f"{src.dtype} is not a permutation element type")
    return src.elem


def _call(sync_fn, enc_fn, ctx, stream, src, dst):
    elem = _same_dtype(src, dst)
    if stream is None:
        check(sync_fn(ctx.handle, elem, ctypes.byref(src.to_c()), ctypes.byref(dst.to_c())))
    else:
        check(enc_fn(ctx.handle, stream.handle, elem, ctypes.byref(src.to_c()),
                     ctypes.byref(dst.to_c())))


def materialize(ctx: Context, src: TensorView, dst: TensorView) -> None:
    """Copies `src` into the row-major `dst` of the same shape and waits (:322-332)."""
    L = N.lib()
    _call(L.lg_materialize, L.lg_encode_materialize, ctx, None, src, dst)


def encode_materialize(ctx: Context, stream: Stream, src: TensorView, dst: TensorView) -> None:
    L = N.lib()
    _call(L.lg_materialize, L.lg_encode_materialize, ctx, stream, src, dst)


def conjugate(ctx: Context, src: TensorView, dst: TensorView) -> None:
    """Conjugate of `src` into row-major `dst`; a copy for real types (:344-357)."""
    L = N.lib()
    _call(L.lg_conjugate, L.lg_encode_conjugate, ctx, None, src, dst)


def encode_conjugate(ctx: Context, stream: Stream, src: TensorView, dst: TensorView) -> None:
    L = N.lib()
    _call(L.lg_conjugate, L.lg_encode_conjugate, ctx, stream, src, dst)


def adjoint(ctx: Context, src: TensorView, dst: TensorView) -> None:
    """Batched adjoint: swap the last two axes and conjugate complex elements (:371-379)."""
    L = N.lib()
    _call(L.lg_adjoint, L.lg_encode_adjoint, ctx, None, src, dst)


def encode_adjoint(ctx: Context, stream: Stream, src: TensorView, dst: TensorView) -> None:
    L = N.lib()
    _call(L.lg_adjoint, L.lg_encode_adjoint, ctx, stream, src, dst)


_OPS = {"materialize": 0, "conjugate": 1, "adjoint": 2}


def plan(op: str, src: TensorView, dst: TensorView) -> dict:
    """The gather plan an op would launch (host only, no device work)."""
    elem = _same_dtype(src, dst)
    out = N.lg_permute_plan()
    check(N.lib().lg_plan_permute(_OPS[op], elem, ctypes.byref(src.to_c()),
                                  ctypes.byref(dst.to_c()), ctypes.byref(out)))
    return {"kind": N.PERMUTE_KINDS[out.kind], "rank": out.rank, "axis_a": out.axis_a,
            "axis_b": out.axis_b, "vector": bool(out.vector), "conj": bool(out.conj),
            "streaming": bool(out.streaming),
            "shape": list(out.shape[:out.rank]), "strides": list(out.strides[:out.rank]),
            "workgroups": out.workgroups}
