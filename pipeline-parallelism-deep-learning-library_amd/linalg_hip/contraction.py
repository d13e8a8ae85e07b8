"""Tensor contraction: C = alpha*A.B + beta*C, batched GEMM, contraction over shared axes.

Mirrors `linalg::ops::contraction` (src/ops/contraction.rs:1024-1130): `contract`,
`encode_contract`, `gemm`, `encode_gemm`, `gemm_nowait`, with operands given as
`(view, labels)` pairs like the reference's `Operand`. Errors raise InvalidArgument or
Overlap and launch nothing. The element type follows the views, as the reference's generic
`T: Element` does (src/ops/contraction.rs:22-32): all-f32 views take the `_f32` entry points,
all-f16 views the `_f16` ones (each output rounded once to f16); mixing them is an error.
"""
from __future__ import annotations

import ctypes

from . import _native as N
from .abi import Context, InvalidArgument, Stream, TensorView, check


def _f32(*views: TensorView) -> str:
    """The entry-point suffix for these views: "f32" or "f16"."""
    kinds = {v.dtype for v in views}
    if len(kinds) != 1 or not kinds <= {"f32", "f16"}:
        raise InvalidArgument(f"contraction needs all-f32 or all-f16 views, got {sorted(kinds)}")
    return kinds.pop()


def _fn(name: str, t: str):
    return getattr(N.lib(), f"{name}_{t}")


def _labels(s: str) -> bytes:
    b = s.encode()
    if len(b) != len(s):
        raise InvalidArgument("labels must be ASCII, one byte per axis")
    return b


def encode_contract(ctx: Context, stream: Stream, alpha: float, a, b, beta: float, c) -> None:
    """Enqueues C = alpha*A.B + beta*C on `stream` (encode_contract, :1036-1048)."""
    (av, la), (bv, lb), (cv, lc) = a, b, c
    t = _f32(av, bv, cv)
    check(_fn("lg_encode_contract", t)(ctx.handle, stream.handle if stream else None, alpha,
                                         ctypes.byref(av.to_c()), _labels(la),
                                         ctypes.byref(bv.to_c()), _labels(lb), beta,
                                         ctypes.byref(cv.to_c()), _labels(lc)))


def contract(ctx: Context, alpha: float, a, b, beta: float, c) -> None:
    """Synchronous encode_contract (contract, :1053-1064)."""
    (av, la), (bv, lb), (cv, lc) = a, b, c
    t = _f32(av, bv, cv)
    check(_fn("lg_contract", t)(ctx.handle, alpha, ctypes.byref(av.to_c()), _labels(la),
                                  ctypes.byref(bv.to_c()), _labels(lb), beta,
                                  ctypes.byref(cv.to_c()), _labels(lc)))


def encode_gemm(ctx: Context, stream: Stream, alpha: float, a: TensorView, b: TensorView,
                beta: float, c: TensorView) -> None:
    """Enqueues the batched matrix product (encode_gemm, :1080-1090)."""
    t = _f32(a, b, c)
    check(_fn("lg_encode_gemm", t)(ctx.handle, stream.handle if stream else None, alpha,
                                     ctypes.byref(a.to_c()), ctypes.byref(b.to_c()), beta,
                                     ctypes.byref(c.to_c())))


def gemm(ctx: Context, alpha: float, a: TensorView, b: TensorView, beta: float,
         c: TensorView) -> None:
    """Synchronous encode_gemm (gemm, :1092-1103)."""
    t = _f32(a, b, c)
    check(_fn("lg_gemm", t)(ctx.handle, alpha, ctypes.byref(a.to_c()), ctypes.byref(b.to_c()),
                              beta, ctypes.byref(c.to_c())))


def gemm_nowait(ctx: Context, alpha: float, a: TensorView, b: TensorView, beta: float,
                c: TensorView) -> Stream:
    """Enqueues on the context stream without waiting and returns it (gemm_nowait, :1105-1130)."""
    t = _f32(a, b, c)
    check(_fn("lg_gemm_nowait", t)(ctx.handle, alpha, ctypes.byref(a.to_c()),
                                     ctypes.byref(b.to_c()), beta, ctypes.byref(c.to_c())))
    return ctx.queue


def _plan_dict(p: N.lg_contract_plan) -> dict:
    return {"kind": N.PLAN_KINDS[p.kind], "a_mode": N.LOAD_MODES[p.a_mode],
            "b_mode": N.LOAD_MODES[p.b_mode], "groups": p.groups, "batch": p.batch, "m": p.m,
            "n": p.n, "k": p.k, "splits": p.splits, "k_chunk": p.k_chunk,
            "workgroups": p.workgroups, "scratch_bytes": p.scratch_bytes,
            "tile": (p.tile_m, p.tile_n), "kernel": N.PLAN_KERNELS[p.kernel],
            "swapped": bool(p.swapped), "kgroups": int(p.kgroups)}


def plan_contract(alpha: float, a, b, beta: float, c) -> dict:
    """The plan `contract` would launch (host only, no device work)."""
    (av, la), (bv, lb), (cv, lc) = a, b, c
    t = _f32(av, bv, cv)
    out = N.lg_contract_plan()
    check(_fn("lg_plan_contract", t)(alpha, ctypes.byref(av.to_c()), _labels(la),
                                       ctypes.byref(bv.to_c()), _labels(lb), beta,
                                       ctypes.byref(cv.to_c()), _labels(lc), ctypes.byref(out)))
    return _plan_dict(out)


def plan_gemm(alpha: float, a: TensorView, b: TensorView, beta: float, c: TensorView) -> dict:
    """The plan `gemm` would launch (host only, no device work)."""
    t = _f32(a, b, c)
    out = N.lg_contract_plan()
    check(_fn("lg_plan_gemm", t)(alpha, ctypes.byref(a.to_c()), ctypes.byref(b.to_c()), beta,
                                   ctypes.byref(c.to_c()), ctypes.byref(out)))
    return _plan_dict(out)
