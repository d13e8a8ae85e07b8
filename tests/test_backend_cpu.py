"""Host-side tests of lg_backend_gemm's operand checks (no device work).

`gemm_checks` calls the entry point with a null context, so it returns the first failing
check, or UnsupportedDevice ("null context") when every check passes. The cases restate
crates/cpu/src/invariants.rs:250-308 (unsupported_layout_and_alias_leave_c_unchanged) and
crates/cuda/src/invariants.rs:228-258, plus the precedence of CpuBackend::gemm
(crates/cpu/src/lib.rs:203-250) where two checks fail at once. Storage bases are fake
addresses that are never dereferenced.
"""
from __future__ import annotations

import math

import pytest

from linalg_hip import backend as B
from linalg_hip import contraction as C
from helpers import Layout
from test_abi_cpu import view

_next = [0x40000000]


def storage(nbytes: int) -> B.Storage:
    base = _next[0]
    _next[0] += ((nbytes + 16383) // 16384 + 1) * 16384
    return B.Storage(base, nbytes)


def rm(shape, dtype=B.DType.F32) -> B.Tensor:
    n = dtype.size_of()
    for d in shape:
        n *= d
    return B.Tensor(storage(n), dtype, list(shape), B.row_major_strides(shape))


def transposed(rows: int, cols: int) -> B.Tensor:
    """transpose_matrix of a row-major [cols, rows] upload (invariants.rs `transposed`)."""
    t = B.transpose_matrix(rm([cols, rows]))
    assert t.shape == [rows, cols] and t.strides == [1, rows] and t.offset == 0
    return t


def kind(a, b, c, alpha=1.0, beta=0.0) -> str:
    with pytest.raises(B.BackendError) as e:
        B.gemm_checks(a, b, c, alpha, beta)
    return e.value.kind


def test_core_helpers_match_the_reference_definitions():
    assert B.row_major_strides([2, 3, 4]) == [12, 4, 1]
    assert B.row_major_strides([5, 0]) == [0, 1]
    assert B.row_major_strides([]) == []
    t = rm([3, 5])
    v = B.transpose_matrix(t)
    assert (v.shape, v.strides, v.storage.storage_id()) == ([5, 3], [1, 5], t.storage.base)
    with pytest.raises(B.BackendError, match="Shape"):
        B.transpose_matrix(rm([2, 2, 2]))


def test_supported_layouts_pass_every_check():
    # All checks pass; the null context is the only failure left.
    for a, b in [(rm([2, 3]), rm([3, 4])), (transposed(2, 3), rm([3, 4])),
                 (rm([2, 3]), transposed(3, 4))]:
        with pytest.raises(B.BackendError, match="null context") as e:
            B.gemm_checks(a, b, rm([2, 4]), 1.0, 0.5)
        assert e.value.kind == "UnsupportedDevice"


def test_unsupported_layout_and_alias_as_the_cpu_backend_reports_them():
    c = rm([2, 2])
    a, b = rm([2, 2]), rm([2, 2])
    a_bad = rm([2, 2])
    a_bad.strides = [1, 1]
    assert kind(a_bad, b, c) == "UnsupportedLayout"
    assert kind(transposed(2, 2), transposed(2, 2), c, 1.0, 1.0) == "UnsupportedLayout"
    c_view = B.transpose_matrix(c)
    assert c_view.storage.storage_id() == c.storage.storage_id()
    assert kind(a, b, c_view) == "UnsupportedLayout"
    shifted = rm([2, 2])
    shifted.offset = 1
    assert kind(shifted, b, c) == "UnsupportedLayout"
    alias_a = B.Tensor(c.storage, B.DType.F32, [2, 2], B.row_major_strides([2, 2]))
    assert kind(alias_a, b, c) == "Alias"
    alias_b = B.Tensor(c.storage, B.DType.F32, [2, 2], B.row_major_strides([2, 2]))
    assert kind(a, alias_b, c) == "Alias"
    shared = rm([2, 2])
    alias_ab = B.Tensor(shared.storage, B.DType.F32, [2, 2], B.row_major_strides([2, 2]))
    assert kind(shared, alias_ab, c) == "Alias"
    # crates/cuda/src/invariants.rs:228-258: gemm(a, a, c) and an offset C.
    assert kind(a, a, c) == "Alias"
    c_off = rm([2, 2])
    c_off.offset = 1
    assert kind(a, b, c_off) == "UnsupportedLayout"


def test_check_precedence():
    a, b, c = rm([2, 3]), rm([3, 4]), rm([2, 4])
    # Shape beats everything: rank, then inner extents.
    bad_rank = rm([2, 3, 1])
    bad_rank.storage = c.storage  # also an alias, also a transposed layout
    assert kind(bad_rank, b, c) == "Shape"
    ragged = rm([2, 3])
    ragged.strides = [3]
    assert kind(ragged, b, c) == "Shape"
    assert kind(rm([2, 5]), b, c) == "Shape"
    assert kind(a, b, rm([3, 4])) == "Shape"
    assert kind(a, b, rm([2, 5])) == "Shape"
    # Dtype beats Alias and layout.
    half = rm([3, 4], B.DType.F16)
    half.storage = a.storage
    half.offset = 1
    assert kind(a, half, c) == "Dtype"
    # Alias beats layout.
    alias = transposed(3, 4)
    alias.storage = a.storage
    alias.offset = 3
    assert kind(a, alias, c) == "Alias"
    # Layout beats the range check.
    short = rm([2, 3])
    short.storage = storage(4)
    short.offset = 2
    assert kind(short, b, c) == "UnsupportedLayout"
    # Range: C is checked whenever M, N > 0; A and B only when they are read.
    short_c = rm([2, 4])
    short_c.storage = storage(31)
    assert kind(a, b, short_c) == "Shape"
    short_a = rm([2, 3])
    short_a.storage = storage(23)
    assert kind(short_a, b, c) == "Shape"
    with pytest.raises(B.BackendError, match="null context"):
        B.gemm_checks(short_a, b, c, 0.0, 1.0)  # alpha = 0: A is not read
    short_b = transposed(3, 4)
    short_b.storage = storage(47)
    assert kind(a, short_b, c) == "Shape"
    with pytest.raises(B.BackendError, match="null context"):
        B.gemm_checks(rm([2, 0]), rm([0, 4]), c, 1.0, 0.0)  # K = 0: nothing read
    # A corner index that overflows 64 bits is Shape, not a wrap-around.
    big = 2 ** 33
    huge = B.Tensor(storage(16), B.DType.F32, [big, big], [big, 1])
    tall_b = B.Tensor(storage(4 * big), B.DType.F32, [big, 1], [1, 1])
    tall_c = B.Tensor(storage(4 * big), B.DType.F32, [big, 1], [1, 1])
    with pytest.raises(B.BackendError, match="overflows") as e:
        B.gemm_checks(huge, tall_b, tall_c, 1.0, 0.0)
    assert e.value.kind == "Shape"
    # Narrow dtypes pass every check (and then need the device, like f32).
    ha, hb, hc = rm([2, 3], B.DType.BF16), rm([3, 4], B.DType.BF16), rm([2, 4], B.DType.BF16)
    with pytest.raises(B.BackendError, match="null context") as e:
        B.gemm_checks(ha, hb, hc, 1.0, 0.0)
    assert e.value.kind == "UnsupportedDevice"
    # An undecodable dtype tag is a wire error (DType::from_tag).
    odd = rm([2, 3])
    odd.dtype = 9
    assert kind(odd, b, c) == "Wire"


def test_empty_outputs_pass_with_no_work():
    # M = 0 or N = 0: nothing is read or written; ranges are not checked.
    with pytest.raises(B.BackendError, match="null context"):
        B.gemm_checks(rm([0, 3]), rm([3, 4]), rm([0, 4]), 1.0, 1.0)
    tiny = rm([2, 0])
    tiny.storage = storage(0)
    with pytest.raises(B.BackendError, match="null context"):
        B.gemm_checks(rm([2, 3]), rm([3, 0]), tiny, 1.0, 1.0)


def dense(shape):
    return view(Layout.dense(shape))


def test_non_finite_alpha_takes_the_general_kernel():
    # The tiled kernel stages alpha*A; only finite alpha keeps its zero padding zero.
    a, b, c = dense([64, 48]), dense([48, 32]), dense([64, 32])
    assert C.plan_gemm(1.0, a, b, 0.0, c)["kind"] == "tiled"
    for alpha in (math.inf, -math.inf, math.nan):
        assert C.plan_gemm(alpha, a, b, 0.0, c)["kind"] == "general"
    assert C.plan_gemm(3.0e38, a, b, 0.0, c)["kind"] == "tiled"


# ---- training ops: crates/cpu/src/training.rs:291-372 and invariants.rs:503-520 ----------
def op_kind(op, *args) -> str:
    with pytest.raises(B.BackendError) as e:
        B.op_checks(op, *args)
    return e.value.kind


def alias_of(t: B.Tensor, **kw) -> B.Tensor:
    fields = dict(storage=t.storage, dtype=t.dtype, shape=list(t.shape), strides=list(t.strides),
                  offset=t.offset)
    fields.update(kw)
    return B.Tensor(**fields)


def test_training_op_errors_come_in_contract_order():
    x, b, b_wrong = rm([2, 3]), rm([3]), rm([4])
    h, hb = rm([2, 3], B.DType.BF16), rm([3], B.DType.BF16)
    y = rm([2, 3])
    odd = alias_of(y, strides=[1, 2])
    # add_bias
    assert op_kind("add_bias", h, b_wrong, y) == "Shape"
    assert op_kind("add_bias", h, b, y) == "Dtype"
    assert op_kind("add_bias", x, b, alias_of(b)) == "Shape"
    assert op_kind("add_bias", x, alias_of(y), y) == "Shape"
    assert op_kind("add_bias", x, alias_of(y, shape=[3], strides=[1]), y) == "Alias"
    assert op_kind("add_bias", x, b, odd) == "UnsupportedLayout"
    # bias_grad
    db = rm([3])
    assert op_kind("bias_grad", h, alias_of(b_wrong)) == "Shape"
    assert op_kind("bias_grad", x, alias_of(hb)) == "Dtype"
    assert op_kind("bias_grad", x, alias_of(x, shape=[3], strides=[1])) == "Alias"
    assert op_kind("bias_grad", alias_of(x, strides=[1, 2]), db) == "UnsupportedLayout"
    # mse_grad
    empty = rm([0, 3])
    assert op_kind("mse_grad", empty, empty, alias_of(empty)) == "Shape"
    assert op_kind("mse_grad", x, b, y) == "Shape"
    assert op_kind("mse_grad", h, x, y) == "Dtype"
    assert op_kind("mse_grad", x, y, alias_of(y)) == "Alias"
    assert op_kind("mse_grad", x, x, odd) == "UnsupportedLayout"
    # sgd_step
    w = rm([3])
    assert op_kind("sgd_step", w, alias_of(x), 0.1) == "Shape"
    assert op_kind("sgd_step", w, alias_of(hb), 0.1) == "Dtype"
    assert op_kind("sgd_step", w, alias_of(w), 0.1) == "Alias"
    assert op_kind("sgd_step", alias_of(w, offset=1), db, 0.1) == "UnsupportedLayout"
    # convert
    h_out = rm([2, 3], B.DType.BF16)
    assert op_kind("convert", x, alias_of(hb)) == "Shape"
    assert op_kind("convert", x, y) == "Dtype"
    assert op_kind("convert", h, alias_of(h)) == "Dtype"
    assert op_kind("convert", x, alias_of(x, dtype=B.DType.BF16)) == "Alias"
    assert op_kind("convert", alias_of(x, strides=[1, 2]), h_out) == "UnsupportedLayout"
    # gelu / gelu_backward (prepare_f32_row_major): Dtype, Shape, layout, storage.
    f16 = rm([4], B.DType.F16)
    assert op_kind("gelu", f16, rm([4])) == "Dtype"
    assert op_kind("gelu", rm([4]), rm([5])) == "Shape"
    assert op_kind("gelu", alias_of(rm([4]), strides=[2]), rm([4])) == "UnsupportedLayout"
    short = rm([4])
    short.storage = storage(12)
    assert op_kind("gelu", short, rm([4])) == "Shape"
    assert op_kind("gelu_backward", rm([4]), rm([4], B.DType.BF16), rm([4])) == "Dtype"
    assert op_kind("gelu_backward", rm([4]), rm([4]), rm([2, 2])) == "Shape"
    # Storage too short after the layout check: Shape.
    tiny = rm([2, 3])
    tiny.storage = storage(20)
    assert op_kind("add_bias", tiny, b, y) == "Shape"
    assert op_kind("sgd_step", rm([6]), alias_of(tiny, shape=[6], strides=[1]), 0.1) == "Shape"
    # An undecodable dtype tag is a wire error everywhere.
    assert op_kind("gelu", alias_of(x, dtype=7), y) == "Wire"


def test_bias_grad_extents_are_31_bit():
    ok = (1 << 31) - 1
    with pytest.raises(B.BackendError, match="null context"):
        B.op_checks("bias_grad", rm([ok, 1]), rm([1]))
    assert op_kind("bias_grad", rm([ok + 1, 1]), rm([1])) == "Shape"
    assert op_kind("bias_grad", rm([1, ok + 1]), rm([ok + 1])) == "Shape"


def test_training_ops_pass_their_checks_on_valid_operands():
    x, b, y = rm([2, 3]), rm([3]), rm([2, 3])
    cases = [("gelu", x, y), ("gelu", x, alias_of(x)), ("gelu_backward", x, rm([2, 3]), y),
             ("add_bias", x, b, y), ("add_bias", x, b, alias_of(x)), ("bias_grad", x, b),
             ("bias_grad", rm([0, 3]), b), ("mse_grad", x, rm([2, 3]), alias_of(x)),
             ("mse_grad", x, alias_of(x), y), ("sgd_step", x, y, 0.5),
             ("convert", x, rm([2, 3], B.DType.BF16)), ("convert", rm([2, 3], B.DType.BF16), x)]
    for op, *args in cases:
        with pytest.raises(B.BackendError, match="null context") as e:
            B.op_checks(op, *args)
        assert e.value.kind == "UnsupportedDevice", op


def transfer_kind(direction: str, t: B.Tensor, length: int) -> str:
    """lg_backend_download_into / upload_into with no context: the first failing check, or
    UnsupportedDevice ("null context") when every check passes."""
    import ctypes
    from linalg_hip import _native as N
    buf = (ctypes.c_uint8 * max(length, 1))()
    if direction == "down":
        code = N.lib().lg_backend_download_into(None, None, ctypes.byref(t.to_c()), buf, length)
    else:
        code = N.lib().lg_backend_upload_into(None, None, buf, length, ctypes.byref(t.to_c()))
    with pytest.raises(B.BackendError) as e:
        B._raise(code)
    return e.value.kind


@pytest.mark.parametrize("direction", ["down", "up"])
def test_transfer_into_checks_in_the_reference_order(direction):
    """download_into / upload_into (crates/cpu/src/lib.rs:328-370): byte count first (Shape),
    then row-major at offset 0 (UnsupportedLayout), then the storage (Shape)."""
    t = rm([3, 5])
    assert transfer_kind(direction, t, 60) == "UnsupportedDevice"
    assert transfer_kind(direction, t, 59) == "Shape"
    assert transfer_kind(direction, t, 61) == "Shape"
    # A wrong length is reported before a wrong layout.
    assert transfer_kind(direction, transposed(3, 5), 59) == "Shape"
    assert transfer_kind(direction, transposed(3, 5), 60) == "UnsupportedLayout"
    shifted = B.Tensor(storage(64), B.DType.F32, [3, 5], [5, 1], 1)
    assert transfer_kind(direction, shifted, 60) == "UnsupportedLayout"
    short = B.Tensor(storage(56), B.DType.F32, [3, 5], [5, 1])
    assert transfer_kind(direction, short, 60) == "Shape"
    half = rm([4], B.DType.BF16)
    assert transfer_kind(direction, half, 8) == "UnsupportedDevice"
    odd = rm([2])
    odd.dtype = 9
    assert transfer_kind(direction, odd, 8) == "Wire"
    assert transfer_kind(direction, rm([0, 3]), 0) == "UnsupportedDevice"
