"""Permutation parity on the GPU: bit-exact against the gather_words oracle.

Restates the cases of tests/permutation_test.rs over the C ABI: destinations start as
SENTINEL words and every word outside the destination view must survive; sources mix random
words and SPECIALS (NaN payloads, -0, infinities, subnormals); all element types (f32, u32,
i32, complex f32). The benchmark configurations run at full size and are compared word for word
with numpy.transpose of the raw bits.
"""
from __future__ import annotations

import json

import numpy as np
import pytest

import linalg_hip as L
from helpers import (GOLDEN, SENTINEL, WORDS, assert_dst, check_materialize, gather, permutations,
                     random_words, rng, span, special_words, word_buffer)
from linalg_hip import permutation as P

pytestmark = pytest.mark.gpu

TYPES = ["f32", "u32", "i32", "c64"]


def check_all_perms(ctx, pool, dtype, base, seed):
    for i, perm in enumerate(permutations(len(base))):
        check_materialize(ctx, pool, dtype, base, perm, 0, None, 0, seed + i)


@pytest.mark.parametrize("dtype", TYPES)
def test_materialize_all_perms_rank_1_to_4_prime_extents(ctx, pool, dtype):
    check_all_perms(ctx, pool, dtype, [101], 1)
    check_all_perms(ctx, pool, dtype, [37, 41], 10)
    check_all_perms(ctx, pool, dtype, [5, 37, 67], 100)
    check_all_perms(ctx, pool, dtype, [5, 7, 37, 41], 1000)


@pytest.mark.parametrize("dtype", TYPES)
def test_materialize_all_perms_rank_5_prime_extents(ctx, pool, dtype):
    check_all_perms(ctx, pool, dtype, [3, 5, 7, 11, 13], 5000)


@pytest.mark.parametrize("dtype", TYPES)
def test_materialize_all_perms_rank_4_with_unit_and_two_extents(ctx, pool, dtype):
    check_all_perms(ctx, pool, dtype, [1, 2, 3, 37], 7000)
    check_all_perms(ctx, pool, dtype, [2, 1, 41, 2], 7100)


def test_materialize_with_source_and_destination_offsets(ctx, pool):
    for n, (so, doff) in enumerate([(0, 0), (1, 3), (13, 7), (33, 1), (4095, 4097)]):
        seed = 200 + n
        check_materialize(ctx, pool, "f32", [37, 41], [1, 0], so, None, doff, seed)
        check_materialize(ctx, pool, "c64", [5, 37, 43], [2, 0, 1], so, None, doff, seed)
        check_materialize(ctx, pool, "u32", [7, 11, 13, 3], [3, 2, 1, 0], so, None, doff, seed)


def test_materialize_multi_tile_transposes_with_ragged_edges(ctx, pool):
    for m, n in [(32, 32), (33, 31), (64, 64), (100, 130), (129, 65), (31, 257), (1000, 33),
                 (65, 129), (128, 256)]:
        check_materialize(ctx, pool, "f32", [m, n], [1, 0], 0, None, 0, 300)
        check_materialize(ctx, pool, "c64", [m, n], [1, 0], 0, None, 0, 301)


def test_materialize_batched_transpose_with_many_batches(ctx, pool):
    check_materialize(ctx, pool, "f32", [257, 33, 35], [0, 2, 1], 0, None, 0, 400)
    check_materialize(ctx, pool, "c64", [1031, 3, 5], [0, 2, 1], 0, None, 0, 401)
    check_materialize(ctx, pool, "u32", [3, 4, 5, 6, 7], [4, 0, 3, 1, 2], 0, None, 0, 402)


def test_materialize_padded_leading_dimension_and_sliced_views(ctx, pool):
    for perm in ([0, 1], [1, 0]):
        check_materialize(ctx, pool, "f32", [45, 40], perm, 5, [64, 1], 3, 500)
        check_materialize(ctx, pool, "c64", [45, 40], perm, 5, [64, 1], 3, 501)
    for perm in ([0, 1], [1, 0]):
        check_materialize(ctx, pool, "u32", [20, 31], perm, 2, [150, 2], 0, 502)
        check_materialize(ctx, pool, "f32", [20, 31], perm, 0, [3 * 64, 1], 0, 503)
    check_materialize(ctx, pool, "f32", [37, 41], [1, 0], 0, [1, 37], 0, 504)
    check_materialize(ctx, pool, "f32", [37, 41], [0, 1], 0, [1, 37], 0, 505)
    check_materialize(ctx, pool, "c64", [4, 9, 33], [2, 0, 1], 1, [9 * 40, 40, 1], 2, 506)
    # Aligned padded rows: the 128-bit tile path with a leading dimension (not in the
    # reference's list; exercises the vector path with a non-dense source).
    check_materialize(ctx, pool, "f32", [96, 200], [1, 0], 4, [256, 1], 8, 507)
    check_materialize(ctx, pool, "c64", [96, 200], [1, 0], 2, [256, 1], 6, 508)


def test_materialize_broadcast_zero_strides(ctx, pool):
    check_materialize(ctx, pool, "f32", [5, 37], [1, 0], 0, [0, 1], 0, 600)
    check_materialize(ctx, pool, "f32", [37, 5], [1, 0], 0, [1, 0], 0, 601)
    check_materialize(ctx, pool, "c64", [3, 4, 33], [2, 1, 0], 0, [0, 0, 1], 0, 602)


def test_materialize_degenerate_extents(ctx, pool):
    for n in [1, 2, 31, 32, 33, 997, 1000]:
        for perm in ([0, 1], [1, 0]):
            check_materialize(ctx, pool, "f32", [1, n], perm, 0, None, 0, 700)
            check_materialize(ctx, pool, "f32", [n, 1], perm, 0, None, 0, 701)
            check_materialize(ctx, pool, "c64", [1, n], perm, 0, None, 0, 702)
            check_materialize(ctx, pool, "c64", [n, 1], perm, 0, None, 0, 703)
    check_materialize(ctx, pool, "f32", [1, 1], [1, 0], 0, None, 0, 704)
    check_materialize(ctx, pool, "f32", [1, 1, 1], [2, 0, 1], 0, None, 0, 705)
    check_materialize(ctx, pool, "f32", [], [], 3, None, 1, 706)


def test_materialize_zero_sized_extents_succeed_and_write_nothing(ctx, pool):
    for shape in ([0, 5], [5, 0], [0, 0], [3, 0, 4], [0]):
        for perm in permutations(len(shape)):
            check_materialize(ctx, pool, "f32", shape, perm, 0, None, 2, 800)
            check_materialize(ctx, pool, "c64", shape, perm, 0, None, 2, 801)


def test_materialize_into_disjoint_region_of_same_buffer(ctx, pool):
    m, n = 37, 41
    buf, host = word_buffer(pool, "f32", 4 * m * n, random_words, rng(900))
    src = L.TensorView.row_major(buf, 0, [m, n])
    view = P.permute_view(src, [1, 0])
    want = gather(host, view)
    dst = L.TensorView.row_major(buf, 2 * m * n, [n, m])
    P.materialize(ctx, view, dst)
    got = buf.words()
    assert np.array_equal(got[2 * m * n: 3 * m * n], want)
    assert np.array_equal(got[: 2 * m * n], host[: 2 * m * n])
    assert np.array_equal(got[3 * m * n:], host[3 * m * n:])


# --------------------------------------------------------------------------------------
# Adjoint and conjugate
# --------------------------------------------------------------------------------------
def reference_adjoint(host, src: L.TensorView):
    r = src.rank()
    perm = list(range(r))
    perm[r - 2], perm[r - 1] = perm[r - 1], perm[r - 2]
    swapped = L.TensorView(src.buffer, src.offset, [src.shape[p] for p in perm],
                           [src.strides[p] for p in perm], src.dtype)
    return gather(host, swapped, conj=True)


def check_involution(ctx, pool, dtype, batch, m, n, seed):
    a_shape, b_shape = batch + [m, n], batch + [n, m]
    length = int(np.prod(a_shape))
    a_buf, a_host = word_buffer(pool, dtype, length, special_words, rng(seed))
    a = L.TensorView.row_major(a_buf, 0, a_shape, dtype)
    a_words = gather(a_host, a)
    b_buf, _ = word_buffer(pool, dtype, length)
    b = L.TensorView.row_major(b_buf, 0, b_shape, dtype)
    c_buf, _ = word_buffer(pool, dtype, length)
    c = L.TensorView.row_major(c_buf, 0, a_shape, dtype)
    label = f"{dtype} batch={batch} {m}x{n}"
    P.adjoint(ctx, a, b)
    assert_dst(label + " B", b_buf, dtype, 0, reference_adjoint(a_host, a))
    P.adjoint(ctx, b, c)
    assert_dst(label + " C", c_buf, dtype, 0, a_words)


def test_adjoint_twice_is_bitwise_identity_with_special_values(ctx, pool):
    shapes = [([], 1, 1), ([], 1, 7), ([], 7, 1), ([], 32, 32), ([], 31, 33), ([], 67, 101),
              ([], 129, 65), ([3], 5, 37), ([2, 3], 41, 7), ([7], 33, 1), ([2], 64, 128),
              ([2], 301, 203)]
    for i, (batch, m, n) in enumerate(shapes):
        check_involution(ctx, pool, "f32", batch, m, n, 1000 + i)
        check_involution(ctx, pool, "c64", batch, m, n, 1100 + i)


def test_adjoint_of_complex_flips_only_the_imaginary_sign_bit(ctx, pool):
    t = json.loads((GOLDEN / "permutation_kats.json").read_text())["complex_adjoint"]
    m, n = t["m"], t["n"]
    a_buf = pool.alloc("c64", m * n)
    host = np.zeros(a_buf.nbytes // 4, dtype=np.uint32)
    host[: 2 * m * n] = t["input_words"]
    a_buf.write(host)
    b_buf, _ = word_buffer(pool, "c64", m * n)
    a = L.TensorView.row_major(a_buf, 0, [m, n], "c64")
    b = L.TensorView.row_major(b_buf, 0, [n, m], "c64")
    P.adjoint(ctx, a, b)
    assert b_buf.words()[: 2 * m * n].tolist() == t["adjoint_words"]


def test_adjoint_of_real_is_plain_transpose(ctx, pool):
    for m, n in [(1, 1), (3, 5), (37, 41), (64, 33)]:
        a_buf, a_host = word_buffer(pool, "f32", m * n, special_words, rng(1200))
        a = L.TensorView.row_major(a_buf, 0, [m, n])
        b_buf, _ = word_buffer(pool, "f32", m * n)
        b = L.TensorView.row_major(b_buf, 0, [n, m])
        P.adjoint(ctx, a, b)
        assert_dst("real adjoint", b_buf, "f32", 0, gather(a_host, P.permute_view(a, [1, 0])))


def test_adjoint_batched_strided_source_with_offsets(ctx, pool):
    batch, m, n, ld = 3, 37, 41, 48
    strides = [m * ld, ld, 1]
    off = 11
    a_buf, a_host = word_buffer(pool, "c64", span(off, [batch, m, n], strides), special_words, rng(1300))
    a = L.TensorView(a_buf, off, [batch, m, n], strides, "c64")
    b_buf, _ = word_buffer(pool, "c64", 5 + batch * m * n + 9)
    b = L.TensorView.row_major(b_buf, 5, [batch, n, m], "c64")
    P.adjoint(ctx, a, b)
    assert_dst("strided adjoint", b_buf, "c64", 5, reference_adjoint(a_host, a))


def test_adjoint_of_a_permuted_view_composes_with_permutation(ctx, pool):
    a_buf, a_host = word_buffer(pool, "c64", 5 * 7 * 11, special_words, rng(1400))
    a = L.TensorView.row_major(a_buf, 0, [5, 7, 11], "c64")
    p = P.permute_view(a, [2, 0, 1])
    b_buf, _ = word_buffer(pool, "c64", 5 * 7 * 11)
    b = L.TensorView.row_major(b_buf, 0, [11, 7, 5], "c64")
    P.adjoint(ctx, p, b)
    assert_dst("adjoint of permuted view", b_buf, "c64", 0, reference_adjoint(a_host, p))


def test_adjoint_zero_sized_and_degenerate_shapes(ctx, pool):
    for batch, m, n in [([], 0, 5), ([], 5, 0), ([2], 0, 0), ([0], 3, 4)]:
        a_buf = pool.alloc("c64", 64)
        b_buf, _ = word_buffer(pool, "c64", 64)
        a = L.TensorView.row_major(a_buf, 0, batch + [m, n], "c64")
        b = L.TensorView.row_major(b_buf, 0, batch + [n, m], "c64")
        P.adjoint(ctx, a, b)
        assert np.all(b_buf.words() == SENTINEL)


def test_conjugate_flips_imaginary_sign_and_is_an_involution(ctx, pool):
    for shape in ([1], [97], [7, 13], [3, 5, 37], [1024]):
        length = int(np.prod(shape))
        a_buf, a_host = word_buffer(pool, "c64", length, special_words, rng(1500))
        a = L.TensorView.row_major(a_buf, 0, shape, "c64")
        b_buf, _ = word_buffer(pool, "c64", length)
        b = L.TensorView.row_major(b_buf, 0, shape, "c64")
        c_buf, _ = word_buffer(pool, "c64", length)
        c = L.TensorView.row_major(c_buf, 0, shape, "c64")
        P.conjugate(ctx, a, b)
        assert_dst("conj", b_buf, "c64", 0, gather(a_host, a, conj=True))
        P.conjugate(ctx, b, c)
        assert_dst("conj conj", c_buf, "c64", 0, gather(a_host, a))


def test_conjugate_of_real_is_a_copy(ctx, pool):
    a_buf, a_host = word_buffer(pool, "f32", 1000, special_words, rng(1600))
    a = L.TensorView.row_major(a_buf, 0, [10, 100])
    b_buf, _ = word_buffer(pool, "f32", 1000)
    b = L.TensorView.row_major(b_buf, 0, [10, 100])
    P.conjugate(ctx, a, b)
    assert_dst("real conj", b_buf, "f32", 0, gather(a_host, a))


# --------------------------------------------------------------------------------------
# Encode-only behaviour: one stream carries several enqueued gathers in order.
# --------------------------------------------------------------------------------------
def test_encode_only_chains_on_one_stream(ctx, pool):
    m, n = 67, 101
    a_buf, a_host = word_buffer(pool, "c64", m * n, special_words, rng(1700))
    a = L.TensorView.row_major(a_buf, 0, [m, n], "c64")
    bufs = [word_buffer(pool, "c64", m * n)[0] for _ in range(3)]
    b = L.TensorView.row_major(bufs[0], 0, [n, m], "c64")
    c = L.TensorView.row_major(bufs[1], 0, [m, n], "c64")
    d = L.TensorView.row_major(bufs[2], 0, [m, n], "c64")
    a_words = gather(a_host, a)
    s = ctx.new_stream()
    try:
        P.encode_adjoint(ctx, s, a, b)
        P.encode_adjoint(ctx, s, b, c)
        P.encode_conjugate(ctx, s, c, d)
        s.wait_until_completed()
    finally:
        s.close()
    assert_dst("chained C", bufs[1], "c64", 0, a_words)
    assert_dst("chained D", bufs[2], "c64", 0, gather(bufs[1].words(), c, conj=True))


def test_encode_materialize_orders_after_earlier_work_on_the_same_stream(ctx, pool):
    m, n = 45, 40
    a_buf, a_host = word_buffer(pool, "f32", m * n, random_words, rng(1800))
    a = L.TensorView.row_major(a_buf, 0, [m, n])
    t = P.permute_view(a, [1, 0])
    b_buf, _ = word_buffer(pool, "f32", m * n)
    b = L.TensorView.row_major(b_buf, 0, [n, m])
    c_buf, _ = word_buffer(pool, "f32", m * n)
    c = L.TensorView.row_major(c_buf, 0, [m, n])
    P.encode_materialize(ctx, ctx.queue, t, b)
    P.encode_materialize(ctx, ctx.queue, P.permute_view(b, [1, 0]), c)
    ctx.queue.wait_until_completed()
    assert_dst("round trip", c_buf, "f32", 0, gather(a_host, a))


# --------------------------------------------------------------------------------------
# Error paths: nothing is launched and nothing written.
# --------------------------------------------------------------------------------------
def test_rejects_aliased_destination(ctx, pool):
    buf, host = word_buffer(pool, "c64", 64 * 64, random_words, rng(2000))
    a = L.TensorView.row_major(buf, 0, [32, 32], "c64")
    shifted = L.TensorView.row_major(buf, 100, [32, 32], "c64")
    n0 = ctx.launches()
    for dst in (a, shifted):
        for fn in (P.adjoint, P.conjugate, P.materialize):
            with pytest.raises(L.Overlap):
                fn(ctx, a, dst)
    with pytest.raises(L.Overlap):
        P.encode_adjoint(ctx, ctx.queue, a, a)
    assert ctx.launches() == n0
    assert np.array_equal(buf.words(), host), "an aliased call must not launch"


def test_rejects_invalid_metadata_without_launching(ctx, pool):
    src_buf, _ = word_buffer(pool, "f32", 1024, random_words, rng(2100))
    dst_buf, _ = word_buffer(pool, "f32", 1024)
    src = L.TensorView.row_major(src_buf, 0, [16, 32])
    inv = lambda: pytest.raises(L.InvalidArgument)
    n0 = ctx.launches()
    with inv():
        P.adjoint(ctx, src, L.TensorView.row_major(dst_buf, 0, [16, 32]))
    swapped = L.TensorView.row_major(dst_buf, 0, [32, 16])
    with inv():
        P.materialize(ctx, src, swapped)
    with inv():
        P.conjugate(ctx, src, swapped)
    with inv():
        P.adjoint(ctx, src, L.TensorView(dst_buf, 0, [32, 16], [1, 32]))
    with inv():
        P.adjoint(ctx, src, L.TensorView(dst_buf, 0, [32, 16], [20, 1]))
    cap = dst_buf.nbytes // 4
    with inv():
        P.adjoint(ctx, src, L.TensorView.row_major(dst_buf, cap - 100, [32, 16]))
    ok_dst = L.TensorView.row_major(dst_buf, 0, [32, 16])
    with inv():
        P.adjoint(ctx, L.TensorView.row_major(src_buf, cap - 100, [16, 32]), ok_dst)
    with inv():
        P.adjoint(ctx, L.TensorView(src_buf, 0, [16, 32], [32]), ok_dst)
    with inv():
        P.adjoint(ctx, L.TensorView.row_major(src_buf, 0, [16]), L.TensorView.row_major(dst_buf, 0, [16]))
    with inv():
        P.adjoint(ctx, src, L.TensorView.row_major(dst_buf, 0, [32, 17]))
    assert ctx.launches() == n0
    assert np.all(dst_buf.words() == SENTINEL)


# --------------------------------------------------------------------------------------
# benchmark configurations at full size: bit-exact against numpy.transpose of the raw words.
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("shape,perm,seed", [([64, 128, 64, 32], [0, 2, 3, 1], 3),
                                             ([512, 1024, 256], [2, 0, 1], 4),
                                             ([1024, 1024, 256], [2, 0, 1], 5)])
def test_baseline_configs_full_size_bit_exact(ctx, pool, shape, perm, seed):
    n = int(np.prod(shape))
    g = rng(seed)
    x = g.uniform(-1.0, 1.0, n).astype(np.float32)
    src_buf = pool.alloc("f32", n)
    src_buf.write(x)
    src = L.TensorView.row_major(src_buf, 0, shape)
    view = P.permute_view(src, perm)
    dst_buf = pool.alloc("f32", n)
    dst = L.TensorView.row_major(dst_buf, 0, view.shape)
    plan = P.plan("materialize", view, dst)
    assert plan["kind"] == "tile" and plan["vector"]
    P.materialize(ctx, view, dst)
    got = dst_buf.read(np.uint32, count=n)
    want = np.ascontiguousarray(np.transpose(x.view(np.uint32).reshape(shape), perm)).ravel()
    assert np.array_equal(got, want)
    # Inverse permutation restores the source exactly (round trip).
    inv = [0] * len(perm)
    for i, p in enumerate(perm):
        inv[p] = i
    back_buf = pool.alloc("f32", n)
    back = L.TensorView.row_major(back_buf, 0, shape)
    P.materialize(ctx, P.permute_view(dst, inv), back)
    assert np.array_equal(back_buf.read(np.uint32, count=n), x.view(np.uint32))


def test_streaming_transposes_with_ragged_edges_and_complex_words(ctx, pool):
    """Permutations moving more than 256 MiB take the streaming tiles (non-temporal accesses,
    their own tile shape; rows a multiple of 16 bytes, as 128-bit access needs): ragged edges
    along both tile axes under a batch axis (f32), a complex transpose (two-word elements) and a
    complex adjoint applied twice (sign flip, then back), each against the gathered words."""
    for dtype, shape, perm in [("f32", [3, 4100, 5004], [0, 2, 1]), ("c64", [4098, 4102], [1, 0])]:
        src_buf = pool.alloc(dtype, int(np.prod(shape)))
        view = P.permute_view(L.TensorView.row_major(src_buf, 0, shape, dtype), perm)
        dst = L.TensorView.row_major(pool.alloc(dtype, view.len()), 0, view.shape, dtype)
        plan = P.plan("materialize", view, dst)
        assert plan["kind"] == "tile" and plan["streaming"], (dtype, plan)
        pool.free_all()
    check_materialize(ctx, pool, "f32", [3, 4100, 5004], [0, 2, 1], 0, None, 0, 1400)
    pool.free_all()
    check_materialize(ctx, pool, "c64", [4098, 4102], [1, 0], 0, None, 0, 1401)
    pool.free_all()
    check_involution(ctx, pool, "c64", [2], 2900, 2902, 1402)


def test_transpose_reads_misaligned_rows_to_the_edges_of_the_buffer(ctx, pool):
    """A view whose rows are not 16-byte aligned, in a buffer that starts 4 bytes into a device
    allocation and ends at the view's last word: interior and edge tiles move every word once
    and touch nothing outside the view, for one-word and two-word (complex) elements."""
    for dtype, (m, n) in (("f32", (131, 1031)), ("c64", (67, 261))):
        words_per = 2 if dtype == "c64" else 1
        real = pool.alloc("f32", (m * n + 8) * words_per)
        buf = L.Buffer(ctx, real.base + 4, m * n * 4 * words_per)
        host = random_words(rng(m + n), m * n * words_per)
        buf.write(host)
        src = L.TensorView.row_major(buf, 0, [m, n], dtype)
        dst_buf = pool.alloc(dtype, m * n)
        dst = L.TensorView.row_major(dst_buf, 0, [n, m], dtype)
        plan = P.plan("materialize", P.permute_view(src, [1, 0]), dst)
        assert plan["kind"] == "tile" and not plan["vector"], plan
        P.materialize(ctx, P.permute_view(src, [1, 0]), dst)
        want = host.reshape(m, n, words_per).transpose(1, 0, 2).ravel()
        assert np.array_equal(dst_buf.read(np.uint32, count=m * n * words_per), want), dtype


def test_transpose_8191x4099_against_copy_spot_check(ctx, pool):
    """The reference benchmark's shape (permutation_test.rs:741-792), checked word for word."""
    m, n = 8191, 4099
    g = rng(3000)
    words = random_words(g, m * n)
    src_buf = pool.alloc("f32", m * n)
    src_buf.write(words)
    dst_buf = pool.alloc("f32", m * n)
    src = L.TensorView.row_major(src_buf, 0, [m, n])
    dst = L.TensorView.row_major(dst_buf, 0, [n, m])
    P.materialize(ctx, P.permute_view(src, [1, 0]), dst)
    got = dst_buf.read(np.uint32, count=m * n)
    assert np.array_equal(got, words.reshape(m, n).T.ravel())
