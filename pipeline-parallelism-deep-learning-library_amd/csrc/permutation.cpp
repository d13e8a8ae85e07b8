// Permutation: axis-permuted views, contiguous materialization, conjugate and adjoint.
//
// Host half of the permutation hot path. Follows the reference's operator semantics
// (src/ops/permutation.rs): permute_view is metadata only (:295-320); every gather checks,
// in this order, both views, equal shapes, a contiguous row-major destination, overlap, and
// emptiness (:163-198); coalesces the source (:107-132); then picks a path (:200-216):
//   * the destination's unit-stride axis is the last one; if the source is not unit stride
//     there but is along some other axis `a`, the two axes are transposed through LDS;
//   * otherwise a gather whose writes are contiguous.
// Differences by design: indexing is 64-bit (no 2^31 element limit), and both paths move
// 128-bit words whenever alignment allows.
#include <algorithm>
#include <cstring>

#include "lg_internal.h"

namespace lg {
namespace {

struct ElemInfo {
    uint32_t bytes;
    int words;
    bool complex;
};

ElemInfo elem_info(lg_elem e) {
    switch (e) {
        case LG_ELEM_F32:
        case LG_ELEM_U32:
        case LG_ELEM_I32:
            return {4, 1, false};
        case LG_ELEM_C32:
            return {8, 2, true};
    }
    fail_invalid("unknown element type " + std::to_string(static_cast<int>(e)));
}

// permute_view (src/ops/permutation.rs:295-320).
View permute(const View& v, const std::vector<uint64_t>& perm) {
    const size_t rank = v.shape.size();
    if (v.strides.size() != rank) {
        fail_invalid("rank mismatch: shape " + fmt_vec(v.shape) + " vs strides " +
                     fmt_vec(v.strides));
    }
    bool ok = perm.size() == rank;
    std::vector<bool> seen(rank, false);
    for (size_t i = 0; ok && i < perm.size(); ++i) {
        if (perm[i] >= rank || seen[perm[i]]) ok = false;
        else seen[perm[i]] = true;
    }
    if (!ok) fail_invalid(fmt_vec(perm) + " is not a permutation of 0.." + std::to_string(rank));
    View out = v;
    for (size_t i = 0; i < rank; ++i) {
        out.shape[i] = v.shape[perm[i]];
        out.strides[i] = v.strides[perm[i]];
    }
    return out;
}

// swap_last_two (src/ops/permutation.rs:284-293).
View swap_last_two(const View& v) {
    const size_t rank = v.shape.size();
    if (rank < 2) fail_invalid("adjoint needs at least 2 axes, got " + std::to_string(rank));
    std::vector<uint64_t> perm(rank);
    for (size_t i = 0; i < rank; ++i) perm[i] = i;
    std::swap(perm[rank - 2], perm[rank - 1]);
    return permute(v, perm);
}

// coalesce (src/ops/permutation.rs:107-132): drop unit axes, merge an axis into the
// previous one when the pair is contiguous in the source. Never empty.
void coalesce(const View& v, std::vector<uint64_t>* shape, std::vector<uint64_t>* strides) {
    shape->clear();
    strides->clear();
    for (size_t d = 0; d < v.shape.size(); ++d) {
        const uint64_t n = v.shape[d], s = v.strides[d];
        if (n == 1) continue;
        if (!shape->empty()) {
            // s * n == previous stride, without overflow.
            const uint64_t prev = strides->back();
            if (n != 0 && s <= UINT64_MAX / n && s * n == prev) {
                shape->back() *= n;
                strides->back() = s;
                continue;
            }
        }
        shape->push_back(n);
        strides->push_back(s);
    }
    if (shape->empty()) {
        shape->push_back(1);
        strides->push_back(1);
    }
}

struct Gather {
    lg_permute_plan info{};
    PermTileArgs tile{};
    PermCopyArgs copy{};
    int words = 1;
    bool conj = false;
};

// Kernel extents are 31-bit: the tile kernels add a tile's extent to a coordinate in 32-bit
// arithmetic, which must not wrap.
uint32_t fit32(uint64_t x, const char* what) {
    if (x > 0x7fffffffull) fail_invalid(std::string(what) + " " + std::to_string(x) +
                                        " does not fit 31-bit kernel extents");
    return static_cast<uint32_t>(x);
}

int64_t fit_stride(uint64_t x, const char* what) {
    if (x > static_cast<uint64_t>(INT64_MAX)) fail_invalid(std::string(what) + " too large");
    return static_cast<int64_t>(x);
}

// Validation and planning of one gather (encode_gather, src/ops/permutation.rs:163-270).
Gather plan_gather(lg_elem elem, const View& src, const View& dst, bool conj_requested) {
    const ElemInfo e = elem_info(elem);
    validate(src, e.bytes);
    validate(dst, e.bytes);
    if (src.shape != dst.shape) {
        fail_invalid("destination shape " + fmt_vec(dst.shape) +
                     " does not match source shape " + fmt_vec(src.shape));
    }
    const std::vector<uint64_t> dense = row_major_strides(dst.shape);
    for (size_t d = 0; d < dst.shape.size(); ++d) {
        if (dst.shape[d] != 1 && dst.strides[d] != dense[d]) {
            fail_invalid("destination must be contiguous row-major, got strides " +
                         fmt_vec(dst.strides) + " for shape " + fmt_vec(dst.shape));
        }
    }
    if (may_overlap(src, e.bytes, dst, e.bytes)) fail_overlap("destination overlaps the source");

    Gather g;
    g.words = e.words;
    g.conj = conj_requested && e.complex;
    g.info.conj = g.conj ? 1 : 0;
    uint64_t f, l;
    if (!element_range(src, &f, &l) || !element_range(dst, &f, &l)) {
        g.info.kind = LG_PERMUTE_EMPTY;
        return g;
    }

    std::vector<uint64_t> shape, strides;
    coalesce(src, &shape, &strides);
    const size_t rank = shape.size();
    if (rank > PERM_MAX_RANK) {
        fail_invalid("rank " + std::to_string(rank) + " exceeds " +
                     std::to_string(PERM_MAX_RANK) + " after merging contiguous axes");
    }
    g.info.rank = static_cast<uint32_t>(rank);
    std::copy(shape.begin(), shape.end(), g.info.shape);
    std::copy(strides.begin(), strides.end(), g.info.strides);
    const std::vector<uint64_t> dst_strides = row_major_strides(shape);
    const uint64_t ve = 4 / static_cast<uint64_t>(e.words);  // elements per 128-bit word

    const size_t b = rank - 1;
    size_t a = rank;
    if (strides[b] != 1) {
        for (size_t d = 0; d < b; ++d) {
            if (strides[d] == 1) {
                a = d;
                break;
            }
        }
    }

    if (a == rank) {
        // Gather with contiguous destination writes.
        g.info.kind = LG_PERMUTE_COPY;
        PermCopyArgs& p = g.copy;
        p.src = reinterpret_cast<const void*>(src.base);
        p.dst = reinterpret_cast<void*>(dst.base);
        p.src_offset = src.offset;
        p.dst_offset = dst.offset;
        p.count = dst.len();
        p.rank = static_cast<uint32_t>(rank);
        for (size_t d = 0; d < rank; ++d) {
            p.shape[d] = shape[d];
            p.strides[d] = fit_stride(strides[d], "source stride");
        }
        p.vec_dst = (dst.base % 16 == 0 && dst.offset % ve == 0) ? 1 : 0;
        p.contiguous = (rank == 1 && strides[0] == 1 && src.base % 16 == 0 &&
                        src.offset % ve == 0 && p.vec_dst) ? 1 : 0;
        p.streaming = (p.contiguous && 2 * p.count * e.bytes > PERM_STREAM_BYTES) ? 1 : 0;
        g.info.vector = p.contiguous;
        g.info.streaming = p.streaming;
        g.info.workgroups = perm_copy_workgroups(p.count, e.words);
        return g;
    }

    g.info.kind = LG_PERMUTE_TILE;
    g.info.axis_a = static_cast<uint32_t>(a);
    g.info.axis_b = static_cast<uint32_t>(b);
    PermTileArgs& p = g.tile;
    p.src = reinterpret_cast<const void*>(src.base);
    p.dst = reinterpret_cast<void*>(dst.base);
    p.src_offset = src.offset;
    p.dst_offset = dst.offset;
    p.ext_a = fit32(shape[a], "extent");
    p.ext_b = fit32(shape[b], "extent");
    p.src_sb = fit_stride(strides[b], "source stride");
    p.dst_sa = fit_stride(dst_strides[a], "destination stride");
    // 128-bit accesses: both views' first elements 16-byte aligned, strides multiples of a
    // 128-bit word.
    bool vec = src.base % 16 == 0 && dst.base % 16 == 0 && src.offset % ve == 0 &&
               dst.offset % ve == 0 && strides[b] % ve == 0 && dst_strides[a] % ve == 0;
    uint32_t o = 0;
    uint64_t outer_count = 1;
    for (size_t d = 0; d < rank; ++d) {
        if (d == a || d == b) continue;
        p.outer_shape[o] = fit32(shape[d], "extent");
        p.outer_src[o] = fit_stride(strides[d], "source stride");
        p.outer_dst[o] = fit_stride(dst_strides[d], "destination stride");
        vec = vec && strides[d] % ve == 0 && dst_strides[d] % ve == 0;
        outer_count *= shape[d];
        ++o;
    }
    p.outer_rank = o;
    const uint64_t moved = 2 * dst.len() * e.bytes;
    g.info.streaming = (vec && moved > PERM_STREAM_BYTES) ? 1 : 0;
    const uint32_t tile_a = g.info.streaming ? PERM_STREAM_TILE_A : PERM_TILE_A;
    const uint32_t tile_b = g.info.streaming ? PERM_STREAM_TILE_B : PERM_TILE_B;
    p.tiles_a = static_cast<uint32_t>((shape[a] + tile_a - 1) / tile_a);
    p.tiles_b = static_cast<uint32_t>((shape[b] + tile_b - 1) / tile_b);
    p.total_tiles = static_cast<uint64_t>(p.tiles_a) * p.tiles_b * outer_count;
    g.info.vector = vec ? 1 : 0;
    g.info.workgroups = perm_tile_workgroups(p.total_tiles);
    return g;
}

Gather plan_op(uint32_t op, lg_elem elem, const lg_view* src_c, const lg_view* dst_c) {
    View src = view_from_c(src_c, "source");
    View dst = view_from_c(dst_c, "destination");
    switch (op) {
        case 0:
            return plan_gather(elem, src, dst, false);
        case 1:
            return plan_gather(elem, src, dst, true);
        case 2:
            return plan_gather(elem, swap_last_two(src), dst, true);
    }
    fail_invalid("unknown permutation op");
}

void run(lg_ctx* ctx, void* stream, uint32_t op, lg_elem elem, const lg_view* src,
         const lg_view* dst, bool wait) {
    if (ctx == nullptr) fail_invalid("null context");
    const Gather g = plan_op(op, elem, src, dst);
    if (g.info.kind == LG_PERMUTE_EMPTY) {
        if (wait) {
            set_device(ctx);
            check_hip(hipStreamSynchronize(pick_stream(ctx, stream)), "hipStreamSynchronize");
        }
        return;
    }
    set_device(ctx);
    hipStream_t s = pick_stream(ctx, stream);
    if (g.info.kind == LG_PERMUTE_TILE) {
        launch_perm_tile(ctx, s, g.tile, g.words, g.conj, g.info.vector != 0,
                         g.info.streaming != 0);
    } else {
        launch_perm_copy(ctx, s, g.copy, g.words, g.conj);
    }
    if (wait) check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
}

}  // namespace
}  // namespace lg

using namespace lg;

extern "C" {

lg_status lg_permute_view(const lg_view* view, const uint64_t* perm, uint32_t perm_len,
                          lg_view* out) {
    return guarded([&] {
        if (out == nullptr) fail_invalid("null output view");
        if (perm == nullptr && perm_len != 0) fail_invalid("null permutation");
        const View v = view_from_c(view, "view");
        std::vector<uint64_t> p(perm, perm + perm_len);
        view_to_c(permute(v, p), out);
    });
}

lg_status lg_encode_materialize(lg_ctx* ctx, void* stream, lg_elem elem, const lg_view* src,
                                const lg_view* dst) {
    return guarded([&] { run(ctx, stream, 0, elem, src, dst, false); });
}
lg_status lg_materialize(lg_ctx* ctx, lg_elem elem, const lg_view* src, const lg_view* dst) {
    return guarded([&] { run(ctx, nullptr, 0, elem, src, dst, true); });
}
lg_status lg_encode_conjugate(lg_ctx* ctx, void* stream, lg_elem elem, const lg_view* src,
                              const lg_view* dst) {
    return guarded([&] { run(ctx, stream, 1, elem, src, dst, false); });
}
lg_status lg_conjugate(lg_ctx* ctx, lg_elem elem, const lg_view* src, const lg_view* dst) {
    return guarded([&] { run(ctx, nullptr, 1, elem, src, dst, true); });
}
lg_status lg_encode_adjoint(lg_ctx* ctx, void* stream, lg_elem elem, const lg_view* src,
                            const lg_view* dst) {
    return guarded([&] { run(ctx, stream, 2, elem, src, dst, false); });
}
lg_status lg_adjoint(lg_ctx* ctx, lg_elem elem, const lg_view* src, const lg_view* dst) {
    return guarded([&] { run(ctx, nullptr, 2, elem, src, dst, true); });
}

lg_status lg_plan_permute(uint32_t op, lg_elem elem, const lg_view* src, const lg_view* dst,
                          lg_permute_plan* out) {
    return guarded([&] {
        if (out == nullptr) fail_invalid("null output plan");
        const Gather g = plan_op(op, elem, src, dst);
        *out = g.info;
    });
}

}  // extern "C"
