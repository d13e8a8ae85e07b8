// gfx950 permutation kernels: the tiled transpose (permutation_tile.h) instantiated at the
// library's tile geometry, and the gather copy.
//
// perm_copy: the destination is contiguous, so each thread produces 128 bits of it from a
// strided gather (odometer over the source strides); a fully contiguous source is a straight
// 128-bit copy.
#include <hip/hip_runtime.h>

#include "lg_internal.h"
#include "permutation_tile.h"

namespace lg {
namespace {

using perm_detail::perm_tile;
using perm_detail::SIGN;
using perm_detail::u32x4;

template <int W, bool CONJ, bool NT>
__global__ __launch_bounds__(PERM_THREADS) void perm_copy(PermCopyArgs p) {
    constexpr int VE = 4 / W;
    const uint32_t* src = static_cast<const uint32_t*>(p.src);
    uint32_t* dst = static_cast<uint32_t*>(p.dst);
    const uint64_t step = static_cast<uint64_t>(gridDim.x) * PERM_THREADS * VE;
    const int rank = static_cast<int>(p.rank);
    for (uint64_t i0 = (static_cast<uint64_t>(blockIdx.x) * PERM_THREADS + threadIdx.x) * VE;
         i0 < p.count; i0 += step) {
        const bool full = i0 + VE <= p.count;
        u32x4 v;
        if (p.contiguous) {
            const uint64_t s0 = p.src_offset + i0;
            if (full) {
                v = perm_detail::load128<NT>(src + s0 * W);
            } else {
                for (int e = 0; e < VE; ++e)
                    if (i0 + e < p.count)
                        for (int w = 0; w < W; ++w) v[e * W + w] = src[(s0 + e) * W + w];
            }
        } else {
            // Decode i0 into a multi-index, then step the odometer VE times.
            uint64_t idx[PERM_MAX_RANK];
            uint64_t r = i0;
            int64_t soff = static_cast<int64_t>(p.src_offset);
            for (int d = rank - 1; d >= 0; --d) {
                const uint64_t q = r / p.shape[d];
                idx[d] = r - q * p.shape[d];
                soff += static_cast<int64_t>(idx[d]) * p.strides[d];
                r = q;
            }
            for (int e = 0; e < VE; ++e) {
                if (i0 + e >= p.count) break;
                for (int w = 0; w < W; ++w) v[e * W + w] = src[soff * W + w];
                for (int d = rank - 1; d >= 0; --d) {
                    soff += p.strides[d];
                    if (++idx[d] < p.shape[d]) break;
                    soff -= static_cast<int64_t>(p.shape[d]) * p.strides[d];
                    idx[d] = 0;
                }
            }
        }
        if constexpr (CONJ) {
            for (int e = 0; e < VE; ++e) v[e * W + 1] ^= SIGN;
        }
        const uint64_t d0 = p.dst_offset + i0;
        if (full && p.vec_dst) {
            perm_detail::store128<NT>(dst + d0 * W, v);
        } else {
            for (int e = 0; e < VE; ++e)
                if (i0 + e < p.count)
                    for (int w = 0; w < W; ++w) dst[(d0 + e) * W + w] = v[e * W + w];
        }
    }
}

constexpr uint64_t TILE_GRID_CAP = 1u << 22;
constexpr uint64_t COPY_GRID_CAP = 1u << 20;

// Streaming (operands beyond the Infinity Cache) tiles are 64 x 256 with 1024 threads, cached
// ones 64 x 64 with 512: measured best on configs 2b and 2a respectively (2b: 6.14 TB/s against
// 6.0 for 128 x 64 tiles of 256 threads, whose destination row segments are 256 B; the 1 GiB
// tensor [1024,1024,256] 5.89 against 5.62. 2a: 6.44 against 6.21 with 256 threads).
template <int W, bool CONJ, bool VEC, int TA, bool NT>
void tile_t(hipStream_t s, const PermTileArgs& a) {
    constexpr int threads = NT ? PERM_STREAM_THREADS : PERM_CACHED_THREADS;
    constexpr int TB = NT ? PERM_STREAM_TILE_B : PERM_TILE_B;
    const uint64_t g = perm_tile_workgroups(a.total_tiles);
    hipLaunchKernelGGL((perm_tile<W, CONJ, VEC, TA, TB, NT ? 3 : 0, threads>),
                       dim3(static_cast<uint32_t>(g)), dim3(threads), 0, s, a);
}

template <int W, bool CONJ, bool NT>
void copy_t(hipStream_t s, const PermCopyArgs& a) {
    const dim3 grid(static_cast<uint32_t>(perm_copy_workgroups(a.count, W)));
    hipLaunchKernelGGL((perm_copy<W, CONJ, NT>), grid, dim3(PERM_THREADS), 0, s, a);
}

}  // namespace

uint64_t perm_tile_workgroups(uint64_t total_tiles) {
    return total_tiles < TILE_GRID_CAP ? (total_tiles ? total_tiles : 1) : TILE_GRID_CAP;
}

uint64_t perm_copy_workgroups(uint64_t count, int words) {
    const uint64_t per = static_cast<uint64_t>(PERM_THREADS) * (4 / words);
    const uint64_t g = (count + per - 1) / per;
    return g < COPY_GRID_CAP ? (g ? g : 1) : COPY_GRID_CAP;
}

void launch_perm_tile(Context* ctx, hipStream_t s, const PermTileArgs& a, int words, bool conj,
                      bool vec, bool streaming) {
    constexpr int TS = PERM_STREAM_TILE_A, TN = PERM_TILE_A;
    const char* name = nullptr;
    if (words == 1) {
        if (streaming) tile_t<1, false, true, TS, true>(s, a), name = "perm_tile_w1_v128_stream";
        else if (vec) tile_t<1, false, true, TN, false>(s, a), name = "perm_tile_w1_v128";
        else tile_t<1, false, false, TN, false>(s, a), name = "perm_tile_w1";
    } else if (!conj) {
        if (streaming) tile_t<2, false, true, TS, true>(s, a), name = "perm_tile_w2_v128_stream";
        else if (vec) tile_t<2, false, true, TN, false>(s, a), name = "perm_tile_w2_v128";
        else tile_t<2, false, false, TN, false>(s, a), name = "perm_tile_w2";
    } else {
        if (streaming) tile_t<2, true, true, TS, true>(s, a), name = "perm_tile_conj_w2_v128_stream";
        else if (vec) tile_t<2, true, true, TN, false>(s, a), name = "perm_tile_conj_w2_v128";
        else tile_t<2, true, false, TN, false>(s, a), name = "perm_tile_conj_w2";
    }
    check_hip(hipGetLastError(), "perm_tile launch");
    note_launch(ctx, name);
}

void launch_perm_copy(Context* ctx, hipStream_t s, const PermCopyArgs& a, int words, bool conj) {
    const bool nt = a.streaming != 0;
    const char* name;
    if (words == 1) {
        if (nt) copy_t<1, false, true>(s, a), name = "perm_copy_w1_stream";
        else copy_t<1, false, false>(s, a), name = "perm_copy_w1";
    } else if (!conj) {
        if (nt) copy_t<2, false, true>(s, a), name = "perm_copy_w2_stream";
        else copy_t<2, false, false>(s, a), name = "perm_copy_w2";
    } else {
        if (nt) copy_t<2, true, true>(s, a), name = "perm_copy_conj_w2_stream";
        else copy_t<2, true, false>(s, a), name = "perm_copy_conj_w2";
    }
    check_hip(hipGetLastError(), "perm_copy launch");
    note_launch(ctx, name);
}

}  // namespace lg
