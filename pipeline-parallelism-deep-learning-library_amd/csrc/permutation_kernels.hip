// gfx950 permutation kernels. Elements move as raw 32-bit words (W = 1 for f32/u32/i32,
// W = 2 for complex f32), so every NaN payload, -0 and subnormal survives bit for bit.
//
// perm_tile: batched 2-axis transpose of axes a (source unit stride) and b (destination
// unit stride). A 64x64-element tile is read with 128-bit loads running along a, staged in
// LDS with an odd word pitch (64*W + 1) so both the row-wise fill and the column-wise drain
// spread over the banks, and written with 128-bit stores running along b. Each workgroup
// walks tiles with a grid stride; the remaining ("outer") axes are decoded per tile.
// Ragged tile edges and misaligned views fall back to 32-bit word accesses.
//
// perm_copy: the destination is contiguous, so each thread produces 128 bits of it from a
// strided gather (odometer over the source strides); a fully contiguous source is a straight
// 128-bit copy.
#include <hip/hip_runtime.h>

#include "lg_internal.h"

namespace lg {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t SIGN = 0x80000000u;
constexpr int T = PERM_TILE;

template <int W, bool CONJ, bool VEC>
__global__ __launch_bounds__(PERM_THREADS) void perm_tile(PermTileArgs p) {
    constexpr int VE = 4 / W;              // elements per 128-bit word
    constexpr int PITCH = T * W + 1;       // LDS row pitch in words
    constexpr int CHUNKS = T * W / 4;      // 128-bit chunks per tile row
    constexpr int ITERS = T * CHUNKS / PERM_THREADS;
    __shared__ uint32_t tile[T * PITCH];

    const uint32_t* src = static_cast<const uint32_t*>(p.src);
    uint32_t* dst = static_cast<uint32_t*>(p.dst);
    const int tid = threadIdx.x;
    const uint64_t per_outer = static_cast<uint64_t>(p.tiles_a) * p.tiles_b;

    for (uint64_t t = blockIdx.x; t < p.total_tiles; t += gridDim.x) {
        uint64_t outer = t / per_outer;
        const uint64_t rem = t - outer * per_outer;
        const uint32_t ta = static_cast<uint32_t>(rem / p.tiles_b);
        const uint32_t tb = static_cast<uint32_t>(rem - static_cast<uint64_t>(ta) * p.tiles_b);
        int64_t sbase = static_cast<int64_t>(p.src_offset);
        int64_t dbase = static_cast<int64_t>(p.dst_offset);
        for (int d = static_cast<int>(p.outer_rank) - 1; d >= 0; --d) {
            const uint64_t q = outer / p.outer_shape[d];
            const int64_t c = static_cast<int64_t>(outer - q * p.outer_shape[d]);
            sbase += c * p.outer_src[d];
            dbase += c * p.outer_dst[d];
            outer = q;
        }
        const uint32_t a0 = ta * T, b0 = tb * T;

        // Fill: rows of the tile are b, 128-bit chunks run along a.
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const int idx = it * PERM_THREADS + tid;
            const int bb = idx / CHUNKS, cw = (idx % CHUNKS) * 4;  // word column
            const uint32_t a = a0 + cw / W, b = b0 + bb;
            uint32_t* row = tile + bb * PITCH + cw;
            const int64_t e0 = sbase + static_cast<int64_t>(b) * p.src_sb + a;  // element index
            if (VEC && b < p.ext_b && a + VE <= p.ext_a) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(src + e0 * W);
                row[0] = v[0];
                row[1] = v[1];
                row[2] = v[2];
                row[3] = v[3];
            } else {
#pragma unroll
                for (int e = 0; e < VE; ++e) {
                    if (b < p.ext_b && a + e < p.ext_a) {
#pragma unroll
                        for (int w = 0; w < W; ++w) row[e * W + w] = src[(e0 + e) * W + w];
                    }
                }
            }
        }
        __syncthreads();

        // Drain: 128-bit chunks run along b, one destination row per a.
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const int idx = it * PERM_THREADS + tid;
            const int aa = idx / CHUNKS, cw = (idx % CHUNKS) * 4;
            const int bl = cw / W;  // first b (local) of this chunk
            const uint32_t a = a0 + aa, b = b0 + bl;
            u32x4 v;
#pragma unroll
            for (int e = 0; e < VE; ++e) {
#pragma unroll
                for (int w = 0; w < W; ++w) {
                    uint32_t word = tile[(bl + e) * PITCH + aa * W + w];
                    if (CONJ && w == 1) word ^= SIGN;
                    v[e * W + w] = word;
                }
            }
            const int64_t e0 = dbase + static_cast<int64_t>(a) * p.dst_sa + b;
            if (VEC && a < p.ext_a && b + VE <= p.ext_b) {
                *reinterpret_cast<u32x4*>(dst + e0 * W) = v;
            } else {
#pragma unroll
                for (int e = 0; e < VE; ++e) {
                    if (a < p.ext_a && b + e < p.ext_b) {
#pragma unroll
                        for (int w = 0; w < W; ++w) dst[(e0 + e) * W + w] = v[e * W + w];
                    }
                }
            }
        }
        __syncthreads();
    }
}

template <int W, bool CONJ>
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
                v = *reinterpret_cast<const u32x4*>(src + s0 * W);
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
            *reinterpret_cast<u32x4*>(dst + d0 * W) = v;
        } else {
            for (int e = 0; e < VE; ++e)
                if (i0 + e < p.count)
                    for (int w = 0; w < W; ++w) dst[(d0 + e) * W + w] = v[e * W + w];
        }
    }
}

constexpr uint64_t TILE_GRID_CAP = 1u << 22;
constexpr uint64_t COPY_GRID_CAP = 1u << 20;

template <int W, bool CONJ, bool VEC>
void tile_t(hipStream_t s, const PermTileArgs& a) {
    const uint64_t g = perm_tile_workgroups(a.total_tiles);
    hipLaunchKernelGGL((perm_tile<W, CONJ, VEC>), dim3(static_cast<uint32_t>(g)),
                       dim3(PERM_THREADS), 0, s, a);
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
                      bool vec) {
    const char* name = nullptr;
    if (words == 1) {
        if (vec) tile_t<1, false, true>(s, a), name = "perm_tile_w1_v128";
        else tile_t<1, false, false>(s, a), name = "perm_tile_w1";
    } else if (!conj) {
        if (vec) tile_t<2, false, true>(s, a), name = "perm_tile_w2_v128";
        else tile_t<2, false, false>(s, a), name = "perm_tile_w2";
    } else {
        if (vec) tile_t<2, true, true>(s, a), name = "perm_tile_conj_w2_v128";
        else tile_t<2, true, false>(s, a), name = "perm_tile_conj_w2";
    }
    check_hip(hipGetLastError(), "perm_tile launch");
    note_launch(ctx, name);
}

void launch_perm_copy(Context* ctx, hipStream_t s, const PermCopyArgs& a, int words, bool conj) {
    const dim3 grid(static_cast<uint32_t>(perm_copy_workgroups(a.count, words)));
    const char* name;
    if (words == 1) {
        hipLaunchKernelGGL((perm_copy<1, false>), grid, dim3(PERM_THREADS), 0, s, a);
        name = "perm_copy_w1";
    } else if (!conj) {
        hipLaunchKernelGGL((perm_copy<2, false>), grid, dim3(PERM_THREADS), 0, s, a);
        name = "perm_copy_w2";
    } else {
        hipLaunchKernelGGL((perm_copy<2, true>), grid, dim3(PERM_THREADS), 0, s, a);
        name = "perm_copy_conj_w2";
    }
    check_hip(hipGetLastError(), "perm_copy launch");
    note_launch(ctx, name);
}

}  // namespace lg
