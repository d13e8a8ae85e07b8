// The LDS-tiled transpose kernel of the permutation path, parameterized by geometry.
//
// Elements move as raw 32-bit words (W = 1 for f32/u32/i32, W = 2 for complex f32), so every
// NaN payload, -0 and subnormal survives bit for bit.
//
// perm_tile<W, CONJ, VEC, TA, TB>: batched 2-axis transpose of axes a (source unit stride) and
// b (destination unit stride). A TA x TB element tile is read with 128-bit loads running along
// a, staged in LDS with an odd word pitch (TA*W + 1) so both the row-wise fill and the
// column-wise drain spread over the banks, and written with 128-bit stores running along b.
// Tiles are walked with a grid stride in the order (outer, tb, ta): the `a` tiles of one band
// of source rows are consecutive, so concurrently running workgroups read whole source rows
// (DRAM pages stay open) and write adjacent TB-element segments of the same destination rows.
// Ragged tile edges and misaligned views fall back to 32-bit word accesses.
#pragma once

#include <hip/hip_runtime.h>

#include "lg_internal.h"

namespace lg {
namespace perm_detail {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t SIGN = 0x80000000u;

template <int W, bool CONJ, bool VEC, int TA, int TB>
__global__ __launch_bounds__(PERM_THREADS) void perm_tile(PermTileArgs p) {
    constexpr int VE = 4 / W;                       // elements per 128-bit word
    constexpr int PITCH = TA * W + 1;               // LDS row pitch in words (rows are b)
    constexpr int FILL_CHUNKS = TA * W / 4;         // 128-bit chunks per tile row (along a)
    constexpr int DRAIN_CHUNKS = TB * W / 4;        // 128-bit chunks per output row (along b)
    constexpr int FILL_ITERS = TB * FILL_CHUNKS / PERM_THREADS;
    constexpr int DRAIN_ITERS = TA * DRAIN_CHUNKS / PERM_THREADS;
    static_assert(FILL_ITERS * PERM_THREADS == TB * FILL_CHUNKS, "fill must split evenly");
    static_assert(DRAIN_ITERS * PERM_THREADS == TA * DRAIN_CHUNKS, "drain must split evenly");
    __shared__ uint32_t tile[TB * PITCH];

    const uint32_t* src = static_cast<const uint32_t*>(p.src);
    uint32_t* dst = static_cast<uint32_t*>(p.dst);
    const int tid = threadIdx.x;
    const uint64_t per_outer = static_cast<uint64_t>(p.tiles_a) * p.tiles_b;

    for (uint64_t t = blockIdx.x; t < p.total_tiles; t += gridDim.x) {
        uint64_t outer = t / per_outer;
        const uint64_t rem = t - outer * per_outer;
        const uint32_t tb = static_cast<uint32_t>(rem / p.tiles_a);
        const uint32_t ta = static_cast<uint32_t>(rem - static_cast<uint64_t>(tb) * p.tiles_a);
        int64_t sbase = static_cast<int64_t>(p.src_offset);
        int64_t dbase = static_cast<int64_t>(p.dst_offset);
        for (int d = static_cast<int>(p.outer_rank) - 1; d >= 0; --d) {
            const uint64_t q = outer / p.outer_shape[d];
            const int64_t c = static_cast<int64_t>(outer - q * p.outer_shape[d]);
            sbase += c * p.outer_src[d];
            dbase += c * p.outer_dst[d];
            outer = q;
        }
        const uint32_t a0 = ta * TA, b0 = tb * TB;

        // Fill: rows of the tile are b, 128-bit chunks run along a.
#pragma unroll
        for (int it = 0; it < FILL_ITERS; ++it) {
            const int idx = it * PERM_THREADS + tid;
            const int bb = idx / FILL_CHUNKS, cw = (idx % FILL_CHUNKS) * 4;  // word column
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
        for (int it = 0; it < DRAIN_ITERS; ++it) {
            const int idx = it * PERM_THREADS + tid;
            const int aa = idx / DRAIN_CHUNKS, cw = (idx % DRAIN_CHUNKS) * 4;
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

}  // namespace perm_detail
}  // namespace lg
