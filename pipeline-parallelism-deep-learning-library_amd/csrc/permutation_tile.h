// The LDS-tiled transpose kernel of the permutation path, parameterized by geometry.
//
// Elements move as raw 32-bit words (W = 1 for f32/u32/i32, W = 2 for complex f32), so every
// NaN payload, -0 and subnormal survives bit for bit.
//
// perm_tile<W, CONJ, VEC, TA, TB>: batched 2-axis transpose of axes a (source unit stride) and
// b (destination unit stride). A TA x TB element tile is read with 128-bit loads running along
// a, staged in LDS with an odd word pitch (TA*W + 1) so both the row-wise fill and the
// column-wise drain spread over the banks, and written with 128-bit stores running along b.
// Tiles are walked with a grid stride in the order (outer, ta, tb), tb fastest: concurrently
// running workgroups write consecutive TB-element segments of the same TA destination rows, so
// every destination row is written front to back, and read consecutive bands of source rows.
// (On a 1 GiB transpose this order measured 2-3% faster than ta fastest on MI355X.)
// A tile that lies wholly inside the view takes a branch-free path: all of its 128-bit loads
// are issued before the first is waited on, and the drain reads LDS before it stores.
// Ragged tile edges and misaligned views fall back to 32-bit word accesses.
#pragma once

#include <hip/hip_runtime.h>

#include "lg_internal.h"

namespace lg {
namespace perm_detail {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t SIGN = 0x80000000u;

// 128-bit global accesses; NT marks them non-temporal (streamed past the caches).
// Tile kernels take NTM: bit 0 makes the loads non-temporal, bit 1 the stores.
template <bool NT>
__device__ inline u32x4 load128(const uint32_t* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    else return *reinterpret_cast<const u32x4*>(p);
}
template <bool NT>
__device__ inline void store128(uint32_t* p, u32x4 v) {
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
    else *reinterpret_cast<u32x4*>(p) = v;
}

template <int W, bool CONJ, bool VEC, int TA, int TB, int NTM, int NTH>
__global__ __launch_bounds__(NTH) void perm_tile(PermTileArgs p) {
    constexpr bool NTL = (NTM & 1) != 0, NTS = (NTM & 2) != 0;
    constexpr int VE = 4 / W;                       // elements per 128-bit word
    constexpr int PITCH = TA * W + 1;               // LDS row pitch in words (rows are b)
    constexpr int FILL_CHUNKS = TA * W / 4;         // 128-bit chunks per tile row (along a)
    constexpr int DRAIN_CHUNKS = TB * W / 4;        // 128-bit chunks per output row (along b)
    constexpr int FILL_ITERS = TB * FILL_CHUNKS / NTH;
    constexpr int DRAIN_ITERS = TA * DRAIN_CHUNKS / NTH;
    static_assert(FILL_ITERS * NTH == TB * FILL_CHUNKS, "fill must split evenly");
    static_assert(DRAIN_ITERS * NTH == TA * DRAIN_CHUNKS, "drain must split evenly");
    __shared__ uint32_t tile[TB * PITCH];

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
        const uint32_t a0 = ta * TA, b0 = tb * TB;
        // Workgroup-uniform: the whole tile lies inside the view and 128-bit accesses are
        // allowed. Then every load of the fill is issued before the first one is waited on,
        // and the drain reads all its LDS words before its stores, with no per-chunk
        // branches to serialize the memory pipeline.
        const bool inside = a0 + TA <= p.ext_a && b0 + TB <= p.ext_b;
        const bool full = VEC && inside;
        // A view that 128-bit accesses cannot serve (rows not 16-byte aligned, such as an odd
        // row pitch) still takes a branch-free path for interior tiles: 32-bit accesses with
        // lane i on word i of a row, so each wave instruction covers 256 contiguous bytes.
        constexpr int ROW_WORDS = TA * W;   // words of one tile row in the source (along a)
        constexpr int COL_WORDS = TB * W;   // words of one destination row segment (along b)
        constexpr int WORDS_IN = TB * ROW_WORDS / NTH;
        constexpr int WORDS_OUT = TA * COL_WORDS / NTH;
        static_assert(WORDS_IN * NTH == TB * ROW_WORDS, "word fill must split evenly");
        static_assert(WORDS_OUT * NTH == TA * COL_WORDS, "word drain must split evenly");
        const bool words_full = !VEC && inside;

        // Fill: rows of the tile are b, 128-bit chunks run along a.
        if (words_full) {
            if constexpr (!VEC) {
                uint32_t r[WORDS_IN];
#pragma unroll
                for (int it = 0; it < WORDS_IN; ++it) {
                    const int idx = it * NTH + tid;
                    const int bb = idx / ROW_WORDS, cw = idx % ROW_WORDS;
                    const int64_t e0 = sbase + static_cast<int64_t>(b0 + bb) * p.src_sb + a0;
                    r[it] = src[e0 * W + cw];
                }
#pragma unroll
                for (int it = 0; it < WORDS_IN; ++it) {
                    const int idx = it * NTH + tid;
                    tile[(idx / ROW_WORDS) * PITCH + idx % ROW_WORDS] = r[it];
                }
            }
        } else if (full) {
            u32x4 r[FILL_ITERS];
#pragma unroll
            for (int it = 0; it < FILL_ITERS; ++it) {
                const int idx = it * NTH + tid;
                const int bb = idx / FILL_CHUNKS, cw = (idx % FILL_CHUNKS) * 4;
                const int64_t e0 = sbase + static_cast<int64_t>(b0 + bb) * p.src_sb + a0 + cw / W;
                r[it] = load128<NTL>(src + e0 * W);
            }
#pragma unroll
            for (int it = 0; it < FILL_ITERS; ++it) {
                const int idx = it * NTH + tid;
                const int bb = idx / FILL_CHUNKS, cw = (idx % FILL_CHUNKS) * 4;
                uint32_t* row = tile + bb * PITCH + cw;
                row[0] = r[it][0];
                row[1] = r[it][1];
                row[2] = r[it][2];
                row[3] = r[it][3];
            }
        } else {
#pragma unroll
            for (int it = 0; it < FILL_ITERS; ++it) {
                const int idx = it * NTH + tid;
                const int bb = idx / FILL_CHUNKS, cw = (idx % FILL_CHUNKS) * 4;  // word column
                const uint32_t a = a0 + cw / W, b = b0 + bb;
                uint32_t* row = tile + bb * PITCH + cw;
                const int64_t e0 = sbase + static_cast<int64_t>(b) * p.src_sb + a;  // element
                if (VEC && b < p.ext_b && a + VE <= p.ext_a) {
                    const u32x4 v = load128<NTL>(src + e0 * W);
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
        }
        __syncthreads();

        // Drain: 128-bit chunks run along b, one destination row per a.
        auto gather = [&](int aa, int bl) {
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
            return v;
        };
        if (words_full) {
            if constexpr (!VEC) {
                uint32_t v[WORDS_OUT];
#pragma unroll
                for (int it = 0; it < WORDS_OUT; ++it) {
                    const int idx = it * NTH + tid;
                    const int aa = idx / COL_WORDS, cwb = idx % COL_WORDS;
                    const int w = cwb % W;
                    uint32_t word = tile[(cwb / W) * PITCH + aa * W + w];
                    if (CONJ && w == 1) word ^= SIGN;
                    v[it] = word;
                }
#pragma unroll
                for (int it = 0; it < WORDS_OUT; ++it) {
                    const int idx = it * NTH + tid;
                    const int aa = idx / COL_WORDS, cwb = idx % COL_WORDS;
                    const int64_t e0 = dbase + static_cast<int64_t>(a0 + aa) * p.dst_sa + b0;
                    dst[e0 * W + cwb] = v[it];
                }
            }
        } else if (full) {
            u32x4 v[DRAIN_ITERS];
#pragma unroll
            for (int it = 0; it < DRAIN_ITERS; ++it) {
                const int idx = it * NTH + tid;
                v[it] = gather(idx / DRAIN_CHUNKS, (idx % DRAIN_CHUNKS) * 4 / W);
            }
#pragma unroll
            for (int it = 0; it < DRAIN_ITERS; ++it) {
                const int idx = it * NTH + tid;
                const int aa = idx / DRAIN_CHUNKS, bl = (idx % DRAIN_CHUNKS) * 4 / W;
                const int64_t e0 = dbase + static_cast<int64_t>(a0 + aa) * p.dst_sa + b0 + bl;
                store128<NTS>(dst + e0 * W, v[it]);
            }
        } else {
#pragma unroll
            for (int it = 0; it < DRAIN_ITERS; ++it) {
                const int idx = it * NTH + tid;
                const int aa = idx / DRAIN_CHUNKS, cw = (idx % DRAIN_CHUNKS) * 4;
                const int bl = cw / W;  // first b (local) of this chunk
                const uint32_t a = a0 + aa, b = b0 + bl;
                const u32x4 v = gather(aa, bl);
                const int64_t e0 = dbase + static_cast<int64_t>(a) * p.dst_sa + b;
                if (VEC && a < p.ext_a && b + VE <= p.ext_b) {
                    store128<NTS>(dst + e0 * W, v);
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
        }
        __syncthreads();
    }
}

}  // namespace perm_detail
}  // namespace lg
