// The fp32 MFMA GEMM kernel of the contraction path, parameterized by pipeline shape.
//
// gemm_f32_mfma<AM, BMD, BK, TM, TN>: C = beta * C + sum_k (alpha * a) * b (or raw split-K
// partials of the sum) for one stride per group. A (64*TM) x (64*TN) output tile per
// 256-thread workgroup (4 waves in 2x2, each wave TM x TN blocks of v_mfma_f32_32x32x2_f32
// accumulating in fp32); the library uses it for 64x64 tiles and for 128x128 tiles of
// operands without a 16-byte aligned unit-stride axis (the others take gemm_f32_dl, with
// slices loaded straight into LDS; gemm_dlds.h). K advances BK at a
// time through two LDS stages: while the MFMAs consume stage s, the next K-slice is already in
// flight from HBM into registers, and is written to stage s^1 before the one barrier per
// slice. Operand loads follow the operand's unit-stride axis so a transposed or permuted
// view is read as it lies, 128 bits per load:
//   LOAD_K  : unit stride along K   -> LDS [row][k] (pitch BK+4), 128-bit LDS reads along k
//   LOAD_MN : unit stride along M/N -> LDS [k][row] (pitch 136), 32-bit LDS reads
//   LOAD_S  : anything else         -> 32-bit predicated loads into the [row][k] layout
// Inside a K-slice, MFMA step s of lane half h uses k = 8*(s/4) + 4*h + s%4, so a [row][k]
// stage hands each lane four consecutive k with one ds_read_b128. A and B agree on this order,
// so every product pairs the same k.
// The 128x128 kernel is held to 128 VGPRs (accumulators included) so four workgroups share a
// compute unit: one wave per SIMD from each, whose LDS waits and barriers the other three
// cover. With that much cover, reading each step group's fragments just before its MFMAs
// beats double-buffering them in registers, and the MFMA block runs at raised wave priority
// so a wave that has its operands issues ahead of waves busy with loads. The strided (LOAD_S)
// forms need more registers than that and keep the compiler's default.
#pragma once

#include <hip/hip_runtime.h>

#include "lg_internal.h"

namespace lg {
namespace gemm_detail {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// Stage geometry of one operand whose tile spans R rows (M for A, N for B) and BK k.
template <int BK, int R>
struct Geo {
    static constexpr int PK = BK + 4;                          // pitch of a [row][k] stage
    static constexpr int PR = R + 8;                           // pitch of a [k][row] stage
    static constexpr int LOADS = (R * BK / 4) / GEMM_THREADS;  // 128-bit loads per thread
    static_assert(LOADS * GEMM_THREADS * 4 == R * BK, "tile must split evenly over threads");
    template <int MODE>
    static constexpr int stage() { return MODE == LOAD_MN ? BK * PR : R * PK; }
};

// Workgroup -> (plane, tile_m, tile_n). Workgroups are dealt round-robin to the 8 XCDs, so
// the linear id is first regrouped so each XCD owns one contiguous run of tiles (sharing
// its L2), then tiles within a plane are walked in groups of GROUP tile-rows for A/B reuse:
// an XCD's resident tiles then cover GROUP tile-rows by a few tile-columns.
template <uint32_t GROUP = 8>
__device__ inline void decode_tile(uint32_t bid, uint32_t total, uint32_t tiles_m,
                                   uint32_t tiles_n, uint32_t* plane, uint32_t* tm,
                                   uint32_t* tn) {
    const uint32_t xcd = bid & 7u, slot = bid >> 3;
    const uint32_t q = total >> 3, r = total & 7u;
    const uint32_t lin = xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
    const uint32_t per_plane = tiles_m * tiles_n;
    *plane = lin / per_plane;
    const uint32_t t = lin - *plane * per_plane;
    const uint32_t group_size = GROUP * tiles_n;
    const uint32_t group = t / group_size;
    const uint32_t first_m = group * GROUP;
    const uint32_t gm = min(tiles_m - first_m, GROUP);
    const uint32_t in_group = t - group * group_size;
    *tm = first_m + in_group % gm;
    *tn = in_group / gm;
}

// Loads one operand's K-slice (rows [0, rows_left) x k [k0, k0+BK) within klen) into
// registers. `p` points at (row 0, k 0) of the tile; srow/sk are the operand's strides.
// FULL (workgroup-uniform: the whole slice is inside the operand) takes branch-free 128-bit
// loads so every load of the slice is in flight at once; edge slices predicate each element.
template <int MODE, bool FULL, int BK, int R, typename G = Geo<BK, R>>
__device__ inline void load_slice(floatx4 (&r)[G::LOADS], const float* __restrict__ p,
                                  int64_t srow, int64_t sk, uint32_t rows_left, uint32_t k0,
                                  uint32_t klen, int tid) {
#pragma unroll
    for (int i = 0; i < Geo<BK, R>::LOADS; ++i) {
        const int idx = i * GEMM_THREADS + tid;
        if constexpr (MODE == LOAD_MN) {
            const uint32_t kr = k0 + idx / (R / 4);
            const uint32_t row = (idx % (R / 4)) * 4;
            const float* q = p + static_cast<int64_t>(kr) * sk + row;
            if (FULL || (kr < klen && row + 4 <= rows_left)) {
                r[i] = *reinterpret_cast<const floatx4*>(q);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) r[i][e] = (kr < klen && row + e < rows_left) ? q[e] : 0.0f;
            }
        } else {
            const uint32_t row = idx / (BK / 4);
            const uint32_t kk = k0 + (idx % (BK / 4)) * 4;
            if constexpr (MODE == LOAD_K) {
                const float* q = p + static_cast<int64_t>(row) * srow + kk;
                if (FULL || (row < rows_left && kk + 4 <= klen)) {
                    r[i] = *reinterpret_cast<const floatx4*>(q);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) r[i][e] = (row < rows_left && kk + e < klen) ? q[e] : 0.0f;
                }
            } else {
                const float* q = p + static_cast<int64_t>(row) * srow;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    r[i][e] = (FULL || (row < rows_left && kk + e < klen))
                                  ? q[static_cast<int64_t>(kk + e) * sk]
                                  : 0.0f;
                }
            }
        }
    }
}

// The thread's first element of load i in a K-slice at k = 0 (LOAD_K and LOAD_MN): the slice
// at k0 then starts k0 (LOAD_K) or k0*sk (LOAD_MN) elements later, one uniform offset, so an
// interior slice costs one address add per load instead of a 64-bit multiply.
template <int MODE, int BK, int R>
__device__ inline const float* slice_ptr(const float* p, int64_t srow, int64_t sk, int i, int tid) {
    const int idx = i * GEMM_THREADS + tid;
    if constexpr (MODE == LOAD_MN) {
        return p + static_cast<int64_t>(idx / (R / 4)) * sk + (idx % (R / 4)) * 4;
    } else {
        return p + static_cast<int64_t>(idx / (BK / 4)) * srow + (idx % (BK / 4)) * 4;
    }
}

// Writes a loaded K-slice into its LDS stage. With SCALE every element is first multiplied by
// alpha (unless alpha is 1), so each product the MFMAs form is (alpha*a)*b. alpha is finite here
// (the planner sends non-finite alpha to the general kernel), so zero padding stays zero.
template <int MODE, int BK, int R, bool SCALE, typename G = Geo<BK, R>>
__device__ inline void store_slice(float* __restrict__ st, const floatx4 (&r)[G::LOADS],
                                   int tid, float alpha) {
#pragma unroll
    for (int i = 0; i < Geo<BK, R>::LOADS; ++i) {
        const int idx = i * GEMM_THREADS + tid;
        floatx4 v = r[i];
        if constexpr (SCALE) {
            if (alpha != 1.0f) v = v * alpha;  // (1*a)*b is a*b: skip the multiply
        }
        if constexpr (MODE == LOAD_MN) {
            const int kr = idx / (R / 4), row = (idx % (R / 4)) * 4;
            *reinterpret_cast<floatx4*>(st + kr * Geo<BK, R>::PR + row) = v;
        } else {
            const int row = idx / (BK / 4), kq = (idx % (BK / 4)) * 4;
            *reinterpret_cast<floatx4*>(st + row * Geo<BK, R>::PK + kq) = v;
        }
    }
}

// Operand values of the NB 32-row blocks `base_row + 32*i` for MFMA steps 4g..4g+3.
template <int MODE, int BK, int R, int NB>
__device__ inline void read_frag(floatx4 (&v)[NB], const float* __restrict__ st, int base_row,
                                 int g, int lr, int h) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int row = base_row + i * 32 + lr;
        if constexpr (MODE == LOAD_MN) {
#pragma unroll
            for (int s = 0; s < 4; ++s) v[i][s] = st[(g * 8 + h * 4 + s) * Geo<BK, R>::PR + row];
        } else {
            v[i] = *reinterpret_cast<const floatx4*>(st + row * Geo<BK, R>::PK + g * 8 + h * 4);
        }
    }
}

template <int TM, int TN>
__device__ inline void mfma_group(floatx16 (&acc)[TM][TN], const floatx4 (&av)[TM],
                                  const floatx4 (&bv)[TN]) {
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][st], bv[j][st], acc[i][j],
                                                                 0, 0, 0);
}

// TM x TN blocks of 32x32 per wave, waves in 2x2: the workgroup tile is (64*TM) x (64*TN). The
// next K-slice is requested at the top of a slice and written to LDS after the slice's MFMAs.
template <int AM, int BMD, int BK, int TM, int TN>
__global__ __launch_bounds__(GEMM_THREADS, (AM == LOAD_S || BMD == LOAD_S) ? 1 : 4)
void gemm_f32_mfma(GemmArgs p) {
    static_assert(TM * TN <= 4, "the occupancy bound assumes at most 2x2 blocks per wave");
    constexpr int TBM = 64 * TM, TBN = 64 * TN;
    using GA = Geo<BK, TBM>;
    using GB = Geo<BK, TBN>;
    constexpr int A_ST = GA::template stage<AM>();
    constexpr int B_ST = GB::template stage<BMD>();
    constexpr int GROUPS = BK / 8;
    __shared__ __attribute__((aligned(16))) float smem[2 * (A_ST + B_ST)];
    float* As = smem;
    float* Bs = smem + 2 * A_ST;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, h = lane >> 5;

    uint32_t plane, tm, tn;
    decode_tile(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, &plane, &tm, &tn);
    const uint32_t bi = plane / p.splits, split = plane - bi * p.splits;
    const uint32_t m0 = tm * TBM, n0 = tn * TBN;
    const uint32_t kb = split * p.k_chunk;
    const uint32_t klen = min(p.k - kb, p.k_chunk);
    const uint32_t mrem = p.m - m0, nrem = p.n - n0;

    const float* A = p.a + static_cast<int64_t>(bi) * p.a_sb + static_cast<int64_t>(m0) * p.a_sm +
                     static_cast<int64_t>(kb) * p.a_sk;
    const float* B = p.b + static_cast<int64_t>(bi) * p.b_sb + static_cast<int64_t>(n0) * p.b_sn +
                     static_cast<int64_t>(kb) * p.b_sk;

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    floatx4 ra[GA::LOADS], rb[GB::LOADS];
    const uint32_t ktiles = (klen + BK - 1) / BK;
    // Workgroup-uniform: the tile's M x N window lies inside the operands, so a K-slice is
    // "full" whenever its k range is.
    const bool inner = mrem >= TBM && nrem >= TBN;
    const float* pa[GA::LOADS];
    const float* pb[GB::LOADS];
#pragma unroll
    for (int i = 0; i < GA::LOADS; ++i) pa[i] = slice_ptr<AM, BK, TBM>(A, p.a_sm, p.a_sk, i, tid);
#pragma unroll
    for (int i = 0; i < GB::LOADS; ++i) pb[i] = slice_ptr<BMD, BK, TBN>(B, p.b_sn, p.b_sk, i, tid);
    auto load = [&](uint32_t k0) {
        if (inner && k0 + BK <= klen) {
            if constexpr (AM == LOAD_S) {
                load_slice<AM, true, BK, TBM>(ra, A, p.a_sm, p.a_sk, mrem, k0, klen, tid);
            } else {
                const int64_t off = AM == LOAD_MN ? static_cast<int64_t>(k0) * p.a_sk : k0;
#pragma unroll
                for (int i = 0; i < GA::LOADS; ++i) ra[i] = *reinterpret_cast<const floatx4*>(pa[i] + off);
            }
            if constexpr (BMD == LOAD_S) {
                load_slice<BMD, true, BK, TBN>(rb, B, p.b_sn, p.b_sk, nrem, k0, klen, tid);
            } else {
                const int64_t off = BMD == LOAD_MN ? static_cast<int64_t>(k0) * p.b_sk : k0;
#pragma unroll
                for (int i = 0; i < GB::LOADS; ++i) rb[i] = *reinterpret_cast<const floatx4*>(pb[i] + off);
            }
        } else {
            load_slice<AM, false, BK, TBM>(ra, A, p.a_sm, p.a_sk, mrem, k0, klen, tid);
            load_slice<BMD, false, BK, TBN>(rb, B, p.b_sn, p.b_sk, nrem, k0, klen, tid);
        }
    };
    // alpha multiplies whichever operand holds the caller's A (1 * x is skipped as x).
    const float alpha_a = p.scale_b ? 1.0f : p.alpha;
    const float alpha_b = p.scale_b ? p.alpha : 1.0f;
    load(0);
    store_slice<AM, BK, TBM, true>(As, ra, tid, alpha_a);
    store_slice<BMD, BK, TBN, true>(Bs, rb, tid, alpha_b);
    __syncthreads();

    uint32_t kt = 0;
    for (; kt < ktiles; ++kt) {
        const int s = kt & 1;
        const bool more = kt + 1 < ktiles;
        if (more) load((kt + 1) * BK);
        const float* as = As + s * A_ST;
        const float* bs = Bs + s * B_ST;
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int g = 0; g < GROUPS; ++g) {
            floatx4 av[TM], bv[TN];
            read_frag<AM, BK, TBM, TM>(av, as, wm * 32 * TM, g, lr, h);
            read_frag<BMD, BK, TBN, TN>(bv, bs, wn * 32 * TN, g, lr, h);
            mfma_group<TM, TN>(acc, av, bv);
        }
        __builtin_amdgcn_s_setprio(0);
        if (more) {
            store_slice<AM, BK, TBM, true>(As + (s ^ 1) * A_ST, ra, tid, alpha_a);
            store_slice<BMD, BK, TBN, true>(Bs + (s ^ 1) * B_ST, rb, tid, alpha_b);
        }
        __syncthreads();
    }

    // Epilogue. Accumulator register r of block (i, j) holds
    // row = 8*(r/4) + 4*h + r%4, col = lane%32 of that 32x32 block.
    if (p.partial != nullptr) {
        float* P = p.partial + static_cast<int64_t>(plane) * p.m * p.n;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t row = m0 + wm * 32 * TM + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
                    const uint32_t col = n0 + wn * 32 * TN + j * 32 + lr;
                    if (inner || (row < p.m && col < p.n)) {
                        P[static_cast<int64_t>(row) * p.n + col] = acc[i][j][r];
                    }
                }
        return;
    }
    float* C = p.c + static_cast<int64_t>(bi) * p.c_sb;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = m0 + wm * 32 * TM + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
                const uint32_t col = n0 + wn * 32 * TN + j * 32 + lr;
                if (inner || (row < p.m && col < p.n)) {
                    float* q = C + static_cast<int64_t>(row) * p.c_sm +
                               static_cast<int64_t>(col) * p.c_sn;
                    float v = acc[i][j][r];
                    if (p.beta != 0.0f) v = p.beta * *q + v;
                    *q = v;
                }
            }
}

// Small products (the 64x64 grid alone under 256 tiles, K <= GEMM_SMALL_K), and small
// outputs with long K split over workgroups: one 32x32 output tile (of one K chunk) per
// workgroup of W waves. The waves take interleaved 8-k groups (wave w: groups w, w+W, ...),
// each accumulating one v_mfma_f32_32x32x2_f32 block straight from registers: the 32 rows are
// shared by the waves but their k ranges are not, so there is nothing for LDS to reuse. Lane
// (r = lane%32, h = lane/32) holds k = 8g + 4h + s at MFMA step s, as in the tiled kernel; an
// operand contiguous along K gives it a 128-bit load, one contiguous along M/N four 32-bit
// loads that coalesce across lanes. The W wave sums meet in LDS and add in wave order, then
// beta*C + sum (or the raw sum into the split partials): the order depends on K, the chunk
// and W alone. The launch uses W = 16 (four waves per SIMD): with K = 512 each wave issues
// all of its loads at once and the SIMD interleaves four accumulation chains (config 1:
// 33 -> 38 TFLOP/s).
constexpr int SMALL_TILE = 32;
constexpr int SMALL_WAVES = 16;  // waves per small-product workgroup
constexpr int SMALL_UNROLL = 4;  // 8-k groups whose loads are issued before their MFMAs

template <int MODE, bool FULL>
__device__ inline floatx4 small_frag(const float* __restrict__ p, int64_t srow, int64_t sk,
                                     bool row_ok, uint32_t k0, uint32_t klen, int r, int h) {
    const uint32_t kk = k0 + 4 * h;
    const float* q = p + static_cast<int64_t>(r) * srow;
    if constexpr (MODE == LOAD_K) {
        if (FULL) return *reinterpret_cast<const floatx4*>(q + kk);
    }
    floatx4 v;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        v[s] = (FULL || (row_ok && kk + s < klen)) ? q[static_cast<int64_t>(kk + s) * sk] : 0.0f;
    }
    return v;
}

// Accumulates the 8-k groups g0, g0 + stride, ... (SMALL_UNROLL of them per batch, every load
// of a batch issued before its MFMAs) of one 32x32 tile into acc. A and B point at the tile's
// (row 0, k 0); klen is the tile's K extent.
template <int AM, int BMD, int STRIDE>
__device__ inline void small_tile_sum(floatx16& acc, const float* A, const float* B,
                                      const GemmArgs& p, uint32_t g0, uint32_t klen, bool inner,
                                      bool a_ok, bool b_ok, int r, int h, float alpha_a,
                                      float alpha_b) {
    const uint32_t groups = (klen + 7) / 8;
    for (; g0 < groups; g0 += STRIDE * SMALL_UNROLL) {
        floatx4 av[SMALL_UNROLL], bv[SMALL_UNROLL];
        const uint32_t last = g0 + STRIDE * (SMALL_UNROLL - 1);
        if (inner && 8 * last + 8 <= klen) {
#pragma unroll
            for (int u = 0; u < SMALL_UNROLL; ++u) {
                const uint32_t k0 = 8 * (g0 + STRIDE * u);
                av[u] = small_frag<AM, true>(A, p.a_sm, p.a_sk, true, k0, klen, r, h);
                bv[u] = small_frag<BMD, true>(B, p.b_sn, p.b_sk, true, k0, klen, r, h);
            }
        } else {
#pragma unroll
            for (int u = 0; u < SMALL_UNROLL; ++u) {
                const uint32_t k0 = 8 * (g0 + STRIDE * u);  // past K: every element predicated to 0
                av[u] = small_frag<AM, false>(A, p.a_sm, p.a_sk, a_ok, k0, klen, r, h);
                bv[u] = small_frag<BMD, false>(B, p.b_sn, p.b_sk, b_ok, k0, klen, r, h);
            }
        }
#pragma unroll
        for (int u = 0; u < SMALL_UNROLL; ++u) {
            floatx4 a = av[u], b = bv[u];
            if (alpha_a != 1.0f) a = a * alpha_a;
            if (alpha_b != 1.0f) b = b * alpha_b;
#pragma unroll
            for (int st = 0; st < 4; ++st)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[st], b[st], acc, 0, 0, 0);
        }
    }
}

template <int AM, int BMD, int W = 4>
__global__ __launch_bounds__(64 * W) void gemm_f32_small(GemmArgs p) {
    constexpr int THREADS = 64 * W;
    __shared__ float red[W][SMALL_TILE * SMALL_TILE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 31, h = lane >> 5;
    uint32_t plane, tm, tn;
    decode_tile(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, &plane, &tm, &tn);
    const uint32_t bi = plane / p.splits, split = plane - bi * p.splits;
    const uint32_t m0 = tm * SMALL_TILE, n0 = tn * SMALL_TILE;
    const uint32_t kb = split * p.k_chunk;
    const uint32_t klen = min(p.k - kb, p.k_chunk);
    const float* A = p.a + static_cast<int64_t>(bi) * p.a_sb + static_cast<int64_t>(m0) * p.a_sm +
                     static_cast<int64_t>(kb) * p.a_sk;
    const float* B = p.b + static_cast<int64_t>(bi) * p.b_sb + static_cast<int64_t>(n0) * p.b_sn +
                     static_cast<int64_t>(kb) * p.b_sk;
    const bool inner = p.m - m0 >= SMALL_TILE && p.n - n0 >= SMALL_TILE;
    const bool a_ok = r < static_cast<int>(p.m - m0), b_ok = r < static_cast<int>(p.n - n0);

    floatx16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    // Wave w takes groups w, w + W, ...
    small_tile_sum<AM, BMD, W>(acc, A, B, p, wave, klen, inner, a_ok, b_ok, r, h,
                               p.scale_b ? 1.0f : p.alpha, p.scale_b ? p.alpha : 1.0f);
    // Accumulator register i: row 8*(i/4) + 4*h + i%4, column r.
#pragma unroll
    for (int i = 0; i < 16; ++i) red[wave][((i >> 2) * 8 + h * 4 + (i & 3)) * SMALL_TILE + r] = acc[i];
    __syncthreads();
    float* C = p.c + static_cast<int64_t>(bi) * p.c_sb;
    float* P = p.partial + static_cast<int64_t>(plane) * p.m * p.n;
#pragma unroll
    for (int j = 0; j < SMALL_TILE * SMALL_TILE / THREADS; ++j) {
        const int e = j * THREADS + tid;
        const uint32_t row = m0 + e / SMALL_TILE, col = n0 + e % SMALL_TILE;
        if (inner || (row < p.m && col < p.n)) {
            float v = red[0][e];
#pragma unroll
            for (int w = 1; w < W; ++w) v = v + red[w][e];
            if (p.partial != nullptr) {
                P[static_cast<int64_t>(row) * p.n + col] = v;
            } else {
                float* q = C + static_cast<int64_t>(row) * p.c_sm + static_cast<int64_t>(col) * p.c_sn;
                if (p.beta != 0.0f) v = p.beta * *q + v;
                *q = v;
            }
        }
    }
}

// Many small products (batched outputs whose 64x64 or 128x128 tiles would be mostly padding):
// one 32x32 output tile per wave over its whole K chunk, four tiles per 256-thread workgroup.
// Operands go straight from memory into MFMA registers, as in gemm_f32_small (no two waves
// read the same rows, so LDS has nothing to share), and each wave stores its accumulators
// directly: no LDS, no barrier. Tiles are numbered plane-major (plane = batch * splits +
// split), row-major within a plane. The sum of one output runs over k in 8-k groups in order.
constexpr int WAVE_TILES = 4;  // tiles (waves) per workgroup

template <int AM, int BMD>
__global__ __launch_bounds__(64 * WAVE_TILES) void gemm_f32_wave(GemmArgs p) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 31, h = lane >> 5;
    const uint32_t per_plane = p.tiles_m * p.tiles_n;
    const uint64_t tile = static_cast<uint64_t>(blockIdx.x) * WAVE_TILES + wave;
    if (tile >= static_cast<uint64_t>(per_plane) * p.batch * p.splits) return;  // whole wave
    const uint32_t plane = static_cast<uint32_t>(tile / per_plane);
    const uint32_t t = static_cast<uint32_t>(tile - static_cast<uint64_t>(plane) * per_plane);
    const uint32_t tm = t / p.tiles_n, tn = t - tm * p.tiles_n;
    const uint32_t bi = plane / p.splits, split = plane - bi * p.splits;
    const uint32_t m0 = tm * SMALL_TILE, n0 = tn * SMALL_TILE;
    const uint32_t kb = split * p.k_chunk;
    const uint32_t klen = min(p.k - kb, p.k_chunk);
    const float* A = p.a + static_cast<int64_t>(bi) * p.a_sb + static_cast<int64_t>(m0) * p.a_sm +
                     static_cast<int64_t>(kb) * p.a_sk;
    const float* B = p.b + static_cast<int64_t>(bi) * p.b_sb + static_cast<int64_t>(n0) * p.b_sn +
                     static_cast<int64_t>(kb) * p.b_sk;
    const bool inner = p.m - m0 >= SMALL_TILE && p.n - n0 >= SMALL_TILE;
    const bool a_ok = r < static_cast<int>(p.m - m0), b_ok = r < static_cast<int>(p.n - n0);
    floatx16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    small_tile_sum<AM, BMD, 1>(acc, A, B, p, 0, klen, inner, a_ok, b_ok, r, h,
                               p.scale_b ? 1.0f : p.alpha, p.scale_b ? p.alpha : 1.0f);
    // Accumulator register i: row 8*(i/4) + 4*h + i%4, column r.
    float* C = p.c + static_cast<int64_t>(bi) * p.c_sb;
    float* P = p.partial + static_cast<int64_t>(plane) * p.m * p.n;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t row = m0 + (i >> 2) * 8 + h * 4 + (i & 3), col = n0 + r;
        if (inner || (row < p.m && col < p.n)) {
            if (p.partial != nullptr) {
                P[static_cast<int64_t>(row) * p.n + col] = acc[i];
            } else {
                float* q = C + static_cast<int64_t>(row) * p.c_sm + static_cast<int64_t>(col) * p.c_sn;
                float v = acc[i];
                if (p.beta != 0.0f) v = p.beta * *q + v;
                *q = v;
            }
        }
    }
}

}  // namespace gemm_detail
}  // namespace lg
