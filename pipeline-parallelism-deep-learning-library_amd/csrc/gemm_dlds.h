// The fp32 MFMA GEMM with operand slices copied from HBM straight into LDS.
//
// gemm_f32_dl<AM, BMD, NS, BK, WN, WM, FM, FN>: WM x WN waves, each FM x FN blocks of
// v_mfma_f32_32x32x2_f32, over a (32 FM WM) x (32 FN WN) output tile (128x128, 128x256, and
// 32x32 with one wave for small outputs split along long K), with K-slices of BK moved by
// global_load_lds_dwordx4: each lane's 16 bytes land in LDS without passing through VGPRs, so
// no staging registers, no LDS write instructions and no wait on the loads before the writes.
// NS unpadded LDS stages keep NS - 1 slices in flight; one barrier per slice. A wave
// instruction fills 1 KB of LDS contiguously (lane l at byte 16*l), so the layout is chosen by
// which global chunk each lane fetches:
//   LOAD_K  (unit stride along K): [row][k], 4*BK bytes per row; 16-byte chunk c of row r at
//            chunk position c ^ swz_k(r) of the row, so the 32 rows an MFMA fragment read
//            touches fall on distinct banks (for 8- and for 16-lane LDS phases);
//   LOAD_MN (unit stride along M/N): [k][row], 4*R bytes per k; chunk c (rows 4c..4c+3) of
//            k-row kr at position c ^ swz_mn(kr), so the two lane halves (k and k + 4) of a
//            32-bit fragment read fall on different banks.
// Edge tiles and a partial last K-slice are loaded through registers into the same layout
// (elements outside the operand as zero). With KG = 2 or 4 the workgroup holds that many such
// wave groups, each with its own stages, taking consecutive parts of the tile's K slices; the
// other groups' sums are added to group 0's through LDS at the end (in group order, the same
// every run), which gives a grid of one workgroup per compute unit more waves per SIMD. alpha scales the fragments of the operand holding
// the caller's A as they are read, so every product is (alpha*a)*b.
#pragma once

#include <hip/hip_runtime.h>

#include "gemm_kernel.h"

namespace lg {
namespace gemm_detail {

constexpr int DL_R = 128;  // rows (M or N) per operand tile

// Stage geometry of an operand tile of R rows and slices of BK, loaded by T threads: floats
// per stage, 16-byte chunks per thread.
template <int R, int BK, int T>
struct DlGeo {
    static constexpr int ST = R * BK;
    static constexpr int LOADS = ST / 4 / T;
    static_assert(LOADS * 4 * T == ST, "a stage splits evenly over the threads");
};

// Chunk swizzles. [row][k] with BK = 16 (four chunks a row): rows r, r+2, r+4, r+6 and r, r+4,
// r+8, r+12 get distinct chunk positions; with BK = 32 (eight chunks): any eight consecutive
// rows, and the rows of one parity among sixteen; with BK = 64 (sixteen chunks): any sixteen
// consecutive rows. [k][row]: k-rows four apart differ by eight
// chunks (128 bytes) when a k-row holds at least 16 chunks (R >= 64); a 32-row k-row (128
// bytes, every bank once) is left as it is.
template <int BK>
__device__ inline uint32_t swz_k(uint32_t r) {
    if constexpr (BK == 16) {
        return ((r >> 1) ^ (r >> 3)) & 3u;
    } else if constexpr (BK == 32) {
        return (r ^ (r >> 3)) & 7u;
    } else {
        return (r ^ (r >> 4)) & 15u;
    }
}
template <int R>
__device__ inline uint32_t swz_mn(uint32_t kr) {
    static_assert(R == 32 || R % 64 == 0, "k-row width");
    return R >= 64 ? ((kr >> 2) & 1u) * 8u : 0u;
}

// Chunk position q of a stage -> (operand row, k) of its first element, relative to the
// tile's (row 0, k of the slice).
template <int MODE, int R, int BK>
__device__ inline void dl_chunk(uint32_t q, uint32_t* row, uint32_t* k) {
    if constexpr (MODE == LOAD_K) {
        constexpr uint32_t CPR = BK / 4;  // chunks per row
        *row = q / CPR;
        *k = 4 * ((q % CPR) ^ swz_k<BK>(q / CPR));
    } else {
        constexpr uint32_t CPK = R / 4;   // chunks per k-row
        *k = q / CPK;
        *row = 4 * ((q % CPK) ^ swz_mn<R>(q / CPK));
    }
}

// Float offset, within one stage, of operand element (row, k).
template <int MODE, int R, int BK>
__device__ inline uint32_t dl_at(uint32_t row, uint32_t k) {
    if constexpr (MODE == LOAD_K) {
        return row * BK + 4 * ((k >> 2) ^ swz_k<BK>(row)) + (k & 3u);
    } else {
        return k * R + 4 * ((row >> 2) ^ swz_mn<R>(k)) + (row & 3u);
    }
}

// Element offset of a chunk's first element from the tile's (row 0, k 0).
template <int MODE, int R, int BK>
__device__ inline int64_t dl_src(uint32_t q, int64_t srow, int64_t sk) {
    uint32_t row, k;
    dl_chunk<MODE, R, BK>(q, &row, &k);
    return static_cast<int64_t>(row) * srow + static_cast<int64_t>(k) * sk;
}

// Registers path: chunk q of the slice at k0 with elements past rows_left or klen as zero.
template <int MODE, int R, int BK>
__device__ inline floatx4 dl_reg_chunk(const float* p, int64_t srow, int64_t sk, uint32_t q,
                                       uint32_t rows_left, uint32_t k0, uint32_t klen) {
    uint32_t row, k;
    dl_chunk<MODE, R, BK>(q, &row, &k);
    floatx4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t r = MODE == LOAD_K ? row : row + e;
        const uint32_t kk = k0 + (MODE == LOAD_K ? k + e : k);
        v[e] = (r < rows_left && kk < klen) ? p[static_cast<int64_t>(r) * srow + static_cast<int64_t>(kk) * sk] : 0.0f;
    }
    return v;
}

template <int MODE, int R, int BK, int NB>
__device__ inline void dl_frag(floatx4 (&v)[NB], const float* __restrict__ st, int base_row, int g,
                               int lr, int h) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const uint32_t row = base_row + i * 32 + lr;
        if constexpr (MODE == LOAD_MN) {
#pragma unroll
            for (int s = 0; s < 4; ++s) v[i][s] = st[dl_at<LOAD_MN, R, BK>(row, g * 8 + h * 4 + s)];
        } else {
            v[i] = *reinterpret_cast<const floatx4*>(st + dl_at<LOAD_K, R, BK>(row, g * 8 + h * 4));
        }
    }
}

// One global_load_lds_dwordx4: each lane's 16 bytes at `src` land at lds + 16 * lane. (A plain
// function, so the builtin is checked once where it is defined rather than inside the kernel
// template, whose host-side stub would otherwise not be emitted.)
__device__ inline void dl_copy16(const float* src, float* lds) {
    __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
}

// s_waitcnt with vmcnt <= N only (gfx9 encoding: expcnt and lgkmcnt at their maximum).
template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// s_waitcnt lgkmcnt(0) only.
__device__ inline void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }

template <int NS, int PER>
__device__ inline void wait_slices(uint32_t newer) {
    // Loads of `newer` later slices may stay in flight: PER instructions per slice.
    if constexpr (NS >= 4) {
        if (newer >= 2) { wait_vm<2 * PER>(); return; }
    }
    if constexpr (NS >= 3) {
        if (newer >= 1) { wait_vm<PER>(); return; }
    }
    wait_vm<0>();
}

// WM x WN waves, each FM x FN blocks of 32x32: a (32 FM WM) x (32 FN WN) tile of 64 WM WN
// threads (2x2 waves of 2x2 blocks: 128x128; 2x4 waves: 128x256, whose B slice serves twice
// the rows; 2x2 waves of 2x4 blocks: 128x256 with half the waves, each reading 6 fragments per
// 8 MFMAs instead of 4 per 4).
template <int WM, int WN>
constexpr int dl_threads() { return 64 * WM * WN; }
template <int NS, int BK, int WM, int WN, int FM, int FN, int KG = 1>
constexpr int dl_occupancy() {
    // workgroups per compute unit by LDS (160 KB), at most what the accumulators allow: 2x2
    // blocks (64 registers) fit four waves per SIMD, 2x4 two, 4x4 one
    constexpr int lds = KG * NS * (32 * FM * WM + 32 * FN * WN) * BK * 4;
    constexpr int by_lds = 160 * 1024 / lds;
    constexpr int waves_per_simd = FM * FN <= 4 ? 4 : FM * FN <= 8 ? 2 : 1;
    constexpr int waves = WM * WN * KG;
    constexpr int by_vgpr = 4 * waves_per_simd / waves > 0 ? 4 * waves_per_simd / waves : 1;
    return by_lds < by_vgpr ? by_lds : by_vgpr;
}

template <int AM, int BMD, int NS, int BK = 16, int WN = 2, int WM = 2, int FM = 2, int FN = 2,
          int KG = 1>
__global__ __launch_bounds__((dl_threads<WM, WN>() * KG), (dl_occupancy<NS, BK, WM, WN, FM, FN, KG>()))
void gemm_f32_dl(GemmArgs p) {
    static_assert(AM != LOAD_S && BMD != LOAD_S, "direct loads need a unit-stride axis");
    static_assert(NS >= 2 && NS <= 4, "stages");
    static_assert(BK == 16 || BK == 32 || BK == 64, "slice depth");
    static_assert(KG >= 1 && KG <= 4, "wave groups");
    constexpr int T = dl_threads<WM, WN>();  // threads of one wave group
    constexpr int RA = 32 * FM * WM, RB = 32 * FN * WN;
    using GA = DlGeo<RA, BK, T>;
    using GB = DlGeo<RB, BK, T>;
    constexpr int NW = T / 64;
    constexpr int GROUP_ST = NS * (GA::ST + GB::ST);  // floats of one group's stages
    constexpr int RED = NW * FM * FN * 16 * 64;      // floats of one group's accumulators
    static_assert((KG / 2) * RED <= KG * GROUP_ST, "the group sums must fit in the stages");
    __shared__ __attribute__((aligned(16))) float smem[KG * GROUP_ST];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // Wave group and wave within it; with one group these are compile-time 0 and the wave id,
    // so the single-group kernel keeps its straight loop.
    const int kg = KG == 1 ? 0 : (tid >> 6) / NW;
    const int wave = KG == 1 ? (tid >> 6) : (tid >> 6) % NW;
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 31, h = lane >> 5;
    float* As = smem + kg * GROUP_ST;
    float* Bs = As + NS * GA::ST;

    uint32_t plane, tm, tn;
    decode_tile(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, &plane, &tm, &tn);
    const uint32_t bi = plane / p.splits, split = plane - bi * p.splits;
    const uint32_t m0 = tm * RA, n0 = tn * RB;
    const uint32_t kb = split * p.k_chunk;
    const uint32_t klen = min(p.k - kb, p.k_chunk);
    const uint32_t mrem = p.m - m0, nrem = p.n - n0;
    const float* A = p.a + static_cast<int64_t>(bi) * p.a_sb + static_cast<int64_t>(m0) * p.a_sm +
                     static_cast<int64_t>(kb) * p.a_sk;
    const float* B = p.b + static_cast<int64_t>(bi) * p.b_sb + static_cast<int64_t>(n0) * p.b_sn +
                     static_cast<int64_t>(kb) * p.b_sk;
    const float alpha_a = p.scale_b ? 1.0f : p.alpha;
    const float alpha_b = p.scale_b ? p.alpha : 1.0f;

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const bool inner = mrem >= RA && nrem >= RB;
    const uint32_t ktiles = (klen + BK - 1) / BK;
    const uint32_t kfull = inner ? klen / BK : 0;  // slices that go by direct loads
    // Group kg takes slices [kg * per, kg * per + mine); every group runs `per` iterations so
    // all waves meet at the same barriers.
    const uint32_t per = KG == 1 ? ktiles : (ktiles + KG - 1) / KG;
    const uint32_t first = KG == 1 ? 0u : min(static_cast<uint32_t>(kg) * per, ktiles);
    const uint32_t mine = KG == 1 ? ktiles : min(per, ktiles - first);
    // Per-thread source offsets of the direct loads at k = 0, and the k step per slice.
    int64_t sa[GA::LOADS], sb[GB::LOADS];
#pragma unroll
    for (int i = 0; i < GA::LOADS; ++i) sa[i] = dl_src<AM, RA, BK>((i * NW + wave) * 64 + lane, p.a_sm, p.a_sk);
#pragma unroll
    for (int i = 0; i < GB::LOADS; ++i) sb[i] = dl_src<BMD, RB, BK>((i * NW + wave) * 64 + lane, p.b_sn, p.b_sk);
    const int64_t a_step = AM == LOAD_K ? BK : static_cast<int64_t>(BK) * p.a_sk;
    const int64_t b_step = BMD == LOAD_K ? BK : static_cast<int64_t>(BK) * p.b_sk;

    // Slice i of this group (global slice first + i) into stage i % NS.
    auto issue = [&](uint32_t i) {
        float* as = As + (i % NS) * GA::ST;
        float* bs = Bs + (i % NS) * GB::ST;
        const uint32_t kt = first + i;
        if (kt < kfull) {
#pragma unroll
            for (int i = 0; i < GA::LOADS; ++i) dl_copy16(A + sa[i] + kt * a_step, as + (i * NW + wave) * 256);
#pragma unroll
            for (int i = 0; i < GB::LOADS; ++i) dl_copy16(B + sb[i] + kt * b_step, bs + (i * NW + wave) * 256);
        } else {
            floatx4 ra[GA::LOADS], rb[GB::LOADS];
#pragma unroll
            for (int i = 0; i < GA::LOADS; ++i)
                ra[i] = dl_reg_chunk<AM, RA, BK>(A, p.a_sm, p.a_sk, (i * NW + wave) * 64 + lane, mrem, kt * BK, klen);
#pragma unroll
            for (int i = 0; i < GB::LOADS; ++i)
                rb[i] = dl_reg_chunk<BMD, RB, BK>(B, p.b_sn, p.b_sk, (i * NW + wave) * 64 + lane, nrem, kt * BK, klen);
#pragma unroll
            for (int i = 0; i < GA::LOADS; ++i)
                *reinterpret_cast<floatx4*>(as + 4 * ((i * NW + wave) * 64 + lane)) = ra[i];
#pragma unroll
            for (int i = 0; i < GB::LOADS; ++i)
                *reinterpret_cast<floatx4*>(bs + 4 * ((i * NW + wave) * 64 + lane)) = rb[i];
        }
    };

#pragma unroll
    for (int s = 0; s < NS - 1; ++s) {
        if (static_cast<uint32_t>(s) < mine) issue(s);
    }
    for (uint32_t kt = 0; kt < per; ++kt) {
        // Group-uniform: a group with fewer slices still meets every barrier.
        const bool live = KG == 1 || kt < mine;
        if (live) wait_slices<NS, GA::LOADS + GB::LOADS>(min(static_cast<uint32_t>(NS - 2), mine - 1 - kt));
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();
        if (!live) continue;
        if (kt + NS - 1 < mine) issue(kt + NS - 1);
        const float* as = As + (kt % NS) * GA::ST;
        const float* bs = Bs + (kt % NS) * GB::ST;
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int g = 0; g < BK / 8; ++g) {
            floatx4 av[FM], bv[FN];
            dl_frag<AM, RA, BK, FM>(av, as, wm * 32 * FM, g, lr, h);
            dl_frag<BMD, RB, BK, FN>(bv, bs, wn * 32 * FN, g, lr, h);
            if (alpha_a != 1.0f) {
#pragma unroll
                for (int i = 0; i < FM; ++i) av[i] = av[i] * alpha_a;
            }
            if (alpha_b != 1.0f) {
#pragma unroll
                for (int j = 0; j < FN; ++j) bv[j] = bv[j] * alpha_b;
            }
            mfma_group<FM, FN>(acc, av, bv);
        }
        __builtin_amdgcn_s_setprio(0);
    }

    if constexpr (KG > 1) {
        // The groups' sums meet through LDS in a fixed tree (every stage read and every load
        // landed: each group waited for its last slice before the final barrier): each round
        // the upper half of the groups still holding sums hands them to the lower half, so
        // four groups add as (g0 + g2) + (g1 + g3), three as (g0 + g2) + g1, two as g0 + g1.
        // Every wave takes part in every barrier; group 0 stores.
        float* red = smem + (wave * FM * FN * 16) * 64 + lane;
#pragma unroll
        for (int n = KG; n > 1; n = (n + 1) / 2) {
            const int half = (n + 1) / 2;
            __syncthreads();
            if (kg >= half && kg < n) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            red[(kg - half) * RED + ((i * FN + j) * 16 + r) * 64] = acc[i][j][r];
            }
            __syncthreads();
            if (kg < n - half) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc[i][j][r] = acc[i][j][r] + red[kg * RED + ((i * FN + j) * 16 + r) * 64];
            }
        }
        if (kg > 0) return;
    }

    // Epilogue: as gemm_f32_mfma.
    if (p.partial != nullptr) {
        float* P = p.partial + static_cast<int64_t>(plane) * p.m * p.n;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t row = m0 + wm * 32 * FM + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
                    const uint32_t col = n0 + wn * 32 * FN + j * 32 + lr;
                    if (inner || (row < p.m && col < p.n)) P[static_cast<int64_t>(row) * p.n + col] = acc[i][j][r];
                }
        return;
    }
    float* C = p.c + static_cast<int64_t>(bi) * p.c_sb;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = m0 + wm * 32 * FM + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
                const uint32_t col = n0 + wn * 32 * FN + j * 32 + lr;
                if (inner || (row < p.m && col < p.n)) {
                    float* q = C + static_cast<int64_t>(row) * p.c_sm + static_cast<int64_t>(col) * p.c_sn;
                    float v = acc[i][j][r];
                    if (p.beta != 0.0f) v = p.beta * *q + v;
                    *q = v;
                }
            }
}

}  // namespace gemm_detail
}  // namespace lg
