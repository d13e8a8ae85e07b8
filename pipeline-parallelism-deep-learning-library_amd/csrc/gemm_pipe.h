// The software-pipelined fp32 MFMA GEMMs: gemm_f32_pl for full 128x128 and 128x64 tiles and,
// below it, gemm_f32_kw for full 64x64 tiles whose waves split K.
//
// gemm_f32_pl<AM, BMD, BK, NS, FN>: four waves (2x2, each 64 x 32*FN as 2 x FN blocks of
// v_mfma_f32_32x32x2_f32) per 128 x 64*FN output tile, operand slices BK deep copied HBM -> LDS
// by global_load_lds_dwordx4 into NS stages with the layouts and swizzles of gemm_f32_dl. The
// latency of every step is hidden inside the wave that waits for it, rather than by other
// waves: with BK = 16 two 128x128 workgroups (or three 128x64 ones) share a compute unit, with
// BK = 32 one 128x128 workgroup does (one wave per SIMD).
//   * A slice's MFMAs come in BK/8 groups of 8 * FN on two alternating fragment register sets;
//     the fragments of group g + 1 are read from LDS among the MFMAs of group g, the loads of
//     the slice NS - 1 ahead among those of the first group, at fixed positions
//     (sched_group_barrier), so each read has most of a group's MFMAs to return in.
//   * The one barrier per slice sits before the last group's MFMAs, not after them: past it
//     the wave issues those MFMAs at once (their fragments are already in registers) while the
//     next slice's first fragments are read, instead of waiting on LDS right after the barrier.
//   * Stage indices are compile-time constants (the slice loop is unrolled NS times), and
//     every slice step issues the same loads (past the last slice it loads the last slice again
//     into a stage no wave reads any more), so each wait on the loads is one constant vmcnt.
// Requirements, checked by the planner: both operands with a 16-byte aligned unit-stride axis,
// M a multiple of 128 and N of 64 * FN, every K chunk a multiple of NS * BK. Split-K partials as in
// gemm_f32_dl. alpha scales the caller's A fragments as they are read (a compile-time branch,
// chosen per launch), so every product is (alpha*a)*b.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "gemm_dlds.h"

namespace lg {
namespace gemm_detail {

// LDS read instructions per fragment group of a wave, at most: one 128-bit read per
// K-contiguous 32-row fragment, four 32-bit reads per M/N-contiguous one (which the compiler
// pairs into two ds_read2st64_b32 where it can; the schedule then has slots to spare).
template <int AM, int BMD, int FM, int FN>
constexpr int pl_reads() {
    return (AM == LOAD_K ? FM : 4 * FM) + (BMD == LOAD_K ? FN : 4 * FN);
}

// Scheduling groups: N times (one MFMA, then PER instructions of kind MASK).
// Masks of __builtin_amdgcn_sched_group_barrier: 0x008 MFMA, 0x010 VMEM, 0x100 DS read.
template <int N, int MASK, int PER>
__device__ inline void pl_after_each_mfma() {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(MASK, PER, 0);
    }
}

// Workgroups of gemm_f32_pl per compute unit, by LDS (160 KB), at most three.
template <int BK, int NS, int FN>
constexpr int pl_workgroups() {
    constexpr int by_lds = 160 * 1024 / (NS * BK * 4 * (128 + 64 * FN));
    return by_lds < 3 ? by_lds : 3;
}

// The pipelined loop of one (32*FM*WM) x (32*FN*WN) output tile, WM x WN waves of FM x FN
// blocks (the loop of gemm_f32_pl): `ktiles` slices of BK along K from A and B (pointers at the
// tile's first row or column and its first k), added into acc. Leaves loads of the last slice in
// flight into the LDS stages: a caller that reuses the stages waits for them. SPLIT issues a
// slice's B loads in the last fragment group of the step that issues its A loads (past that
// step's barrier, where the stage they fill is free as well) instead of beside them.
template <int AM, int BMD, int BK, int NS, int FN, int WM = 2, int FM = 2, int WN = 2,
          bool SPLIT = false>
__device__ __forceinline__ void pl_tile_loop(const GemmArgs& p, float* smem, const float* A,
                                             const float* B, uint32_t ktiles,
                                             floatx16 (&acc)[FM][FN]) {
    static_assert(AM != LOAD_S && BMD != LOAD_S, "direct loads need a unit-stride axis");
    static_assert(FN == 1 || FN == 2, "waves of FM x 1 or FM x 2 blocks");
    static_assert(FM == 2 || FM == 4, "waves of 2 x FN or 4 x FN blocks");
    static_assert(WM * WN == 4 || WM * WN == 8, "four or eight waves");
    constexpr int NW = WM * WN, T = 64 * NW, RA = 32 * FM * WM, RB = 32 * FN * WN;
    using GA = DlGeo<RA, BK, T>;
    using GB = DlGeo<RB, BK, T>;
    constexpr int PER = GA::LOADS + GB::LOADS;  // load instructions per slice per thread
    constexpr int G = BK / 8;                   // fragment groups per slice
    constexpr int MG = 4 * FM * FN;             // MFMAs per group
    static_assert(G >= 2 && G % 2 == 0, "groups alternate between two fragment register sets");
    static_assert(NS >= 2 && (NS - 1) * PER < 64, "stages (vmcnt counts at most 63)");
    // Reads of one group after the first RM MFMAs of the previous group, RPM after each; the
    // first group's loads, up to two after each of NV MFMAs, from the tenth MFMA on where the
    // group is that long (earlier positions measured 2-4 % slower on batched 1024^3 products).
    constexpr int RD = pl_reads<AM, BMD, FM, FN>();
    constexpr int RPM = RD > MG * 3 / 4 ? 2 : 1;
    constexpr int RM = (RD + RPM - 1) / RPM;
    constexpr int NV = ((SPLIT ? GA::LOADS : PER) + 1) / 2;
    constexpr int NVB = SPLIT ? (GB::LOADS + 1) / 2 : 0;
    // Loads issued after slice kt + 1's last one when step kt reaches its barrier.
    constexpr int AFTER = SPLIT ? (NS - 3) * PER + GA::LOADS : (NS - 2) * PER;
    static_assert(!SPLIT || NS >= 3, "split loads keep two slices ahead");
    constexpr int VF0 = 10 - RM < MG - RM - NV ? 10 - RM : MG - RM - NV;
    constexpr int VF = VF0 > 0 ? VF0 : 0;
    static_assert(RM + VF + NV <= MG, "MFMAs of a group");

    float* As = smem;
    // The B stages start past the A stages. Where that start is beyond the 64 KiB reach of a
    // DS instruction's offset, the compiler, folding it into every read, holds one address
    // register per B fragment read; hidden from it (an empty asm), every read is one register
    // plus an offset.
    uint32_t b_first = NS * GA::ST;
    if constexpr (FM == 4) __asm__ volatile("" : "+s"(b_first));
    float* Bs = smem + b_first;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 31, h = lane >> 5;

    const float alpha_a = p.scale_b ? 1.0f : p.alpha;
    const float alpha_b = p.scale_b ? p.alpha : 1.0f;

    int64_t sa[GA::LOADS], sb[GB::LOADS];
#pragma unroll
    for (int i = 0; i < GA::LOADS; ++i) sa[i] = dl_src<AM, RA, BK>((i * NW + wave) * 64 + lane, p.a_sm, p.a_sk);
#pragma unroll
    for (int i = 0; i < GB::LOADS; ++i) sb[i] = dl_src<BMD, RB, BK>((i * NW + wave) * 64 + lane, p.b_sn, p.b_sk);
    const int64_t a_step = AM == LOAD_K ? BK : static_cast<int64_t>(BK) * p.a_sk;
    const int64_t b_step = BMD == LOAD_K ? BK : static_cast<int64_t>(BK) * p.b_sk;
    // Slice kt into `stage`.
    auto issue_a = [&](uint32_t kt, int stage) {
        float* as = As + stage * GA::ST;
#pragma unroll
        for (int i = 0; i < GA::LOADS; ++i) dl_copy16(A + sa[i] + kt * a_step, as + (i * NW + wave) * 256);
    };
    auto issue_b = [&](uint32_t kt, int stage) {
        float* bs = Bs + stage * GB::ST;
#pragma unroll
        for (int i = 0; i < GB::LOADS; ++i) dl_copy16(B + sb[i] + kt * b_step, bs + (i * NW + wave) * 256);
    };
    auto issue = [&](uint32_t kt, int stage) {
        issue_a(kt, stage);
        issue_b(kt, stage);
    };

    auto run = [&](auto scale) {
        constexpr bool SCALE = decltype(scale)::value;
        floatx4 fa[2][FM], fb[2][FN];
        // Fragment group g of the slice in `stage` into register set `set`.
        auto read = [&](int set, int g, int stage) {
            dl_frag<AM, RA, BK, FM>(fa[set], As + stage * GA::ST, wm * 32 * FM, g, lr, h);
            dl_frag<BMD, RB, BK, FN>(fb[set], Bs + stage * GB::ST, wn * 32 * FN, g, lr, h);
            if constexpr (SCALE) {
#pragma unroll
                for (int i = 0; i < FM; ++i) fa[set][i] = fa[set][i] * alpha_a;
#pragma unroll
                for (int j = 0; j < FN; ++j) fb[set][j] = fb[set][j] * alpha_b;
            }
        };
        // Slices 0 .. NS-2 in flight; slice step kt then issues slice kt + NS - 1 into the
        // stage slice kt - 1 used (clamped to the last slice), so at the barrier of step kt the
        // loads issued after slice kt + 1's are always those of the NS - 2 slices behind it.
#pragma unroll
        for (int s = 0; s + 1 < NS; ++s) issue(min(static_cast<uint32_t>(s), ktiles - 1), s);
        wait_vm<(NS - 2) * PER>();
        __builtin_amdgcn_s_barrier();
        read(0, 0, 0);
        for (uint32_t k0 = 0; k0 < ktiles; k0 += NS) {
#pragma unroll
            for (int u = 0; u < NS; ++u) {
                const uint32_t kt = k0 + u;
#pragma unroll
                for (int g = 0; g + 1 < G; ++g) {
                    read((g + 1) & 1, g + 1, u);
                    if (g == 0) {
                        if constexpr (SPLIT) {
                            issue_a(min(kt + NS - 1, ktiles - 1), (u + NS - 1) % NS);
                        } else {
                            issue(min(kt + NS - 1, ktiles - 1), (u + NS - 1) % NS);
                        }
                    }
                    mfma_group<FM, FN>(acc, fa[g & 1], fb[g & 1]);
                    pl_after_each_mfma<RM, 0x100, RPM>();
                    if (g == 0) {
                        if constexpr (VF > 0) __builtin_amdgcn_sched_group_barrier(0x008, VF, 0);
                        pl_after_each_mfma<NV, 0x010, 2>();
                        __builtin_amdgcn_sched_group_barrier(0x008, MG - RM - VF - NV, 0);
                    } else {
                        __builtin_amdgcn_sched_group_barrier(0x008, MG - RM, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                // Slice kt + 1 landed for every wave, slice kt read by every wave.
                wait_vm<AFTER>();
                wait_lgkm0();
                __builtin_amdgcn_s_barrier();
                constexpr int L = (G - 1) & 1;
                read(0, 0, (u + 1) % NS);  // past the last slice: unused
                if constexpr (SPLIT) issue_b(min(kt + NS - 1, ktiles - 1), (u + NS - 1) % NS);
                mfma_group<FM, FN>(acc, fa[L], fb[L]);
                pl_after_each_mfma<RM, 0x100, RPM>();
                if constexpr (SPLIT) {
                    pl_after_each_mfma<NVB, 0x010, 2>();
                    __builtin_amdgcn_sched_group_barrier(0x008, MG - RM - NVB, 0);
                } else {
                    __builtin_amdgcn_sched_group_barrier(0x008, MG - RM, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    if (alpha_a != 1.0f || alpha_b != 1.0f) {
        run(std::true_type{});
    } else {
        run(std::false_type{});
    }

}

// Stores one tile of C of waves in WN columns with FM x FN blocks each (plane bi, first row m0,
// first column n0): beta * C + acc, or acc alone when beta is 0 (C never read).
template <int FN, int FM = 2, int WN = 2>
__device__ __forceinline__ void pl_store_c(const GemmArgs& p, const floatx16 (&acc)[FM][FN],
                                           uint32_t bi, uint32_t m0, uint32_t n0) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 31, h = lane >> 5;
    float* C = p.c + static_cast<int64_t>(bi) * p.c_sb;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = m0 + wm * 32 * FM + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
                const uint32_t col = n0 + wn * 32 * FN + j * 32 + lr;
                float* q = C + static_cast<int64_t>(row) * p.c_sm + static_cast<int64_t>(col) * p.c_sn;
                float v = acc[i][j][r];
                if (p.beta != 0.0f) v = p.beta * *q + v;
                *q = v;
            }
}

template <int AM, int BMD, int BK, int NS, int FN = 2>
__global__ __launch_bounds__(256, (pl_workgroups<BK, NS, FN>()))
void gemm_f32_pl(GemmArgs p) {
    static_assert(AM != LOAD_S && BMD != LOAD_S, "direct loads need a unit-stride axis");
    static_assert(FN == 1 || FN == 2, "128x64 or 128x128 tiles");
    constexpr int T = 256, NW = 4, FM = 2, RA = 128, RB = 64 * FN;
    using GA = DlGeo<RA, BK, T>;
    using GB = DlGeo<RB, BK, T>;
    constexpr int PER = GA::LOADS + GB::LOADS;  // load instructions per slice per thread
    constexpr int G = BK / 8;                   // fragment groups per slice
    constexpr int MG = 4 * FM * FN;             // MFMAs per group
    static_assert(G >= 2 && G % 2 == 0, "groups alternate between two fragment register sets");
    static_assert(NS >= 2 && (NS - 1) * PER < 64, "stages (vmcnt counts at most 63)");
    // Reads of one group after the first RM MFMAs of the previous group, RPM after each; the
    // first group's loads, up to two after each of NV MFMAs, from the tenth MFMA on where the
    // group is that long (earlier positions measured 2-4 % slower on batched 1024^3 products).
    constexpr int RD = pl_reads<AM, BMD, FM, FN>();
    constexpr int RPM = RD > MG * 3 / 4 ? 2 : 1;
    constexpr int RM = (RD + RPM - 1) / RPM;
    constexpr int NV = (PER + 1) / 2;
    constexpr int VF0 = 10 - RM < MG - RM - NV ? 10 - RM : MG - RM - NV;
    constexpr int VF = VF0 > 0 ? VF0 : 0;
    static_assert(RM + VF + NV <= MG, "MFMAs of a group");

    __shared__ __attribute__((aligned(16))) float smem[NS * (GA::ST + GB::ST)];
    float* As = smem;
    float* Bs = smem + NS * GA::ST;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / 2, wn = wave % 2;
    const int lr = lane & 31, h = lane >> 5;

    uint32_t plane, tm, tn;
    decode_tile(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, &plane, &tm, &tn);
    const uint32_t bi = plane / p.splits, split = plane - bi * p.splits;
    const uint32_t m0 = tm * RA, n0 = tn * RB;
    const uint32_t kb = split * p.k_chunk;
    const uint32_t ktiles = min(p.k - kb, p.k_chunk) / BK;
    const float* A = p.a + static_cast<int64_t>(bi) * p.a_sb + static_cast<int64_t>(m0) * p.a_sm +
                     static_cast<int64_t>(kb) * p.a_sk;
    const float* B = p.b + static_cast<int64_t>(bi) * p.b_sb + static_cast<int64_t>(n0) * p.b_sn +
                     static_cast<int64_t>(kb) * p.b_sk;
    const float alpha_a = p.scale_b ? 1.0f : p.alpha;
    const float alpha_b = p.scale_b ? p.alpha : 1.0f;

    int64_t sa[GA::LOADS], sb[GB::LOADS];
#pragma unroll
    for (int i = 0; i < GA::LOADS; ++i) sa[i] = dl_src<AM, RA, BK>((i * NW + wave) * 64 + lane, p.a_sm, p.a_sk);
#pragma unroll
    for (int i = 0; i < GB::LOADS; ++i) sb[i] = dl_src<BMD, RB, BK>((i * NW + wave) * 64 + lane, p.b_sn, p.b_sk);
    const int64_t a_step = AM == LOAD_K ? BK : static_cast<int64_t>(BK) * p.a_sk;
    const int64_t b_step = BMD == LOAD_K ? BK : static_cast<int64_t>(BK) * p.b_sk;
    // Slice kt into `stage`.
    auto issue = [&](uint32_t kt, int stage) {
        float* as = As + stage * GA::ST;
        float* bs = Bs + stage * GB::ST;
#pragma unroll
        for (int i = 0; i < GA::LOADS; ++i) dl_copy16(A + sa[i] + kt * a_step, as + (i * NW + wave) * 256);
#pragma unroll
        for (int i = 0; i < GB::LOADS; ++i) dl_copy16(B + sb[i] + kt * b_step, bs + (i * NW + wave) * 256);
    };

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    auto run = [&](auto scale) {
        constexpr bool SCALE = decltype(scale)::value;
        floatx4 fa[2][FM], fb[2][FN];
        // Fragment group g of the slice in `stage` into register set `set`.
        auto read = [&](int set, int g, int stage) {
            dl_frag<AM, RA, BK, FM>(fa[set], As + stage * GA::ST, wm * 32 * FM, g, lr, h);
            dl_frag<BMD, RB, BK, FN>(fb[set], Bs + stage * GB::ST, wn * 32 * FN, g, lr, h);
            if constexpr (SCALE) {
#pragma unroll
                for (int i = 0; i < FM; ++i) fa[set][i] = fa[set][i] * alpha_a;
#pragma unroll
                for (int j = 0; j < FN; ++j) fb[set][j] = fb[set][j] * alpha_b;
            }
        };
        // Slices 0 .. NS-2 in flight; slice step kt then issues slice kt + NS - 1 into the
        // stage slice kt - 1 used (clamped to the last slice), so at the barrier of step kt the
        // loads issued after slice kt + 1's are always those of the NS - 2 slices behind it.
#pragma unroll
        for (int s = 0; s + 1 < NS; ++s) issue(min(static_cast<uint32_t>(s), ktiles - 1), s);
        wait_vm<(NS - 2) * PER>();
        __builtin_amdgcn_s_barrier();
        read(0, 0, 0);
        for (uint32_t k0 = 0; k0 < ktiles; k0 += NS) {
#pragma unroll
            for (int u = 0; u < NS; ++u) {
                const uint32_t kt = k0 + u;
#pragma unroll
                for (int g = 0; g + 1 < G; ++g) {
                    read((g + 1) & 1, g + 1, u);
                    if (g == 0) issue(min(kt + NS - 1, ktiles - 1), (u + NS - 1) % NS);
                    mfma_group<FM, FN>(acc, fa[g & 1], fb[g & 1]);
                    pl_after_each_mfma<RM, 0x100, RPM>();
                    if (g == 0) {
                        if constexpr (VF > 0) __builtin_amdgcn_sched_group_barrier(0x008, VF, 0);
                        pl_after_each_mfma<NV, 0x010, 2>();
                        __builtin_amdgcn_sched_group_barrier(0x008, MG - RM - VF - NV, 0);
                    } else {
                        __builtin_amdgcn_sched_group_barrier(0x008, MG - RM, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                // Slice kt + 1 landed for every wave, slice kt read by every wave.
                wait_vm<(NS - 2) * PER>();
                wait_lgkm0();
                __builtin_amdgcn_s_barrier();
                constexpr int L = (G - 1) & 1;
                read(0, 0, (u + 1) % NS);  // past the last slice: unused
                mfma_group<FM, FN>(acc, fa[L], fb[L]);
                pl_after_each_mfma<RM, 0x100, RPM>();
                __builtin_amdgcn_sched_group_barrier(0x008, MG - RM, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    if (alpha_a != 1.0f || alpha_b != 1.0f) {
        run(std::true_type{});
    } else {
        run(std::false_type{});
    }

    // Epilogue as gemm_f32_dl's, every element inside the output.
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
                    P[static_cast<int64_t>(row) * p.n + col] = acc[i][j][r];
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
                float* q = C + static_cast<int64_t>(row) * p.c_sm + static_cast<int64_t>(col) * p.c_sn;
                float v = acc[i][j][r];
                if (p.beta != 0.0f) v = p.beta * *q + v;
                *q = v;
            }
}

// gemm_f32_pl256<AM, BMD, BK, NS>: the pipelined loop on full 256x128 tiles with eight waves
// (4x2, each 2x2 blocks of 32x32 as in gemm_f32_pl). The waves keep gemm_f32_pl's fragment
// reads per MFMA and two waves per SIMD, while one workgroup's stages serve twice the rows of
// B: it loads 3/4 of the operand bytes per FLOP that two 128x128 workgroups do. One workgroup
// per compute unit (96 KiB of stages). Every K in whole steps of NS slices; M a multiple of 256,
// N of 128; no split.
// Tiles are walked in groups of PL256_GROUP tile-rows: an XCD's 32 resident tiles then form a
// 4 x 8 block, 1024 x 1024 of C, which reads the fewest A rows plus B columns at a time (traffic
// below the L2 on 4096^3: 3.0x the algorithmic bytes, against 3.7x in groups of 8).
constexpr uint32_t PL256_GROUP = 4;
template <int AM, int BMD, int BK, int NS>
__global__ __launch_bounds__(512, 1) void gemm_f32_pl256(GemmArgs p) {
    constexpr int FN = 2, RA = 256, RB = 128;
    using GA = DlGeo<RA, BK, 512>;
    using GB = DlGeo<RB, BK, 512>;
    __shared__ __attribute__((aligned(16))) float smem[NS * (GA::ST + GB::ST)];
    uint32_t plane, tm, tn;
    decode_tile<PL256_GROUP>(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, &plane, &tm, &tn);
    const uint32_t m0 = tm * RA, n0 = tn * RB;
    const float* A = p.a + static_cast<int64_t>(plane) * p.a_sb + static_cast<int64_t>(m0) * p.a_sm;
    const float* B = p.b + static_cast<int64_t>(plane) * p.b_sb + static_cast<int64_t>(n0) * p.b_sn;
    floatx16 acc[2][FN];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    pl_tile_loop<AM, BMD, BK, NS, FN, 4>(p, smem, A, B, p.k / BK, acc);
    pl_store_c<FN>(p, acc, plane, m0, n0);
}

// gemm_f32_pl2x<AM, BMD, BK, NS>: the pipelined loop on full 256x256 tiles with eight waves (2x4,
// each 4x2 blocks of 32x32: 128 x 64 of C, 128 accumulators), two per SIMD, one workgroup per
// compute unit (128 KiB of stages): per FLOP 2/3 of the operand loads of the 256x128 tiles and
// 3/4 of their fragment reads. With B contiguous along N (each wave instruction a 1 KiB k-row
// of B) a slice's B loads go out in the step's last fragment group, apart from its A loads:
// issued together they held 4096^3 at 134 TFLOP/s, apart 148. Every K in whole steps of NS
// slices; M and N multiples of 256; no split.
template <int AM, int BMD, int BK, int NS>
__global__ __launch_bounds__(512, 1) void gemm_f32_pl2x(GemmArgs p) {
    constexpr int FM = 4, FN = 2, WM = 2, WN = 4, RA = 256, RB = 256;
    using GA = DlGeo<RA, BK, 512>;
    using GB = DlGeo<RB, BK, 512>;
    __shared__ __attribute__((aligned(16))) float smem[NS * (GA::ST + GB::ST)];
    uint32_t plane, tm, tn;
    decode_tile<PL256_GROUP>(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, &plane, &tm, &tn);
    const uint32_t m0 = tm * RA, n0 = tn * RB;
    const float* A = p.a + static_cast<int64_t>(plane) * p.a_sb + static_cast<int64_t>(m0) * p.a_sm;
    const float* B = p.b + static_cast<int64_t>(plane) * p.b_sb + static_cast<int64_t>(n0) * p.b_sn;
    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    pl_tile_loop<AM, BMD, BK, NS, FN, WM, FM, WN, BMD == LOAD_MN>(p, smem, A, B, p.k / BK, acc);
    pl_store_c<FN, FM, WN>(p, acc, plane, m0, n0);
}

// gemm_f32_sk<AM, BMD, BK, NS>: stream-K over the pipelined loop of full 128x128 tiles. The T
// output tiles of S = K / (NS * BK) pipeline steps each make T * S steps, cut into gridDim.x
// = G contiguous runs as even as integers allow (run r: [r * T * S / G, (r + 1) * T * S / G)),
// so every compute unit gets the same work whatever T is. The planner keeps every run at
// least S long (T >= G), so a tile's steps fall to at most two runs: a tile split at run
// boundary b (1 <= b < G) is the last part of run b - 1 and the first part of run b. The
// first part, which run b takes at its start, covers the tile's first K steps and the last
// part, which run b - 1 takes at its end, the rest: every run starts at k = 0 like a plain
// grid, and the last part usually finds the first one done. The two sums meet in slots 2b
// (last part) and 2b + 1 (first part) of `partial` and a ticket counter, counters[b]:
//   * the first part stores its sum, then takes a ticket;
//   * the last part first reads the counter: when the first part's ticket is there, it adds
//     that part's sum to its own at once; otherwise it stores its sum and takes a ticket too;
//   * whichever holds the second ticket adds the other's sum to its own (a + b and b + a are
//     the same float), applies beta * C, stores the tile and clears the counter for the next
//     launch.
// No workgroup waits for another, and every result depends on the shape alone. Tiles a run
// covers whole are stored directly. The sums and tickets move through device-scope (agent)
// accesses, which no XCD's L2 keeps a stale copy of: relaxed atomic stores acknowledged before
// the ticket is taken, relaxed atomic loads issued only after the ticket is seen. No fence
// writes back or invalidates an XCD's L2, which holds the operand panels of the other runs.
// Runs are numbered in XCD order (run r on XCD r * 8 / G), so consecutive runs, which share
// tiles and operand panels, sit on one XCD. One workgroup per compute unit (BK = 32); partial
// holds 2G slots of 128x128 floats.
template <int AM, int BMD, int BK, int NS>
__global__ __launch_bounds__(256, 1) void gemm_f32_sk(GemmArgs p) {
    constexpr int FN = 2, RA = 128, RB = 128, SLOT = 128 * 128;  // floats per partial slot
    using GA = DlGeo<RA, BK, 256>;
    using GB = DlGeo<RB, BK, 256>;
    // The ticket word lives in the stages' own LDS array, past the stages: a second LDS object
    // would keep the compiler from telling the stages' direct loads apart from its fragment
    // reads, and it would then wait for every load in flight before each read.
    __shared__ __attribute__((aligned(16))) float smem[NS * (GA::ST + GB::ST) + 4];
    uint32_t& ticket = *reinterpret_cast<uint32_t*>(smem + NS * (GA::ST + GB::ST));
    const int tid = threadIdx.x;

    const uint32_t G = gridDim.x, bid = blockIdx.x;
    const uint32_t xcd = bid & 7u, slot_in = bid >> 3, q8 = G >> 3, r8 = G & 7u;
    const uint32_t r = xcd < r8 ? xcd * (q8 + 1) + slot_in : r8 * (q8 + 1) + (xcd - r8) * q8 + slot_in;
    const uint32_t per_plane = p.tiles_m * p.tiles_n;
    const uint64_t T = static_cast<uint64_t>(per_plane) * p.batch;
    const uint32_t S = p.k / (NS * BK);
    const uint64_t steps = T * S;
    uint64_t x = static_cast<uint64_t>(r) * steps / G;
    const uint64_t end = static_cast<uint64_t>(r + 1) * steps / G;

    auto add_other = [&](floatx16 (&acc)[2][FN], const float* other) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    acc[i][j][e] = acc[i][j][e] + __hip_atomic_load(other + ((i * FN + j) * 16 + e) * 256,
                                                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
    };

    while (x < end) {
        const uint64_t t = x / S;
        const uint32_t s0 = static_cast<uint32_t>(x - t * S);
        const uint32_t s1 = static_cast<uint32_t>(min(static_cast<uint64_t>(S), s0 + (end - x)));
        const uint32_t len = s1 - s0;
        const bool whole = len == S;
        const bool first_part = s0 > 0;            // the run started inside this tile
        const uint32_t b = first_part ? r : r + 1;  // the run boundary splitting the tile
        // K steps of this part: the first part from k = 0, the last part the rest.
        const uint32_t k0 = whole || first_part ? 0 : S - len;
        // Tile t: plane, then groups of eight tile rows walked column by column (decode_tile's
        // order), so a run of consecutive tiles reuses A and B panels in the XCD's L2.
        const uint32_t bi = static_cast<uint32_t>(t / per_plane);
        const uint32_t tp = static_cast<uint32_t>(t - static_cast<uint64_t>(bi) * per_plane);
        const uint32_t group = tp / (8 * p.tiles_n), first_m = group * 8;
        const uint32_t gm = min(p.tiles_m - first_m, 8u), in_group = tp - group * 8 * p.tiles_n;
        const uint32_t m0 = (first_m + in_group % gm) * RA, n0 = (in_group / gm) * RB;
        const uint32_t kb = k0 * NS * BK;
        const float* A = p.a + static_cast<int64_t>(bi) * p.a_sb + static_cast<int64_t>(m0) * p.a_sm +
                         static_cast<int64_t>(kb) * p.a_sk;
        const float* B = p.b + static_cast<int64_t>(bi) * p.b_sb + static_cast<int64_t>(n0) * p.b_sn +
                         static_cast<int64_t>(kb) * p.b_sk;
        floatx16 acc[2][FN];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
        pl_tile_loop<AM, BMD, BK, NS, FN>(p, smem, A, B, len * NS, acc);

        if (whole) {
            pl_store_c<FN>(p, acc, bi, m0, n0);
        } else {
            float* mine = p.partial + static_cast<int64_t>(2 * b + (first_part ? 1 : 0)) * SLOT + tid;
            const float* other = p.partial + static_cast<int64_t>(2 * b + (first_part ? 0 : 1)) * SLOT + tid;
            bool done = false;
            if (!first_part) {
                if (tid == 0) {
                    ticket = __hip_atomic_load(p.counters + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                __syncthreads();
                done = ticket == 1;  // the first part's sum is complete
                __syncthreads();     // every thread has read `ticket` before it is reused
            }
            if (!done) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
#pragma unroll
                        for (int e = 0; e < 16; ++e) {
                            __hip_atomic_store(mine + ((i * FN + j) * 16 + e) * 256, acc[i][j][e],
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        }
                wait_vm<0>();  // every store of this thread acknowledged
                __syncthreads();
                if (tid == 0) {
                    ticket = __hip_atomic_fetch_add(p.counters + b, 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
                }
                __syncthreads();
                done = ticket == 1;
            }
            if (done) {
                add_other(acc, other);
                pl_store_c<FN>(p, acc, bi, m0, n0);
                if (tid == 0) __hip_atomic_store(p.counters + b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        x += len;
        // The loop leaves loads of its last slice in flight into the stages: let them land,
        // and every wave finish reading, before the next tile's loads reuse the stages.
        wait_vm<0>();
        wait_lgkm0();
        __syncthreads();
    }
}

// gemm_f32_kw<AM, BMD, BK, NS>: a 64x64 output tile per workgroup whose four waves each
// compute the whole tile (2x2 blocks of 32x32) over a quarter of the K chunk, through their own
// NS LDS stages filled by their own direct loads: no barrier inside the loop (each wave waits
// only for its own loads), the same in-wave pipelining as gemm_f32_pl. Launched with two stages
// of 32-deep slices: a slice's A loads go out in the first fragment group of the slice before
// it, its B loads in the second, and each slice waits for all of them: every A row segment is
// then a whole 128-byte line (against four stages of 16, A loads in one step's first group and B
// loads in its last: 1024^3 and config 4 the same within 1-2 %). With more stages the B loads
// go out in the last group. The four sums meet
// through LDS at the end in a fixed order, (s0 + s1) + (s2 + s3), each wave adding and storing
// one 32x32 block. One workgroup per compute unit (128 KB of stages): for grids of about one
// 64x64 tile per compute unit (1024^3: 75 -> 97-99 TFLOP/s against four wave groups of four
// waves sharing stages). Full 64x64 tiles, K chunks in whole multiples of 4 * NS * BK.
template <int AM, int BMD, int BK, int NS>
__global__ __launch_bounds__(256, 1) void gemm_f32_kw(GemmArgs p) {
    constexpr int R = 64, FM = 2, FN = 2, W = 4;
    using GA = DlGeo<R, BK, 64>;
    using GB = DlGeo<R, BK, 64>;
    constexpr int PER = GA::LOADS + GB::LOADS;
    constexpr int G = BK / 8;
    static_assert(G >= 2 && G % 2 == 0, "groups alternate between two fragment register sets");
    static_assert(NS >= 2 && (NS - 1) * PER < 64, "stages");
    constexpr int RD = pl_reads<AM, BMD, FM, FN>();
    constexpr int RPM = RD > 12 ? 2 : 1;
    constexpr int RM = (RD + RPM - 1) / RPM;
    constexpr int VF = RM < 10 ? 10 - RM : 0;
    constexpr int VPM = PER / 4;  // loads after each of two MFMAs (A or B: half the slice)
    static_assert(RM + VF + 2 <= 16, "a group has 16 MFMAs");
    constexpr int WST = NS * (GA::ST + GB::ST);
    static_assert(W * WST >= W * FM * FN * 16 * 64, "the sums fit in the stages");
    __shared__ __attribute__((aligned(16))) float smem[W * WST];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 31, h = lane >> 5;
    float* As = smem + wave * WST;
    float* Bs = As + NS * GA::ST;

    uint32_t plane, tm, tn;
    decode_tile(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, &plane, &tm, &tn);
    const uint32_t bi = plane / p.splits, split = plane - bi * p.splits;
    const uint32_t m0 = tm * R, n0 = tn * R;
    const uint32_t kb = split * p.k_chunk;
    const uint32_t per = min(p.k - kb, p.k_chunk) / W;
    const uint32_t ktiles = per / BK;
    const uint32_t k0w = kb + wave * per;
    const float* A = p.a + static_cast<int64_t>(bi) * p.a_sb + static_cast<int64_t>(m0) * p.a_sm +
                     static_cast<int64_t>(k0w) * p.a_sk;
    const float* B = p.b + static_cast<int64_t>(bi) * p.b_sb + static_cast<int64_t>(n0) * p.b_sn +
                     static_cast<int64_t>(k0w) * p.b_sk;
    const float alpha_a = p.scale_b ? 1.0f : p.alpha;
    const float alpha_b = p.scale_b ? p.alpha : 1.0f;

    int64_t sa[GA::LOADS], sb[GB::LOADS];
#pragma unroll
    for (int i = 0; i < GA::LOADS; ++i) sa[i] = dl_src<AM, R, BK>(i * 64 + lane, p.a_sm, p.a_sk);
#pragma unroll
    for (int i = 0; i < GB::LOADS; ++i) sb[i] = dl_src<BMD, R, BK>(i * 64 + lane, p.b_sn, p.b_sk);
    const int64_t a_step = AM == LOAD_K ? BK : static_cast<int64_t>(BK) * p.a_sk;
    const int64_t b_step = BMD == LOAD_K ? BK : static_cast<int64_t>(BK) * p.b_sk;
    // A slice's A loads go out in the first fragment group of the step three slices ahead of
    // it, its B loads in that step's last group (1024^3: 98-99 -> 101.5 TFLOP/s, config 4
    // 114-115 -> 117-120 against all eight together in the first group).
    auto issue_a = [&](uint32_t kt, int stage) {
        float* as = As + stage * GA::ST;
#pragma unroll
        for (int i = 0; i < GA::LOADS; ++i) dl_copy16(A + sa[i] + kt * a_step, as + i * 256);
    };
    auto issue_b = [&](uint32_t kt, int stage) {
        float* bs = Bs + stage * GB::ST;
#pragma unroll
        for (int i = 0; i < GB::LOADS; ++i) dl_copy16(B + sb[i] + kt * b_step, bs + i * 256);
    };
    auto issue = [&](uint32_t kt, int stage) {
        issue_a(kt, stage);
        issue_b(kt, stage);
    };
    constexpr bool TWO = NS == 2;  // two stages: B loads in the second group, wait for all
    static_assert(!TWO || G >= 4, "two stages need four groups a slice");
    constexpr int AFTER = TWO ? 0 : (NS - 3) * PER + GA::LOADS;
    static_assert(TWO || NS >= 3, "A and B loads of a slice go out in different steps' groups");

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    auto run = [&](auto scale) {
        constexpr bool SCALE = decltype(scale)::value;
        floatx4 fa[2][FM], fb[2][FN];
        auto read = [&](int set, int g, int stage) {
            dl_frag<AM, R, BK, FM>(fa[set], As + stage * GA::ST, 0, g, lr, h);
            dl_frag<BMD, R, BK, FN>(fb[set], Bs + stage * GB::ST, 0, g, lr, h);
            if constexpr (SCALE) {
#pragma unroll
                for (int i = 0; i < FM; ++i) fa[set][i] = fa[set][i] * alpha_a;
#pragma unroll
                for (int j = 0; j < FN; ++j) fb[set][j] = fb[set][j] * alpha_b;
            }
        };
#pragma unroll
        for (int s = 0; s + 1 < NS; ++s) issue(min(static_cast<uint32_t>(s), ktiles - 1), s);
        wait_vm<(NS - 2) * PER>();
        read(0, 0, 0);
        for (uint32_t k0 = 0; k0 < ktiles; k0 += NS) {
#pragma unroll
            for (int u = 0; u < NS; ++u) {
                const uint32_t kt = k0 + u;
#pragma unroll
                for (int g = 0; g + 1 < G; ++g) {
                    read((g + 1) & 1, g + 1, u);
                    if (g == 0) issue_a(min(kt + NS - 1, ktiles - 1), (u + NS - 1) % NS);
                    if (TWO && g == 1) issue_b(min(kt + NS - 1, ktiles - 1), (u + NS - 1) % NS);
                    mfma_group<FM, FN>(acc, fa[g & 1], fb[g & 1]);
                    pl_after_each_mfma<RM, 0x100, RPM>();
                    if (g == 0) {
                        if constexpr (VF > 0) __builtin_amdgcn_sched_group_barrier(0x008, VF, 0);
                        pl_after_each_mfma<2, 0x010, VPM>();
                        __builtin_amdgcn_sched_group_barrier(0x008, 16 - RM - VF - 2, 0);
                    } else if (TWO && g == 1) {
                        pl_after_each_mfma<2, 0x010, VPM>();
                        __builtin_amdgcn_sched_group_barrier(0x008, 16 - RM - 2, 0);
                    } else {
                        __builtin_amdgcn_sched_group_barrier(0x008, 16 - RM, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                wait_vm<AFTER>();  // slice kt + 1 landed (this wave's own loads)
                constexpr int L = (G - 1) & 1;
                read(0, 0, (u + 1) % NS);
                if constexpr (!TWO) issue_b(min(kt + NS - 1, ktiles - 1), (u + NS - 1) % NS);
                mfma_group<FM, FN>(acc, fa[L], fb[L]);
                pl_after_each_mfma<RM, 0x100, RPM>();
                if constexpr (!TWO) pl_after_each_mfma<2, 0x010, VPM>();
                __builtin_amdgcn_sched_group_barrier(0x008, 16 - RM - (TWO ? 0 : 2), 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    if (alpha_a != 1.0f || alpha_b != 1.0f) {
        run(std::true_type{});
    } else {
        run(std::false_type{});
    }

    // The four sums meet through LDS: wave w adds block w of every wave's sum as
    // (s0 + s1) + (s2 + s3) and stores it.
    wait_vm<0>();
    __syncthreads();
    {
        float* mine = smem + wave * (FM * FN * 16 * 64) + lane;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) mine[((i * FN + j) * 16 + r) * 64] = acc[i][j][r];
    }
    __syncthreads();
    const int bi_ = wave >> 1, bj = wave & 1;
    float v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float* q = smem + ((bi_ * FN + bj) * 16 + r) * 64 + lane;
        constexpr int S = FM * FN * 16 * 64;
        v[r] = (q[0] + q[S]) + (q[2 * S] + q[3 * S]);
    }
    if (p.partial != nullptr) {
        float* P = p.partial + static_cast<int64_t>(plane) * p.m * p.n;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = m0 + bi_ * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
            const uint32_t col = n0 + bj * 32 + lr;
            P[static_cast<int64_t>(row) * p.n + col] = v[r];
        }
        return;
    }
    float* C = p.c + static_cast<int64_t>(bi) * p.c_sb;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t row = m0 + bi_ * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
        const uint32_t col = n0 + bj * 32 + lr;
        float* q = C + static_cast<int64_t>(row) * p.c_sm + static_cast<int64_t>(col) * p.c_sn;
        float x = v[r];
        if (p.beta != 0.0f) x = p.beta * *q + x;
        *q = x;
    }
}

}  // namespace gemm_detail
}  // namespace lg
