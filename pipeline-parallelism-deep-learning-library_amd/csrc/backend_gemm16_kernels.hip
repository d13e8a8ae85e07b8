// gfx950 kernel of the Backend's 16-bit gemm (F16 / BF16 tensors): CpuBackend's arithmetic,
// bit for bit.
//
// crates/cpu/src/lib.rs:270-291 runs `accumulate` (:664-691) with loaders that widen each
// element exactly to f32 and a store that rounds to 16 bits, so every output is
//   acc = beta == 0 ? +0 : beta * widen(C)                        (C unread when beta is 0)
//   if alpha != 0: for k ascending: acc = acc + (alpha * widen(A[row, k])) * widen(B[k, col])
//   C = narrow(acc)
// with one f32 rounding per multiply and per add, and narrow = the half crate's (2.7.1)
// from_f32_const: round to nearest even on the f32 bits, NaN kept quiet with its sign and top
// payload bits. Here each output is one lane's private f32 accumulator that sees exactly these
// operations in this order; the file is compiled with -ffp-contract=off, so no multiply and add
// fuse. alpha * widen(a) does not depend on the column, so it is formed once per A element as
// the slice is staged: the same rounding the loop performs at every use. That leaves one
// multiply and one add per term, on the VALU (the f32 matrix cores sum in their own order).
//
// Tiling: 128x128 outputs per 256-thread workgroup, 8x8 per thread as two 4-row by two
// 4-column blocks 64 apart, so each k costs a thread four 128-bit LDS reads (a wave's reads
// are 4 broadcast addresses of A and 16 consecutive 16-byte words of B: no bank conflicts) for
// 128 VALU operations; 64x64 tiles (4x4 per thread, two reads for 32 operations) where the
// 128x128 grid would leave compute units idle. K advances in slices of 16 staged in LDS as f32, [k][row] and
// [k][col], double buffered; the next slice's 16-bit elements are in flight in registers while
// the current slice is consumed. The last slice runs only its valid k: a padded term would
// add +0 (turning a -0 sum into +0) or 0 * inf.
#include <hip/hip_runtime.h>

#include "lg_internal.h"

namespace lg {
namespace {

constexpr int QT = 256;  // threads per workgroup, 16 x 16
constexpr int QK = 16;   // K slice
// Square tiles of QM = 16 * TM outputs a side, TM x TM per thread as (TM/4)^2 blocks of 4x4
// whose rows and columns are 64 apart: TM = 8 (128x128 tiles), or TM = 4 (64x64 tiles, for
// grids that would leave compute units idle).
template <int TM>
struct Geo16 {
    static constexpr int QM = 16 * TM;       // output tile edge
    static constexpr int QP = QM + 4;        // LDS row pitch in floats: 16-byte rows, k rows 4 banks apart
    static constexpr int QL = QM * QK / QT;  // elements per thread and operand per slice
    static constexpr int NB = TM / 4;        // 4x4 blocks per thread along each axis
    static_assert((TM == 4 || TM == 8) && QL * QT == QM * QK, "whole slices per thread");
};

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Exact widening (every finite 16-bit value is an f32).
template <int HK>
__device__ inline float widen(uint16_t h) {
    if constexpr (HK == 1) return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
    else return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// f32 -> f16 bits as the half crate's f16::from_f32_const: ties to even on the f32 bits,
// f16 subnormals kept, overflow to infinity, NaN quiet (0x0200) with the top ten payload bits.
__device__ inline uint16_t to_f16(float v) {
    const uint32_t x = __builtin_bit_cast(uint32_t, v);
    const uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xffu, man = x & 0x7fffffu;
    if (exp == 0xffu) return static_cast<uint16_t>(sign | 0x7c00u | (man ? 0x0200u | (man >> 13) : 0u));
    const int e = static_cast<int>(exp) - 112;  // the f16 biased exponent
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    if (e > 0) {
        // Normal: drop 13 bits; a round-up carry may ripple into the exponent (up to infinity).
        const uint32_t kept = sign | (static_cast<uint32_t>(e) << 10) | (man >> 13);
        const uint32_t rest = man & 0x1fffu;
        return static_cast<uint16_t>(kept + ((rest > 0x1000u || (rest == 0x1000u && (kept & 1u))) ? 1u : 0u));
    }
    const int shift = 14 - e;  // f16 subnormal: units of 2^-24
    if (shift > 24) return static_cast<uint16_t>(sign);
    const uint32_t sig = man | 0x800000u;
    const uint32_t kept = sig >> shift, rest = sig & ((1u << shift) - 1u), half = 1u << (shift - 1);
    return static_cast<uint16_t>(sign | (kept + ((rest > half || (rest == half && (kept & 1u))) ? 1u : 0u)));
}

// f32 -> bf16 bits as bf16::from_f32_const: the high half rounded to nearest even, NaN | 0x40.
__device__ inline uint16_t to_bf16(float v) {
    const uint32_t x = __builtin_bit_cast(uint32_t, v);
    if ((x & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((x >> 16) | 0x40u);
    return static_cast<uint16_t>((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

template <int HK>
__device__ inline uint16_t narrow(float v) {
    if constexpr (HK == 1) return to_bf16(v);
    else return to_f16(v);
}

// One operand's slice [k0, k0+QK) x [r0, r0+QM) into registers: element e of the slice is
// (k = e % QK, row = e / QK) when the operand is contiguous along K, else (k = e / QM,
// row = e % QM), so consecutive lanes read consecutive addresses either way. Outside the
// operand: 0 (never summed: rows past the edge are not stored, k past the end not run).
template <int TM, typename G = Geo16<TM>>
__device__ inline void load_slice(uint16_t (&r)[G::QL], const uint16_t* __restrict__ p, int64_t s_row,
                                  int64_t s_k, uint32_t kfast, uint32_t rows_left, uint32_t k0,
                                  uint32_t k, int tid) {
#pragma unroll
    for (int it = 0; it < G::QL; ++it) {
        const int e = it * QT + tid;
        const uint32_t kk = kfast ? e % QK : e / G::QM, row = kfast ? e / QK : e % G::QM;
        r[it] = (row < rows_left && k0 + kk < k)
                    ? p[static_cast<int64_t>(row) * s_row + static_cast<int64_t>(k0 + kk) * s_k]
                    : uint16_t(0);
    }
}

// Registers -> LDS stage [k][row] as f32, each value times `scale` (alpha for A, so the stage
// holds alpha*a rounded to f32; 1 for B, an exact copy).
template <int HK, bool SCALE, int TM, typename G = Geo16<TM>>
__device__ inline void stage_slice(float* __restrict__ st, const uint16_t (&r)[G::QL], uint32_t kfast,
                                   float scale, int tid) {
#pragma unroll
    for (int it = 0; it < G::QL; ++it) {
        const int e = it * QT + tid;
        const int kk = kfast ? e % QK : e / G::QM, row = kfast ? e / QK : e % G::QM;
        const float v = widen<HK>(r[it]);
        st[kk * G::QP + row] = SCALE ? scale * v : v;
    }
}

template <int HK, int TM>
__global__ __launch_bounds__(QT) void gemm16_seq(Gemm16SeqArgs p) {
    using G = Geo16<TM>;
    constexpr int QM = G::QM, QP = G::QP, QL = G::QL, NB = G::NB;
    __shared__ __attribute__((aligned(16))) float As[2][QK * QP];
    __shared__ __attribute__((aligned(16))) float Bs[2][QK * QP];
    const uint32_t tm = blockIdx.x / p.tiles_n, tn = blockIdx.x - tm * p.tiles_n;
    const uint32_t m0 = tm * QM, n0 = tn * QM;
    const uint32_t mrem = p.m - m0, nrem = p.n - n0;
    const int tid = threadIdx.x, tx = tid % 16, ty = tid / 16;

    // Output (i, j) of this thread: row ty*4 + i%4 + 64*(i/4), column tx*4 + j%4 + 64*(j/4).
    float acc[TM][TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const uint32_t row = ty * 4 + (i & 3) + 64 * (i >> 2);
#pragma unroll
        for (int j = 0; j < TM; ++j) {
            const uint32_t col = tx * 4 + (j & 3) + 64 * (j >> 2);
            acc[i][j] = 0.0f;
            if (p.beta != 0.0f && row < mrem && col < nrem) {
                acc[i][j] = p.beta * widen<HK>(p.c[static_cast<int64_t>(m0 + row) * p.c_sm + (n0 + col)]);
            }
        }
    }

    if (p.alpha != 0.0f && p.k > 0) {
        const uint16_t* A = p.a + static_cast<int64_t>(m0) * p.a_sm;
        const uint16_t* B = p.b + static_cast<int64_t>(n0) * p.b_sn;
        uint16_t ra[QL], rb[QL];
        const uint32_t ktiles = (p.k + QK - 1) / QK;
        load_slice<TM>(ra, A, p.a_sm, p.a_sk, p.a_kfast, mrem, 0, p.k, tid);
        load_slice<TM>(rb, B, p.b_sn, p.b_sk, p.b_kfast, nrem, 0, p.k, tid);
        stage_slice<HK, true, TM>(As[0], ra, p.a_kfast, p.alpha, tid);
        stage_slice<HK, false, TM>(Bs[0], rb, p.b_kfast, 1.0f, tid);
        __syncthreads();
        for (uint32_t kt = 0; kt < ktiles; ++kt) {
            const int s = kt & 1;
            const bool more = kt + 1 < ktiles;
            if (more) {
                load_slice<TM>(ra, A, p.a_sm, p.a_sk, p.a_kfast, mrem, (kt + 1) * QK, p.k, tid);
                load_slice<TM>(rb, B, p.b_sn, p.b_sk, p.b_kfast, nrem, (kt + 1) * QK, p.k, tid);
            }
            const float* as = As[s];
            const float* bs = Bs[s];
            auto term = [&](int kk) {
                float av[TM], bv[TM];
#pragma unroll
                for (int q = 0; q < NB; ++q) {
                    const f32x4 a4 = *reinterpret_cast<const f32x4*>(as + kk * QP + 64 * q + ty * 4);
                    const f32x4 b4 = *reinterpret_cast<const f32x4*>(bs + kk * QP + 64 * q + tx * 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        av[4 * q + e] = a4[e];
                        bv[4 * q + e] = b4[e];
                    }
                }
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j) {
                        const float prod = av[i] * bv[j];
                        acc[i][j] = acc[i][j] + prod;
                    }
            };
            const uint32_t klen = more ? QK : p.k - kt * QK;
            if (klen == QK) {
#pragma unroll
                for (int kk = 0; kk < QK; ++kk) term(kk);
            } else {
                for (uint32_t kk = 0; kk < klen; ++kk) term(static_cast<int>(kk));
            }
            if (more) {
                stage_slice<HK, true, TM>(As[s ^ 1], ra, p.a_kfast, p.alpha, tid);
                stage_slice<HK, false, TM>(Bs[s ^ 1], rb, p.b_kfast, 1.0f, tid);
            }
            __syncthreads();
        }
    }

#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const uint32_t row = ty * 4 + (i & 3) + 64 * (i >> 2);
#pragma unroll
        for (int j = 0; j < TM; ++j) {
            const uint32_t col = tx * 4 + (j & 3) + 64 * (j >> 2);
            if (row < mrem && col < nrem) {
                p.c[static_cast<int64_t>(m0 + row) * p.c_sm + (n0 + col)] = narrow<HK>(acc[i][j]);
            }
        }
    }
}

}  // namespace

uint64_t gemm16_seq_workgroups(uint32_t m, uint32_t n, uint32_t tile) {
    return static_cast<uint64_t>((m + tile - 1) / tile) * ((n + tile - 1) / tile);
}

void launch_gemm16_seq(Context* ctx, hipStream_t s, const Gemm16SeqArgs& args) {
    const uint64_t groups = static_cast<uint64_t>(args.tiles_m) * args.tiles_n;
    if ((args.tile != 64 && args.tile != 128) || groups == 0 ||
        groups != gemm16_seq_workgroups(args.m, args.n, args.tile) || groups * QT > 0xffffffffull) {
        fail_invalid("16-bit gemm grid does not match its extents");
    }
    const dim3 grid(static_cast<uint32_t>(groups));
    if (args.kind == 1) {
        if (args.tile == 64) {
            hipLaunchKernelGGL((gemm16_seq<1, 4>), grid, dim3(QT), 0, s, args);
        } else {
            hipLaunchKernelGGL((gemm16_seq<1, 8>), grid, dim3(QT), 0, s, args);
        }
    } else {
        if (args.tile == 64) {
            hipLaunchKernelGGL((gemm16_seq<0, 4>), grid, dim3(QT), 0, s, args);
        } else {
            hipLaunchKernelGGL((gemm16_seq<0, 8>), grid, dim3(QT), 0, s, args);
        }
    }
    check_hip(hipGetLastError(), "gemm16_seq");
    note_launch(ctx, args.kind == 1 ? "gemm_bf16_seq" : "gemm_f16_seq");
}

}  // namespace lg
