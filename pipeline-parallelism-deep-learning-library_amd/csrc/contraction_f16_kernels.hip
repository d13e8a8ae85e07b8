// gfx950 kernels of the f16 contraction: C = alpha * A.B + beta * C on half operands.
//
// The reference sums exact f16 products in double-float f32 and rounds once to f16
// (shaders/contraction.metal:444-678), because an f32 accumulator can cross an f16 rounding
// midpoint. Here the products (22 significant bits) are exact in f64 and the sums run in f64
// on the f64 matrix cores (v_mfma_f64_16x16x4_f64), relative error ~2^-53 per step; alpha*acc
// and beta*C (exact in f64: 24 x 11 bits) add in f64, and each output rounds ONCE, f64 -> f16,
// to nearest even. Where the exact result fits in 53 bits this is the correctly rounded f16 of
// the exact value, which is also what the reference's double-float path returns.
#include <hip/hip_runtime.h>

#include "gemm_kernel.h"
#include "lg_internal.h"

namespace lg {
namespace {

typedef double f64x4 __attribute__((ext_vector_type(4)));

// Exact: every finite f16 is an f32, every f32 an f64.
__device__ inline double h2d(uint16_t bits) {
    return static_cast<double>(static_cast<float>(__builtin_bit_cast(_Float16, bits)));
}

// f64 -> f16 bits, round to nearest even, with f16 subnormals, overflow to infinity and NaN
// as the quiet NaN of the same sign (the reference's f32_to_f16_bits convention). Integer
// arithmetic on the f64 fields, so there is exactly one rounding.
__device__ inline uint16_t d2h(double x) {
    const uint64_t b = __builtin_bit_cast(uint64_t, x);
    const uint32_t sign = static_cast<uint32_t>(b >> 48) & 0x8000u;
    const uint64_t rest = b & 0x7fffffffffffffffull;
    if (rest > 0x7ff0000000000000ull) return static_cast<uint16_t>(sign | 0x7e00u);
    if (rest == 0x7ff0000000000000ull) return static_cast<uint16_t>(sign | 0x7c00u);
    const int e = static_cast<int>(rest >> 52) - 1023;
    const uint64_t mant = rest & 0xfffffffffffffull;
    if (e > 15) return static_cast<uint16_t>(sign | 0x7c00u);
    if (e >= -14) {
        uint32_t exp16 = static_cast<uint32_t>(e + 15);
        uint64_t kept = mant >> 42;
        const uint64_t dropped = mant & ((1ull << 42) - 1);
        const uint64_t halfway = 1ull << 41;
        if (dropped > halfway || (dropped == halfway && (kept & 1))) {
            if (++kept == 0x400) {
                kept = 0;
                if (++exp16 >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
            }
        }
        return static_cast<uint16_t>(sign | (exp16 << 10) | static_cast<uint32_t>(kept));
    }
    if (e < -25) return static_cast<uint16_t>(sign);  // below half the smallest subnormal
    // Subnormal f16: units of 2^-24. x = sig * 2^(e-52) with the implicit bit at 52.
    const uint64_t sig = mant | (1ull << 52);
    const int shift = 28 - e;  // 43 .. 53
    uint64_t kept = sig >> shift;
    const uint64_t dropped = sig & ((1ull << shift) - 1);
    const uint64_t halfway = 1ull << (shift - 1);
    if (dropped > halfway || (dropped == halfway && (kept & 1))) ++kept;  // 0x400 = min normal
    return static_cast<uint16_t>(sign | static_cast<uint32_t>(kept));
}

__device__ inline uint16_t finish(double acc, float alpha, float beta, const uint16_t* c) {
    double r = acc * static_cast<double>(alpha);
    if (beta != 0.0f) r = r + static_cast<double>(beta) * h2d(*c);
    return d2h(r);
}

// 64x64 output tile per 256-thread workgroup: 4 waves in 2x2, each 32x32 = 2x2 blocks of
// v_mfma_f64_16x16x4_f64. Block operand layout (checked on gfx950): A lane l holds row l%16,
// k l/16; B lane l holds column l%16, k l/16; accumulator value v of lane l is row 4*v + l/16,
// column l%16 (rows interleave across the four 16-lane groups).
// K advances 64 at a time through two LDS stages that hold the halves as they are (the f64
// values are formed when a fragment is read, exactly), so a 64-deep slice costs 18 KB per
// stage and each barrier serves 64 MFMAs per wave. While the MFMAs consume stage s, the next
// slice is in flight into registers: two 128-bit loads of eight halves per thread and operand
// when the operand is contiguous along K (stage [row][k]) or along M/N (stage [k][row]),
// predicated 16-bit loads otherwise. 36 KB of LDS keeps four workgroups on a compute unit.
constexpr int HT = 256;
constexpr int HP = HGEMM_BK + 8;        // halves per stage row: 128-bit rows stay 16-byte aligned
constexpr int H_STAGE = HGEMM_BM * HP;  // halves per operand stage (both operands are 64 x 64)
constexpr int HCH = HGEMM_BM * HGEMM_BK / 8 / HT;  // 128-bit chunks per thread and operand
static_assert(HGEMM_BM == 64 && HGEMM_BN == 64 && HGEMM_BK == 64, "stage geometry");
static_assert(HCH * HT * 8 == HGEMM_BM * HGEMM_BK, "each thread stages whole chunks");

typedef uint16_t h8 __attribute__((ext_vector_type(8)));

// One operand's K-slice for thread `tid`: HCH runs of eight halves. `p` is (row 0, k 0) of the
// tile, srow/sk its strides; the runs go along k (LOAD_K, LOAD_S) or along the row axis
// (LOAD_MN). FULL: the slice lies inside the operand, so no predicates.
template <int MODE, bool FULL>
__device__ inline void hload(h8 (&r)[HCH], const uint16_t* __restrict__ p, int64_t srow,
                             int64_t sk, uint32_t rows_left, uint32_t k0, uint32_t klen,
                             int tid) {
#pragma unroll
    for (int it = 0; it < HCH; ++it) {
        const int idx = it * HT + tid;
        if constexpr (MODE == LOAD_MN) {
            const uint32_t kr = k0 + idx / 8, row = (idx % 8) * 8;
            const uint16_t* q = p + static_cast<int64_t>(kr) * sk + row;
            if (FULL) {
                r[it] = *reinterpret_cast<const h8*>(q);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) r[it][e] = (kr < klen && row + e < rows_left) ? q[e] : uint16_t(0);
            }
        } else {
            const uint32_t row = idx / 8, kk = k0 + (idx % 8) * 8;
            const uint16_t* q = p + static_cast<int64_t>(row) * srow;
            if (MODE == LOAD_K && FULL) {
                r[it] = *reinterpret_cast<const h8*>(q + kk);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    r[it][e] = (FULL || (row < rows_left && kk + e < klen))
                                   ? q[static_cast<int64_t>(kk + e) * sk] : uint16_t(0);
                }
            }
        }
    }
}

// Writes the runs to a stage: [k][row] for LOAD_MN, [row][k] otherwise (pitch HP halves).
__device__ inline void hstage(uint16_t* __restrict__ st, const h8 (&r)[HCH], int tid) {
#pragma unroll
    for (int it = 0; it < HCH; ++it) {
        const int idx = it * HT + tid;
        *reinterpret_cast<h8*>(st + (idx / 8) * HP + (idx % 8) * 8) = r[it];
    }
}

// Elements (row, k0 .. k0+3) of a stage, widened exactly: one 64-bit LDS read from a
// [row][k] stage (k0 is a multiple of four, rows are 144 bytes), four 16-bit reads from a
// [k][row] one.
template <int MODE>
__device__ inline void hval4(double (&v)[4], const uint16_t* __restrict__ st, int row, int k0) {
    if constexpr (MODE == LOAD_MN) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = h2d(st[(k0 + j) * HP + row]);
    } else {
        typedef uint16_t h4 __attribute__((ext_vector_type(4)));
        const h4 w = *reinterpret_cast<const h4*>(st + row * HP + k0);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = h2d(w[j]);
    }
}

template <int AM, int BMD>
__global__ __launch_bounds__(HT, 4) void gemm_f16_f64mfma(GemmHalfArgs p) {
    __shared__ __attribute__((aligned(16))) uint16_t smem[4 * H_STAGE];
    uint16_t* As = smem;
    uint16_t* Bs = smem + 2 * H_STAGE;
    uint32_t plane, tm, tn;
    gemm_detail::decode_tile(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, &plane, &tm, &tn);
    const uint32_t m0 = tm * HGEMM_BM, n0 = tn * HGEMM_BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int li = lane & 15, lk = lane >> 4;
    const uint16_t* A = p.a + static_cast<int64_t>(plane) * p.a_sb + static_cast<int64_t>(m0) * p.a_sm;
    const uint16_t* B = p.b + static_cast<int64_t>(plane) * p.b_sb + static_cast<int64_t>(n0) * p.b_sn;
    uint16_t* C = p.c + static_cast<int64_t>(plane) * p.c_sb;
    const uint32_t mrem = p.m - m0, nrem = p.n - n0;
    const bool inner = mrem >= HGEMM_BM && nrem >= HGEMM_BN;

    f64x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};

    h8 ra[HCH], rb[HCH];
    auto load = [&](uint32_t k0) {
        if (inner && k0 + HGEMM_BK <= p.k) {
            hload<AM, true>(ra, A, p.a_sm, p.a_sk, mrem, k0, p.k, tid);
            hload<BMD, true>(rb, B, p.b_sn, p.b_sk, nrem, k0, p.k, tid);
        } else {
            hload<AM, false>(ra, A, p.a_sm, p.a_sk, mrem, k0, p.k, tid);
            hload<BMD, false>(rb, B, p.b_sn, p.b_sk, nrem, k0, p.k, tid);
        }
    };
    const uint32_t ktiles = (p.k + HGEMM_BK - 1) / HGEMM_BK;
    load(0);
    hstage(As, ra, tid);
    hstage(Bs, rb, tid);
    __syncthreads();
    for (uint32_t kt = 0; kt < ktiles; ++kt) {
        const int s = kt & 1;
        const bool more = kt + 1 < ktiles;
        if (more) load((kt + 1) * HGEMM_BK);
        const uint16_t* as = As + s * H_STAGE;
        const uint16_t* bs = Bs + s * H_STAGE;
        // 16-k groups: MFMA step s of group q gives lane group lk the k = 16q + 4lk + s, so
        // a [row][k] stage hands a lane its four k of the group in one 64-bit read. A and B
        // agree on the order, so every product pairs the same k.
#pragma unroll 1
        for (int q = 0; q < HGEMM_BK / 16; ++q) {
            double av[2][4], bv[2][4];
#pragma unroll
            for (int i = 0; i < 2; ++i) hval4<AM>(av[i], as, wm * 32 + i * 16 + li, q * 16 + lk * 4);
#pragma unroll
            for (int j = 0; j < 2; ++j) hval4<BMD>(bv[j], bs, wn * 32 + j * 16 + li, q * 16 + lk * 4);
#pragma unroll
            for (int st = 0; st < 4; ++st)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[i][st], bv[j][st],
                                                                         acc[i][j], 0, 0, 0);
        }
        if (more) {
            hstage(As + (s ^ 1) * H_STAGE, ra, tid);
            hstage(Bs + (s ^ 1) * H_STAGE, rb, tid);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t row = m0 + wm * 32 + i * 16 + v * 4 + lk;
                const uint32_t col = n0 + wn * 32 + j * 16 + li;
                if (inner || (row < p.m && col < p.n)) {
                    uint16_t* q = C + static_cast<int64_t>(row) * p.c_sm + static_cast<int64_t>(col) * p.c_sn;
                    *q = finish(acc[i][j][v], p.alpha, p.beta, q);
                }
            }
}

__device__ inline int64_t decode4(const Axes4& ax, uint64_t idx) {
    int64_t off = 0;
#pragma unroll
    for (int d = 3; d >= 0; --d) {
        const uint64_t q = idx / ax.ext[d];
        off += static_cast<int64_t>(idx - q * ax.ext[d]) * ax.stride[d];
        idx = q;
    }
    return off;
}

// Groups that keep several strides after merging: one thread per output, K in order.
__global__ __launch_bounds__(256) void general_f16(GeneralHalfArgs p) {
    const uint64_t mn = static_cast<uint64_t>(p.m) * p.n;
    const uint64_t count = mn * p.batch;
    for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < count;
         e += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t bi = e / mn, rem = e - bi * mn;
        const uint64_t mi = rem / p.n, ni = rem - mi * p.n;
        const uint16_t* a = p.a + decode4(p.a_batch, bi) + decode4(p.a_m, mi);
        const uint16_t* b = p.b + decode4(p.b_batch, bi) + decode4(p.b_n, ni);
        double acc = 0.0;
        uint32_t dig[4] = {0, 0, 0, 0};
        int64_t oa = 0, ob = 0;
        for (uint32_t kk = 0; kk < p.k; ++kk) {
            acc = acc + h2d(a[oa]) * h2d(b[ob]);
#pragma unroll
            for (int d = 3; d >= 0; --d) {
                oa += p.a_k.stride[d];
                ob += p.b_k.stride[d];
                if (++dig[d] < p.a_k.ext[d]) break;
                oa -= static_cast<int64_t>(p.a_k.ext[d]) * p.a_k.stride[d];
                ob -= static_cast<int64_t>(p.b_k.ext[d]) * p.b_k.stride[d];
                dig[d] = 0;
            }
        }
        uint16_t* q = p.c + decode4(p.c_batch, bi) + decode4(p.c_m, mi) + decode4(p.c_n, ni);
        *q = finish(acc, p.alpha, p.beta, q);
    }
}

// C = 0 without reading C, or C = beta*C rounded once (the product is exact in f64).
__global__ __launch_bounds__(256) void fill_f16(FillHalfArgs p) {
    const uint64_t mn = static_cast<uint64_t>(p.m) * p.n;
    for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < p.count;
         e += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t bi = e / mn, rem = e - bi * mn;
        const uint64_t mi = rem / p.n, ni = rem - mi * p.n;
        uint16_t* q = p.c + decode4(p.c_batch, bi) + decode4(p.c_m, mi) + decode4(p.c_n, ni);
        *q = p.beta == 0.0f ? static_cast<uint16_t>(0)
                            : d2h(static_cast<double>(p.beta) * h2d(*q));
    }
}

uint32_t grid_for(uint64_t items) {
    const uint64_t g = (items + 255) / 256;
    return static_cast<uint32_t>(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

}  // namespace

uint64_t gemm_half_workgroups(uint32_t m, uint32_t n, uint32_t batch) {
    return static_cast<uint64_t>((m + HGEMM_BM - 1) / HGEMM_BM) * ((n + HGEMM_BN - 1) / HGEMM_BN) * batch;
}

void launch_gemm_half(Context* ctx, hipStream_t s, const GemmHalfArgs& args, int a_mode,
                      int b_mode) {
    const dim3 grid(static_cast<uint32_t>(gemm_half_workgroups(args.m, args.n, args.batch)));
#define LG_HGEMM_CASE(AMV, BMV)                                                       \
    if (a_mode == AMV && b_mode == BMV) {                                             \
        hipLaunchKernelGGL((gemm_f16_f64mfma<AMV, BMV>), grid, dim3(HT), 0, s, args); \
    } else
    LG_HGEMM_CASE(LOAD_K, LOAD_K)
    LG_HGEMM_CASE(LOAD_K, LOAD_MN)
    LG_HGEMM_CASE(LOAD_K, LOAD_S)
    LG_HGEMM_CASE(LOAD_MN, LOAD_K)
    LG_HGEMM_CASE(LOAD_MN, LOAD_MN)
    LG_HGEMM_CASE(LOAD_MN, LOAD_S)
    LG_HGEMM_CASE(LOAD_S, LOAD_K)
    LG_HGEMM_CASE(LOAD_S, LOAD_MN)
    LG_HGEMM_CASE(LOAD_S, LOAD_S) { fail_invalid("unknown operand load mode"); }
#undef LG_HGEMM_CASE
    check_hip(hipGetLastError(), "gemm_f16_f64mfma");
    note_launch(ctx, "gemm_f16_f64mfma");
}

void launch_general_half(Context* ctx, hipStream_t s, const GeneralHalfArgs& args) {
    const uint64_t count = static_cast<uint64_t>(args.m) * args.n * args.batch;
    hipLaunchKernelGGL(general_f16, dim3(grid_for(count)), dim3(256), 0, s, args);
    check_hip(hipGetLastError(), "general_f16");
    note_launch(ctx, "general_f16");
}

void launch_fill_half(Context* ctx, hipStream_t s, const FillHalfArgs& args) {
    hipLaunchKernelGGL(fill_f16, dim3(grid_for(args.count)), dim3(256), 0, s, args);
    check_hip(hipGetLastError(), "fill_f16");
    note_launch(ctx, args.beta == 0.0f ? "zero_f16" : "scale_f16");
}

}  // namespace lg
