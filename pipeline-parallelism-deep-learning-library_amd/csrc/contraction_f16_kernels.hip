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
// K advances 16 at a time: the slice is loaded as halves (all 8 loads in flight when the tile
// and slice lie inside the operands), widened to f64 and staged in LDS.
constexpr int HT = 256;
constexpr int APITCH = HGEMM_BK + 1;  // doubles; odd pitch spreads the k-column reads
constexpr int BPITCH = HGEMM_BN + 1;

__global__ __launch_bounds__(HT) void gemm_f16_f64mfma(GemmHalfArgs p) {
    __shared__ double As[HGEMM_BM * APITCH];
    __shared__ double Bs[HGEMM_BK * BPITCH];
    uint32_t plane, tm, tn;
    gemm_detail::decode_tile(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, &plane, &tm, &tn);
    const uint32_t m0 = tm * HGEMM_BM, n0 = tn * HGEMM_BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int li = lane & 15, lk = lane >> 4;
    const uint16_t* A = p.a + static_cast<int64_t>(plane) * p.a_sb;
    const uint16_t* B = p.b + static_cast<int64_t>(plane) * p.b_sb;
    uint16_t* C = p.c + static_cast<int64_t>(plane) * p.c_sb;
    const bool inner = m0 + HGEMM_BM <= p.m && n0 + HGEMM_BN <= p.n;

    f64x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};

    constexpr int LOADS = HGEMM_BM * HGEMM_BK / HT;  // 4 halves of A and 4 of B per thread
    for (uint32_t k0 = 0; k0 < p.k; k0 += HGEMM_BK) {
        uint16_t ra[LOADS], rb[LOADS];
        if (inner && k0 + HGEMM_BK <= p.k) {
#pragma unroll
            for (int it = 0; it < LOADS; ++it) {
                const int idx = it * HT + tid;
                const int row = idx / HGEMM_BK, kk = idx % HGEMM_BK;
                ra[it] = A[static_cast<int64_t>(m0 + row) * p.a_sm + static_cast<int64_t>(k0 + kk) * p.a_sk];
                const int kb = idx / HGEMM_BN, col = idx % HGEMM_BN;
                rb[it] = B[static_cast<int64_t>(k0 + kb) * p.b_sk + static_cast<int64_t>(n0 + col) * p.b_sn];
            }
        } else {
#pragma unroll
            for (int it = 0; it < LOADS; ++it) {
                const int idx = it * HT + tid;
                const int row = idx / HGEMM_BK, kk = idx % HGEMM_BK;
                const bool ia = m0 + row < p.m && k0 + kk < p.k;
                ra[it] = ia ? A[static_cast<int64_t>(m0 + row) * p.a_sm + static_cast<int64_t>(k0 + kk) * p.a_sk]
                            : static_cast<uint16_t>(0);
                const int kb = idx / HGEMM_BN, col = idx % HGEMM_BN;
                const bool ib = k0 + kb < p.k && n0 + col < p.n;
                rb[it] = ib ? B[static_cast<int64_t>(k0 + kb) * p.b_sk + static_cast<int64_t>(n0 + col) * p.b_sn]
                            : static_cast<uint16_t>(0);
            }
        }
#pragma unroll
        for (int it = 0; it < LOADS; ++it) {
            const int idx = it * HT + tid;
            As[(idx / HGEMM_BK) * APITCH + idx % HGEMM_BK] = h2d(ra[it]);
            Bs[(idx / HGEMM_BN) * BPITCH + idx % HGEMM_BN] = h2d(rb[it]);
        }
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < HGEMM_BK / 4; ++ks) {
            double av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) av[i] = As[(wm * 32 + i * 16 + li) * APITCH + ks * 4 + lk];
#pragma unroll
            for (int j = 0; j < 2; ++j) bv[j] = Bs[(ks * 4 + lk) * BPITCH + wn * 32 + j * 16 + li];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[i], bv[j], acc[i][j], 0, 0, 0);
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
        *q = p.beta == 0.0f ? static_cast<uint16_t>(0) : d2h(static_cast<double>(p.beta) * h2d(*q));
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

void launch_gemm_half(Context* ctx, hipStream_t s, const GemmHalfArgs& args) {
    const uint64_t g = gemm_half_workgroups(args.m, args.n, args.batch);
    hipLaunchKernelGGL(gemm_f16_f64mfma, dim3(static_cast<uint32_t>(g)), dim3(HT), 0, s, args);
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
