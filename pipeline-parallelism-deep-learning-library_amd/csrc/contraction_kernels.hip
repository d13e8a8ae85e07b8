// gfx950 contraction kernels: the fp32 MFMA GEMM (gemm_kernel.h) instantiated at the
// library's pipeline shape, the split-K reduction (fixed order over splits, so results are
// bit-reproducible), the mixed-radix general fallback, and the C = 0 / C = beta*C fill.
// Every product is formed as (alpha * a) * b, the grouping of the reference's sequential loop.
// Everything is compiled with -ffp-contract=off: products and sums round separately.
#include <hip/hip_runtime.h>

#include "gemm_kernel.h"
#include "lg_internal.h"

namespace lg {
namespace {

using gemm_detail::gemm_f32_mfma;
using gemm_detail::gemm_f32_small;
using gemm_detail::SMALL_WAVES;

// Split-K second pass. Partials are [batch][splits][m][n], dense. A workgroup owns 64 runs
// of V consecutive outputs; its four waves each sum a fixed quarter of the splits in
// ascending order (8 loads in flight), the quarters are added in order 0+1+2+3, and beta*C
// is added once (alpha is already inside the partials). The order depends only on the split
// count, so results are
// bit-reproducible from run to run. V = 4 (128-bit loads) whenever n is a multiple of 4.
constexpr int RED_LANES = 64;
constexpr int RED_SLICES = 4;

template <int V>
__global__ __launch_bounds__(RED_LANES * RED_SLICES) void reduce_f32(ReduceArgs p) {
    typedef float vec __attribute__((ext_vector_type(4)));
    __shared__ vec part[RED_SLICES][RED_LANES];
    const int lane = threadIdx.x % RED_LANES, q = threadIdx.x / RED_LANES;
    const uint64_t mn = static_cast<uint64_t>(p.m) * p.n;
    const uint64_t count = mn * p.batch;
    const uint32_t s0 = static_cast<uint32_t>(static_cast<uint64_t>(q) * p.splits / RED_SLICES);
    const uint32_t s1 = static_cast<uint32_t>(static_cast<uint64_t>(q + 1) * p.splits / RED_SLICES);
    const uint64_t step = static_cast<uint64_t>(gridDim.x) * RED_LANES * V;
    for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * RED_LANES * V; base < count; base += step) {
        const uint64_t e = base + static_cast<uint64_t>(lane) * V;
        vec acc = {0.0f, 0.0f, 0.0f, 0.0f};
        uint64_t bi = 0, rem = 0;
        if (e < count) {
            bi = e / mn;
            rem = e - bi * mn;
            const float* src = p.partial + bi * p.splits * mn + rem;
            uint32_t s = s0;
            for (; s + 8 <= s1; s += 8) {
                vec x[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    if constexpr (V == 4) {
                        x[u] = *reinterpret_cast<const vec*>(src + (s + u) * mn);
                    } else {
                        x[u][0] = src[(s + u) * mn];
                    }
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) acc = acc + x[u];
            }
            for (; s < s1; ++s) {
                if constexpr (V == 4) {
                    acc = acc + *reinterpret_cast<const vec*>(src + s * mn);
                } else {
                    acc[0] = acc[0] + src[s * mn];
                }
            }
        }
        part[q][lane] = acc;
        __syncthreads();
        if (q == 0 && e < count) {
            vec t = part[0][lane];
#pragma unroll
            for (int k = 1; k < RED_SLICES; ++k) t = t + part[k][lane];
#pragma unroll
            for (int v = 0; v < V; ++v) {
                const uint64_t r = rem + v;
                const uint32_t row = static_cast<uint32_t>(r / p.n), col = static_cast<uint32_t>(r % p.n);
                float* out = p.c + static_cast<int64_t>(bi) * p.c_sb + static_cast<int64_t>(row) * p.c_sm +
                             static_cast<int64_t>(col) * p.c_sn;
                float val = t[v];
                if (p.beta != 0.0f) val = p.beta * *out + val;
                *out = val;
            }
        }
        __syncthreads();
    }
}

// Mixed-radix offset of index `idx` within a right-aligned 4-axis group.
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

// Fallback for groups that keep more than one stride after merging, and for non-finite alpha:
// one thread per output, acc = (beta == 0 ? 0 : beta*C), then acc += (alpha*a)*b in k order
// with an odometer over the (up to four) K axes of A and B -- the reference's sequential
// loop, so this kernel's results are bit-identical to it.
__global__ __launch_bounds__(256) void general_f32(GeneralArgs p) {
    const uint64_t mn = static_cast<uint64_t>(p.m) * p.n;
    const uint64_t count = mn * p.batch;
    for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < count;
         e += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t bi = e / mn, rem = e - bi * mn;
        const uint64_t mi = rem / p.n, ni = rem - mi * p.n;
        const float* a = p.a + decode4(p.a_batch, bi) + decode4(p.a_m, mi);
        const float* b = p.b + decode4(p.b_batch, bi) + decode4(p.b_n, ni);
        float* q = p.c + decode4(p.c_batch, bi) + decode4(p.c_m, mi) + decode4(p.c_n, ni);
        float acc = p.beta == 0.0f ? 0.0f : p.beta * *q;
        uint32_t dig[4] = {0, 0, 0, 0};
        int64_t oa = 0, ob = 0;
        for (uint32_t kk = 0; kk < p.k; ++kk) {
            acc = acc + (p.alpha * a[oa]) * b[ob];
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
        *q = acc;
    }
}

// C = 0 (beta == 0, C never read) or C = beta * C, one rounding.
__global__ __launch_bounds__(256) void fill_f32(FillArgs p) {
    const uint64_t mn = static_cast<uint64_t>(p.m) * p.n;
    for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < p.count;
         e += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t bi = e / mn, rem = e - bi * mn;
        const uint64_t mi = rem / p.n, ni = rem - mi * p.n;
        float* q = p.c + decode4(p.c_batch, bi) + decode4(p.c_m, mi) + decode4(p.c_n, ni);
        *q = p.beta == 0.0f ? 0.0f : p.beta * *q;
    }
}

uint32_t grid_for(uint64_t count) {
    const uint64_t g = (count + 255) / 256;
    return static_cast<uint32_t>(g < 65536 ? (g == 0 ? 1 : g) : 65536);
}

void check_launch(const char* what) { check_hip(hipGetLastError(), what); }

template <int AM, int BMD>
void launch_gemm_t(hipStream_t s, const GemmArgs& a, uint32_t groups) {
    if (a.tile == GEMM_TINY_TILE) {
        hipLaunchKernelGGL((gemm_f32_small<AM, BMD, SMALL_WAVES>), dim3(groups), dim3(64 * SMALL_WAVES), 0,
                           s, a);
    } else if (a.tile == GEMM_SMALL_TILE) {
        hipLaunchKernelGGL((gemm_f32_mfma<AM, BMD, GEMM_BK, 1, 1>), dim3(groups),
                           dim3(GEMM_THREADS), 0, s, a);
    } else {
        // A read along M (a transposed A) takes the two-ahead pipeline.
        constexpr bool ahead = AM == LOAD_MN && BMD != LOAD_S;
        hipLaunchKernelGGL((gemm_f32_mfma<AM, BMD, GEMM_BK, 2, 2, ahead>), dim3(groups),
                           dim3(GEMM_THREADS), 0, s, a);
    }
}

}  // namespace

uint64_t gemm_workgroups(uint32_t m, uint32_t n, uint32_t batch, uint32_t splits, uint32_t tile) {
    const uint64_t tm = (m + tile - 1) / tile, tn = (n + tile - 1) / tile;
    return tm * tn * batch * splits;
}

void launch_gemm(Context* ctx, hipStream_t s, const GemmArgs& args, int a_mode, int b_mode) {
    const uint32_t groups =
        static_cast<uint32_t>(gemm_workgroups(args.m, args.n, args.batch, args.splits, args.tile));
    static const char* const names[3][3] = {
        {"gemm_f32_mfma<K,K>", "gemm_f32_mfma<K,MN>", "gemm_f32_mfma<K,S>"},
        {"gemm_f32_mfma<MN,K>", "gemm_f32_mfma<MN,MN>", "gemm_f32_mfma<MN,S>"},
        {"gemm_f32_mfma<S,K>", "gemm_f32_mfma<S,MN>", "gemm_f32_mfma<S,S>"}};
#define LG_GEMM_CASE(AMV, BMV)                       \
    if (a_mode == AMV && b_mode == BMV) {            \
        launch_gemm_t<AMV, BMV>(s, args, groups);    \
    } else
    LG_GEMM_CASE(LOAD_K, LOAD_K)
    LG_GEMM_CASE(LOAD_K, LOAD_MN)
    LG_GEMM_CASE(LOAD_K, LOAD_S)
    LG_GEMM_CASE(LOAD_MN, LOAD_K)
    LG_GEMM_CASE(LOAD_MN, LOAD_MN)
    LG_GEMM_CASE(LOAD_MN, LOAD_S)
    LG_GEMM_CASE(LOAD_S, LOAD_K)
    LG_GEMM_CASE(LOAD_S, LOAD_MN)
    LG_GEMM_CASE(LOAD_S, LOAD_S) { fail_invalid("unknown operand load mode"); }
#undef LG_GEMM_CASE
    check_launch("gemm_f32_mfma launch");
    note_launch(ctx, names[a_mode][b_mode]);
}

void launch_reduce(Context* ctx, hipStream_t s, const ReduceArgs& args) {
    const uint64_t count = static_cast<uint64_t>(args.m) * args.n * args.batch;
    const int v = args.n % 4 == 0 ? 4 : 1;
    const uint64_t per = static_cast<uint64_t>(RED_LANES) * v;
    const uint64_t g = (count + per - 1) / per;
    const dim3 grid(static_cast<uint32_t>(g < 65536 ? (g ? g : 1) : 65536));
    if (v == 4) {
        hipLaunchKernelGGL(reduce_f32<4>, grid, dim3(RED_LANES * RED_SLICES), 0, s, args);
    } else {
        hipLaunchKernelGGL(reduce_f32<1>, grid, dim3(RED_LANES * RED_SLICES), 0, s, args);
    }
    check_launch("reduce_f32 launch");
    note_launch(ctx, "reduce_f32");
}

void launch_general(Context* ctx, hipStream_t s, const GeneralArgs& args) {
    const uint64_t count = static_cast<uint64_t>(args.m) * args.n * args.batch;
    hipLaunchKernelGGL(general_f32, dim3(grid_for(count)), dim3(256), 0, s, args);
    check_launch("general_f32 launch");
    note_launch(ctx, "general_f32");
}

void launch_fill(Context* ctx, hipStream_t s, const FillArgs& args) {
    hipLaunchKernelGGL(fill_f32, dim3(grid_for(args.count)), dim3(256), 0, s, args);
    check_launch("fill_f32 launch");
    note_launch(ctx, args.beta == 0.0f ? "zero_f32" : "scale_f32");
}

}  // namespace lg
