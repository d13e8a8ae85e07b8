// gfx950 contraction kernels: the fp32 MFMA GEMM kernels (gemm_kernel.h) instantiated at the
// library's pipeline shapes, the split-K reduction (fixed order over splits, so results are
// bit-reproducible), dot products, the mixed-radix general fallback, and the C = 0 /
// C = beta*C fill.
// Every product is formed as (alpha * a) * b, the grouping of the reference's sequential loop.
// Everything is compiled with -ffp-contract=off: products and sums round separately.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "gemm_dlds.h"
#include "gemm_pipe.h"
#include "gemm_kernel.h"
#include "lg_internal.h"

namespace lg {
namespace {

using gemm_detail::gemm_f32_dl;
using gemm_detail::gemm_f32_mfma;
using gemm_detail::gemm_f32_kw;
using gemm_detail::gemm_f32_pl;
using gemm_detail::gemm_f32_pl256;
using gemm_detail::gemm_f32_pl2x;
using gemm_detail::gemm_f32_sk;
using gemm_detail::gemm_f32_small;
using gemm_detail::gemm_f32_wave;
using gemm_detail::SMALL_WAVES;
using gemm_detail::WAVE_TILES;

// Split-K second pass. Partials are [batch][splits][m][n], dense. A workgroup owns 64 runs
// of V consecutive outputs; its SL waves each sum a fixed 1/SL of the splits in ascending
// order (8 loads in flight), the slices are added in order 0+1+...+(SL-1), and beta*C is added
// once (alpha is already inside the partials). The order depends only on the split count and
// SL (the planner picks SL from the shape), so results are bit-reproducible from run to run.
// V = 4 (128-bit loads) whenever n is a multiple of 4. SL = 16 serves few outputs with many
// splits (the small-output split path), where four waves per output run would leave the
// loads of one output's splits mostly in series.
constexpr int RED_LANES = 64;

template <int V, int SL>
__global__ __launch_bounds__(RED_LANES * SL) void reduce_f32(ReduceArgs p) {
    typedef float vec __attribute__((ext_vector_type(4)));
    __shared__ vec part[SL][RED_LANES];
    const int lane = threadIdx.x % RED_LANES, q = threadIdx.x / RED_LANES;
    const uint64_t mn = static_cast<uint64_t>(p.m) * p.n;
    const uint64_t count = mn * p.batch;
    const uint32_t s0 = static_cast<uint32_t>(static_cast<uint64_t>(q) * p.splits / SL);
    const uint32_t s1 = static_cast<uint32_t>(static_cast<uint64_t>(q + 1) * p.splits / SL);
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
            for (int k = 1; k < SL; ++k) t = t + part[k][lane];
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

// Dot products, C[b] = beta*C[b] + sum_k (alpha*a[b][k])*b[b][k] (M = N = 1, memory-bound:
// 8 bytes per multiply-add, so the VALU rather than a mostly-padded MFMA tile). Workgroup
// (b, s) takes K chunk s of product b; thread t sums the elements t, t + 256, ... of the chunk
// (128-bit runs of 4 when VEC, DOT_UNROLL runs' loads issued before their products) in index
// order, and the workgroup adds the 256 thread sums in a fixed tree. With one split that is
// the result; otherwise it is partial[b][s], and dot_finish (the next launch on the stream, so
// every partial is complete and visible) adds product b's partials: thread t sums splits
// t, t + 256, ... in order, then the same tree. No workgroup waits on another and no device-
// scope fence runs per workgroup. The order depends only on K, the chunk and the split count.
constexpr int DOT_UNROLL = 8;

__device__ inline float dot_tree(float* red, float v) {
    red[threadIdx.x] = v;
    __syncthreads();
#pragma unroll
    for (int w = DOT_THREADS / 2; w > 0; w /= 2) {
        if (static_cast<int>(threadIdx.x) < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    return red[0];
}

template <bool VEC>
__global__ __launch_bounds__(DOT_THREADS) void dot_f32(DotArgs p) {
    typedef float vec __attribute__((ext_vector_type(4)));
    __shared__ float red[DOT_THREADS];
    const uint32_t bi = blockIdx.x / p.splits, split = blockIdx.x - bi * p.splits;
    const uint32_t kb = split * p.k_chunk;
    const uint32_t klen = min(p.k - kb, p.k_chunk);
    const float* a = p.a + static_cast<int64_t>(bi) * p.a_sb + static_cast<int64_t>(kb) * p.a_sk;
    const float* b = p.b + static_cast<int64_t>(bi) * p.b_sb + static_cast<int64_t>(kb) * p.b_sk;
    const float alpha_a = p.scale_b ? 1.0f : p.alpha, alpha_b = p.scale_b ? p.alpha : 1.0f;
    float acc = 0.0f;
    auto add = [&](float x, float y) {
        if (alpha_a != 1.0f) x = alpha_a * x;
        if (alpha_b != 1.0f) y = alpha_b * y;
        acc = acc + x * y;
    };
    uint32_t i = threadIdx.x;
    if constexpr (VEC) {
        // klen is a multiple of 4 except in the last chunk, whose tail the scalar step takes.
        const vec* av = reinterpret_cast<const vec*>(a);
        const vec* bv = reinterpret_cast<const vec*>(b);
        const uint32_t nv = klen / 4;
        for (; i + (DOT_UNROLL - 1) * DOT_THREADS < nv; i += DOT_UNROLL * DOT_THREADS) {
            vec x[DOT_UNROLL], y[DOT_UNROLL];
#pragma unroll
            for (int u = 0; u < DOT_UNROLL; ++u) {
                x[u] = av[i + u * DOT_THREADS];
                y[u] = bv[i + u * DOT_THREADS];
            }
#pragma unroll
            for (int u = 0; u < DOT_UNROLL; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) add(x[u][e], y[u][e]);
        }
        for (; i < nv; i += DOT_THREADS) {
            const vec x = av[i], y = bv[i];
#pragma unroll
            for (int e = 0; e < 4; ++e) add(x[e], y[e]);
        }
        // The chunk's last klen % 4 elements go to the threads after the vector runs.
        i = nv * 4 + threadIdx.x;
        if (i < klen) add(a[i], b[i]);
    } else {
        for (; i < klen; i += DOT_THREADS) {
            add(a[static_cast<int64_t>(i) * p.a_sk], b[static_cast<int64_t>(i) * p.b_sk]);
        }
    }
    const float sum = dot_tree(red, acc);
    if (threadIdx.x != 0) return;
    if (p.splits == 1) {
        float* c = p.c + static_cast<int64_t>(bi) * p.c_sb;
        *c = p.beta != 0.0f ? p.beta * *c + sum : sum;
    } else {
        p.partial[blockIdx.x] = sum;
    }
}

// Products with K <= OUTER_MAX_K (rank-1 and other low-rank updates): memory-bound on C, so
// the VALU does them in crates/cpu's own order, acc = beta == 0 ? +0 : beta*C, then
// acc = acc + (alpha*a)*b for k in order, one rounding per operation: the reference's bits.
// Thread t owns four consecutive columns of one row (128-bit loads of B and non-temporal
// 128-bit stores of C when VB / VC); a grid-stride loop of at most OUTER_MAX_GROUPS workgroups
// covers batch * m * ceil(n / 4) such quads (measured on rank-1 4096^2: 17.1 -> 15.8 us
// against one quad per thread with ordinary stores; 4096 workgroups, four quads a thread,
// 12.6-12.8 us back to back against 13.2-13.4 for 2048 and 14.8-16.5 for 16384).
constexpr uint32_t OUTER_THREADS = 256;
constexpr uint32_t OUTER_MAX_GROUPS = 4096;

template <bool VB, bool VC>
__global__ __launch_bounds__(OUTER_THREADS) void outer_f32(GemmArgs p) {
    typedef float vec __attribute__((ext_vector_type(4)));
    const uint32_t nq = (p.n + 3) / 4;
    const uint64_t total = static_cast<uint64_t>(p.batch) * p.m * nq;
    const float alpha_a = p.scale_b ? 1.0f : p.alpha, alpha_b = p.scale_b ? p.alpha : 1.0f;
    // Index arithmetic in 32 bits when every output quad's index fits (the 64-bit divisions
    // otherwise cost more VALU time than the thread's 16 bytes of stores).
    const bool narrow = total <= 0xffffffffull;
    for (uint64_t t = static_cast<uint64_t>(blockIdx.x) * OUTER_THREADS + threadIdx.x; t < total;
         t += static_cast<uint64_t>(gridDim.x) * OUTER_THREADS) {
        uint32_t j0, bi, i;
        if (narrow) {
            const uint32_t t32 = static_cast<uint32_t>(t), row32 = t32 / nq;
            j0 = (t32 - row32 * nq) * 4;
            bi = p.batch == 1 ? 0u : row32 / p.m;
            i = row32 - bi * p.m;
        } else {
            const uint64_t row = t / nq;
            j0 = static_cast<uint32_t>(t - row * nq) * 4;
            bi = static_cast<uint32_t>(row / p.m);
            i = static_cast<uint32_t>(row - static_cast<uint64_t>(bi) * p.m);
        }
        const uint32_t cnt = min(4u, p.n - j0);
        const float* a = p.a + static_cast<int64_t>(bi) * p.a_sb + static_cast<int64_t>(i) * p.a_sm;
        const float* b = p.b + static_cast<int64_t>(bi) * p.b_sb + static_cast<int64_t>(j0) * p.b_sn;
        float* c = p.c + static_cast<int64_t>(bi) * p.c_sb + static_cast<int64_t>(i) * p.c_sm +
                   static_cast<int64_t>(j0) * p.c_sn;
        vec acc = {0.0f, 0.0f, 0.0f, 0.0f};
        if (p.beta != 0.0f) {
            if constexpr (VC) {
                acc = p.beta * *reinterpret_cast<const vec*>(c);
            } else {
                for (uint32_t e = 0; e < cnt; ++e) acc[e] = p.beta * c[static_cast<int64_t>(e) * p.c_sn];
            }
        }
        for (uint32_t k = 0; k < p.k; ++k) {
            float x = a[static_cast<int64_t>(k) * p.a_sk];
            vec y;
            if constexpr (VB) {
                y = *reinterpret_cast<const vec*>(b + static_cast<int64_t>(k) * p.b_sk);
            } else {
#pragma unroll
                for (uint32_t e = 0; e < 4; ++e) {
                    y[e] = e < cnt ? b[static_cast<int64_t>(k) * p.b_sk + static_cast<int64_t>(e) * p.b_sn] : 0.0f;
                }
            }
            if (alpha_a != 1.0f) x = alpha_a * x;
            if (alpha_b != 1.0f) y = alpha_b * y;
            acc = acc + x * y;
        }
        if constexpr (VC) {
            __builtin_nontemporal_store(acc, reinterpret_cast<vec*>(c));
        } else {
            for (uint32_t e = 0; e < cnt; ++e) c[static_cast<int64_t>(e) * p.c_sn] = acc[e];
        }
    }
}

// Second launch of a split dot: workgroup b adds product b's partials in split order.
__global__ __launch_bounds__(DOT_THREADS) void dot_finish_f32(DotArgs p) {
    __shared__ float red[DOT_THREADS];
    const uint32_t bi = blockIdx.x;
    const float* part = p.partial + static_cast<uint64_t>(bi) * p.splits;
    float t = 0.0f;
    for (uint32_t g = threadIdx.x; g < p.splits; g += DOT_THREADS) t = t + part[g];
    const float total = dot_tree(red, t);
    if (threadIdx.x == 0) {
        float* c = p.c + static_cast<int64_t>(bi) * p.c_sb;
        *c = p.beta != 0.0f ? p.beta * *c + total : total;
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
    if (a.kernel == KERN_OUTER) {
        if (a.vec_b && a.vec_c) {
            hipLaunchKernelGGL((outer_f32<true, true>), dim3(groups), dim3(OUTER_THREADS), 0, s, a);
        } else if (a.vec_c) {
            hipLaunchKernelGGL((outer_f32<false, true>), dim3(groups), dim3(OUTER_THREADS), 0, s, a);
        } else if (a.vec_b) {
            hipLaunchKernelGGL((outer_f32<true, false>), dim3(groups), dim3(OUTER_THREADS), 0, s, a);
        } else {
            hipLaunchKernelGGL((outer_f32<false, false>), dim3(groups), dim3(OUTER_THREADS), 0, s, a);
        }
    } else if (a.kernel == KERN_SK) {
        if constexpr (AM != LOAD_S && BMD != LOAD_S) {
            const uint64_t tiles = static_cast<uint64_t>(a.tiles_m) * a.tiles_n * a.batch;
            if (a.tile != GEMM_BM || a.tile_n != GEMM_BN || a.m % GEMM_BM != 0 || a.n % GEMM_BN != 0 ||
                a.slice_k != 32 || a.k % (PIPE_STAGES * 32) != 0 || a.splits != 1 || tiles < groups ||
                groups != SK_RANGES || a.partial == nullptr || a.counters == nullptr) {
                fail_invalid("the stream-K GEMM needs full 128x128 tiles, at least one per range, "
                             "K in whole steps and its scratch");
            }
            hipLaunchKernelGGL((gemm_f32_sk<AM, BMD, 32, PIPE_STAGES>), dim3(groups), dim3(256), 0, s, a);
        } else {
            fail_invalid("the stream-K GEMM needs a unit-stride axis in both operands");
        }
    } else if (a.kernel == KERN_PIPE) {
        if constexpr (AM != LOAD_S && BMD != LOAD_S) {
            const uint32_t last = a.k - (a.splits - 1) * a.k_chunk;
            if (a.tile == GEMM_SMALL_TILE) {
                if (a.tile_n != GEMM_SMALL_TILE || a.m % GEMM_SMALL_TILE != 0 || a.n % GEMM_SMALL_TILE != 0 ||
                    a.slice_k != KW_BK || a.k_chunk % KW_STEP != 0 || last % KW_STEP != 0) {
                    fail_invalid("the K-split GEMM needs full 64x64 tiles and K chunks in whole steps");
                }
                hipLaunchKernelGGL((gemm_f32_kw<AM, BMD, KW_BK, KW_STAGES>), dim3(groups), dim3(256), 0, s, a);
                return;
            }
            const uint32_t step = PIPE_STAGES * a.slice_k;
            if (a.tile == PIPE_TALL_M && a.tile_n == PIPE_WIDE_N) {
                if constexpr (AM == LOAD_K && BMD != LOAD_S) {
                    if (a.m % PIPE_TALL_M != 0 || a.n % PIPE_WIDE_N != 0 || a.slice_k != 16 || a.splits != 1 ||
                        a.k % step != 0) {
                        fail_invalid("the 256x256 pipelined GEMM needs full tiles and K in whole steps");
                    }
                    hipLaunchKernelGGL((gemm_f32_pl2x<AM, BMD, 16, PIPE_STAGES>), dim3(groups), dim3(512), 0, s, a);
                    return;
                } else {
                    fail_invalid("the 256x256 pipelined GEMM needs A contiguous along K");
                }
            }
            if (a.tile == PIPE_TALL_M) {
                if (a.tile_n != GEMM_BN || a.m % PIPE_TALL_M != 0 || a.n % GEMM_BN != 0 || a.slice_k != 16 ||
                    a.splits != 1 || a.k % step != 0) {
                    fail_invalid("the 256x128 pipelined GEMM needs full tiles and K in whole steps");
                }
                hipLaunchKernelGGL((gemm_f32_pl256<AM, BMD, 16, PIPE_STAGES>), dim3(groups), dim3(512), 0, s, a);
                return;
            }
            if (a.tile_n == PIPE_NARROW_N) {
                if (a.tile != GEMM_BM || a.m % GEMM_BM != 0 || a.n % PIPE_NARROW_N != 0 || a.slice_k != 16 ||
                    a.k_chunk % step != 0 || last % step != 0) {
                    fail_invalid("the pipelined GEMM needs full 128x64 tiles and K chunks in whole steps");
                }
                hipLaunchKernelGGL((gemm_f32_pl<AM, BMD, 16, PIPE_STAGES, 1>), dim3(groups), dim3(256), 0, s, a);
                return;
            }
            if (a.tile != GEMM_BM || a.tile_n != GEMM_BN || a.m % GEMM_BM != 0 || a.n % GEMM_BN != 0 ||
                (a.slice_k != 16 && a.slice_k != 32) || a.k_chunk % step != 0 || last % step != 0) {
                fail_invalid("the pipelined GEMM needs full 128x128 tiles and K chunks in whole steps");
            }
            if (a.slice_k == 32) {
                hipLaunchKernelGGL((gemm_f32_pl<AM, BMD, 32, PIPE_STAGES>), dim3(groups), dim3(256), 0, s, a);
            } else {
                hipLaunchKernelGGL((gemm_f32_pl<AM, BMD, 16, PIPE_STAGES>), dim3(groups), dim3(256), 0, s, a);
            }
        } else {
            fail_invalid("the pipelined GEMM needs a unit-stride axis in both operands");
        }
    } else if (a.kernel == KERN_DIRECT) {
        if constexpr (AM != LOAD_S && BMD != LOAD_S) {
            if (a.tile == GEMM_TINY_TILE) {
                hipLaunchKernelGGL((gemm_f32_dl<AM, BMD, 3, 32, 1, 1, 1, 1>), dim3(groups), dim3(64), 0, s, a);
            } else if (a.tile == GEMM_SMALL_TILE) {
                if (a.kgroups != 4) fail_invalid("64x64 direct-load tiles run four wave groups");
                hipLaunchKernelGGL((gemm_f32_dl<AM, BMD, 2, 32, 2, 2, 1, 1, 4>), dim3(groups), dim3(1024), 0, s, a);
            } else if (a.kgroups == 2) {
                hipLaunchKernelGGL((gemm_f32_dl<AM, BMD, 2, 32, 2, 2, 2, 2, 2>), dim3(groups), dim3(512), 0, s, a);
            } else if (a.tile_n == GEMM_WIDE_N) {
                hipLaunchKernelGGL((gemm_f32_dl<AM, BMD, 3, 16, 4>), dim3(groups), dim3(512), 0, s, a);
            } else {
                hipLaunchKernelGGL((gemm_f32_dl<AM, BMD, 3, 16, 2>), dim3(groups), dim3(256), 0, s, a);
            }
        } else {
            fail_invalid("direct-load GEMM needs a unit-stride axis in both operands");
        }
    } else if (a.kernel == KERN_WAVE) {
        hipLaunchKernelGGL((gemm_f32_wave<AM, BMD>), dim3(groups), dim3(64 * WAVE_TILES), 0, s, a);
    } else if (a.kernel == KERN_SMALL) {
        hipLaunchKernelGGL((gemm_f32_small<AM, BMD, SMALL_WAVES>), dim3(groups), dim3(64 * SMALL_WAVES), 0,
                           s, a);
    } else if (a.tile == GEMM_SMALL_TILE) {
        hipLaunchKernelGGL((gemm_f32_mfma<AM, BMD, GEMM_BK, 1, 1>), dim3(groups),
                           dim3(GEMM_THREADS), 0, s, a);
    } else {
        hipLaunchKernelGGL((gemm_f32_mfma<AM, BMD, GEMM_BK, 2, 2>), dim3(groups),
                           dim3(GEMM_THREADS), 0, s, a);
    }
}

}  // namespace

uint64_t gemm_workgroups(const GemmArgs& a) {
    if (a.kernel == KERN_SK) return SK_RANGES;
    if (a.kernel == KERN_OUTER) {
        const uint64_t quads = static_cast<uint64_t>(a.batch) * a.m * ((a.n + 3) / 4);
        return std::max<uint64_t>(1, std::min<uint64_t>((quads + OUTER_THREADS - 1) / OUTER_THREADS,
                                                         OUTER_MAX_GROUPS));
    }
    const uint64_t tiles = static_cast<uint64_t>((a.m + a.tile - 1) / a.tile) *
                           ((a.n + a.tile_n - 1) / a.tile_n) * a.batch * a.splits;
    return a.kernel == KERN_WAVE ? (tiles + WAVE_TILES - 1) / WAVE_TILES : tiles;
}

void launch_gemm(Context* ctx, hipStream_t s, const GemmArgs& args, int a_mode, int b_mode) {
    const uint32_t groups = static_cast<uint32_t>(gemm_workgroups(args));
    static const char* const names[6][3][3] = {
        {{"gemm_f32_mfma<K,K>", "gemm_f32_mfma<K,MN>", "gemm_f32_mfma<K,S>"},
         {"gemm_f32_mfma<MN,K>", "gemm_f32_mfma<MN,MN>", "gemm_f32_mfma<MN,S>"},
         {"gemm_f32_mfma<S,K>", "gemm_f32_mfma<S,MN>", "gemm_f32_mfma<S,S>"}},
        {{"gemm_f32_small<K,K>", "gemm_f32_small<K,MN>", "gemm_f32_small<K,S>"},
         {"gemm_f32_small<MN,K>", "gemm_f32_small<MN,MN>", "gemm_f32_small<MN,S>"},
         {"gemm_f32_small<S,K>", "gemm_f32_small<S,MN>", "gemm_f32_small<S,S>"}},
        {{"gemm_f32_wave<K,K>", "gemm_f32_wave<K,MN>", "gemm_f32_wave<K,S>"},
         {"gemm_f32_wave<MN,K>", "gemm_f32_wave<MN,MN>", "gemm_f32_wave<MN,S>"},
         {"gemm_f32_wave<S,K>", "gemm_f32_wave<S,MN>", "gemm_f32_wave<S,S>"}},
        {{"gemm_f32_outer", "gemm_f32_outer", "gemm_f32_outer"},
         {"gemm_f32_outer", "gemm_f32_outer", "gemm_f32_outer"},
         {"gemm_f32_outer", "gemm_f32_outer", "gemm_f32_outer"}},
        {{"gemm_f32_dl<K,K>", "gemm_f32_dl<K,MN>", "gemm_f32_dl<K,S>"},
         {"gemm_f32_dl<MN,K>", "gemm_f32_dl<MN,MN>", "gemm_f32_dl<MN,S>"},
         {"gemm_f32_dl<S,K>", "gemm_f32_dl<S,MN>", "gemm_f32_dl<S,S>"}},
        {{"gemm_f32_pl<K,K>", "gemm_f32_pl<K,MN>", "gemm_f32_pl<K,S>"},
         {"gemm_f32_pl<MN,K>", "gemm_f32_pl<MN,MN>", "gemm_f32_pl<MN,S>"},
         {"gemm_f32_pl<S,K>", "gemm_f32_pl<S,MN>", "gemm_f32_pl<S,S>"}}};
    if (args.kernel > KERN_SK) fail_invalid("unknown GEMM kernel");
    static const char* const deep[3][3] = {
        {"gemm_f32_pl32<K,K>", "gemm_f32_pl32<K,MN>", "gemm_f32_pl32<K,S>"},
        {"gemm_f32_pl32<MN,K>", "gemm_f32_pl32<MN,MN>", "gemm_f32_pl32<MN,S>"},
        {"gemm_f32_pl32<S,K>", "gemm_f32_pl32<S,MN>", "gemm_f32_pl32<S,S>"}};
    static const char* const kw[3][3] = {
        {"gemm_f32_kw<K,K>", "gemm_f32_kw<K,MN>", "gemm_f32_kw<K,S>"},
        {"gemm_f32_kw<MN,K>", "gemm_f32_kw<MN,MN>", "gemm_f32_kw<MN,S>"},
        {"gemm_f32_kw<S,K>", "gemm_f32_kw<S,MN>", "gemm_f32_kw<S,S>"}};
    static const char* const narrow[3][3] = {
        {"gemm_f32_pl_n64<K,K>", "gemm_f32_pl_n64<K,MN>", "gemm_f32_pl_n64<K,S>"},
        {"gemm_f32_pl_n64<MN,K>", "gemm_f32_pl_n64<MN,MN>", "gemm_f32_pl_n64<MN,S>"},
        {"gemm_f32_pl_n64<S,K>", "gemm_f32_pl_n64<S,MN>", "gemm_f32_pl_n64<S,S>"}};
    static const char* const sk[3][3] = {
        {"gemm_f32_sk<K,K>", "gemm_f32_sk<K,MN>", "gemm_f32_sk<K,S>"},
        {"gemm_f32_sk<MN,K>", "gemm_f32_sk<MN,MN>", "gemm_f32_sk<MN,S>"},
        {"gemm_f32_sk<S,K>", "gemm_f32_sk<S,MN>", "gemm_f32_sk<S,S>"}};
    const char* name = args.kernel == KERN_SK ? sk[a_mode][b_mode] : names[args.kernel][a_mode][b_mode];
    static const char* const tall[3][3] = {
        {"gemm_f32_pl256<K,K>", "gemm_f32_pl256<K,MN>", "gemm_f32_pl256<K,S>"},
        {"gemm_f32_pl256<MN,K>", "gemm_f32_pl256<MN,MN>", "gemm_f32_pl256<MN,S>"},
        {"gemm_f32_pl256<S,K>", "gemm_f32_pl256<S,MN>", "gemm_f32_pl256<S,S>"}};
    if (args.kernel == KERN_PIPE && args.tile == PIPE_TALL_M && args.tile_n == PIPE_WIDE_N) {
        name = a_mode != LOAD_K ? tall[a_mode][b_mode]
               : b_mode == LOAD_K ? "gemm_f32_pl2x<K,K>"
               : "gemm_f32_pl2x<K,MN>";
    } else if (args.kernel == KERN_PIPE && args.tile == PIPE_TALL_M) {
        name = tall[a_mode][b_mode];
    } else if (args.kernel == KERN_PIPE && args.tile == GEMM_BM && args.tile_n == PIPE_NARROW_N) {
        name = narrow[a_mode][b_mode];
    } else if (args.kernel == KERN_PIPE && args.tile == GEMM_SMALL_TILE) {
        name = kw[a_mode][b_mode];
    } else if (args.kernel == KERN_PIPE && args.slice_k == 32) {
        name = deep[a_mode][b_mode];
    }
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
    check_launch("gemm launch");
    note_launch(ctx, name);
}

void launch_reduce(Context* ctx, hipStream_t s, const ReduceArgs& args) {
    const uint64_t count = static_cast<uint64_t>(args.m) * args.n * args.batch;
    // Small outputs take one output per lane, so more workgroups share the splits' loads
    // (32x32 outputs: 16 workgroups instead of 4). The sum's order does not depend on V.
    const int v = args.n % 4 == 0 && count >= 65536 ? 4 : 1;
    const uint64_t per = static_cast<uint64_t>(RED_LANES) * v;
    const uint64_t g = (count + per - 1) / per;
    const dim3 grid(static_cast<uint32_t>(g < 65536 ? (g ? g : 1) : 65536));
    if (args.slices == 16) {
        if (v == 4) {
            hipLaunchKernelGGL((reduce_f32<4, 16>), grid, dim3(RED_LANES * 16), 0, s, args);
        } else {
            hipLaunchKernelGGL((reduce_f32<1, 16>), grid, dim3(RED_LANES * 16), 0, s, args);
        }
    } else if (args.slices == 4) {
        if (v == 4) {
            hipLaunchKernelGGL((reduce_f32<4, 4>), grid, dim3(RED_LANES * 4), 0, s, args);
        } else {
            hipLaunchKernelGGL((reduce_f32<1, 4>), grid, dim3(RED_LANES * 4), 0, s, args);
        }
    } else {
        fail_invalid("reduction slices must be 4 or 16");
    }
    check_launch("reduce_f32 launch");
    note_launch(ctx, "reduce_f32");
}

void launch_dot(Context* ctx, hipStream_t s, const DotArgs& args, bool vec) {
    const uint64_t groups = static_cast<uint64_t>(args.batch) * args.splits;
    if (vec) {
        hipLaunchKernelGGL(dot_f32<true>, dim3(static_cast<uint32_t>(groups)), dim3(DOT_THREADS), 0, s, args);
    } else {
        hipLaunchKernelGGL(dot_f32<false>, dim3(static_cast<uint32_t>(groups)), dim3(DOT_THREADS), 0, s, args);
    }
    check_launch("dot_f32 launch");
    note_launch(ctx, "dot_f32");
    if (args.splits > 1) {
        hipLaunchKernelGGL(dot_finish_f32, dim3(args.batch), dim3(DOT_THREADS), 0, s, args);
        check_launch("dot_finish_f32 launch");
        note_launch(ctx, "dot_finish_f32");
    }
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
