// gfx950 kernels of the Backend training ops: GELU and its derivative, bias add, bias
// gradient, MSE gradient + loss, SGD step and f32 <-> bf16 conversion. All operands are
// row-major contiguous f32 (bf16 for one side of a conversion) at offset 0.
//
// Every formula is evaluated as written, one rounding per operation (-ffp-contract=off; f32
// division is IEEE-correctly rounded in HIP device code), so the elementwise ops return the
// reference loop's bits; GELU differs only where the device expf rounds differently. HBM-bound:
// 128-bit accesses whenever the operands allow them (element count a multiple of 4, bases
// 16-byte aligned), grid-stride loops over at most GRID_CAP workgroups.
#include <hip/hip_runtime.h>

#include "lg_internal.h"

namespace lg {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int THREADS = 256;
constexpr uint64_t GRID_CAP = 8192;

// Abramowitz & Stegun 7.1.26 (max |error| 1.5e-7 on erf), with the coefficients rounded to
// f32: 0.254829592, -0.284496736, 1.421413741, -1.453152027, 1.061405429, p = 0.3275911.
// The same rounding and evaluation order as crates/cpu/src/lib.rs:809-842.
constexpr float ERF_A1 = 0.2548296f;
constexpr float ERF_A2 = 0.28449672f;
constexpr float ERF_A3 = 1.4214138f;
constexpr float ERF_A4 = 1.4531521f;
constexpr float ERF_A5 = 1.0614054f;
constexpr float ERF_P = 0.3275911f;
constexpr float INV_SQRT_2PI = 0.3989423f;
constexpr float FRAC_1_SQRT_2 = 0.70710677f;

__device__ inline float erf_as(float x) {
    const float sign = __builtin_signbit(x) ? -1.0f : 1.0f;
    const float a = __builtin_fabsf(x);
    const float t = 1.0f / (1.0f + ERF_P * a);
    const float poly = (((((ERF_A5 * t - ERF_A4) * t) + ERF_A3) * t - ERF_A2) * t + ERF_A1) * t;
    return sign * (1.0f - poly * expf(-a * a));
}

__device__ inline float gelu_one(float x) {
    const float inner = x * FRAC_1_SQRT_2;
    return 0.5f * x * (1.0f + erf_as(inner));
}

__device__ inline float gelu_prime_one(float x) {
    const float phi = 0.5f * (1.0f + erf_as(x * FRAC_1_SQRT_2));
    const float pdf = expf(-0.5f * x * x) * INV_SQRT_2PI;
    return phi + x * pdf;
}

__device__ inline uint64_t first_index() {
    return static_cast<uint64_t>(blockIdx.x) * THREADS + threadIdx.x;
}
__device__ inline uint64_t grid_step() { return static_cast<uint64_t>(gridDim.x) * THREADS; }

// y = GELU(x); y may be x. VEC: n % 4 == 0 and both bases 16-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(THREADS) void gelu_f32(const float* x, float* y, uint64_t n) {
    if constexpr (VEC) {
        const uint64_t n4 = n / 4;
        for (uint64_t i = first_index(); i < n4; i += grid_step()) {
            f32x4 v = reinterpret_cast<const f32x4*>(x)[i];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = gelu_one(v[e]);
            reinterpret_cast<f32x4*>(y)[i] = v;
        }
    } else {
        for (uint64_t i = first_index(); i < n; i += grid_step()) y[i] = gelu_one(x[i]);
    }
}

// dx = dy * GELU'(pre).
template <bool VEC>
__global__ __launch_bounds__(THREADS) void gelu_backward_f32(const float* pre, const float* dy,
                                                             float* dx, uint64_t n) {
    if constexpr (VEC) {
        const uint64_t n4 = n / 4;
        for (uint64_t i = first_index(); i < n4; i += grid_step()) {
            const f32x4 p = reinterpret_cast<const f32x4*>(pre)[i];
            const f32x4 g = reinterpret_cast<const f32x4*>(dy)[i];
            f32x4 r;
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = g[e] * gelu_prime_one(p[e]);
            reinterpret_cast<f32x4*>(dx)[i] = r;
        }
    } else {
        for (uint64_t i = first_index(); i < n; i += grid_step()) dx[i] = dy[i] * gelu_prime_one(pre[i]);
    }
}

// y[i][j] = x[i][j] + b[j]; y may be x. VEC additionally needs cols % 4 == 0.
template <bool VEC>
__global__ __launch_bounds__(THREADS) void add_bias_f32(const float* x, const float* b, float* y,
                                                        uint64_t n, uint64_t cols) {
    if constexpr (VEC) {
        const uint64_t n4 = n / 4;
        for (uint64_t i = first_index(); i < n4; i += grid_step()) {
            const uint64_t col = (i * 4) % cols;
            const f32x4 v = reinterpret_cast<const f32x4*>(x)[i];
            const f32x4 bb = *reinterpret_cast<const f32x4*>(b + col);
            reinterpret_cast<f32x4*>(y)[i] = v + bb;
        }
    } else {
        for (uint64_t i = first_index(); i < n; i += grid_step()) y[i] = x[i] + b[i % cols];
    }
}

// db[j] = db[j] + s[j], s[j] = dpre[0][j] + dpre[1][j] + ... in row order: the reference's
// sequential column sum, one lane per column (loads coalesce across lanes). UNROLL loads are
// issued before they are added, in order, so each lane keeps UNROLL loads in flight.
constexpr int BIAS_UNROLL = 16;
__global__ __launch_bounds__(THREADS) void bias_grad_f32(const float* dpre, float* db,
                                                         uint32_t rows, uint32_t cols) {
    const uint32_t j = blockIdx.x * THREADS + threadIdx.x;
    if (j >= cols) return;
    const float* p = dpre + j;
    float s = 0.0f;
    uint32_t r = 0;
    for (; r + BIAS_UNROLL <= rows; r += BIAS_UNROLL) {
        float v[BIAS_UNROLL];
#pragma unroll
        for (int u = 0; u < BIAS_UNROLL; ++u) v[u] = p[static_cast<uint64_t>(r + u) * cols];
#pragma unroll
        for (int u = 0; u < BIAS_UNROLL; ++u) s = s + v[u];
    }
    for (; r < rows; ++r) s = s + p[static_cast<uint64_t>(r) * cols];
    db[j] = db[j] + s;
}

// MSE: d = y - target; dy = (2*d) / n; loss = (sum d*d) / n, in one launch. Workgroup g owns
// the contiguous run [g*chunk, (g+1)*chunk); each lane sums its strided share in index order,
// the 256 lane sums meet in a fixed LDS tree, and the workgroup's sum goes to partial[g]. The
// workgroup that finishes last (ticket from a device-wide counter) adds partial[0..G) in a
// fixed order and writes the loss, so the summation order depends only on n. dy may be y.
// The counter starts at zero (the host clears it before the launch); nothing waits on another
// workgroup, so no schedule can hang.
__global__ __launch_bounds__(THREADS) void mse_grad_f32(const float* y, const float* target,
                                                        float* dy, uint64_t n, uint64_t chunk,
                                                        float nf, float* partial,
                                                        uint32_t* counter, float* loss) {
    __shared__ float red[THREADS];
    __shared__ bool last;
    const uint32_t groups = gridDim.x;
    const uint64_t lo = static_cast<uint64_t>(blockIdx.x) * chunk;
    const uint64_t hi = lo + chunk < n ? lo + chunk : n;
    float s = 0.0f;
    for (uint64_t i = lo + threadIdx.x; i < hi; i += THREADS) {
        const float d = y[i] - target[i];
        s = s + d * d;
        dy[i] = (2.0f * d) / nf;
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = THREADS / 2; w > 0; w /= 2) {
        if (static_cast<int>(threadIdx.x) < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        // Device-scope store, release fence, then the ticket: partials of every workgroup are
        // visible (across XCDs) to whichever workgroup draws the last ticket.
        __hip_atomic_store(partial + blockIdx.x, red[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __threadfence();
        last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
               groups - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    float t = 0.0f;
    for (uint32_t g = threadIdx.x; g < groups; g += THREADS) {
        t = t + __hip_atomic_load(partial + g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    red[threadIdx.x] = t;
    __syncthreads();
    for (int w = THREADS / 2; w > 0; w /= 2) {
        if (static_cast<int>(threadIdx.x) < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) *loss = red[0] / nf;
}

// w = w - (lr * dw); dw = +0.
template <bool VEC>
__global__ __launch_bounds__(THREADS) void sgd_step_f32(float* w, float* dw, float lr, uint64_t n) {
    if constexpr (VEC) {
        const uint64_t n4 = n / 4;
        for (uint64_t i = first_index(); i < n4; i += grid_step()) {
            const f32x4 g = reinterpret_cast<const f32x4*>(dw)[i];
            const f32x4 v = reinterpret_cast<const f32x4*>(w)[i];
            reinterpret_cast<f32x4*>(w)[i] = v - lr * g;
            reinterpret_cast<f32x4*>(dw)[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    } else {
        for (uint64_t i = first_index(); i < n; i += grid_step()) {
            const float step = lr * dw[i];
            w[i] = w[i] - step;
            dw[i] = 0.0f;
        }
    }
}

// f32 bits -> bf16 bits: nearest, ties to even; NaN stays NaN (quiet, same sign, top payload
// bits); the rounding carry takes the largest finite values to infinity and keeps subnormals.
__device__ inline uint32_t bf16_bits(uint32_t bits) {
    if ((bits & 0x7fffffffu) > 0x7f800000u) return ((bits >> 16) | 0x0040u) & 0xffffu;
    const uint32_t lsb = (bits >> 16) & 1u;
    return (bits + 0x7fffu + lsb) >> 16;
}

// VEC: n % 4 == 0, source 16-byte and destination 8-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(THREADS) void convert_f32_bf16(const uint32_t* x, uint16_t* y, uint64_t n) {
    if constexpr (VEC) {
        const uint64_t n4 = n / 4;
        for (uint64_t i = first_index(); i < n4; i += grid_step()) {
            const u32x4 v = reinterpret_cast<const u32x4*>(x)[i];
            u32x2 o;
            o[0] = bf16_bits(v[0]) | (bf16_bits(v[1]) << 16);
            o[1] = bf16_bits(v[2]) | (bf16_bits(v[3]) << 16);
            reinterpret_cast<u32x2*>(y)[i] = o;
        }
    } else {
        for (uint64_t i = first_index(); i < n; i += grid_step()) y[i] = static_cast<uint16_t>(bf16_bits(x[i]));
    }
}

// bf16 bits -> f32: exact, the bits move to the upper half.
template <bool VEC>
__global__ __launch_bounds__(THREADS) void convert_bf16_f32(const uint16_t* x, uint32_t* y, uint64_t n) {
    if constexpr (VEC) {
        const uint64_t n4 = n / 4;
        for (uint64_t i = first_index(); i < n4; i += grid_step()) {
            const u32x2 v = reinterpret_cast<const u32x2*>(x)[i];
            u32x4 o;
            o[0] = v[0] << 16;
            o[1] = v[0] & 0xffff0000u;
            o[2] = v[1] << 16;
            o[3] = v[1] & 0xffff0000u;
            reinterpret_cast<u32x4*>(y)[i] = o;
        }
    } else {
        for (uint64_t i = first_index(); i < n; i += grid_step()) y[i] = static_cast<uint32_t>(x[i]) << 16;
    }
}

uint32_t grid(uint64_t items) {
    const uint64_t g = (items + THREADS - 1) / THREADS;
    return static_cast<uint32_t>(g < 1 ? 1 : (g > GRID_CAP ? GRID_CAP : g));
}

bool aligned(const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

void after_launch(Context* ctx, const char* name) {
    check_hip(hipGetLastError(), name);
    note_launch(ctx, name);
}

}  // namespace

void launch_gelu(Context* ctx, hipStream_t s, const float* x, float* y, uint64_t n) {
    if (n % 4 == 0 && aligned(x, 16) && aligned(y, 16)) {
        hipLaunchKernelGGL(gelu_f32<true>, dim3(grid(n / 4)), dim3(THREADS), 0, s, x, y, n);
    } else {
        hipLaunchKernelGGL(gelu_f32<false>, dim3(grid(n)), dim3(THREADS), 0, s, x, y, n);
    }
    after_launch(ctx, "gelu_f32");
}

void launch_gelu_backward(Context* ctx, hipStream_t s, const float* pre, const float* dy,
                          float* dx, uint64_t n) {
    if (n % 4 == 0 && aligned(pre, 16) && aligned(dy, 16) && aligned(dx, 16)) {
        hipLaunchKernelGGL(gelu_backward_f32<true>, dim3(grid(n / 4)), dim3(THREADS), 0, s, pre, dy,
                           dx, n);
    } else {
        hipLaunchKernelGGL(gelu_backward_f32<false>, dim3(grid(n)), dim3(THREADS), 0, s, pre, dy, dx,
                           n);
    }
    after_launch(ctx, "gelu_backward_f32");
}

void launch_add_bias(Context* ctx, hipStream_t s, const float* x, const float* b, float* y,
                     uint64_t rows, uint64_t cols) {
    const uint64_t n = rows * cols;
    if (cols % 4 == 0 && aligned(x, 16) && aligned(b, 16) && aligned(y, 16)) {
        hipLaunchKernelGGL(add_bias_f32<true>, dim3(grid(n / 4)), dim3(THREADS), 0, s, x, b, y, n,
                           cols);
    } else {
        hipLaunchKernelGGL(add_bias_f32<false>, dim3(grid(n)), dim3(THREADS), 0, s, x, b, y, n, cols);
    }
    after_launch(ctx, "add_bias_f32");
}

void launch_bias_grad(Context* ctx, hipStream_t s, const float* dpre, float* db, uint32_t rows,
                      uint32_t cols) {
    const uint32_t g = (cols + THREADS - 1) / THREADS;
    hipLaunchKernelGGL(bias_grad_f32, dim3(g), dim3(THREADS), 0, s, dpre, db, rows, cols);
    after_launch(ctx, "bias_grad_f32");
}

uint64_t mse_groups(uint64_t n, uint64_t* chunk) {
    // At least 4096 elements per workgroup, at most 4096 workgroups; shape-only, so the
    // summation order is a function of n alone.
    uint64_t c = (n + MSE_MAX_GROUPS - 1) / MSE_MAX_GROUPS;
    if (c < MSE_MIN_CHUNK) c = MSE_MIN_CHUNK;
    *chunk = c;
    return (n + c - 1) / c;
}

void launch_mse_grad(Context* ctx, hipStream_t s, const float* y, const float* target, float* dy,
                     uint64_t n, float* partial, uint32_t* counter, float* loss) {
    uint64_t chunk = 0;
    const uint64_t g = mse_groups(n, &chunk);
    const float nf = static_cast<float>(n);
    hipLaunchKernelGGL(mse_grad_f32, dim3(static_cast<uint32_t>(g)), dim3(THREADS), 0, s, y, target,
                       dy, n, chunk, nf, partial, counter, loss);
    after_launch(ctx, "mse_grad_f32");
}

void launch_sgd_step(Context* ctx, hipStream_t s, float* w, float* dw, float lr, uint64_t n) {
    if (n % 4 == 0 && aligned(w, 16) && aligned(dw, 16)) {
        hipLaunchKernelGGL(sgd_step_f32<true>, dim3(grid(n / 4)), dim3(THREADS), 0, s, w, dw, lr, n);
    } else {
        hipLaunchKernelGGL(sgd_step_f32<false>, dim3(grid(n)), dim3(THREADS), 0, s, w, dw, lr, n);
    }
    after_launch(ctx, "sgd_step_f32");
}

void launch_convert(Context* ctx, hipStream_t s, bool to_bf16, const void* x, void* y, uint64_t n) {
    if (to_bf16) {
        const uint32_t* src = static_cast<const uint32_t*>(x);
        uint16_t* dst = static_cast<uint16_t*>(y);
        if (n % 4 == 0 && aligned(x, 16) && aligned(y, 8)) {
            hipLaunchKernelGGL(convert_f32_bf16<true>, dim3(grid(n / 4)), dim3(THREADS), 0, s, src, dst, n);
        } else {
            hipLaunchKernelGGL(convert_f32_bf16<false>, dim3(grid(n)), dim3(THREADS), 0, s, src, dst, n);
        }
        after_launch(ctx, "convert_f32_bf16");
    } else {
        const uint16_t* src = static_cast<const uint16_t*>(x);
        uint32_t* dst = static_cast<uint32_t*>(y);
        if (n % 4 == 0 && aligned(x, 8) && aligned(y, 16)) {
            hipLaunchKernelGGL(convert_bf16_f32<true>, dim3(grid(n / 4)), dim3(THREADS), 0, s, src, dst, n);
        } else {
            hipLaunchKernelGGL(convert_bf16_f32<false>, dim3(grid(n)), dim3(THREADS), 0, s, src, dst, n);
        }
        after_launch(ctx, "convert_bf16_f32");
    }
}

}  // namespace lg
