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
// One 128-bit vector per thread for every tensor up to 2^30 vectors: many short-lived
// workgroups keep more loads in flight than a grid-stride loop over a capped grid.
constexpr uint64_t GRID_CAP = 1u << 20;

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
// sequential column sum, bit for bit. The dependency chain runs down each column, so the
// loads are decoupled from it: a workgroup owns BG_COLS columns; all four waves stream blocks
// of BG_ROWS rows into a double-buffered LDS tile (the next block's loads are in flight while
// the current one is summed), and wave 0 -- one lane per column -- adds the block's rows in
// order. One workgroup per 64 columns keeps 64 KB of loads in flight per CU (128 KB of LDS).
constexpr int BG_COLS = 64;
constexpr int BG_ROWS = 256;
constexpr int BG_LOADS = BG_ROWS * BG_COLS / 4 / THREADS;  // 128-bit loads per thread per block
static_assert(BG_LOADS * THREADS * 4 == BG_ROWS * BG_COLS, "block must split evenly");

template <bool VEC>
__global__ __launch_bounds__(THREADS) void bias_grad_f32(const float* dpre, float* db,
                                                         uint32_t rows, uint32_t cols) {
    __shared__ f32x4 tile[2][BG_ROWS * BG_COLS / 4];
    const int tid = threadIdx.x;
    const uint32_t c0 = blockIdx.x * BG_COLS;
    const uint32_t nblk = (rows + BG_ROWS - 1) / BG_ROWS;
    f32x4 r[BG_LOADS];
    // Element (row, col) of block b: thread t's i-th vector covers row (i*THREADS+t) / 16,
    // columns 4*((i*THREADS+t) % 16) .. +3 of the workgroup's 64.
    auto fetch = [&](uint32_t b) {
#pragma unroll
        for (int i = 0; i < BG_LOADS; ++i) {
            const int v = i * THREADS + tid;
            const uint32_t row = b * BG_ROWS + v / (BG_COLS / 4);
            const uint32_t col = c0 + (v % (BG_COLS / 4)) * 4;
            const float* p = dpre + static_cast<uint64_t>(row) * cols + col;
            if (VEC && row < rows && col + 4 <= cols) {
                r[i] = *reinterpret_cast<const f32x4*>(p);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) r[i][e] = (row < rows && col + e < cols) ? p[e] : 0.0f;
            }
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int i = 0; i < BG_LOADS; ++i) tile[buf][i * THREADS + tid] = r[i];
    };
    fetch(0);
    stash(0);
    __syncthreads();
    float s = 0.0f;
    const float* lane_col = reinterpret_cast<const float*>(tile[0]) + tid;  // wave 0 only
    for (uint32_t b = 0; b < nblk; ++b) {
        const int buf = b & 1;
        if (b + 1 < nblk) fetch(b + 1);
        if (tid < BG_COLS) {
            const uint32_t n = min(static_cast<uint32_t>(BG_ROWS), rows - b * BG_ROWS);
            const float* col = lane_col + buf * BG_ROWS * BG_COLS;
            for (uint32_t i = 0; i < n; ++i) s = s + col[i * BG_COLS];
        }
        if (b + 1 < nblk) stash(buf ^ 1);
        __syncthreads();
    }
    const uint32_t j = c0 + tid;
    if (tid < BG_COLS && j < cols) db[j] = db[j] + s;
}

// MSE: d = y - target; dy = (2*d) / n; loss = (sum d*d) / n, in one launch. At most
// MSE_MAX_GROUPS workgroups: each pays one device-scope release (an L2 write-back on this
// multi-XCD part), which measured 0.1 us apiece when 4096 workgroups issued them. Workgroup g owns
// the contiguous run [g*chunk, (g+1)*chunk); each lane sums its strided share in index order,
// the 256 lane sums meet in a fixed LDS tree, and the workgroup's sum goes to partial[g]. The
// workgroup that finishes last (ticket from a device-wide counter) adds partial[0..G) in a
// fixed order and writes the loss, so the summation order depends only on n (VEC, 128-bit
// accesses, is chosen by n % 4 and alignment alone). dy may be y.
// The counter starts at zero (the host clears it before the launch); nothing waits on another
// workgroup, so no schedule can hang.
constexpr int MSE_UNROLL = 4;

template <bool VEC>
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
    if (VEC) {
        // chunk and lo are multiples of 4: lane t takes vectors t, t + 256, ... of the run and
        // adds the four squares of each in index order; MSE_UNROLL vectors' loads are issued
        // before the first is used.
        const f32x4* yv = reinterpret_cast<const f32x4*>(y + lo);
        const f32x4* tv = reinterpret_cast<const f32x4*>(target + lo);
        f32x4* dv = reinterpret_cast<f32x4*>(dy + lo);
        const uint64_t nv = (hi - lo) / 4;
        auto one = [&](f32x4 a, f32x4 b, uint64_t i) {
            const f32x4 d = a - b;
            s = s + d[0] * d[0];
            s = s + d[1] * d[1];
            s = s + d[2] * d[2];
            s = s + d[3] * d[3];
            dv[i] = (2.0f * d) / nf;
        };
        uint64_t i = threadIdx.x;
        for (; i + (MSE_UNROLL - 1) * THREADS < nv; i += MSE_UNROLL * THREADS) {
            f32x4 a[MSE_UNROLL], b[MSE_UNROLL];
#pragma unroll
            for (int u = 0; u < MSE_UNROLL; ++u) {
                a[u] = yv[i + u * THREADS];
                b[u] = tv[i + u * THREADS];
            }
#pragma unroll
            for (int u = 0; u < MSE_UNROLL; ++u) one(a[u], b[u], i + u * THREADS);
        }
        for (; i < nv; i += THREADS) one(yv[i], tv[i], i);
    } else {
        for (uint64_t i = lo + threadIdx.x; i < hi; i += THREADS) {
            const float d = y[i] - target[i];
            s = s + d * d;
            dy[i] = (2.0f * d) / nf;
        }
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
    const uint32_t g = (cols + BG_COLS - 1) / BG_COLS;
    if (cols % 4 == 0 && aligned(dpre, 16)) {
        hipLaunchKernelGGL(bias_grad_f32<true>, dim3(g), dim3(THREADS), 0, s, dpre, db, rows, cols);
    } else {
        hipLaunchKernelGGL(bias_grad_f32<false>, dim3(g), dim3(THREADS), 0, s, dpre, db, rows, cols);
    }
    after_launch(ctx, "bias_grad_f32");
}

uint64_t mse_groups(uint64_t n, uint64_t* chunk) {
    // At least MSE_MIN_CHUNK elements per workgroup, at most MSE_MAX_GROUPS workgroups;
    // shape-only, so the summation order is a function of n alone.
    uint64_t c = (n + MSE_MAX_GROUPS - 1) / MSE_MAX_GROUPS;
    if (c < MSE_MIN_CHUNK) c = MSE_MIN_CHUNK;
    c = (c + 3) / 4 * 4;  // whole 128-bit vectors per workgroup
    *chunk = c;
    return (n + c - 1) / c;
}

void launch_mse_grad(Context* ctx, hipStream_t s, const float* y, const float* target, float* dy,
                     uint64_t n, float* partial, uint32_t* counter, float* loss) {
    uint64_t chunk = 0;
    const uint64_t g = mse_groups(n, &chunk);
    const float nf = static_cast<float>(n);
    if (n % 4 == 0 && aligned(y, 16) && aligned(target, 16) && aligned(dy, 16)) {
        hipLaunchKernelGGL(mse_grad_f32<true>, dim3(static_cast<uint32_t>(g)), dim3(THREADS), 0, s,
                           y, target, dy, n, chunk, nf, partial, counter, loss);
    } else {
        hipLaunchKernelGGL(mse_grad_f32<false>, dim3(static_cast<uint32_t>(g)), dim3(THREADS), 0, s,
                           y, target, dy, n, chunk, nf, partial, counter, loss);
    }
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
