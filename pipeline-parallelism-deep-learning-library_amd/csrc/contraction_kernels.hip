// gfx950 contraction kernels.
//
// gemm_f32_mfma: C = alpha * A.B + beta * C (or raw split-K partials) for one stride per
// group. 128x128 output tile per 256-thread workgroup (4 waves in 2x2, each wave 64x64 =
// 2x2 blocks of v_mfma_f32_32x32x2_f32 with fp32 accumulation). K advances 32 at a time
// through two LDS stages: while the MFMAs consume stage s, the next K-slice is already in
// flight from HBM into registers, and is written to stage s^1 before the one barrier per
// slice. Operand loads follow the operand's unit-stride axis so a transposed or permuted
// view is read as it lies, 128 bits per load:
//   LOAD_K  : unit stride along K  -> LDS [row][k]   (pitch 36), 128-bit LDS reads along k
//   LOAD_MN : unit stride along M/N-> LDS [k][row]   (pitch 136), 32-bit LDS reads
//   LOAD_S  : anything else        -> 32-bit predicated loads into the [row][k] layout
// Inside a 32-wide K slice, MFMA step s of lane half h uses k = 8*(s/4) + 4*h + s%4, so a
// [row][k] stage hands each lane four consecutive k with one ds_read_b128. A and B agree on
// this order, so every product pairs the same k.
//
// The other kernels are the split-K reduction (fixed order over splits, so results are
// bit-reproducible), the mixed-radix general fallback, and the C = 0 / C = beta*C fill.
// Everything is compiled with -ffp-contract=off: alpha*acc and beta*C round separately.
#include <hip/hip_runtime.h>

#include "lg_internal.h"

namespace lg {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = GEMM_BM, BN = GEMM_BN, BK = GEMM_BK;
constexpr int PK = BK + 4;   // pitch of a [row][k] stage (floats)
constexpr int PMN = BM + 8;  // pitch of a [k][row] stage (floats)
static_assert(BM == BN, "stage pitches assume square tiles");
constexpr int LOADS = (BM * BK / 4) / GEMM_THREADS;  // 128-bit loads per thread per operand
static_assert(LOADS * GEMM_THREADS * 4 == BM * BK, "tile must split evenly over the threads");

// Workgroup -> (plane, tile_m, tile_n). Workgroups are dealt round-robin to the 8 XCDs, so
// the linear id is first regrouped so each XCD owns one contiguous run of tiles (sharing
// its L2), then tiles within a plane are walked in groups of 8 tile-rows for A/B reuse.
__device__ inline void decode_tile(uint32_t bid, uint32_t total, uint32_t tiles_m,
                                   uint32_t tiles_n, uint32_t* plane, uint32_t* tm,
                                   uint32_t* tn) {
    const uint32_t xcd = bid & 7u, slot = bid >> 3;
    const uint32_t q = total >> 3, r = total & 7u;
    const uint32_t lin = xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
    const uint32_t per_plane = tiles_m * tiles_n;
    *plane = lin / per_plane;
    const uint32_t t = lin - *plane * per_plane;
    constexpr uint32_t GROUP = 8;
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
template <int MODE>
__device__ inline void load_slice(floatx4 (&r)[LOADS], const float* __restrict__ p, int64_t srow,
                                  int64_t sk, uint32_t rows_left, uint32_t k0, uint32_t klen,
                                  int tid) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int idx = i * GEMM_THREADS + tid;
        if constexpr (MODE == LOAD_MN) {
            const uint32_t kr = k0 + idx / (BM / 4);
            const uint32_t row = (idx % (BM / 4)) * 4;
            const float* q = p + static_cast<int64_t>(kr) * sk + row;
            if (kr < klen && row + 4 <= rows_left) {
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
                if (row < rows_left && kk + 4 <= klen) {
                    r[i] = *reinterpret_cast<const floatx4*>(q);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) r[i][e] = (row < rows_left && kk + e < klen) ? q[e] : 0.0f;
                }
            } else {
                const float* q = p + static_cast<int64_t>(row) * srow;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    r[i][e] = (row < rows_left && kk + e < klen)
                                  ? q[static_cast<int64_t>(kk + e) * sk]
                                  : 0.0f;
                }
            }
        }
    }
}

template <int MODE>
__device__ inline void store_slice(float* __restrict__ st, const floatx4 (&r)[LOADS], int tid) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int idx = i * GEMM_THREADS + tid;
        if constexpr (MODE == LOAD_MN) {
            const int kr = idx / (BM / 4), row = (idx % (BM / 4)) * 4;
            *reinterpret_cast<floatx4*>(st + kr * PMN + row) = r[i];
        } else {
            const int row = idx / (BK / 4), kq = (idx % (BK / 4)) * 4;
            *reinterpret_cast<floatx4*>(st + row * PK + kq) = r[i];
        }
    }
}

// Operand values of the two 32-row blocks `base_row + {0, 32}` for MFMA steps 4g..4g+3.
template <int MODE>
__device__ inline void read_frag(floatx4 (&v)[2], const float* __restrict__ st, int base_row,
                                 int g, int lr, int h) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int row = base_row + i * 32 + lr;
        if constexpr (MODE == LOAD_MN) {
#pragma unroll
            for (int s = 0; s < 4; ++s) v[i][s] = st[(g * 8 + h * 4 + s) * PMN + row];
        } else {
            v[i] = *reinterpret_cast<const floatx4*>(st + row * PK + g * 8 + h * 4);
        }
    }
}

template <int AM, int BMD>
__global__ __launch_bounds__(GEMM_THREADS) void gemm_f32_mfma(GemmArgs p) {
    constexpr int A_ST = (AM == LOAD_MN) ? BK * PMN : BM * PK;
    constexpr int B_ST = (BMD == LOAD_MN) ? BK * PMN : BN * PK;
    __shared__ __attribute__((aligned(16))) float smem[2 * (A_ST + B_ST)];
    float* As = smem;
    float* Bs = smem + 2 * A_ST;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, h = lane >> 5;

    const uint32_t total = gridDim.x;
    uint32_t plane, tm, tn;
    decode_tile(blockIdx.x, total, p.tiles_m, p.tiles_n, &plane, &tm, &tn);
    const uint32_t bi = plane / p.splits, split = plane - bi * p.splits;
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t kb = split * p.k_chunk;
    const uint32_t klen = min(p.k - kb, p.k_chunk);
    const uint32_t mrem = p.m - m0, nrem = p.n - n0;

    const float* A = p.a + static_cast<int64_t>(bi) * p.a_sb + static_cast<int64_t>(m0) * p.a_sm +
                     static_cast<int64_t>(kb) * p.a_sk;
    const float* B = p.b + static_cast<int64_t>(bi) * p.b_sb + static_cast<int64_t>(n0) * p.b_sn +
                     static_cast<int64_t>(kb) * p.b_sk;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    floatx4 ra[LOADS], rb[LOADS];
    const uint32_t ktiles = (klen + BK - 1) / BK;
    load_slice<AM>(ra, A, p.a_sm, p.a_sk, mrem, 0, klen, tid);
    load_slice<BMD>(rb, B, p.b_sn, p.b_sk, nrem, 0, klen, tid);
    store_slice<AM>(As, ra, tid);
    store_slice<BMD>(Bs, rb, tid);
    __syncthreads();

    for (uint32_t kt = 0; kt < ktiles; ++kt) {
        const int s = kt & 1;
        const bool more = kt + 1 < ktiles;
        if (more) {
            load_slice<AM>(ra, A, p.a_sm, p.a_sk, mrem, (kt + 1) * BK, klen, tid);
            load_slice<BMD>(rb, B, p.b_sn, p.b_sk, nrem, (kt + 1) * BK, klen, tid);
        }
        const float* as = As + s * A_ST;
        const float* bs = Bs + s * B_ST;
#pragma unroll
        for (int g = 0; g < BK / 8; ++g) {
            floatx4 av[2], bv[2];
            read_frag<AM>(av, as, wm * 64, g, lr, h);
            read_frag<BMD>(bv, bs, wn * 64, g, lr, h);
#pragma unroll
            for (int st = 0; st < 4; ++st)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][st], bv[j][st],
                                                                         acc[i][j], 0, 0, 0);
        }
        if (more) {
            store_slice<AM>(As + (s ^ 1) * A_ST, ra, tid);
            store_slice<BMD>(Bs + (s ^ 1) * B_ST, rb, tid);
        }
        __syncthreads();
    }

    // Epilogue. Accumulator register r of block (i, j) holds
    // row = 8*(r/4) + 4*h + r%4, col = lane%32 of that 32x32 block.
    if (p.partial != nullptr) {
        float* P = p.partial + static_cast<int64_t>(plane) * p.m * p.n;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
                    const uint32_t col = n0 + wn * 64 + j * 32 + lr;
                    if (row < p.m && col < p.n) P[static_cast<int64_t>(row) * p.n + col] = acc[i][j][r];
                }
        return;
    }
    float* C = p.c + static_cast<int64_t>(bi) * p.c_sb;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
                const uint32_t col = n0 + wn * 64 + j * 32 + lr;
                if (row < p.m && col < p.n) {
                    float* q = C + static_cast<int64_t>(row) * p.c_sm + static_cast<int64_t>(col) * p.c_sn;
                    float v = p.alpha * acc[i][j][r];
                    if (p.beta != 0.0f) v = v + p.beta * *q;
                    *q = v;
                }
            }
}

// Split-K second pass: for every output, sum the partials of splits 0..S-1 in order, then
// apply alpha and beta once. Partials are [batch][splits][m][n], dense.
__global__ __launch_bounds__(256) void reduce_f32(ReduceArgs p) {
    const uint64_t mn = static_cast<uint64_t>(p.m) * p.n;
    const uint64_t count = mn * p.batch;
    for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < count;
         e += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t bi = e / mn, rem = e - bi * mn;
        const uint32_t row = static_cast<uint32_t>(rem / p.n), col = static_cast<uint32_t>(rem % p.n);
        const float* src = p.partial + bi * p.splits * mn + rem;
        float acc = 0.0f;
        for (uint32_t s = 0; s < p.splits; ++s) acc = acc + src[s * mn];
        float* q = p.c + static_cast<int64_t>(bi) * p.c_sb + static_cast<int64_t>(row) * p.c_sm +
                   static_cast<int64_t>(col) * p.c_sn;
        float v = p.alpha * acc;
        if (p.beta != 0.0f) v = v + p.beta * *q;
        *q = v;
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

// Fallback for groups that keep more than one stride after merging: one thread per output,
// K walked in order with an odometer over the (up to four) K axes of A and B.
__global__ __launch_bounds__(256) void general_f32(GeneralArgs p) {
    const uint64_t mn = static_cast<uint64_t>(p.m) * p.n;
    const uint64_t count = mn * p.batch;
    for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < count;
         e += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t bi = e / mn, rem = e - bi * mn;
        const uint64_t mi = rem / p.n, ni = rem - mi * p.n;
        const float* a = p.a + decode4(p.a_batch, bi) + decode4(p.a_m, mi);
        const float* b = p.b + decode4(p.b_batch, bi) + decode4(p.b_n, ni);
        float acc = 0.0f;
        uint32_t dig[4] = {0, 0, 0, 0};
        int64_t oa = 0, ob = 0;
        for (uint32_t kk = 0; kk < p.k; ++kk) {
            acc = acc + a[oa] * b[ob];
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
        float* q = p.c + decode4(p.c_batch, bi) + decode4(p.c_m, mi) + decode4(p.c_n, ni);
        float v = p.alpha * acc;
        if (p.beta != 0.0f) v = v + p.beta * *q;
        *q = v;
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
    hipLaunchKernelGGL((gemm_f32_mfma<AM, BMD>), dim3(groups), dim3(GEMM_THREADS), 0, s, a);
}

}  // namespace

uint64_t gemm_workgroups(uint32_t m, uint32_t n, uint32_t batch, uint32_t splits) {
    const uint64_t tm = (m + GEMM_BM - 1) / GEMM_BM, tn = (n + GEMM_BN - 1) / GEMM_BN;
    return tm * tn * batch * splits;
}

void launch_gemm(Context* ctx, hipStream_t s, const GemmArgs& args, int a_mode, int b_mode) {
    const uint32_t groups =
        static_cast<uint32_t>(gemm_workgroups(args.m, args.n, args.batch, args.splits));
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
    hipLaunchKernelGGL(reduce_f32, dim3(grid_for(count)), dim3(256), 0, s, args);
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
