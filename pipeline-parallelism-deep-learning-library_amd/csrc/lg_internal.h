// Internal interfaces between the host planner (C++) and the gfx950 kernels (HIP).
//
// Kernel argument structs are passed by value. All element offsets and strides are 64-bit
// (one MI355X holds 288 GB, so views far past 2^32 elements are legal); extents handed to
// a kernel are 32-bit and the planner proves they fit.
#pragma once

#include <atomic>
#include <cstdint>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "linalg_hip.h"

namespace lg {

// ---------------------------------------------------------------------------------------
// Errors: thrown inside the library, turned into lg_status at the C boundary.
// ---------------------------------------------------------------------------------------
struct Failure {
    lg_status status;
    std::string message;
};
[[noreturn]] void fail_invalid(const std::string& msg);
[[noreturn]] void fail_overlap(const std::string& msg);
[[noreturn]] void fail_kernel(const std::string& msg);
[[noreturn]] void fail_no_device(const std::string& msg);
void check_hip(hipError_t err, const char* what);

// ---------------------------------------------------------------------------------------
// Host copy of an lg_view (TensorView, src/abi.rs:64-76).
// ---------------------------------------------------------------------------------------
struct View {
    uintptr_t base = 0;
    uint64_t bytes = 0;
    uint64_t offset = 0;
    std::vector<uint64_t> shape;
    std::vector<uint64_t> strides;

    size_t rank() const { return shape.size(); }
    bool is_empty() const;
    // Product of extents; fails InvalidArgument on overflow.
    uint64_t len() const;
};

View view_from_c(const lg_view* v, const char* name);
void view_to_c(const View& v, lg_view* out);
// TensorView::validate (src/abi.rs:140-177).
void validate(const View& v, uint32_t elem_bytes);
// One past the last reachable element, or false for an empty view (element_range).
bool element_range(const View& v, uint64_t* first, uint64_t* end_exclusive);
// TensorView::may_overlap (src/abi.rs:193-204).
bool may_overlap(const View& a, uint32_t ea, const View& b, uint32_t eb);
std::vector<uint64_t> row_major_strides(const std::vector<uint64_t>& shape);
std::string fmt_vec(const std::vector<uint64_t>& v);

// ---------------------------------------------------------------------------------------
// Context: one device, one default stream, a launch log.
// ---------------------------------------------------------------------------------------
struct Context {
    int device = 0;
    hipStream_t stream = nullptr;
    std::atomic<uint64_t> launches{0};
    std::atomic<const char*> names[256];
    // The MSE reduction's scratch (partials, ticket counter, loss) and the pinned host word
    // the loss is read back into; made on first use, freed with the context. mse_grad holds
    // mse_lock from its launch until the loss is back, so concurrent calls take turns.
    std::mutex mse_lock;
    void* mse_scratch = nullptr;
    float* mse_host = nullptr;
    // Split-K and split-dot partials: one buffer per context, SCRATCH_BYTES long, allocated
    // with the context and never grown, so a split call never allocates or synchronizes --
    // also under stream capture. split_lock is held while
    // a call hands the buffer to its launches. Calls on one stream are ordered by the stream;
    // an eager call on another stream first waits for split_event, which marks the end of the
    // previous user's work.
    std::mutex split_lock;
    void* split_scratch = nullptr;
    hipStream_t split_stream = nullptr;  // stream of the last eager call that used the buffer
    hipEvent_t split_event = nullptr;
};
void note_launch(Context* ctx, const char* name);
void set_last_error(const std::string& msg);
void clear_last_error();

// Runs `body`, translating failures into a status and the thread's last-error message.
template <typename F>
lg_status guarded(F&& body) {
    try {
        body();
        clear_last_error();
        return LG_OK;
    } catch (const Failure& f) {
        set_last_error(f.message);
        return f.status;
    } catch (const std::bad_alloc&) {
        set_last_error("host allocation failed");
        return LG_KERNEL;
    } catch (const std::exception& e) {
        // Nothing may unwind through the C ABI; a library exception is an internal failure.
        set_last_error(std::string("internal error: ") + e.what());
        return LG_KERNEL;
    } catch (...) {
        set_last_error("internal error: unknown exception");
        return LG_KERNEL;
    }
}

// ---------------------------------------------------------------------------------------
// Contraction kernels
// ---------------------------------------------------------------------------------------
enum LoadMode : int { LOAD_K = 0, LOAD_MN = 1, LOAD_S = 2 };

// Tile geometry of the MFMA GEMM kernel: 128x128 output tiles, or 64x64 (GEMM_SMALL_TILE)
// when the 128x128 grid, even split along K, has fewer than GEMM_SMALL_BELOW workgroups.
constexpr uint32_t GEMM_BM = 128;
constexpr uint32_t GEMM_BN = 128;
#ifndef LG_GEMM_SMALL_BELOW
#define LG_GEMM_SMALL_BELOW 256
#endif
constexpr uint32_t GEMM_SMALL_TILE = 64;
constexpr uint64_t GEMM_SMALL_BELOW = LG_GEMM_SMALL_BELOW;
// Products whose 64x64 grid is under GEMM_SMALL_BELOW tiles and whose K is at most
// GEMM_SMALL_K take the single-launch 32x32 kernel (gemm_f32_small) instead of split-K.
#ifndef LG_GEMM_SMALL_K
#define LG_GEMM_SMALL_K 1024
#endif
constexpr uint32_t GEMM_TINY_TILE = 32;
constexpr uint32_t GEMM_SMALL_K = LG_GEMM_SMALL_K;
constexpr uint32_t GEMM_BK = 16;       // K-slice depth per LDS stage
constexpr uint32_t GEMM_THREADS = 256;

// Kernels of the tiled plan.
enum GemmKernel : uint32_t {
    KERN_TILE = 0,   // gemm_f32_mfma: 128x128 (or 64x64) tile per 256-thread workgroup
    KERN_SMALL = 1,  // gemm_f32_small: one 32x32 tile per workgroup, sixteen waves split K
    KERN_WAVE = 2,   // gemm_f32_wave: one 32x32 tile per wave, four tiles per workgroup
    KERN_OUTER = 3,  // outer_f32: K <= OUTER_MAX_K on the VALU, four outputs per thread
    KERN_DIRECT = 4, // gemm_f32_dl: 128x128 or 128x256 tiles, slices loaded straight into LDS
    KERN_PIPE = 5,   // gemm_f32_pl (full 128x128 tiles) / gemm_f32_kw (full 64x64 tiles): software-pipelined direct loads
    KERN_SK = 6      // gemm_f32_sk: stream-K over full 128x128 tiles, one workgroup per compute unit
};
// N extent of the wide direct-load tile (eight waves, 128x256).
constexpr uint32_t GEMM_WIDE_N = 256;
// KERN_PIPE: K chunks are whole multiples of four slices of `slice_k` (16: two workgroups per
// compute unit; 32: one), on 128x128 tiles; on 64x64 tiles four waves each take a quarter of
// every chunk (K chunks in whole multiples of 4 * PIPE_STAGES * 16).
constexpr uint32_t PIPE_STAGES = 4;
constexpr uint32_t PIPE_KW = 4;  // waves splitting K on 64x64 tiles
// gemm_f32_kw's slices and stages: two stages of 32-deep slices per wave, so a K chunk is a
// whole number of KW_STEP (each of the PIPE_KW waves takes whole pairs of slices).
constexpr uint32_t KW_BK = 32;
constexpr uint32_t KW_STAGES = 2;
constexpr uint32_t KW_STEP = PIPE_KW * KW_STAGES * KW_BK;
constexpr uint32_t PIPE_NARROW_N = 64;  // N extent of the 128x64 pipelined tile
constexpr uint32_t PIPE_TALL_M = 256;   // M extent of the 256x128 pipelined tile (gemm_f32_pl256)
constexpr uint32_t PIPE_WIDE_N = 256;   // N extent of the 256x256 pipelined tile (gemm_f32_pl2x)
constexpr uint32_t PIPE_DEEP_K = 4096;  // (K, K) chunks from this long take 32-deep slices
constexpr uint32_t OUTER_MAX_K = 8;

struct GemmArgs {
    const float* a;  // element pointer of A's view offset
    const float* b;
    float* c;
    float* partial;  // split-K partials [batch][splits][m][n], or null; KERN_SK: 2G tile slots
    int64_t a_sb, a_sm, a_sk;
    int64_t b_sb, b_sn, b_sk;
    int64_t c_sb, c_sm, c_sn;
    uint32_t m, n, k, batch;
    uint32_t k_chunk, splits;
    uint32_t tiles_m, tiles_n;
    float alpha, beta;
    uint32_t tile;     // output tile edge along M: 128, 64 or 32 (1 for KERN_OUTER)
    uint32_t tile_n;   // along N: `tile`, or GEMM_WIDE_N for the wide direct-load tile
    uint32_t kernel;   // GemmKernel
    // 0: alpha scales the A-role operand as it is loaded; 1: the B-role one. The planner swaps
    // the operands (C^T = B^T.A^T) when C is contiguous along M, and the operand it then
    // loads as B is the caller's A: every product stays (alpha*a)*b.
    uint32_t scale_b;
    // KERN_OUTER: 1 when C is contiguous along N, n % 4 == 0 and every row 16-byte aligned
    // (128-bit stores), and (vec_b) the same for B (128-bit loads).
    uint32_t vec_c, vec_b;
    // KERN_DIRECT: wave groups per workgroup that take the tile's K slices in halves and add
    // their sums in group order at the end (1 or 2).
    uint32_t kgroups;
    // KERN_PIPE: K depth of one LDS slice, 16 or 32.
    uint32_t slice_k;
    uint32_t* counters;  // KERN_SK: one ticket counter per range boundary, zero between launches
};

// Dot products (M = N = 1): C[b] = beta*C[b] + sum_k (alpha*a[b][k])*b[b][k]. Split along K
// into `splits` workgroups per product writing partial sums, which a second launch adds in
// split order.
struct DotArgs {
    const float* a;
    const float* b;
    float* c;
    float* partial;     // [batch][splits] when splits > 1
    int64_t a_sb, a_sk, b_sb, b_sk, c_sb;
    uint32_t k, batch, k_chunk, splits;
    float alpha, beta;
    uint32_t scale_b;
};
constexpr uint32_t DOT_THREADS = 256;
constexpr uint32_t DOT_MIN_CHUNK = 4096;   // K elements per split, at least
constexpr uint32_t DOT_TARGET = 2048;      // workgroups the split dot path aims for

// The per-context scratch of split partials. Plans never need more than SPLIT_PARTIAL_MAX
// bytes of partials (the planner caps the split count to fit).
constexpr uint64_t SPLIT_PARTIAL_MAX = 32ull << 20;
// Stream-K (KERN_SK): SK_RANGES workgroups, one per compute unit of the part (a constant, so
// plans and results depend on the shape alone); 2 * SK_RANGES partial slots of a 128x128 tile
// fill SPLIT_PARTIAL_MAX exactly. Its ticket counters follow the partials in the scratch,
// zeroed when the scratch is made and cleared again by every launch that uses them.
constexpr uint32_t SK_RANGES = 256;
constexpr uint64_t SK_PARTIAL_BYTES = 2ull * SK_RANGES * 128 * 128 * sizeof(float);
static_assert(SK_PARTIAL_BYTES <= SPLIT_PARTIAL_MAX, "stream-K slots fit the partials");
constexpr uint64_t SK_COUNTER_BYTES = 4096;
static_assert(SK_COUNTER_BYTES >= SK_RANGES * sizeof(uint32_t), "one counter per boundary");
constexpr uint64_t SCRATCH_BYTES = SPLIT_PARTIAL_MAX + SK_COUNTER_BYTES;

struct ReduceArgs {
    const float* partial;
    float* c;
    int64_t c_sb, c_sm, c_sn;
    uint32_t m, n, batch, splits;
    float beta;
    uint32_t slices;  // waves that split the split range of each output: 4 or 16
};

// Right-aligned mixed radix of up to 4 axes (slot 3 fastest); unused slots have extent 1.
struct Axes4 {
    uint32_t ext[4];
    int64_t stride[4];
};

struct GeneralArgs {
    const float* a;
    const float* b;
    float* c;
    uint32_t m, n, k, batch;
    float alpha, beta;
    Axes4 a_batch, a_m, a_k, b_batch, b_n, b_k, c_batch, c_m, c_n;
};

struct FillArgs {
    float* c;
    uint64_t count;
    uint32_t m, n, batch;
    float beta;
    Axes4 c_batch, c_m, c_n;
};

// f16 contraction (half operands as raw 16-bit patterns): products of halves are exact in
// f64, sums run in f64 on the f64 matrix cores, and each output rounds once to f16.
constexpr int HGEMM_BM = 64, HGEMM_BN = 64, HGEMM_BK = 64;
struct GemmHalfArgs {
    const uint16_t* a;
    const uint16_t* b;
    uint16_t* c;
    int64_t a_sb, a_sm, a_sk, b_sb, b_sn, b_sk, c_sb, c_sm, c_sn;
    uint32_t m, n, k, batch, tiles_m, tiles_n;
    float alpha, beta;
};
struct GeneralHalfArgs {
    const uint16_t* a;
    const uint16_t* b;
    uint16_t* c;
    uint32_t m, n, k, batch;
    float alpha, beta;
    Axes4 a_batch, a_m, a_k, b_batch, b_n, b_k, c_batch, c_m, c_n;
};
struct FillHalfArgs {
    uint16_t* c;
    uint64_t count;
    uint32_t m, n, batch;
    float beta;
    Axes4 c_batch, c_m, c_n;
};
// The Backend's 16-bit gemm with CpuBackend's f32 arithmetic (one lane per output, k in
// order, one rounding per multiply and add, one 16-bit rounding at the end). Operands are 2-D
// with element strides; C's column stride is 1. *_kfast: the operand's K stride is 1.
struct Gemm16SeqArgs {
    const uint16_t* a;
    const uint16_t* b;
    uint16_t* c;
    int64_t a_sm, a_sk, b_sk, b_sn, c_sm;
    uint32_t m, n, k, tiles_m, tiles_n;
    float alpha, beta;
    uint32_t kind;  // 0 = f16, 1 = bf16
    uint32_t a_kfast, b_kfast;
    uint32_t tile;  // square output tile: 128, or 64 where 128x128 tiles would not fill two
                    // workgroups per compute unit (fewer than 2 * GEMM16_SEQ_CUS tiles)
};
constexpr uint32_t GEMM16_SEQ_TILE = 128;
constexpr uint32_t GEMM16_SEQ_CUS = 256;  // compute units of the part
void launch_gemm16_seq(Context* ctx, hipStream_t s, const Gemm16SeqArgs& args);
uint64_t gemm16_seq_workgroups(uint32_t m, uint32_t n, uint32_t tile);

void launch_gemm_half(Context* ctx, hipStream_t s, const GemmHalfArgs& args, int a_mode,
                      int b_mode);
void launch_general_half(Context* ctx, hipStream_t s, const GeneralHalfArgs& args);
void launch_fill_half(Context* ctx, hipStream_t s, const FillHalfArgs& args);
uint64_t gemm_half_workgroups(uint32_t m, uint32_t n, uint32_t batch);

void launch_gemm(Context* ctx, hipStream_t s, const GemmArgs& args, int a_mode, int b_mode);
void launch_reduce(Context* ctx, hipStream_t s, const ReduceArgs& args);
// The dot kernel, then (split dots) the ordered sum of the partials.
void launch_dot(Context* ctx, hipStream_t s, const DotArgs& args, bool vec);
void launch_general(Context* ctx, hipStream_t s, const GeneralArgs& args);
void launch_fill(Context* ctx, hipStream_t s, const FillArgs& args);
uint64_t gemm_workgroups(const GemmArgs& args);

// ---------------------------------------------------------------------------------------
// Permutation kernels
// ---------------------------------------------------------------------------------------
constexpr uint32_t PERM_MAX_RANK = 8;  // MAX_RANK, src/ops/permutation.rs:14-16
constexpr uint32_t PERM_TILE_A = 64;   // transpose tile extent along a (source unit stride)
constexpr uint32_t PERM_TILE_B = 64;   // transpose tile extent along b (destination unit stride)
// Streaming configuration, used when source + destination exceed the 256 MiB Infinity Cache
// (nothing of the operands survives in cache between uses, so accesses are non-temporal):
// 64 x 256 tiles of 1024 threads, so each destination row segment a tile writes is 1 KiB, as
// long as one wave's 128-bit store.
constexpr uint32_t PERM_STREAM_TILE_A = 64;
constexpr uint32_t PERM_STREAM_TILE_B = 256;
constexpr uint32_t PERM_STREAM_THREADS = 1024;
constexpr uint64_t PERM_STREAM_BYTES = 256ull << 20;
constexpr uint32_t PERM_THREADS = 256;         // copy kernel
constexpr uint32_t PERM_CACHED_THREADS = 512;  // transpose tiles that stay in the cache

struct PermTileArgs {
    const void* src;  // allocation bases
    void* dst;
    uint64_t src_offset, dst_offset;  // elements
    uint32_t ext_a, ext_b;            // a: source unit-stride axis; b: destination unit-stride axis
    int64_t src_sb, dst_sa;           // source stride of b, destination stride of a
    uint32_t outer_rank;
    uint32_t tiles_a, tiles_b;
    uint64_t total_tiles;
    uint32_t outer_shape[PERM_MAX_RANK];
    int64_t outer_src[PERM_MAX_RANK];
    int64_t outer_dst[PERM_MAX_RANK];
};

struct PermCopyArgs {
    const void* src;
    void* dst;
    uint64_t src_offset, dst_offset, count;
    uint32_t rank;
    uint32_t contiguous;  // rank 1, unit stride, aligned: straight vector copy
    uint32_t vec_dst;     // destination offset aligned for 128-bit stores
    uint32_t streaming;   // non-temporal 128-bit accesses
    uint64_t shape[PERM_MAX_RANK];
    int64_t strides[PERM_MAX_RANK];
};

// words: 1 (4-byte elements) or 2 (8-byte complex); conj flips the imaginary sign bit.
void launch_perm_tile(Context* ctx, hipStream_t s, const PermTileArgs& args, int words, bool conj,
                      bool vec, bool streaming);
void launch_perm_copy(Context* ctx, hipStream_t s, const PermCopyArgs& args, int words, bool conj);
uint64_t perm_copy_workgroups(uint64_t count, int words);
uint64_t perm_tile_workgroups(uint64_t total_tiles);

}  // namespace lg

namespace lg {
// Backend training-op kernels (training_kernels.hip). Operands are dense, offset 0, n > 0.
constexpr uint64_t MSE_MAX_GROUPS = 256;   // workgroups of the MSE reduction, at most
constexpr uint64_t MSE_MIN_CHUNK = 4096;   // elements per MSE workgroup, at least
uint64_t mse_groups(uint64_t n, uint64_t* chunk);
void launch_gelu(Context* ctx, hipStream_t s, const float* x, float* y, uint64_t n);
void launch_gelu_backward(Context* ctx, hipStream_t s, const float* pre, const float* dy,
                          float* dx, uint64_t n);
void launch_add_bias(Context* ctx, hipStream_t s, const float* x, const float* b, float* y,
                     uint64_t rows, uint64_t cols);
void launch_bias_grad(Context* ctx, hipStream_t s, const float* dpre, float* db, uint32_t rows,
                      uint32_t cols);
// partial: mse_groups(n) floats; counter: one zeroed uint32; loss: one float (all device).
void launch_mse_grad(Context* ctx, hipStream_t s, const float* y, const float* target, float* dy,
                     uint64_t n, float* partial, uint32_t* counter, float* loss);
void launch_sgd_step(Context* ctx, hipStream_t s, float* w, float* dw, float lr, uint64_t n);
void launch_convert(Context* ctx, hipStream_t s, bool to_bf16, const void* x, void* y, uint64_t n);
}  // namespace lg

struct lg_ctx : lg::Context {};

namespace lg {
void set_device(const lg_ctx* ctx);
// Plans and enqueues the f32 matrix product C = alpha*A.B + beta*C on views whose ranges
// the caller has already checked (the gemm form of the contraction planner; alias rules and
// the scalar rules apply, views are not re-validated).
void enqueue_gemm_views(lg_ctx* ctx, hipStream_t s, float alpha, const View& a, const View& b,
                        float beta, const View& c);
// Plans C = alpha*A.B + beta*C (the gemm form, f32) and enqueues it on `stream` with device
// scratch from the caller: once validation and planning have passed, and only when the plan
// needs scratch, `scratch(ctx)` is called with the context's device current and returns
// `partial_cap` bytes of device memory for split partials. A plan needing more than
// partial_cap fails with InvalidArgument before anything is launched.
void enqueue_gemm_fixed_scratch(lg_ctx* ctx, void* stream, float alpha, const lg_view* a,
                                const lg_view* b, float beta, const lg_view* c,
                                uint64_t partial_cap, float* (*scratch)(lg_ctx*));
// Looks up the no-allocation entry point's static scratch on the context's device (current
// when called), so its code object is loaded at context creation and never inside a capture.
void noalloc_prepare(lg_ctx* ctx);
inline hipStream_t pick_stream(const lg_ctx* ctx, void* stream) {
    return stream ? static_cast<hipStream_t>(stream) : ctx->stream;
}
}  // namespace lg
