// lg_encode_gemm_f32_noalloc: lg_encode_gemm_f32 for callers that may not allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that forbid it).
//
// Its split-K and split-dot partials live in `scratch`, a file-scope device array of
// SCRATCH_BYTES (32 MiB of partials, the most any plan uses: the planner caps split counts to
// fit, and 4 KiB of stream-K ticket counters, cleared once when the array is looked up), which
// each GPU holds from the first context made on it until the process ends. In host code the
// array's name is only a stand-in: its device address on each GPU is looked up once per device
// with hipGetSymbolAddress, when lg_ctx_create makes the first context there (so the code
// object holding the array is loaded then, never under a later stream capture), and only that
// address is handed to kernels. Every partial is written before it is read within one call, and every
// launch that takes a stream-K ticket leaves its counter at zero again, so nothing needs clearing
// between calls. Every call on one GPU shares that GPU's array, so calls that overlap on one
// GPU (several streams, several contexts, or graph replays running at once) race on it: the
// caller orders them. Nothing here allocates: no hipMalloc, no hipFree, no allocating library
// routine.
#include <hip/hip_runtime.h>

#include <mutex>

#include "lg_internal.h"

namespace lg {
namespace {

static_assert(SCRATCH_BYTES % 256 == 0, "scratch is whole 256-byte granules");
static __device__ __align__(256) float scratch[SCRATCH_BYTES / sizeof(float)];

constexpr int MAX_DEVICES = 64;
std::mutex table_lock;
void* table[MAX_DEVICES] = {};  // device address of `scratch` on each device, once looked up

// The device address of `scratch` on the context's device (current when called), looked up
// the first time.
float* scratch_on(lg_ctx* ctx) {
    const int device = ctx->device;
    if (device < 0 || device >= MAX_DEVICES) fail_invalid("device index beyond the scratch table");
    std::lock_guard<std::mutex> hold(table_lock);
    if (table[device] == nullptr) {
        void* ptr = nullptr;
        check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (ptr == nullptr) fail_kernel("hipGetSymbolAddress(scratch) returned no address");
        // The stream-K ticket counters after the partials start at zero (launches leave them
        // so); cleared here once per device, before any call can use them.
        check_hip(hipMemset(static_cast<char*>(ptr) + SPLIT_PARTIAL_MAX, 0, SK_COUNTER_BYTES),
                  "hipMemset(scratch counters)");
        table[device] = ptr;
    }
    return static_cast<float*>(table[device]);
}

}  // namespace

void noalloc_prepare(lg_ctx* ctx) { (void)scratch_on(ctx); }

}  // namespace lg

using namespace lg;

extern "C" lg_status lg_encode_gemm_f32_noalloc(lg_ctx* ctx, void* stream, float alpha,
                                                const lg_view* a, const lg_view* b, float beta,
                                                const lg_view* c) {
    return guarded([&] {
        if (ctx == nullptr) fail_invalid("null context");
        enqueue_gemm_fixed_scratch(ctx, stream, alpha, a, b, beta, c, SPLIT_PARTIAL_MAX, scratch_on);
    });
}
