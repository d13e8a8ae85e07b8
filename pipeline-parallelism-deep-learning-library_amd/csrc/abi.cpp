// L0 data model: errors, context, allocation, view validation.
//
// Restates the behaviour of the reference's frozen data model (src/abi.rs) for HIP device
// memory: views are element-strided windows into one allocation; validation checks rank,
// bounds and overflow; overlap is a conservative byte-range test within one allocation.
#include <algorithm>
#include <atomic>
#include <cstring>
#include <memory>
#include <sstream>

#include "lg_internal.h"

namespace lg {

namespace {
thread_local std::string g_last_error;
}

[[noreturn]] void fail_invalid(const std::string& msg) {
    throw Failure{LG_INVALID_ARGUMENT, "invalid argument: " + msg};
}
[[noreturn]] void fail_overlap(const std::string& msg) {
    throw Failure{LG_OVERLAP, "overlapping views: " + msg};
}
[[noreturn]] void fail_kernel(const std::string& msg) {
    throw Failure{LG_KERNEL, "kernel failure: " + msg};
}
[[noreturn]] void fail_no_device(const std::string& msg) {
    throw Failure{LG_NO_DEVICE, "no HIP device available: " + msg};
}

void check_hip(hipError_t err, const char* what) {
    if (err != hipSuccess) {
        fail_kernel(std::string(what) + ": " + hipGetErrorString(err));
    }
}

std::string fmt_vec(const std::vector<uint64_t>& v) {
    std::ostringstream os;
    os << "[";
    for (size_t i = 0; i < v.size(); ++i) os << (i ? ", " : "") << v[i];
    os << "]";
    return os.str();
}

bool View::is_empty() const {
    return std::find(shape.begin(), shape.end(), uint64_t{0}) != shape.end();
}

uint64_t View::len() const {
    uint64_t n = 1;
    for (uint64_t e : shape) {
        if (e != 0 && n > UINT64_MAX / e) fail_invalid("element count overflows");
        n *= e;
    }
    return n;
}

View view_from_c(const lg_view* v, const char* name) {
    if (v == nullptr) fail_invalid(std::string("null view ") + name);
    if (v->rank > LG_MAX_RANK || v->nstrides > LG_MAX_RANK) {
        fail_invalid(std::string(name) + " rank exceeds LG_MAX_RANK");
    }
    View out;
    out.base = reinterpret_cast<uintptr_t>(v->base);
    out.bytes = v->bytes;
    out.offset = v->offset;
    out.shape.assign(v->shape, v->shape + v->rank);
    out.strides.assign(v->strides, v->strides + v->nstrides);
    return out;
}

void view_to_c(const View& v, lg_view* out) {
    std::memset(out, 0, sizeof(*out));
    out->base = reinterpret_cast<void*>(v.base);
    out->bytes = v.bytes;
    out->offset = v.offset;
    out->rank = static_cast<uint32_t>(v.shape.size());
    out->nstrides = static_cast<uint32_t>(v.strides.size());
    std::copy(v.shape.begin(), v.shape.end(), out->shape);
    std::copy(v.strides.begin(), v.strides.end(), out->strides);
}

std::vector<uint64_t> row_major_strides(const std::vector<uint64_t>& shape) {
    std::vector<uint64_t> s(shape.size(), 1);
    for (size_t d = shape.size(); d-- > 1;) s[d - 1] = s[d] * shape[d];
    return s;
}

// Highest reachable element index with checked arithmetic (max_element_index,
// src/abi.rs:206-210). False on overflow. The view must be non-empty.
static bool max_element_index(const View& v, uint64_t* last) {
    uint64_t acc = v.offset;
    for (size_t d = 0; d < v.shape.size(); ++d) {
        const uint64_t n1 = v.shape[d] - 1;
        const uint64_t s = v.strides[d];
        if (s != 0 && n1 > UINT64_MAX / s) return false;
        const uint64_t t = n1 * s;
        if (acc > UINT64_MAX - t) return false;
        acc += t;
    }
    *last = acc;
    return true;
}

void validate(const View& v, uint32_t elem_bytes) {
    if (elem_bytes == 0) fail_invalid("zero-sized element type");
    if (v.shape.size() != v.strides.size()) {
        fail_invalid("rank mismatch: shape " + fmt_vec(v.shape) + " vs strides " +
                     fmt_vec(v.strides));
    }
    if (v.base == 0) fail_invalid("null buffer base");
    // Alignment of the element type: 2 bytes for f16, 4 for f32, u32, i32 and [f32; 2].
    const uint32_t align = elem_bytes < 4 ? elem_bytes : 4;
    if (v.base % align != 0) fail_invalid("buffer base is misaligned for the element type");
    const uint64_t capacity = v.bytes / elem_bytes;
    if (v.is_empty()) {
        if (v.offset <= capacity) return;
        fail_invalid("offset " + std::to_string(v.offset) + " beyond buffer capacity " +
                     std::to_string(capacity));
    }
    uint64_t last = 0;
    if (!max_element_index(v, &last)) {
        fail_invalid("index overflow in view with shape " + fmt_vec(v.shape) + " strides " +
                     fmt_vec(v.strides));
    }
    if (last >= capacity) {
        fail_invalid("view reaches element " + std::to_string(last) + ", buffer holds " +
                     std::to_string(capacity));
    }
}

bool element_range(const View& v, uint64_t* first, uint64_t* end_exclusive) {
    if (v.is_empty()) return false;
    uint64_t last = 0;
    if (!max_element_index(v, &last)) return false;
    *first = v.offset;
    *end_exclusive = last + 1;
    return true;
}

bool may_overlap(const View& a, uint32_t ea, const View& b, uint32_t eb) {
    if (a.base != b.base) return false;
    uint64_t a0, a1, b0, b1;
    if (!element_range(a, &a0, &a1) || !element_range(b, &b0, &b1)) return false;
    // Byte ranges; element indices were validated against the allocation, so these fit.
    const uint64_t as = a0 * ea, ae = a1 * ea, bs = b0 * eb, be = b1 * eb;
    return as < be && bs < ae;
}

void set_last_error(const std::string& msg) { g_last_error = msg; }
void clear_last_error() { g_last_error.clear(); }

void note_launch(Context* ctx, const char* name) {
    if (ctx == nullptr) return;
    const uint64_t i = ctx->launches.fetch_add(1, std::memory_order_relaxed);
    ctx->names[i % 256].store(name, std::memory_order_relaxed);
}

}  // namespace lg

namespace lg {
void set_device(const lg_ctx* ctx) {
    if (ctx == nullptr) fail_invalid("null context");
    check_hip(hipSetDevice(ctx->device), "hipSetDevice");
}
}  // namespace lg

using namespace lg;

extern "C" {

const char* lg_last_error(void) { return g_last_error.c_str(); }

lg_status lg_ctx_create(int32_t device, lg_ctx** out) {
    return guarded([&] {
        if (out == nullptr) fail_invalid("null output pointer");
        *out = nullptr;
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
            (void)hipGetLastError();
            fail_no_device("hipGetDeviceCount reports no device");
        }
        if (device < 0 || device >= count) {
            fail_no_device("device " + std::to_string(device) + " not present");
        }
        check_hip(hipSetDevice(device), "hipSetDevice");
        std::unique_ptr<lg_ctx> ctx(new lg_ctx());
        ctx->device = device;
        for (auto& n : ctx->names) n.store(nullptr);
        noalloc_prepare(ctx.get());  // before anything the context would have to release
        check_hip(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking), "hipStreamCreate");
        // The split partials' scratch, made once here so no enqueue ever allocates (stream
        // capture included).
        void* scratch = nullptr;
        hipError_t err = hipMalloc(&scratch, SCRATCH_BYTES);
        if (err == hipSuccess) err = hipMemset(scratch, 0, SCRATCH_BYTES);  // stream-K counters
        if (err == hipSuccess) err = hipEventCreateWithFlags(&ctx->split_event, hipEventDisableTiming);
        if (err != hipSuccess) {
            if (scratch != nullptr) (void)hipFree(scratch);
            (void)hipStreamDestroy(ctx->stream);
            check_hip(err, "context scratch");
        }
        ctx->split_scratch = scratch;
        *out = ctx.release();
    });
}

void lg_ctx_destroy(lg_ctx* ctx) {
    if (ctx == nullptr) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->mse_scratch != nullptr) (void)hipFree(ctx->mse_scratch);
    if (ctx->mse_host != nullptr) (void)hipHostFree(ctx->mse_host);
    if (ctx->split_stream != nullptr && ctx->split_stream != ctx->stream) {
        (void)hipEventSynchronize(ctx->split_event);  // the last use was on a caller's stream
    }
    if (ctx->split_scratch != nullptr) (void)hipFree(ctx->split_scratch);
    if (ctx->split_event != nullptr) (void)hipEventDestroy(ctx->split_event);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

void* lg_ctx_stream(const lg_ctx* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

lg_status lg_ctx_sync(lg_ctx* ctx) {
    return guarded([&] {
        set_device(ctx);
        check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    });
}

lg_status lg_stream_sync(lg_ctx* ctx, void* stream) {
    return guarded([&] {
        set_device(ctx);
        check_hip(hipStreamSynchronize(pick_stream(ctx, stream)), "hipStreamSynchronize");
    });
}

lg_status lg_stream_create(lg_ctx* ctx, void** stream) {
    return guarded([&] {
        if (stream == nullptr) fail_invalid("null output pointer");
        set_device(ctx);
        hipStream_t s = nullptr;
        check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
        *stream = s;
    });
}

lg_status lg_stream_destroy(lg_ctx* ctx, void* stream) {
    return guarded([&] {
        if (stream == nullptr) fail_invalid("null stream");
        set_device(ctx);
        check_hip(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
        check_hip(hipStreamDestroy(static_cast<hipStream_t>(stream)), "hipStreamDestroy");
    });
}

lg_status lg_alloc(lg_ctx* ctx, uint64_t elem_bytes, uint64_t len, void** base, uint64_t* bytes) {
    return guarded([&] {
        if (base == nullptr || bytes == nullptr) fail_invalid("null output pointer");
        if (elem_bytes != 0 && len > UINT64_MAX / elem_bytes) {
            fail_invalid("alloc: byte length overflows");
        }
        uint64_t n = std::max<uint64_t>(len * elem_bytes, 1);
        if (n > UINT64_MAX - (LG_ALLOC_GRANULE - 1)) fail_invalid("alloc: byte length overflows");
        n = (n + LG_ALLOC_GRANULE - 1) / LG_ALLOC_GRANULE * LG_ALLOC_GRANULE;
        set_device(ctx);
        void* p = nullptr;
        check_hip(hipMalloc(&p, n), "hipMalloc");
        const hipError_t e = hipMemsetAsync(p, 0, n, ctx->stream);
        if (e != hipSuccess) {
            (void)hipFree(p);
            check_hip(e, "hipMemsetAsync");
        }
        check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        *base = p;
        *bytes = n;
    });
}

lg_status lg_free(lg_ctx* ctx, void* base) {
    return guarded([&] {
        set_device(ctx);
        check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        check_hip(hipFree(base), "hipFree");
    });
}

lg_status lg_upload(lg_ctx* ctx, void* base, uint64_t byte_offset, const void* src, uint64_t nbytes) {
    return guarded([&] {
        if (nbytes == 0) return;
        if (base == nullptr || src == nullptr) fail_invalid("null pointer");
        set_device(ctx);
        check_hip(hipMemcpyAsync(static_cast<char*>(base) + byte_offset, src, nbytes,
                                 hipMemcpyHostToDevice, ctx->stream),
                  "hipMemcpyAsync");
        check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    });
}

lg_status lg_download(lg_ctx* ctx, const void* base, uint64_t byte_offset, void* dst, uint64_t nbytes) {
    return guarded([&] {
        if (nbytes == 0) return;
        if (base == nullptr || dst == nullptr) fail_invalid("null pointer");
        set_device(ctx);
        check_hip(hipMemcpyAsync(dst, static_cast<const char*>(base) + byte_offset, nbytes,
                                 hipMemcpyDeviceToHost, ctx->stream),
                  "hipMemcpyAsync");
        check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    });
}

lg_status lg_view_validate(const lg_view* view, uint32_t elem_bytes) {
    return guarded([&] { validate(view_from_c(view, "view"), elem_bytes); });
}

int32_t lg_view_may_overlap(const lg_view* a, uint32_t a_elem_bytes, const lg_view* b,
                            uint32_t b_elem_bytes) {
    int32_t result = 0;
    (void)guarded([&] {
        result = may_overlap(view_from_c(a, "a"), a_elem_bytes, view_from_c(b, "b"), b_elem_bytes)
                     ? 1
                     : 0;
    });
    return result;
}

uint64_t lg_debug_launch_count(const lg_ctx* ctx) {
    return ctx ? ctx->launches.load(std::memory_order_relaxed) : 0;
}

const char* lg_debug_launch_name(const lg_ctx* ctx, uint64_t i) {
    if (ctx == nullptr) return nullptr;
    const uint64_t n = ctx->launches.load(std::memory_order_relaxed);
    if (i >= n || n - i > 256) return nullptr;
    return ctx->names[i % 256].load(std::memory_order_relaxed);
}

}  // extern "C"
