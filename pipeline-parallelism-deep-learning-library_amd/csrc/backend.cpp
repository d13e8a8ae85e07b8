// Backend-style gemm: the linalg_core::Backend::gemm contract (crates/core/src/lib.rs:143-164)
// with CpuBackend::gemm's check order and error codes (crates/cpu/src/lib.rs:203-295,
// 606-661), running on the contraction path's MFMA kernels.
//
// Checks, first failure wins, nothing launched on error:
//   Wire              a dtype tag that is not F32, F16 or BF16 (no such Tensor exists)
//   Shape             every operand is rank 2 (shape and strides); inner extents agree
//   Dtype             all three dtypes equal
//   Alias             distinct storage (storage id = allocation base)
//   UnsupportedLayout offset 0; (row-major, row-major, row-major), (transpose_matrix of a
//                     row-major matrix, row-major, row-major) or (row-major, transposed,
//                     row-major), where "transposed" means strides == [1, rows]
//   Shape             C reaches past its storage (when M, N > 0); A or B reach past theirs
//                     (when alpha != 0 and K > 0)
// Then f32 runs on the device; F16 and BF16 report UnsupportedDevice (not built here).
#include "lg_internal.h"

namespace lg {
namespace {

struct TensorErr {
    lg_core_error code;
    std::string message;
};

[[noreturn]] void core_fail(lg_core_error code, const std::string& msg) { throw TensorErr{code, msg}; }

uint64_t dtype_size(uint32_t dtype) {
    switch (dtype) {
        case LG_DTYPE_F32:
            return 4;
        case LG_DTYPE_F16:
        case LG_DTYPE_BF16:
            return 2;
    }
    // DType::from_tag (crates/core/src/lib.rs:25-32): an unknown tag is a wire error.
    core_fail(LG_CORE_WIRE, "unknown dtype tag " + std::to_string(dtype));
}

// matrix_dims (crates/cpu/src/lib.rs:606-611).
void matrix_dims(const lg_tensor* t, uint64_t* rows, uint64_t* cols, const char* name) {
    if (t->rank != 2 || t->nstrides != 2) core_fail(LG_CORE_SHAPE, std::string(name) + " is not rank 2");
    *rows = t->shape[0];
    *cols = t->shape[1];
}

enum class Layout { RowMajor, Transposed };

// matrix_layout (crates/cpu/src/lib.rs:619-631).
Layout matrix_layout(const lg_tensor* t) {
    if (t->offset != 0) core_fail(LG_CORE_UNSUPPORTED_LAYOUT, "offset must be 0");
    const std::vector<uint64_t> rm = row_major_strides({t->shape[0], t->shape[1]});
    if (t->strides[0] == rm[0] && t->strides[1] == rm[1]) return Layout::RowMajor;
    if (t->strides[0] == 1 && t->strides[1] == t->shape[0]) return Layout::Transposed;
    core_fail(LG_CORE_UNSUPPORTED_LAYOUT, "strides are neither row-major nor a transposed row-major");
}

// corner + require_range (crates/cpu/src/lib.rs:633-649).
void require_range(const lg_tensor* t, uint64_t rows, uint64_t cols, uint64_t size, const char* name) {
    uint64_t last = 0;
    if (rows != 0 && cols != 0) {
        const uint64_t s0 = t->strides[0], s1 = t->strides[1];
        if ((s0 != 0 && rows - 1 > UINT64_MAX / s0) || (s1 != 0 && cols - 1 > UINT64_MAX / s1)) {
            core_fail(LG_CORE_SHAPE, std::string(name) + " index overflows");
        }
        const uint64_t r = (rows - 1) * s0, c = (cols - 1) * s1;
        if (r > UINT64_MAX - c || r + c > UINT64_MAX - t->offset) {
            core_fail(LG_CORE_SHAPE, std::string(name) + " index overflows");
        }
        last = t->offset + r + c;
    }
    if (last == UINT64_MAX || last + 1 > UINT64_MAX / size) core_fail(LG_CORE_SHAPE, std::string(name) + " index overflows");
    if ((last + 1) * size > t->bytes) {
        core_fail(LG_CORE_SHAPE, std::string(name) + " reaches past its storage");
    }
}

View to_view(const lg_tensor* t) {
    View v;
    v.base = reinterpret_cast<uintptr_t>(t->base);
    v.bytes = t->bytes;
    v.offset = t->offset;
    v.shape = {t->shape[0], t->shape[1]};
    v.strides = {t->strides[0], t->strides[1]};
    return v;
}

}  // namespace
}  // namespace lg

using namespace lg;

extern "C" lg_core_error lg_backend_gemm(lg_ctx* ctx, void* stream, const lg_tensor* a,
                                         const lg_tensor* b, const lg_tensor* c, float alpha,
                                         float beta) {
    try {
        if (a == nullptr || b == nullptr || c == nullptr) core_fail(LG_CORE_SHAPE, "null tensor");
        for (const lg_tensor* t : {a, b, c}) dtype_size(t->dtype);  // decodable tags only
        uint64_t m, k, kb, n, mc, nc;
        matrix_dims(a, &m, &k, "a");
        matrix_dims(b, &kb, &n, "b");
        matrix_dims(c, &mc, &nc, "c");
        if (k != kb || m != mc || n != nc) core_fail(LG_CORE_SHAPE, "extents of a, b and c disagree");
        if (a->dtype != b->dtype || a->dtype != c->dtype) core_fail(LG_CORE_DTYPE, "dtypes differ");
        const uint64_t size = dtype_size(a->dtype);
        if (a->base == b->base || a->base == c->base || b->base == c->base) {
            core_fail(LG_CORE_ALIAS, "a, b and c must have distinct storage");
        }
        const Layout la = matrix_layout(a), lb = matrix_layout(b), lc = matrix_layout(c);
        const bool supported = lc == Layout::RowMajor &&
                               !(la == Layout::Transposed && lb == Layout::Transposed);
        if (!supported) core_fail(LG_CORE_UNSUPPORTED_LAYOUT, "unsupported layout combination");
        if (m > 0 && n > 0) {
            require_range(c, m, n, size, "c");
            if (alpha != 0.0f && k > 0) {
                require_range(a, m, k, size, "a");
                require_range(b, k, n, size, "b");
            }
        }
        if (a->dtype != LG_DTYPE_F32) {
            core_fail(LG_CORE_UNSUPPORTED_DEVICE, "only f32 gemm runs on the HIP backend");
        }
        if (ctx == nullptr) core_fail(LG_CORE_UNSUPPORTED_DEVICE, "null context");
        if (m == 0 || n == 0) {
            clear_last_error();
            return LG_CORE_OK;
        }
        const lg_status st = guarded([&] {
            enqueue_gemm_views(ctx, pick_stream(ctx, stream), alpha, to_view(a), to_view(b), beta,
                               to_view(c));
        });
        if (st != LG_OK) return LG_CORE_UNSUPPORTED_DEVICE;  // launch failure; message kept
        return LG_CORE_OK;
    } catch (const TensorErr& e) {
        set_last_error(e.message);
        return e.code;
    } catch (const Failure& f) {
        set_last_error(f.message);
        return LG_CORE_UNSUPPORTED_DEVICE;
    }
}
