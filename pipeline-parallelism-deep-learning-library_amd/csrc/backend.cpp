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

// ---- training-op checks (crates/cpu/src/lib.rs:297-533,595-604,731-807) ----------------

// Every tensor handed in: non-null, a decodable dtype tag, rank and stride count that fit.
void decode(std::initializer_list<const lg_tensor*> ts) {
    for (const lg_tensor* t : ts) {
        if (t == nullptr) core_fail(LG_CORE_SHAPE, "null tensor");
        if (t->rank > LG_MAX_RANK || t->nstrides > LG_MAX_RANK) {
            core_fail(LG_CORE_SHAPE, "rank above LG_MAX_RANK");
        }
    }
    for (const lg_tensor* t : ts) dtype_size(t->dtype);
}

bool same_shape(const lg_tensor* a, const lg_tensor* b) {
    if (a->rank != b->rank) return false;
    for (uint32_t d = 0; d < a->rank; ++d) {
        if (a->shape[d] != b->shape[d]) return false;
    }
    return true;
}

// numel with overflow as Shape (numel, crates/cpu/src/lib.rs:595-601).
uint64_t numel(const lg_tensor* t) {
    uint64_t n = 1;
    for (uint32_t d = 0; d < t->rank; ++d) {
        if (t->shape[d] != 0 && n > UINT64_MAX / t->shape[d]) core_fail(LG_CORE_SHAPE, "element count overflows");
        n *= t->shape[d];
    }
    return n;
}

uint64_t nbytes(const lg_tensor* t) {
    const uint64_t n = numel(t), size = dtype_size(t->dtype);
    if (n > UINT64_MAX / size) core_fail(LG_CORE_SHAPE, "byte count overflows");
    return n * size;
}

// packed_layout (crates/cpu/src/lib.rs:731-744): offset 0, row-major strides.
bool packed_layout(const lg_tensor* t) {
    if (t->offset != 0 || t->nstrides != t->rank) return false;
    uint64_t stride = 1;
    for (uint32_t d = t->rank; d-- > 0;) {
        if (t->strides[d] != stride) return false;
        stride *= t->shape[d];  // wraps like the reference's wrapping_mul
    }
    return true;
}

void all_f32(std::initializer_list<const lg_tensor*> ts) {
    for (const lg_tensor* t : ts) {
        if (t->dtype != LG_DTYPE_F32) core_fail(LG_CORE_DTYPE, "operand is not f32");
    }
}

// packed (crates/cpu/src/lib.rs:769-781): layout first, then each storage holds its bytes.
void packed(std::initializer_list<const lg_tensor*> ts) {
    for (const lg_tensor* t : ts) {
        if (!packed_layout(t)) core_fail(LG_CORE_UNSUPPORTED_LAYOUT, "operand is not row-major contiguous at offset 0");
    }
    for (const lg_tensor* t : ts) {
        if (nbytes(t) > t->bytes) core_fail(LG_CORE_SHAPE, "operand reaches past its storage");
    }
}

// prepare_f32_row_major (crates/cpu/src/lib.rs:783-807): Dtype, Shape, layout, storage.
uint64_t prepare_f32_row_major(std::initializer_list<const lg_tensor*> ts) {
    all_f32(ts);
    const lg_tensor* first = *ts.begin();
    for (const lg_tensor* t : ts) {
        if (!same_shape(t, first)) core_fail(LG_CORE_SHAPE, "shapes differ");
    }
    for (const lg_tensor* t : ts) {
        if (t->offset != 0 || t->nstrides != t->rank) {
            core_fail(LG_CORE_UNSUPPORTED_LAYOUT, "operand is not row-major contiguous at offset 0");
        }
        uint64_t stride = 1;
        for (uint32_t d = t->rank; d-- > 0;) {
            if (t->strides[d] != stride) {
                core_fail(LG_CORE_UNSUPPORTED_LAYOUT, "operand is not row-major contiguous at offset 0");
            }
            stride *= t->shape[d];
        }
    }
    const uint64_t count = numel(first);
    if (count > UINT64_MAX / 4) core_fail(LG_CORE_SHAPE, "byte count overflows");
    for (const lg_tensor* t : ts) {
        if (t->bytes < count * 4) core_fail(LG_CORE_SHAPE, "operand reaches past its storage");
    }
    return count;
}

// Runs `body` (checks, then launches) with the entry points' error mapping: check failures
// return their code; device failures return UnsupportedDevice with the HIP message.
template <typename F>
lg_core_error run_op(F&& body) {
    try {
        body();
        clear_last_error();
        return LG_CORE_OK;
    } catch (const TensorErr& e) {
        set_last_error(e.message);
        return e.code;
    } catch (const Failure& f) {
        set_last_error(f.message);
        return LG_CORE_UNSUPPORTED_DEVICE;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return LG_CORE_UNSUPPORTED_DEVICE;
    } catch (...) {
        set_last_error("internal error: unknown exception");
        return LG_CORE_UNSUPPORTED_DEVICE;
    }
}

hipStream_t device_stream(lg_ctx* ctx, void* stream) {
    if (ctx == nullptr) core_fail(LG_CORE_UNSUPPORTED_DEVICE, "null context");
    set_device(ctx);
    return pick_stream(ctx, stream);
}

template <typename T>
T* dev(const lg_tensor* t) {
    return static_cast<T*>(t->base);
}

}  // namespace
}  // namespace lg

using namespace lg;

extern "C" {

lg_core_error lg_backend_gelu(lg_ctx* ctx, void* stream, const lg_tensor* x, const lg_tensor* y) {
    return run_op([&] {
        decode({x, y});
        const uint64_t n = prepare_f32_row_major({x, y});
        hipStream_t s = device_stream(ctx, stream);
        if (n > 0) launch_gelu(ctx, s, dev<const float>(x), dev<float>(y), n);
    });
}

lg_core_error lg_backend_gelu_backward(lg_ctx* ctx, void* stream, const lg_tensor* pre,
                                       const lg_tensor* dy, const lg_tensor* dx) {
    return run_op([&] {
        decode({pre, dy, dx});
        const uint64_t n = prepare_f32_row_major({pre, dy, dx});
        hipStream_t s = device_stream(ctx, stream);
        if (n > 0) launch_gelu_backward(ctx, s, dev<const float>(pre), dev<const float>(dy), dev<float>(dx), n);
    });
}

lg_core_error lg_backend_add_bias(lg_ctx* ctx, void* stream, const lg_tensor* x,
                                  const lg_tensor* b, const lg_tensor* y) {
    return run_op([&] {
        decode({x, b, y});
        // bias_shapes (crates/cpu/src/lib.rs:746-757).
        if (x->rank != 2 || !same_shape(y, x) || b->rank != 1 || b->shape[0] != x->shape[1]) {
            core_fail(LG_CORE_SHAPE, "add_bias needs x [B, N], b [N], y [B, N]");
        }
        all_f32({x, b, y});
        if (b->base == x->base || b->base == y->base) core_fail(LG_CORE_ALIAS, "b shares storage with x or y");
        packed({x, b, y});
        hipStream_t s = device_stream(ctx, stream);
        const uint64_t rows = x->shape[0], cols = x->shape[1];
        if (rows > 0 && cols > 0) launch_add_bias(ctx, s, dev<const float>(x), dev<const float>(b), dev<float>(y), rows, cols);
    });
}

lg_core_error lg_backend_bias_grad(lg_ctx* ctx, void* stream, const lg_tensor* dpre,
                                   const lg_tensor* db) {
    return run_op([&] {
        decode({dpre, db});
        if (dpre->rank != 2 || db->rank != 1 || db->shape[0] != dpre->shape[1]) {
            core_fail(LG_CORE_SHAPE, "bias_grad needs dpre [B, N] and db [N]");
        }
        all_f32({dpre, db});
        if (dpre->base == db->base) core_fail(LG_CORE_ALIAS, "db shares storage with dpre");
        packed({dpre, db});
        const uint64_t rows = dpre->shape[0], cols = dpre->shape[1];
        // The kernel walks rows in blocks with 32-bit arithmetic (rows + block - 1 must not
        // wrap): extents are 31-bit.
        if (rows > 0x7fffffffull || cols > 0x7fffffffull) {
            core_fail(LG_CORE_SHAPE, "bias_grad extents must fit 31 bits");
        }
        hipStream_t s = device_stream(ctx, stream);
        if (rows > 0 && cols > 0) {
            launch_bias_grad(ctx, s, dev<const float>(dpre), dev<float>(db), static_cast<uint32_t>(rows),
                             static_cast<uint32_t>(cols));
        }
    });
}

lg_core_error lg_backend_mse_grad(lg_ctx* ctx, void* stream, const lg_tensor* y,
                                  const lg_tensor* target, const lg_tensor* dy, float* loss) {
    return run_op([&] {
        decode({y, target, dy});
        if (!same_shape(target, y) || !same_shape(dy, y)) core_fail(LG_CORE_SHAPE, "shapes differ");
        const uint64_t n = numel(y);
        if (n == 0) core_fail(LG_CORE_SHAPE, "mse_grad of zero elements");
        all_f32({y, target, dy});
        if (dy->base == target->base) core_fail(LG_CORE_ALIAS, "dy shares storage with target");
        packed({y, target, dy});
        if (loss == nullptr) core_fail(LG_CORE_SHAPE, "null loss pointer");
        hipStream_t s = device_stream(ctx, stream);
        std::lock_guard<std::mutex> hold(ctx->mse_lock);
        // Scratch: partial[MSE_MAX_GROUPS], then the counter, then the loss.
        if (ctx->mse_scratch == nullptr) {
            check_hip(hipMalloc(&ctx->mse_scratch, (MSE_MAX_GROUPS + 2) * sizeof(float)), "hipMalloc");
        }
        if (ctx->mse_host == nullptr) {
            check_hip(hipHostMalloc(reinterpret_cast<void**>(&ctx->mse_host), sizeof(float)), "hipHostMalloc");
        }
        float* partial = static_cast<float*>(ctx->mse_scratch);
        uint32_t* counter = reinterpret_cast<uint32_t*>(partial + MSE_MAX_GROUPS);
        float* dloss = partial + MSE_MAX_GROUPS + 1;
        check_hip(hipMemsetAsync(counter, 0, sizeof(uint32_t), s), "hipMemsetAsync");
        launch_mse_grad(ctx, s, dev<const float>(y), dev<const float>(target), dev<float>(dy), n,
                        partial, counter, dloss);
        check_hip(hipMemcpyAsync(ctx->mse_host, dloss, sizeof(float), hipMemcpyDeviceToHost, s),
                  "hipMemcpyAsync");
        check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
        const float host = *ctx->mse_host;
        *loss = host;  // final: every earlier call and this one have completed
    });
}

lg_core_error lg_backend_download_into(lg_ctx* ctx, void* stream, const lg_tensor* t,
                                       uint8_t* out, uint64_t out_len) {
    return run_op([&] {
        decode({t});
        const uint64_t len = nbytes(t);
        if (out_len != len) core_fail(LG_CORE_SHAPE, "output length differs from the tensor's bytes");
        if (!packed_layout(t)) core_fail(LG_CORE_UNSUPPORTED_LAYOUT, "tensor is not row-major at offset 0");
        if (len > t->bytes) core_fail(LG_CORE_SHAPE, "tensor reaches past its storage");
        if (len != 0 && out == nullptr) core_fail(LG_CORE_SHAPE, "null output");
        hipStream_t s = device_stream(ctx, stream);
        // After every earlier call on the stream; `out` holds the bytes when this returns.
        if (len) check_hip(hipMemcpyAsync(out, t->base, len, hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
        check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
    });
}

lg_core_error lg_backend_upload_into(lg_ctx* ctx, void* stream, const uint8_t* bytes,
                                     uint64_t len, const lg_tensor* t) {
    return run_op([&] {
        decode({t});
        const uint64_t need = nbytes(t);
        if (len != need) core_fail(LG_CORE_SHAPE, "byte count differs from the tensor's bytes");
        if (!packed_layout(t)) core_fail(LG_CORE_UNSUPPORTED_LAYOUT, "tensor is not row-major at offset 0");
        if (need > t->bytes) core_fail(LG_CORE_SHAPE, "tensor reaches past its storage");
        if (need != 0 && bytes == nullptr) core_fail(LG_CORE_SHAPE, "null bytes");
        hipStream_t s = device_stream(ctx, stream);
        // Ordered after every earlier call and before every later one on the stream; `bytes`
        // may be reused as soon as this returns.
        if (need) {
            check_hip(hipMemcpyAsync(t->base, bytes, need, hipMemcpyHostToDevice, s), "hipMemcpyAsync");
        }
        check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
    });
}

lg_core_error lg_backend_sgd_step(lg_ctx* ctx, void* stream, const lg_tensor* w,
                                  const lg_tensor* dw, float lr) {
    return run_op([&] {
        decode({w, dw});
        if (!same_shape(dw, w)) core_fail(LG_CORE_SHAPE, "shapes differ");
        const uint64_t n = numel(w);
        all_f32({w, dw});
        if (w->base == dw->base) core_fail(LG_CORE_ALIAS, "w and dw share storage");
        packed({w, dw});
        hipStream_t s = device_stream(ctx, stream);
        if (n > 0) launch_sgd_step(ctx, s, dev<float>(w), dev<float>(dw), lr, n);
    });
}

lg_core_error lg_backend_convert(lg_ctx* ctx, void* stream, const lg_tensor* x, const lg_tensor* y) {
    return run_op([&] {
        decode({x, y});
        if (!same_shape(y, x)) core_fail(LG_CORE_SHAPE, "shapes differ");
        const uint64_t n = numel(x);
        const bool to_bf16 = x->dtype == LG_DTYPE_F32 && y->dtype == LG_DTYPE_BF16;
        const bool to_f32 = x->dtype == LG_DTYPE_BF16 && y->dtype == LG_DTYPE_F32;
        if (!to_bf16 && !to_f32) core_fail(LG_CORE_DTYPE, "convert needs (F32, BF16) or (BF16, F32)");
        if (x->base == y->base) core_fail(LG_CORE_ALIAS, "x and y share storage");
        packed({x, y});
        hipStream_t s = device_stream(ctx, stream);
        if (n > 0) launch_convert(ctx, s, to_bf16, x->base, y->base, n);
    });
}

}  // extern "C"

// CpuBackend::gemm on F16 / BF16 tensors (crates/cpu/src/lib.rs:270-291): the checked
// row-major or transposed operands, offset 0, handed to the kernel that repeats
// `accumulate`'s f32 arithmetic per output. A and B are not read when alpha or k is 0.
static void enqueue_gemm16(lg_ctx* ctx, hipStream_t s, const lg_tensor* a, const lg_tensor* b,
                           const lg_tensor* c, uint64_t m, uint64_t n, uint64_t k, float alpha,
                           float beta) {
    if (m > UINT32_MAX - GEMM16_SEQ_TILE || n > UINT32_MAX - GEMM16_SEQ_TILE || k > UINT32_MAX) {
        fail_invalid("16-bit gemm extents exceed 2^32 - 129");
    }
    Gemm16SeqArgs g{};
    g.a = static_cast<const uint16_t*>(a->base);
    g.b = static_cast<const uint16_t*>(b->base);
    g.c = static_cast<uint16_t*>(c->base);
    g.a_sm = static_cast<int64_t>(a->strides[0]);
    g.a_sk = static_cast<int64_t>(a->strides[1]);
    g.b_sk = static_cast<int64_t>(b->strides[0]);
    g.b_sn = static_cast<int64_t>(b->strides[1]);
    g.c_sm = static_cast<int64_t>(c->strides[0]);
    g.m = static_cast<uint32_t>(m);
    g.n = static_cast<uint32_t>(n);
    g.k = static_cast<uint32_t>(k);
    g.tile = gemm16_seq_workgroups(g.m, g.n, GEMM16_SEQ_TILE) < 2 * GEMM16_SEQ_CUS ? 64 : GEMM16_SEQ_TILE;
    g.tiles_m = (g.m + g.tile - 1) / g.tile;
    g.tiles_n = (g.n + g.tile - 1) / g.tile;
    g.alpha = alpha;
    g.beta = beta;
    g.kind = a->dtype == LG_DTYPE_BF16 ? 1 : 0;
    g.a_kfast = g.a_sk == 1;
    g.b_kfast = g.b_sk == 1;
    set_device(ctx);
    launch_gemm16_seq(ctx, s, g);
}

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
        if (ctx == nullptr) core_fail(LG_CORE_UNSUPPORTED_DEVICE, "null context");
        if (m == 0 || n == 0) {
            clear_last_error();
            return LG_CORE_OK;
        }
        const lg_status st = guarded([&] {
            if (a->dtype == LG_DTYPE_F32) {
                enqueue_gemm_views(ctx, pick_stream(ctx, stream), alpha, to_view(a), to_view(b),
                                   beta, to_view(c));
            } else {
                enqueue_gemm16(ctx, pick_stream(ctx, stream), a, b, c, m, n, k, alpha, beta);
            }
        });
        if (st != LG_OK) return LG_CORE_UNSUPPORTED_DEVICE;  // launch failure; message kept
        return LG_CORE_OK;
    } catch (const TensorErr& e) {
        set_last_error(e.message);
        return e.code;
    } catch (const Failure& f) {
        set_last_error(f.message);
        return LG_CORE_UNSUPPORTED_DEVICE;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return LG_CORE_UNSUPPORTED_DEVICE;
    } catch (...) {
        set_last_error("internal error: unknown exception");
        return LG_CORE_UNSUPPORTED_DEVICE;
    }
}
