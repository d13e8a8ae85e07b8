/*
 * linalg_hip.h — C ABI of the MI355X (gfx950) tensor-contraction and permutation backend.
 *
 * This is the drop-in boundary for the reference's L1 operator surface
 * (`linalg::ops::contraction`, `linalg::ops::permutation`) and its L0 data model
 * (`linalg::abi`). Every entry point below names the reference item it replaces
 * (paths relative to the reference repository root).
 *
 * Conventions
 *  - Plain C types only: pointers, fixed-width integers, floats. No HIP or torch types;
 *    streams travel as `void*` (a `hipStream_t`), NULL meaning the context's own stream.
 *  - Views are in ELEMENTS: the element at multi-index idx lives at element
 *    `offset + sum(idx[d] * strides[d])` counted from `base`, exactly as
 *    `TensorView` (src/abi.rs:64-76). `base` is always the allocation base returned by
 *    lg_alloc (never an offset-adjusted pointer) and `bytes` its length, which play the
 *    roles of `buffer.contents()` and `buffer.length()`.
 *  - Every call validates everything first. On any error it launches nothing and writes
 *    nothing, returns a non-zero lg_status, and lg_last_error() describes the failure
 *    (src/ops/contraction.rs:1024-1035, src/ops/permutation.rs:163-198). Nothing aborts
 *    on bad metadata.
 *  - `lg_encode_*` only enqueue on the given stream (the reference's `encode_*` into a
 *    command buffer); the un-prefixed forms enqueue on the context stream and wait for
 *    completion (the reference's synchronous `contract`, `gemm`, `materialize`, ...).
 *    Enqueue order on one stream is execution order.
 *  - Thread safety: calls on different streams may run concurrently. As in
 *    crates/core/src/lib.rs:67-70, the caller must not let two in-flight calls write
 *    overlapping memory.
 *  - Split scratch: every split-K and split-dot plan (lg_contract_plan.scratch_bytes > 0)
 *    of one context shares that context's one scratch buffer. Eager calls are ordered on it
 *    by the library (stream order, or an event when the stream changes). A call recorded
 *    under stream capture is ordered only by its own stream: replays of that graph must not
 *    overlap one another or any other split call on the same context, whatever the stream
 *    (the caller orders them, or gives each concurrent stream its own context).
 */
#ifndef LINALG_HIP_H
#define LINALG_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Largest rank a view may carry. The reference's TensorView holds a Vec of any length;
 * 16 is far beyond every caller of the hot path. */
#define LG_MAX_RANK 16
/* Allocation granularity of lg_alloc, as ALLOC_GRANULE (src/abi.rs:221-223). */
#define LG_ALLOC_GRANULE 16384u

/* Status codes: LinalgError (src/abi.rs:20-33). */
typedef enum lg_status {
    LG_OK = 0,
    LG_NO_DEVICE = 1,        /* LinalgError::NoDevice */
    LG_INVALID_ARGUMENT = 2, /* LinalgError::InvalidArgument */
    LG_OVERLAP = 3,          /* LinalgError::Overlap */
    LG_KERNEL = 4            /* LinalgError::ShaderCompile: code-object, launch or runtime failure */
} lg_status;

/* Element types the permutation kernels move as raw bits
 * (permutation::Element, src/ops/permutation.rs:26-54). Contraction is f32-only here. */
typedef enum lg_elem {
    LG_ELEM_F32 = 0, /* one 32-bit word */
    LG_ELEM_U32 = 1, /* one 32-bit word */
    LG_ELEM_I32 = 2, /* one 32-bit word */
    LG_ELEM_C32 = 3  /* complex f32 [re, im]: two words; conjugation flips the sign bit of im */
} lg_elem;

/* A strided window into one allocation (TensorView, src/abi.rs:64-76).
 * `rank` entries of `shape` and `nstrides` entries of `strides` are meaningful; they must be
 * equal for the view to validate (the reference's "rank mismatch" check). */
typedef struct lg_view {
    void* base;                      /* allocation base (device memory) */
    uint64_t bytes;                  /* allocation length in bytes */
    uint64_t offset;                 /* in elements */
    uint32_t rank;                   /* number of axes in `shape` */
    uint32_t nstrides;               /* number of entries in `strides` */
    uint64_t shape[LG_MAX_RANK];     /* extents */
    uint64_t strides[LG_MAX_RANK];   /* in elements */
} lg_view;

/* ---------------------------------------------------------------------------------------
 * Errors
 * ------------------------------------------------------------------------------------- */

/* Message of the last failing call on this thread ("" if none). The LinalgError payload
 * (src/abi.rs:24-43). Valid until the next call on the same thread. */
const char* lg_last_error(void);

/* ---------------------------------------------------------------------------------------
 * Context and memory (src/abi.rs:51-62, 221-243)
 * ------------------------------------------------------------------------------------- */

typedef struct lg_ctx lg_ctx;

/* Opens HIP device `device` and creates one stream on it: MetalContext::new
 * (src/abi.rs:55-61). LG_NO_DEVICE when no such device exists. */
lg_status lg_ctx_create(int32_t device, lg_ctx** out);
/* Waits for the context stream, then releases it. NULL is ignored. */
void lg_ctx_destroy(lg_ctx* ctx);
/* The context's hipStream_t (MetalContext::queue). */
void* lg_ctx_stream(const lg_ctx* ctx);
/* Blocks until all work enqueued on the context stream has completed
 * (`wait_until_completed`, src/ops/contraction.rs:1015-1022). */
lg_status lg_ctx_sync(lg_ctx* ctx);
/* Blocks until all work on `stream` (a hipStream_t; NULL = context stream) has completed. */
lg_status lg_stream_sync(lg_ctx* ctx, void* stream);
/* A new stream on the context's device: the analogue of `queue.new_command_buffer()`
 * that the reference's `encode_*` calls fill (src/ops/contraction.rs:1057-1063). Work
 * enqueued on it starts without an explicit commit. */
lg_status lg_stream_create(lg_ctx* ctx, void** stream);
/* Waits for `stream` and destroys it. */
lg_status lg_stream_destroy(lg_ctx* ctx, void* stream);

/* Zero-filled device allocation holding at least `len` elements of `elem_bytes` bytes,
 * rounded up to whole LG_ALLOC_GRANULE granules (at least one, so len = 0 is legal):
 * alloc_shared (src/abi.rs:225-243). MI355X memory is not host-visible, so contents move
 * with lg_upload / lg_download. */
lg_status lg_alloc(lg_ctx* ctx, uint64_t elem_bytes, uint64_t len, void** base, uint64_t* bytes);
/* Frees an lg_alloc allocation after the context stream has drained. */
lg_status lg_free(lg_ctx* ctx, void* base);
/* Host -> device copy of `nbytes` at byte offset `byte_offset` of allocation `base`,
 * ordered after all earlier work on the context stream; returns once complete. */
lg_status lg_upload(lg_ctx* ctx, void* base, uint64_t byte_offset, const void* src, uint64_t nbytes);
/* Device -> host copy, ordered after all earlier work on the context stream. */
lg_status lg_download(lg_ctx* ctx, const void* base, uint64_t byte_offset, void* dst, uint64_t nbytes);

/* ---------------------------------------------------------------------------------------
 * View metadata (host only, no device work)
 * ------------------------------------------------------------------------------------- */

/* TensorView::validate (src/abi.rs:140-177) for elements of `elem_bytes` bytes. */
lg_status lg_view_validate(const lg_view* view, uint32_t elem_bytes);
/* TensorView::may_overlap (src/abi.rs:193-204): 1 when both views live in the same
 * allocation and their byte ranges intersect, else 0. Views must have validated. */
int32_t lg_view_may_overlap(const lg_view* a, uint32_t a_elem_bytes, const lg_view* b,
                            uint32_t b_elem_bytes);

/* ---------------------------------------------------------------------------------------
 * Permutation (src/ops/permutation.rs:272-387)
 * ------------------------------------------------------------------------------------- */

/* permute_view (src/ops/permutation.rs:295-320): axis i of *out is axis perm[i] of *view.
 * Metadata only. LG_INVALID_ARGUMENT unless perm is a permutation of 0..rank. */
lg_status lg_permute_view(const lg_view* view, const uint64_t* perm, uint32_t perm_len,
                          lg_view* out);

/* encode_materialize / materialize (src/ops/permutation.rs:322-342): copies `src` (any
 * strided view) into the contiguous row-major `dst` of the same shape, bit for bit. */
lg_status lg_encode_materialize(lg_ctx* ctx, void* stream, lg_elem elem, const lg_view* src,
                                const lg_view* dst);
lg_status lg_materialize(lg_ctx* ctx, lg_elem elem, const lg_view* src, const lg_view* dst);

/* encode_conjugate / conjugate (src/ops/permutation.rs:344-369): as materialize, flipping
 * the sign bit of the imaginary word of complex elements (a plain copy for real types). */
lg_status lg_encode_conjugate(lg_ctx* ctx, void* stream, lg_elem elem, const lg_view* src,
                              const lg_view* dst);
lg_status lg_conjugate(lg_ctx* ctx, lg_elem elem, const lg_view* src, const lg_view* dst);

/* encode_adjoint / adjoint (src/ops/permutation.rs:371-387): swaps the last two axes of
 * `src` (rank >= 2) and conjugates complex elements into the row-major `dst`. */
lg_status lg_encode_adjoint(lg_ctx* ctx, void* stream, lg_elem elem, const lg_view* src,
                            const lg_view* dst);
lg_status lg_adjoint(lg_ctx* ctx, lg_elem elem, const lg_view* src, const lg_view* dst);

/* ---------------------------------------------------------------------------------------
 * Contraction (src/ops/contraction.rs:1024-1130), f32
 * ------------------------------------------------------------------------------------- */

/* encode_contract / contract (src/ops/contraction.rs:1036-1064):
 *   C = alpha * A.B + beta * C over einsum labels (one ASCII byte per axis).
 * A label in A and B but not C is contracted; A and C: an M axis; B and C: an N axis; all
 * three: a batch axis. beta = 0 never reads C, alpha = 0 never reads A or B, K = 0 gives
 * C = beta * C, an empty M, N or batch launches nothing. LG_OVERLAP when C aliases an input
 * it reads or writes an element twice (the in-place scale with the other extents 1 is
 * allowed). Split plans use the context's shared scratch: under stream capture see
 * "Split scratch" above. */
lg_status lg_encode_contract_f32(lg_ctx* ctx, void* stream, float alpha, const lg_view* a,
                                 const char* a_labels, const lg_view* b, const char* b_labels,
                                 float beta, const lg_view* c, const char* c_labels);
lg_status lg_contract_f32(lg_ctx* ctx, float alpha, const lg_view* a, const char* a_labels,
                          const lg_view* b, const char* b_labels, float beta, const lg_view* c,
                          const char* c_labels);

/* encode_gemm / gemm / gemm_nowait (src/ops/contraction.rs:1066-1130): batched matrix form.
 * Equal ranks r >= 2; leading r-2 axes are batch; A[..., M, K], B[..., K, N], C[..., M, N].
 * Strides may describe transposes or windows; nothing is copied. gemm_nowait enqueues on
 * the context stream and returns without waiting. Split plans use the context's shared
 * scratch: under stream capture see "Split scratch" above. */
lg_status lg_encode_gemm_f32(lg_ctx* ctx, void* stream, float alpha, const lg_view* a,
                             const lg_view* b, float beta, const lg_view* c);
lg_status lg_gemm_f32(lg_ctx* ctx, float alpha, const lg_view* a, const lg_view* b, float beta,
                      const lg_view* c);
lg_status lg_gemm_nowait_f32(lg_ctx* ctx, float alpha, const lg_view* a, const lg_view* b,
                             float beta, const lg_view* c);

/* No counterpart in the reference: lg_encode_gemm_f32 for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid allocation).
 * Same arguments, validation, plans and results as lg_encode_gemm_f32. It allocates nothing:
 * split-K, split-dot and stream-K partials live in a static device array of 32 MiB (plus
 * 4 KiB of stream-K ticket counters) that each GPU holds from the first lg_ctx_create on it
 * until the process ends (no plan needs more; a product that did would fail with
 * LG_INVALID_ARGUMENT before launching anything). Every call on one GPU shares that GPU's
 * array, so calls that overlap on one GPU race on it and must be ordered by the caller (one
 * stream, or events). */
lg_status lg_encode_gemm_f32_noalloc(lg_ctx* ctx, void* stream, float alpha, const lg_view* a,
                                     const lg_view* b, float beta, const lg_view* c);

/* The same five entry points for half operands: contract / gemm / gemm_nowait instantiated at
 * `T = half::f16` (src/ops/contraction.rs:22-32,147-162,1036-1130). Views are in f16
 * elements (2 bytes, 2-byte aligned base); alpha and beta stay f32. Validation, label and
 * alias rules are the f32 ones. Each output is the exact-product dot rounded ONCE to f16:
 * products of halves are exact in f64 and summed in f64 (the reference sums them in
 * double-float f32 and rounds once, shaders/contraction.metal:444-678); alpha*acc and beta*C
 * add in f64 and round to nearest even. beta*C alone (alpha = 0 or K = 0) is the exact product
 * rounded once (contract_scale_f16, shaders/contraction.metal:730-756). */
lg_status lg_encode_contract_f16(lg_ctx* ctx, void* stream, float alpha, const lg_view* a,
                                 const char* a_labels, const lg_view* b, const char* b_labels,
                                 float beta, const lg_view* c, const char* c_labels);
lg_status lg_contract_f16(lg_ctx* ctx, float alpha, const lg_view* a, const char* a_labels,
                          const lg_view* b, const char* b_labels, float beta, const lg_view* c,
                          const char* c_labels);
lg_status lg_encode_gemm_f16(lg_ctx* ctx, void* stream, float alpha, const lg_view* a,
                             const lg_view* b, float beta, const lg_view* c);
lg_status lg_gemm_f16(lg_ctx* ctx, float alpha, const lg_view* a, const lg_view* b, float beta,
                      const lg_view* c);
lg_status lg_gemm_nowait_f16(lg_ctx* ctx, float alpha, const lg_view* a, const lg_view* b,
                             float beta, const lg_view* c);

/* ---------------------------------------------------------------------------------------
 * Backend-style gemm: linalg_core::Backend::gemm (crates/core/src/lib.rs:143-164)
 * ------------------------------------------------------------------------------------- */

/* core::Error (crates/core/src/lib.rs:43-53). */
typedef enum lg_core_error {
    LG_CORE_OK = 0,
    LG_CORE_SHAPE = 1,
    LG_CORE_DTYPE = 2,
    LG_CORE_UNSUPPORTED_LAYOUT = 3,
    LG_CORE_UNSUPPORTED_DEVICE = 4,
    LG_CORE_ALIAS = 5,
    LG_CORE_TRANSPORT = 6,
    LG_CORE_WIRE = 7,
    LG_CORE_SCHEDULE = 8
} lg_core_error;

/* DType wire tags (crates/core/src/lib.rs:18-24). */
typedef enum lg_dtype { LG_DTYPE_F32 = 1, LG_DTYPE_F16 = 2, LG_DTYPE_BF16 = 3 } lg_dtype;

/* core::Tensor<S> (crates/core/src/lib.rs:55-61): one storage allocation (its base pointer is
 * the storage id) plus dtype, shape, strides and offset in elements. */
typedef struct lg_tensor {
    void* base;                      /* storage allocation base (device memory) */
    uint64_t bytes;                  /* storage length in bytes */
    uint32_t dtype;                  /* lg_dtype */
    uint32_t rank;                   /* entries of `shape` */
    uint32_t nstrides;               /* entries of `strides` */
    uint32_t reserved;
    uint64_t offset;                 /* in elements */
    uint64_t shape[LG_MAX_RANK];
    uint64_t strides[LG_MAX_RANK];
} lg_tensor;

/* Backend::gemm as CpuBackend::gemm checks it (crates/cpu/src/lib.rs:203-295): `a` is [M, K],
 * `b` [K, N], `c` [M, N]; a dtype tag outside lg_dtype is LG_CORE_WIRE (DType::from_tag,
 * crates/core/src/lib.rs:25-32); then checks in order Shape (rank 2, inner extents), Dtype
 * (all equal), Alias (distinct storage), UnsupportedLayout (offset 0; all row-major, or A or
 * B a transpose_matrix of a row-major matrix with C row-major), then Shape again for every
 * operand that is read reaching past its storage. Stores beta*C + alpha*A*B (beta = 0 does
 * not read C, alpha = 0 does not read A or B, K = 0 with beta = 0 stores zeros); every
 * product is (alpha*a)*b, as in the reference's loop, summed in the kernel's fixed order.
 * F16 and BF16 operands return CpuBackend::gemm's bits (crates/cpu/src/lib.rs:270-291 with
 * `accumulate`, :664-691): per output, acc = beta*C in f32 (0 when beta is 0), then
 * acc = acc + (alpha*a)*b in k order, every multiply and add rounded to f32, stored rounded
 * to the 16-bit type to nearest even (the half crate's from_f32_const); only NaN payloads may
 * differ. This runs on the vector ALUs (one lane per output), not the matrix cores, whose
 * summation order is their own. The checks run before `ctx` is used.
 * Enqueues on `stream` (NULL = context stream) and returns before the device finishes, as
 * the GPU backends do (crates/core/src/lib.rs:72-82). On any error nothing is launched. */
lg_core_error lg_backend_gemm(lg_ctx* ctx, void* stream, const lg_tensor* a, const lg_tensor* b,
                              const lg_tensor* c, float alpha, float beta);

/* The Backend trait's activation and training ops (crates/core/src/lib.rs:165-255), each with
 * CpuBackend's check order and error codes (crates/cpu/src/lib.rs:297-533) and one kernel
 * launch. Every check runs before `ctx` is used, and on any error nothing is launched or
 * written. A dtype tag outside lg_dtype is LG_CORE_WIRE. Operands are row-major contiguous at
 * offset 0 (else LG_CORE_UNSUPPORTED_LAYOUT) whose storage holds all their bytes (else
 * LG_CORE_SHAPE). Each formula is evaluated as written, one rounding per operation; empty
 * operands launch nothing. All but mse_grad enqueue on `stream` (NULL = context stream) and
 * return before the device finishes. */

/* gelu (crates/cpu/src/lib.rs:297-307): y = 0.5*x*(1 + erf(x/sqrt 2)), erf by Abramowitz &
 * Stegun 7.1.26 in f32 as the reference evaluates it. Checks: Dtype (all f32), Shape (equal
 * shapes), layout, storage. y may be x. */
lg_core_error lg_backend_gelu(lg_ctx* ctx, void* stream, const lg_tensor* x, const lg_tensor* y);

/* gelu_backward (crates/cpu/src/lib.rs:309-326): dx = dy * (Phi(pre) + pre*phi(pre)).
 * Checks as gelu over (pre, dy, dx). */
lg_core_error lg_backend_gelu_backward(lg_ctx* ctx, void* stream, const lg_tensor* pre,
                                       const lg_tensor* dy, const lg_tensor* dx);

/* add_bias (crates/cpu/src/lib.rs:372-401): y[i][j] = x[i][j] + b[j]; x, y [B, N], b [N].
 * Checks: Shape, Dtype, Alias (b distinct from x and y; y may be x), layout, storage. */
lg_core_error lg_backend_add_bias(lg_ctx* ctx, void* stream, const lg_tensor* x,
                                  const lg_tensor* b, const lg_tensor* y);

/* bias_grad (crates/cpu/src/lib.rs:403-435): db[j] = db[j] + (dpre[0][j] + dpre[1][j] + ...),
 * rows summed in order as the reference does, so the result is the reference's bits.
 * Checks: Shape (dpre [B, N], db [N]), Dtype, Alias, layout, storage; B, N < 2^31. */
lg_core_error lg_backend_bias_grad(lg_ctx* ctx, void* stream, const lg_tensor* dpre,
                                   const lg_tensor* db);

/* mse_grad (crates/cpu/src/lib.rs:437-472): d = y - target, dy = (2*d)/n, *loss = (sum of
 * d*d)/n with n rounded to f32. The loss sums in a fixed order that depends only on n (the
 * contract leaves the order to the backend). Checks: Shape (equal shapes, n > 0), Dtype,
 * Alias (dy distinct from target; dy may be y, y may share target's storage), layout,
 * storage. Waits for every earlier call and this one before returning; *loss is unchanged on
 * error. */
lg_core_error lg_backend_mse_grad(lg_ctx* ctx, void* stream, const lg_tensor* y,
                                  const lg_tensor* target, const lg_tensor* dy, float* loss);

/* sgd_step (crates/cpu/src/lib.rs:474-501): w = w - (lr*dw), then dw = +0. Checks: Shape,
 * Dtype, Alias (distinct storage), layout, storage. */
lg_core_error lg_backend_sgd_step(lg_ctx* ctx, void* stream, const lg_tensor* w,
                                  const lg_tensor* dw, float lr);

/* convert (crates/cpu/src/lib.rs:503-533,725-732): F32 -> BF16 nearest, ties to even (NaN
 * stays a quiet NaN of the same sign, overflow to infinity, subnormals kept); BF16 -> F32
 * exact. Checks: Shape, Dtype ((F32, BF16) or (BF16, F32)), Alias, layout, storage. */
lg_core_error lg_backend_convert(lg_ctx* ctx, void* stream, const lg_tensor* x,
                                 const lg_tensor* y);

/* Backend::download_into and Backend::upload_into (crates/core/src/lib.rs:118-133, as
 * CpuBackend checks them at crates/cpu/src/lib.rs:328-370): a tensor's row-major bytes into
 * caller memory, or caller bytes over every element of an existing tensor, allocating
 * nothing. Checks in order: decodable tensor, byte count equal to the tensor's (else Shape),
 * row-major at offset 0 (else UnsupportedLayout), storage holding the bytes (else Shape).
 * Both copy on `stream` (NULL = context stream) after every earlier call there and return
 * when the copy is done: `out` holds the bytes, and `bytes` may be reused. */
lg_core_error lg_backend_download_into(lg_ctx* ctx, void* stream, const lg_tensor* t,
                                       uint8_t* out, uint64_t out_len);
lg_core_error lg_backend_upload_into(lg_ctx* ctx, void* stream, const uint8_t* bytes,
                                     uint64_t len, const lg_tensor* t);

/* ---------------------------------------------------------------------------------------
 * Wire format of stage boundaries (crates/core/src/lib.rs:298-412)
 *
 * "LNGL", u32 version 1, u32 dtype tag, u32 ndim (at most 8), ndim u32 extents, then the
 * row-major payload; little-endian. A malformed message, more than 8 extents or an
 * undecodable tag is LG_CORE_WIRE; an extent above u32::MAX or an overflowing byte count is
 * LG_CORE_SHAPE. On error nothing is written.
 * ------------------------------------------------------------------------------------- */

#define LG_WIRE_HEADER_MAX 48 /* WIRE_HEADER_MAX: 16 + 4 * 8 */

/* write_wire_header (crates/core/src/lib.rs:328-335): writes 16 + 4*rank bytes to `out`. */
lg_core_error lg_wire_write_header(uint32_t dtype, const uint64_t* shape, uint32_t rank,
                                   uint8_t out[LG_WIRE_HEADER_MAX], uint64_t* len);
/* parse_wire_header (crates/core/src/lib.rs:361-389): the payload is bytes[*payload_offset..]
 * and its length has been checked against the shape. */
lg_core_error lg_wire_parse_header(const uint8_t* bytes, uint64_t len, uint32_t* dtype,
                                   uint64_t shape[8], uint32_t* rank, uint64_t* payload_offset);
/* encode_wire (crates/core/src/lib.rs:309-322) into a caller buffer of `out_cap` bytes (too
 * small: LG_CORE_SHAPE); a payload of the wrong length is LG_CORE_WIRE. */
lg_core_error lg_wire_encode(uint32_t dtype, const uint64_t* shape, uint32_t rank,
                             const void* payload, uint64_t payload_len, uint8_t* out,
                             uint64_t out_cap, uint64_t* written);
/* send_tensor's download + encode_wire (crates/pipeline/src/lib.rs:71-80) in one device-to-host
 * copy straight into the wire buffer: after every earlier call on the context stream, returns
 * when the bytes are final. Checks in the reference's order: the dtype tag (LG_CORE_WIRE);
 * download's (crates/cpu/src/lib.rs:183-194): row-major strides at any offset (else
 * LG_CORE_UNSUPPORTED_LAYOUT), the byte range inside the storage (else LG_CORE_SHAPE); then
 * encode_wire's header checks (rank above 8: LG_CORE_WIRE; extent above u32::MAX: LG_CORE_SHAPE);
 * `out_cap` too small: LG_CORE_SHAPE. Host-memory rate; no kernel runs. */
lg_core_error lg_wire_encode_tensor(lg_ctx* ctx, const lg_tensor* t, uint8_t* out,
                                    uint64_t out_cap, uint64_t* written);
/* recv_tensor's decode_wire + upload (crates/pipeline/src/lib.rs:82-98) into an existing tensor
 * (Backend::upload_into's rules, crates/core/src/lib.rs:127-134): the message's dtype must be
 * the tensor's (else LG_CORE_DTYPE) and its shape the tensor's (else LG_CORE_SHAPE); one
 * host-to-device copy; `bytes` may be reused once this returns. */
lg_core_error lg_wire_decode_into(lg_ctx* ctx, const uint8_t* bytes, uint64_t len,
                                  const lg_tensor* t);

/* ---------------------------------------------------------------------------------------
 * Plan inspection (host only; no context, no device work). These run the exact
 * validation and planning of the entry points above and report the plan instead of
 * launching it, so the planner is testable without a GPU.
 * ------------------------------------------------------------------------------------- */

/* Plan kinds of a contraction (Plan, src/ops/contraction.rs:664-675). */
typedef enum lg_plan_kind {
    LG_PLAN_EMPTY = 0,   /* nothing to do */
    LG_PLAN_ZERO = 1,    /* Fill with beta = 0: C = 0 without reading C */
    LG_PLAN_SCALE = 2,   /* Fill with beta != 0: C = beta * C */
    LG_PLAN_TILED = 3,   /* one MFMA GEMM launch */
    LG_PLAN_SPLIT = 4,   /* split-K MFMA partials + ordered reduction */
    LG_PLAN_GENERAL = 5, /* mixed-radix fallback (more than one stride per group) */
    LG_PLAN_DOT = 6      /* M = N = 1: VALU dot products, split along K with ordered partials */
} lg_plan_kind;

/* Kernel of a tiled, split or dot plan. */
typedef enum lg_plan_kernel {
    LG_KERNEL_NONE = 0,  /* empty, fill or general plans */
    LG_KERNEL_TILE = 1,  /* 128x128 (or 64x64) output tile per 256-thread workgroup */
    LG_KERNEL_SMALL = 2, /* one 32x32 tile per workgroup, sixteen waves splitting its K */
    LG_KERNEL_WAVE = 3,  /* one 32x32 tile per wave (batches of small products) */
    LG_KERNEL_DOT = 4,   /* one dot product (chunk) per workgroup */
    LG_KERNEL_OUTER = 5, /* K <= 8: four outputs per thread on the VALU, summed in k order */
    LG_KERNEL_DIRECT = 6, /* 128x128 or 128x256 tile, operand slices loaded straight into LDS */
    LG_KERNEL_PIPELINED = 7, /* full tiles, direct loads, software-pipelined waves: 128x128,
                                128x64, 64x64 (K split over the waves), and with A contiguous
                                along K 256x128 or 256x256 tiles of eight waves */
    LG_KERNEL_STREAMK = 8   /* full 128x128 tiles spread unevenly over the compute units: one
                               workgroup per compute unit takes an equal run of the pipelined
                               kernel's K steps across tiles; a tile two runs share is summed by
                               the run finishing second (scratch_bytes of the context's scratch) */
} lg_plan_kernel;

/* Operand load modes of the tiled kernel. */
typedef enum lg_load_mode {
    LG_LOAD_K_CONTIG = 0,  /* unit stride along K: 128-bit loads along K */
    LG_LOAD_MN_CONTIG = 1, /* unit stride along M (A) or N (B): 128-bit loads along M/N */
    LG_LOAD_STRIDED = 2    /* neither, or misaligned: 32-bit predicated loads */
} lg_load_mode;

typedef struct lg_contract_plan {
    uint32_t kind;        /* lg_plan_kind */
    uint32_t a_mode;      /* lg_load_mode of A (tiled/split) */
    uint32_t b_mode;      /* lg_load_mode of B (tiled/split) */
    uint32_t groups;      /* max number of strides in any merged group */
    uint64_t batch, m, n, k;
    uint64_t splits;      /* 1 unless LG_PLAN_SPLIT */
    uint64_t k_chunk;     /* K elements per split */
    uint64_t workgroups;  /* workgroups of the main launch */
    uint64_t scratch_bytes; /* device scratch of the split-K partials */
    uint32_t tile_m;      /* output tile of one workgroup or wave (tiled/split): 128x128 on */
    uint32_t tile_n;      /* the pipelined kernel (full tiles, at least 512 workgroups; with A
                             contiguous along K 256x128, or 256x256 where at least 256 of
                             those fill the output), else
                             128x256 for grids of at least 512 such tiles, else 128x128; 64x64
                             when 128x128 tiles would leave most compute units idle or be
                             mostly padding;
                             32x32 for small outputs (sixteen waves per tile splitting K) and
                             batches of small products (one tile per wave); 1x1 for dot
                             products, 1x4 for K <= 8; f16: 64x64 */
    uint32_t kernel;      /* lg_plan_kernel */
    uint32_t swapped;     /* 1 when C is contiguous along M and is computed as C^T = B^T.A^T */
    uint32_t kgroups;     /* LG_KERNEL_DIRECT: wave groups per workgroup splitting the tile's K
                             slices when the grid leaves at most one workgroup per compute unit
                             (2 for 128x128 tiles, 4 for 64x64); LG_KERNEL_PIPELINED on 64x64
                             tiles: 4 (each wave takes a quarter of every K chunk); else 1 */
    uint32_t reserved;
} lg_contract_plan;

lg_status lg_plan_contract_f32(float alpha, const lg_view* a, const char* a_labels,
                               const lg_view* b, const char* b_labels, float beta,
                               const lg_view* c, const char* c_labels, lg_contract_plan* out);
lg_status lg_plan_gemm_f32(float alpha, const lg_view* a, const lg_view* b, float beta,
                           const lg_view* c, lg_contract_plan* out);
/* The plans of the f16 entry points: kinds EMPTY, ZERO, SCALE, TILED (the f64 matrix-core
 * tile kernel, a 64x64 tile per workgroup, 16-bit strided loads) or GENERAL. */
lg_status lg_plan_contract_f16(float alpha, const lg_view* a, const char* a_labels,
                               const lg_view* b, const char* b_labels, float beta,
                               const lg_view* c, const char* c_labels, lg_contract_plan* out);
lg_status lg_plan_gemm_f16(float alpha, const lg_view* a, const lg_view* b, float beta,
                           const lg_view* c, lg_contract_plan* out);

/* Permutation plan (encode_gather's path choice, src/ops/permutation.rs:200-268). */
typedef enum lg_permute_kind {
    LG_PERMUTE_EMPTY = 0, /* nothing to move */
    LG_PERMUTE_COPY = 1,  /* gather with contiguous 128-bit writes */
    LG_PERMUTE_TILE = 2   /* LDS-tiled 2-axis transpose, 128-bit reads and writes */
} lg_permute_kind;

typedef struct lg_permute_plan {
    uint32_t kind;          /* lg_permute_kind */
    uint32_t rank;          /* rank after coalescing */
    uint32_t axis_a;        /* tile: source unit-stride axis */
    uint32_t axis_b;        /* tile: destination unit-stride axis (rank - 1) */
    uint32_t vector;        /* 1 when the 128-bit path is legal (alignment) */
    uint32_t conj;          /* 1 when the imaginary sign bit is flipped */
    uint32_t streaming;     /* 1 when accesses are non-temporal (operands exceed the cache) */
    uint32_t reserved;
    uint64_t shape[8];      /* coalesced extents */
    uint64_t strides[8];    /* coalesced source strides */
    uint64_t workgroups;    /* workgroups of the launch */
} lg_permute_plan;

/* `op`: 0 materialize, 1 conjugate, 2 adjoint. */
lg_status lg_plan_permute(uint32_t op, lg_elem elem, const lg_view* src, const lg_view* dst,
                          lg_permute_plan* out);

/* ---------------------------------------------------------------------------------------
 * Debug counters (the reference's debug launch log, crates/cpu/src/lib.rs:79-148)
 * ------------------------------------------------------------------------------------- */

/* Number of kernels this context has launched. */
uint64_t lg_debug_launch_count(const lg_ctx* ctx);
/* Name of launch `i` counted from 0, for the last 256 launches; NULL if out of range. */
const char* lg_debug_launch_name(const lg_ctx* ctx, uint64_t i);

#ifdef __cplusplus
}
#endif

#endif /* LINALG_HIP_H */
