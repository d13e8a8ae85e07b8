//! Raw declarations of include/linalg_hip.h, one for one: every function, struct and constant
//! of the header under the same name, with the same parameters in the same order and the same
//! C types (tests/test_crates_hip_cpu.py checks this against the header). C enums are `i32` /
//! `u32` type aliases of the same name; arrays passed as parameters are pointers.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_void};

pub const LG_MAX_RANK: usize = 16;
pub const LG_ALLOC_GRANULE: u32 = 16384;
pub const LG_WIRE_HEADER_MAX: usize = 48;

pub type lg_status = i32;
pub const LG_OK: lg_status = 0;
pub const LG_NO_DEVICE: lg_status = 1;
pub const LG_INVALID_ARGUMENT: lg_status = 2;
pub const LG_OVERLAP: lg_status = 3;
pub const LG_KERNEL: lg_status = 4;

pub type lg_elem = i32;
pub const LG_ELEM_F32: lg_elem = 0;
pub const LG_ELEM_U32: lg_elem = 1;
pub const LG_ELEM_I32: lg_elem = 2;
pub const LG_ELEM_C32: lg_elem = 3;

pub type lg_core_error = i32;
pub const LG_CORE_OK: lg_core_error = 0;
pub const LG_CORE_SHAPE: lg_core_error = 1;
pub const LG_CORE_DTYPE: lg_core_error = 2;
pub const LG_CORE_UNSUPPORTED_LAYOUT: lg_core_error = 3;
pub const LG_CORE_UNSUPPORTED_DEVICE: lg_core_error = 4;
pub const LG_CORE_ALIAS: lg_core_error = 5;
pub const LG_CORE_TRANSPORT: lg_core_error = 6;
pub const LG_CORE_WIRE: lg_core_error = 7;
pub const LG_CORE_SCHEDULE: lg_core_error = 8;

pub type lg_dtype = u32;
pub const LG_DTYPE_F32: lg_dtype = 1;
pub const LG_DTYPE_F16: lg_dtype = 2;
pub const LG_DTYPE_BF16: lg_dtype = 3;

#[repr(C)]
#[derive(Clone, Copy)]
pub struct lg_view {
    pub base: *mut c_void,
    pub bytes: u64,
    pub offset: u64,
    pub rank: u32,
    pub nstrides: u32,
    pub shape: [u64; LG_MAX_RANK],
    pub strides: [u64; LG_MAX_RANK],
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct lg_tensor {
    pub base: *mut c_void,
    pub bytes: u64,
    pub dtype: u32,
    pub rank: u32,
    pub nstrides: u32,
    pub reserved: u32,
    pub offset: u64,
    pub shape: [u64; LG_MAX_RANK],
    pub strides: [u64; LG_MAX_RANK],
}

#[repr(C)]
#[derive(Clone, Copy, Default, Debug)]
pub struct lg_contract_plan {
    pub kind: u32,
    pub a_mode: u32,
    pub b_mode: u32,
    pub groups: u32,
    pub batch: u64,
    pub m: u64,
    pub n: u64,
    pub k: u64,
    pub splits: u64,
    pub k_chunk: u64,
    pub workgroups: u64,
    pub scratch_bytes: u64,
    pub tile_m: u32,
    pub tile_n: u32,
    pub kernel: u32,
    pub swapped: u32,
    pub kgroups: u32,
    pub reserved: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Default, Debug)]
pub struct lg_permute_plan {
    pub kind: u32,
    pub rank: u32,
    pub axis_a: u32,
    pub axis_b: u32,
    pub vector: u32,
    pub conj: u32,
    pub streaming: u32,
    pub reserved: u32,
    pub shape: [u64; 8],
    pub strides: [u64; 8],
    pub workgroups: u64,
}

/// Opaque context: one device and its stream.
#[repr(C)]
pub struct lg_ctx {
    _private: [u8; 0],
}

#[link(name = "linalg_hip")]
extern "C" {
    // Errors, context and memory.
    pub fn lg_last_error() -> *const c_char;
    pub fn lg_ctx_create(device: i32, out: *mut *mut lg_ctx) -> lg_status;
    pub fn lg_ctx_destroy(ctx: *mut lg_ctx);
    pub fn lg_ctx_stream(ctx: *const lg_ctx) -> *mut c_void;
    pub fn lg_ctx_sync(ctx: *mut lg_ctx) -> lg_status;
    pub fn lg_stream_sync(ctx: *mut lg_ctx, stream: *mut c_void) -> lg_status;
    pub fn lg_stream_create(ctx: *mut lg_ctx, stream: *mut *mut c_void) -> lg_status;
    pub fn lg_stream_destroy(ctx: *mut lg_ctx, stream: *mut c_void) -> lg_status;
    pub fn lg_alloc(ctx: *mut lg_ctx, elem_bytes: u64, len: u64, base: *mut *mut c_void,
                    bytes: *mut u64) -> lg_status;
    pub fn lg_free(ctx: *mut lg_ctx, base: *mut c_void) -> lg_status;
    pub fn lg_upload(ctx: *mut lg_ctx, base: *mut c_void, byte_offset: u64, src: *const c_void,
                     nbytes: u64) -> lg_status;
    pub fn lg_download(ctx: *mut lg_ctx, base: *const c_void, byte_offset: u64, dst: *mut c_void,
                       nbytes: u64) -> lg_status;

    // View metadata.
    pub fn lg_view_validate(view: *const lg_view, elem_bytes: u32) -> lg_status;
    pub fn lg_view_may_overlap(a: *const lg_view, a_elem_bytes: u32, b: *const lg_view,
                               b_elem_bytes: u32) -> i32;

    // Permutation.
    pub fn lg_permute_view(view: *const lg_view, perm: *const u64, perm_len: u32,
                           out: *mut lg_view) -> lg_status;
    pub fn lg_encode_materialize(ctx: *mut lg_ctx, stream: *mut c_void, elem: lg_elem,
                                 src: *const lg_view, dst: *const lg_view) -> lg_status;
    pub fn lg_materialize(ctx: *mut lg_ctx, elem: lg_elem, src: *const lg_view,
                          dst: *const lg_view) -> lg_status;
    pub fn lg_encode_conjugate(ctx: *mut lg_ctx, stream: *mut c_void, elem: lg_elem,
                               src: *const lg_view, dst: *const lg_view) -> lg_status;
    pub fn lg_conjugate(ctx: *mut lg_ctx, elem: lg_elem, src: *const lg_view,
                        dst: *const lg_view) -> lg_status;
    pub fn lg_encode_adjoint(ctx: *mut lg_ctx, stream: *mut c_void, elem: lg_elem,
                             src: *const lg_view, dst: *const lg_view) -> lg_status;
    pub fn lg_adjoint(ctx: *mut lg_ctx, elem: lg_elem, src: *const lg_view, dst: *const lg_view)
        -> lg_status;

    // Contraction, f32.
    pub fn lg_encode_contract_f32(ctx: *mut lg_ctx, stream: *mut c_void, alpha: f32,
                                  a: *const lg_view, a_labels: *const c_char, b: *const lg_view,
                                  b_labels: *const c_char, beta: f32, c: *const lg_view,
                                  c_labels: *const c_char) -> lg_status;
    pub fn lg_contract_f32(ctx: *mut lg_ctx, alpha: f32, a: *const lg_view,
                           a_labels: *const c_char, b: *const lg_view, b_labels: *const c_char,
                           beta: f32, c: *const lg_view, c_labels: *const c_char) -> lg_status;
    pub fn lg_encode_gemm_f32(ctx: *mut lg_ctx, stream: *mut c_void, alpha: f32,
                              a: *const lg_view, b: *const lg_view, beta: f32,
                              c: *const lg_view) -> lg_status;
    pub fn lg_gemm_f32(ctx: *mut lg_ctx, alpha: f32, a: *const lg_view, b: *const lg_view,
                       beta: f32, c: *const lg_view) -> lg_status;
    pub fn lg_gemm_nowait_f32(ctx: *mut lg_ctx, alpha: f32, a: *const lg_view,
                              b: *const lg_view, beta: f32, c: *const lg_view) -> lg_status;
    pub fn lg_encode_gemm_f32_noalloc(ctx: *mut lg_ctx, stream: *mut c_void, alpha: f32,
                                      a: *const lg_view, b: *const lg_view, beta: f32,
                                      c: *const lg_view) -> lg_status;

    // Contraction, f16 (views of half elements; alpha and beta stay f32).
    pub fn lg_encode_contract_f16(ctx: *mut lg_ctx, stream: *mut c_void, alpha: f32,
                                  a: *const lg_view, a_labels: *const c_char, b: *const lg_view,
                                  b_labels: *const c_char, beta: f32, c: *const lg_view,
                                  c_labels: *const c_char) -> lg_status;
    pub fn lg_contract_f16(ctx: *mut lg_ctx, alpha: f32, a: *const lg_view,
                           a_labels: *const c_char, b: *const lg_view, b_labels: *const c_char,
                           beta: f32, c: *const lg_view, c_labels: *const c_char) -> lg_status;
    pub fn lg_encode_gemm_f16(ctx: *mut lg_ctx, stream: *mut c_void, alpha: f32,
                              a: *const lg_view, b: *const lg_view, beta: f32,
                              c: *const lg_view) -> lg_status;
    pub fn lg_gemm_f16(ctx: *mut lg_ctx, alpha: f32, a: *const lg_view, b: *const lg_view,
                       beta: f32, c: *const lg_view) -> lg_status;
    pub fn lg_gemm_nowait_f16(ctx: *mut lg_ctx, alpha: f32, a: *const lg_view,
                              b: *const lg_view, beta: f32, c: *const lg_view) -> lg_status;

    // Backend-style operations (linalg_core::Backend).
    pub fn lg_backend_gemm(ctx: *mut lg_ctx, stream: *mut c_void, a: *const lg_tensor,
                           b: *const lg_tensor, c: *const lg_tensor, alpha: f32, beta: f32)
        -> lg_core_error;
    pub fn lg_backend_gelu(ctx: *mut lg_ctx, stream: *mut c_void, x: *const lg_tensor,
                           y: *const lg_tensor) -> lg_core_error;
    pub fn lg_backend_gelu_backward(ctx: *mut lg_ctx, stream: *mut c_void, pre: *const lg_tensor,
                                    dy: *const lg_tensor, dx: *const lg_tensor) -> lg_core_error;
    pub fn lg_backend_add_bias(ctx: *mut lg_ctx, stream: *mut c_void, x: *const lg_tensor,
                               b: *const lg_tensor, y: *const lg_tensor) -> lg_core_error;
    pub fn lg_backend_bias_grad(ctx: *mut lg_ctx, stream: *mut c_void, dpre: *const lg_tensor,
                                db: *const lg_tensor) -> lg_core_error;
    pub fn lg_backend_mse_grad(ctx: *mut lg_ctx, stream: *mut c_void, y: *const lg_tensor,
                               target: *const lg_tensor, dy: *const lg_tensor, loss: *mut f32)
        -> lg_core_error;
    pub fn lg_backend_sgd_step(ctx: *mut lg_ctx, stream: *mut c_void, w: *const lg_tensor,
                               dw: *const lg_tensor, lr: f32) -> lg_core_error;
    pub fn lg_backend_convert(ctx: *mut lg_ctx, stream: *mut c_void, x: *const lg_tensor,
                              y: *const lg_tensor) -> lg_core_error;
    pub fn lg_backend_download_into(ctx: *mut lg_ctx, stream: *mut c_void, t: *const lg_tensor,
                                    out: *mut u8, out_len: u64) -> lg_core_error;
    pub fn lg_backend_upload_into(ctx: *mut lg_ctx, stream: *mut c_void, bytes: *const u8,
                                  len: u64, t: *const lg_tensor) -> lg_core_error;

    // The wire format and its device-buffer ends.
    pub fn lg_wire_write_header(dtype: u32, shape: *const u64, rank: u32, out: *mut u8,
                                len: *mut u64) -> lg_core_error;
    pub fn lg_wire_parse_header(bytes: *const u8, len: u64, dtype: *mut u32, shape: *mut u64,
                                rank: *mut u32, payload_offset: *mut u64) -> lg_core_error;
    pub fn lg_wire_encode(dtype: u32, shape: *const u64, rank: u32, payload: *const c_void,
                          payload_len: u64, out: *mut u8, out_cap: u64, written: *mut u64)
        -> lg_core_error;
    pub fn lg_wire_encode_tensor(ctx: *mut lg_ctx, t: *const lg_tensor, out: *mut u8,
                                 out_cap: u64, written: *mut u64) -> lg_core_error;
    pub fn lg_wire_decode_into(ctx: *mut lg_ctx, bytes: *const u8, len: u64,
                               t: *const lg_tensor) -> lg_core_error;

    // Plan inspection (host only) and the debug launch log.
    pub fn lg_plan_contract_f32(alpha: f32, a: *const lg_view, a_labels: *const c_char,
                                b: *const lg_view, b_labels: *const c_char, beta: f32,
                                c: *const lg_view, c_labels: *const c_char,
                                out: *mut lg_contract_plan) -> lg_status;
    pub fn lg_plan_gemm_f32(alpha: f32, a: *const lg_view, b: *const lg_view, beta: f32,
                            c: *const lg_view, out: *mut lg_contract_plan) -> lg_status;
    pub fn lg_plan_contract_f16(alpha: f32, a: *const lg_view, a_labels: *const c_char,
                                b: *const lg_view, b_labels: *const c_char, beta: f32,
                                c: *const lg_view, c_labels: *const c_char,
                                out: *mut lg_contract_plan) -> lg_status;
    pub fn lg_plan_gemm_f16(alpha: f32, a: *const lg_view, b: *const lg_view, beta: f32,
                            c: *const lg_view, out: *mut lg_contract_plan) -> lg_status;
    pub fn lg_plan_permute(op: u32, elem: lg_elem, src: *const lg_view, dst: *const lg_view,
                           out: *mut lg_permute_plan) -> lg_status;
    pub fn lg_debug_launch_count(ctx: *const lg_ctx) -> u64;
    pub fn lg_debug_launch_name(ctx: *const lg_ctx, i: u64) -> *const c_char;
}
