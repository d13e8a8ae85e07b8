//! linalg's contraction and permutation operators on MI355X (gfx950), through liblinalg_hip.
//!
//! The surface mirrors the reference crate's: `LinalgError` / `Result` / the context /
//! `TensorView` / `alloc_shared` / `row_major_strides` of `linalg::abi` (src/abi.rs:20-243),
//! `ops::contraction::{contract, encode_contract, gemm, encode_gemm, gemm_nowait}`
//! (src/ops/contraction.rs:1036-1130) and `ops::permutation::{permute_view, materialize,
//! encode_materialize, conjugate, encode_conjugate, adjoint, encode_adjoint}`
//! (src/ops/permutation.rs:299-387), with the same argument meaning and errors. What differs is
//! what a discrete GPU needs: buffers are device memory with explicit `upload` / `download`,
//! and `encode_*` enqueue on a `HipStream` (work starts when enqueued; `wait_until_completed`
//! waits) where the reference encodes into a Metal command buffer.

pub mod ffi;

use std::ffi::{CStr, CString};
use std::fmt;
use std::marker::PhantomData;

/// Errors of every fallible operation (src/abi.rs:20-33). On error nothing was enqueued.
#[derive(Clone, Debug, PartialEq, Eq)]
pub enum LinalgError {
    /// No HIP device with the requested index.
    NoDevice,
    /// A shape, stride, offset, extent, or parameter is invalid for the requested operation.
    InvalidArgument(String),
    /// A destination overlaps a source in a way the operation does not allow.
    Overlap(String),
    /// A code-object, launch or runtime failure (the reference's shader-compile failure).
    ShaderCompile(String),
}

impl fmt::Display for LinalgError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        match self {
            Self::NoDevice => write!(f, "no HIP device available"),
            Self::InvalidArgument(msg) => write!(f, "invalid argument: {msg}"),
            Self::Overlap(msg) => write!(f, "overlapping views: {msg}"),
            Self::ShaderCompile(msg) => write!(f, "kernel failure: {msg}"),
        }
    }
}

impl std::error::Error for LinalgError {}

/// Crate-wide result type.
pub type Result<T> = std::result::Result<T, LinalgError>;

fn check(status: ffi::lg_status) -> Result<()> {
    if status == ffi::LG_OK {
        return Ok(());
    }
    // SAFETY: lg_last_error returns a NUL-terminated thread-local string that stays valid
    // until the next call on this thread.
    let msg = unsafe { CStr::from_ptr(ffi::lg_last_error()) }.to_string_lossy().into_owned();
    Err(match status {
        ffi::LG_NO_DEVICE => LinalgError::NoDevice,
        ffi::LG_INVALID_ARGUMENT => LinalgError::InvalidArgument(msg),
        ffi::LG_OVERLAP => LinalgError::Overlap(msg),
        _ => LinalgError::ShaderCompile(msg),
    })
}

/// One HIP device and the stream the synchronous operations run on (MetalContext,
/// src/abi.rs:51-62).
pub struct HipContext {
    raw: *mut ffi::lg_ctx,
}

// SAFETY: the library's entry points may be called from any thread; calls on different streams
// may run concurrently (include/linalg_hip.h, "Thread safety").
unsafe impl Send for HipContext {}
unsafe impl Sync for HipContext {}

impl HipContext {
    /// Opens device 0 (MetalContext::new).
    pub fn new() -> Result<Self> {
        Self::with_device(0)
    }

    /// Opens HIP device `device`.
    pub fn with_device(device: i32) -> Result<Self> {
        let mut raw = std::ptr::null_mut();
        // SAFETY: `raw` is a valid out-pointer.
        check(unsafe { ffi::lg_ctx_create(device, &mut raw) })?;
        Ok(Self { raw })
    }

    /// A new stream: what the reference's `queue.new_command_buffer()` gives `encode_*`.
    pub fn new_stream(&self) -> Result<HipStream<'_>> {
        let mut raw = std::ptr::null_mut();
        // SAFETY: the context is live and `raw` a valid out-pointer.
        check(unsafe { ffi::lg_stream_create(self.raw, &mut raw) })?;
        Ok(HipStream { ctx: self, raw })
    }

    /// Blocks until everything enqueued on the context's stream has completed.
    pub fn sync(&self) -> Result<()> {
        // SAFETY: the context is live.
        check(unsafe { ffi::lg_ctx_sync(self.raw) })
    }

    /// Names of the kernels launched so far (at most the last 256): the debug launch log.
    pub fn launches(&self) -> Vec<String> {
        // SAFETY: the context is live; names are static NUL-terminated strings.
        unsafe {
            let n = ffi::lg_debug_launch_count(self.raw);
            (n.saturating_sub(256)..n)
                .filter_map(|i| {
                    let p = ffi::lg_debug_launch_name(self.raw, i);
                    (!p.is_null()).then(|| CStr::from_ptr(p).to_string_lossy().into_owned())
                })
                .collect()
        }
    }

    pub fn raw(&self) -> *mut ffi::lg_ctx {
        self.raw
    }
}

impl Drop for HipContext {
    fn drop(&mut self) {
        // SAFETY: created by lg_ctx_create and destroyed once.
        unsafe { ffi::lg_ctx_destroy(self.raw) }
    }
}

/// A stream of one context: `encode_*` enqueue on it in call order.
pub struct HipStream<'c> {
    ctx: &'c HipContext,
    raw: *mut std::ffi::c_void,
}

impl HipStream<'_> {
    /// Blocks until everything enqueued on this stream has completed (`wait_until_completed`).
    pub fn wait_until_completed(&self) -> Result<()> {
        // SAFETY: the stream belongs to the live context.
        check(unsafe { ffi::lg_stream_sync(self.ctx.raw, self.raw) })
    }
}

impl Drop for HipStream<'_> {
    fn drop(&mut self) {
        // SAFETY: created by lg_stream_create on this context; waits, then destroys.
        unsafe {
            ffi::lg_stream_destroy(self.ctx.raw, self.raw);
        }
    }
}

/// A device allocation (the reference's shared metal::Buffer): zero-filled, whole 16 KiB
/// granules, contents moved with `upload` / `download`.
pub struct HipBuffer<'c> {
    ctx: &'c HipContext,
    base: *mut std::ffi::c_void,
    bytes: u64,
}

impl HipBuffer<'_> {
    /// Allocation length in bytes (`buffer.length()`).
    pub fn length(&self) -> u64 {
        self.bytes
    }

    /// The device base address (`buffer.contents()`): views count elements from here.
    pub fn contents(&self) -> *mut std::ffi::c_void {
        self.base
    }

    /// Copies `data` into the buffer at `byte_offset`, after every earlier call on the
    /// context's stream; returns once the copy is done.
    pub fn upload<T: Copy>(&self, byte_offset: u64, data: &[T]) -> Result<()> {
        let n = std::mem::size_of_val(data) as u64;
        // SAFETY: `data` is valid for `n` bytes; the library checks the range.
        check(unsafe { ffi::lg_upload(self.ctx.raw, self.base, byte_offset, data.as_ptr().cast(), n) })
    }

    /// Copies bytes from `byte_offset` into `out`, after every earlier call on the context's
    /// stream.
    pub fn download<T: Copy>(&self, byte_offset: u64, out: &mut [T]) -> Result<()> {
        let n = std::mem::size_of_val(out) as u64;
        // SAFETY: `out` is valid for `n` bytes of writes; the library checks the range.
        check(unsafe { ffi::lg_download(self.ctx.raw, self.base, byte_offset, out.as_mut_ptr().cast(), n) })
    }
}

impl Drop for HipBuffer<'_> {
    fn drop(&mut self) {
        // SAFETY: allocated by lg_alloc on this context; freed once after its stream drains.
        unsafe {
            ffi::lg_free(self.ctx.raw, self.base);
        }
    }
}

/// A zero-filled device buffer of at least `len` elements of `T` (alloc_shared,
/// src/abi.rs:225-243).
pub fn alloc_shared<T>(ctx: &HipContext, len: usize) -> Result<HipBuffer<'_>> {
    let (mut base, mut bytes) = (std::ptr::null_mut(), 0u64);
    // SAFETY: out-pointers are valid.
    check(unsafe {
        ffi::lg_alloc(ctx.raw, std::mem::size_of::<T>() as u64, len as u64, &mut base, &mut bytes)
    })?;
    Ok(HipBuffer { ctx, base, bytes })
}

/// Row-major strides of `shape`, in elements (src/abi.rs:214-220).
pub fn row_major_strides(shape: &[usize]) -> Vec<usize> {
    let mut strides = vec![0; shape.len()];
    let mut stride = 1usize;
    for d in (0..shape.len()).rev() {
        strides[d] = stride;
        stride *= shape[d];
    }
    strides
}

/// A strided view of elements of type `T` in one buffer (TensorView, src/abi.rs:64-211): the
/// element at multi-index idx is element `offset + sum(idx[d] * strides[d])` of the buffer.
pub struct TensorView<'a, T> {
    pub buffer: &'a HipBuffer<'a>,
    pub offset: usize,
    pub shape: Vec<usize>,
    pub strides: Vec<usize>,
    _elem: PhantomData<T>,
}

impl<T> Clone for TensorView<'_, T> {
    fn clone(&self) -> Self {
        Self {
            buffer: self.buffer,
            offset: self.offset,
            shape: self.shape.clone(),
            strides: self.strides.clone(),
            _elem: PhantomData,
        }
    }
}

impl<'a, T> TensorView<'a, T> {
    /// Explicit metadata; nothing is validated here (operations validate).
    pub fn new(buffer: &'a HipBuffer<'a>, offset: usize, shape: Vec<usize>, strides: Vec<usize>) -> Self {
        Self { buffer, offset, shape, strides, _elem: PhantomData }
    }

    /// A contiguous row-major view of `shape` starting at element `offset`.
    pub fn row_major(buffer: &'a HipBuffer<'a>, offset: usize, shape: Vec<usize>) -> Self {
        let strides = row_major_strides(&shape);
        Self::new(buffer, offset, shape, strides)
    }

    pub fn rank(&self) -> usize {
        self.shape.len()
    }

    pub fn len(&self) -> usize {
        self.shape.iter().product()
    }

    pub fn is_empty(&self) -> bool {
        self.shape.contains(&0)
    }

    /// Buffer element index of multi-index `idx`.
    pub fn element_index(&self, idx: &[usize]) -> usize {
        self.offset + idx.iter().zip(&self.strides).map(|(i, s)| i * s).sum::<usize>()
    }

    /// TensorView::validate (src/abi.rs:140-177).
    pub fn validate(&self) -> Result<()> {
        let v = self.to_c()?;
        // SAFETY: `v` is a fully initialised view descriptor.
        check(unsafe { ffi::lg_view_validate(&v, std::mem::size_of::<T>() as u32) })
    }

    /// TensorView::may_overlap (src/abi.rs:193-204); both views must validate.
    pub fn may_overlap<U>(&self, other: &TensorView<'_, U>) -> bool {
        match (self.to_c(), other.to_c()) {
            // SAFETY: both descriptors are fully initialised.
            (Ok(a), Ok(b)) => unsafe {
                ffi::lg_view_may_overlap(&a, std::mem::size_of::<T>() as u32, &b,
                                         std::mem::size_of::<U>() as u32) != 0
            },
            _ => true,
        }
    }

    /// The C descriptor; a rank above LG_MAX_RANK is InvalidArgument.
    pub fn to_c(&self) -> Result<ffi::lg_view> {
        if self.shape.len() > ffi::LG_MAX_RANK || self.strides.len() > ffi::LG_MAX_RANK {
            return Err(LinalgError::InvalidArgument(format!(
                "rank {} exceeds {}", self.shape.len().max(self.strides.len()), ffi::LG_MAX_RANK)));
        }
        let mut v = ffi::lg_view {
            base: self.buffer.base,
            bytes: self.buffer.bytes,
            offset: self.offset as u64,
            rank: self.shape.len() as u32,
            nstrides: self.strides.len() as u32,
            shape: [0; ffi::LG_MAX_RANK],
            strides: [0; ffi::LG_MAX_RANK],
        };
        for (d, &e) in self.shape.iter().enumerate() {
            v.shape[d] = e as u64;
        }
        for (d, &s) in self.strides.iter().enumerate() {
            v.strides[d] = s as u64;
        }
        Ok(v)
    }
}

fn labels(s: &str) -> Result<CString> {
    if !s.is_ascii() {
        return Err(LinalgError::InvalidArgument("labels must be ASCII, one byte per axis".into()));
    }
    CString::new(s).map_err(|_| LinalgError::InvalidArgument("labels hold a NUL byte".into()))
}

pub mod ops {
    pub mod contraction {
        //! C = alpha * A.B + beta * C over einsum labels, and the batched matrix form
        //! (src/ops/contraction.rs:1036-1130).
        use crate::{check, ffi, labels, HipContext, HipStream, Result, TensorView};
        use std::ffi::{c_char, c_void};

        mod sealed {
            pub trait Sealed {}
            impl Sealed for f32 {}
            impl Sealed for half::f16 {}
        }

        type ContractFn = unsafe extern "C" fn(*mut ffi::lg_ctx, *mut c_void, f32, *const ffi::lg_view,
                                               *const c_char, *const ffi::lg_view, *const c_char, f32,
                                               *const ffi::lg_view, *const c_char) -> ffi::lg_status;
        type GemmFn = unsafe extern "C" fn(*mut ffi::lg_ctx, *mut c_void, f32, *const ffi::lg_view,
                                           *const ffi::lg_view, f32, *const ffi::lg_view) -> ffi::lg_status;

        /// Element types of a contraction (src/ops/contraction.rs:22-32): f32, and f16 with
        /// each output rounded once.
        pub trait Element: sealed::Sealed + Copy + 'static {
            const ENCODE_CONTRACT: ContractFn;
            const ENCODE_GEMM: GemmFn;
        }
        impl Element for f32 {
            const ENCODE_CONTRACT: ContractFn = ffi::lg_encode_contract_f32;
            const ENCODE_GEMM: GemmFn = ffi::lg_encode_gemm_f32;
        }
        impl Element for half::f16 {
            const ENCODE_CONTRACT: ContractFn = ffi::lg_encode_contract_f16;
            const ENCODE_GEMM: GemmFn = ffi::lg_encode_gemm_f16;
        }

        /// A view and its labels, one ASCII byte per axis (src/ops/contraction.rs:35).
        pub type Operand<'v, 'b, T> = (&'v TensorView<'b, T>, &'v str);

        fn contract_on<T: Element>(ctx: &HipContext, stream: *mut c_void, alpha: f32,
                                   a: Operand<'_, '_, T>, b: Operand<'_, '_, T>, beta: f32,
                                   c: Operand<'_, '_, T>) -> Result<()> {
            let (va, vb, vc) = (a.0.to_c()?, b.0.to_c()?, c.0.to_c()?);
            let (la, lb, lc) = (labels(a.1)?, labels(b.1)?, labels(c.1)?);
            // SAFETY: descriptors and labels outlive the call, which copies what it keeps.
            check(unsafe {
                T::ENCODE_CONTRACT(ctx.raw(), stream, alpha, &va, la.as_ptr(), &vb, lb.as_ptr(),
                                   beta, &vc, lc.as_ptr())
            })
        }

        fn gemm_on<T: Element>(ctx: &HipContext, stream: *mut c_void, alpha: f32, a: &TensorView<'_, T>,
                               b: &TensorView<'_, T>, beta: f32, c: &TensorView<'_, T>) -> Result<()> {
            let (va, vb, vc) = (a.to_c()?, b.to_c()?, c.to_c()?);
            // SAFETY: the descriptors outlive the call.
            check(unsafe { T::ENCODE_GEMM(ctx.raw(), stream, alpha, &va, &vb, beta, &vc) })
        }

        /// Enqueues C = alpha*A.B + beta*C on `stream` (encode_contract).
        pub fn encode_contract<T: Element>(ctx: &HipContext, stream: &HipStream<'_>, alpha: f32,
                                           a: Operand<'_, '_, T>, b: Operand<'_, '_, T>, beta: f32,
                                           c: Operand<'_, '_, T>) -> Result<()> {
            contract_on(ctx, stream.raw, alpha, a, b, beta, c)
        }

        /// encode_contract on the context's stream, then waits (contract).
        pub fn contract<T: Element>(ctx: &HipContext, alpha: f32, a: Operand<'_, '_, T>,
                                    b: Operand<'_, '_, T>, beta: f32, c: Operand<'_, '_, T>) -> Result<()> {
            contract_on(ctx, std::ptr::null_mut(), alpha, a, b, beta, c)?;
            ctx.sync()
        }

        /// Enqueues the batched matrix product on `stream` (encode_gemm).
        pub fn encode_gemm<T: Element>(ctx: &HipContext, stream: &HipStream<'_>, alpha: f32,
                                       a: &TensorView<'_, T>, b: &TensorView<'_, T>, beta: f32,
                                       c: &TensorView<'_, T>) -> Result<()> {
            gemm_on(ctx, stream.raw, alpha, a, b, beta, c)
        }

        /// encode_gemm on the context's stream, then waits (gemm).
        pub fn gemm<T: Element>(ctx: &HipContext, alpha: f32, a: &TensorView<'_, T>,
                                b: &TensorView<'_, T>, beta: f32, c: &TensorView<'_, T>) -> Result<()> {
            gemm_on(ctx, std::ptr::null_mut(), alpha, a, b, beta, c)?;
            ctx.sync()
        }

        /// Enqueues on the context's stream and returns before the device finishes
        /// (gemm_nowait); `ctx.sync()` or a download waits for it.
        pub fn gemm_nowait<T: Element>(ctx: &HipContext, alpha: f32, a: &TensorView<'_, T>,
                                       b: &TensorView<'_, T>, beta: f32, c: &TensorView<'_, T>) -> Result<()> {
            gemm_on(ctx, std::ptr::null_mut(), alpha, a, b, beta, c)
        }
    }

    pub mod permutation {
        //! Axis permutation and the bit-exact copies built on it (src/ops/permutation.rs:272-387).
        use crate::{check, ffi, HipContext, HipStream, LinalgError, Result, TensorView};
        use std::ffi::c_void;

        mod sealed {
            pub trait Sealed {}
            impl Sealed for f32 {}
            impl Sealed for u32 {}
            impl Sealed for i32 {}
            impl Sealed for [f32; 2] {}
        }

        /// Element types moved as raw bits (src/ops/permutation.rs:26-54).
        pub trait Element: sealed::Sealed + Copy {
            const ELEM: ffi::lg_elem;
        }
        impl Element for f32 {
            const ELEM: ffi::lg_elem = ffi::LG_ELEM_F32;
        }
        impl Element for u32 {
            const ELEM: ffi::lg_elem = ffi::LG_ELEM_U32;
        }
        impl Element for i32 {
            const ELEM: ffi::lg_elem = ffi::LG_ELEM_I32;
        }
        impl Element for [f32; 2] {
            const ELEM: ffi::lg_elem = ffi::LG_ELEM_C32;
        }

        /// Axis i of the result is axis perm[i] of `view`; metadata only (permute_view).
        pub fn permute_view<'a, T>(view: &TensorView<'a, T>, perm: &[usize]) -> Result<TensorView<'a, T>> {
            let v = view.to_c()?;
            let p: Vec<u64> = perm.iter().map(|&x| x as u64).collect();
            // SAFETY: every pointer is valid for the call; `out` is fully written on success.
            let mut out = v;
            check(unsafe { ffi::lg_permute_view(&v, p.as_ptr(), p.len() as u32, &mut out) })?;
            let rank = out.rank as usize;
            if rank > ffi::LG_MAX_RANK {
                return Err(LinalgError::InvalidArgument("rank out of range".into()));
            }
            Ok(TensorView::new(view.buffer, out.offset as usize,
                               out.shape[..rank].iter().map(|&e| e as usize).collect(),
                               out.strides[..rank].iter().map(|&s| s as usize).collect()))
        }

        type CopyFn = unsafe extern "C" fn(*mut ffi::lg_ctx, *mut c_void, ffi::lg_elem,
                                           *const ffi::lg_view, *const ffi::lg_view) -> ffi::lg_status;

        fn copy_on<T: Element>(f: CopyFn, ctx: &HipContext, stream: *mut c_void, src: &TensorView<'_, T>,
                               dst: &TensorView<'_, T>) -> Result<()> {
            let (s, d) = (src.to_c()?, dst.to_c()?);
            // SAFETY: the descriptors outlive the call.
            check(unsafe { f(ctx.raw(), stream, T::ELEM, &s, &d) })
        }

        /// Copies `src` into the row-major `dst`, bit for bit (encode_materialize).
        pub fn encode_materialize<T: Element>(ctx: &HipContext, stream: &HipStream<'_>,
                                              src: &TensorView<'_, T>, dst: &TensorView<'_, T>) -> Result<()> {
            copy_on(ffi::lg_encode_materialize, ctx, stream.raw, src, dst)
        }

        pub fn materialize<T: Element>(ctx: &HipContext, src: &TensorView<'_, T>,
                                       dst: &TensorView<'_, T>) -> Result<()> {
            copy_on(ffi::lg_encode_materialize, ctx, std::ptr::null_mut(), src, dst)?;
            ctx.sync()
        }

        /// As materialize, flipping the imaginary sign bit of complex elements (encode_conjugate).
        pub fn encode_conjugate<T: Element>(ctx: &HipContext, stream: &HipStream<'_>,
                                            src: &TensorView<'_, T>, dst: &TensorView<'_, T>) -> Result<()> {
            copy_on(ffi::lg_encode_conjugate, ctx, stream.raw, src, dst)
        }

        pub fn conjugate<T: Element>(ctx: &HipContext, src: &TensorView<'_, T>,
                                     dst: &TensorView<'_, T>) -> Result<()> {
            copy_on(ffi::lg_encode_conjugate, ctx, std::ptr::null_mut(), src, dst)?;
            ctx.sync()
        }

        /// Swaps the last two axes and conjugates complex elements (encode_adjoint).
        pub fn encode_adjoint<T: Element>(ctx: &HipContext, stream: &HipStream<'_>,
                                          src: &TensorView<'_, T>, dst: &TensorView<'_, T>) -> Result<()> {
            copy_on(ffi::lg_encode_adjoint, ctx, stream.raw, src, dst)
        }

        pub fn adjoint<T: Element>(ctx: &HipContext, src: &TensorView<'_, T>,
                                   dst: &TensorView<'_, T>) -> Result<()> {
            copy_on(ffi::lg_encode_adjoint, ctx, std::ptr::null_mut(), src, dst)?;
            ctx.sync()
        }
    }
}
