//! Raw bindings to `include/oxm.h`, the C-ABI of the MI355X (gfx950)
//! backend.  Every item mirrors one declaration of the header; the header's
//! comments state the contracts.  The safe wrapper is the `oxmera-hip`
//! crate, which implements `oxmera_runtime::Backend`
//! (crates/oxmera-runtime/src/lib.rs:25-34) on top of these functions.
//!
//! Stable oxmera crates are `#![forbid(unsafe_code)]`
//! (crates/oxmera-core/src/lib.rs:13); the `unsafe` of the FFI lives here, in
//! a crate of its own, as `research/` is isolated (ADR-0003).

#![allow(non_camel_case_types)]
#![warn(missing_docs)]

use std::ffi::{c_char, c_void};

/// `oxm_status`: one code per `oxmera_core::Error` variant
/// (crates/oxmera-core/src/error.rs:14-102), plus runtime failures, ABI
/// argument errors and integer division by zero.
pub type oxm_status = i32;
/// Success.
pub const OXM_OK: oxm_status = 0;
/// `Error::ShapeMismatch`.
pub const OXM_E_SHAPE_MISMATCH: oxm_status = 1;
/// `Error::BroadcastIncompatible`.
pub const OXM_E_BROADCAST_INCOMPATIBLE: oxm_status = 2;
/// `Error::DTypeMismatch`.
pub const OXM_E_DTYPE_MISMATCH: oxm_status = 3;
/// `Error::UnsupportedDType`.
pub const OXM_E_UNSUPPORTED_DTYPE: oxm_status = 4;
/// `Error::DeviceMismatch`.
pub const OXM_E_DEVICE_MISMATCH: oxm_status = 5;
/// `Error::IndexOutOfBounds`.
pub const OXM_E_INDEX_OUT_OF_BOUNDS: oxm_status = 6;
/// `Error::RankMismatch`.
pub const OXM_E_RANK_MISMATCH: oxm_status = 7;
/// `Error::BackendUnavailable`.
pub const OXM_E_BACKEND_UNAVAILABLE: oxm_status = 8;
/// `Error::NotImplemented`.
pub const OXM_E_NOT_IMPLEMENTED: oxm_status = 9;
/// A HIP runtime failure (no `Error` variant: reported as `NotImplemented`
/// with the runtime's message by the safe crate).
pub const OXM_E_HIP: oxm_status = 10;
/// A NULL or malformed argument at the ABI itself (including an output that
/// overlaps an input).
pub const OXM_E_INVALID_ARGUMENT: oxm_status = 11;
/// Integer division by zero (BinaryOps::div, crates/oxmera-ops/src/lib.rs:47-48).
pub const OXM_E_DIVISION_BY_ZERO: oxm_status = 12;

/// `oxm_dtype`: `oxmera_core::DType` in declaration order (dtype.rs:9-22),
/// then BF16 and F16.
pub type oxm_dtype = i32;
/// F32.
pub const OXM_F32: oxm_dtype = 0;
/// F64.
pub const OXM_F64: oxm_dtype = 1;
/// I32.
pub const OXM_I32: oxm_dtype = 2;
/// I64.
pub const OXM_I64: oxm_dtype = 3;
/// U8.
pub const OXM_U8: oxm_dtype = 4;
/// Bool (one byte, 0 or 1).
pub const OXM_BOOL: oxm_dtype = 5;
/// bfloat16.
pub const OXM_BF16: oxm_dtype = 6;
/// IEEE half.
pub const OXM_F16: oxm_dtype = 7;

/// `oxm_act`: the GEMM epilogue's activation.
pub type oxm_act = i32;
/// out = acc + bias.
pub const OXM_ACT_NONE: oxm_act = 0;
/// aux = acc + bias; out = GELU(aux).
pub const OXM_ACT_GELU: oxm_act = 1;
/// out = acc * GELU'(aux).
pub const OXM_ACT_DGELU: oxm_act = 2;
/// aux = GELU'(acc + bias); out = GELU(acc + bias).
pub const OXM_ACT_GELU_GRAD: oxm_act = 3;
/// out = acc * aux.
pub const OXM_ACT_MUL_AUX: oxm_act = 4;

/// Unary ops (`oxm_unary_op`).
pub const OXM_UN_NEG: i32 = 0;
/// exp.
pub const OXM_UN_EXP: i32 = 1;
/// ln.
pub const OXM_UN_LN: i32 = 2;
/// abs.
pub const OXM_UN_ABS: i32 = 3;
/// sign (autograd helper).
pub const OXM_UN_SIGN: i32 = 4;
/// Binary ops (`oxm_binary_op`).
pub const OXM_BIN_ADD: i32 = 0;
/// sub.
pub const OXM_BIN_SUB: i32 = 1;
/// mul.
pub const OXM_BIN_MUL: i32 = 2;
/// div.
pub const OXM_BIN_DIV: i32 = 3;
/// eq (autograd helper).
pub const OXM_BIN_EQ: i32 = 4;
/// grad * GELU'(z) (autograd helper).
pub const OXM_BIN_DGELU: i32 = 5;
/// Reductions (`oxm_reduce_op`).
pub const OXM_RED_SUM: i32 = 0;
/// max.
pub const OXM_RED_MAX: i32 = 1;

/// Maximum rank of a view.
pub const OXM_MAX_DIMS: usize = 8;
/// Size of the static scratch of `oxm_reduce_noalloc`.
pub const OXM_REDUCE_SCRATCH_BYTES: usize = 8 << 20;

/// A strided view (`oxm_view`): oxmera's `Layout` over a buffer
/// (crates/oxmera-core/src/layout.rs:24-34).  Strides and offset are in
/// elements; `device` is -1 for host memory, else the HIP device index.
#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct oxm_view {
    /// Buffer start (element `offset` is the view's first element).
    pub data: *mut c_void,
    /// `oxm_dtype`.
    pub dtype: i32,
    /// Rank.
    pub ndim: i32,
    /// `ndim` extents.
    pub shape: *const i64,
    /// `ndim` signed element strides.
    pub strides: *const i64,
    /// Element offset.
    pub offset: i64,
    /// -1 = host, >= 0 = HIP device.
    pub device: i32,
}

/// The GEMM epilogue (`oxm_epilogue`).
#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct oxm_epilogue {
    /// `[N]` bias on the device, or NULL.
    pub bias: *const c_void,
    /// The bias's `oxm_dtype`.
    pub bias_dtype: i32,
    /// `oxm_act`.
    pub act: i32,
    /// Pre-activation written (GELU) or read (DGELU), or NULL.
    pub aux: *mut c_void,
    /// `[N]` f32 column sums of the stored output, or NULL.
    pub colsum: *mut f32,
}

unsafe extern "C" {
    /// Library version string.
    pub fn oxm_version() -> *const c_char;
    /// Thread-local message of the last failure.
    pub fn oxm_last_error() -> *const c_char;
    /// Number of HIP devices; `OXM_E_BACKEND_UNAVAILABLE` when none.
    pub fn oxm_device_count(count: *mut i32) -> oxm_status;
    /// `Backend::name()`.
    pub fn oxm_backend_name() -> *const c_char;
    /// Bytes a view addresses, overflow-checked (host only).
    pub fn oxm_view_byte_range(v: *const oxm_view, lo_bytes: *mut i64, hi_bytes: *mut i64) -> oxm_status;
    /// `broadcast_shapes` (shape.rs:45-58).
    pub fn oxm_broadcast_shapes(
        lhs_ndim: i32,
        lhs: *const i64,
        rhs_ndim: i32,
        rhs: *const i64,
        out_ndim: *mut i32,
        out_shape: *mut i64,
    ) -> oxm_status;
    /// Shape rules of `MatmulOps::matmul`.
    pub fn oxm_gemm_infer(a: *const oxm_view, b: *const oxm_view, out_ndim: *mut i32, out_shape: *mut i64)
    -> oxm_status;
    /// `MatmulOps::matmul` with an optional fused epilogue.
    pub fn oxm_gemm(
        a: *const oxm_view,
        b: *const oxm_view,
        c: *const oxm_view,
        ep: *const oxm_epilogue,
        stream: *mut c_void,
    ) -> oxm_status;
    /// Column sums of a rank-2 tensor into f32.
    pub fn oxm_sum_rows(x: *const oxm_view, out: *const oxm_view, stream: *mut c_void) -> oxm_status;
    /// MSE loss and its gradient in one pass.
    pub fn oxm_mse_loss_grad(
        y: *const oxm_view,
        t: *const oxm_view,
        loss: *const oxm_view,
        dy: *const oxm_view,
        dy_colsum: *const oxm_view,
        stream: *mut c_void,
    ) -> oxm_status;
    /// `UnaryOps`.
    pub fn oxm_unary(op: i32, x: *const oxm_view, out: *const oxm_view, stream: *mut c_void) -> oxm_status;
    /// `BinaryOps` with broadcasting.
    pub fn oxm_binary(op: i32, a: *const oxm_view, b: *const oxm_view, out: *const oxm_view, stream: *mut c_void)
    -> oxm_status;
    /// Output shape of a reduction.
    pub fn oxm_reduce_infer(
        x: *const oxm_view,
        axes: *const i32,
        naxes: i32,
        out_ndim: *mut i32,
        out_shape: *mut i64,
    ) -> oxm_status;
    /// `ReduceOps`.
    pub fn oxm_reduce(
        op: i32,
        x: *const oxm_view,
        axes: *const i32,
        naxes: i32,
        out: *const oxm_view,
        stream: *mut c_void,
    ) -> oxm_status;
    /// `ReduceOps` with no allocation (static per-GPU scratch).
    pub fn oxm_reduce_noalloc(
        op: i32,
        x: *const oxm_view,
        axes: *const i32,
        naxes: i32,
        out: *const oxm_view,
        stream: *mut c_void,
    ) -> oxm_status;
    /// `Tensor::contiguous`'s element copy.
    pub fn oxm_copy_view(src: *const oxm_view, dst: *const oxm_view, stream: *mut c_void) -> oxm_status;
    /// Float dtype conversion.
    pub fn oxm_convert(src: *const oxm_view, dst: *const oxm_view, stream: *mut c_void) -> oxm_status;
    /// One fused SGD step.
    pub fn oxm_sgd_step(
        param: *const oxm_view,
        grad: *const oxm_view,
        velocity: *const oxm_view,
        lr: f32,
        momentum: f32,
        weight_decay: f32,
        nesterov: i32,
        stream: *mut c_void,
    ) -> oxm_status;
    /// Device allocation (`Storage`'s device variant).
    pub fn oxm_alloc(device: i32, bytes: usize, out: *mut *mut c_void) -> oxm_status;
    /// Frees an `oxm_alloc` block.
    pub fn oxm_free(device: i32, ptr: *mut c_void) -> oxm_status;
    /// Byte copy between host (-1) and device memory.
    pub fn oxm_copy(
        dst: *mut c_void,
        dst_device: i32,
        src: *const c_void,
        src_device: i32,
        bytes: usize,
        stream: *mut c_void,
    ) -> oxm_status;
    /// Waits for all work on a device.
    pub fn oxm_synchronize(device: i32) -> oxm_status;
}
