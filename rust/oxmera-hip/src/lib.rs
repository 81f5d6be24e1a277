//! oxmera's `Backend` (crates/oxmera-runtime/src/lib.rs:25-34) on one
//! AMD Instinct MI355X (gfx950), over the C-ABI of `liboxm.so`
//! (include/oxm.h, bound by `oxmera-hip-sys`).
//!
//! * `MatmulOps::matmul` (crates/oxmera-ops/src/lib.rs:52-59) runs the MFMA
//!   GEMM on the operands' own strided views (transposed, sliced and
//!   batch-broadcast operands are read in place, never copied); the output
//!   is a fresh contiguous tensor (:16-17), F32 for F32, BF16 and F16 inputs
//!   (f32 accumulation).
//! * `UnaryOps`, `BinaryOps` (NumPy broadcasting) and `ReduceOps` run the
//!   HBM-bound kernels, for float, integer and boolean dtypes.
//! * Every call is synchronous (the value is ready when it returns), the
//!   library validates everything before launching, and every failure is a
//!   typed `oxmera_core::Error` (`check`).
//!
//! Seam additions this crate relies on in oxmera-core / oxmera-tensor: the
//! `Device::Rocm { index }` variant, `DType::BF16` / `DType::F16`, and a
//! device variant of `Storage` (`DeviceBuffer`, `Storage::from_device_buffer`,
//! `Storage::device_buffer`).

use std::ffi::{CStr, c_void};
use std::sync::Arc;

use oxmera_core::{DType, Device, Error, Layout, Result, Shape, Strides};
use oxmera_hip_sys as sys;
use oxmera_ops::{BinaryOps, MatmulOps, ReduceOps, UnaryOps};
use oxmera_runtime::{Backend, register_backend};
use oxmera_tensor::{DeviceBuffer, Storage, Tensor};

// ---- errors ----------------------------------------------------------------------

/// The operands of a call, for building the typed error of a failed status.
struct Ctx<'a> {
    op: &'static str,
    lhs: Option<&'a Tensor>,
    rhs: Option<&'a Tensor>,
    device: Device,
}

fn last_error() -> String {
    // SAFETY: oxm_last_error returns a NUL-terminated thread-local string that
    // stays valid until the next call on this thread; it is copied at once.
    unsafe { CStr::from_ptr(sys::oxm_last_error()) }.to_string_lossy().into_owned()
}

fn shape_of(t: Option<&Tensor>) -> Shape {
    t.map(|t| t.shape().clone()).unwrap_or_else(|| Shape::new(vec![]))
}

/// Map a C-ABI status onto `oxmera_core::Error` (error.rs:14-102): codes 1-9
/// are the nine variants, one to one, with fields taken from the call's
/// operands and the library's message as the detail where the variant has
/// one.  Codes with no variant (10: a HIP runtime failure, 11: an argument
/// the ABI refuses, such as an output overlapping an input, 12: integer
/// division by zero) become `NotImplemented` carrying the message, until the
/// taxonomy grows variants for them (it is `#[non_exhaustive]`).
fn check(status: sys::oxm_status, cx: &Ctx<'_>) -> Result<()> {
    let lhs_dt = cx.lhs.map(|t| t.dtype()).unwrap_or(DType::F32);
    let rhs_dt = cx.rhs.map(|t| t.dtype()).unwrap_or(lhs_dt);
    let lhs_dev = cx.lhs.map(|t| t.device()).unwrap_or(cx.device);
    let rhs_dev = cx.rhs.map(|t| t.device()).unwrap_or(cx.device);
    match status {
        sys::OXM_OK => Ok(()),
        sys::OXM_E_SHAPE_MISMATCH => Err(Error::ShapeMismatch { expected: shape_of(cx.lhs), got: shape_of(cx.rhs), op: cx.op }),
        sys::OXM_E_BROADCAST_INCOMPATIBLE => Err(Error::BroadcastIncompatible { lhs: shape_of(cx.lhs), rhs: shape_of(cx.rhs) }),
        sys::OXM_E_DTYPE_MISMATCH => Err(Error::DTypeMismatch { expected: lhs_dt, got: rhs_dt, op: cx.op }),
        sys::OXM_E_UNSUPPORTED_DTYPE => Err(Error::UnsupportedDType { dtype: lhs_dt, op: cx.op }),
        sys::OXM_E_DEVICE_MISMATCH => Err(Error::DeviceMismatch { lhs: lhs_dev, rhs: rhs_dev, op: cx.op }),
        sys::OXM_E_INDEX_OUT_OF_BOUNDS => Err(Error::IndexOutOfBounds { index: vec![], shape: shape_of(cx.lhs) }),
        sys::OXM_E_RANK_MISMATCH => Err(Error::RankMismatch {
            index_rank: cx.lhs.map(|t| t.shape().ndim()).unwrap_or(0),
            shape_rank: cx.rhs.map(|t| t.shape().ndim()).unwrap_or(0),
        }),
        sys::OXM_E_BACKEND_UNAVAILABLE => Err(Error::BackendUnavailable { device: cx.device }),
        sys::OXM_E_NOT_IMPLEMENTED => Err(Error::NotImplemented { op: cx.op, detail: last_error() }),
        // no variant in the taxonomy yet: the message says what happened
        _ => Err(Error::NotImplemented { op: cx.op, detail: format!("status {status}: {}", last_error()) }),
    }
}

// ---- device storage ------------------------------------------------------------

/// One `oxm_alloc` block: the opaque handle behind `Storage`'s device
/// variant (crates/oxmera-tensor/src/storage.rs:19-24).  Freed on drop.
#[derive(Debug)]
pub struct HipBuffer {
    ptr: *mut c_void,
    bytes: usize,
    device: i32,
}

// SAFETY: the pointer is a device address owned by this value alone; HIP
// allows freeing and using it from any thread.
unsafe impl Send for HipBuffer {}
// SAFETY: shared references only read the address and the length.
unsafe impl Sync for HipBuffer {}

impl HipBuffer {
    /// `bytes` of device memory on HIP device `device`.
    pub fn alloc(device: usize, bytes: usize) -> Result<Self> {
        let mut ptr = std::ptr::null_mut();
        // SAFETY: `ptr` is a valid out-pointer.
        let st = unsafe { sys::oxm_alloc(device as i32, bytes, &mut ptr) };
        check(st, &Ctx { op: "alloc", lhs: None, rhs: None, device: Device::Rocm { index: device } })?;
        Ok(Self { ptr, bytes, device: device as i32 })
    }
}

impl Drop for HipBuffer {
    fn drop(&mut self) {
        // SAFETY: `ptr` came from oxm_alloc on `device` and is freed once.
        let _ = unsafe { sys::oxm_free(self.device, self.ptr) };
    }
}

impl DeviceBuffer for HipBuffer {
    fn addr(&self) -> u64 {
        self.ptr as u64
    }
    fn len_bytes(&self) -> usize {
        self.bytes
    }
}

/// The C-ABI dtype code.
pub fn dtype_code(dt: DType) -> Result<i32> {
    Ok(match dt {
        DType::F32 => sys::OXM_F32,
        DType::F64 => sys::OXM_F64,
        DType::I32 => sys::OXM_I32,
        DType::I64 => sys::OXM_I64,
        DType::U8 => sys::OXM_U8,
        DType::Bool => sys::OXM_BOOL,
        DType::BF16 => sys::OXM_BF16,
        DType::F16 => sys::OXM_F16,
        other => return Err(Error::UnsupportedDType { dtype: other, op: "hip" }),
    })
}

/// The extents of a shape as the C-ABI's i64s.
pub fn dims(shape: &Shape) -> Vec<i64> {
    shape.dims().iter().map(|&d| d as i64).collect()
}

/// A fresh contiguous tensor of `shape` and `dtype` on HIP device `index`
/// (uninitialised device memory; every op overwrites its output).
pub fn device_empty(shape: Shape, dtype: DType, index: usize) -> Result<Tensor> {
    let bytes = shape.numel() * dtype.size_in_bytes();
    let buf: Arc<dyn DeviceBuffer> = Arc::new(HipBuffer::alloc(index, bytes.max(1))?);
    let storage = Storage::from_device_buffer(buf, dtype, Device::Rocm { index });
    Tensor::from_storage(Arc::new(storage), Layout::contiguous(shape))
}

/// A tensor's `oxm_view` plus the arrays it points into (kept alive with it).
struct View {
    v: sys::oxm_view,
    _shape: Vec<i64>,
    _strides: Vec<i64>,
}

fn view(t: &Tensor) -> Result<View> {
    let storage = t.storage();
    let (data, device) = match (storage.device_buffer(), t.device()) {
        (Some(b), Device::Rocm { index }) => (b.addr() as *mut c_void, index as i32),
        (None, Device::Cpu) => (storage.cpu_bytes().map_or(std::ptr::null(), |b| b.as_ptr()) as *mut c_void, -1),
        (_, dev) => return Err(Error::DeviceMismatch { lhs: dev, rhs: dev, op: "hip" }),
    };
    let layout = t.layout();
    let shape = dims(&layout.shape);
    let strides: Vec<i64> = layout.strides.values().iter().map(|&s| s as i64).collect();
    let v = sys::oxm_view {
        data,
        dtype: dtype_code(t.dtype())?,
        ndim: shape.len() as i32,
        shape: shape.as_ptr(),
        strides: strides.as_ptr(),
        offset: layout.offset as i64,
        device,
    };
    Ok(View { v, _shape: shape, _strides: strides })
}

// ---- the backend -----------------------------------------------------------------

/// The MI355X backend for HIP device `index`.
#[derive(Debug)]
pub struct HipBackend {
    index: usize,
}

impl HipBackend {
    /// A backend for HIP device `index`; `BackendUnavailable` when the HIP
    /// runtime does not see that device.
    pub fn new(index: usize) -> Result<Self> {
        let mut n = 0i32;
        // SAFETY: `n` is a valid out-pointer.
        let st = unsafe { sys::oxm_device_count(&mut n) };
        let device = Device::Rocm { index };
        check(st, &Ctx { op: "device_count", lhs: None, rhs: None, device })?;
        if index >= n as usize {
            return Err(Error::BackendUnavailable { device });
        }
        Ok(Self { index })
    }

    fn cx<'a>(&self, op: &'static str, lhs: Option<&'a Tensor>, rhs: Option<&'a Tensor>) -> Ctx<'a> {
        Ctx { op, lhs, rhs, device: Device::Rocm { index: self.index } }
    }

    /// `lhs . rhs` into `out` (caller-allocated, contiguous, of the inferred
    /// shape; F32, or BF16 / F16 for 16-bit inputs) with a fused epilogue:
    /// the path oxmera-nn's Linear layers take (bias + GELU forward, GELU'
    /// backward, column sums of the output for the bias gradient).
    pub fn matmul_into(&self, lhs: &Tensor, rhs: &Tensor, out: &Tensor, ep: Option<&sys::oxm_epilogue>) -> Result<()> {
        let (a, b, c) = (view(lhs)?, view(rhs)?, view(out)?);
        let epp = ep.map_or(std::ptr::null(), |e| e as *const _);
        // SAFETY: the views point at live storage and arrays held by `a`,
        // `b`, `c`; a NULL stream makes the call synchronous.
        let st = unsafe { sys::oxm_gemm(&a.v, &b.v, &c.v, epp, std::ptr::null_mut()) };
        check(st, &self.cx("matmul", Some(lhs), Some(rhs)))
    }

    fn unary(&self, op: i32, name: &'static str, a: &Tensor) -> Result<Tensor> {
        let out = device_empty(a.shape().clone(), a.dtype(), self.index)?;
        let (x, o) = (view(a)?, view(&out)?);
        // SAFETY: as in matmul_into.
        let st = unsafe { sys::oxm_unary(op, &x.v, &o.v, std::ptr::null_mut()) };
        check(st, &self.cx(name, Some(a), None))?;
        Ok(out)
    }

    fn binary(&self, op: i32, name: &'static str, lhs: &Tensor, rhs: &Tensor) -> Result<Tensor> {
        let shape = oxmera_core::shape::broadcast_shapes(lhs.shape(), rhs.shape())?;
        let out = device_empty(shape, lhs.dtype(), self.index)?;
        let (a, b, o) = (view(lhs)?, view(rhs)?, view(&out)?);
        // SAFETY: as in matmul_into.
        let st = unsafe { sys::oxm_binary(op, &a.v, &b.v, &o.v, std::ptr::null_mut()) };
        check(st, &self.cx(name, Some(lhs), Some(rhs)))?;
        Ok(out)
    }

    fn reduce(&self, op: i32, name: &'static str, a: &Tensor, axes: &[usize]) -> Result<Tensor> {
        let ax: Vec<i32> = axes.iter().map(|&x| x as i32).collect();
        let x = view(a)?;
        let mut nd = 0i32;
        let mut shp = [0i64; sys::OXM_MAX_DIMS];
        // SAFETY: `ax` and `shp` are live arrays of the stated lengths.
        let st = unsafe { sys::oxm_reduce_infer(&x.v, ax.as_ptr(), ax.len() as i32, &mut nd, shp.as_mut_ptr()) };
        check(st, &self.cx(name, Some(a), None))?;
        let shape = Shape::new(shp[..nd as usize].iter().map(|&d| d as usize).collect());
        let out = device_empty(shape, a.dtype(), self.index)?;
        let o = view(&out)?;
        // SAFETY: as above.
        let st = unsafe { sys::oxm_reduce(op, &x.v, ax.as_ptr(), ax.len() as i32, &o.v, std::ptr::null_mut()) };
        check(st, &self.cx(name, Some(a), None))?;
        Ok(out)
    }

    /// `Tensor::contiguous` on the device (crates/oxmera-tensor/src/tensor.rs:
    /// 86-90): a clone when already contiguous, else a fresh copy.
    pub fn contiguous(&self, a: &Tensor) -> Result<Tensor> {
        if a.layout().is_contiguous() {
            return Ok(a.clone());
        }
        let out = device_empty(a.shape().clone(), a.dtype(), self.index)?;
        let (x, o) = (view(a)?, view(&out)?);
        // SAFETY: as in matmul_into.
        let st = unsafe { sys::oxm_copy_view(&x.v, &o.v, std::ptr::null_mut()) };
        check(st, &self.cx("contiguous", Some(a), None))?;
        Ok(out)
    }

    /// A contiguous CPU tensor's bytes copied into fresh device storage.
    pub fn to_device(&self, host: &Tensor) -> Result<Tensor> {
        let bytes = host
            .storage()
            .cpu_bytes()
            .ok_or(Error::DeviceMismatch { lhs: host.device(), rhs: Device::Cpu, op: "to_device" })?;
        if !host.layout().is_contiguous() {
            return Err(Error::NotImplemented { op: "to_device", detail: "a non-contiguous host view".into() });
        }
        let es = host.dtype().size_in_bytes();
        let n = host.shape().numel() * es;
        let start = host.layout().offset * es;
        let out = device_empty(host.shape().clone(), host.dtype(), self.index)?;
        let dst = out.storage().device_buffer().map(|b| b.addr()).unwrap_or(0) as *mut c_void;
        // SAFETY: `bytes[start..start + n]` lies in the host storage (the
        // layout is contiguous and was validated by Tensor::from_storage);
        // `dst` is a fresh allocation of n bytes.
        let st = unsafe {
            sys::oxm_copy(dst, self.index as i32, bytes[start..start + n].as_ptr() as *const c_void, -1, n, std::ptr::null_mut())
        };
        check(st, &self.cx("to_device", Some(host), None))?;
        Ok(out)
    }

    /// A device tensor's elements in logical order, as a contiguous CPU tensor.
    pub fn to_host(&self, t: &Tensor) -> Result<Tensor> {
        let c = self.contiguous(t)?;
        let es = c.dtype().size_in_bytes();
        let n = c.shape().numel() * es;
        let mut bytes = vec![0u8; n];
        let src = c.storage().device_buffer().map(|b| b.addr()).unwrap_or(0) + (c.layout().offset * es) as u64;
        // SAFETY: `bytes` holds n bytes; the source range lies in the device
        // allocation (the library checks it against its allocation registry).
        let st = unsafe {
            sys::oxm_copy(bytes.as_mut_ptr() as *mut c_void, -1, src as *const c_void, self.index as i32, n, std::ptr::null_mut())
        };
        check(st, &self.cx("to_host", Some(t), None))?;
        let storage = Storage::cpu_from_bytes(bytes, c.dtype());
        Tensor::from_storage(Arc::new(storage), Layout::contiguous(c.shape().clone()))
    }
}

impl MatmulOps for HipBackend {
    fn matmul(&self, lhs: &Tensor, rhs: &Tensor) -> Result<Tensor> {
        let (a, b) = (view(lhs)?, view(rhs)?);
        let mut nd = 0i32;
        let mut shp = [0i64; sys::OXM_MAX_DIMS];
        // SAFETY: `shp` holds OXM_MAX_DIMS entries.
        let st = unsafe { sys::oxm_gemm_infer(&a.v, &b.v, &mut nd, shp.as_mut_ptr()) };
        check(st, &self.cx("matmul", Some(lhs), Some(rhs)))?;
        let shape = Shape::new(shp[..nd as usize].iter().map(|&d| d as usize).collect());
        let out = device_empty(shape, DType::F32, self.index)?;
        self.matmul_into(lhs, rhs, &out, None)?;
        Ok(out)
    }
}

impl UnaryOps for HipBackend {
    fn neg(&self, a: &Tensor) -> Result<Tensor> {
        self.unary(sys::OXM_UN_NEG, "neg", a)
    }
    fn exp(&self, a: &Tensor) -> Result<Tensor> {
        self.unary(sys::OXM_UN_EXP, "exp", a)
    }
    fn ln(&self, a: &Tensor) -> Result<Tensor> {
        self.unary(sys::OXM_UN_LN, "ln", a)
    }
    fn abs(&self, a: &Tensor) -> Result<Tensor> {
        self.unary(sys::OXM_UN_ABS, "abs", a)
    }
}

impl BinaryOps for HipBackend {
    fn add(&self, lhs: &Tensor, rhs: &Tensor) -> Result<Tensor> {
        self.binary(sys::OXM_BIN_ADD, "add", lhs, rhs)
    }
    fn sub(&self, lhs: &Tensor, rhs: &Tensor) -> Result<Tensor> {
        self.binary(sys::OXM_BIN_SUB, "sub", lhs, rhs)
    }
    fn mul(&self, lhs: &Tensor, rhs: &Tensor) -> Result<Tensor> {
        self.binary(sys::OXM_BIN_MUL, "mul", lhs, rhs)
    }
    fn div(&self, lhs: &Tensor, rhs: &Tensor) -> Result<Tensor> {
        self.binary(sys::OXM_BIN_DIV, "div", lhs, rhs)
    }
}

impl ReduceOps for HipBackend {
    fn sum(&self, a: &Tensor, axes: &[usize]) -> Result<Tensor> {
        self.reduce(sys::OXM_RED_SUM, "sum", a, axes)
    }
    fn max(&self, a: &Tensor, axes: &[usize]) -> Result<Tensor> {
        self.reduce(sys::OXM_RED_MAX, "max", a, axes)
    }
}

impl Backend for HipBackend {
    fn device(&self) -> Device {
        Device::Rocm { index: self.index }
    }
    fn name(&self) -> &'static str {
        "hip-gfx950"
    }
}

/// Register the backend of HIP device `index` with the runtime
/// (crates/oxmera-runtime/src/lib.rs:46-53), so that `backend_for(Device::
/// Rocm { index })` and `TensorOps` resolve to it.
pub fn register(index: usize) -> Result<Arc<HipBackend>> {
    let be = Arc::new(HipBackend::new(index)?);
    register_backend(be.clone());
    Ok(be)
}

/// Strides of a contiguous row-major shape, as oxmera's `Strides`.
pub fn row_major(shape: &Shape) -> Strides {
    let mut acc = 1isize;
    let mut s = vec![0isize; shape.ndim()];
    for (i, &d) in shape.dims().iter().enumerate().rev() {
        s[i] = acc;
        acc *= d as isize;
    }
    Strides::new(s)
}

#[cfg(test)]
mod tests {
    //! The A4 spec cases (exercises/a4-reference-matmul/tests/spec.rs:31-94)
    //! on the GPU when one is present; skipped (returning early) otherwise.
    use super::*;

    fn dev() -> Option<HipBackend> {
        HipBackend::new(0).ok()
    }

    fn t(be: &HipBackend, v: &[f32], shape: &[usize]) -> Tensor {
        let host = Tensor::from_vec_f32(v.to_vec(), Shape::new(shape.to_vec())).unwrap();
        be.to_device(&host).unwrap()
    }

    fn vals(be: &HipBackend, x: &Tensor) -> Vec<f32> {
        let h = be.to_host(x).unwrap();
        h.storage().cpu_bytes().unwrap().chunks(4).map(|c| f32::from_le_bytes([c[0], c[1], c[2], c[3]])).collect()
    }

    #[test]
    fn a4_cases_on_the_device() {
        let Some(be) = dev() else { return };
        let a = t(&be, &[1., 2., 3., 4.], &[2, 2]);
        let b = t(&be, &[5., 6., 7., 8.], &[2, 2]);
        assert_eq!(vals(&be, &be.matmul(&a, &b).unwrap()), vec![19., 22., 43., 50.]);
        let r = t(&be, &[1., 2., 3., 4., 5., 6.], &[2, 3]);
        let c = t(&be, &[1., 10., 100.], &[3, 1]);
        assert_eq!(vals(&be, &be.matmul(&r, &c).unwrap()), vec![321., 654.]);
        // a transposed view, read in place
        let bt = t(&be, &[5., 7., 6., 8.], &[2, 2]).permute(&[1, 0]).unwrap();
        assert_eq!(vals(&be, &be.matmul(&a, &bt).unwrap()), vec![19., 22., 43., 50.]);
    }

    #[test]
    fn refusals_are_typed() {
        let Some(be) = dev() else { return };
        let a = t(&be, &[0.; 6], &[2, 3]);
        let b = t(&be, &[0.; 8], &[4, 2]);
        assert!(matches!(be.matmul(&a, &b), Err(Error::ShapeMismatch { .. })));
        let v = t(&be, &[0.; 6], &[6]);
        assert!(matches!(be.matmul(&v, &v), Err(Error::RankMismatch { .. })));
    }
}
