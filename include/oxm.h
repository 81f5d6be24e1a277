/*
 * oxm.h -- C-ABI of the MI355X (gfx950) GEMM backend for oxmera.
 *
 * This is the boundary a Rust FFI crate (`oxmera-hip-sys`) binds; a safe
 * `oxmera-hip` crate implements oxmera's `Backend` on top of it and registers
 * it with the runtime.  Every entry point below names the reference interface
 * it serves.  Plain pointers and sizes only; no exception or abort crosses it.
 *
 * Conventions
 *  - Views follow oxmera's Layout (crates/oxmera-core/src/layout.rs:24-34):
 *    shape, ELEMENT strides (signed: flipped views are representable,
 *    layout.rs:6-10) and an element offset into the buffer at `data`.
 *  - The caller owns every buffer.  Outputs are caller-allocated, contiguous,
 *    sized by oxm_gemm_infer ("the output of every operation is a fresh
 *    contiguous tensor on the operands' device", crates/oxmera-ops/src/lib.rs:16-17).
 *  - Status codes map 1:1 onto oxmera_core::Error variants
 *    (crates/oxmera-core/src/error.rs:14-102); oxm_last_error() returns a
 *    thread-local message naming the operation and its operands.
 *  - Validation runs completely before any device work is launched.  A view
 *    whose element count or byte range would overflow int64 is
 *    OXM_E_INDEX_OUT_OF_BOUNDS.  An output that shares memory with an input
 *    (or with another output of the same call) is OXM_E_INVALID_ARGUMENT:
 *    outputs are fresh storage (crates/oxmera-ops/src/lib.rs:16-17).  The
 *    one exception is an elementwise input that IS the output element for
 *    element (same first element and strides), which unary and binary ops
 *    accept (in-place update).
 *  - stream == NULL: the call is synchronous (the result may be read as soon
 *    as it returns, as MatmulOps::matmul returns a value).  A non-NULL
 *    hipStream_t makes it asynchronous on that stream.
 *  - Entry points are thread-safe (Backend: Send + Sync,
 *    crates/oxmera-runtime/src/lib.rs:29).
 */
#ifndef OXM_H
#define OXM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* oxmera_core::Error (error.rs:14-102), one code per variant, plus OXM_E_HIP
 * for a HIP runtime failure and OXM_E_INVALID_ARGUMENT for a NULL or
 * malformed argument at the ABI itself. */
typedef enum {
    OXM_OK = 0,
    OXM_E_SHAPE_MISMATCH = 1,         /* Error::ShapeMismatch          error.rs:16-25 */
    OXM_E_BROADCAST_INCOMPATIBLE = 2, /* Error::BroadcastIncompatible  error.rs:27-34 */
    OXM_E_DTYPE_MISMATCH = 3,         /* Error::DTypeMismatch          error.rs:36-45 */
    OXM_E_UNSUPPORTED_DTYPE = 4,      /* Error::UnsupportedDType       error.rs:47-54 */
    OXM_E_DEVICE_MISMATCH = 5,        /* Error::DeviceMismatch         error.rs:56-65 */
    OXM_E_INDEX_OUT_OF_BOUNDS = 6,    /* Error::IndexOutOfBounds       error.rs:67-74 */
    OXM_E_RANK_MISMATCH = 7,          /* Error::RankMismatch           error.rs:76-83 */
    OXM_E_BACKEND_UNAVAILABLE = 8,    /* Error::BackendUnavailable     error.rs:85-90 */
    OXM_E_NOT_IMPLEMENTED = 9,        /* Error::NotImplemented         error.rs:92-101 */
    OXM_E_HIP = 10,
    OXM_E_INVALID_ARGUMENT = 11,
    /* The typed error BinaryOps::div promises for integer division by zero
     * (crates/oxmera-ops/src/lib.rs:47-48).  oxmera_core::Error has no
     * variant for it yet (the enum is #[non_exhaustive], error.rs:13). */
    OXM_E_DIVISION_BY_ZERO = 12
} oxm_status;

/* oxmera_core::DType (dtype.rs:9-22) in declaration order, plus BF16 and F16,
 * which this backend carries end to end (dtype.rs:5-6). */
typedef enum {
    OXM_F32 = 0,
    OXM_F64 = 1,
    OXM_I32 = 2,
    OXM_I64 = 3,
    OXM_U8 = 4,
    OXM_BOOL = 5,
    OXM_BF16 = 6,
    OXM_F16 = 7
} oxm_dtype;

/* Epilogue activation applied in the GEMM's store stage.  GELU_GRAD and
 * MUL_AUX are the pair a training step uses: the forward saves GELU'(z) (one
 * more multiply-add on the normal CDF and density GELU computes anyway) and
 * the backward multiplies by it, instead of saving z and evaluating GELU'(z)
 * again in the backward's epilogue. */
typedef enum {
    OXM_ACT_NONE = 0,      /* out = acc + bias                                        */
    OXM_ACT_GELU = 1,      /* aux_out = acc + bias; out = GELU_erf(acc + bias)        */
    OXM_ACT_DGELU = 2,     /* out = acc * GELU_erf'(aux[m,n])  (backward of GELU)      */
    OXM_ACT_GELU_GRAD = 3, /* aux_out = GELU_erf'(acc + bias); out = GELU_erf(acc + bias) */
    OXM_ACT_MUL_AUX = 4    /* out = acc * aux[m,n]  (backward of GELU from GELU_GRAD's aux) */
} oxm_act;

#define OXM_MAX_DIMS 8

/* A strided view: oxmera_tensor::Tensor's Layout over its Storage
 * (crates/oxmera-tensor/src/tensor.rs:15-19, layout.rs:24-34).
 * device: -1 = host memory, >= 0 = HIP device index (Device, device.rs:10-24). */
typedef struct {
    void *data;
    int32_t dtype;           /* oxm_dtype */
    int32_t ndim;
    const int64_t *shape;
    const int64_t *strides;  /* elements, signed */
    int64_t offset;          /* elements */
    int32_t device;
} oxm_view;

/* Fused epilogue.  bias: [N] of bias_dtype on the device, or NULL (not
 * applied under DGELU / MUL_AUX).  aux: a contiguous [batch..., M, N] buffer of
 * out_dtype: written with the pre-activation for OXM_ACT_GELU or with
 * GELU'(pre-activation) for OXM_ACT_GELU_GRAD (may be NULL), read as Z for
 * OXM_ACT_DGELU and as the factor for OXM_ACT_MUL_AUX (required).  out_dtype must equal the dtype of the output view.
 * colsum: an F32 [N] device buffer, or NULL; when set, the call overwrites it
 * with the sums over all rows (and batches) of the output AS STORED (after
 * rounding to the output dtype) -- the bias gradient of a Linear layer whose
 * input gradient this GEMM produces (ReduceOps::sum over rows,
 * crates/oxmera-ops/src/lib.rs:61-69, fused into the producer). */
typedef struct {
    const void *bias;
    int32_t bias_dtype;
    int32_t act;             /* oxm_act */
    void *aux;
    float *colsum;
} oxm_epilogue;

/* Library version string. */
const char *oxm_version(void);

/* Thread-local description of the last failure on this thread: the operation
 * and its operands (exercises/a5-error-taxonomy/tests/spec.rs:62-80). */
const char *oxm_last_error(void);

/* Number of HIP devices this backend can serve; OXM_E_BACKEND_UNAVAILABLE when
 * the HIP runtime finds none (backend_for's typed refusal,
 * crates/oxmera-runtime/src/lib.rs:36-44). */
oxm_status oxm_device_count(int32_t *count);

/* Backend::name() (crates/oxmera-runtime/src/lib.rs:33). */
const char *oxm_backend_name(void);

/* The bytes a view can address, relative to v->data: [*lo_bytes, *hi_bytes)
 * (both 0 for an empty view).  Tensor::from_storage's rule
 * (crates/oxmera-tensor/src/tensor.rs:21-28) needs exactly this range to lie
 * inside the storage; every product and sum is overflow-checked, and a range
 * that does not fit int64 is OXM_E_INDEX_OUT_OF_BOUNDS.  Host-only: it
 * touches no device and needs no GPU. */
oxm_status oxm_view_byte_range(const oxm_view *v, int64_t *lo_bytes, int64_t *hi_bytes);

/* broadcast_shapes (crates/oxmera-core/src/shape.rs:45-58): NumPy rules; on
 * refusal OXM_E_BROADCAST_INCOMPATIBLE and the message carries both operands
 * verbatim (exercises/a2-broadcasting/tests/spec.rs:38-54). */
oxm_status oxm_broadcast_shapes(int32_t lhs_ndim, const int64_t *lhs, int32_t rhs_ndim, const int64_t *rhs,
                                int32_t *out_ndim, int64_t *out_shape);

/* Shape rules of MatmulOps::matmul (crates/oxmera-ops/src/lib.rs:52-59),
 * extended to rank >= 2 with NumPy batch broadcasting over the leading dims:
 * [..., m, k] x [..., k, n] -> [broadcast(...), m, n].  Rank < 2 is
 * OXM_E_RANK_MISMATCH, an inner-dim mismatch OXM_E_SHAPE_MISMATCH,
 * differing dtypes OXM_E_DTYPE_MISMATCH.  out_shape holds OXM_MAX_DIMS. */
oxm_status oxm_gemm_infer(const oxm_view *a, const oxm_view *b, int32_t *out_ndim, int64_t *out_shape);

/* MatmulOps::matmul (crates/oxmera-ops/src/lib.rs:52-59; reference body
 * CpuBackend::matmul, crates/oxmera-cpu/src/lib.rs:71-76), on the GPU:
 * c = epilogue(a . b).  a, b: any strided views (transposed, sliced,
 * broadcast batch dims) of F32, BF16 or F16 on one device; they are read in
 * place, never copied.  c: contiguous view of the inferred shape, F32 for F32
 * inputs, F32/BF16/F16 for 16-bit inputs (f32 accumulation throughout).
 * ep may be NULL (plain matmul).  stream: hipStream_t or NULL. */
oxm_status oxm_gemm(const oxm_view *a, const oxm_view *b, const oxm_view *c, const oxm_epilogue *ep,
                    void *stream);

/* ReduceOps::sum over one axis of a rank-2 contiguous tensor
 * (crates/oxmera-ops/src/lib.rs:61-69): out[c] = sum_r x[r, c] (axis 0) with
 * f32 accumulation.  The bias gradient of oxmera-nn Linear.  x: F32/BF16/F16
 * [R, C] contiguous view on the device; out: F32 [C] contiguous view. */
oxm_status oxm_sum_rows(const oxm_view *x, const oxm_view *out, void *stream);

/* Mean-squared-error loss and its gradient (the MLP's objective; composed in
 * the reference from BinaryOps::sub/mul and ReduceOps::sum,
 * crates/oxmera-ops/src/lib.rs:39-69): loss[0] = mean((y - t)^2) (f32, device),
 * dy = 2 (y - t) / numel in dy's dtype.  y, t, dy: contiguous, same shape.
 * dy_colsum: NULL, or an F32 [C] view (C = the last dimension) that receives
 * the sums over the leading dimensions of dy as stored -- the bias gradient of
 * the layer that produced y, in the same pass. */
oxm_status oxm_mse_loss_grad(const oxm_view *y, const oxm_view *t, const oxm_view *loss, const oxm_view *dy,
                             const oxm_view *dy_colsum, void *stream);

/* UnaryOps (crates/oxmera-ops/src/lib.rs:27-37): out = op(x) elementwise.
 * x: any strided view on a HIP device; out: a contiguous view of x's shape
 * and dtype ("a fresh contiguous tensor", :16-17).  Float dtypes (F32, F64,
 * BF16, F16): every op; exp and ln follow the device's IEEE-754 float
 * functions (ln of a negative is NaN, of zero -inf).  I32 / I64 / U8: neg
 * and abs, wrapping (neg(i32::MIN) = abs(i32::MIN) = i32::MIN, neg of a U8
 * is 256 - x mod 256); Bool: abs (the identity).  exp and ln are "float
 * dtypes only" (:31-34): OXM_E_UNSUPPORTED_DTYPE, as is any other
 * unsupported pairing. */
typedef enum {
    OXM_UN_NEG = 0,
    OXM_UN_EXP = 1,
    OXM_UN_LN = 2,
    OXM_UN_ABS = 3,
    /* sign(x) in {-1, 0, +1}, NaN for NaN: no counterpart among the
     * reference's UnaryOps; the derivative of abs for the autograd tape. */
    OXM_UN_SIGN = 4
} oxm_unary_op;
oxm_status oxm_unary(int32_t op, const oxm_view *x, const oxm_view *out, void *stream);

/* BinaryOps (crates/oxmera-ops/src/lib.rs:39-50): out = a op b with NumPy
 * broadcasting (crates/oxmera-core/src/shape.rs:45-58; BroadcastIncompatible
 * otherwise).  a, b: same dtype and device, any strides; out: contiguous,
 * the broadcast shape.  Float division follows IEEE-754.  I32 / I64 / U8:
 * add, sub, mul wrap; div truncates toward zero (i32::MIN / -1 wraps to
 * i32::MIN) and a zero divisor anywhere is OXM_E_DIVISION_BY_ZERO (integer
 * div then runs synchronously on `stream`, to know it before returning;
 * the output holds 0 where the divisor was 0).  Bool: add is OR, mul is
 * AND; sub and div are OXM_E_UNSUPPORTED_DTYPE.  eq: every dtype. */
typedef enum {
    OXM_BIN_ADD = 0,
    OXM_BIN_SUB = 1,
    OXM_BIN_MUL = 2,
    OXM_BIN_DIV = 3,
    /* The two below have no counterpart among the reference's BinaryOps;
     * the autograd tape uses them.  EQ: 1 where a == b, else 0 (the mask of
     * max's gradient).  DGELU: a * GELU'(b) with the erf GELU, the
     * gradient through a GELU whose pre-activation is b. */
    OXM_BIN_EQ = 4,
    OXM_BIN_DGELU = 5
} oxm_binary_op;
oxm_status oxm_binary(int32_t op, const oxm_view *a, const oxm_view *b, const oxm_view *out, void *stream);

/* ReduceOps (crates/oxmera-ops/src/lib.rs:61-69): sum or max over `axes`,
 * removing them from the shape; naxes == 0 means every axis (a rank-0
 * result).  Float dtypes: accumulation in f32 (f64 for F64), one rounding to
 * the output dtype, a fixed combination order (results do not depend on
 * scheduling).  I32 / I64 / U8: sum wraps in the dtype (the exact sum modulo
 * 2^bits, whatever the order), max is exact; Bool: sum and max are OR.
 * max propagates NaN and refuses an empty reduced extent (ShapeMismatch:
 * "there is no identity to invent").  oxm_reduce_infer gives the output
 * shape; out must be contiguous with it and x's dtype. */
typedef enum { OXM_RED_SUM = 0, OXM_RED_MAX = 1 } oxm_reduce_op;
oxm_status oxm_reduce_infer(const oxm_view *x, const int32_t *axes, int32_t naxes, int32_t *out_ndim,
                            int64_t *out_shape);
oxm_status oxm_reduce(int32_t op, const oxm_view *x, const int32_t *axes, int32_t naxes, const oxm_view *out,
                      void *stream);

/* oxm_reduce with no allocation: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): the partial results
 * of a split reduction go to a static per-GPU scratch area of
 * OXM_REDUCE_SCRATCH_BYTES that the library holds until the process ends,
 * instead of a stream allocation, and the call allocates nothing (integer
 * reductions never need it).  Same arguments, checks and results as
 * oxm_reduce; a reduction whose partials would not fit is
 * OXM_E_NOT_IMPLEMENTED.  Every call on one GPU shares that GPU's scratch:
 * calls that overlap in time on one GPU (other threads, other streams) race
 * and must be serialised by the caller. */
#define OXM_REDUCE_SCRATCH_BYTES (8u << 20)
oxm_status oxm_reduce_noalloc(int32_t op, const oxm_view *x, const int32_t *axes, int32_t naxes,
                              const oxm_view *out, void *stream);

/* Tensor::contiguous's copy (crates/oxmera-tensor/src/tensor.rs:86-90):
 * dst = src element by element, bits unchanged.  Same shape and dtype, same
 * HIP device; src any strides, dst any strides that do not repeat elements
 * (a contiguous dst gives contiguous()). */
oxm_status oxm_copy_view(const oxm_view *src, const oxm_view *dst, void *stream);

/* dst = src converted element by element between float dtypes (F32, F64,
 * BF16, F16): widened exactly, rounded once to nearest-even (F64 -> 16-bit
 * rounds through f32).  Same shape and HIP device; src any strides, dst any
 * strides that do not repeat elements.  No counterpart in the reference
 * (it has no dtype conversion yet); the autograd tape uses it where a
 * gradient's dtype differs from its operand's (an f32 GEMM result flowing
 * back into a 16-bit operand). */
oxm_status oxm_convert(const oxm_view *src, const oxm_view *dst, void *stream);

/* One SGD step over one parameter, in place, fused (the reserved
 * crates/oxmera-optim/src/lib.rs:1-11 defines no optimizer yet; semantics
 * as torch.optim.SGD with dampening 0), per element in f32 with each
 * operation rounded separately (no fused multiply-add):
 *   g = grad (+ weight_decay * p)
 *   momentum != 0:  v = momentum * v + g;  g = nesterov ? g + momentum * v : v
 *   p = p - lr * g, rounded once to p's dtype.
 * param: contiguous F32, BF16 or F16; grad: contiguous, same shape, F32 or
 * param's dtype; velocity: NULL when momentum == 0, else a contiguous F32
 * buffer of the same shape (zeros before the first step). */
oxm_status oxm_sgd_step(const oxm_view *param, const oxm_view *grad, const oxm_view *velocity, float lr,
                        float momentum, float weight_decay, int32_t nesterov, void *stream);

/* Storage for device tensors (crates/oxmera-tensor/src/storage.rs:12-32,
 * "GPU variants hold opaque backend handles", :19-24). */
oxm_status oxm_alloc(int32_t device, size_t bytes, void **out);
oxm_status oxm_free(int32_t device, void *ptr);

/* Byte copy between host (-1) and device (>= 0) memory.  stream == NULL:
 * synchronous.  Otherwise the copy is ordered after the work already queued
 * on `stream`; a copy to or from host memory also completes before the call
 * returns (so the host buffer may be read or freed at once), a device-to-
 * device copy stays asynchronous.  Overlapping device ranges are
 * OXM_E_INVALID_ARGUMENT. */
oxm_status oxm_copy(void *dst, int32_t dst_device, const void *src, int32_t src_device, size_t bytes, void *stream);

/* Wait for all work on the device. */
oxm_status oxm_synchronize(int32_t device);

#ifdef __cplusplus
}
#endif

#endif /* OXM_H */
