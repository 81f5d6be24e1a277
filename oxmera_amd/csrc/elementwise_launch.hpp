// elementwise_launch.hpp -- host <-> kernel interface of elementwise.hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace oxm {

constexpr int kDtF64 = 1;  // oxm_dtype F64 (F32 = 0, BF16 = 6, F16 = 7 are in gemm_kernels.hpp)
constexpr int kDtI32 = 2, kDtI64 = 3, kDtU8 = 4, kDtBool = 5;  // oxm_dtype integer / boolean codes

enum UnaryOp : int { kUnNeg = 0, kUnExp = 1, kUnLn = 2, kUnAbs = 3, kUnSign = 4 };
enum BinaryOp : int { kBinAdd = 0, kBinSub = 1, kBinMul = 2, kBinDiv = 3, kBinEq = 4, kBinDGelu = 5 };
enum ReduceOp : int { kRedSum = 0, kRedMax = 1 };

constexpr int kEwMaxDims = 8;

// A row-major iteration space over the output shape and, per operand
// (0 = output, 1 and 2 = inputs), its element strides (0 on broadcast dims).
struct EwShape {
    int32_t ndim;  // >= 1
    int64_t numel;
    int64_t shape[kEwMaxDims];
    int64_t st[3][kEwMaxDims];
};

// out[o] = reduce over the reduced dims; the output (kept dims, row-major)
// is contiguous.  Strides are the input's.
struct RedGeom {
    int32_t nk, nr;  // nk >= 1 (a scalar output is one kept dim of extent 1), nr >= 1
    int64_t n_out, n_red;
    int64_t kshape[kEwMaxDims], kst[kEwMaxDims];
    int64_t rshape[kEwMaxDims], rst[kEwMaxDims];
};

// Vector paths of an elementwise launch.  kEwContig16: every operand
// contiguous over s (one dim), 16-byte aligned, numel a multiple of 16 bytes.
// kEwInner16: every operand of stride 1 or 0 along the innermost dim (the
// output 1), that extent a multiple of 16 bytes, stride-1 operands' vectors
// 16-byte aligned.  kEwScalar: anything else.
enum EwVec { kEwScalar = 0, kEwContig16 = 1, kEwInner16 = 2 };

// nops 1: out = op(x); nops 2: out = op(x, y).  vec: an EwVec the caller has
// checked s and the pointers against.
hipError_t launch_elementwise(int dtype, int nops, int op, const EwShape &s, void *out, const void *x, const void *y,
                              int vec, hipStream_t st);

// Element copy of elem_bytes-sized elements from a strided view (operand 1)
// to a strided destination (operand 0), bits unchanged.
hipError_t launch_copy(int elem_bytes, const EwShape &s, void *dst, const void *src, bool contig16, hipStream_t st);

// ws: nullptr (a workspace is allocated on the stream when the schedule
// splits), or a device buffer of at least reduce_workspace_bytes(...).
hipError_t launch_reduce(int dtype, int op, const RedGeom &g, const void *x, void *out, hipStream_t st,
                         void *ws = nullptr);
size_t reduce_workspace_bytes(int dtype, const RedGeom &g, const void *x);

// The static workspace of oxm_reduce_noalloc (elementwise.hip): its size, and
// its device address on the current device (looked up once per device).
constexpr size_t kReduceScratchBytes = size_t(8) << 20;
constexpr int kMaxScratchDevices = 64;
hipError_t reduce_scratch(void **ptr);

// The same for I32 / I64 / U8 / Bool (elementwise_int.hip): unary neg / abs,
// binary add / sub / mul / div / eq, reduce sum / max; the host has refused
// the combinations a dtype does not carry.  Integer div stores 1 to
// *zero_div (a device int the caller cleared) when a divisor is zero.
hipError_t launch_elementwise_int(int dtype, int nops, int op, const EwShape &s, void *out, const void *x,
                                  const void *y, int *zero_div, hipStream_t st);
hipError_t launch_reduce_int(int dtype, int op, const RedGeom &g, const void *x, void *out, hipStream_t st);

// dst = src converted from dtype dti to dtype dto (float dtypes); operand 0
// of s is dst, operand 1 src.
hipError_t launch_convert(int dti, int dto, const EwShape &s, void *dst, const void *src, hipStream_t st);

// One fused SGD step over n contiguous elements (see oxm_sgd_step); v is
// null when momentum == 0.
hipError_t launch_sgd(int pdt, int gdt, int64_t n, void *p, const void *g, float *v, float lr, float momentum,
                      float weight_decay, bool nesterov, hipStream_t st);

}  // namespace oxm
