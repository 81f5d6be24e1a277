// elementwise_int.hip -- UnaryOps, BinaryOps and ReduceOps for oxmera's
// integer and boolean dtypes (I32, I64, U8, Bool; crates/oxmera-core/src/
// dtype.rs:9-22) on gfx950.
//
// Semantics (the float ops live in elementwise.hip):
//  * I32 / I64 / U8 arithmetic wraps (two's complement / modulo 2^8), as
//    Rust's wrapping_* operations and NumPy's fixed-width integers do:
//    i32::MIN negated or made absolute stays i32::MIN, 250u8 + 10 = 4.
//  * div truncates toward zero (Rust's `/`); i32::MIN / -1 wraps to
//    i32::MIN (wrapping_div).  A zero divisor anywhere makes the call fail
//    with the typed division-by-zero error (crates/oxmera-ops/src/lib.rs:
//    47-48): the kernel raises a flag the host reads back.
//  * Bool holds 0 or 1 per byte: add is OR, mul is AND, abs is the
//    identity; neg, sub and div are refused by the host (NumPy refuses them
//    too).  sum over Bool is OR, max is OR.
//  * sum accumulates in the output dtype with wrapping: addition modulo 2^n
//    is associative, so the result is the exact sum modulo 2^n whatever the
//    order -- bit-exact against any summation order.  max is order-free too.
//
// All of these are HBM-bound: one read of each input element, one write of
// each output element.  Elementwise kernels walk runs of kRun consecutive
// elements of the innermost dim (coalesced for unit strides), the same
// iteration space the host collapsed for the float kernels.  Reductions: a
// block per output when the reduced elements are one unit-stride run, a
// thread per output otherwise.
#include <limits>
#include <type_traits>

#include "elementwise_launch.hpp"

namespace oxm {

namespace {

constexpr int kRunI = 4;

// Wrapping arithmetic through the unsigned type of the same width (signed
// overflow is undefined in C++; unsigned arithmetic wraps by definition).
template <typename T>
struct IntOps {
    using U = typename std::make_unsigned<T>::type;
    __device__ static T add(T a, T b) { return (T)((U)a + (U)b); }
    __device__ static T sub(T a, T b) { return (T)((U)a - (U)b); }
    __device__ static T mul(T a, T b) { return (T)((U)a * (U)b); }
    __device__ static T neg(T a) { return (T)((U)0 - (U)a); }
    __device__ static T abs(T a) {
        if constexpr (std::is_signed<T>::value)
            return a < 0 ? neg(a) : a;
        else
            return a;
    }
    // truncating division; b != 0 (checked by the caller); MIN / -1 wraps
    __device__ static T div(T a, T b) {
        if constexpr (std::is_signed<T>::value) {
            if (b == (T)-1) return neg(a);
        }
        return a / b;
    }
};

// OP codes: the UnaryOp / BinaryOp values of elementwise_launch.hpp.
template <typename T, bool BOOL, int OP>
__device__ __forceinline__ T int_unary(T x) {
    if constexpr (OP == kUnNeg)
        return IntOps<T>::neg(x);
    else
        return BOOL ? x : IntOps<T>::abs(x);  // kUnAbs
}

template <typename T, bool BOOL, int OP>
__device__ __forceinline__ T int_binary(T a, T b, int *zero_div) {
    if constexpr (BOOL) {
        if constexpr (OP == kBinAdd)
            return (T)((a | b) != 0);
        else if constexpr (OP == kBinMul)
            return (T)((a & b) != 0);
        else
            return (T)(a == b);  // kBinEq
    } else {
        if constexpr (OP == kBinAdd)
            return IntOps<T>::add(a, b);
        else if constexpr (OP == kBinSub)
            return IntOps<T>::sub(a, b);
        else if constexpr (OP == kBinMul)
            return IntOps<T>::mul(a, b);
        else if constexpr (OP == kBinDiv) {
            if (b == 0) {
                *zero_div = 1;  // plain vector store; every writer stores the same value
                return 0;
            }
            return IntOps<T>::div(a, b);
        } else
            return (T)(a == b);  // kBinEq
    }
}

__device__ __forceinline__ void offsets3(const EwShape &s, int64_t i, int64_t &o0, int64_t &o1, int64_t &o2) {
    o0 = o1 = o2 = 0;
    for (int d = s.ndim - 1; d >= 0; --d) {
        const int64_t e = s.shape[d];
        const int64_t c = i % e;
        i /= e;
        o0 += c * s.st[0][d];
        o1 += c * s.st[1][d];
        o2 += c * s.st[2][d];
    }
}

// Unary (NOPS 1) or binary (NOPS 2); operand 0 is the output.
template <typename T, bool BOOL, int NOPS, int OP>
__global__ void __launch_bounds__(256) int_ew(EwShape s, T *out, const T *x, const T *y, int *zero_div) {
    const int64_t inner = s.shape[s.ndim - 1];
    const int64_t runs_per_row = (inner + kRunI - 1) / kRunI;
    const int64_t nruns = s.numel / inner * runs_per_row;
    const int64_t s0 = s.st[0][s.ndim - 1], s1 = s.st[1][s.ndim - 1], s2 = s.st[2][s.ndim - 1];
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < nruns; r += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = r / runs_per_row, c0 = (r - row * runs_per_row) * kRunI;
        int64_t oo, ox, oy;
        offsets3(s, row * inner + c0, oo, ox, oy);
#pragma unroll
        for (int k = 0; k < kRunI; ++k) {
            if (c0 + k >= inner) break;
            const T a = x[ox + k * s1];
            T v;
            if constexpr (NOPS == 1)
                v = int_unary<T, BOOL, OP>(a);
            else
                v = int_binary<T, BOOL, OP>(a, y[oy + k * s2], zero_div);
            out[oo + k * s0] = v;
        }
    }
}

template <typename T, bool BOOL, int OP>
__device__ __forceinline__ T red_comb(T acc, T v) {
    if constexpr (BOOL)
        return (T)((acc | v) != 0);  // sum and max over Bool: OR
    else if constexpr (OP == kRedSum)
        return IntOps<T>::add(acc, v);
    else
        return v > acc ? v : acc;
}

template <typename T, bool BOOL, int OP>
__device__ __forceinline__ T red_init() {
    if constexpr (BOOL || OP == kRedSum)
        return (T)0;
    else
        return std::numeric_limits<T>::lowest();
}

__device__ __forceinline__ int64_t dims_off(int n, const int64_t *shape, const int64_t *st, int64_t i) {
    int64_t o = 0;
    for (int d = n - 1; d >= 0; --d) {
        const int64_t c = i % shape[d];
        i /= shape[d];
        o += c * st[d];
    }
    return o;
}

// A thread per output, the reduced elements in row-major order.
template <typename T, bool BOOL, int OP>
__global__ void __launch_bounds__(256) int_reduce_per_thread(RedGeom g, const T *x, T *out) {
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < g.n_out;
         o += (int64_t)gridDim.x * blockDim.x) {
        const int64_t base = dims_off(g.nk, g.kshape, g.kst, o);
        T acc = red_init<T, BOOL, OP>();
        for (int64_t r = 0; r < g.n_red; ++r)
            acc = red_comb<T, BOOL, OP>(acc, x[base + (g.nr == 1 ? r * g.rst[0] : dims_off(g.nr, g.rshape, g.rst, r))]);
        out[o] = acc;
    }
}

// A block per output whose reduced elements are one unit-stride run: the
// threads read it coalesced, then combine through LDS.
template <typename T, bool BOOL, int OP>
__global__ void __launch_bounds__(256) int_reduce_rows(RedGeom g, const T *x, T *out) {
    __shared__ T red[256];
    const int64_t o = blockIdx.x;
    const T *row = x + dims_off(g.nk, g.kshape, g.kst, o);
    T acc = red_init<T, BOOL, OP>();
    for (int64_t r = threadIdx.x; r < g.n_red; r += 256) acc = red_comb<T, BOOL, OP>(acc, row[r]);
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] = red_comb<T, BOOL, OP>(red[threadIdx.x], red[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0) out[o] = red[0];
}

unsigned grid_i(int64_t work) {
    int64_t g = (work + 255) / 256;
    if (g > 65536) g = 65536;
    return (unsigned)(g < 1 ? 1 : g);
}

template <typename T, bool BOOL, int NOPS, int OP>
hipError_t ew_go(const EwShape &s, void *out, const void *x, const void *y, int *zero_div, hipStream_t st) {
    const int64_t runs = s.numel / s.shape[s.ndim - 1] * ((s.shape[s.ndim - 1] + kRunI - 1) / kRunI);
    hipLaunchKernelGGL((int_ew<T, BOOL, NOPS, OP>), dim3(grid_i(runs)), dim3(256), 0, st, s, (T *)out, (const T *)x,
                       (const T *)y, zero_div);
    return hipGetLastError();
}

template <typename T, bool BOOL>
hipError_t ew_typed(int nops, int op, const EwShape &s, void *out, const void *x, const void *y, int *zero_div,
                    hipStream_t st) {
    if (nops == 1) {
        if constexpr (!BOOL) {
            if (op == kUnNeg) return ew_go<T, BOOL, 1, kUnNeg>(s, out, x, y, zero_div, st);
        }
        return ew_go<T, BOOL, 1, kUnAbs>(s, out, x, y, zero_div, st);
    }
    switch (op) {
    case kBinAdd: return ew_go<T, BOOL, 2, kBinAdd>(s, out, x, y, zero_div, st);
    case kBinMul: return ew_go<T, BOOL, 2, kBinMul>(s, out, x, y, zero_div, st);
    case kBinEq: return ew_go<T, BOOL, 2, kBinEq>(s, out, x, y, zero_div, st);
    default: break;
    }
    if constexpr (!BOOL) {
        if (op == kBinSub) return ew_go<T, BOOL, 2, kBinSub>(s, out, x, y, zero_div, st);
        if (op == kBinDiv) return ew_go<T, BOOL, 2, kBinDiv>(s, out, x, y, zero_div, st);
    }
    return hipErrorInvalidValue;  // refused by the host before it gets here
}

template <typename T, bool BOOL, int OP>
hipError_t red_go(const RedGeom &g, const void *x, void *out, hipStream_t st) {
    if (g.n_out == 0) return hipSuccess;
    if (g.nr == 1 && g.rst[0] == 1 && g.n_red >= 1024 && g.n_out <= INT32_MAX)
        hipLaunchKernelGGL((int_reduce_rows<T, BOOL, OP>), dim3((unsigned)g.n_out), dim3(256), 0, st, g, (const T *)x,
                           (T *)out);
    else
        hipLaunchKernelGGL((int_reduce_per_thread<T, BOOL, OP>), dim3(grid_i(g.n_out)), dim3(256), 0, st, g,
                           (const T *)x, (T *)out);
    return hipGetLastError();
}

template <typename T, bool BOOL>
hipError_t red_typed(int op, const RedGeom &g, const void *x, void *out, hipStream_t st) {
    return op == kRedSum ? red_go<T, BOOL, kRedSum>(g, x, out, st) : red_go<T, BOOL, kRedMax>(g, x, out, st);
}

}  // namespace

hipError_t launch_elementwise_int(int dtype, int nops, int op, const EwShape &s, void *out, const void *x,
                                  const void *y, int *zero_div, hipStream_t st) {
    if (s.numel == 0) return hipSuccess;
    switch (dtype) {
    case kDtI32: return ew_typed<int32_t, false>(nops, op, s, out, x, y, zero_div, st);
    case kDtI64: return ew_typed<int64_t, false>(nops, op, s, out, x, y, zero_div, st);
    case kDtU8: return ew_typed<uint8_t, false>(nops, op, s, out, x, y, zero_div, st);
    default: return ew_typed<uint8_t, true>(nops, op, s, out, x, y, zero_div, st);
    }
}

hipError_t launch_reduce_int(int dtype, int op, const RedGeom &g, const void *x, void *out, hipStream_t st) {
    switch (dtype) {
    case kDtI32: return red_typed<int32_t, false>(op, g, x, out, st);
    case kDtI64: return red_typed<int64_t, false>(op, g, x, out, st);
    case kDtU8: return red_typed<uint8_t, false>(op, g, x, out, st);
    default: return red_typed<uint8_t, true>(op, g, x, out, st);
    }
}

}  // namespace oxm
