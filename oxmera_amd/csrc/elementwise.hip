// elementwise.hip -- the rest of oxmera's Backend on gfx950: UnaryOps,
// BinaryOps (NumPy broadcasting), ReduceOps (sum / max over axes) and the
// strided copy behind Tensor::contiguous (crates/oxmera-ops/src/lib.rs:27-69,
// crates/oxmera-tensor/src/tensor.rs:86-90).
//
// All of these are HBM-bound: one read of each input element, one write of
// each output element.  Operands are strided views (element strides, may be
// zero for broadcast dims or negative); outputs are contiguous.  The host
// collapses dimensions that are contiguous with each other, so most views
// reach the kernels as one or two dims.  Contiguous same-shape operands take
// a 16-byte-per-lane path; everything else decodes coordinates once per run
// of consecutive elements along the innermost dimension.
//
// Reductions accumulate in f32 (f64 for F64 input) and round once.  Two
// coalesced schedules: rows (an output's reduced elements contiguous: a
// block walks them) and columns (consecutive outputs contiguous: a thread per
// output walks the reduced elements); both keep several loads in flight per
// thread and may split the reduced range over blocks, writing partials to a
// workspace that a second pass combines in a fixed order -- no atomics, so
// results do not depend on scheduling.  Other layouts: a thread per output.
#include <mutex>

#include "elementwise_launch.hpp"
#include "gemm_kernels.hpp"

namespace oxm {

namespace {

// ---- element access ----------------------------------------------------------

template <int DT>
struct El;
template <>
struct El<kDtF32> {
    using Acc = float;
    __device__ static float load(const void *p, int64_t i) { return ((const float *)p)[i]; }
    __device__ static void store(void *p, int64_t i, float v) { ((float *)p)[i] = v; }
};
template <>
struct El<kDtBF16> {
    using Acc = float;
    __device__ static float load(const void *p, int64_t i) { return bf16_bits_to_f32(((const uint16_t *)p)[i]); }
    __device__ static void store(void *p, int64_t i, float v) { ((uint16_t *)p)[i] = f32_to_bf16_bits(v); }
};
template <>
struct El<kDtF16> {
    using Acc = float;
    __device__ static float load(const void *p, int64_t i) { return f16_bits_to_f32(((const uint16_t *)p)[i]); }
    __device__ static void store(void *p, int64_t i, float v) { ((uint16_t *)p)[i] = f32_to_f16_bits(v); }
};
template <>
struct El<kDtF64> {
    using Acc = double;
    __device__ static double load(const void *p, int64_t i) { return ((const double *)p)[i]; }
    __device__ static void store(void *p, int64_t i, double v) { ((double *)p)[i] = v; }
};

// The op is a template parameter: each kernel is straight-line code (a
// run-time switch per element compiled to branchy code that mishandled one
// of its cases).
template <int OP, typename A>
__device__ __forceinline__ A apply_unary(A x) {
    if constexpr (OP == kUnNeg)
        return -x;
    else if constexpr (OP == kUnExp)
        return exp(x);
    else if constexpr (OP == kUnLn)
        return log(x);
    else if constexpr (OP == kUnAbs)
        return fabs(x);
    else  // sign; NaN stays NaN
        return x > A(0) ? A(1) : (x < A(0) ? A(-1) : x * A(0));
}

// GELU'(x) for the erf GELU: Phi(x) + x phi(x).
template <typename A>
__device__ __forceinline__ A dgelu_acc(A x) {
    if constexpr (std::is_same<A, float>::value) {
        return dgelu_erf(x);
    } else {
        return 0.5 * (1.0 + erf(x * 0.70710678118654752440)) + x * 0.39894228040143267794 * exp(-0.5 * x * x);
    }
}

template <int OP, typename A>
__device__ __forceinline__ A apply_binary(A a, A b) {
    if constexpr (OP == kBinAdd)
        return a + b;
    else if constexpr (OP == kBinSub)
        return a - b;
    else if constexpr (OP == kBinMul)
        return a * b;
    else if constexpr (OP == kBinDiv)
        return a / b;
    else if constexpr (OP == kBinEq)
        return a == b ? A(1) : A(0);
    else
        return a * dgelu_acc<A>(b);
}

// Offsets of element `i` (row-major over `shape`) in up to three strided
// operands.
struct Coord {
    __device__ static void offsets(const EwShape &s, int64_t i, int64_t &o0, int64_t &o1, int64_t &o2) {
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
};

// ---- elementwise: strided (runs of kRun along the innermost dim) --------------

constexpr int kRun = 4;

// Unary (NOPS = 1) or binary (NOPS = 2) over a strided iteration space; the
// output is operand index 0 (contiguous), inputs 1 and 2.
template <int DT, int NOPS, int OP>
__global__ void __launch_bounds__(256) ew_strided(EwShape s, void *out, const void *x, const void *y) {
    using A = typename El<DT>::Acc;
    const int64_t inner = s.shape[s.ndim - 1];
    const int64_t runs_per_row = (inner + kRun - 1) / kRun;
    const int64_t rows = s.numel / inner;
    const int64_t nruns = rows * runs_per_row;
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < nruns; r += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = r / runs_per_row, c0 = (r - row * runs_per_row) * kRun;
        int64_t oo, ox, oy;
        Coord::offsets(s, row * inner + c0, oo, ox, oy);
        const int64_t si0 = s.st[0][s.ndim - 1], si1 = s.st[1][s.ndim - 1], si2 = s.st[2][s.ndim - 1];
#pragma unroll
        for (int k = 0; k < kRun; ++k) {
            if (c0 + k >= inner) break;
            const A a = El<DT>::load(x, ox + k * si1);
            A v;
            if constexpr (NOPS == 1)
                v = apply_unary<OP, A>(a);
            else
                v = apply_binary<OP, A>(a, El<DT>::load(y, oy + k * si2));
            El<DT>::store(out, oo + k * si0, v);
        }
    }
}

// ---- elementwise: contiguous, same shape (16 bytes per lane) -------------------

template <int DT>
__device__ __forceinline__ void ld16(const void *p, int64_t i, float (&v)[DT == kDtF32 ? 4 : 8]) {
    const uint4 u = *(const uint4 *)((const char *)p + i * (DT == kDtF32 ? 4 : 2));
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    if constexpr (DT == kDtF32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(w[e]);
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t h = (w[e >> 1] >> (16 * (e & 1))) & 0xffffu;
            v[e] = DT == kDtBF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
        }
    }
}

template <int DT>
__device__ __forceinline__ void st16(void *p, int64_t i, const float (&v)[DT == kDtF32 ? 4 : 8]) {
    uint32_t w[4];
    if constexpr (DT == kDtF32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = __float_as_uint(v[e]);
    } else {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t lo = DT == kDtBF16 ? f32_to_bf16_bits(v[2 * d]) : f32_to_f16_bits(v[2 * d]);
            const uint32_t hi = DT == kDtBF16 ? f32_to_bf16_bits(v[2 * d + 1]) : f32_to_f16_bits(v[2 * d + 1]);
            w[d] = lo | (hi << 16);
        }
    }
    *(uint4 *)((char *)p + i * (DT == kDtF32 ? 4 : 2)) = make_uint4(w[0], w[1], w[2], w[3]);
}

// st16 with a non-temporal store.
template <int DT>
__device__ __forceinline__ void st16_nt(void *p, int64_t i, const float (&v)[DT == kDtF32 ? 4 : 8]) {
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    uint32_t w[4];
    if constexpr (DT == kDtF32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = __float_as_uint(v[e]);
    } else {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t lo = DT == kDtBF16 ? f32_to_bf16_bits(v[2 * d]) : f32_to_f16_bits(v[2 * d]);
            const uint32_t hi = DT == kDtBF16 ? f32_to_bf16_bits(v[2 * d + 1]) : f32_to_f16_bits(v[2 * d + 1]);
            w[d] = lo | (hi << 16);
        }
    }
    __builtin_nontemporal_store(u32x4v{w[0], w[1], w[2], w[3]}, (u32x4v *)((char *)p + i * (DT == kDtF32 ? 4 : 2)));
}

// n is a multiple of the vector width; every pointer 16-byte aligned.  Each
// thread takes two vectors a grid apart per iteration (both loads of each
// operand in flight together); stores are non-temporal (the output is not
// read again by this kernel).
template <int DT, int NOPS, int OP>
__global__ void __launch_bounds__(256) ew_contig16(int64_t n, void *out, const void *x, const void *y) {
    constexpr int V = DT == kDtF32 ? 4 : 8;
    const int64_t nv = n / V;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    auto one = [&](int64_t j, float (&a)[V], const float (&b)[V]) {
#pragma unroll
        for (int e = 0; e < V; ++e) {
            if constexpr (NOPS == 1)
                a[e] = apply_unary<OP, float>(a[e]);
            else
                a[e] = apply_binary<OP, float>(a[e], b[e]);
        }
        st16_nt<DT>(out, j * V, a);
    };
    int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; j + stride < nv; j += 2 * stride) {
        float a0[V], b0[V], a1[V], b1[V];
        ld16<DT>(x, j * V, a0);
        ld16<DT>(x, (j + stride) * V, a1);
        if constexpr (NOPS == 2) {
            ld16<DT>(y, j * V, b0);
            ld16<DT>(y, (j + stride) * V, b1);
        }
        one(j, a0, b0);
        one(j + stride, a1, b1);
    }
    if (j < nv) {
        float a[V], b[V];
        ld16<DT>(x, j * V, a);
        if constexpr (NOPS == 2) ld16<DT>(y, j * V, b);
        one(j, a, b);
    }
}

// Rows of vectors: every operand of stride 1 (a vector load) or 0 (one
// element repeated) along the innermost dim; outer dims through strides.
template <int DT, int NOPS, int OP>
__global__ void __launch_bounds__(256) ew_inner16(EwShape s, void *out, const void *x, const void *y) {
    constexpr int V = DT == kDtF32 ? 4 : 8;
    const int L = s.ndim - 1;
    const int64_t inner = s.shape[L], vpr = inner / V, nv = s.numel / V;
    const bool xv = s.st[1][L] != 0, yv = s.st[2][L] != 0;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < nv; j += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = j / vpr, c = (j - row * vpr) * V;
        int64_t oo, ox, oy;
        Coord::offsets(s, row * inner, oo, ox, oy);
        float a[V], b[V];
        if (xv) {
            ld16<DT>(x, ox + c, a);
        } else {
            const float v = El<DT>::load(x, ox);
#pragma unroll
            for (int e = 0; e < V; ++e) a[e] = v;
        }
        if constexpr (NOPS == 2) {
            if (yv) {
                ld16<DT>(y, oy + c, b);
            } else {
                const float v = El<DT>::load(y, oy);
#pragma unroll
                for (int e = 0; e < V; ++e) b[e] = v;
            }
        }
#pragma unroll
        for (int e = 0; e < V; ++e) {
            if constexpr (NOPS == 1)
                a[e] = apply_unary<OP, float>(a[e]);
            else
                a[e] = apply_binary<OP, float>(a[e], b[e]);
        }
        st16<DT>(out, oo + c, a);
    }
}

// ---- strided copy (bits unchanged) ------------------------------------------------

template <typename U>
__global__ void __launch_bounds__(256) copy_strided(EwShape s, U *dst, const U *src) {
    const int64_t inner = s.shape[s.ndim - 1];
    const int64_t runs_per_row = (inner + kRun - 1) / kRun;
    const int64_t nruns = s.numel / inner * runs_per_row;
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < nruns; r += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = r / runs_per_row, c0 = (r - row * runs_per_row) * kRun;
        int64_t od, os, unused;
        Coord::offsets(s, row * inner + c0, od, os, unused);
        const int64_t sd = s.st[0][s.ndim - 1], ss = s.st[1][s.ndim - 1];
#pragma unroll
        for (int k = 0; k < kRun; ++k) {
            if (c0 + k >= inner) break;
            dst[od + k * sd] = src[os + k * ss];
        }
    }
}

__global__ void __launch_bounds__(256) copy_contig16(int64_t n16, uint4 *dst, const uint4 *src) {
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n16; j += (int64_t)gridDim.x * blockDim.x)
        dst[j] = src[j];
}

// Transposing copy: the source is contiguous along dim p, the destination
// along the innermost dim L.  A block moves a kTT x kTT tile of (p, L) for
// one combination of the other ("batch") dims through LDS, reading along p
// and writing along L, so both sides are coalesced.
constexpr int kTT = 64;

template <typename U>
__global__ void __launch_bounds__(256) copy_transpose(EwShape s, int p, U *dst, const U *src) {
    __shared__ U tile[kTT][kTT + 1];
    const int L = s.ndim - 1;
    const int64_t np_ = s.shape[p], nl = s.shape[L];
    const int64_t tiles_p = (np_ + kTT - 1) / kTT, tiles_l = (nl + kTT - 1) / kTT;
    int64_t b = blockIdx.x;
    const int64_t tl = b % tiles_l;
    b /= tiles_l;
    const int64_t tp = b % tiles_p;
    b /= tiles_p;
    int64_t od = 0, os = 0;  // batch offsets, dims other than p and L
    for (int d = L - 1; d >= 0; --d) {
        if (d == p) continue;
        const int64_t c = b % s.shape[d];
        b /= s.shape[d];
        od += c * s.st[0][d];
        os += c * s.st[1][d];
    }
    const int64_t p0 = tp * kTT, l0 = tl * kTT;
    const int tx = threadIdx.x % kTT, ty = threadIdx.x / kTT;
    const int64_t sl = s.st[1][L], dp = s.st[0][p];
#pragma unroll
    for (int k = 0; k < kTT / 4; ++k) {
        const int j = ty + 4 * k;
        if (p0 + tx < np_ && l0 + j < nl) tile[j][tx] = src[os + (p0 + tx) + (l0 + j) * sl];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kTT / 4; ++k) {
        const int i = ty + 4 * k;
        if (p0 + i < np_ && l0 + tx < nl) dst[od + (p0 + i) * dp + (l0 + tx)] = tile[tx][i];
    }
}

// The same with 16-byte accesses on both sides, for 2- and 4-byte elements
// (the launcher has checked that both pointers are 16-byte aligned, that both
// extents and every stride other than the unit ones are multiples of the
// vector width W, so every vector below is aligned and wholly in or out of
// range).  A lane reads W consecutive p of one l and stores them as one
// 16-byte chunk of LDS row l, the chunk index XORed with (l / W) % C (C =
// chunks per 64-element row); a lane then gathers W consecutive l of one p
// from the columns -- with the XOR, the W-row groups of a wave's lanes fall
// on different banks -- and writes them as one 16-byte vector.
template <typename U>
__global__ void __launch_bounds__(256) copy_transpose_vec(EwShape s, int p, U *dst, const U *src) {
    constexpr int W = 16 / sizeof(U);
    constexpr int C = kTT / W;        // 16-byte chunks per tile row
    constexpr int kRowsPass = 256 / C;
    __shared__ __attribute__((aligned(16))) U tile[kTT * kTT];
    const int L = s.ndim - 1;
    const int64_t np_ = s.shape[p], nl = s.shape[L];
    const int64_t tiles_p = (np_ + kTT - 1) / kTT, tiles_l = (nl + kTT - 1) / kTT;
    int64_t b = blockIdx.x;
    const int64_t tl = b % tiles_l;
    b /= tiles_l;
    const int64_t tp = b % tiles_p;
    b /= tiles_p;
    int64_t od = 0, os = 0;
    for (int d = L - 1; d >= 0; --d) {
        if (d == p) continue;
        const int64_t c = b % s.shape[d];
        b /= s.shape[d];
        od += c * s.st[0][d];
        os += c * s.st[1][d];
    }
    const int64_t p0 = tp * kTT, l0 = tl * kTT;
    const int64_t sl = s.st[1][L], dp = s.st[0][p];
    const int c = threadIdx.x % C, r = threadIdx.x / C;
#pragma unroll
    for (int k = 0; k < kTT / kRowsPass; ++k) {
        const int l = r + k * kRowsPass;
        if (l0 + l < nl && p0 + c * W < np_)
            *(uint4 *)&tile[l * kTT + ((c ^ ((l / W) % C)) * W)] =
                *(const uint4 *)&src[os + (p0 + c * W) + (l0 + l) * sl];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kTT / kRowsPass; ++k) {
        const int pp = r + k * kRowsPass;  // this lane's p in the tile; c: its group of W l's
        if (p0 + pp < np_ && l0 + c * W < nl) {
            alignas(16) U v[W];
#pragma unroll
            for (int i = 0; i < W; ++i) {
                const int l = c * W + i;
                v[i] = tile[l * kTT + (((pp / W) ^ ((l / W) % C)) * W) + pp % W];
            }
            *(uint4 *)&dst[od + (p0 + pp) * dp + (l0 + c * W)] = *(const uint4 *)v;
        }
    }
}

// ---- dtype conversion --------------------------------------------------------------

template <int DI, int DO>
__global__ void __launch_bounds__(256) convert_strided(EwShape s, void *dst, const void *src) {
    const int64_t inner = s.shape[s.ndim - 1];
    const int64_t runs_per_row = (inner + kRun - 1) / kRun;
    const int64_t nruns = s.numel / inner * runs_per_row;
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < nruns; r += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = r / runs_per_row, c0 = (r - row * runs_per_row) * kRun;
        int64_t od, os, unused;
        Coord::offsets(s, row * inner + c0, od, os, unused);
        const int64_t sd = s.st[0][s.ndim - 1], ss = s.st[1][s.ndim - 1];
#pragma unroll
        for (int k = 0; k < kRun; ++k) {
            if (c0 + k >= inner) break;
            El<DO>::store(dst, od + k * sd, (typename El<DO>::Acc)El<DI>::load(src, os + k * ss));
        }
    }
}

// ---- SGD ---------------------------------------------------------------------------

// A product the compiler may not fuse into a following add: the empty asm
// takes the value through a VGPR, so the multiply is rounded on its own.
__device__ __forceinline__ float unfused_mul(float a, float b) {
    float m = a * b;
    asm volatile("" : "+v"(m));
    return m;
}

// One parameter's update: MODE 0 plain, 1 momentum, 2 Nesterov momentum.
// Each f32 operation is rounded on its own (no fused multiply-adds), so the
// result is reproducible operation by operation.
template <int MODE, bool WD>
__device__ __forceinline__ float sgd_one(float pv, float gv, float &vv, float lr, float mu, float wd) {
    if constexpr (WD) gv = gv + unfused_mul(wd, pv);
    if constexpr (MODE != 0) {
        vv = unfused_mul(mu, vv) + gv;
        gv = MODE == 2 ? gv + unfused_mul(mu, vv) : vv;
    }
    return pv - unfused_mul(lr, gv);
}

// Eight consecutive elements as f32: one 16-byte access for a 16-bit type,
// two for f32 (i a multiple of 8, the pointer 16-byte aligned).
template <int DT>
__device__ __forceinline__ void ld8(const void *p, int64_t i, float (&v)[8]) {
    if constexpr (DT == kDtF32) {
        float a[4], b[4];
        ld16<kDtF32>(p, i, a);
        ld16<kDtF32>(p, i + 4, b);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = a[e], v[e + 4] = b[e];
    } else {
        ld16<DT>(p, i, v);
    }
}
template <int DT>
__device__ __forceinline__ void st8(void *p, int64_t i, const float (&v)[8]) {
    if constexpr (DT == kDtF32) {
        const float a[4] = {v[0], v[1], v[2], v[3]}, b[4] = {v[4], v[5], v[6], v[7]};
        st16<kDtF32>(p, i, a);
        st16<kDtF32>(p, i + 4, b);
    } else {
        st16<DT>(p, i, v);
    }
}

template <int PDT, int GDT, int MODE, bool WD>
__global__ void __launch_bounds__(256) sgd_kernel(int64_t n, void *p, const void *g, float *v, float lr, float mu,
                                                  float wd) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float vv = MODE != 0 ? v[i] : 0.f;
        El<PDT>::store(p, i, sgd_one<MODE, WD>(El<PDT>::load(p, i), El<GDT>::load(g, i), vv, lr, mu, wd));
        if constexpr (MODE != 0) v[i] = vv;
    }
}

// The same with eight elements per thread and 16-byte accesses (n a multiple
// of 8, every array 16-byte aligned: checked by the launcher).
template <int PDT, int GDT, int MODE, bool WD>
__global__ void __launch_bounds__(256) sgd_kernel_vec(int64_t n, void *p, const void *g, float *v, float lr,
                                                      float mu, float wd) {
    for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8; i < n;
         i += (int64_t)gridDim.x * blockDim.x * 8) {
        float pv[8], gv[8], vv[8];
        ld8<PDT>(p, i, pv);
        ld8<GDT>(g, i, gv);
        if constexpr (MODE != 0) ld8<kDtF32>(v, i, vv);
#pragma unroll
        for (int e = 0; e < 8; ++e) pv[e] = sgd_one<MODE, WD>(pv[e], gv[e], vv[e], lr, mu, wd);
        st8<PDT>(p, i, pv);
        if constexpr (MODE != 0) st8<kDtF32>(v, i, vv);
    }
}

// ---- reductions -------------------------------------------------------------------

// Reduction geometry: the output's (kept) dims and the reduced dims, each
// with the input's strides.
template <int OP, typename A>
__device__ __forceinline__ A red_identity() {
    return OP == kRedSum ? (A)0 : -(A)INFINITY;
}

template <int OP, typename A>
__device__ __forceinline__ A red_combine(A acc, A v) {
    if constexpr (OP == kRedSum) {
        return acc + v;
    } else {
        // max with NaN propagation (a NaN anywhere makes the result NaN)
        if (v != v || acc != acc) return v != v ? v : acc;
        return v > acc ? v : acc;
    }
}

__device__ __forceinline__ int64_t dims_offset(int n, const int64_t *shape, const int64_t *st, int64_t i) {
    int64_t o = 0;
    for (int d = n - 1; d >= 0; --d) {
        const int64_t c = i % shape[d];
        i /= shape[d];
        o += c * st[d];
    }
    return o;
}

// Element r (row-major over the reduced dims) of output o's reduction.
__device__ __forceinline__ int64_t red_offset(const RedGeom &g, int64_t r) {
    return g.nr == 1 ? r * g.rst[0] : dims_offset(g.nr, g.rshape, g.rst, r);
}

constexpr int kRedU = 8;  // independent loads in flight per thread

// Generic: one thread per output element, the reduced elements in order.
template <int DT, int OP>
__global__ void __launch_bounds__(256) reduce_per_thread(RedGeom g, const void *x, void *out) {
    using A = typename El<DT>::Acc;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < g.n_out;
         o += (int64_t)gridDim.x * blockDim.x) {
        const int64_t base = dims_offset(g.nk, g.kshape, g.kst, o);
        A acc = red_identity<OP, A>();
        for (int64_t r = 0; r < g.n_red; ++r) acc = red_combine<OP, A>(acc, (A)El<DT>::load(x, base + red_offset(g, r)));
        El<DT>::store(out, o, acc);
    }
}

// Rows: output o's reduced elements are contiguous in memory (one reduced
// dim of stride 1).  Block (o, s) takes split s of the row; each thread
// keeps kRedU independent partials so kRedU coalesced loads are in flight.
// VEC: the loads are 16-byte vectors (the launcher has checked that every
// row starts 16-byte aligned and n_red is a multiple of the vector); the
// split size is then rounded up to a whole number of vectors.
// Result to out (splits == 1) or to ws[o * splits + s].
template <int DT, int OP, bool VEC>
__global__ void __launch_bounds__(256) reduce_rows(RedGeom g, const void *x, void *out, typename El<DT>::Acc *ws,
                                                   int splits) {
    using A = typename El<DT>::Acc;
    __shared__ A red[256];
    const int64_t o = blockIdx.x / splits;
    const int s = blockIdx.x % splits;
    const int64_t base = dims_offset(g.nk, g.kshape, g.kst, o);
    int64_t chunk = (g.n_red + splits - 1) / splits;
    A acc[kRedU];
#pragma unroll
    for (int u = 0; u < kRedU; ++u) acc[u] = red_identity<OP, A>();
    if constexpr (VEC) {
        constexpr int V = DT == kDtF32 ? 4 : 8;
        chunk = (chunk + V - 1) / V * V;
        const int64_t r0 = s * chunk, r1 = r0 + chunk < g.n_red ? r0 + chunk : g.n_red;
        for (int64_t r = r0 + threadIdx.x * V; r < r1; r += 256 * V * kRedU) {
            float v[kRedU][V];
#pragma unroll
            for (int u = 0; u < kRedU; ++u) {
                if (r + u * 256 * V < r1) {
                    ld16<DT>(x, base + r + u * 256 * V, v[u]);
                } else {
#pragma unroll
                    for (int e = 0; e < V; ++e) v[u][e] = red_identity<OP, A>();
                }
            }
#pragma unroll
            for (int u = 0; u < kRedU; ++u)
#pragma unroll
                for (int e = 0; e < V; ++e) acc[u] = red_combine<OP, A>(acc[u], v[u][e]);
        }
    } else {
        const int64_t r0 = s * chunk, r1 = r0 + chunk < g.n_red ? r0 + chunk : g.n_red;
        for (int64_t r = r0 + threadIdx.x; r < r1; r += 256 * kRedU) {
            A v[kRedU];
#pragma unroll
            for (int u = 0; u < kRedU; ++u)
                v[u] = r + u * 256 < r1 ? (A)El<DT>::load(x, base + r + u * 256) : red_identity<OP, A>();
#pragma unroll
            for (int u = 0; u < kRedU; ++u) acc[u] = red_combine<OP, A>(acc[u], v[u]);
        }
    }
#pragma unroll
    for (int u = 1; u < kRedU; ++u) acc[0] = red_combine<OP, A>(acc[0], acc[u]);
    red[threadIdx.x] = acc[0];
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] = red_combine<OP, A>(red[threadIdx.x], red[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        if (splits == 1)
            El<DT>::store(out, o, red[0]);
        else
            ws[o * splits + s] = red[0];
    }
}

// Rows, one wave per output (many short rows, 16-byte vectors): wave w of
// block b reduces row 4 b + w, lane l taking vectors l, l + 64, ... (kRedU
// in flight), then the 64 lanes combine through cross-lane exchanges in a
// fixed pattern -- no LDS and no block barrier per row.
template <int DT, int OP>
__global__ void __launch_bounds__(256) reduce_rows_wave(RedGeom g, const void *x, void *out) {
    constexpr int V = DT == kDtF32 ? 4 : 8;
    const int lane = threadIdx.x & 63;
    const int64_t o = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (o >= g.n_out) return;  // whole waves leave together
    const int64_t base = dims_offset(g.nk, g.kshape, g.kst, o);
    float acc[kRedU];
#pragma unroll
    for (int u = 0; u < kRedU; ++u) acc[u] = red_identity<OP, float>();
    for (int64_t r = (int64_t)lane * V; r < g.n_red; r += 64 * V * kRedU) {
        float v[kRedU][V];
#pragma unroll
        for (int u = 0; u < kRedU; ++u) {
            if (r + u * 64 * V < g.n_red) {
                ld16<DT>(x, base + r + u * 64 * V, v[u]);
            } else {
#pragma unroll
                for (int e = 0; e < V; ++e) v[u][e] = red_identity<OP, float>();
            }
        }
#pragma unroll
        for (int u = 0; u < kRedU; ++u)
#pragma unroll
            for (int e = 0; e < V; ++e) acc[u] = red_combine<OP, float>(acc[u], v[u][e]);
    }
#pragma unroll
    for (int u = 1; u < kRedU; ++u) acc[0] = red_combine<OP, float>(acc[0], acc[u]);
    float t = acc[0];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) t = red_combine<OP, float>(t, __shfl_xor(t, off));
    if (lane == 0) El<DT>::store(out, o, t);
}

// Columns: consecutive outputs are consecutive in memory (the innermost kept
// dim has stride 1), so a block of 256 threads takes 256 consecutive outputs
// (coalesced) over split s of the reduced range, kRedU reduced elements in
// flight per thread.  Result to out (splits == 1) or to ws[s * n_out + o].
template <int DT, int OP>
__global__ void __launch_bounds__(256) reduce_cols(RedGeom g, const void *x, void *out, typename El<DT>::Acc *ws,
                                                   int splits) {
    using A = typename El<DT>::Acc;
    const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int s = blockIdx.y;
    if (o >= g.n_out) return;
    const int64_t base = dims_offset(g.nk, g.kshape, g.kst, o);
    const int64_t chunk = (g.n_red + splits - 1) / splits;
    const int64_t r0 = s * chunk, r1 = r0 + chunk < g.n_red ? r0 + chunk : g.n_red;
    A acc[kRedU];
#pragma unroll
    for (int u = 0; u < kRedU; ++u) acc[u] = red_identity<OP, A>();
    for (int64_t r = r0; r < r1; r += kRedU) {
        A v[kRedU];
#pragma unroll
        for (int u = 0; u < kRedU; ++u) v[u] = r + u < r1 ? (A)El<DT>::load(x, base + red_offset(g, r + u)) : red_identity<OP, A>();
#pragma unroll
        for (int u = 0; u < kRedU; ++u) acc[u] = red_combine<OP, A>(acc[u], v[u]);
    }
#pragma unroll
    for (int u = 1; u < kRedU; ++u) acc[0] = red_combine<OP, A>(acc[0], acc[u]);
    if (splits == 1)
        El<DT>::store(out, o, acc[0]);
    else
        ws[(int64_t)s * g.n_out + o] = acc[0];
}

// Columns with 16-byte loads: as reduce_cols, but thread t takes V = 16 /
// sizeof(elem) consecutive outputs (the launcher has checked that the
// innermost kept dim is contiguous with a length that is a multiple of V,
// and that every V-group of outputs starts 16-byte aligned for every reduced
// element), one vector load per reduced element, the reduced offset computed
// once per vector.  Per output the same order as reduce_cols: kRedU partials
// over interleaved reduced elements, combined 0..kRedU-1.
template <int DT, int OP>
__global__ void __launch_bounds__(256) reduce_cols_vec(RedGeom g, const void *x, void *out, float *ws, int splits) {
    constexpr int V = DT == kDtF32 ? 4 : 8;
    const int64_t o = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
    const int s = blockIdx.y;
    if (o >= g.n_out) return;
    const int64_t base = dims_offset(g.nk, g.kshape, g.kst, o);
    const int64_t chunk = (g.n_red + splits - 1) / splits;
    const int64_t r0 = s * chunk, r1 = r0 + chunk < g.n_red ? r0 + chunk : g.n_red;
    float acc[kRedU][V];
#pragma unroll
    for (int u = 0; u < kRedU; ++u)
#pragma unroll
        for (int e = 0; e < V; ++e) acc[u][e] = red_identity<OP, float>();
    for (int64_t r = r0; r < r1; r += kRedU) {
        float v[kRedU][V];
#pragma unroll
        for (int u = 0; u < kRedU; ++u) {
            if (r + u < r1) {
                ld16<DT>(x, base + red_offset(g, r + u), v[u]);
            } else {
#pragma unroll
                for (int e = 0; e < V; ++e) v[u][e] = red_identity<OP, float>();
            }
        }
#pragma unroll
        for (int u = 0; u < kRedU; ++u)
#pragma unroll
            for (int e = 0; e < V; ++e) acc[u][e] = red_combine<OP, float>(acc[u][e], v[u][e]);
    }
#pragma unroll
    for (int e = 0; e < V; ++e) {
        float t = acc[0][e];
#pragma unroll
        for (int u = 1; u < kRedU; ++u) t = red_combine<OP, float>(t, acc[u][e]);
        if (splits == 1)
            El<DT>::store(out, o + e, t);
        else
            ws[(int64_t)s * g.n_out + o + e] = t;
    }
}

// Columns of a tall input in one pass, no workspace: block b takes the
// 8 * V consecutive outputs 8 V b .. (eight 16-byte vectors: 128 bytes of a
// row), thread (j, q) vector j over reduced elements q, q + 64, q + 128, ...
// (kRedU loads in flight), and the 64 phases of an output are combined in q
// order through LDS -- a fixed order.  Used when there are enough 128-byte
// column groups to give every CU a block (the [8192, 8192] f32 column sum:
// 256 blocks, against 2048 split blocks + a finishing pass before).
constexpr int kTallPhases = 64;

template <int DT, int OP>
__global__ void __launch_bounds__(8 * kTallPhases) reduce_cols_tall(RedGeom g, const void *x, void *out) {
    constexpr int V = DT == kDtF32 ? 4 : 8;
    __shared__ float part[kTallPhases][8 * V];
    const int j = threadIdx.x % 8, q = threadIdx.x / 8;
    const int64_t o = ((int64_t)blockIdx.x * 8 + j) * V;
    float acc[kRedU][V];
#pragma unroll
    for (int u = 0; u < kRedU; ++u)
#pragma unroll
        for (int e = 0; e < V; ++e) acc[u][e] = red_identity<OP, float>();
    if (o < g.n_out) {
        const int64_t base = dims_offset(g.nk, g.kshape, g.kst, o);
        for (int64_t r = q; r < g.n_red; r += (int64_t)kTallPhases * kRedU) {
            float v[kRedU][V];
#pragma unroll
            for (int u = 0; u < kRedU; ++u) {
                const int64_t rr = r + (int64_t)u * kTallPhases;
                if (rr < g.n_red) {
                    ld16<DT>(x, base + red_offset(g, rr), v[u]);
                } else {
#pragma unroll
                    for (int e = 0; e < V; ++e) v[u][e] = red_identity<OP, float>();
                }
            }
#pragma unroll
            for (int u = 0; u < kRedU; ++u)
#pragma unroll
                for (int e = 0; e < V; ++e) acc[u][e] = red_combine<OP, float>(acc[u][e], v[u][e]);
        }
    }
#pragma unroll
    for (int e = 0; e < V; ++e) {
        float t = acc[0][e];
#pragma unroll
        for (int u = 1; u < kRedU; ++u) t = red_combine<OP, float>(t, acc[u][e]);
        part[q][j * V + e] = t;
    }
    __syncthreads();
    if (threadIdx.x < 8 * V) {
        const int64_t oo = (int64_t)blockIdx.x * 8 * V + threadIdx.x;
        if (oo < g.n_out) {
            float t = part[0][threadIdx.x];
            for (int k = 1; k < kTallPhases; ++k) t = red_combine<OP, float>(t, part[k][threadIdx.x]);
            El<DT>::store(out, oo, t);
        }
    }
}

// The finishing pass for the column schedule (ws[s * n_out + o]): 64
// consecutive outputs per block, four threads per output; thread (o, q)
// combines splits q, q + 4, q + 8, ... (kRedU loads in flight), then the
// four partials of an output are combined in q order through LDS -- a fixed
// order, so results do not depend on scheduling.  A wave reads 64
// consecutive outputs of one split (coalesced).
template <int DT, int OP>
__global__ void __launch_bounds__(256) reduce_finish_cols(const typename El<DT>::Acc *ws, int64_t n_out, int splits,
                                                          void *out) {
    using A = typename El<DT>::Acc;
    __shared__ A part[4][64];
    const int ol = threadIdx.x % 64, q = threadIdx.x / 64;
    const int64_t o = (int64_t)blockIdx.x * 64 + ol;
    A acc = red_identity<OP, A>();
    if (o < n_out) {
        for (int s0 = q; s0 < splits; s0 += 4 * kRedU) {
            A v[kRedU];
#pragma unroll
            for (int u = 0; u < kRedU; ++u) {
                const int sp = s0 + 4 * u;
                v[u] = sp < splits ? ws[(int64_t)sp * n_out + o] : red_identity<OP, A>();
            }
#pragma unroll
            for (int u = 0; u < kRedU; ++u) acc = red_combine<OP, A>(acc, v[u]);
        }
    }
    part[q][ol] = acc;
    __syncthreads();
    if (q == 0 && o < n_out) {
        A t = part[0][ol];
#pragma unroll
        for (int k = 1; k < 4; ++k) t = red_combine<OP, A>(t, part[k][ol]);
        El<DT>::store(out, o, t);
    }
}

// out[o] = the splits' partials combined, in a fixed order.  stride_o /
// stride_s address ws[o * stride_o + s * stride_s].  A thread per output,
// kRedU partials in flight.
template <int DT, int OP>
__global__ void __launch_bounds__(256) reduce_finish(const typename El<DT>::Acc *ws, int64_t n_out, int splits,
                                                     int64_t stride_o, int64_t stride_s, void *out) {
    using A = typename El<DT>::Acc;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < n_out; o += (int64_t)gridDim.x * blockDim.x) {
        A acc[kRedU];
#pragma unroll
        for (int u = 0; u < kRedU; ++u) acc[u] = red_identity<OP, A>();
        for (int s = 0; s < splits; s += kRedU) {
            A v[kRedU];
#pragma unroll
            for (int u = 0; u < kRedU; ++u) v[u] = s + u < splits ? ws[o * stride_o + (s + u) * stride_s] : red_identity<OP, A>();
#pragma unroll
            for (int u = 0; u < kRedU; ++u) acc[u] = red_combine<OP, A>(acc[u], v[u]);
        }
#pragma unroll
        for (int u = 1; u < kRedU; ++u) acc[0] = red_combine<OP, A>(acc[0], acc[u]);
        El<DT>::store(out, o, acc[0]);
    }
}

// The same with a block per output (few outputs, many splits): thread t
// takes partials t, t + 256, ..., then a tree over the block.
template <int DT, int OP>
__global__ void __launch_bounds__(256) reduce_finish_block(const typename El<DT>::Acc *ws, int splits, int64_t stride_o,
                                                           int64_t stride_s, void *out) {
    using A = typename El<DT>::Acc;
    __shared__ A red[256];
    const int64_t o = blockIdx.x;
    A acc = red_identity<OP, A>();
    for (int s = threadIdx.x; s < splits; s += 256) acc = red_combine<OP, A>(acc, ws[o * stride_o + s * stride_s]);
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] = red_combine<OP, A>(red[threadIdx.x], red[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0) El<DT>::store(out, o, red[0]);
}

// ---- dispatch helpers ------------------------------------------------------------

unsigned grid_for(int64_t work) {
    int64_t g = (work + 255) / 256;
    if (g > 65536) g = 65536;
    return (unsigned)(g < 1 ? 1 : g);
}

template <int DT, int NOPS, int OP>
hipError_t ew_launch(const EwShape &s, void *out, const void *x, const void *y, int vec, hipStream_t st) {
    if constexpr (DT != kDtF64) {
        constexpr int V = DT == kDtF32 ? 4 : 8;
        if (vec == kEwContig16) {
            hipLaunchKernelGGL((ew_contig16<DT, NOPS, OP>), dim3(grid_for(s.numel / V)), dim3(256), 0, st, s.numel, out,
                               x, y);
            return hipGetLastError();
        }
        if (vec == kEwInner16) {
            hipLaunchKernelGGL((ew_inner16<DT, NOPS, OP>), dim3(grid_for(s.numel / V)), dim3(256), 0, st, s, out, x, y);
            return hipGetLastError();
        }
    }
    const int64_t runs = s.numel / s.shape[s.ndim - 1] * ((s.shape[s.ndim - 1] + kRun - 1) / kRun);
    hipLaunchKernelGGL((ew_strided<DT, NOPS, OP>), dim3(grid_for(runs)), dim3(256), 0, st, s, out, x, y);
    return hipGetLastError();
}

template <int DT>
hipError_t ew_dispatch(int nops, int op, const EwShape &s, void *out, const void *x, const void *y, int vec,
                       hipStream_t st) {
    if (s.numel == 0) return hipSuccess;
    if (nops == 1) {
        switch (op) {
        case kUnNeg: return ew_launch<DT, 1, kUnNeg>(s, out, x, y, vec, st);
        case kUnExp: return ew_launch<DT, 1, kUnExp>(s, out, x, y, vec, st);
        case kUnLn: return ew_launch<DT, 1, kUnLn>(s, out, x, y, vec, st);
        case kUnAbs: return ew_launch<DT, 1, kUnAbs>(s, out, x, y, vec, st);
        default: return ew_launch<DT, 1, kUnSign>(s, out, x, y, vec, st);
        }
    }
    switch (op) {
    case kBinAdd: return ew_launch<DT, 2, kBinAdd>(s, out, x, y, vec, st);
    case kBinSub: return ew_launch<DT, 2, kBinSub>(s, out, x, y, vec, st);
    case kBinMul: return ew_launch<DT, 2, kBinMul>(s, out, x, y, vec, st);
    case kBinDiv: return ew_launch<DT, 2, kBinDiv>(s, out, x, y, vec, st);
    case kBinEq: return ew_launch<DT, 2, kBinEq>(s, out, x, y, vec, st);
    default: return ew_launch<DT, 2, kBinDGelu>(s, out, x, y, vec, st);
    }
}

// How a reduction is scheduled (red_launch): rows, columns (with 16-byte
// loads when cols_vec), or a thread per output; splits > 1 combines partial
// results from a workspace of sizeof(Acc) * n_out * splits bytes.
struct RedPlan {
    bool rows, cols, cols_vec, cols_tall;
    int64_t splits;
};

template <int DT>
RedPlan plan_reduce(const RedGeom &g, const void *x) {
    RedPlan pl{};
    pl.rows = g.nr == 1 && g.rst[0] == 1 && g.n_red >= 256;
    pl.cols = !pl.rows && g.kst[g.nk - 1] == 1 && g.n_out >= 64 && g.n_red >= 2 * kRedU;
    // column schedule with 16-byte loads: every V-group of consecutive
    // outputs starts 16-byte aligned at every reduced element (x aligned, the
    // innermost kept dim a multiple of V long, every other stride a multiple
    // of V)
    pl.cols_vec = false;
    if constexpr (DT != kDtF64) {
        constexpr int V = DT == kDtF32 ? 4 : 8;
        pl.cols_vec = pl.cols && (uintptr_t)x % 16 == 0 && g.kshape[g.nk - 1] % V == 0;
        for (int d = 0; d + 1 < g.nk; ++d) pl.cols_vec = pl.cols_vec && g.kst[d] % V == 0;
        for (int d = 0; d < g.nr; ++d) pl.cols_vec = pl.cols_vec && g.rst[d] % V == 0;
    }
    // one pass over 128-byte column groups when they give every CU a block and
    // each of the 64 row phases a few loads
    if constexpr (DT != kDtF64) {
        constexpr int V = DT == kDtF32 ? 4 : 8;
        pl.cols_tall = pl.cols_vec && g.n_out / (8 * V) >= 256 && g.n_red >= 4 * kTallPhases;
    }
    int64_t splits = 1;
    if (pl.cols_tall) {
        pl.splits = 1;
        return pl;
    }
    if (pl.rows) {
        splits = 2048 / g.n_out;  // (8192 blocks for one output measured slower: 0.057 vs 0.051 ms)
        const int64_t cap = g.n_red / 4096;  // >= 4096 elements per block
        if (splits > cap) splits = cap;
    } else if (pl.cols) {
        // ~2048 blocks of 256 threads: a streaming pass needs the waves (the
        // [8192, 8192] f32 column sum ran 58 % of HBM peak with 512 blocks,
        // 63-65 % with 2048)
        const int64_t per_block = pl.cols_vec ? 256 * (DT == kDtF32 ? 4 : 8) : 256;
        const int64_t col_blocks = (g.n_out + per_block - 1) / per_block;
        splits = 2048 / col_blocks;
        const int64_t cap = g.n_red / 32;  // >= 32 reduced elements per thread
        if (splits > cap) splits = cap;
    }
    pl.splits = splits < 1 ? 1 : splits;
    return pl;
}

// ws_ext: a caller-provided workspace of at least the plan's size (the
// static scratch of oxm_reduce_noalloc), or nullptr to allocate one on the
// stream.
template <int DT, int OP>
hipError_t red_launch(const RedGeom &g, const void *x, void *out, hipStream_t st, void *ws_ext) {
    using A = typename El<DT>::Acc;
    if (g.n_out == 0) return hipSuccess;
    const RedPlan pl = plan_reduce<DT>(g, x);
    const bool rows = pl.rows, cols = pl.cols, cols_vec = pl.cols_vec;
    const int64_t splits = pl.splits;
    if (!rows && !cols) {
        hipLaunchKernelGGL((reduce_per_thread<DT, OP>), dim3(grid_for(g.n_out)), dim3(256), 0, st, g, x, out);
        return hipGetLastError();
    }
    if constexpr (DT != kDtF64) {
        if (pl.cols_tall) {
            constexpr int V = DT == kDtF32 ? 4 : 8;
            hipLaunchKernelGGL((reduce_cols_tall<DT, OP>), dim3((unsigned)((g.n_out + 8 * V - 1) / (8 * V))),
                               dim3(8 * kTallPhases), 0, st, g, x, out);
            return hipGetLastError();
        }
    }
    A *ws = nullptr;
    bool owned = false;
    hipError_t e;
    if (splits > 1) {
        if (ws_ext) {
            ws = (A *)ws_ext;
        } else {
            if ((e = hipMallocAsync((void **)&ws, sizeof(A) * g.n_out * splits, st)) != hipSuccess) return e;
            owned = true;
        }
    }
    auto finish = [&](int64_t stride_o, int64_t stride_s) {
        if (g.n_out <= 1024 && splits >= 64)
            hipLaunchKernelGGL((reduce_finish_block<DT, OP>), dim3((unsigned)g.n_out), dim3(256), 0, st, ws, (int)splits,
                               stride_o, stride_s, out);
        else
            hipLaunchKernelGGL((reduce_finish<DT, OP>), dim3(grid_for(g.n_out)), dim3(256), 0, st, ws, g.n_out,
                               (int)splits, stride_o, stride_s, out);
    };
    if (rows) {
        bool vec = false;
        if constexpr (DT != kDtF64) {
            constexpr int V = DT == kDtF32 ? 4 : 8;
            vec = (uintptr_t)x % 16 == 0 && g.n_red % V == 0;
            for (int d = 0; d < g.nk; ++d) vec = vec && g.kst[d] % V == 0;
            if (vec && splits == 1 && g.n_out >= 1024) {
                hipLaunchKernelGGL((reduce_rows_wave<DT, OP>), dim3((unsigned)((g.n_out + 3) / 4)), dim3(256), 0, st, g,
                                   x, out);
                return hipGetLastError();
            }
            if (vec)
                hipLaunchKernelGGL((reduce_rows<DT, OP, true>), dim3((unsigned)(g.n_out * splits)), dim3(256), 0, st, g,
                                   x, out, ws, (int)splits);
        }
        if (!vec)
            hipLaunchKernelGGL((reduce_rows<DT, OP, false>), dim3((unsigned)(g.n_out * splits)), dim3(256), 0, st, g, x,
                               out, ws, (int)splits);
        if (splits > 1) finish(splits, (int64_t)1);
    } else {
        if constexpr (DT != kDtF64) {
            constexpr int V = DT == kDtF32 ? 4 : 8;
            if (cols_vec)
                hipLaunchKernelGGL((reduce_cols_vec<DT, OP>),
                                   dim3((unsigned)((g.n_out / V + 255) / 256), (unsigned)splits), dim3(256), 0, st, g,
                                   x, out, (float *)ws, (int)splits);
        }
        if (!cols_vec)
            hipLaunchKernelGGL((reduce_cols<DT, OP>), dim3((unsigned)((g.n_out + 255) / 256), (unsigned)splits),
                               dim3(256), 0, st, g, x, out, ws, (int)splits);
        if (splits > 1)
            hipLaunchKernelGGL((reduce_finish_cols<DT, OP>), dim3((unsigned)((g.n_out + 63) / 64)), dim3(256), 0, st,
                               ws, g.n_out, (int)splits, out);
    }
    e = hipGetLastError();
    if (owned) {
        hipError_t f = hipFreeAsync(ws, st);
        if (e == hipSuccess) e = f;
    }
    return e;
}

template <int DT>
hipError_t red_dispatch(int op, const RedGeom &g, const void *x, void *out, hipStream_t st, void *ws) {
    return op == kRedSum ? red_launch<DT, kRedSum>(g, x, out, st, ws) : red_launch<DT, kRedMax>(g, x, out, st, ws);
}

template <int DT>
size_t ws_bytes(const RedGeom &g, const void *x) {
    if (g.n_out == 0) return 0;
    const RedPlan pl = plan_reduce<DT>(g, x);
    return (pl.rows || pl.cols) && pl.splits > 1 ? sizeof(typename El<DT>::Acc) * g.n_out * pl.splits : 0;
}

}  // namespace

hipError_t launch_elementwise(int dtype, int nops, int op, const EwShape &s, void *out, const void *x, const void *y,
                              int vec, hipStream_t st) {
    switch (dtype) {
    case kDtF32: return ew_dispatch<kDtF32>(nops, op, s, out, x, y, vec, st);
    case kDtBF16: return ew_dispatch<kDtBF16>(nops, op, s, out, x, y, vec, st);
    case kDtF16: return ew_dispatch<kDtF16>(nops, op, s, out, x, y, vec, st);
    default: return ew_dispatch<kDtF64>(nops, op, s, out, x, y, vec, st);
    }
}

hipError_t launch_copy(int elem_bytes, const EwShape &s, void *dst, const void *src, bool contig16, hipStream_t st) {
    if (s.numel == 0) return hipSuccess;
    if (contig16) {
        const int64_t n16 = s.numel * elem_bytes / 16;
        hipLaunchKernelGGL(copy_contig16, dim3(grid_for(n16)), dim3(256), 0, st, n16, (uint4 *)dst, (const uint4 *)src);
        return hipGetLastError();
    }
    const int L = s.ndim - 1;
    int p = -1;
    if (s.ndim >= 2 && s.st[0][L] == 1 && s.st[1][L] != 1 && s.shape[L] >= 16)
        for (int d = L - 1; d >= 0; --d)
            if (s.st[1][d] == 1 && s.shape[d] >= 16) {
                p = d;
                break;
            }
    const int64_t blocks = p < 0 ? 0
                                 : s.numel / (s.shape[p] * s.shape[L]) * ((s.shape[p] + kTT - 1) / kTT) *
                                       ((s.shape[L] + kTT - 1) / kTT);
    if (p >= 0 && blocks <= INT32_MAX) {
        const dim3 g((unsigned)blocks);
        if (elem_bytes == 2 || elem_bytes == 4) {
            const int w = 16 / elem_bytes;
            bool vec = (uintptr_t)dst % 16 == 0 && (uintptr_t)src % 16 == 0 && s.shape[p] % w == 0 &&
                       s.shape[L] % w == 0;
            for (int d = 0; d <= L; ++d) {
                if (d != L) vec = vec && s.st[0][d] % w == 0;
                if (d != p) vec = vec && s.st[1][d] % w == 0;
            }
            if (vec) {
                if (elem_bytes == 2)
                    hipLaunchKernelGGL(copy_transpose_vec<uint16_t>, g, dim3(256), 0, st, s, p, (uint16_t *)dst,
                                       (const uint16_t *)src);
                else
                    hipLaunchKernelGGL(copy_transpose_vec<uint32_t>, g, dim3(256), 0, st, s, p, (uint32_t *)dst,
                                       (const uint32_t *)src);
                return hipGetLastError();
            }
        }
        switch (elem_bytes) {
        case 1: hipLaunchKernelGGL(copy_transpose<uint8_t>, g, dim3(256), 0, st, s, p, (uint8_t *)dst, (const uint8_t *)src); break;
        case 2: hipLaunchKernelGGL(copy_transpose<uint16_t>, g, dim3(256), 0, st, s, p, (uint16_t *)dst, (const uint16_t *)src); break;
        case 4: hipLaunchKernelGGL(copy_transpose<uint32_t>, g, dim3(256), 0, st, s, p, (uint32_t *)dst, (const uint32_t *)src); break;
        default: hipLaunchKernelGGL(copy_transpose<uint64_t>, g, dim3(256), 0, st, s, p, (uint64_t *)dst, (const uint64_t *)src); break;
        }
        return hipGetLastError();
    }
    const int64_t runs = s.numel / s.shape[L] * ((s.shape[L] + kRun - 1) / kRun);
    const dim3 grid(grid_for(runs));
    switch (elem_bytes) {
    case 1: hipLaunchKernelGGL(copy_strided<uint8_t>, grid, dim3(256), 0, st, s, (uint8_t *)dst, (const uint8_t *)src); break;
    case 2: hipLaunchKernelGGL(copy_strided<uint16_t>, grid, dim3(256), 0, st, s, (uint16_t *)dst, (const uint16_t *)src); break;
    case 4: hipLaunchKernelGGL(copy_strided<uint32_t>, grid, dim3(256), 0, st, s, (uint32_t *)dst, (const uint32_t *)src); break;
    default: hipLaunchKernelGGL(copy_strided<uint64_t>, grid, dim3(256), 0, st, s, (uint64_t *)dst, (const uint64_t *)src); break;
    }
    return hipGetLastError();
}

namespace {
template <int DI>
hipError_t convert_from(int dto, const EwShape &s, void *dst, const void *src, hipStream_t st) {
    const int64_t runs = s.numel / s.shape[s.ndim - 1] * ((s.shape[s.ndim - 1] + kRun - 1) / kRun);
    const dim3 grid(grid_for(runs));
    switch (dto) {
    case kDtF32: hipLaunchKernelGGL((convert_strided<DI, kDtF32>), grid, dim3(256), 0, st, s, dst, src); break;
    case kDtBF16: hipLaunchKernelGGL((convert_strided<DI, kDtBF16>), grid, dim3(256), 0, st, s, dst, src); break;
    case kDtF16: hipLaunchKernelGGL((convert_strided<DI, kDtF16>), grid, dim3(256), 0, st, s, dst, src); break;
    default: hipLaunchKernelGGL((convert_strided<DI, kDtF64>), grid, dim3(256), 0, st, s, dst, src); break;
    }
    return hipGetLastError();
}

template <int PDT, int GDT, int MODE, bool WD>
void sgd_go(int64_t n, void *p, const void *g, float *v, float lr, float mu, float wd, hipStream_t st) {
    const bool vec = n % 8 == 0 && (uintptr_t)p % 16 == 0 && (uintptr_t)g % 16 == 0 &&
                     (MODE == 0 || (uintptr_t)v % 16 == 0);
    if (vec)
        hipLaunchKernelGGL((sgd_kernel_vec<PDT, GDT, MODE, WD>), dim3(grid_for(n / 8)), dim3(256), 0, st, n, p, g, v,
                           lr, mu, wd);
    else
        hipLaunchKernelGGL((sgd_kernel<PDT, GDT, MODE, WD>), dim3(grid_for(n)), dim3(256), 0, st, n, p, g, v, lr, mu,
                           wd);
}

template <int PDT, int GDT>
hipError_t sgd_typed(int64_t n, void *p, const void *g, float *v, float lr, float mu, float wd, bool nesterov,
                     hipStream_t st) {
    const bool w = wd != 0.0f;
    if (mu == 0.0f) {
        if (w) sgd_go<PDT, GDT, 0, true>(n, p, g, v, lr, mu, wd, st);
        else sgd_go<PDT, GDT, 0, false>(n, p, g, v, lr, mu, wd, st);
    } else if (!nesterov) {
        if (w) sgd_go<PDT, GDT, 1, true>(n, p, g, v, lr, mu, wd, st);
        else sgd_go<PDT, GDT, 1, false>(n, p, g, v, lr, mu, wd, st);
    } else {
        if (w) sgd_go<PDT, GDT, 2, true>(n, p, g, v, lr, mu, wd, st);
        else sgd_go<PDT, GDT, 2, false>(n, p, g, v, lr, mu, wd, st);
    }
    return hipGetLastError();
}
}  // namespace

hipError_t launch_convert(int dti, int dto, const EwShape &s, void *dst, const void *src, hipStream_t st) {
    if (s.numel == 0) return hipSuccess;
    switch (dti) {
    case kDtF32: return convert_from<kDtF32>(dto, s, dst, src, st);
    case kDtBF16: return convert_from<kDtBF16>(dto, s, dst, src, st);
    case kDtF16: return convert_from<kDtF16>(dto, s, dst, src, st);
    default: return convert_from<kDtF64>(dto, s, dst, src, st);
    }
}

hipError_t launch_sgd(int pdt, int gdt, int64_t n, void *p, const void *g, float *v, float lr, float momentum,
                      float weight_decay, bool nesterov, hipStream_t st) {
    if (n == 0) return hipSuccess;
    if (pdt == kDtF32) return sgd_typed<kDtF32, kDtF32>(n, p, g, v, lr, momentum, weight_decay, nesterov, st);
    if (pdt == kDtBF16)
        return gdt == kDtF32 ? sgd_typed<kDtBF16, kDtF32>(n, p, g, v, lr, momentum, weight_decay, nesterov, st)
                             : sgd_typed<kDtBF16, kDtBF16>(n, p, g, v, lr, momentum, weight_decay, nesterov, st);
    return gdt == kDtF32 ? sgd_typed<kDtF16, kDtF32>(n, p, g, v, lr, momentum, weight_decay, nesterov, st)
                         : sgd_typed<kDtF16, kDtF16>(n, p, g, v, lr, momentum, weight_decay, nesterov, st);
}

hipError_t launch_reduce(int dtype, int op, const RedGeom &g, const void *x, void *out, hipStream_t st, void *ws) {
    switch (dtype) {
    case kDtF32: return red_dispatch<kDtF32>(op, g, x, out, st, ws);
    case kDtBF16: return red_dispatch<kDtBF16>(op, g, x, out, st, ws);
    case kDtF16: return red_dispatch<kDtF16>(op, g, x, out, st, ws);
    default: return red_dispatch<kDtF64>(op, g, x, out, st, ws);
    }
}

size_t reduce_workspace_bytes(int dtype, const RedGeom &g, const void *x) {
    switch (dtype) {
    case kDtF32: return ws_bytes<kDtF32>(g, x);
    case kDtBF16: return ws_bytes<kDtBF16>(g, x);
    case kDtF16: return ws_bytes<kDtF16>(g, x);
    case kDtF64: return ws_bytes<kDtF64>(g, x);
    default: return 0;  // integer reductions take no workspace
    }
}

// The workspace of oxm_reduce_noalloc: device memory the library owns from
// load to exit, one copy per GPU, so callers that cannot allocate (graph
// capture, serving loops) can still split a reduction.  Host code never uses
// this name as an address (in host code it is only a stand-in for the device
// symbol): reduce_scratch() looks the device address up with
// hipGetSymbolAddress once per device and hands that out.
__device__ __align__(256) unsigned char scratch[kReduceScratchBytes];

namespace {
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxScratchDevices] = {};
}  // namespace

hipError_t reduce_scratch(void **ptr) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return hipSuccess;
}

}  // namespace oxm
