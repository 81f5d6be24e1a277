// gemm_strip.hip -- the last few rows of a GEMM whose other rows run on
// 256x256 MFMA tiles.
//
// When M % 256 leftover rows alone would cost one more round of 256x256
// tiles (4097 x 4095 x 4093: 16 tile-rows fill the 256 CUs once, the 17th
// holds a single row), the dispatcher runs the whole 256-row tiles as usual
// and hands the leftover rows -- at most kStripMaxRows -- to this kernel.
// A strip that thin is bound by reading B once (the MFMA tile kernel would
// compute a full tile per column block for it), so here every block owns 16
// columns and reads B's rows for them exactly once, with plain f32 FMAs:
// thread (c, q) accumulates every strip row of column j0 + c over
// k = q, q + 64, q + 128, ...; the 64 partial sums of a column meet in LDS
// and are added in q order.  Reading B is bound by memory latency, so the
// grid spreads it over all CUs (N / 16 blocks of 1024 threads) and each
// thread keeps 16 loads in flight (K = 4093: four rounds of them; 32 in
// flight measured slower, 55 vs 48 us; 32 columns x 8 phases of 256
// threads 90 us; 16-byte loads of four columns per lane 118 us).  Operands
// are read through their element strides (any layout); the epilogue is a
// plain store.
#include <hip/hip_runtime.h>

#include "gemm_kernels.hpp"
#include "gemm_launch.hpp"

namespace oxm {
namespace {

constexpr int kCols = 16;    // columns per block
constexpr int kPhases = 64;  // k-phases per block (kCols * kPhases = 1024 threads)
constexpr int kUnroll = 16;  // loads of B in flight per thread

template <typename T>
__device__ __forceinline__ float ld_elem(const void *p, int64_t i) {
    if constexpr (Elem<T>::kBytes == 4)
        return ((const float *)p)[i];
    else if constexpr (std::is_same<T, bf16_t>::value)
        return bf16_bits_to_f32(((const uint16_t *)p)[i]);
    else
        return f16_bits_to_f32(((const uint16_t *)p)[i]);
}

template <typename T, int OUT_DT>
__global__ void __launch_bounds__(kCols *kPhases) gemm_strip(GemmArgs p) {
    __shared__ float part[kPhases][kStripMaxRows][kCols];
    const int c = threadIdx.x % kCols, q = threadIdx.x / kCols;
    const int64_t j = (int64_t)blockIdx.x * kCols + c;
    const int rows = (int)p.M;
    float acc[kStripMaxRows];
#pragma unroll
    for (int r = 0; r < kStripMaxRows; ++r) acc[r] = 0.f;
    if (j < p.N) {
        const int64_t boff = j * p.sbn;
        int64_t k = q;
        for (; k + (kUnroll - 1) * kPhases < p.K; k += kUnroll * kPhases) {
            float bk[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) bk[u] = ld_elem<T>(p.b, (k + u * kPhases) * p.sbk + boff);
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
#pragma unroll
                for (int r = 0; r < kStripMaxRows; ++r)
                    if (r < rows) acc[r] = fmaf(ld_elem<T>(p.a, r * p.sam + (k + u * kPhases) * p.sak), bk[u], acc[r]);
        }
        for (; k < p.K; k += kPhases) {
            const float bk = ld_elem<T>(p.b, k * p.sbk + boff);
#pragma unroll
            for (int r = 0; r < kStripMaxRows; ++r)
                if (r < rows) acc[r] = fmaf(ld_elem<T>(p.a, r * p.sam + k * p.sak), bk, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < kStripMaxRows; ++r) part[q][r][c] = acc[r];
    __syncthreads();
    if (q == 0 && j < p.N) {
        for (int r = 0; r < rows; ++r) {
            float s = part[0][r][c];
#pragma unroll
            for (int u = 1; u < kPhases; ++u) s += part[u][r][c];
            store_out<OUT_DT>(p.c, (int64_t)r * p.N + j, s);
        }
    }
}

// Split over K for a row-major (N-contiguous) B: block (g, s) streams the
// slab of B's rows s * kc .. (s + 1) * kc - 1 over the 1024 columns of group
// g (thread t: column 1024 g + t, kSplitU loads in flight), A's slab in LDS,
// and writes its partial sums of every strip row to ws[s][r][j]; strip_sum
// then adds an output's splits in s order (16 phases per output, combined in
// phase order).  A CU then reads 4 KB of each of its B rows instead of 64
// bytes of every row.
constexpr int kSplitCols = 1024;  // columns per block (one per thread)
constexpr int kSplitU = 16;       // loads of B in flight per thread
constexpr int kSumPhases = 16;    // strip_sum: threads per output

template <typename T>
__global__ void __launch_bounds__(kSplitCols) gemm_strip_splitk(GemmArgs p, float *ws, int64_t kc) {
    __shared__ float as[kStripMaxRows][kSplitU];
    const int rows = (int)p.M;
    const int64_t k0 = (int64_t)blockIdx.y * kc;
    const int64_t k1 = k0 + kc < p.K ? k0 + kc : p.K;
    const int64_t j = (int64_t)blockIdx.x * kSplitCols + threadIdx.x;
    const bool col_ok = j < p.N;
    float acc[kStripMaxRows];
#pragma unroll
    for (int r = 0; r < kStripMaxRows; ++r) acc[r] = 0.f;
    for (int64_t k = k0; k < k1; k += kSplitU) {
        __syncthreads();  // the previous step's reads of as
        if (threadIdx.x < kStripMaxRows * kSplitU) {
            const int r = threadIdx.x / kSplitU, u = threadIdx.x % kSplitU;
            as[r][u] = (r < rows && k + u < k1) ? ld_elem<T>(p.a, r * p.sam + (k + u) * p.sak) : 0.f;
        }
        __syncthreads();
        float bk[kSplitU];
#pragma unroll
        for (int u = 0; u < kSplitU; ++u) bk[u] = (col_ok && k + u < k1) ? ld_elem<T>(p.b, (k + u) * p.sbk + j) : 0.f;
#pragma unroll
        for (int r = 0; r < kStripMaxRows; ++r)
            if (r < rows) {
#pragma unroll
                for (int u = 0; u < kSplitU; ++u) acc[r] = fmaf(as[r][u], bk[u], acc[r]);
            }
    }
    if (col_ok) {
        float *dst = ws + (int64_t)blockIdx.y * rows * p.N;
#pragma unroll
        for (int r = 0; r < kStripMaxRows; ++r)
            if (r < rows) dst[(int64_t)r * p.N + j] = acc[r];
    }
}

// out[i] (i over rows x N) = sum over s of ws[s][i] in s order: thread
// (o, q) of a block adds splits q, q + 16, ... of output 64 b + o, and the
// 16 phases are combined in q order.
template <int OUT_DT>
__global__ void __launch_bounds__(64 * kSumPhases) strip_sum(GemmArgs p, const float *ws, int splits) {
    __shared__ float part[kSumPhases][64];
    const int64_t n = p.M * p.N;
    const int o = threadIdx.x % 64, q = threadIdx.x / 64;
    const int64_t i = (int64_t)blockIdx.x * 64 + o;
    float t = 0.f;
    if (i < n)
        for (int s = q; s < splits; s += kSumPhases) t += ws[(int64_t)s * n + i];
    part[q][o] = t;
    __syncthreads();
    if (q == 0 && i < n) {
        float u = part[0][o];
#pragma unroll
        for (int k = 1; k < kSumPhases; ++k) u += part[k][o];
        store_out<OUT_DT>(p.c, i, u);
    }
}

template <typename T>
hipError_t launch_splitk(const GemmArgs &a, hipStream_t s) {
    const int64_t groups = (a.N + kSplitCols - 1) / kSplitCols;
    int64_t splits = 256 / groups;  // about one block per CU
    const int64_t kc = (a.K + splits - 1) / splits;
    splits = (a.K + kc - 1) / kc;
    float *ws = nullptr;
    hipError_t e = hipMallocAsync((void **)&ws, sizeof(float) * splits * a.M * a.N, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((gemm_strip_splitk<T>), dim3((unsigned)groups, (unsigned)splits), dim3(kSplitCols), 0, s, a,
                       ws, kc);
    e = hipGetLastError();
    if (e == hipSuccess) {
        const unsigned grid = (unsigned)((a.M * a.N + 63) / 64);
        if (a.out_dtype == kDtF32)
            hipLaunchKernelGGL((strip_sum<kDtF32>), dim3(grid), dim3(64 * kSumPhases), 0, s, a, ws, (int)splits);
        else if (a.out_dtype == kDtBF16)
            hipLaunchKernelGGL((strip_sum<kDtBF16>), dim3(grid), dim3(64 * kSumPhases), 0, s, a, ws, (int)splits);
        else
            hipLaunchKernelGGL((strip_sum<kDtF16>), dim3(grid), dim3(64 * kSumPhases), 0, s, a, ws, (int)splits);
        e = hipGetLastError();
    }
    const hipError_t f = hipFreeAsync(ws, s);
    return e != hipSuccess ? e : f;
}

template <typename T>
hipError_t launch_t(const GemmArgs &a, hipStream_t s) {
    dim3 grid((unsigned)((a.N + kCols - 1) / kCols)), block(kCols * kPhases);
    if (a.out_dtype == kDtF32)
        hipLaunchKernelGGL((gemm_strip<T, kDtF32>), grid, block, 0, s, a);
    else if (a.out_dtype == kDtBF16)
        hipLaunchKernelGGL((gemm_strip<T, kDtBF16>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((gemm_strip<T, kDtF16>), grid, block, 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_strip(const GemmArgs &a, int dtype, hipStream_t s) {
    if (a.M < 1 || a.M > kStripMaxRows || a.batch != 1) return hipErrorInvalidValue;
    // N-contiguous B of at most 64 column groups, K of at least 4 rows per
    // split: the split-K form (partials of splits x M x N floats, <= 64 MB)
    const int64_t groups = (a.N + kSplitCols - 1) / kSplitCols;
    if (a.sbn == 1 && groups <= 64 && a.K >= 4 * (256 / groups) && (256 / groups) * a.M * a.N * 4 <= (64ll << 20)) {
        if (dtype == kDtF32) return launch_splitk<float>(a, s);
        if (dtype == kDtBF16) return launch_splitk<bf16_t>(a, s);
        return launch_splitk<f16_t>(a, s);
    }
    if (dtype == kDtF32) return launch_t<float>(a, s);
    if (dtype == kDtBF16) return launch_t<bf16_t>(a, s);
    return launch_t<f16_t>(a, s);
}

}  // namespace oxm
