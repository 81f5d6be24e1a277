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
    if (dtype == kDtF32) return launch_t<float>(a, s);
    if (dtype == kDtBF16) return launch_t<bf16_t>(a, s);
    return launch_t<f16_t>(a, s);
}

}  // namespace oxm
