// gemm_dispatch.hpp -- maps runtime loader kinds onto kernel instantiations.
#pragma once
#include "gemm_kernels.hpp"
#include "gemm_launch.hpp"

namespace oxm {

template <typename T, int BM, int BN, int WM, int WN, Ld LA, Ld LB, bool SCHED = true>
hipError_t launch_one(const GemmArgs &a, hipStream_t s) {
    int64_t ntiles = (int64_t)a.tiles_m * a.tiles_n * a.batch;
    dim3 grid((unsigned)ntiles), block(WM * WN * 64);
    hipLaunchKernelGGL((gemm_kernel<T, BM, BN, WM, WN, LA, LB, SCHED>), grid, block, 0, s, a);
    return hipGetLastError();
}

// Whether the direct-to-LDS kernels may issue their DMA through
// global_load_lds_dwordx4 (DirectLoader GLB): K a whole number of 64-k
// stages, and not switched off with OXM_GEMM_GLOBAL_DMA=0 (read at each
// call, like OXM_GEMM_CFG).
bool use_global_dma(const GemmArgs &a);

// The f32 direct-to-LDS kernel's DMA goes through global_load_lds when K is
// a multiple of 32 and OXM_GEMM_GLOBAL_DMA is not 0 (use_f32_dma: gemm_launch.hpp).
bool use_global_dma_f32(const GemmArgs &a);

template <int BM, int BN, int WM, int WN, bool AMN, bool BMN, int NS>
hipError_t launch_dlf32(GemmArgs a, hipStream_t s) {
    a.group_m = 4;
    int64_t ntiles = (int64_t)a.tiles_m * a.tiles_n * a.batch;
    dim3 grid((unsigned)ntiles), block(WM * WN * 64);
    if (use_global_dma_f32(a))
        hipLaunchKernelGGL((gemm_kernel_dlf32<BM, BN, WM, WN, AMN, BMN, true, NS>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((gemm_kernel_dlf32<BM, BN, WM, WN, AMN, BMN, false, NS>), grid, block, 0, s, a);
    return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int NS = 2>
hipError_t pick_dlf32(const GemmArgs &a, int la, int lb, hipStream_t s) {
    if (la == kLdK && lb == kLdK) return launch_dlf32<BM, BN, WM, WN, false, false, NS>(a, s);
    if (la == kLdK) return launch_dlf32<BM, BN, WM, WN, false, true, NS>(a, s);
    if (lb == kLdK) return launch_dlf32<BM, BN, WM, WN, true, false, NS>(a, s);
    return launch_dlf32<BM, BN, WM, WN, true, true, NS>(a, s);
}

// Direct-to-LDS kernel (16-bit operands, each K- or M/N-contiguous).
template <typename T, int BM, int BN, int WM, int WN, int NS, int BKS, bool AMN, bool BMN, bool GLB = false>
hipError_t launch_dl(GemmArgs a, hipStream_t s) {
    a.group_m = 4;
    int64_t ntiles = (int64_t)a.tiles_m * a.tiles_n * a.batch;
    dim3 grid((unsigned)ntiles), block(WM * WN * 64);
    hipLaunchKernelGGL((gemm_kernel_dl<T, BM, BN, WM, WN, NS, BKS, AMN, BMN, GLB>), grid, block, 0, s, a);
    return hipGetLastError();
}

// GLB: also instantiate the global_load_lds variant and take it when
// use_global_dma allows (the default configurations).
template <typename T, int BM, int BN, int WM, int WN, int NS, int BKS, bool GLB = false>
hipError_t pick_dl(const GemmArgs &a, int la, int lb, hipStream_t s) {
    if constexpr (GLB) {
        static_assert(BKS == 64, "global DMA with 64-k stages");
        if (use_global_dma(a)) {
            if (la == kLdK && lb == kLdK) return launch_dl<T, BM, BN, WM, WN, NS, BKS, false, false, true>(a, s);
            if (la == kLdK) return launch_dl<T, BM, BN, WM, WN, NS, BKS, false, true, true>(a, s);
            if (lb == kLdK) return launch_dl<T, BM, BN, WM, WN, NS, BKS, true, false, true>(a, s);
            return launch_dl<T, BM, BN, WM, WN, NS, BKS, true, true, true>(a, s);
        }
    }
    if (la == kLdK && lb == kLdK) return launch_dl<T, BM, BN, WM, WN, NS, BKS, false, false>(a, s);
    if (la == kLdK) return launch_dl<T, BM, BN, WM, WN, NS, BKS, false, true>(a, s);
    if (lb == kLdK) return launch_dl<T, BM, BN, WM, WN, NS, BKS, true, false>(a, s);
    return launch_dl<T, BM, BN, WM, WN, NS, BKS, true, true>(a, s);
}

// Direct-to-LDS kernel with one wave per SIMD (2x2 waves, hand-placed stream;
// the OXM_GEMM_CFG=6 tuning configuration).  Measured against the default
// 2x4-wave kernel with the same epilogue: 8192^3 NT, f32 out 0.805 vs 0.807
// ms; the MLP's GEMMs 0.91-1.54 ms vs 0.91-1.26 ms (with a per-element
// epilogue its four waves per CU hide the epilogue's memory traffic worse).
template <typename T, bool AMN, bool BMN>
hipError_t launch_dli(GemmArgs a, hipStream_t s) {
    a.group_m = 4;
    int64_t ntiles = (int64_t)a.tiles_m * a.tiles_n * a.batch;
    dim3 grid((unsigned)ntiles), block(256);
    hipLaunchKernelGGL((gemm_kernel_dli<T, 256, 256, 64, AMN, BMN>), grid, block, 0, s, a);
    return hipGetLastError();
}

template <typename T>
hipError_t pick_dli(const GemmArgs &a, int la, int lb, hipStream_t s) {
    if (la == kLdK && lb == kLdK) return launch_dli<T, false, false>(a, s);
    if (la == kLdK) return launch_dli<T, false, true>(a, s);
    if (lb == kLdK) return launch_dli<T, true, false>(a, s);
    return launch_dli<T, true, true>(a, s);
}

// One wave per SIMD on 16x16x32 MFMAs (AMN / BMN: the operand is M/N-major).
template <typename T, bool AMN, bool BMN>
hipError_t launch_dli16(GemmArgs a, hipStream_t s) {
    a.group_m = 4;
    int64_t ntiles = (int64_t)a.tiles_m * a.tiles_n * a.batch;
    dim3 grid((unsigned)ntiles), block(256);
    if (use_global_dma(a))
        hipLaunchKernelGGL((gemm_kernel_dli16<T, true, 8, 4, 2, AMN, BMN>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((gemm_kernel_dli16<T, false, 8, 4, 2, AMN, BMN>), grid, block, 0, s, a);
    return hipGetLastError();
}

// The 16x16x32 one-wave kernel for K- or M/N-contiguous operands.
template <typename T>
hipError_t pick_dli16(const GemmArgs &a, int la, int lb, hipStream_t s) {
    if (la == kLdK && lb == kLdK) return launch_dli16<T, false, false>(a, s);
    if (la == kLdK) return launch_dli16<T, false, true>(a, s);
    if (lb == kLdK) return launch_dli16<T, true, false>(a, s);
    return launch_dli16<T, true, true>(a, s);
}

template <typename T, int BM, int BN, int WM, int WN, Ld LA>
hipError_t pick_b(const GemmArgs &a, int lb, hipStream_t s) {
    switch (lb) {
    case kLdK: return launch_one<T, BM, BN, WM, WN, LA, Ld::K>(a, s);
    case kLdMN: return launch_one<T, BM, BN, WM, WN, LA, Ld::MN>(a, s);
    default: return launch_one<T, BM, BN, WM, WN, LA, Ld::G>(a, s);
    }
}

template <typename T, int BM, int BN, int WM, int WN>
hipError_t pick_a(const GemmArgs &a, int la, int lb, hipStream_t s) {
    switch (la) {
    case kLdK: return pick_b<T, BM, BN, WM, WN, Ld::K>(a, lb, s);
    case kLdMN: return pick_b<T, BM, BN, WM, WN, Ld::MN>(a, lb, s);
    default: return pick_b<T, BM, BN, WM, WN, Ld::G>(a, lb, s);
    }
}

// f32 with at least one ragged operand: both vector operands take the
// ragged loaders (they are correct for whole rows too).
template <int BM, int BN, int WM, int WN, Ld LA>
hipError_t pick_b_ragged(const GemmArgs &a, int lb, hipStream_t s) {
    switch (lb) {
    case kLdK:
    case kLdKR: return launch_one<float, BM, BN, WM, WN, LA, Ld::KR>(a, s);
    case kLdMN:
    case kLdMNR: return launch_one<float, BM, BN, WM, WN, LA, Ld::MNR>(a, s);
    default: return launch_one<float, BM, BN, WM, WN, LA, Ld::G>(a, s);
    }
}

template <int BM, int BN, int WM, int WN>
hipError_t pick_a_f32(const GemmArgs &a, int la, int lb, hipStream_t s) {
    if (la != kLdKR && la != kLdMNR && lb != kLdKR && lb != kLdMNR) return pick_a<float, BM, BN, WM, WN>(a, la, lb, s);
    switch (la) {
    case kLdK:
    case kLdKR: return pick_b_ragged<BM, BN, WM, WN, Ld::KR>(a, lb, s);
    case kLdMN:
    case kLdMNR: return pick_b_ragged<BM, BN, WM, WN, Ld::MNR>(a, lb, s);
    default: return pick_b_ragged<BM, BN, WM, WN, Ld::G>(a, lb, s);
    }
}

}  // namespace oxm
