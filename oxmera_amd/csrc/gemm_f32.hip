// gemm_f32.hip -- f32 instantiations (v_mfma_f32_32x32x2_f32): the register-staged kernels and,
// for K- or M/N-contiguous operands, the direct-to-LDS kernel (256x256, 256x192, 128x128 and 64x64 tiles).
#include "gemm_dispatch.hpp"

namespace oxm {

hipError_t launch_gemm_f32(const GemmArgs &a, int ld_a, int ld_b, int cfg, hipStream_t s) {
    if (cfg == kCfgF32_256 && use_f32_dma(a, ld_a, ld_b)) return pick_dlf32<256, 256, 2, 4>(a, ld_a, ld_b, s);
    if (cfg == kCfgF32_256x192) {
        // the host takes this configuration only for operands use_f32_dma accepts
        if (!use_f32_dma(a, ld_a, ld_b)) return hipErrorInvalidValue;
        return pick_dlf32<256, 192, 4, 3>(a, ld_a, ld_b, s);
    }
    if (cfg == kCfgF32_256) return pick_a_f32<256, 256, 2, 4>(a, ld_a, ld_b, s);
    if (cfg == kCfgF32_128 && use_f32_dma(a, ld_a, ld_b)) return pick_dlf32<128, 128, 2, 2>(a, ld_a, ld_b, s);
    if (cfg == kCfgF32_64 && use_f32_dma(a, ld_a, ld_b)) return pick_dlf32<64, 64, 2, 2, 8>(a, ld_a, ld_b, s);
    if (cfg == kCfgF32_64) return pick_a_f32<64, 64, 2, 2>(a, ld_a, ld_b, s);
    return pick_a_f32<128, 128, 2, 2>(a, ld_a, ld_b, s);
}

}  // namespace oxm
