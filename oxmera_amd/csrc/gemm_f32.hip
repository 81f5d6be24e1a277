// gemm_f32.hip -- f32 dispatch (v_mfma_f32_32x32x2_f32) and the register-staged kernel on
// 128x128 and 64x64 tiles.  The other instantiations sit in units of their own so they build in
// parallel: gemm_f32_rs.hip (register-staged, 256x256 tiles), gemm_f32_dl256.hip (direct-to-LDS,
// 256x256 and 256x192 tiles) and gemm_f32_dl64.hip (direct-to-LDS, 128x128 and 64x64 tiles).
#include "gemm_dispatch.hpp"

namespace oxm {

hipError_t launch_gemm_f32_rs(const GemmArgs &a, int ld_a, int ld_b, int cfg, hipStream_t s);
hipError_t launch_gemm_f32_dl256(const GemmArgs &a, int ld_a, int ld_b, int cfg, hipStream_t s);
hipError_t launch_gemm_f32_dl64(const GemmArgs &a, int ld_a, int ld_b, int cfg, hipStream_t s);

hipError_t launch_gemm_f32(const GemmArgs &a, int ld_a, int ld_b, int cfg, hipStream_t s) {
    if (cfg == kCfgF32_256x192) {
        // the host takes this configuration only for operands use_f32_dma accepts
        if (!use_f32_dma(a, ld_a, ld_b)) return hipErrorInvalidValue;
        return launch_gemm_f32_dl256(a, ld_a, ld_b, cfg, s);
    }
    if (use_f32_dma(a, ld_a, ld_b)) {
        if (cfg == kCfgF32_256) return launch_gemm_f32_dl256(a, ld_a, ld_b, cfg, s);
        return launch_gemm_f32_dl64(a, ld_a, ld_b, cfg, s);
    }
    if (cfg == kCfgF32_256) return launch_gemm_f32_rs(a, ld_a, ld_b, cfg, s);
    if (cfg == kCfgF32_64) return pick_a_f32<64, 64, 2, 2>(a, ld_a, ld_b, s);
    return pick_a_f32<128, 128, 2, 2>(a, ld_a, ld_b, s);
}

}  // namespace oxm
