// gemm_bf16.hip -- bf16-input instantiations (v_mfma_f32_32x32x16_bf16): the direct-to-LDS and
// register-staged kernels; the one-wave-per-SIMD kernels are in gemm_bf16_1w.hip.
#include "gemm_dispatch.hpp"

namespace oxm {

hipError_t launch_gemm_bf16_1w(const GemmArgs &a, int ld_a, int ld_b, int cfg, hipStream_t s);

hipError_t launch_gemm_bf16(const GemmArgs &a, int ld_a, int ld_b, int cfg, hipStream_t s) {
    if (ld_a != kLdG && ld_b != kLdG && cfg != kCfgH_256_NS) {
        // K- or M/N-contiguous operands: direct-to-LDS ring
        if (cfg == kCfgH_128) return pick_dl<bf16_t, 128, 128, 2, 2, 2, 64, true>(a, ld_a, ld_b, s);
        if (cfg == kCfgH_256_4W) return pick_dl<bf16_t, 256, 256, 2, 2, 2, 64>(a, ld_a, ld_b, s);
        if (cfg == kCfgH_256_1W16 || cfg == kCfgH_256_1W) return launch_gemm_bf16_1w(a, ld_a, ld_b, cfg, s);
        return pick_dl<bf16_t, 256, 256, 2, 4, 2, 64, true>(a, ld_a, ld_b, s);
    }
    if (cfg == kCfgH_128) return pick_a<bf16_t, 128, 128, 2, 2>(a, ld_a, ld_b, s);
    return pick_a<bf16_t, 256, 256, 2, 2>(a, ld_a, ld_b, s);
}

}  // namespace oxm
