// gemm_bf16_1w.hip -- the one-wave-per-SIMD bf16 kernels (configurations 6 and 7, the latter on
// v_mfma_f32_16x16x32_bf16), in a unit of their own so it builds in parallel with gemm_bf16.hip.
#include "gemm_dispatch.hpp"

namespace oxm {

hipError_t launch_gemm_bf16_1w(const GemmArgs &a, int ld_a, int ld_b, int cfg, hipStream_t s) {
    if (cfg == kCfgH_256_1W16) return pick_dli16<bf16_t>(a, ld_a, ld_b, s);
    return pick_dli<bf16_t>(a, ld_a, ld_b, s);
}

}  // namespace oxm
