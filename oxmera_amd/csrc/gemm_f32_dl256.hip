// gemm_f32_dl256.hip -- the f32 direct-to-LDS kernel on 256x256 and 256x192 tiles (the
// operands checked by use_f32_dma in gemm_f32.hip).
#include "gemm_dispatch.hpp"

namespace oxm {

hipError_t launch_gemm_f32_dl256(const GemmArgs &a, int ld_a, int ld_b, int cfg, hipStream_t s) {
    if (cfg == kCfgF32_256x192) return pick_dlf32<256, 192, 4, 3>(a, ld_a, ld_b, s);
    return pick_dlf32<256, 256, 2, 4>(a, ld_a, ld_b, s);
}

}  // namespace oxm
