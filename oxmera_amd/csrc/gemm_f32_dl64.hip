// gemm_f32_dl64.hip -- the f32 direct-to-LDS kernel on 128x128 tiles and on 64x64 tiles with a
// ring of 8 stages (the operands checked by use_f32_dma in gemm_f32.hip).
#include "gemm_dispatch.hpp"

namespace oxm {

hipError_t launch_gemm_f32_dl64(const GemmArgs &a, int ld_a, int ld_b, int cfg, hipStream_t s) {
    if (cfg == kCfgF32_64) return pick_dlf32<64, 64, 2, 2, 8>(a, ld_a, ld_b, s);
    return pick_dlf32<128, 128, 2, 2>(a, ld_a, ld_b, s);
}

}  // namespace oxm
