// gemm_f32_rs.hip -- the register-staged f32 kernel on 256x256 tiles (operands the direct-to-LDS
// kernel does not take: ragged rows, gathers, misaligned rows).
#include "gemm_dispatch.hpp"

namespace oxm {

hipError_t launch_gemm_f32_rs(const GemmArgs &a, int ld_a, int ld_b, int /*cfg*/, hipStream_t s) {
    return pick_a_f32<256, 256, 2, 4>(a, ld_a, ld_b, s);
}

}  // namespace oxm
