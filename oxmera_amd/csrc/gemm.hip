// gemm.hip -- tile-shape table and dtype dispatch of the GEMM kernels.
// The instantiations live in translation units per dtype (gemm_f32*.hip,
// gemm_bf16*.hip, gemm_f16*.hip) so they build in parallel.
#include <cstdlib>

#include "gemm_dispatch.hpp"
#include "gemm_launch.hpp"
#include "gemm_kernels.hpp"

namespace oxm {

hipError_t launch_gemm_f32(const GemmArgs &a, int ld_a, int ld_b, int cfg, hipStream_t s);
hipError_t launch_gemm_bf16(const GemmArgs &a, int ld_a, int ld_b, int cfg, hipStream_t s);
hipError_t launch_gemm_f16(const GemmArgs &a, int ld_a, int ld_b, int cfg, hipStream_t s);

static bool env_off(const char *name) {
    const char *v = getenv(name);
    return v && v[0] == '0';
}

bool use_global_dma(const GemmArgs &a) {
    return a.K >= 64 && a.K % 64 == 0 && !env_off("OXM_GEMM_GLOBAL_DMA");
}

bool use_global_dma_f32(const GemmArgs &a) {
    return a.K >= 32 && a.K % 32 == 0 && !env_off("OXM_GEMM_GLOBAL_DMA");
}

bool use_f32_dma(const GemmArgs &a, int la, int lb) {
    if (env_off("OXM_GEMM_F32_DMA")) return false;
    if ((la != kLdK && la != kLdMN) || (lb != kLdK && lb != kLdMN)) return false;
    // every row (K-major) or k-row (M/N-major) of both operands starts 16-byte aligned
    if ((uintptr_t)a.a % 16 != 0 || (uintptr_t)a.b % 16 != 0) return false;
    const int64_t ra = la == kLdK ? a.sam : a.sak, rb = lb == kLdK ? a.sbn : a.sbk;
    if (ra % 4 != 0 || rb % 4 != 0) return false;
    for (int d = 0; d < a.nbd; ++d)
        if (a.bsa[d] % 4 != 0 || a.bsb[d] % 4 != 0) return false;
    return true;
}

TileShape tile_shape(int cfg) {
    switch (cfg) {
    case kCfgH_256:
    case kCfgH_256_4W:
    case kCfgH_256_1W:
    case kCfgH_256_1W16:
    case kCfgH_256_NS:
    case kCfgF32_256: return {256, 256};
    case kCfgH_128: return {128, 128};
    case kCfgF32_64: return {64, 64};
    case kCfgF32_256x192: return {256, 192};
    default: return {128, 128};
    }
}

hipError_t launch_gemm(GemmArgs args, int dtype, int ld_a, int ld_b, int cfg, hipStream_t stream) {
    TileShape ts = tile_shape(cfg);
    args.tiles_m = (int32_t)((args.M + ts.bm - 1) / ts.bm);
    args.tiles_n = (int32_t)((args.N + ts.bn - 1) / ts.bn);
    args.group_m = 8;
    args.xcd_remap = 1;
    if (dtype == kDtF32) return launch_gemm_f32(args, ld_a, ld_b, cfg, stream);
    if (dtype == kDtBF16) return launch_gemm_bf16(args, ld_a, ld_b, cfg, stream);
    return launch_gemm_f16(args, ld_a, ld_b, cfg, stream);
}

}  // namespace oxm
