// gemm_launch.hpp -- host-side entry into the GEMM kernels.
#pragma once
#include <hip/hip_runtime.h>

#include "gemm_args.hpp"

namespace oxm {

// Operand loader kinds (the kernel's Ld enum, as plain ints for the host).
// kLdKR / kLdMNR: f32 K- / M/N-contiguous rows whose length is not a
// multiple of 4 (the kernels shift the straddling chunk into place).
enum LoaderKind : int { kLdK = 0, kLdMN = 1, kLdG = 2, kLdKR = 3, kLdMNR = 4 };

// Tile configurations.
enum TileCfg : int {
    kCfgF32_128 = 0,   // f32: 128x128 tile, 2x2 waves of 64x64, BK 32
    kCfgH_256 = 1,     // bf16/f16: 256x256 tile, 2x4 waves of 128x64 (direct-to-LDS), BK 64
    kCfgH_128 = 2,     // bf16/f16: 128x128 tile, 2x2 waves of 64x64, BK 64
                       // (K- or M/N-contiguous operands use the direct-to-LDS kernel:
                       //  2 stages of 64 k, 128-byte rows)
    // tuning variants (16-bit; selected by OXM_GEMM_CFG)
    kCfgH_256_4W = 3,  // direct-to-LDS 256x256 with 2x2 waves of 128x128
    kCfgH_256_NS = 4,  // 256x256 register-staged kernel instead of the direct-to-LDS one
    kCfgF32_256 = 5,   // f32: 256x256 tile, 2x4 waves of 128x64, BK 32 (problems of >= 256 tiles)
    kCfgH_256_1W = 6,  // 16-bit direct-to-LDS 256x256, 2x2 waves of 128x128, one wave per SIMD,
                       // hand-interleaved MFMA / fragment-read / DMA stream
    kCfgH_256_1W16 = 7,  // as kCfgH_256_1W on 16x16x32 MFMAs (K- or M/N-contiguous operands)
    kCfgF32_64 = 8,    // f32: 64x64 tile, 2x2 waves of 32x32, BK 32 (problems of <= 64 128x128 tiles)
    kCfgF32_256x192 = 9,  // f32: 256x192 tile, 4x3 waves of 64x64, direct-to-LDS only (K- or
                          // M/N-contiguous, 16-byte aligned rows): a whole number of rounds where
                          // 256x256 tiles leave CUs idle (C4: 256 tiles instead of 192)
};

struct TileShape {
    int bm, bn;
};
TileShape tile_shape(int cfg);

// Row strip: at most this many leftover rows of a GEMM run on the strip
// kernel (gemm_strip.hip) instead of a round of mostly empty 256x256 tiles.
constexpr int kStripMaxRows = 16;

// C[0..M) = A[0..M) . B for a strip of M <= kStripMaxRows rows, one batch, a
// plain store epilogue (no bias, activation or column sums); `args` is
// validated by the caller.
hipError_t launch_gemm_strip(const GemmArgs &args, int dtype, hipStream_t stream);

// f32 on 256x256, 256x192 and 128x128 tiles: the direct-to-LDS kernel
// (gemm_kernel_dlf32) serves K- or M/N-contiguous operands (la, lb: kLdK or
// kLdMN) whose rows all start 16-byte aligned, unless OXM_GEMM_F32_DMA=0
// (read at each call) keeps the register-staged kernel.  256x192 tiles exist
// on this kernel only.
bool use_f32_dma(const GemmArgs &a, int la, int lb);

// Launch one batched GEMM.  `args` must be fully validated by the caller;
// tiles_m/tiles_n/group_m/xcd_remap are filled in here.
hipError_t launch_gemm(GemmArgs args, int dtype, int ld_a, int ld_b, int cfg, hipStream_t stream);

}  // namespace oxm
