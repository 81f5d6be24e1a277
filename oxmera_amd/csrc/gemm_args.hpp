// gemm_args.hpp -- the argument block shared by the host dispatcher and the
// gfx950 GEMM kernels.  Plain data only (it is passed by value as a kernel
// argument).
#pragma once
#include <stdint.h>

namespace oxm {

constexpr int kMaxBatchDims = 6;

// One batched GEMM C[b] = epilogue(A[b] . B[b]) over strided views.
// All strides and offsets are in ELEMENTS (oxmera Layout semantics,
// crates/oxmera-core/src/layout.rs:6-34) and may be negative.
struct GemmArgs {
    const void *a;      // element (b, m, k) at a + boff_a(b) + m*sam + k*sak
    const void *b;      // element (b, k, n) at b + boff_b(b) + k*sbk + n*sbn
    void *c;            // contiguous [batch, M, N] of out_dtype
    const void *bias;   // [N] of bias_dtype or nullptr
    void *aux;          // [batch, M, N] of out_dtype (GELU: pre-act out; DGELU: Z in)
    int64_t M, N, K;
    int64_t sam, sak, sbk, sbn;
    int64_t bsa[kMaxBatchDims];   // a's stride per output batch dim (0 = broadcast)
    int64_t bsb[kMaxBatchDims];
    int64_t bext[kMaxBatchDims];  // output batch extents
    int64_t batch;                // product of bext
    int32_t nbd;                  // number of batch dims
    int32_t act;                  // oxm_act
    int32_t out_dtype;            // oxm_dtype of c / aux
    int32_t bias_dtype;
    int32_t tiles_m, tiles_n;     // tiles per batch
    int32_t group_m;              // tile-row grouping for L2 reuse
    int32_t xcd_remap;            // 1: spread consecutive tiles per XCD
    float *colsum;                // [N] f32 (zeroed by the host), += column sums of the stored C, or nullptr
};

}  // namespace oxm
