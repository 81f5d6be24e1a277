// gemm_kernels.hpp -- gfx950 (CDNA4) MFMA GEMM kernels for strided views.
//
// Design (MI355X-first):
//  * One workgroup computes a BM x BN tile of C for one batch.  Waves are laid
//    out WAVES_M x WAVES_N; each wave owns a (BM/WAVES_M) x (BN/WAVES_N)
//    sub-tile built from 32x32 MFMA blocks whose f32 accumulators live in
//    AGPRs.
//  * K is walked in steps of BK elements = 128 bytes per row.  Both operands
//    are staged through LDS in ONE canonical layout -- K-major rows of 128 B
//    split into eight 16-byte chunks, chunk c of row r stored at position
//    c ^ swz(r) -- so every MFMA fragment is a single ds_read_b128 per lane
//    whatever the operand's layout in HBM.  The XOR swizzle keeps the eight
//    lanes of a ds_read_b128 phase on distinct banks.
//  * Operands are read in place through their element strides.  The global
//    loader is chosen per operand from its layout (no copies, no transposes
//    in HBM):
//      Ld::K   K-contiguous rows, 16-byte loads along K;
//      Ld::MN  M/N-contiguous columns, 16-byte loads along M/N and a
//              register transpose before the LDS store;
//      Ld::G   anything else (odd leading dims, non-unit strides, negative
//              strides): element loads with per-element bounds.
//  * Two LDS buffers: the global loads for step k+1 are issued before the
//    MFMAs of step k and stored to the other buffer after them; one
//    workgroup barrier per step.
//  * Tiles are ordered in groups of GROUP_M tile-rows and spread so that
//    each of the 8 XCDs (each with its own L2) works on a compact region.
//  * Epilogue fused in the store stage: + bias[n], GELU(erf) with the
//    pre-activation saved to aux, or * GELU'(aux) for the backward pass;
//    output in f32, bf16 or f16.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm_args.hpp"

namespace oxm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Storage tags for the 16-bit element types (bit patterns are moved, never
// converted, until the MFMA consumes them).
struct bf16_t {
    uint16_t bits;
};
struct f16_t {
    uint16_t bits;
};

enum class Ld : int { K = 0, MN = 1, G = 2 };

template <typename T>
struct Elem;
template <>
struct Elem<float> {
    static constexpr int kBytes = 4;
};
template <>
struct Elem<bf16_t> {
    static constexpr int kBytes = 2;
};
template <>
struct Elem<f16_t> {
    static constexpr int kBytes = 2;
};

enum : int { kDtF32 = 0, kDtBF16 = 6, kDtF16 = 7 };
enum : int { kActNone = 0, kActGelu = 1, kActDGelu = 2 };

// ---- scalar helpers ------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    _Float16 x = __builtin_bit_cast(_Float16, (uint16_t)h);
    return (float)x;
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);  // RNE conversion
}

__device__ __forceinline__ float load_as_f32(const void *p, int dtype, int64_t i) {
    if (dtype == kDtF32) return ((const float *)p)[i];
    if (dtype == kDtBF16) return bf16_bits_to_f32(((const uint16_t *)p)[i]);
    return f16_bits_to_f32(((const uint16_t *)p)[i]);
}

// GELU with the exact erf form, x * Phi(x), and its derivative
// Phi(x) + x * phi(x).  erff/expf are HIP's device math functions.
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f)); }

__device__ __forceinline__ float dgelu_erf(float x) {
    float cdf = 0.5f * (1.0f + erff(x * 0.70710678118654752440f));
    float pdf = expf(-0.5f * x * x) * 0.39894228040143267794f;
    return cdf + x * pdf;
}

// ---- LDS layout ----------------------------------------------------------

// Byte offset of 16-byte chunk `c` (0..7) of K-major row `r` in an operand
// region.  SWZ selects the XOR pattern (measured with SQ_LDS_BANK_CONFLICT).
template <int SWZ>
__device__ __forceinline__ uint32_t lds_off(int r, int c) {
    int s = (SWZ == 0) ? (r & 7) : ((r >> 1) & 7);
    return (uint32_t)(r * 128 + ((c ^ s) << 4));
}

// ---- global -> LDS loaders -----------------------------------------------

// Loads one operand tile (ROWS rows of the M or N dimension, BK = 128 B of K
// per row) per K step.  `base` already points at (batch, row 0 of the tile,
// k = 0); `s_mn`/`s_k` are element strides; `rows_left` = rows of the tile
// that exist (MN - tile origin); K is the full reduction length.
template <typename T, Ld KIND, int ROWS, int NT, int SWZ>
struct Loader;

// K-contiguous rows: thread t owns chunk (t % 8) of rows t/8, t/8 + NT/8, ...
template <typename T, int ROWS, int NT, int SWZ>
struct Loader<T, Ld::K, ROWS, NT, SWZ> {
    static constexpr int kBytes = Elem<T>::kBytes;
    static constexpr int kVec = 16 / kBytes;
    static constexpr int kBK = 128 / kBytes;
    static constexpr int kPer = ROWS * 8 / NT;
    static_assert(ROWS * 8 % NT == 0, "tile rows must cover the workgroup");
    const char *base;
    int64_t row_off[kPer];  // byte offsets of this thread's rows
    bool row_ok[kPer];
    int chunk;
    int64_t K;
    uint4 regs[kPer];

    __device__ __forceinline__ Loader(const char *b, int64_t s_mn, int64_t /*s_k*/, int64_t rows_left, int64_t k,
                                      int tid)
        : base(b), K(k) {
        chunk = tid & 7;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            int r = (tid >> 3) + i * (NT / 8);
            row_off[i] = (int64_t)r * s_mn * kBytes + chunk * 16;
            row_ok[i] = r < rows_left;
        }
    }
    __device__ __forceinline__ void prefetch(int kt) {
        int64_t k0 = (int64_t)kt * kBK;
        bool k_ok = k0 + chunk * kVec < K;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            if (row_ok[i] && k_ok)
                regs[i] = *(const uint4 *)(base + row_off[i] + k0 * kBytes);
            else
                regs[i] = make_uint4(0, 0, 0, 0);
        }
    }
    __device__ __forceinline__ void store(uint8_t *lds, int tid, int /*kt*/) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            int r = (tid >> 3) + i * (NT / 8);
            *(uint4 *)(lds + lds_off<SWZ>(r, chunk)) = regs[i];
        }
    }
};

// M/N-contiguous columns: thread t owns a kVec(mn) x kVec(k) block: k-block
// t % 8, mn-block t / 8 (+ NT/8 per repeat).  kVec 16-byte loads along MN,
// transposed in registers into kVec K-major 16-byte chunks.
template <typename T, int ROWS, int NT, int SWZ>
struct Loader<T, Ld::MN, ROWS, NT, SWZ> {
    static constexpr int kBytes = Elem<T>::kBytes;
    static constexpr int kVec = 16 / kBytes;
    static constexpr int kBK = 128 / kBytes;
    static constexpr int kBlocks = (ROWS / kVec) * 8;
    static constexpr int kPer = kBlocks >= NT ? kBlocks / NT : 1;
    static_assert(kBlocks % NT == 0 || NT % kBlocks == 0, "block count must tile the workgroup");
    const char *base;
    int64_t s_k_bytes;
    int64_t blk_off[kPer];
    bool blk_ok[kPer];
    bool active;
    int kb;
    int64_t K;
    uint4 regs[kPer][kVec];

    __device__ __forceinline__ Loader(const char *b, int64_t /*s_mn*/, int64_t s_k, int64_t rows_left, int64_t k,
                                      int tid)
        : base(b), K(k) {
        s_k_bytes = s_k * kBytes;
        kb = tid & 7;
        active = tid < kBlocks * kPer;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            int mb = (tid >> 3) + i * (NT / 8);
            blk_off[i] = (int64_t)mb * 16 + (int64_t)kb * kVec * s_k_bytes;
            blk_ok[i] = active && (int64_t)mb * kVec < rows_left;
        }
    }
    __device__ __forceinline__ void prefetch(int kt) {
        int64_t k0 = (int64_t)kt * kBK;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const char *p = base + blk_off[i] + k0 * s_k_bytes;
#pragma unroll
            for (int j = 0; j < kVec; ++j) {
                if (blk_ok[i] && k0 + kb * kVec + j < K)
                    regs[i][j] = *(const uint4 *)(p + j * s_k_bytes);
                else
                    regs[i][j] = make_uint4(0, 0, 0, 0);
            }
        }
    }
    __device__ __forceinline__ void store(uint8_t *lds, int tid, int /*kt*/) {
        if (!active) return;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            int mb = (tid >> 3) + i * (NT / 8);
            if constexpr (kBytes == 4) {
                // 4x4 f32 transpose: pure register renaming.
                const uint32_t *in = (const uint32_t *)regs[i];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    uint4 v = make_uint4(in[0 * 4 + r], in[1 * 4 + r], in[2 * 4 + r], in[3 * 4 + r]);
                    *(uint4 *)(lds + lds_off<SWZ>(mb * 4 + r, kb)) = v;
                }
            } else {
                // 8x8 16-bit transpose: out row r, dword d = (in[2d][r], in[2d+1][r]).
                const uint32_t *in = (const uint32_t *)regs[i];  // in[j*4 + w]: k=j, mn=2w,2w+1
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    uint32_t o[4];
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        uint32_t lo = in[(2 * d) * 4 + (r >> 1)];
                        uint32_t hi = in[(2 * d + 1) * 4 + (r >> 1)];
                        if (r & 1)
                            o[d] = (lo >> 16) | (hi & 0xffff0000u);
                        else
                            o[d] = (lo & 0xffffu) | (hi << 16);
                    }
                    *(uint4 *)(lds + lds_off<SWZ>(mb * 8 + r, kb)) = make_uint4(o[0], o[1], o[2], o[3]);
                }
            }
        }
    }
};

// Generic strided operand: element loads with full bounds checks, issued in
// the store phase (no register staging).  Threads walk the operand's
// unit-ish dimension so neighbouring lanes touch neighbouring addresses.
template <typename T, int ROWS, int NT, int SWZ>
struct Loader<T, Ld::G, ROWS, NT, SWZ> {
    static constexpr int kBytes = Elem<T>::kBytes;
    static constexpr int kVec = 16 / kBytes;
    static constexpr int kBK = 128 / kBytes;
    static constexpr int kPer = ROWS * kBK / NT;
    const char *base;
    int64_t s_mn, s_k, rows_left, K;
    bool along_k;

    __device__ __forceinline__ Loader(const char *b, int64_t smn, int64_t sk, int64_t rl, int64_t k, int /*tid*/)
        : base(b), s_mn(smn), s_k(sk), rows_left(rl), K(k) {
        int64_t am = smn < 0 ? -smn : smn, ak = sk < 0 ? -sk : sk;
        along_k = ak <= am;
    }
    __device__ __forceinline__ void prefetch(int) {}
    __device__ __forceinline__ void store(uint8_t *lds, int tid, int kt) {
        int64_t k0 = (int64_t)kt * kBK;
#pragma unroll 4
        for (int i = 0; i < kPer; ++i) {
            int e = tid + i * NT;
            int r, kk;
            if (along_k) {
                r = e / kBK;
                kk = e % kBK;
            } else {
                r = e % ROWS;
                kk = e / ROWS;
            }
            bool ok = r < rows_left && k0 + kk < K;
            const char *p = base + ((int64_t)r * s_mn + (k0 + kk) * s_k) * kBytes;
            uint32_t off = lds_off<SWZ>(r, kk / kVec) + (kk % kVec) * kBytes;
            if constexpr (kBytes == 4) {
                float v = ok ? *(const float *)p : 0.0f;
                *(float *)(lds + off) = v;
            } else {
                uint16_t v = ok ? *(const uint16_t *)p : (uint16_t)0;
                *(uint16_t *)(lds + off) = v;
            }
        }
    }
};

// ---- MFMA step ------------------------------------------------------------

template <typename T>
struct Mma;

// f32: v_mfma_f32_32x32x2_f32.  A 16-byte fragment holds 4 k values per lane:
// step s uses k = 8g + 4*(lane/32) + s, identically for A and B.
template <>
struct Mma<float> {
    __device__ __forceinline__ static void run(f32x16_t &acc, const uint4 &a, const uint4 &b) {
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
    }
};

// bf16 / f16: v_mfma_f32_32x32x16_{bf16,f16}.  A 16-byte fragment holds the
// 8 k values one lane contributes; lanes 0-31 and 32-63 hold the two k
// halves, identically for A and B.
template <>
struct Mma<bf16_t> {
    __device__ __forceinline__ static void run(f32x16_t &acc, const uint4 &a, const uint4 &b) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                      acc, 0, 0, 0);
    }
};
template <>
struct Mma<f16_t> {
    __device__ __forceinline__ static void run(f32x16_t &acc, const uint4 &a, const uint4 &b) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                     acc, 0, 0, 0);
    }
};

// ---- epilogue -------------------------------------------------------------

template <int OUT_DT>
__device__ __forceinline__ void store_out(void *c, int64_t i, float v) {
    if constexpr (OUT_DT == kDtF32)
        ((float *)c)[i] = v;
    else if constexpr (OUT_DT == kDtBF16)
        ((uint16_t *)c)[i] = f32_to_bf16_bits(v);
    else
        ((uint16_t *)c)[i] = f32_to_f16_bits(v);
}

template <int OUT_DT>
__device__ __forceinline__ float load_out(const void *c, int64_t i) {
    if constexpr (OUT_DT == kDtF32)
        return ((const float *)c)[i];
    else if constexpr (OUT_DT == kDtBF16)
        return bf16_bits_to_f32(((const uint16_t *)c)[i]);
    else
        return f16_bits_to_f32(((const uint16_t *)c)[i]);
}

// Stores four consecutive outputs C[o .. o+3] (o = row*N + col), applying the
// epilogue.  `vec` = the four are in range and 4-element aligned.
template <int OUT_DT>
__device__ __forceinline__ void store4(const GemmArgs &p, int64_t o, int64_t col, float4 v, bool vec, int nvalid) {
    float x[4] = {v.x, v.y, v.z, v.w};
    if (p.act == kActDGelu) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < nvalid) x[i] *= dgelu_erf(load_out<OUT_DT>(p.aux, o + i));
    } else {
        if (p.bias) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (i < nvalid) x[i] += load_as_f32(p.bias, p.bias_dtype, col + i);
        }
        if (p.act == kActGelu) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (i < nvalid) {
                    if (p.aux) store_out<OUT_DT>(p.aux, o + i, x[i]);
                    x[i] = gelu_erf(x[i]);
                }
            }
        }
    }
    if (vec) {
        if constexpr (OUT_DT == kDtF32) {
            *(float4 *)((float *)p.c + o) = make_float4(x[0], x[1], x[2], x[3]);
        } else {
            uint32_t lo, hi;
            if constexpr (OUT_DT == kDtBF16) {
                lo = f32_to_bf16_bits(x[0]) | ((uint32_t)f32_to_bf16_bits(x[1]) << 16);
                hi = f32_to_bf16_bits(x[2]) | ((uint32_t)f32_to_bf16_bits(x[3]) << 16);
            } else {
                lo = f32_to_f16_bits(x[0]) | ((uint32_t)f32_to_f16_bits(x[1]) << 16);
                hi = f32_to_f16_bits(x[2]) | ((uint32_t)f32_to_f16_bits(x[3]) << 16);
            }
            *(uint2 *)((uint16_t *)p.c + o) = make_uint2(lo, hi);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < nvalid) store_out<OUT_DT>(p.c, o + i, x[i]);
    }
}

// Writes one 32-row slab of a wave's accumulators (already staged in LDS as
// f32 [32][WN + 4]) to C with coalesced 4-element stores.
template <int OUT_DT, int WN>
__device__ __forceinline__ void write_slab(const GemmArgs &p, const float *ws, int64_t cbase, int64_t row0,
                                           int64_t col0, int lane) {
    constexpr int kLanesPerRow = WN / 4;
    constexpr int kRowsPerIter = 64 / kLanesPerRow;
    constexpr int kSld = WN + 4;
    const int c4 = (lane % kLanesPerRow) * 4;
    const int64_t col = col0 + c4;
    const int nvalid = (int)(p.N - col < 4 ? (p.N - col < 0 ? 0 : p.N - col) : 4);
    const bool aligned = (p.N & 3) == 0 && (((uintptr_t)p.c) & 15) == 0;
    for (int it = 0; it < 32 / kRowsPerIter; ++it) {
        int r = it * kRowsPerIter + lane / kLanesPerRow;
        int64_t row = row0 + r;
        if (row >= p.M || nvalid == 0) continue;
        float4 v = *(const float4 *)(ws + r * kSld + c4);
        int64_t o = cbase + row * p.N + col;
        store4<OUT_DT>(p, o, col, v, aligned && nvalid == 4, nvalid);
    }
}

// ---- the kernel -------------------------------------------------------------

template <typename T, int BM, int BN, int WAVES_M, int WAVES_N, Ld LA, Ld LB, int SWZ>
__global__ void __launch_bounds__(WAVES_M *WAVES_N * 64) gemm_kernel(GemmArgs p) {
    constexpr int NT = WAVES_M * WAVES_N * 64;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int kBytes = Elem<T>::kBytes;
    constexpr int kBK = 128 / kBytes;
    constexpr int kRegionA = BM * 128, kRegionB = BN * 128;
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be a multiple of 32");
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * (kRegionA + kRegionB)];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    // Tile decode: XCD spreading, then GROUP_M tile-row groups per batch.
    const int64_t per_batch = (int64_t)p.tiles_m * p.tiles_n;
    const int64_t ntiles = per_batch * p.batch;
    int64_t wg = blockIdx.x;
    if (p.xcd_remap && (ntiles & 7) == 0) wg = (wg & 7) * (ntiles >> 3) + (wg >> 3);
    const int64_t bidx = wg / per_batch;
    const int64_t t = wg - bidx * per_batch;
    const int64_t gsz = (int64_t)p.group_m * p.tiles_n;
    const int64_t grp = t / gsz;
    const int64_t first_m = grp * p.group_m;
    const int64_t gm = (p.tiles_m - first_m) < p.group_m ? (p.tiles_m - first_m) : p.group_m;
    const int64_t tin = t - grp * gsz;
    const int64_t tile_m = first_m + tin % gm;
    const int64_t tile_n = tin / gm;
    const int64_t m0 = tile_m * BM, n0 = tile_n * BN;

    int64_t offa = 0, offb = 0, rem = bidx;
    for (int d = p.nbd - 1; d >= 0; --d) {
        int64_t i = rem % p.bext[d];
        rem /= p.bext[d];
        offa += i * p.bsa[d];
        offb += i * p.bsb[d];
    }
    const char *abase = (const char *)p.a + (offa + m0 * p.sam) * kBytes;
    const char *bbase = (const char *)p.b + (offb + n0 * p.sbn) * kBytes;

    Loader<T, LA, BM, NT, SWZ> la(abase, p.sam, p.sak, p.M - m0, p.K, tid);
    Loader<T, LB, BN, NT, SWZ> lb(bbase, p.sbn, p.sbk, p.N - n0, p.K, tid);

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};

    const int nk = (int)((p.K + kBK - 1) / kBK);
    constexpr int kStage = kRegionA + kRegionB;  // bytes per LDS buffer

    if (nk > 0) {
        la.prefetch(0);
        lb.prefetch(0);
        la.store(lds, tid, 0);
        lb.store(lds + kRegionA, tid, 0);
        __syncthreads();
    }
    const int arow = wm * WM + (lane & 31);
    const int brow = wn * WN + (lane & 31);
    const int half = lane >> 5;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {
            la.prefetch(kt + 1);
            lb.prefetch(kt + 1);
        }
        const uint8_t *sa = lds + cur * kStage;
        const uint8_t *sb = sa + kRegionA;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint4 af[TM], bfr[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = *(const uint4 *)(sa + lds_off<SWZ>(arow + i * 32, 2 * g + half));
#pragma unroll
            for (int j = 0; j < TN; ++j) bfr[j] = *(const uint4 *)(sb + lds_off<SWZ>(brow + j * 32, 2 * g + half));
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) Mma<T>::run(acc[i][j], af[i], bfr[j]);
        }
        if (kt + 1 < nk) {
            uint8_t *nxt = lds + (cur ^ 1) * kStage;
            la.store(nxt, tid, kt + 1);
            lb.store(nxt + kRegionA, tid, kt + 1);
        }
        __syncthreads();
    }

    // Epilogue: each wave stages one 32-row slab of its accumulators in LDS
    // (the operand buffers are free after the last barrier), then stores it
    // row-contiguously.  32x32 MFMA accumulator layout: lane l, element e is
    // C[8*(e/4) + 4*(l/32) + e%4][l%32].
    constexpr int kSld = WN + 4;
    static_assert(NT / 64 * 32 * kSld * 4 <= 2 * (kRegionA + kRegionB), "epilogue staging must fit in LDS");
    float *ws = (float *)lds + wave * 32 * kSld;
    const int64_t cbase = bidx * p.M * p.N;
    const int64_t col0 = n0 + wn * WN;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                ws[(8 * (e >> 2) + 4 * half + (e & 3)) * kSld + j * 32 + (lane & 31)] = acc[i][j][e];
        __syncthreads();
        const int64_t row0 = m0 + wm * WM + i * 32;
        if (p.out_dtype == kDtF32)
            write_slab<kDtF32, WN>(p, ws, cbase, row0, col0, lane);
        else if (p.out_dtype == kDtBF16)
            write_slab<kDtBF16, WN>(p, ws, cbase, row0, col0, lane);
        else
            write_slab<kDtF16, WN>(p, ws, cbase, row0, col0, lane);
        __syncthreads();
    }
}

}  // namespace oxm
