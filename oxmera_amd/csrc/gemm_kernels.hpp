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
//      Ld::KR, Ld::MNR  the same for f32 rows whose length (K, or M/N) is
//              not a multiple of 4: the straddling chunk is loaded as the
//              row's last 16 bytes and shifted into place;
//      Ld::G   anything else (non-unit or negative strides, 16-bit rows
//              not 16-byte aligned): element loads with per-element bounds.
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

#include <type_traits>

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

enum class Ld : int { K = 0, MN = 1, G = 2, KR = 3, MNR = 4 };

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
enum : int { kActNone = 0, kActGelu = 1, kActDGelu = 2, kActGeluGrad = 3, kActMulAux = 4 };

// Whether the epilogue reads aux (as Z, or as the factor) rather than writing it.
__device__ __forceinline__ bool act_reads_aux(int act) { return act == kActDGelu || act == kActMulAux; }

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

// GELU in the erf form, x * Phi(x), and its derivative Phi(x) + x * phi(x),
// with the normal CDF from Abramowitz & Stegun, Handbook of Mathematical
// Functions (1964), formula 7.1.26: for u >= 0
//   erfc(u) = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-u^2) + eps,
//   t = 1 / (1 + p u),  |eps| <= 1.5e-7.
// With u = |x| / sqrt(2), exp(-u^2) = exp(-x^2 / 2) is also phi(x) * sqrt(2 pi),
// so GELU' costs one exponential and one reciprocal (HIP's erff + expf cost
// ~3x more per element, and in a GEMM epilogue the MFMA pipes idle meanwhile).
// Measured in f32 against float64 erf on [-12, 12]: |error| <= 1.9e-7
// (GELU) and 3.2e-7 (GELU') times max(1, |x|); NaN propagates.
struct NormalParts {
    float cdf;  // Phi(x)
    float e;    // exp(-x^2 / 2)
};

__device__ __forceinline__ NormalParts normal_parts(float x) {
    const float u = fabsf(x) * 0.70710678118654752440f;
    const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * u);
    const float e = __builtin_amdgcn_exp2f(-0.72134752044448170368f * x * x);  // log2(e) / 2
    const float poly = t * (0.254829592f + t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f +
                                                                                       t * 1.061405429f))));
    const float q = 0.5f * poly * e;  // Phi(-|x|)
    return {x >= 0.0f ? 1.0f - q : q, e};
}

__device__ __forceinline__ float gelu_erf(float x) { return x * normal_parts(x).cdf; }

__device__ __forceinline__ float dgelu_erf(float x) {
    const NormalParts n = normal_parts(x);
    return n.cdf + x * n.e * 0.39894228040143267794f;  // 1 / sqrt(2 pi)
}

// GELU(x) and GELU'(x) from one evaluation of the normal parts.
__device__ __forceinline__ void gelu_and_grad(float x, float &g, float &d) {
    const NormalParts n = normal_parts(x);
    g = x * n.cdf;
    d = n.cdf + x * n.e * 0.39894228040143267794f;
}

// ---- LDS layout ----------------------------------------------------------

// Byte offset of 16-byte chunk `c` (0..7) of K-major row `r` (128 B per row)
// in an operand region.  The LDS serves 256 B per cycle, so a ds_read_b128
// phase covers 16 lanes: rows are paired into 256-byte lines, the pair's
// halves are exchanged when bit 3 of the row is set, and chunks are XORed
// with bits 1..3 of the row.  Then
//   * fragment reads (16 consecutive rows, one chunk) hit 16 distinct
//     16-byte bank groups;
//   * K-loader writes (2 rows x 8 chunks per 16 lanes) and M/N-loader writes
//     (rows r and r+8 x 8 chunks) do as well.
__device__ __forceinline__ uint32_t lds_off(int r, int c) {
    const int half = (r & 1) ^ ((r >> 3) & 1);
    return (uint32_t)((r >> 1) * 256 + half * 128 + ((c ^ ((r >> 1) & 7)) << 4));
}

// ---- buffer loads ---------------------------------------------------------

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Byte offsets at or beyond a resource's num_records read as zero; kOob is
// never inside a resource (num_records <= kMaxRec).
constexpr uint32_t kMaxRec = 0x7FFFFF00u;
constexpr uint32_t kOob = 0x7FFFFFE0u;  // + up to 16 bytes stays below 2^31

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const char *base, int64_t nbytes) {
    if (nbytes < 0) nbytes = 0;
    if (nbytes > (int64_t)kMaxRec) nbytes = kMaxRec;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(base), (short)0, (int)nbytes, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// A 16-byte chunk moved down by `bytes` (0 < bytes < 16) with zeros shifted
// in at the top: element e of the result is element e + bytes/size of `v`.
// Used for the chunk that straddles the end of a row whose length is not a
// multiple of the vector width: the last 16 bytes of the row are loaded
// (always inside it) and shifted so the chunk's valid elements come first.
__device__ __forceinline__ uint4 shift_down_bytes(uint4 v, int bytes) {
    // branch-free in `bytes` (0 <= bytes < 16; 0 returns v)
    const uint64_t lo = (uint64_t)v.x | ((uint64_t)v.y << 32), hi = (uint64_t)v.z | ((uint64_t)v.w << 32);
    const int b = 8 * bytes;
    const uint64_t lo_small = (lo >> (b & 63)) | (b ? hi << ((64 - b) & 63) : 0);
    const uint64_t lo_big = hi >> ((b - 64) & 63);
    const uint64_t nlo = b >= 64 ? lo_big : lo_small;
    const uint64_t nhi = b >= 64 ? 0 : hi >> (b & 63);
    return make_uint4((uint32_t)nlo, (uint32_t)(nlo >> 32), (uint32_t)nhi, (uint32_t)(nhi >> 32));
}

// ---- global -> LDS loaders -----------------------------------------------

// Loads one operand tile (ROWS rows of the M or N dimension, BK = 128 B of K
// per row) per K step.  `base` points at (batch, first row of the tile,
// k = 0); `s_mn`/`s_k` are element strides; `rows_left` = rows of the tile
// that exist (MN - tile origin); K is the full reduction length.  The host
// only selects Ld::K / Ld::MN when the strides are non-negative and the
// tile's byte range fits a buffer resource; 16-bit operands must also be
// 16-byte aligned with K (Ld::K) or M/N (Ld::MN) a multiple of 8, while f32
// rows may start at any 4-byte boundary (16-byte loads need only dword
// alignment) and end mid-chunk, provided a row (Ld::K: K; Ld::MN: every
// tile's M/N extent) holds at least one whole chunk.
template <typename T, Ld KIND, int ROWS, int NT, int NSET>
struct Loader;

// K-contiguous rows: thread t owns chunk (t % 8) of rows t/8, t/8 + NT/8, ...
// RG: K need not be a multiple of kVec (Ld::KR).
template <typename T, int ROWS, int NT, int NSET, bool RG>
struct LoaderK {
    static constexpr int kBytes = Elem<T>::kBytes;
    static constexpr int kVec = 16 / kBytes;
    static constexpr int kBK = 128 / kBytes;
    static constexpr int kPer = ROWS * 8 / NT;
    static_assert(ROWS * 8 % NT == 0, "tile rows must cover the workgroup");
    static constexpr int kVmem = kPer, kDsWrite = kPer;  // instructions per K step
    const char *base;
    int64_t nbytes;
    uint32_t off[kPer];  // byte offsets of this thread's chunks (kOob: row absent)
    int chunk;
    int64_t K;
    uint4 regs[NSET][kPer];  // staging sets (NSET = prefetch distance)

    __device__ __forceinline__ LoaderK(const char *b, int64_t s_mn, int64_t /*s_k*/, int64_t rows_left, int64_t k,
                                       int tid)
        : base(b), K(k) {
        chunk = tid & 7;
        const int64_t rows_here = rows_left < ROWS ? rows_left : ROWS;
        nbytes = ((rows_here - 1) * s_mn + k) * kBytes;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            int r = (tid >> 3) + i * (NT / 8);
            off[i] = r < rows_left ? (uint32_t)(r * s_mn * kBytes + chunk * 16) : kOob;
        }
    }
    // Bytes the chunk of step kt must be shifted down by: non-zero only for
    // the chunk that straddles K (K not a multiple of kVec, K >= kVec), which
    // is loaded as the row's last kVec elements.
    __device__ __forceinline__ int tail_shift(int kt) const {
        const int64_t kc = (int64_t)kt * kBK + chunk * kVec;
        return (kc < K && kc + kVec > K) ? (int)(kc + kVec - K) * kBytes : 0;
    }
    template <int S>
    __device__ __forceinline__ void prefetch(int kt) {
        const int64_t k0 = (int64_t)kt * kBK;
        if constexpr (!RG) {
            const __amdgpu_buffer_rsrc_t rs = make_rsrc(base + k0 * kBytes, nbytes - k0 * kBytes);
            const bool k_ok = (k0 + kBK <= K) || (k0 + chunk * kVec < K);
#pragma unroll
            for (int i = 0; i < kPer; ++i) regs[S][i] = buf_load16(rs, k_ok ? off[i] : kOob);
        } else if (k0 + kBK <= K) {
            const __amdgpu_buffer_rsrc_t rs = make_rsrc(base + k0 * kBytes, nbytes - k0 * kBytes);
#pragma unroll
            for (int i = 0; i < kPer; ++i) regs[S][i] = buf_load16(rs, off[i]);
        } else {
            // last step: the resource starts kVec elements early so a shifted
            // chunk's offset stays non-negative
            const int64_t back = k0 >= kVec ? kVec : 0;
            const __amdgpu_buffer_rsrc_t rs = make_rsrc(base + (k0 - back) * kBytes, nbytes - (k0 - back) * kBytes);
            const bool in = k0 + chunk * kVec < K;
            const uint32_t adj = (uint32_t)(back * kBytes - tail_shift(kt));
#pragma unroll
            for (int i = 0; i < kPer; ++i) regs[S][i] = buf_load16(rs, in ? off[i] + adj : kOob);
        }
    }
    template <int S>
    __device__ __forceinline__ void store(uint8_t *lds, int tid, int kt) {
        if (RG && (int64_t)kt * kBK + kBK > K && (K & (kVec - 1)) != 0) {  // uniform: ragged last step
            const int sh = tail_shift(kt);
#pragma unroll
            for (int i = 0; i < kPer; ++i) regs[S][i] = shift_down_bytes(regs[S][i], sh);
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            int r = (tid >> 3) + i * (NT / 8);
            *(uint4 *)(lds + lds_off(r, chunk)) = regs[S][i];
        }
    }
};

template <typename T, int ROWS, int NT, int NSET>
struct Loader<T, Ld::K, ROWS, NT, NSET> : LoaderK<T, ROWS, NT, NSET, false> {
    using LoaderK<T, ROWS, NT, NSET, false>::LoaderK;
};
template <typename T, int ROWS, int NT, int NSET>
struct Loader<T, Ld::KR, ROWS, NT, NSET> : LoaderK<T, ROWS, NT, NSET, true> {
    using LoaderK<T, ROWS, NT, NSET, true>::LoaderK;
};

// M/N-contiguous columns: thread t owns a kVec(mn) x kVec(k) block, k-block
// t % 8; kVec 16-byte loads along MN are transposed in registers into kVec
// K-major 16-byte chunks.  Blocks are assigned so that the two 8-lane halves
// of every 16-lane LDS phase write rows 8 apart (opposite bank halves).
// RG: M/N need not be a multiple of kVec (Ld::MNR).
template <typename T, int ROWS, int NT, int NSET, bool RG>
struct LoaderMN {
    static constexpr int kBytes = Elem<T>::kBytes;
    static constexpr int kVec = 16 / kBytes;
    static constexpr int kBK = 128 / kBytes;
    static constexpr int kBlocks = (ROWS / kVec) * 8;
    static constexpr int kPer = kBlocks >= NT ? kBlocks / NT : 1;
    static_assert(kBlocks % NT == 0 || NT % kBlocks == 0, "block count must tile the workgroup");
    static constexpr int kVmem = kPer * kVec, kDsWrite = kPer * kVec;
    const char *base;
    int64_t nbytes, sk_bytes;
    uint32_t off[kPer];
    int mb[kPer];
    int shift[kPer];  // bytes a block straddling a ragged M/N edge is shifted down by
    bool ok[kPer];
    bool ragged;      // tile-uniform: some block straddles the M/N edge
    bool active;
    int kb;
    int64_t K;
    uint4 regs[NSET][kPer][kVec];

    __device__ __forceinline__ static int block_of(int q) {
        if constexpr (kVec == 8) {
            return q;  // rows 8q..8q+7: neighbours q, q+1 are 8 rows apart
        } else {
            // 4-row blocks: pair q = 2j + s with blocks j' and j' + 2 (8 rows apart)
            const int j = (q & 7) >> 1, s = q & 1;
            return (q & ~7) + (j & 1) + 4 * (j >> 1) + 2 * s;
        }
    }

    __device__ __forceinline__ LoaderMN(const char *b, int64_t /*s_mn*/, int64_t s_k, int64_t rows_left, int64_t k,
                                        int tid)
        : base(b), K(k) {
        sk_bytes = s_k * kBytes;
        kb = tid & 7;
        active = tid < kBlocks * kPer;
        const int64_t rows_here = rows_left < ROWS ? rows_left : ROWS;
        ragged = RG && (rows_here & (kVec - 1)) != 0;
        nbytes = (k - 1) * sk_bytes + rows_here * kBytes;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            mb[i] = block_of((tid >> 3) + i * (NT / 8));
            ok[i] = active && (int64_t)mb[i] * kVec < rows_left;
            // A block that straddles the edge (the tile holds >= kVec rows, so
            // it is not the first) loads the last kVec rows and is shifted.
            const int nv = (int)rows_here - mb[i] * kVec;
            shift[i] = (RG && ok[i] && nv < kVec) ? (kVec - nv) * kBytes : 0;
            off[i] = (uint32_t)(mb[i] * 16 - shift[i] + kb * kVec * sk_bytes);
        }
    }
    template <int S>
    __device__ __forceinline__ void prefetch(int kt) {
        const int64_t k0 = (int64_t)kt * kBK;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(base + k0 * sk_bytes, nbytes - k0 * sk_bytes);
        const bool full = k0 + kBK <= K;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
#pragma unroll
            for (int j = 0; j < kVec; ++j) {
                const bool v = ok[i] && (full || k0 + kb * kVec + j < K);
                regs[S][i][j] = buf_load16(rs, v ? off[i] + (uint32_t)(j * sk_bytes) : kOob);
            }
        }
    }
    template <int S>
    __device__ __forceinline__ void store(uint8_t *lds, int /*tid*/, int /*kt*/) {
        if (!active) return;
        if (RG && ragged) {
#pragma unroll
            for (int i = 0; i < kPer; ++i)
#pragma unroll
                for (int j = 0; j < kVec; ++j) regs[S][i][j] = shift_down_bytes(regs[S][i][j], shift[i]);
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            if constexpr (kBytes == 4) {
                // 4x4 f32 transpose: register renaming only.
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    uint4 v;
                    v.x = (&regs[S][i][0].x)[r];
                    v.y = (&regs[S][i][1].x)[r];
                    v.z = (&regs[S][i][2].x)[r];
                    v.w = (&regs[S][i][3].x)[r];
                    *(uint4 *)(lds + lds_off(mb[i] * 4 + r, kb)) = v;
                }
            } else {
                // 8x8 16-bit transpose: output row r, dword d = (in[2d][r], in[2d+1][r]).
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    uint32_t o[4];
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const uint32_t lo = (&regs[S][i][2 * d].x)[r >> 1];
                        const uint32_t hi = (&regs[S][i][2 * d + 1].x)[r >> 1];
                        o[d] = (r & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
                    }
                    *(uint4 *)(lds + lds_off(mb[i] * 8 + r, kb)) = make_uint4(o[0], o[1], o[2], o[3]);
                }
            }
        }
    }
};

template <typename T, int ROWS, int NT, int NSET>
struct Loader<T, Ld::MN, ROWS, NT, NSET> : LoaderMN<T, ROWS, NT, NSET, false> {
    using LoaderMN<T, ROWS, NT, NSET, false>::LoaderMN;
};
template <typename T, int ROWS, int NT, int NSET>
struct Loader<T, Ld::MNR, ROWS, NT, NSET> : LoaderMN<T, ROWS, NT, NSET, true> {
    using LoaderMN<T, ROWS, NT, NSET, true>::LoaderMN;
};

// Generic strided operand: element loads with full bounds checks, issued in
// the store phase (no register staging).  Threads walk the operand's
// smaller-stride dimension so neighbouring lanes touch neighbouring addresses.
template <typename T, int ROWS, int NT, int NSET>
struct Loader<T, Ld::G, ROWS, NT, NSET> {
    static constexpr int kBytes = Elem<T>::kBytes;
    static constexpr int kVec = 16 / kBytes;
    static constexpr int kBK = 128 / kBytes;
    static constexpr int kPer = ROWS * kBK / NT;
    static constexpr int kVmem = -1, kDsWrite = -1;  // data-dependent: no fixed schedule
    const char *base;
    int64_t s_mn, s_k, rows_left, K;
    bool along_k;

    __device__ __forceinline__ Loader(const char *b, int64_t smn, int64_t sk, int64_t rl, int64_t k, int /*tid*/)
        : base(b), s_mn(smn), s_k(sk), rows_left(rl), K(k) {
        int64_t am = smn < 0 ? -smn : smn, ak = sk < 0 ? -sk : sk;
        along_k = ak <= am;
    }
    template <int S>
    __device__ __forceinline__ void prefetch(int) {}
    template <int S>
    __device__ __forceinline__ void store(uint8_t *lds, int tid, int kt) {
        const int64_t k0 = (int64_t)kt * kBK;
#pragma unroll 4
        for (int i = 0; i < kPer; ++i) {
            const int e = tid + i * NT;
            int r, kk;
            if (along_k) {
                r = e / kBK;
                kk = e % kBK;
            } else {
                r = e % ROWS;
                kk = e / ROWS;
            }
            const bool ok = r < rows_left && k0 + kk < K;
            const char *p = base + ((int64_t)r * s_mn + (k0 + kk) * s_k) * kBytes;
            const uint32_t o = lds_off(r, kk / kVec) + (kk % kVec) * kBytes;
            if constexpr (kBytes == 4) {
                float v = ok ? *(const float *)p : 0.0f;
                *(float *)(lds + o) = v;
            } else {
                uint16_t v = ok ? *(const uint16_t *)p : (uint16_t)0;
                *(uint16_t *)(lds + o) = v;
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
// The value a store of OUT_DT keeps, as f32 (what a later read sees).
template <int OUT_DT>
__device__ __forceinline__ float stored_value(float x) {
    if constexpr (OUT_DT == kDtF32)
        return x;
    else if constexpr (OUT_DT == kDtBF16)
        return bf16_bits_to_f32(f32_to_bf16_bits(x));
    else
        return f16_bits_to_f32(f32_to_f16_bits(x));
}

// Four consecutive elements of a C-shaped array (OUT_DT) at element offset o,
// as f32.  `vec`: the four are in range and 16-byte aligned (one vector load);
// otherwise the first nvalid are loaded one by one and the rest read as 0.
template <int OUT_DT>
__device__ __forceinline__ void load4_out(const void *c, int64_t o, bool vec, int nvalid, float (&z)[4]) {
    if (vec) {
        if constexpr (OUT_DT == kDtF32) {
            const f32x4_t v = *(const f32x4_t *)((const float *)c + o);
            z[0] = v[0], z[1] = v[1], z[2] = v[2], z[3] = v[3];
        } else {
            const uint2 u = *(const uint2 *)((const uint16_t *)c + o);
            const uint32_t h[4] = {u.x & 0xffffu, u.x >> 16, u.y & 0xffffu, u.y >> 16};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                z[i] = OUT_DT == kDtBF16 ? bf16_bits_to_f32(h[i]) : f16_bits_to_f32(h[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) z[i] = i < nvalid ? load_out<OUT_DT>(c, o + i) : 0.f;
    }
}

// Stores four consecutive values (rounded to OUT_DT) at element offset o of a
// C-shaped array; `vec` as in load4_out.  Vector stores are non-temporal: the
// epilogue's arrays are written once and read by no later work of this
// kernel, and keeping them out of the caches' way keeps the operand lines
// that other tiles still read (8192^3 bf16 with f32 output: 0.805 ms instead
// of 0.852 ms).
template <int OUT_DT>
__device__ __forceinline__ void store4_out(void *c, int64_t o, const float (&x)[4], bool vec, int nvalid) {
    if (vec) {
        if constexpr (OUT_DT == kDtF32) {
            __builtin_nontemporal_store(f32x4_t{x[0], x[1], x[2], x[3]}, (f32x4_t *)((float *)c + o));
        } else {
            typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
            uint32_t lo, hi;
            if constexpr (OUT_DT == kDtBF16) {
                lo = f32_to_bf16_bits(x[0]) | ((uint32_t)f32_to_bf16_bits(x[1]) << 16);
                hi = f32_to_bf16_bits(x[2]) | ((uint32_t)f32_to_bf16_bits(x[3]) << 16);
            } else {
                lo = f32_to_f16_bits(x[0]) | ((uint32_t)f32_to_f16_bits(x[1]) << 16);
                hi = f32_to_f16_bits(x[2]) | ((uint32_t)f32_to_f16_bits(x[3]) << 16);
            }
            __builtin_nontemporal_store(u32x2_t{lo, hi}, (u32x2_t *)((uint16_t *)c + o));
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < nvalid) store_out<OUT_DT>(c, o + i, x[i]);
    }
}

// Applies the epilogue to 4 adjacent outputs (row-major offset o, nvalid of
// them inside N) and stores them: + bias (b4, this lane's four columns) and
// GELU with the pre-activation saved to aux, or * GELU'(z4) (z4: the aux
// values of these outputs, loaded by the caller); with p.colsum, adds the
// stored values to cs.
template <int OUT_DT>
__device__ __forceinline__ void store4(const GemmArgs &p, int64_t o, float4 v, bool vec, int nvalid,
                                       const float (&b4)[4], const float (&z4)[4], float (&cs)[4]) {
    float x[4] = {v.x, v.y, v.z, v.w};
    if (p.act == kActDGelu) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < nvalid) x[i] *= dgelu_erf(z4[i]);
    } else if (p.act == kActMulAux) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < nvalid) x[i] *= z4[i];
    } else {
        if (p.bias) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (i < nvalid) x[i] += b4[i];
        }
        if (p.act == kActGelu) {
            if (p.aux) store4_out<OUT_DT>(p.aux, o, x, vec, nvalid);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (i < nvalid) x[i] = gelu_erf(x[i]);
        } else if (p.act == kActGeluGrad) {
            float d[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (i < nvalid) gelu_and_grad(x[i], x[i], d[i]);
            if (p.aux) store4_out<OUT_DT>(p.aux, o, d, vec, nvalid);
        }
    }
    if (p.colsum) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < nvalid) cs[i] += stored_value<OUT_DT>(x[i]);
    }
    store4_out<OUT_DT>(p.c, o, x, vec, nvalid);
}

// The aux (pre-activation) values one lane multiplies into a 32-row slab under
// GELU' (lane l owns columns 4 (l % (WN/4)) .. +3 of rows l / (WN/4),
// + 64/(WN/4), ..., as in write_slab), as raw 8- or 16-byte loads converted
// when used.  The epilogue issues the loads of all its slabs before its first
// store: vmcnt counts loads and stores alike, so once a store is outstanding a
// load can only be waited for with every earlier store, and per-row loads
// would wait out the write latency again and again.
template <int OUT_DT, int WN>
struct AuxSlab {
    static constexpr int kIters = 32 / (64 / (WN / 4));
    using Raw = typename std::conditional<OUT_DT == kDtF32, f32x4_t, uint2>::type;
    Raw raw[kIters];
};

// Whether the stores (and aux reads) of four columns take one vector access:
// 16-byte aligned C and aux rows of a multiple of 4 columns.
__device__ __forceinline__ bool slab_aligned(const GemmArgs &p) {
    return (p.N & 3) == 0 && (((uintptr_t)p.c) & 15) == 0 && (((uintptr_t)p.aux) & 15) == 0;
}

// Loads a slab's aux values for a lane; only called when slab_aligned(p).
// Rows past M and columns past N read row M-1 / columns N-4 .. N-1 instead
// (in bounds; write_slab skips those rows and loads edge columns itself), so
// the loads take no branches.
template <int OUT_DT, int WN>
__device__ __forceinline__ void load_aux_slab(const GemmArgs &p, int64_t cbase, int64_t row0, int64_t col0, int lane,
                                              AuxSlab<OUT_DT, WN> &s) {
    using Raw = typename AuxSlab<OUT_DT, WN>::Raw;
    constexpr int kLanesPerRow = WN / 4;
    constexpr int kRowsPerIter = 64 / kLanesPerRow;
    constexpr int kEs = OUT_DT == kDtF32 ? 4 : 2;
    int64_t col = col0 + (lane % kLanesPerRow) * 4;
    col = col + 4 <= p.N ? col : p.N - 4;
    const int r0 = lane / kLanesPerRow;
    const char *base = (const char *)p.aux + (cbase + col) * kEs;
#pragma unroll
    for (int it = 0; it < AuxSlab<OUT_DT, WN>::kIters; ++it) {
        int64_t row = row0 + it * kRowsPerIter + r0;
        row = row < p.M ? row : p.M - 1;
        s.raw[it] = *(const Raw *)(base + row * p.N * kEs);
    }
}

template <int OUT_DT>
__device__ __forceinline__ void unpack4(const f32x4_t &v, float (&z)[4]) {
    z[0] = v[0], z[1] = v[1], z[2] = v[2], z[3] = v[3];
}
template <int OUT_DT>
__device__ __forceinline__ void unpack4(const uint2 &u, float (&z)[4]) {
    const uint32_t h[4] = {u.x & 0xffffu, u.x >> 16, u.y & 0xffffu, u.y >> 16};
#pragma unroll
    for (int i = 0; i < 4; ++i) z[i] = OUT_DT == kDtBF16 ? bf16_bits_to_f32(h[i]) : f16_bits_to_f32(h[i]);
}

// Writes one 32-row slab of a wave's accumulators (already staged in LDS as
// f32 [32][WN + 8]) to C with coalesced 4-element stores; lane l owns columns
// col0 + 4 (l % (WN/4)) .. +3 of rows l / (WN/4), + 64/(WN/4), ...  b4: the
// bias of the lane's four columns.  PRE: an aux-reading epilogue (GELU',
// MUL_AUX) with the slab's aux values prefetched in `pre` (lanes that could
// not prefetch load them here).
template <int OUT_DT, int WN, bool PRE>
__device__ __forceinline__ void write_slab(const GemmArgs &p, const float *ws, int64_t cbase, int64_t row0,
                                           int64_t col0, int lane, const float (&b4)[4], float (&cs)[4],
                                           const AuxSlab<OUT_DT, WN> &pre) {
    constexpr int kLanesPerRow = WN / 4;
    constexpr int kRowsPerIter = 64 / kLanesPerRow;
    constexpr int kIters = 32 / kRowsPerIter;
    constexpr int kSld = WN + 8;
    const int c4 = (lane % kLanesPerRow) * 4;
    const int64_t col = col0 + c4;
    const int nvalid = (int)(p.N - col < 4 ? (p.N - col < 0 ? 0 : p.N - col) : 4);
    const bool vec = slab_aligned(p) && nvalid == 4;
    const int r0 = lane / kLanesPerRow;
    if constexpr (PRE) {
#pragma unroll
        for (int it = 0; it < kIters; ++it) {
            const int r = it * kRowsPerIter + r0;
            const int64_t row = row0 + r;
            if (row >= p.M || nvalid == 0) continue;
            const int64_t o = cbase + row * p.N + col;
            float z4[4];
            if (vec)
                unpack4<OUT_DT>(pre.raw[it], z4);
            else
                load4_out<OUT_DT>(p.aux, o, false, nvalid, z4);
            const float4 v = *(const float4 *)(ws + r * kSld + c4);
            store4<OUT_DT>(p, o, v, vec, nvalid, b4, z4, cs);
        }
    } else {
#pragma unroll 2
        for (int it = 0; it < kIters; ++it) {
            const int r = it * kRowsPerIter + r0;
            const int64_t row = row0 + r;
            if (row >= p.M || nvalid == 0) continue;
            const int64_t o = cbase + row * p.N + col;
            float z4[4] = {0.f, 0.f, 0.f, 0.f};
            if (act_reads_aux(p.act)) load4_out<OUT_DT>(p.aux, o, vec, nvalid, z4);
            const float4 v = *(const float4 *)(ws + r * kSld + c4);
            store4<OUT_DT>(p, o, v, vec, nvalid, b4, z4, cs);
        }
    }
}

// Adds a wave's column partial sums (cs, per lane as in write_slab) into
// p.colsum: lanes that own the same columns are summed with cross-lane
// shuffles, then one lane per column group issues the atomics.
template <int WN>
__device__ __forceinline__ void colsum_flush(const GemmArgs &p, float (&cs)[4], int64_t col0, int lane) {
    constexpr int kLanesPerRow = WN / 4;
#pragma unroll
    for (int off = kLanesPerRow; off < 64; off <<= 1)
#pragma unroll
        for (int i = 0; i < 4; ++i) cs[i] += __shfl_xor(cs[i], off);
    if (lane < kLanesPerRow) {
        const int64_t col = col0 + lane * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (col + i < p.N) atomicAdd(p.colsum + col + i, cs[i]);
    }
}

// Orders this wave's LDS accesses before and after it for all of the wave's
// lanes (the epilogue's staging area is per wave, so no other wave is waited
// for: waves write their slabs out independently; against block barriers
// here it measured the same, within 0.3 %, on C3, C2, C4 and the MLP).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// f(integral_constant<I>), f(integral_constant<I + 1>), ..., f(integral_constant<N - 1>).
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// Writes 32-row slab I of a wave's accumulators into the LDS slab ws (f32
// [32][WN + 8]).  32x32 blocks (f32x16_t): lane l holds column l % 32 of rows
// 8 (e / 4) + 4 (l / 32) + e % 4 of block row I.  16x16 blocks (f32x4_t):
// lane l holds column l % 16 of rows 4 (l / 16) + e; the slab is block rows
// 2I and 2I + 1.
template <int I, int WN, int TM, int TN>
__device__ __forceinline__ void fill_slab(float *ws, f32x16_t (&acc)[TM][TN], int lane) {
    constexpr int kSld = WN + 8;
    const int half = lane >> 5;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e)
            ws[(8 * (e >> 2) + 4 * half + (e & 3)) * kSld + j * 32 + (lane & 31)] = acc[I][j][e];
}
template <int I, int WN, int TM, int TN>
__device__ __forceinline__ void fill_slab(float *ws, f32x4_t (&acc)[TM][TN], int lane) {
    constexpr int kSld = WN + 8;
    const int q = lane >> 4;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) ws[(16 * h + 4 * q + e) * kSld + j * 16 + (lane & 15)] = acc[2 * I + h][j][e];
}

// 32-row slabs in a wave tile of TM block rows.
template <typename Acc, int TM>
constexpr int kSlabs = std::is_same<Acc, f32x16_t>::value ? TM : TM / 2;

// LDS-staged epilogue: each wave writes its WM x WN accumulators one 32-row
// slab at a time through a padded LDS slab (row stride WN + 8 floats), then
// stores rows with 16-byte writes, applying the bias and activation (under
// GELU' the next slab's aux values load while a slab is written).  The caller
// has drained every DMA into `lds` and synchronised.
template <int OUT_DT, int WN, typename Acc, int TM, int TN>
__device__ __forceinline__ void epilogue_slabs(const GemmArgs &p, Acc (&acc)[TM][TN], float *ws, int lane,
                                               int64_t cbase, int64_t row_base, int64_t col0, const float (&b4)[4],
                                               float (&cs)[4]) {
    constexpr int NSLAB = kSlabs<Acc, TM>;
    // an aux-reading epilogue (GELU', MUL_AUX) with 16-bit output and
    // 64-column wave tiles: every slab's aux values (64 VGPRs at most) load
    // before the first store; otherwise write_slab loads them per row
    constexpr bool kPre = OUT_DT != kDtF32 && WN <= 64;
    const bool pre_ok = kPre && act_reads_aux(p.act) && slab_aligned(p);
    AuxSlab<OUT_DT, WN> pre[kPre ? NSLAB : 1];
    if constexpr (kPre) {
        if (pre_ok) {
#pragma unroll
            for (int i = 0; i < NSLAB; ++i) load_aux_slab<OUT_DT, WN>(p, cbase, row_base + i * 32, col0, lane, pre[i]);
        }
    }
    static_for<0, NSLAB>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        fill_slab<i, WN>(ws, acc, lane);
        wave_sync();
        const int64_t row0 = row_base + i * 32;
        if (pre_ok)
            write_slab<OUT_DT, WN, kPre>(p, ws, cbase, row0, col0, lane, b4, cs, pre[kPre ? i : 0]);
        else
            write_slab<OUT_DT, WN, false>(p, ws, cbase, row0, col0, lane, b4, cs, pre[0]);
        wave_sync();
    });
}

template <int NT, int WM, int WN, int TM, int TN, int LDS_BYTES, typename Acc>
__device__ __forceinline__ void epilogue_lds(const GemmArgs &p, Acc (&acc)[TM][TN], uint8_t *lds, int wave,
                                             int lane, int64_t cbase, int64_t row_base, int64_t col0) {
    constexpr int kSld = WN + 8;
    static_assert(NT / 64 * 32 * kSld * 4 <= LDS_BYTES, "epilogue staging must fit in LDS");
    float *ws = (float *)lds + wave * 32 * kSld;
    float cs[4] = {0.f, 0.f, 0.f, 0.f};  // column sums of the stored output (p.colsum)
    float b4[4] = {0.f, 0.f, 0.f, 0.f};  // bias of this lane's four columns (the same in every row)
    if (p.bias && !act_reads_aux(p.act)) {
        const int64_t col = col0 + (lane % (WN / 4)) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (col + i < p.N) b4[i] = load_as_f32(p.bias, p.bias_dtype, col + i);
    }
    if (p.out_dtype == kDtF32)
        epilogue_slabs<kDtF32, WN>(p, acc, ws, lane, cbase, row_base, col0, b4, cs);
    else if (p.out_dtype == kDtBF16)
        epilogue_slabs<kDtBF16, WN>(p, acc, ws, lane, cbase, row_base, col0, b4, cs);
    else
        epilogue_slabs<kDtF16, WN>(p, acc, ws, lane, cbase, row_base, col0, b4, cs);
    if (p.colsum) colsum_flush<WN>(p, cs, col0, lane);
}

// ---- the kernel -------------------------------------------------------------

template <typename T, int BM, int BN, int WAVES_M, int WAVES_N, Ld LA, Ld LB, bool SCHED = true, int PF = 1>
__global__ void __launch_bounds__(WAVES_M *WAVES_N * 64) gemm_kernel(GemmArgs p) {
    constexpr int NT = WAVES_M * WAVES_N * 64;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int kBytes = Elem<T>::kBytes;
    constexpr int kBK = 128 / kBytes;
    constexpr int kRegionA = BM * 128, kRegionB = BN * 128;
    constexpr int kStage = kRegionA + kRegionB;  // bytes per LDS buffer
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be a multiple of 32");
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kStage];

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

    int64_t offa = 0, offb = 0;
    if (p.nbd > 0) {
        int64_t rem = bidx;
        for (int d = p.nbd - 1; d >= 0; --d) {
            int64_t i = rem % p.bext[d];
            rem /= p.bext[d];
            offa += i * p.bsa[d];
            offb += i * p.bsb[d];
        }
    }
    const char *abase = (const char *)p.a + (offa + m0 * p.sam) * kBytes;
    const char *bbase = (const char *)p.b + (offb + n0 * p.sbn) * kBytes;

    Loader<T, LA, BM, NT, PF> la(abase, p.sam, p.sak, p.M - m0, p.K, tid);
    Loader<T, LB, BN, NT, PF> lb(bbase, p.sbn, p.sbk, p.N - n0, p.K, tid);
    // f32: the step's global loads go out spread over group 0's MFMAs, one
    // every kLoadGap (4096^3 on 256x256 tiles: 1.015 ms back to back, 1.002
    // one per MFMA, 0.988 one every 4 MFMAs)
    constexpr int kLoads = decltype(la)::kVmem + decltype(lb)::kVmem;
    constexpr int kLoadGapMax = kLoads > 0 ? TM * TN * 4 / kLoads : 1;
    constexpr int kLoadGap = kLoadGapMax < 1 ? 1 : (kLoadGapMax > 4 ? 4 : kLoadGapMax);
    constexpr bool kSpreadLoads = SCHED && NT >= 256 && kBytes == 4 && decltype(la)::kVmem > 0 &&
                                  decltype(lb)::kVmem > 0 && kLoads <= TM * TN * 4;

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};

    // Fragment addressing: lane l reads chunk 2g + l/32 of row (base + l%32 +
    // 32 i); rows 32 apart share the swizzle, so tile i adds i * 4096 bytes.
    const int half = lane >> 5;
    const int arow = wm * WM + (lane & 31);
    const int brow = wn * WN + (lane & 31);
    uint32_t aoff[4], boff[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        aoff[g] = lds_off(arow, 2 * g + half);
        boff[g] = kRegionA + lds_off(brow, 2 * g + half);
    }
    uint4 fa[2][TM], fb[2][TN];
    auto read_frags = [&](const uint8_t *stage, int g, uint4(&A)[TM], uint4(&B)[TN]) {
#pragma unroll
        for (int i = 0; i < TM; ++i) A[i] = *(const uint4 *)(stage + aoff[g] + i * 4096);
#pragma unroll
        for (int j = 0; j < TN; ++j) B[j] = *(const uint4 *)(stage + boff[g] + j * 4096);
    };

    // Pipeline: LDS double buffer (stage kt&1 is computed while stage
    // (kt+1)&1 is filled) and PF register sets for the global loads: step
    // kt+PF is loaded into set (kt+PF)%PF while set (kt+1)%PF is stored.
    // Order of one K step, pinned with scheduling fences (without them the
    // compiler sinks the global loads next to their LDS stores and exposes
    // the full memory latency every step):
    //   global loads of step kt+PF
    //   for g = 0..2: LDS reads of group g+1, MFMAs of group g
    //   LDS stores of step kt+1, barrier, LDS reads of group 0 of kt+1,
    //   MFMAs of group 3 (under the latency of those reads).
    // Loads past the end of K are out of range and read zeros.
    static_assert(PF == 1 || PF == 2, "prefetch distance 1 or 2");
    const int nk = (int)((p.K + kBK - 1) / kBK);
    if (nk > 0) {
        la.template prefetch<0>(0);
        lb.template prefetch<0>(0);
        la.template store<0>(lds, tid, 0);
        lb.template store<0>(lds + kRegionA, tid, 0);
        if constexpr (PF == 2) {
            la.template prefetch<1>(1);
            lb.template prefetch<1>(1);
        }
        __syncthreads();
        read_frags(lds, 0, fa[0], fb[0]);
    }
    auto k_step = [&](auto sc, int kt) {
        constexpr int S = decltype(sc)::value;  // kt % 2 for PF == 2
        const int cur = PF == 2 ? S : (kt & 1);
        const uint8_t *stage = lds + cur * kStage;
        uint8_t *nxt = lds + (cur ^ 1) * kStage;
        constexpr int kLoadSet = PF == 2 ? S : 0, kStoreSet = PF == 2 ? (S ^ 1) : 0;
        la.template prefetch<kLoadSet>(kt + PF);
        lb.template prefetch<kLoadSet>(kt + PF);
        if constexpr (SCHED && !kSpreadLoads) __builtin_amdgcn_sched_barrier(0);
        static_for<0, 3>([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            read_frags(stage, g + 1, fa[(g + 1) & 1], fb[(g + 1) & 1]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) Mma<T>::run(acc[i][j], fa[g & 1][i], fb[g & 1][j]);
            if constexpr (kSpreadLoads && g == 0) {
                static_for<0, kLoads>([&](auto) {
                    __builtin_amdgcn_sched_group_barrier(0x008, kLoadGap, 0);  // kLoadGap MFMAs
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);         // one global load
                });
            }
            if constexpr (SCHED) __builtin_amdgcn_sched_barrier(0);
        });
        la.template store<kStoreSet>(nxt, tid, kt + 1);
        lb.template store<kStoreSet>(nxt + kRegionA, tid, kt + 1);
        __syncthreads();
        // group 3's MFMAs use registers only: issued after the barrier, they
        // keep the MFMA pipe busy while the next step's first fragments load
        read_frags(nxt, 0, fa[0], fb[0]);
        if constexpr (SCHED) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) Mma<T>::run(acc[i][j], fa[1][i], fb[1][j]);
        if constexpr (SCHED) __builtin_amdgcn_sched_barrier(0);
    };
    if constexpr (PF == 2) {
        for (int kt = 0; kt < nk; kt += 2) {
            k_step(std::integral_constant<int, 0>{}, kt);
            if (kt + 1 < nk) k_step(std::integral_constant<int, 1>{}, kt + 1);
        }
    } else {
        for (int kt = 0; kt < nk; ++kt) k_step(std::integral_constant<int, 0>{}, kt);
    }

    // Epilogue (the operand buffers are free after the last barrier).
    epilogue_lds<NT, WM, WN, TM, TN, 2 * kStage>(p, acc, lds, wave, lane, bidx * p.M * p.N, m0 + wm * WM, n0 + wn * WN);
}

// ===========================================================================
// Direct-to-LDS pipeline for 16-bit operands that are both K-contiguous.
//
// The register-staged kernel above keeps one K step (64 KB for a 256x256
// tile) in flight per CU, and at 8192^3 that leaves the MFMAs waiting on
// global-load latency.  Here global loads go straight into LDS
// (buffer_load_dwordx4 ... lds: no VGPR staging, no ds_write) and the LDS is
// a ring of NS stages of 32 k each, so NS-1 stages (96-128 KB) are in flight
// while one is consumed.  One barrier per stage.
// ===========================================================================

// K-major stage layout (operand K-contiguous in HBM): 64-byte rows (32 k of
// a 16-bit type, four 16-byte chunks), four rows per 256-byte line; chunk c
// of row r sits at position (r % 4) * 4 + (c ^ ((r / 4) % 4)) of its line.  A
// fragment read (16 consecutive rows, one chunk) covers all 16 positions of
// the 256-byte bank width.
__device__ __forceinline__ uint32_t lds_off64(int r, int c) {
    return (uint32_t)((r >> 2) * 256 + (((r & 3) << 2) | (c ^ ((r >> 2) & 3))) * 16);
}

// M/N-major stage layout (operand M/N-contiguous in HBM): one row of ROWS
// elements per k (32 rows), in 64-byte segments; segment s of k-row r is
// stored at segment s ^ (r % 4).  The DMA copies k-rows as they lie in HBM;
// fragments are formed with transposing reads (ds_read_b64_tr_b16).
template <int ROWS>
__device__ __forceinline__ uint32_t lds_off_mn(int r, int byte_in_row) {
    return (uint32_t)(r * ROWS * 2 + ((((byte_in_row >> 6) ^ (r & 3)) << 6) | (byte_in_row & 63)));
}

// s_waitcnt immediate that waits for vmcnt <= n and nothing else (gfx9
// encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
constexpr int waitcnt_vm(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | ((n >> 4) << 14); }

// Global -> LDS DMA of one operand tile (ROWS rows of M or N, BKS k) per
// stage.  Each wave instruction fills one 1 KB block; every lane fetches the
// 16 bytes that belong at its position (lane L writes block byte 16 L), so
// the stage layout is produced by the choice of global addresses.  With
// BKS = 64 a K-major row is 128 bytes and every row is one 128-byte request
// (BKS = 32 halves the bytes per L2 request).
//
// GLB: the DMA goes through global_load_lds_dwordx4 (64-bit base + 32-bit
// lane offset) instead of buffer_load_dwordx4 ... lds: the same data
// movement, but its issue stalls the wave about half as long (8192^3 bf16 on
// the one-wave kernel: 2554 against 2850 cycles per 64-k stage).  It has no
// range check, so it serves only K a multiple of BKS (no partial chunk to
// zero): rows (K-major) or 8-element column chunks (M/N-major) past the
// operand's edge read the last valid ones instead -- they feed only outputs
// past M or N, which are never stored -- and steps past K re-read the last
// step into a stage that is never consumed.
//
// SW16 (M/N-major, read by FragReader16MN): within each 64-byte segment the
// two 32-byte halves are exchanged when bit 3 of the k-row is set.
template <int ROWS, int NT, bool MN, int BKS, bool GLB = false, bool SW16 = false>
struct DirectLoader {
    static constexpr int kWaves = NT / 64;
    static constexpr int kBlocks = ROWS * BKS * 2 / 1024;
    static constexpr int kPer = kBlocks / kWaves;  // load instructions per wave per stage
    static_assert(kBlocks % kWaves == 0, "blocks must divide among the waves");
    static_assert(BKS == 32 || BKS == 64, "32 or 64 k per stage");
    const char *base;
    int64_t nbytes, K, sk_bytes;
    uint32_t voff[kPer];
    int krow[kPer];  // M/N-major: the k-row each lane fills
    int chunk;       // K-major: the k-chunk each lane fills

    __device__ __forceinline__ DirectLoader(const char *b, int64_t s_mn, int64_t s_k, int64_t rows_left, int64_t k,
                                            int wave, int lane)
        : base(b), K(k) {
        const int64_t rows_here = rows_left < ROWS ? rows_left : ROWS;
        if constexpr (!MN) {
            sk_bytes = 2;
            nbytes = ((rows_here - 1) * s_mn + k) * 2;
            const int line = lane >> 4, pos = lane & 15;
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                const int blk = wave + i * kWaves;
                int r;
                if constexpr (BKS == 32) {
                    // 16 rows x 64 B per block: row 16 b + 4 (L/16) + (L%16)/4, chunk (L%4) ^ (L/16)
                    chunk = (pos & 3) ^ line;
                    r = blk * 16 + line * 4 + (pos >> 2);
                } else {
                    // 8 rows x 128 B per block (inverse of lds_off): line sr = 4 b + L/16,
                    // half h = (L%16)/8, position p = L%8
                    const int sr = blk * 4 + line, h = pos >> 3, pc = pos & 7;
                    r = 2 * sr + (h ^ ((sr >> 2) & 1));
                    chunk = pc ^ (sr & 7);
                }
                if constexpr (GLB) {
                    const int64_t rc = r < rows_left ? r : rows_left - 1;
                    voff[i] = (uint32_t)(rc * s_mn * 2 + chunk * 16);
                } else {
                    voff[i] = r < rows_left ? (uint32_t)(r * s_mn * 2 + chunk * 16) : kOob;
                }
                krow[i] = 0;
            }
        } else {
            // block b covers 1024 / (2 ROWS) k-rows; lane L's byte in the stage
            // is 1024 b + 16 L
            sk_bytes = s_k * 2;
            chunk = 0;
            nbytes = (k - 1) * sk_bytes + rows_here * 2;
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                const int blk = wave + i * kWaves;
                const int pos = blk * 1024 + lane * 16;
                const int r = pos / (ROWS * 2), bir = pos % (ROWS * 2);
                const int w = SW16 ? ((bir & 63) ^ (((r >> 3) & 1) << 5)) : (bir & 63);
                const int mn = (((bir >> 6) ^ (r & 3)) << 5) + (w >> 1);
                krow[i] = r;
                if constexpr (GLB) {
                    // rows_left is a multiple of 8 for an M/N-major 16-bit operand
                    const int64_t mc = mn < rows_left ? mn : rows_left - 8;
                    voff[i] = (uint32_t)(r * sk_bytes + mc * 2);
                } else {
                    voff[i] = mn < rows_left ? (uint32_t)(r * sk_bytes + mn * 2) : kOob;
                }
            }
        }
    }
    // The buffer resource (GLB: the 64-bit base in x, y) and K bound of one
    // stage's DMA.
    struct Stage {
        i32x4_t rsrc;
        int64_t k0;
        bool k_ok;
        uint32_t lds_base;
    };
    __device__ __forceinline__ Stage prep(uint8_t *dst, int kt) const {
        Stage st;
        if constexpr (GLB) {
            const int last = (int)(K / BKS) - 1;  // K >= BKS, a multiple of BKS
            st.k0 = (int64_t)(kt < last ? kt : last) * BKS;
            const uint64_t addr = (uint64_t)(base + st.k0 * sk_bytes);
            st.rsrc.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)addr);
            st.rsrc.y = __builtin_amdgcn_readfirstlane((int)(uint32_t)(addr >> 32));
            st.rsrc.z = st.rsrc.w = 0;
            st.k_ok = true;
            st.lds_base = (uint32_t)(uintptr_t)dst;
            return st;
        }
        st.k0 = (int64_t)kt * BKS;
        int64_t nb = nbytes - st.k0 * sk_bytes;
        nb = nb < 0 ? 0 : (nb > (int64_t)kMaxRec ? (int64_t)kMaxRec : nb);
        const uint64_t addr = (uint64_t)(base + st.k0 * sk_bytes);
        st.rsrc.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)addr);
        st.rsrc.y = __builtin_amdgcn_readfirstlane((int)(uint32_t)(addr >> 32) & 0xffff);
        st.rsrc.z = __builtin_amdgcn_readfirstlane((int)nb);
        st.rsrc.w = 0x00020000;
        st.k_ok = st.k0 + chunk * 8 < K;
        st.lds_base = (uint32_t)(uintptr_t)dst;
        return st;
    }
    // Instruction I (of kPer) of a prepared stage.
    template <int I>
    __device__ __forceinline__ void issue_one(const Stage &st, int wave) const {
        const int blk = wave + I * kWaves;
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(st.lds_base + blk * 1024);
        if constexpr (GLB) {
            const char *gb = (const char *)(((uint64_t)(uint32_t)st.rsrc.y << 32) | (uint32_t)st.rsrc.x);
            // M0 is written inside the asm by an SALU move, which the DMA may
            // read after one wait state (s_nop 0).  The base SGPRs come from
            // prep(), possibly through v_readfirstlane: a VMEM read of an SGPR
            // a VALU wrote needs 5 wait states, which the first instruction of
            // each prepared stage (I == 0, issued before the others) supplies
            // with s_nop 4; the later ones follow it.  The short pad took the
            // one-wave kernel's stage from 2554 to 2316 cycles.  The build
            // checks the emitted code for a VALU write of a DMA's base SGPRs
            // within 5 wait states (oxmera_amd/build.py).
            if constexpr (I == 0)
                asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff[I]), "s"(gb),
                             "s"(m0)
                             : "memory", "m0");
            else
                asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff[I]), "s"(gb),
                             "s"(m0)
                             : "memory", "m0");
            return;
        }
        bool ok;
        if constexpr (MN)
            ok = st.k0 + krow[I] < K;
        else
            ok = st.k_ok;
        const uint32_t vo = ok ? voff[I] : kOob;
        // The compiler cannot see that this asm is a VMEM instruction reading
        // the descriptor SGPRs and M0, so it inserts none of the wait states
        // that reading needs: 5 after a VALU write of an SGPR it reads (the
        // compiler forms the descriptor with v_readfirstlane when it keeps the
        // inputs in VGPRs, and reloads spilled SGPRs with v_readlane) and 1
        // after an SALU write of M0.  Without them the DMA can use a stale
        // descriptor or LDS address: stage data landed in the wrong rows when
        // an unrelated change moved v_readfirstlane next to the DMA.  s_nop 4
        // supplies the 5 cycles whatever precedes the asm.
        asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(vo), "s"(st.rsrc), "{m0}"(m0)
                     : "memory");
    }
    // Issue the DMA of K step kt (BKS k) into the stage at `dst`.  Inline asm
    // keeps the compiler from treating it as an LDS store it must drain before
    // every LDS read; the kernel orders it explicitly (vmcnt + s_barrier).
    __device__ __forceinline__ void issue(uint8_t *dst, int kt, int wave) {
        const Stage st = prep(dst, kt);
        static_for<0, kPer>([&](auto ic) { issue_one<decltype(ic)::value>(st, wave); });
    }
};

typedef short i16x4_t __attribute__((ext_vector_type(4)));

// MFMA fragments of one operand from a stage: TILES tiles of 32 rows
// starting at row0, fragment g = k 16g .. 16g+15 (g < BKS/16).  Lane l
// supplies row l % 32 and k 16g + 8 (l / 32) + 0..7, for A and B alike.
template <int ROWS, int TILES, bool MN, int BKS>
struct FragReader {
    static constexpr int kG = BKS / 16;
    static constexpr int kTileStride = BKS == 32 ? 2048 : 4096;  // K-major: bytes between tiles
    uint32_t off[kG];           // K-major: per g
    uint32_t rowpart[kG][2];    // M/N-major: per (g, t)
    uint32_t seg[TILES];        // M/N-major: per tile

    __device__ __forceinline__ FragReader(uint32_t region, int row0, int lane) {
        if constexpr (!MN) {
            const int half = lane >> 5;
            const int r = row0 + (lane & 31);
#pragma unroll
            for (int g = 0; g < kG; ++g)
                off[g] = region + (BKS == 32 ? lds_off64(r, 2 * g + half) : lds_off(r, 2 * g + half));
        } else {
            // ds_read_b64_tr_b16: in each 16-lane group, output lane 4a + b gets
            // element b of the 8-byte blocks addressed by lanes a, a+4, a+8, a+12.
            // Lane a + 4j addresses k-row k0 + j at columns mnb + 4a .. +3, so
            // lane i of the group receives k0 .. k0+3 of column mnb + i.
            const int grp = lane >> 4, h = grp >> 1, mnb = (grp & 1) * 16;
            const int a = lane & 3, j = (lane >> 2) & 3;
#pragma unroll
            for (int g = 0; g < kG; ++g)
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    rowpart[g][t] = region + (16 * g + 8 * h + 4 * t + j) * ROWS * 2 + (mnb + 4 * a) * 2;
#pragma unroll
            for (int i = 0; i < TILES; ++i) seg[i] = (uint32_t)((((row0 >> 5) + i) ^ j) << 6);
        }
    }
    // Fragment of tile I of group g (one ds_read_b128, or two transposing
    // reads for an M/N-major operand).
    template <int I>
    __device__ __forceinline__ uint4 read1(const uint8_t *stage, int g) const {
        if constexpr (!MN) {
            return *(const uint4 *)(stage + off[g] + I * kTileStride);
        } else {
            typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
            const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_i16x4 *)(uintptr_t)(uint32_t)(uintptr_t)(stage + rowpart[g][0] + seg[I]));
            const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_i16x4 *)(uintptr_t)(uint32_t)(uintptr_t)(stage + rowpart[g][1] + seg[I]));
            const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
            return make_uint4(l2.x, l2.y, h2.x, h2.y);
        }
    }
    __device__ __forceinline__ void read(const uint8_t *stage, int g, uint4 (&out)[TILES]) const {
#pragma unroll
        for (int i = 0; i < TILES; ++i) {
            if constexpr (!MN) {
                out[i] = *(const uint4 *)(stage + off[g] + i * kTileStride);
            } else {
                typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
                const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_i16x4 *)(uintptr_t)(uint32_t)(uintptr_t)(stage + rowpart[g][0] + seg[i]));
                const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_i16x4 *)(uintptr_t)(uint32_t)(uintptr_t)(stage + rowpart[g][1] + seg[i]));
                const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
                out[i] = make_uint4(l2.x, l2.y, h2.x, h2.y);
            }
        }
    }
};

// Where workgroup `blk` works: tiles are spread across the 8 XCDs
// (consecutive workgroups land on different XCDs, so each XCD gets a
// contiguous run of tiles) and ordered in groups of group_m tile-rows, so an
// XCD's L2 holds a compact block of A and B panels.
struct TileCoord {
    int64_t bidx, m0, n0, offa, offb;
};

template <int BM, int BN>
__device__ __forceinline__ TileCoord tile_coord(const GemmArgs &p, int64_t wg) {
    const int64_t per_batch = (int64_t)p.tiles_m * p.tiles_n;
    const int64_t ntiles = per_batch * p.batch;
    if (p.xcd_remap && (ntiles & 7) == 0) wg = (wg & 7) * (ntiles >> 3) + (wg >> 3);
    TileCoord tc;
    tc.bidx = wg / per_batch;
    const int64_t t = wg - tc.bidx * per_batch;
    const int64_t gsz = (int64_t)p.group_m * p.tiles_n;
    const int64_t grp = t / gsz;
    const int64_t first_m = grp * p.group_m;
    const int64_t gm = (p.tiles_m - first_m) < p.group_m ? (p.tiles_m - first_m) : p.group_m;
    const int64_t tin = t - grp * gsz;
    tc.m0 = (first_m + tin % gm) * BM;
    tc.n0 = (tin / gm) * BN;
    tc.offa = tc.offb = 0;
    if (p.nbd > 0) {
        int64_t rem = tc.bidx;
        for (int d = p.nbd - 1; d >= 0; --d) {
            const int64_t i = rem % p.bext[d];
            rem /= p.bext[d];
            tc.offa += i * p.bsa[d];
            tc.offb += i * p.bsb[d];
        }
    }
    return tc;
}

// Direct-to-LDS GEMM for 16-bit operands that are K- or M/N-contiguous
// (AMN / BMN: the operand is M/N-major).  NS stages of BKS k form a ring;
// NS-1 stages are in flight while one is consumed; one barrier per stage.
// After the barrier the stage's DMA instructions are interleaved with the
// deferred MFMAs (one or more after each) rather than issued as a burst, so
// the MFMA pipe keeps running while the DMA is issued (at 8192^3 this
// measured between even and 4 % faster than a burst, depending on the GPU).
template <typename T, int BM, int BN, int WAVES_M, int WAVES_N, int NS, int BKS, bool AMN, bool BMN,
          bool GLB = false>
__global__ void __launch_bounds__(WAVES_M *WAVES_N * 64) gemm_kernel_dl(GemmArgs p) {
    constexpr int NT = WAVES_M * WAVES_N * 64;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int kStageA = BM * BKS * 2, kStageB = BN * BKS * 2;
    constexpr int kStage = kStageA + kStageB;
    constexpr int kG = BKS / 16;
    constexpr int kQ = TM * TN;                                       // MFMAs per fragment group
    constexpr int kReads = TM * (AMN ? 2 : 1) + TN * (BMN ? 2 : 1);  // LDS reads per fragment group
    constexpr int kPer = (kReads + kQ / 2 - 1) / (kQ / 2);            // reads after each early MFMA
    static_assert(Elem<T>::kBytes == 2, "direct-to-LDS path is for 16-bit operands");
    static_assert(NS >= 2, "at least two stages");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * kStage];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const TileCoord tc = tile_coord<BM, BN>(p, blockIdx.x);
    const int64_t m0 = tc.m0, n0 = tc.n0;
    // The stage's DMA is issued by waves 0-3 only, one per SIMD, so that under
    // memory backpressure (a DMA instruction waits to issue) every SIMD keeps
    // a wave that issues MFMAs: 8192^3 NT 0.827 -> 0.817 ms, the MLP step
    // 5.94 -> 5.80 ms (spreading all 8 waves' DMA over two fragment groups
    // instead measured the same).
    constexpr int DW = NT / 64 < 4 ? NT / 64 : 4;
    const bool dma_wave = wave < DW;
    using LA = DirectLoader<BM, DW * 64, AMN, BKS, GLB>;
    using LB = DirectLoader<BN, DW * 64, BMN, BKS, GLB>;
    LA la((const char *)p.a + (tc.offa + m0 * p.sam) * 2, p.sam, p.sak, p.M - m0, p.K, wave, lane);
    LB lb((const char *)p.b + (tc.offb + n0 * p.sbn) * 2, p.sbn, p.sbk, p.N - n0, p.K, wave, lane);
    constexpr int kLoadsPerStage = LA::kPer + LB::kPer;
    const FragReader<BM, TM, AMN, BKS> fra(0, wm * WM, lane);
    const FragReader<BN, TN, BMN, BKS> frb(kStageA, wn * WN, lane);

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};
    uint4 fa[2][TM], fb[2][TN];

    const int nk = (int)((p.K + BKS - 1) / BKS);
    // Software pipeline.  Step kt computes stage kt % NS while NS-1 later
    // stages are in flight.  The MFMAs of the last fragment group of step kt
    // use registers only, so they are issued AFTER the barrier, under the LDS
    // latency of step kt+1's first fragment reads; before the barrier every
    // LDS read of step kt has landed (lgkmcnt 0), which is what lets the DMA
    // of step kt+NS overwrite stage kt % NS right after it.
    if (dma_wave) {
#pragma unroll
        for (int s = 0; s < NS - 1; ++s) {
            la.issue(lds + s * kStage, s, wave);
            lb.issue(lds + s * kStage + kStageA, s, wave);
        }
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm((NS - 2) * kLoadsPerStage));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (dma_wave) {
        la.issue(lds + (NS - 1) * kStage, NS - 1, wave);
        lb.issue(lds + (NS - 1) * kStage + kStageA, NS - 1, wave);
    }
    fra.read(lds, 0, fa[0]);
    frb.read(lds, 0, fb[0]);
    int cur = 0;  // stage of step kt
    for (int kt = 0; kt < nk; ++kt) {
        uint8_t *stage = lds + cur * kStage;
        // Buffer resources of step kt+NS's DMA (into this stage once it is
        // consumed), computed here so the scalar work overlaps the MFMAs.
        const int knext = kt + NS;
        const typename LA::Stage sta = la.prep(stage, knext);
        const typename LB::Stage stb = lb.prep(stage + kStageA, knext);
        static_for<0, kG - 1>([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            fra.read(stage, g + 1, fa[(g + 1) & 1]);
            frb.read(stage, g + 1, fb[(g + 1) & 1]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) Mma<T>::run(acc[i][j], fa[g & 1][i], fb[g & 1][j]);
            // Group g+1's fragment reads go out over the first half of group
            // g's MFMAs, kPer after each, so at least half the group covers
            // their latency (left alone, the compiler issues them after
            // group g's next-to-last MFMA and waits one MFMA later)
            static_for<0, kQ>([&](auto qc) {
                constexpr int q = decltype(qc)::value;
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                constexpr int left = kReads - q * kPer;
                constexpr int nr = q < kQ / 2 ? (left < kPer ? (left > 0 ? left : 0) : kPer) : 0;
                if constexpr (nr > 0) __builtin_amdgcn_sched_group_barrier(0x100, nr, 0);  // LDS reads
            });
            __builtin_amdgcn_sched_barrier(0);
        });
        // every LDS read of step kt landed; this wave's DMA of step kt+1 landed
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm((NS - 2) * kLoadsPerStage) & ~(0xF << 8));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        constexpr int gl = (kG - 1) & 1;
        cur = cur + 1 == NS ? 0 : cur + 1;
        const uint8_t *next = lds + cur * kStage;
        fra.read(next, 0, fa[0]);
        frb.read(next, 0, fb[0]);
        __builtin_amdgcn_sched_barrier(0);
        // MFMA q of the deferred group, then (DMA waves) DMA instructions
        // [q*L/Q, (q+1)*L/Q) of the stage (L loads, Q MFMAs).
        constexpr int Q = TM * TN, L = kLoadsPerStage;
        static_for<0, Q>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            Mma<T>::run(acc[q / TN][q % TN], fa[gl][q / TN], fb[gl][q % TN]);
            if (dma_wave) {
                static_for<q * L / Q, (q + 1) * L / Q>([&](auto lc) {
                    constexpr int l = decltype(lc)::value;
                    if constexpr (l < LA::kPer)
                        la.template issue_one<l>(sta, wave);
                    else
                        lb.template issue_one<l - LA::kPer>(stb, wave);
                });
            }
            __builtin_amdgcn_sched_barrier(0);
        });
        __builtin_amdgcn_sched_barrier(0);
    }
    // DMA past the end of K was issued (out of range: it writes zeros to
    // LDS); drain it before the LDS is reused for the epilogue.
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();
    epilogue_lds<NT, WM, WN, TM, TN, NS * kStage>(p, acc, lds, wave, lane, tc.bidx * p.M * p.N, m0 + wm * WM,
                                                  n0 + wn * WN);
}

// Direct-to-LDS GEMM with one wave per SIMD: 4 waves (2 x 2) of 128 x 128,
// two stages of BKS = 64 k.  A 128 x 128 wave tile reads a third less from
// LDS per flop than 128 x 64 (the LDS serves both the DMA writes and the
// fragment reads, and its occupancy is what idles the MFMA pipe), but a lone
// wave must keep its own MFMA pipe fed, so its instruction stream is placed
// by hand: a stage is four groups of 16 MFMAs (one per 32 x 32 block), and
// every MFMA slot carries at most one other instruction -- a fragment read
// for the next group (slots 0-7, in the order the next group's MFMAs consume
// them) or a DMA instruction of the next stage (slots 8-15 of the first two
// groups after the barrier).  The last group of each stage is deferred past
// the barrier so the MFMA pipe works while the next stage's first fragments
// are read.
template <typename T, int BM, int BN, int BKS, bool AMN, bool BMN, int DF = 8, int DS = 2>
__global__ void __launch_bounds__(256) gemm_kernel_dli(GemmArgs p) {
    constexpr int NT = 256, WAVES_N = 2;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int kStageA = BM * BKS * 2, kStageB = BN * BKS * 2;
    constexpr int kStage = kStageA + kStageB;
    constexpr int kG = BKS / 16;
    static_assert(Elem<T>::kBytes == 2, "direct-to-LDS path is for 16-bit operands");
    static_assert(kG == 4, "four fragment groups per stage");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * kStage];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const TileCoord tc = tile_coord<BM, BN>(p, blockIdx.x);
    const int64_t m0 = tc.m0, n0 = tc.n0;
    using LA = DirectLoader<BM, NT, AMN, BKS>;
    using LB = DirectLoader<BN, NT, BMN, BKS>;
    LA la((const char *)p.a + (tc.offa + m0 * p.sam) * 2, p.sam, p.sak, p.M - m0, p.K, wave, lane);
    LB lb((const char *)p.b + (tc.offb + n0 * p.sbn) * 2, p.sbn, p.sbk, p.N - n0, p.K, wave, lane);
    constexpr int L = LA::kPer + LB::kPer;  // DMA instructions per wave per stage
    constexpr int Q = TM * TN;              // MFMA slots per group
    constexpr int R = TM + TN;              // fragment reads per group
    static_assert(R <= Q && DF + (L - 1) * DS < kG * Q, "DMA must fit the slots of one iteration");
    const FragReader<BM, TM, AMN, BKS> fra(0, wm * WM, lane);
    const FragReader<BN, TN, BMN, BKS> frb(kStageA, wn * WN, lane);

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};
    uint4 fa[2][TM], fb[2][TN];

    // One group (GI-th of an iteration; GI < 0: no DMA): the MFMAs of register
    // set USE (MF = false: none); slot s < R also reads fragment s of group GN
    // (GN < 0: none) of stage `rs` into set USE ^ 1 (A0, B0 .. B(TN-1), A1 ..
    // A(TM-1): the order the next group consumes them); DMA instruction l of
    // the next stage goes into iteration slot DF + l * DS.
    auto group = [&](auto usec, auto mfc, auto gnc, auto gic, const uint8_t *rs, const typename LA::Stage &sta,
                     const typename LB::Stage &stb) {
        constexpr int USE = decltype(usec)::value, GN = decltype(gnc)::value, GI = decltype(gic)::value;
        constexpr bool MF = decltype(mfc)::value;
        static_for<0, Q>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            if constexpr (MF) Mma<T>::run(acc[q / TN][q % TN], fa[USE][q / TN], fb[USE][q % TN]);
            if constexpr (GN >= 0 && q < R) {
                if constexpr (q == 0)
                    fa[USE ^ 1][0] = fra.template read1<0>(rs, GN);
                else if constexpr (q <= TN)
                    fb[USE ^ 1][q - 1] = frb.template read1<(q > 0 && q <= TN ? q - 1 : 0)>(rs, GN);
                else
                    fa[USE ^ 1][q - TN] = fra.template read1<(q > TN ? q - TN : 0)>(rs, GN);
            }
            constexpr int sg = GI * Q + q;
            if constexpr (GI >= 0 && sg >= DF && (sg - DF) % DS == 0 && (sg - DF) / DS < L) {
                constexpr int l = (sg - DF) / DS;
                if constexpr (l < LA::kPer)
                    la.template issue_one<(l < LA::kPer ? l : 0)>(sta, wave);
                else
                    lb.template issue_one<(l >= LA::kPer ? l - LA::kPer : 0)>(stb, wave);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using INone = std::integral_constant<int, -1>;
    using YES = std::integral_constant<bool, true>;
    using NO = std::integral_constant<bool, false>;
    // every LDS read of this wave landed; its DMA into the next stage landed;
    // then all waves
    auto stage_barrier = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0) & ~(0xF << 8));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };

    const int nk = (int)((p.K + BKS - 1) / BKS);
    // Prologue: DMA of steps 0 and 1, wait for step 0, its group-0 fragments.
    la.issue(lds, 0, wave);
    lb.issue(lds + kStageA, 0, wave);
    la.issue(lds + kStage, 1, wave);
    lb.issue(lds + kStage + kStageA, 1, wave);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(L));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    {
        const typename LA::Stage sta = la.prep(lds, 0);
        const typename LB::Stage stb = lb.prep(lds + kStageA, 0);
        // group-0 fragment reads of step 0, no MFMAs yet
        group(I1{}, NO{}, I0{}, INone{}, lds, sta, stb);
        group(I0{}, YES{}, I1{}, INone{}, lds, sta, stb);
        group(I1{}, YES{}, I2{}, INone{}, lds, sta, stb);
        group(I0{}, YES{}, I3{}, INone{}, lds, sta, stb);
    }
    for (int kt = 1; kt < nk; ++kt) {
        stage_barrier();
        const uint8_t *stage = lds + (kt & 1) * kStage;
        uint8_t *other = lds + ((kt & 1) ^ 1) * kStage;
        // DMA of step kt+1 into the stage step kt-1 used (past K: zeros)
        const typename LA::Stage sta = la.prep(other, kt + 1);
        const typename LB::Stage stb = lb.prep(other + kStageA, kt + 1);
        group(I1{}, YES{}, I0{}, I0{}, stage, sta, stb);  // group 3 of step kt-1
        group(I0{}, YES{}, I1{}, I1{}, stage, sta, stb);  // groups 0-2 of step kt
        group(I1{}, YES{}, I2{}, I2{}, stage, sta, stb);
        group(I0{}, YES{}, I3{}, I3{}, stage, sta, stb);
    }
    {
        const typename LA::Stage sta = la.prep(lds, 0);
        const typename LB::Stage stb = lb.prep(lds + kStageA, 0);
        group(I1{}, YES{}, INone{}, INone{}, lds, sta, stb);  // group 3 of the last step
    }
    // drain every DMA (the last steps' are out of range) before the LDS is reused
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();
    epilogue_lds<NT, WM, WN, TM, TN, 2 * kStage>(p, acc, lds, wave, lane, tc.bidx * p.M * p.N, m0 + wm * WM,
                                                 n0 + wn * WN);
}

// ---- one wave per SIMD on 16x16x32 MFMAs ------------------------------------

// bf16 / f16 on v_mfma_f32_16x16x32_{bf16,f16}: a 16-byte fragment holds the
// 8 k values one lane contributes (lane l: row l % 16, k 8 (l / 16) .. +7 of
// the 32), identically for A and B; the 4 accumulators of lane l are column
// l % 16 of rows 4 (l / 16) .. +3.
template <typename T>
struct Mma16;
template <>
struct Mma16<bf16_t> {
    __device__ __forceinline__ static void run(f32x4_t &acc, const uint4 &a, const uint4 &b) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                      acc, 0, 0, 0);
    }
};
template <>
struct Mma16<f16_t> {
    __device__ __forceinline__ static void run(f32x4_t &acc, const uint4 &a, const uint4 &b) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                     acc, 0, 0, 0);
    }
};

// 16x16x32 fragments of a K-major operand from a BKS = 64 stage (lds_off
// layout): tile I is rows row0 + 16 I .. +15, group g is k 32 g .. +31; lane l
// reads row l % 16 at 16-byte chunk 4 g + l / 16.  Sixteen rows of one chunk
// fall in sixteen distinct bank groups, and rows r and r + 16 differ by 8 row
// pairs (2048 bytes) with the same swizzle.
struct FragReader16 {
    uint32_t off[2];
    __device__ __forceinline__ FragReader16(uint32_t region, int row0, int lane) {
        const int r = row0 + (lane & 15);
#pragma unroll
        for (int g = 0; g < 2; ++g) off[g] = region + lds_off(r, 4 * g + (lane >> 4));
    }
    template <int I>
    __device__ __forceinline__ uint4 read1(const uint8_t *stage, int g) const {
        return *(const uint4 *)(stage + off[g] + I * 2048);
    }
};

// 16x16x32 fragments of an M/N-major 16-bit operand from a BKS = 64 stage of
// a 256-row tile (DirectLoader SW16 layout: 512-byte k-rows, 64-byte segment
// s of k-row r stored at s ^ (r % 4), its 32-byte halves exchanged when bit
// 3 of r is set).  Tile I is mn0 + 16 I .. +15, group g is k 32 g .. +31;
// lane l supplies column mn0 + 16 I + l % 16 at k 32 g + 8 (l / 16) .. +7,
// as FragReader16 does for a K-major operand, from two ds_read_b64_tr_b16
// (in a 16-lane group, lane a + 4 j addresses k-row k0 + j at columns
// 4 a .. 4 a + 3 of the 16, and lane i receives k0 .. k0 + 3 of column i).
// A half-wave's accesses (8 k-rows: k0 + j and k0 + 8 + j, 32 bytes each)
// fall in distinct banks.
struct FragReader16MN {
    uint32_t rb[2][2];  // per (g, t): k-row 32 g + 8 (l / 16) + 4 t + j, plus 8 a
    uint32_t x[8];      // per tile: the segment and half swizzle
    __device__ __forceinline__ FragReader16MN(uint32_t region, int mn0, int lane) {
        const int q = lane >> 4, i = lane & 15, a = i & 3, j = i >> 2;
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int t = 0; t < 2; ++t) rb[g][t] = region + (32 * g + 8 * q + 4 * t + j) * 512 + 8 * a;
#pragma unroll
        for (int I = 0; I < 8; ++I) {
            const int c = (mn0 >> 4) + I;  // 32-byte column chunk of tile I
            x[I] = (uint32_t)((((c >> 1) ^ j) << 6) | (((c & 1) ^ (q & 1)) << 5));
        }
    }
    template <int I>
    __device__ __forceinline__ uint4 read1(const uint8_t *stage, int g) const {
        typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4 *)(uintptr_t)(uint32_t)(uintptr_t)(stage + rb[g][0] + x[I]));
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4 *)(uintptr_t)(uint32_t)(uintptr_t)(stage + rb[g][1] + x[I]));
        const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
        return make_uint4(l2.x, l2.y, h2.x, h2.y);
    }
};

// 256x256 tile, 2x2 waves of 128x128, one wave per SIMD, 16-bit operands
// (each K- or, AMN / BMN, M/N-major), 16x16x32 MFMAs (OXM_GEMM_CFG=7).  Against the 32x32x16 kernels a
// 16x16x32 MFMA is half as long, so each fragment read and DMA instruction
// of the hand-placed stream has twice as many MFMA slots to hide in: a
// 64-k stage is two groups of 64 MFMA slots (8 x 8 blocks); slot 2r of a
// group reads fragment r of the next group (A0, B0 .. B7, A1 .. A7, the order
// its MFMAs consume them) and the stage's 16 DMA instructions take every
// fourth slot from slot 8 of the step (placements swept: DMA offset 0 / 8 /
// 16 / 24 / 40 / 64 slots, spacing 2 / 3 / 4 / 6 / 7 / 8, fragment-read
// spacing 1 / 2 / 3, per-wave DMA offsets; this one measured best).  The
// second group of each stage is deferred past the barrier.  The MFMA sums
// equal those of the 32x32x16 kernels bit for bit on the shapes tested.
template <typename T, bool GLB = false, int DF = 8, int DS = 4, int RS = 2, bool AMN = false, bool BMN = false>
__global__ void __launch_bounds__(256) gemm_kernel_dli16(GemmArgs p) {
    constexpr int BM = 256, BN = 256, BKS = 64, NT = 256, WAVES_N = 2;
    constexpr int WM = 128, WN = 128, TM = 8, TN = 8;  // 16x16 blocks per wave
    constexpr int kStageA = BM * BKS * 2, kStageB = BN * BKS * 2;
    constexpr int kStage = kStageA + kStageB;
    static_assert(Elem<T>::kBytes == 2, "direct-to-LDS path is for 16-bit operands");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * kStage];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const TileCoord tc = tile_coord<BM, BN>(p, blockIdx.x);
    const int64_t m0 = tc.m0, n0 = tc.n0;
    using LA = DirectLoader<BM, NT, AMN, BKS, GLB, AMN>;
    using LB = DirectLoader<BN, NT, BMN, BKS, GLB, BMN>;
    LA la((const char *)p.a + (tc.offa + m0 * p.sam) * 2, p.sam, p.sak, p.M - m0, p.K, wave, lane);
    LB lb((const char *)p.b + (tc.offb + n0 * p.sbn) * 2, p.sbn, p.sbk, p.N - n0, p.K, wave, lane);
    constexpr int L = LA::kPer + LB::kPer;  // DMA instructions per wave per stage
    constexpr int Q = TM * TN;              // MFMA slots per group
    constexpr int R = TM + TN;              // fragment reads per group (two instructions when M/N-major)
    static_assert(DF + (L - 1) * DS < 2 * Q, "DMA must fit the slots of one stage");
    static_assert((R - 1) * RS < Q, "fragment reads must fit the slots of one group");
    using FA = typename std::conditional<AMN, FragReader16MN, FragReader16>::type;
    using FB = typename std::conditional<BMN, FragReader16MN, FragReader16>::type;
    const FA fra(0, wm * WM, lane);
    const FB frb(kStageA, wn * WN, lane);

    f32x4_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{};
    uint4 fa[2][TM], fb[2][TN];

    // One group (GI-th of a stage; GI < 0: no DMA): the MFMAs of register set
    // USE (MF = false: none); fragment reads of group GN (GN < 0: none) of
    // stage `rs` into set USE ^ 1; DMA instruction l of the next stage in
    // stage slot DF + l * DS.
    auto group = [&](auto usec, auto mfc, auto gnc, auto gic, const uint8_t *rs, const typename LA::Stage &sta,
                     const typename LB::Stage &stb) {
        constexpr int USE = decltype(usec)::value, GN = decltype(gnc)::value, GI = decltype(gic)::value;
        constexpr bool MF = decltype(mfc)::value;
        static_for<0, Q>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            if constexpr (MF) Mma16<T>::run(acc[q / TN][q % TN], fa[USE][q / TN], fb[USE][q % TN]);
            if constexpr (GN >= 0 && q % RS == 0 && q / RS < R) {
                constexpr int r = q / RS;
                if constexpr (r == 0)
                    fa[USE ^ 1][0] = fra.template read1<0>(rs, GN);
                else if constexpr (r <= TN)
                    fb[USE ^ 1][r - 1] = frb.template read1<(r >= 1 && r <= TN ? r - 1 : 0)>(rs, GN);
                else
                    fa[USE ^ 1][r - TN] = fra.template read1<(r > TN ? r - TN : 0)>(rs, GN);
            }
            constexpr int sg = GI * Q + q;
            if constexpr (GI >= 0 && sg >= DF && (sg - DF) % DS == 0 && (sg - DF) / DS < L) {
                constexpr int l = (sg - DF) / DS;
                if constexpr (l < LA::kPer)
                    la.template issue_one<(l < LA::kPer ? l : 0)>(sta, wave);
                else
                    lb.template issue_one<(l >= LA::kPer ? l - LA::kPer : 0)>(stb, wave);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using INone = std::integral_constant<int, -1>;
    using YES = std::integral_constant<bool, true>;
    using NO = std::integral_constant<bool, false>;
    // every LDS read of this wave landed; its DMA into the next stage landed;
    // then all waves
    auto stage_barrier = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0) & ~(0xF << 8));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };

    const int nk = (int)((p.K + BKS - 1) / BKS);
    // Prologue: DMA of steps 0 and 1, wait for step 0, its group-0 fragments.
    la.issue(lds, 0, wave);
    lb.issue(lds + kStageA, 0, wave);
    la.issue(lds + kStage, 1, wave);
    lb.issue(lds + kStage + kStageA, 1, wave);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(L));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    {
        const typename LA::Stage sta = la.prep(lds, 0);
        const typename LB::Stage stb = lb.prep(lds + kStageA, 0);
        group(I1{}, NO{}, I0{}, INone{}, lds, sta, stb);
        group(I0{}, YES{}, I1{}, INone{}, lds, sta, stb);
    }
    for (int kt = 1; kt < nk; ++kt) {
        stage_barrier();
        const uint8_t *stage = lds + (kt & 1) * kStage;
        uint8_t *other = lds + ((kt & 1) ^ 1) * kStage;
        // DMA of step kt+1 into the stage step kt-1 used (past K: zeros)
        const typename LA::Stage sta = la.prep(other, kt + 1);
        const typename LB::Stage stb = lb.prep(other + kStageA, kt + 1);
        group(I1{}, YES{}, I0{}, I0{}, stage, sta, stb);  // group 1 of step kt-1
        group(I0{}, YES{}, I1{}, I1{}, stage, sta, stb);  // group 0 of step kt
    }
    {
        const typename LA::Stage sta = la.prep(lds, 0);
        const typename LB::Stage stb = lb.prep(lds + kStageA, 0);
        group(I1{}, YES{}, INone{}, INone{}, lds, sta, stb);  // group 1 of the last step
    }
    // drain every DMA (the last steps' are out of range) before the LDS is reused
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();
    epilogue_lds<NT, WM, WN, TM, TN, 2 * kStage>(p, acc, lds, wave, lane, tc.bidx * p.M * p.N, m0 + wm * WM,
                                                 n0 + wn * WN);
}

// ---- f32 direct-to-LDS (256x256 tiles) -----------------------------------------
//
// The register-staged f32 kernel moves every operand byte through VGPRs
// (global loads, a 4x4 transpose for an M/N-major operand, ds_write_b128).
// Here both operands go global -> LDS by DMA, as in the 16-bit kernels:
// 4096^3 row-major x row-major 0.987 -> 0.924 ms (88.5 -> 94.6 % of the f32
// MFMA peak), bit-identical.  A 32-k stage of a 256-row operand is 32 KB in
// either orientation.

// K-major f32 operand: a 32-k row is 128 bytes, the same bytes as a 64-k row
// of a 16-bit operand, so DirectLoader / FragReader serve it unchanged with
// strides and K counted in 16-bit units.  The fragments then hold 4 f32 k
// values per lane, k = 8 g + 4 (lane / 32) + s, as Mma<float> takes them.
template <int ROWS, bool GLB>
struct F32LoaderK : DirectLoader<ROWS, 256, false, 64, GLB> {
    using Base = DirectLoader<ROWS, 256, false, 64, GLB>;
    static constexpr int kStageBytes = ROWS * 128;
    __device__ __forceinline__ F32LoaderK(const char *b, int64_t s_mn, int64_t rows_left, int64_t k, int wave,
                                          int lane)
        : Base(b, 2 * s_mn, 1, rows_left, 2 * k, wave, lane) {}
};

// M/N-major f32 operand (ROWS = 256, 192, 128 or 64 values along M or N
// contiguous per k): a k-row of the tile takes 4 ROWS bytes of the stage
// (1 KB, 192 of them used, for ROWS = 192), a 1 KB DMA block
// holds 1024 / kRowBytes of them; the k-rows whose bit 2 is set are stored
// rotated by 128 bytes, so a fragment read (lanes 0-31 at k-row k, lanes
// 32-63 at k + 4, 32 consecutive values each) touches 64 distinct banks.
// Lane L of block b fills k-row b * kRowsPerBlock + L / kLanesPerRow with
// the 16 bytes of column chunk (L mod kLanesPerRow - rot) mod kLanesPerRow
// (ROWS = 192: the chunks from 48 on are not used).  Chunks past the tile's
// or the operand's M/N edge: kOob (buffer form, reads zeros) or the last
// valid chunk (GLB: those columns feed only outputs that are never stored,
// or no output); past K: kOob, or (GLB, K a multiple of 32) the last step
// again into a stage nobody reads.
template <int ROWS, bool GLB>
struct F32LoaderMN {
    static_assert(ROWS == 256 || ROWS == 192 || ROWS == 128 || ROWS == 64, "256-, 192-, 128- or 64-wide tiles");
    static constexpr int kWaves = 4;
    static constexpr int kRowBytes = ROWS == 64 ? 256 : (ROWS == 128 ? 512 : 1024), kRowsPerBlock = 1024 / kRowBytes,
                         kLanesPerRow = kRowBytes / 16;
    static constexpr int kStageBytes = 32 * kRowBytes;
    static constexpr int kPer = 32 / kRowsPerBlock / kWaves;  // DMA instructions per wave per stage
    const char *base;
    int64_t K, sk_bytes, nbytes, cols_left;
    int lane;
    struct Stage {
        i32x4_t rsrc;
        int64_t k0;
        uint32_t lds_base;
    };
    __device__ __forceinline__ F32LoaderMN(const char *b, int64_t s_k, int64_t cols, int64_t k, int /*wave*/,
                                           int ln)
        : base(b), K(k), sk_bytes(s_k * 4), cols_left(cols), lane(ln) {
        const int64_t cols_here = cols < ROWS ? cols : ROWS;
        nbytes = (k - 1) * sk_bytes + cols_here * 4;
    }
    __device__ __forceinline__ Stage prep(uint8_t *dst, int kt) const {
        Stage st;
        if constexpr (GLB) {
            const int last = (int)(K / 32) - 1;  // K >= 32, a multiple of 32
            st.k0 = (int64_t)(kt < last ? kt : last) * 32;
            const uint64_t addr = (uint64_t)(base + st.k0 * sk_bytes);
            st.rsrc.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)addr);
            st.rsrc.y = __builtin_amdgcn_readfirstlane((int)(uint32_t)(addr >> 32));
            st.rsrc.z = st.rsrc.w = 0;
        } else {
            st.k0 = (int64_t)kt * 32;
            int64_t nb = nbytes - st.k0 * sk_bytes;
            nb = nb < 0 ? 0 : (nb > (int64_t)kMaxRec ? (int64_t)kMaxRec : nb);
            const uint64_t addr = (uint64_t)(base + st.k0 * sk_bytes);
            st.rsrc.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)addr);
            st.rsrc.y = __builtin_amdgcn_readfirstlane((int)(uint32_t)(addr >> 32) & 0xffff);
            st.rsrc.z = __builtin_amdgcn_readfirstlane((int)nb);
            st.rsrc.w = 0x00020000;
        }
        st.lds_base = (uint32_t)(uintptr_t)dst;
        return st;
    }
    template <int I>
    __device__ __forceinline__ void issue_one(const Stage &st, int wave) const {
        const int blk = wave + I * kWaves;
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(st.lds_base + blk * 1024);
        const int kr = blk * kRowsPerBlock + lane / kLanesPerRow;
        const int c = ((lane % kLanesPerRow) - ((kr >> 2) & 1) * 8) & (kLanesPerRow - 1);
        int64_t col = 4 * c;
        // the columns this tile reads: a multiple of 4 (M/N a multiple of 4)
        const int64_t lim = cols_left < ROWS ? cols_left : ROWS;
        if constexpr (GLB) {
            if (col >= lim) col = lim - 4;
            const uint32_t vo = (uint32_t)(kr * sk_bytes + col * 4);
            const char *gb = (const char *)(((uint64_t)(uint32_t)st.rsrc.y << 32) | (uint32_t)st.rsrc.x);
            // pads as in DirectLoader: the first DMA of a prepared stage waits
            // out a VALU write of the base SGPRs, the later ones only M0's
            if constexpr (I == 0)
                asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(vo), "s"(gb),
                             "s"(m0)
                             : "memory", "m0");
            else
                asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(vo), "s"(gb),
                             "s"(m0)
                             : "memory", "m0");
        } else {
            const uint32_t vo =
                (col < lim && st.k0 + kr < K) ? (uint32_t)(kr * sk_bytes + col * 4) : kOob;
            asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(vo), "s"(st.rsrc), "{m0}"(m0)
                         : "memory");
        }
    }
    __device__ __forceinline__ void issue(uint8_t *dst, int kt, int wave) {
        const Stage st = prep(dst, kt);
        static_for<0, kPer>([&](auto ic) { issue_one<decltype(ic)::value>(st, wave); });
    }
};

// Fragments of an M/N-major f32 operand from the rotated stage: TILES tiles
// of 32 values starting at mn0; lane l supplies mn0 + 32 I + l % 32 at
// k = 8 g + 4 (l / 32) + s (s = 0..3), four ds_read_b32 per fragment.
template <int TILES, int ROWS>
struct F32FragMN {
    static constexpr int kRowBytes = ROWS == 64 ? 256 : (ROWS == 128 ? 512 : 1024);
    uint32_t region;
    int mn0, lane;
    __device__ __forceinline__ F32FragMN(uint32_t r, int m, int l) : region(r), mn0(m), lane(l) {}
    __device__ __forceinline__ void read(const uint8_t *stage, int g, uint4 (&out)[TILES]) const {
#pragma unroll
        for (int i = 0; i < TILES; ++i) {
            const int c = mn0 + 32 * i + (lane & 31);
            uint32_t v[4];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int k = 8 * g + 4 * (lane >> 5) + s;
                v[s] = *(const uint32_t *)(stage + region + k * kRowBytes +
                                           ((c * 4 + ((k >> 2) & 1) * 128) & (kRowBytes - 1)));
            }
            out[i] = make_uint4(v[0], v[1], v[2], v[3]);
        }
    }
};

// BM x BN tile (256x256 with 2x4 waves of 128x64; 256x192 with 4x3 waves of
// 64x64; 128x128 with 2x2 waves of 64x64, two blocks per CU; 64x64 with 2x2
// waves of 32x32), a ring of NS stages of 32 k (NS - 1 in flight while one
// is consumed: 2 for the large tiles; 8 for 64x64 tiles, whose problems are
// small enough that the latency of each step, not the MFMAs, sets the
// time), the DMA issued by waves 0-3; the same pipeline as gemm_kernel_dl.
template <int BM, int BN, int WAVES_M, int WAVES_N, bool AMN, bool BMN, bool GLB, int NS = 2>
__global__ void __launch_bounds__(WAVES_M *WAVES_N * 64) gemm_kernel_dlf32(GemmArgs p) {
    constexpr int NT = WAVES_M * WAVES_N * 64;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N, TM = WM / 32, TN = WN / 32, kG = 4;
    static_assert(NT / 64 >= 4 && WM % 32 == 0 && WN % 32 == 0, "four DMA waves, 32x32 blocks");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const TileCoord tc = tile_coord<BM, BN>(p, blockIdx.x);
    const int64_t m0 = tc.m0, n0 = tc.n0;
    const bool dma_wave = wave < 4;
    using LA = typename std::conditional<AMN, F32LoaderMN<BM, GLB>, F32LoaderK<BM, GLB>>::type;
    using LB = typename std::conditional<BMN, F32LoaderMN<BN, GLB>, F32LoaderK<BN, GLB>>::type;
    constexpr int kStageA = LA::kStageBytes, kStageB = LB::kStageBytes, kStage = kStageA + kStageB;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * kStage];
    LA la((const char *)p.a + (tc.offa + m0 * p.sam) * 4, AMN ? p.sak : p.sam, p.M - m0, p.K, wave, lane);
    LB lb((const char *)p.b + (tc.offb + n0 * p.sbn) * 4, BMN ? p.sbk : p.sbn, p.N - n0, p.K, wave, lane);
    constexpr int kLoadsPerStage = LA::kPer + LB::kPer;
    using FA = typename std::conditional<AMN, F32FragMN<TM, BM>, FragReader<BM, TM, false, 64>>::type;
    using FB = typename std::conditional<BMN, F32FragMN<TN, BN>, FragReader<BN, TN, false, 64>>::type;
    const FA fra(0, wm * WM, lane);
    const FB frb(kStageA, wn * WN, lane);

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};
    uint4 fa[2][TM], fb[2][TN];

    const int nk = (int)((p.K + 31) / 32);
    static_assert((NS - 1) * (LA::kPer + LB::kPer) <= 63, "vmcnt counts at most 63 DMA instructions");
    if constexpr (NS == 2) {
        // prologue: stage 0, then (after it landed) stage 1 in flight
        if (dma_wave) {
            la.issue(lds, 0, wave);
            lb.issue(lds + kStageA, 0, wave);
        }
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (dma_wave) {
            la.issue(lds + kStage, 1, wave);
            lb.issue(lds + kStage + kStageA, 1, wave);
        }
    } else {
        // prologue: the first NS stages (those within K) at once, wait for stage 0
        if (dma_wave) {
            static_for<0, NS>([&](auto sc) {
                constexpr int st = decltype(sc)::value;
                if (st < nk) {
                    la.issue(lds + st * kStage, st, wave);
                    lb.issue(lds + st * kStage + kStageA, st, wave);
                }
            });
        }
        // stage 0 landed: at most (stages issued - 1) x L instructions outstanding
        static_for<1, NS + 1>([&](auto ic) {
            constexpr int issued = decltype(ic)::value;
            if ((nk < NS ? nk : NS) == issued)
                __builtin_amdgcn_s_waitcnt(waitcnt_vm((issued - 1) * (LA::kPer + LB::kPer)));
        });
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    }
    fra.read(lds, 0, fa[0]);
    frb.read(lds, 0, fb[0]);
    constexpr int kQ = TM * TN * 4;  // MFMAs per fragment group (Mma<float> issues four)
    constexpr int kReads = TM * (AMN ? 4 : 1) + TN * (BMN ? 4 : 1);
    constexpr int kPerR = (kReads + kQ / 2 - 1) / (kQ / 2);
    int cur = 0;
    for (int kt = 0; kt < nk; ++kt) {
        uint8_t *stage = lds + cur * kStage;
        const typename LA::Stage sta = la.prep(stage, kt + NS);
        const typename LB::Stage stb = lb.prep(stage + kStageA, kt + NS);
        // DMA instructions that may stay in flight once step kt+1 has landed:
        // those of the issued steps after it, min(nk - 1, kt + NS - 1) - (kt + 1)
        const int after = nk - 2 - kt < NS - 2 ? nk - 2 - kt : NS - 2;
        const int ahead = (after > 0 ? after : 0) * (LA::kPer + LB::kPer);
        static_for<0, kG - 1>([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            fra.read(stage, g + 1, fa[(g + 1) & 1]);
            frb.read(stage, g + 1, fb[(g + 1) & 1]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) Mma<float>::run(acc[i][j], fa[g & 1][i], fb[g & 1][j]);
            // group g+1's fragment reads over the first half of group g's MFMAs
            static_for<0, kQ>([&](auto qc) {
                constexpr int q = decltype(qc)::value;
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                constexpr int left = kReads - q * kPerR;
                constexpr int nr = q < kQ / 2 ? (left < kPerR ? (left > 0 ? left : 0) : kPerR) : 0;
                if constexpr (nr > 0) __builtin_amdgcn_sched_group_barrier(0x100, nr, 0);
            });
            __builtin_amdgcn_sched_barrier(0);
        });
        // every LDS read of step kt landed; this wave's DMA of step kt+1 landed
        // (NS > 2: the later stages' may still be in flight)
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (NS == 2) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(0) & ~(0xF << 8));
        } else {
            static_for<0, NS - 1>([&](auto ac) {
                constexpr int a = decltype(ac)::value * (LA::kPer + LB::kPer);
                if (ahead == a) __builtin_amdgcn_s_waitcnt(waitcnt_vm(a) & ~(0xF << 8));
            });
        }
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        constexpr int gl = (kG - 1) & 1;
        cur = cur + 1 == NS ? 0 : cur + 1;
        const uint8_t *next = lds + cur * kStage;
        fra.read(next, 0, fa[0]);
        frb.read(next, 0, fb[0]);
        __builtin_amdgcn_sched_barrier(0);
        // the deferred group's MFMAs, the DMA of step kt+2 (into the stage
        // just consumed) spread over them
        constexpr int Q = TM * TN, L = kLoadsPerStage;
        const bool more = NS == 2 || kt + NS < nk;  // NS > 2: no DMA past K
        static_for<0, Q>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            Mma<float>::run(acc[q / TN][q % TN], fa[gl][q / TN], fb[gl][q % TN]);
            if (dma_wave && more) {
                static_for<q * L / Q, (q + 1) * L / Q>([&](auto lc) {
                    constexpr int l = decltype(lc)::value;
                    if constexpr (l < LA::kPer)
                        la.template issue_one<l>(sta, wave);
                    else
                        lb.template issue_one<l - LA::kPer>(stb, wave);
                });
            }
            __builtin_amdgcn_sched_barrier(0);
        });
        __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();
    epilogue_lds<NT, WM, WN, TM, TN, NS * kStage>(p, acc, lds, wave, lane, tc.bidx * p.M * p.N, m0 + wm * WM,
                                                  n0 + wn * WN);
}

}  // namespace oxm

