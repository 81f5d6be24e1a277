// glue.hip -- HBM-bound helper kernels for the Linear / MLP training step.
// Each reads its operands once and writes its results once; rows whose
// length and start allow it move 16 bytes per lane per access (8 bf16/f16
// or 4 f32 elements), other shapes take an element-wise fallback.
#include "gemm_kernels.hpp"
#include "glue_launch.hpp"

namespace oxm {

namespace {

__global__ void fill_zero_f32(float *p, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

// ---- element-wise fallbacks (any row length, any alignment) ----------------

// Column sums: block (bx, by) sums rows [by*kRowsPerBlock, +kRowsPerBlock) of
// columns [bx*1024, +1024); each thread owns 4 adjacent columns.
constexpr int kRowsPerBlock = 64;

__global__ void __launch_bounds__(256) sum_rows_kernel(const void *x, int dtype, int64_t R, int64_t C, float *out) {
    const int64_t c0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    const int64_t r0 = (int64_t)blockIdx.y * kRowsPerBlock;
    if (c0 >= C) return;
    const int64_t r1 = r0 + kRowsPerBlock < R ? r0 + kRowsPerBlock : R;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t r = r0; r < r1; ++r) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (c0 + i < C) acc[i] += load_as_f32(x, dtype, r * C + c0 + i);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (c0 + i < C) atomicAdd(out + c0 + i, acc[i]);
}

__global__ void __launch_bounds__(256) mse_kernel(const void *y, const void *t, void *dy, int dtype, int64_t n,
                                                  float *loss) {
    __shared__ float red[256];
    const float scale = 2.0f / (float)n;
    float acc = 0.0f;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float d = load_as_f32(y, dtype, i) - load_as_f32(t, dtype, i);
        acc += d * d;
        float g = d * scale;
        if (dtype == kDtF32)
            ((float *)dy)[i] = g;
        else if (dtype == kDtBF16)
            ((uint16_t *)dy)[i] = f32_to_bf16_bits(g);
        else
            ((uint16_t *)dy)[i] = f32_to_f16_bits(g);
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) atomicAdd(loss, red[0] / (float)n);
}

// ---- 16-byte paths ------------------------------------------------------------

// 16 bytes of DT as floats (VEC = 16 / element size).
template <int DT>
struct Vec16 {
    static constexpr int kVec = DT == kDtF32 ? 4 : 8;
    __device__ static void load(const void *p, int64_t i, float (&v)[kVec]) {
        const uint4 u = *(const uint4 *)((const char *)p + i * (DT == kDtF32 ? 4 : 2));
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
        if constexpr (DT == kDtF32) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(w[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t h = (w[e >> 1] >> (16 * (e & 1))) & 0xffffu;
                v[e] = DT == kDtBF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
            }
        }
    }
    // Rounds v to DT in place (so callers can reuse the stored values) and
    // stores it.
    __device__ static void round_store(void *p, int64_t i, float (&v)[kVec]) {
        uint32_t w[4];
        if constexpr (DT == kDtF32) {
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = __float_as_uint(v[e]);
        } else {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                uint32_t h[2];
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const float x = v[2 * d + q];
                    h[q] = DT == kDtBF16 ? f32_to_bf16_bits(x) : f32_to_f16_bits(x);
                    v[2 * d + q] = DT == kDtBF16 ? bf16_bits_to_f32(h[q]) : f16_bits_to_f32(h[q]);
                }
                w[d] = h[0] | (h[1] << 16);
            }
        }
        *(uint4 *)((char *)p + i * (DT == kDtF32 ? 4 : 2)) = make_uint4(w[0], w[1], w[2], w[3]);
    }
};

// The 16-byte kernels below share one shape: a block is 64 column chunks
// (16 bytes each: 512 bf16/f16 or 256 f32 columns) x 4 row lanes; wave w
// walks rows r0 + w, r0 + w + 4, ... of the block's kBlockRows, its 64 lanes
// reading 1 KB of contiguous row per access.  Column partials are summed
// over the 4 waves in LDS, so each column takes one atomic per block: with
// kBlockRows = 128 that is R / 128 atomics per column (same-address atomics
// are what bound an earlier version of this pass).
constexpr int kBlockRows = 128;
constexpr int kRowLanes = 4;

// cacc (this thread's V column partials) summed over the block's row lanes
// and added to out[c0 ..) by row lane 0.
template <int V>
__device__ __forceinline__ void flush_columns(float (&cacc)[V], float *out, int64_t c0, bool valid) {
    __shared__ float part[kRowLanes - 1][64 * V];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    if (ty > 0) {
#pragma unroll
        for (int e = 0; e < V; ++e) part[ty - 1][tx * V + e] = cacc[e];
    }
    __syncthreads();
    if (ty == 0 && valid) {
#pragma unroll
        for (int e = 0; e < V; ++e) {
            float v = cacc[e];
#pragma unroll
            for (int q = 0; q < kRowLanes - 1; ++q) v += part[q][tx * V + e];
            atomicAdd(out + c0 + e, v);
        }
    }
}

// Column sums over R rows of a contiguous [R, C] matrix, C a multiple of the
// vector width.
template <int DT>
__global__ void __launch_bounds__(256) sum_rows_vec_kernel(const void *x, int64_t R, int64_t C, float *out) {
    constexpr int V = Vec16<DT>::kVec, kU = 8;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int64_t c0 = ((int64_t)blockIdx.x * 64 + tx) * V;
    const int64_t r0 = (int64_t)blockIdx.y * kBlockRows;
    const int64_t r1 = r0 + kBlockRows < R ? r0 + kBlockRows : R;
    const bool valid = c0 < C;
    float acc[V] = {};
    if (valid) {
        // kU rows per iteration: their loads are all in flight before the adds
        for (int64_t r = r0 + ty; r < r1; r += kU * kRowLanes) {
            float v[kU][V];
#pragma unroll
            for (int q = 0; q < kU; ++q)
                if (r + q * kRowLanes < r1) Vec16<DT>::load(x, (r + q * kRowLanes) * C + c0, v[q]);
#pragma unroll
            for (int q = 0; q < kU; ++q) {
                if (r + q * kRowLanes >= r1) break;
#pragma unroll
                for (int e = 0; e < V; ++e) acc[e] += v[q][e];
            }
        }
    }
    flush_columns<V>(acc, out, c0, valid);
}

// MSE over a contiguous [R, C] pair, C a multiple of the vector width:
// loss += sum (y - t)^2 / n, dy = round(2 (y - t) / n), and (colsum != null)
// colsum[c] += sum over rows of the ROUNDED dy -- the bias gradient of the
// layer that produced y, formed from the same values the GEMMs will read.
template <int DT>
__global__ void __launch_bounds__(256) mse_vec_kernel(const void *y, const void *t, void *dy, int64_t R, int64_t C,
                                                      float *loss, float *colsum) {
    constexpr int V = Vec16<DT>::kVec, kU = 4;
    __shared__ float red[4];
    const float inv_n = 1.0f / ((float)R * (float)C);
    const float scale = 2.0f * inv_n;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int64_t c0 = ((int64_t)blockIdx.x * 64 + tx) * V;
    const int64_t r0 = (int64_t)blockIdx.y * kBlockRows;
    const int64_t r1 = r0 + kBlockRows < R ? r0 + kBlockRows : R;
    const bool valid = c0 < C;
    float lacc = 0.0f, cacc[V] = {};
    if (valid) {
        // kU rows per iteration: their 2 kU loads are all in flight before use
        for (int64_t r = r0 + ty; r < r1; r += kU * kRowLanes) {
            float a[kU][V], b[kU][V];
#pragma unroll
            for (int q = 0; q < kU; ++q) {
                if (r + q * kRowLanes < r1) {
                    Vec16<DT>::load(y, (r + q * kRowLanes) * C + c0, a[q]);
                    Vec16<DT>::load(t, (r + q * kRowLanes) * C + c0, b[q]);
                }
            }
#pragma unroll
            for (int q = 0; q < kU; ++q) {
                if (r + q * kRowLanes >= r1) break;
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const float d = a[q][e] - b[q][e];
                    lacc += d * d;
                    a[q][e] = d * scale;
                }
                Vec16<DT>::round_store(dy, (r + q * kRowLanes) * C + c0, a[q]);
#pragma unroll
                for (int e = 0; e < V; ++e) cacc[e] += a[q][e];
            }
        }
    }
    if (colsum) flush_columns<V>(cacc, colsum, c0, valid);
    // block sum of the squared differences: wave shuffles, then 4 partials
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) lacc += __shfl_xor(lacc, off);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = lacc;
    __syncthreads();
    if (threadIdx.x == 0) atomicAdd(loss, (red[0] + red[1] + red[2] + red[3]) * inv_n);
}

template <int DT>
void launch_mse_vec(const void *y, const void *t, void *dy, int64_t R, int64_t C, float *loss, float *colsum,
                    hipStream_t s) {
    constexpr int V = Vec16<DT>::kVec;
    dim3 grid((unsigned)((C / V + 63) / 64), (unsigned)((R + kBlockRows - 1) / kBlockRows));
    hipLaunchKernelGGL(mse_vec_kernel<DT>, grid, dim3(256), 0, s, y, t, dy, R, C, loss, colsum);
}

template <int DT>
void launch_sum_rows_vec(const void *x, int64_t R, int64_t C, float *out, hipStream_t s) {
    constexpr int V = Vec16<DT>::kVec;
    dim3 grid((unsigned)((C / V + 63) / 64), (unsigned)((R + kBlockRows - 1) / kBlockRows));
    hipLaunchKernelGGL(sum_rows_vec_kernel<DT>, grid, dim3(256), 0, s, x, R, C, out);
}

// The 16-byte paths need every row to start on a 16-byte boundary.
bool rows_vectorisable(const void *p, int dtype, int64_t C) {
    const int64_t es = dtype == kDtF32 ? 4 : 2;
    return ((uintptr_t)p % 16) == 0 && (C * es) % 16 == 0;
}

void zero(float *p, int64_t n, hipStream_t s) {
    if (n > 0) hipLaunchKernelGGL(fill_zero_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n);
}

}  // namespace

hipError_t launch_sum_rows(const void *x, int dtype, int64_t R, int64_t C, float *out, hipStream_t s) {
    zero(out, C, s);
    if (R == 0 || C == 0) return hipGetLastError();
    if (rows_vectorisable(x, dtype, C)) {
        if (dtype == kDtF32)
            launch_sum_rows_vec<kDtF32>(x, R, C, out, s);
        else if (dtype == kDtBF16)
            launch_sum_rows_vec<kDtBF16>(x, R, C, out, s);
        else
            launch_sum_rows_vec<kDtF16>(x, R, C, out, s);
        return hipGetLastError();
    }
    dim3 grid((unsigned)((C + 1023) / 1024), (unsigned)((R + kRowsPerBlock - 1) / kRowsPerBlock));
    hipLaunchKernelGGL(sum_rows_kernel, grid, dim3(256), 0, s, x, dtype, R, C, out);
    return hipGetLastError();
}

hipError_t launch_mse(const void *y, const void *t, void *dy, int dtype, int64_t R, int64_t C, float *loss,
                      float *colsum, hipStream_t s) {
    zero(loss, 1, s);
    if (colsum) zero(colsum, C, s);
    const int64_t n = R * C;
    if (rows_vectorisable(y, dtype, C) && rows_vectorisable(t, dtype, C) && rows_vectorisable(dy, dtype, C)) {
        if (dtype == kDtF32)
            launch_mse_vec<kDtF32>(y, t, dy, R, C, loss, colsum, s);
        else if (dtype == kDtBF16)
            launch_mse_vec<kDtBF16>(y, t, dy, R, C, loss, colsum, s);
        else
            launch_mse_vec<kDtF16>(y, t, dy, R, C, loss, colsum, s);
        return hipGetLastError();
    }
    int64_t blocks = (n + 1023) / 1024;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(mse_kernel, dim3((unsigned)blocks), dim3(256), 0, s, y, t, dy, dtype, n, loss);
    if (colsum) {
        dim3 grid((unsigned)((C + 1023) / 1024), (unsigned)((R + kRowsPerBlock - 1) / kRowsPerBlock));
        hipLaunchKernelGGL(sum_rows_kernel, grid, dim3(256), 0, s, dy, dtype, R, C, colsum);
    }
    return hipGetLastError();
}

hipError_t launch_fill_zero(float *p, int64_t n, hipStream_t s) {
    zero(p, n, s);
    return hipGetLastError();
}

}  // namespace oxm
