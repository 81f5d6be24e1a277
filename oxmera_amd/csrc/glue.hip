// glue.hip -- HBM-bound helper kernels for the Linear / MLP training step.
// These are memory-bound (one read of each operand, one write of each
// result); they use wide grids and coalesced row-major access.
#include "gemm_kernels.hpp"
#include "glue_launch.hpp"

namespace oxm {

namespace {

__global__ void fill_zero_f32(float *p, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

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

}  // namespace

hipError_t launch_sum_rows(const void *x, int dtype, int64_t R, int64_t C, float *out, hipStream_t s) {
    hipLaunchKernelGGL(fill_zero_f32, dim3((unsigned)((C + 255) / 256)), dim3(256), 0, s, out, C);
    if (R == 0) return hipGetLastError();
    dim3 grid((unsigned)((C + 1023) / 1024), (unsigned)((R + kRowsPerBlock - 1) / kRowsPerBlock));
    hipLaunchKernelGGL(sum_rows_kernel, grid, dim3(256), 0, s, x, dtype, R, C, out);
    return hipGetLastError();
}

hipError_t launch_mse(const void *y, const void *t, void *dy, int dtype, int64_t n, float *loss, hipStream_t s) {
    hipLaunchKernelGGL(fill_zero_f32, dim3(1), dim3(256), 0, s, loss, (int64_t)1);
    int64_t blocks = (n + 1023) / 1024;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(mse_kernel, dim3((unsigned)blocks), dim3(256), 0, s, y, t, dy, dtype, n, loss);
    return hipGetLastError();
}

}  // namespace oxm
