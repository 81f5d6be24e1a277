// glue_launch.hpp -- HBM-bound helper kernels used around the GEMMs by the
// Linear / MLP training step (bias gradient, MSE loss and gradient).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace oxm {

// out[c] = sum_r x[r, c] (f32 accumulate); x contiguous [R, C] of dtype.
hipError_t launch_sum_rows(const void *x, int dtype, int64_t R, int64_t C, float *out, hipStream_t s);

// loss[0] = mean((y - t)^2); dy = 2 (y - t) / n in dtype.
// loss = mean((y - t)^2), dy = 2 (y - t) / n over a contiguous [R, C] pair;
// colsum (nullable, [C] f32) receives the column sums of the rounded dy.
hipError_t launch_mse(const void *y, const void *t, void *dy, int dtype, int64_t R, int64_t C, float *loss,
                      float *colsum, hipStream_t s);

// p[0 .. n) = 0 with a fill kernel (safe inside captured graphs).
hipError_t launch_fill_zero(float *p, int64_t n, hipStream_t s);

}  // namespace oxm
