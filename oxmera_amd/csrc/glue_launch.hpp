// glue_launch.hpp -- HBM-bound helper kernels used around the GEMMs by the
// Linear / MLP training step (bias gradient, MSE loss and gradient).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace oxm {

// out[c] = sum_r x[r, c] (f32 accumulate); x contiguous [R, C] of dtype.
hipError_t launch_sum_rows(const void *x, int dtype, int64_t R, int64_t C, float *out, hipStream_t s);

// loss[0] = mean((y - t)^2); dy = 2 (y - t) / n in dtype.
hipError_t launch_mse(const void *y, const void *t, void *dy, int dtype, int64_t n, float *loss, hipStream_t s);

}  // namespace oxm
