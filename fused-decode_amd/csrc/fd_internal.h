// Entry points shared between the library's translation units (not exported).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fd {

// RMSNorm of `rows` contiguous rows of n elements (16-byte aligned, n % 8 == 0):
// y = round(x * rsqrt(mean(x^2) + eps) * w). Defined in norm.hip.
int rms_rows(void* y, const void* x, const void* w, int w_dtype, int64_t rows, int64_t n,
             float eps, int act_dtype, hipStream_t st);

}  // namespace fd
