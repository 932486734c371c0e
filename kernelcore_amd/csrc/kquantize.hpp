// kquantize.hpp -- launchers of the weight quantizers and the normal generator (kquantize.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace kcamd {

// nsb super-blocks of 256 f32 values (contiguous) -> nsb ggml blocks (144 or 210 bytes each).
int launchQuantizeKquant(bool q6k, const float* x, void* blocks, long long nsb, hipStream_t s);
// y[0..n) = mean + stdev * N(0, 1), a function of (seed, index) only.
int launchFillNormal(float* y, long long n, unsigned long long seed, float mean, float stdev, hipStream_t s);

}  // namespace kcamd
