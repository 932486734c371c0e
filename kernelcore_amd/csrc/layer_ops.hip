// layer_ops.hip -- bandwidth-bound elementwise and row kernels around the K-quant matvecs (gfx950).
#include <hip/hip_runtime.h>

#include "internal.hpp"
#include "launch.hpp"

namespace kcamd {
namespace {

// kernels/vector_add.cu: out[i] = a[i] + b[i].
__global__ void vector_add_kernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ out,
                                  int count) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) out[i] = a[i] + b[i];
}

}  // namespace

int launchVectorAdd(const float* a, const float* b, float* out, int count, hipStream_t s) {
    if (count == 0) return 0;
    hipLaunchKernelGGL(vector_add_kernel, dim3((count + 255) / 256), dim3(256), 0, s, a, b, out, count);
    return fromHip(hipGetLastError(), "vector_add");
}

}  // namespace kcamd
