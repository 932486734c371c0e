// kmatmul_mfma.hpp -- shared between the two prefill MFMA kernels (kmatmul_mfma.hip: 128 rows x 64
// columns per workgroup, each wavefront dequantizing its own rows; kmatmul_mfmaw.hip: 128 rows x
// 128 columns, every weight dequantized once per workgroup into LDS).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace kcamd {

// Up to three weight matrices over the same activations, each split over K into ks ranges
// (blockIdx.z; split z writes its partial sums to y[z]). tile0: the part's first row tile
// (blockIdx.x) of 128 rows.
struct MfmaPart {
    const uint8_t* qw;
    float* y[2];
    int rows;
    int q6;
    int tile0;
};
struct MfmaGroup {
    MfmaPart p[3];
    int nparts;
    int ks;
};

// The wide-tile kernel over `tiles` row tiles: act (fp16, 16 x), mins (Q4_K min operands) and xdT
// (column scales, ncp columns per super-block) as act_to_f16 writes them.
int launchMfmaW(const MfmaGroup& g, int tiles, const void* act, const void* mins, const float* xdT, int nsb, int ncols,
                int ncp, hipStream_t s);

}  // namespace kcamd
