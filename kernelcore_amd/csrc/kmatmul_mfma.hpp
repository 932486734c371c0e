// kmatmul_mfma.hpp -- shared between the two prefill MFMA kernels (kmatmul_mfma.hip: 128 rows x 64
// columns per workgroup, each wavefront dequantizing its own rows; kmatmul_mfmaw.hip: 128 rows x
// 128 columns, every weight dequantized once per workgroup into LDS).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace kcamd {

// Up to three weight matrices over the same activations, each split over K into ks ranges
// (blockIdx.z; split z writes its partial sums to y[z]). tile0: the part's first row tile
// (blockIdx.x) of 128 rows. ks (the producer-wavefront kernel only; 0 = the group's split over
// blockIdx.z): the part's own split, its ks x ntiles workgroups at blockIdx.x = tile0 + z ntiles +
// row tile (the group's ks is then 1).
struct MfmaPart {
    const uint8_t* qw;
    float* y[2];
    int rows;
    int q6;
    int tile0;
    int ks;
    int ntiles;
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

// The producer-wavefront kernel (kmatmul_mfmaws.hip): Q4_K and Q6_K parts, 256-row tiles (tile0 in
// units of mfmaWsRows()); mfmaWsFits says whether g's parts and the activations fit its 32-bit
// buffer offsets.
int mfmaWsRows();
bool mfmaWsFits(const MfmaGroup& g, int nsb, int ncols);
int launchMfmaWs(const MfmaGroup& g, int tiles, const void* act, const void* mins, const float* xdT, int nsb, int ncols,
                 int ncp, hipStream_t s);
// The same kernel reading the per-256 int8 slots (xq) itself: no fp16 conversion launch before it
// (Q4_K parts only; k a multiple of 1024: mfmaWsSlotsFits).
bool mfmaWsSlotsFits(int nsb);
int launchMfmaWsSlots(const MfmaGroup& g, int tiles, const int* xq, int nsb, int ncols, hipStream_t s);

}  // namespace kcamd
