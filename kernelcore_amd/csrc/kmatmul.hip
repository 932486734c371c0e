// kmatmul.hip -- Y = W X for K-quant weights and several 8-bit activation columns (gfx950).
//
// Names and results follow the reference's matmul kernels (arasheedu/Kernelcore
// kernels/llm/matmul_{q4k,q6k}_q8x{4,8}.cu: per-32 slots, bit-identical per column to the
// matvec; matmul_{q4k,q6k}_q8kx{4,8}.cu: per-256 slots, mirror llm/llm_reference.cpp:529-596).
// Column c of X is the activation slot xq + c * slot_ints; its outputs go to y + c * rows.
//
// This file holds the column-tiled ("skinny") kernel: the matvec's tile layout with each lane
// computing NC columns from one load of its weights, and the per-row sum of super-block terms
// done in registers in super-block order (the four lanes of a row pass their terms with
// cross-lane reads, in order), which keeps every column bit-identical to the reference. It serves
// small batches and the per-32 names; large per-256 batches go to the MFMA kernel.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "internal.hpp"
#include "kquant.hpp"
#include "kquant_device.hpp"
#include "launch.hpp"

namespace kcamd {
namespace {

// The per-32 terms read their column's activations straight from global memory (16 lanes read
// the same words; L1 serves them). dx / dxs / sums are formed in registers with the reference's
// float products (xd[2b] * xd[2b+1]).
template <bool A16>
__device__ __forceinline__ float q4k_term_g(const uint32_t* c, const int* slot, int nb, int s) {
    const float* xd = reinterpret_cast<const float*>(slot + nb * 8) + 16 * s;
    float dx[8], dxs[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        dx[b] = xd[2 * b];
        dxs[b] = xd[2 * b] * xd[2 * b + 1];
    }
    return q4k_term<A16>(c, slot + 64 * s, dx, dxs);
}

template <bool A16>
__device__ __forceinline__ void q6k_terms_g(const uint32_t* c, uint32_t dbits, const int* slot, int nb, int s,
                                            float* t0, float* t1) {
    const float* xd = reinterpret_cast<const float*>(slot + nb * 8) + 16 * s;
    const int* xs = slot + 64 * s;
    float dx[8];
    int s32[8], s16[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        dx[b] = xd[2 * b];
        s32[b] = (int)xd[2 * b + 1];
        int w[8];
        load8<A16>(xs + 8 * b, w);
        s16[b] = dot4(0x01010101, w[3], dot4(0x01010101, w[2], dot4(0x01010101, w[1], dot4(0x01010101, w[0], 0))));
    }
    q6k_terms<A16>(c, dbits, xs, dx, s32, s16, t0, t1);
}

// Adds the terms of super-blocks 4g .. 4g+3 (held by lanes kq = 0..3 of this row) to acc in order.
__device__ __forceinline__ float addInOrder(float acc, float t, int r, int valid) {
#pragma unroll
    for (int q = 0; q < kGroupSb; ++q) {
        const float v = __shfl(t, q * 16 + r);
        if (q < valid) acc += v;
    }
    return acc;
}

template <bool Q6, bool K8, int NC, bool A16>
__global__ __launch_bounds__(256) void matmul_cols_kernel(const uint8_t* __restrict__ qw, const int* __restrict__ xq,
                                                          float* __restrict__ y, int rows, int nsb, int ntiles,
                                                          int ncols) {
    constexpr int kSeg = Q6 ? kQ6kSeg : kQ4kSeg;
    const int lane = threadIdx.x & 63;
    const int tile = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (tile >= ntiles) return;  // whole wavefronts; no barrier follows
    const int kq = lane >> 4, r = lane & 15;
    const int col0 = blockIdx.y * NC;
    const int ngroups = (nsb + kGroupSb - 1) / kGroupSb;
    const int nb = nsb * 8;
    const int slot_ints = K8 ? nsb * 85 : nb * 11;
    const uint8_t* seg0 = qw + (size_t)tile * ngroups * kSeg;
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
    for (int g = 0; g < ngroups; ++g) {
        Pieces<Q6, true> p;
        p.load(seg0 + (size_t)g * kSeg, lane);
        const uint32_t* cw = reinterpret_cast<const uint32_t*>(p.c);
        const int s = g * kGroupSb + kq;
        const bool real = s < nsb;
        const int valid = min(kGroupSb, nsb - g * kGroupSb);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (col0 + c >= ncols) break;  // uniform
            const int* slot = xq + (size_t)(col0 + c) * slot_ints;
            if (K8) {
                float t = 0.0f;
                if (real) {
                    const float xd = reinterpret_cast<const float*>(slot + nsb * 64)[s];
                    const int* b16 = slot + nsb * 65 + s * 16;
                    t = Q6 ? q6k_term_k<A16>(cw, p.dbits, slot + s * 64, xd, b16)
                           : q4k_term_k<A16>(cw, slot + s * 64, xd, b16);
                }
                acc[c] = addInOrder(acc[c], t, r, valid);
            } else if (Q6) {
                float t0 = 0.0f, t1 = 0.0f;
                if (real) q6k_terms_g<A16>(cw, p.dbits, slot, nb, s, &t0, &t1);
#pragma unroll
                for (int q = 0; q < kGroupSb; ++q) {  // both halves of super-block 4g+q, in order
                    const float v0 = __shfl(t0, q * 16 + r), v1 = __shfl(t1, q * 16 + r);
                    if (q < valid) {
                        acc[c] += v0;
                        acc[c] += v1;
                    }
                }
            } else {
                const float t = real ? q4k_term_g<A16>(cw, slot, nb, s) : 0.0f;
                acc[c] = addInOrder(acc[c], t, r, valid);
            }
        }
    }
    const int row = tile * kTileRows + r;
    if (kq == 0 && row < rows) {
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (col0 + c < ncols) y[(size_t)(col0 + c) * rows + row] = acc[c];
    }
}

template <bool Q6, bool K8, int NC>
int runCols(const kcMatmulKQ8Args& a, hipStream_t s) {
    const int ntiles = tilesOf(a.rows);
    const dim3 grid((ntiles + 3) / 4, (a.ncols + NC - 1) / NC);
    // 16-byte activation loads when every slot starts 16-byte aligned
    const int slot_ints = K8 ? a.k / 256 * 85 : a.k / 32 * 11;
    const bool a16 = (reinterpret_cast<uintptr_t>(a.xq) & 15) == 0 && slot_ints % 4 == 0;
    const uint8_t* qw = reinterpret_cast<const uint8_t*>(a.qw);
    if (a16)
        hipLaunchKernelGGL((matmul_cols_kernel<Q6, K8, NC, true>), grid, dim3(256), 0, s, qw, a.xq, a.y, a.rows,
                           a.k / 256, ntiles, a.ncols);
    else
        hipLaunchKernelGGL((matmul_cols_kernel<Q6, K8, NC, false>), grid, dim3(256), 0, s, qw, a.xq, a.y, a.rows,
                           a.k / 256, ntiles, a.ncols);
    return fromHip(hipGetLastError(), "matmul (column tiles)");
}

template <bool Q6, bool K8>
int pickCols(const kcMatmulKQ8Args& a, hipStream_t s) {
    if (a.ncols <= 1) return runCols<Q6, K8, 1>(a, s);
    if (a.ncols <= 2) return runCols<Q6, K8, 2>(a, s);
    if (a.ncols <= 4) return runCols<Q6, K8, 4>(a, s);
    return runCols<Q6, K8, 8>(a, s);
}

}  // namespace

int launchMatmulCols(bool q6k, bool per256, const kcMatmulKQ8Args& a, hipStream_t s) {
    if (q6k) return per256 ? pickCols<true, true>(a, s) : pickCols<true, false>(a, s);
    return per256 ? pickCols<false, true>(a, s) : pickCols<false, false>(a, s);
}

int launchMatmulKq(bool q6k, bool per256, const kcMatmulKQ8Args& a, hipStream_t s) {
    // "matmul_path": 0 default (MFMA from 64 columns with per-256 slots), 1 column tiles; 2 and up
    // force the MFMA kernels: 2 default MFMA kernel, 3 register-staged 2 x 2 blocks per wavefront,
    // 4 / 5 register-staged one-wavefront-per-SIMD rows (two / one super-block groups), 7 the
    // wide-tile kernel (kmatmul_mfmaw.hip).
    const int path = option("matmul_path");
    const bool mfma = per256 && (path >= 2 || (path == 0 && a.ncols >= 64));
    if (mfma) return launchMatmulMfma(q6k, a, s);
    return launchMatmulCols(q6k, per256, a, s);
}

}  // namespace kcamd
