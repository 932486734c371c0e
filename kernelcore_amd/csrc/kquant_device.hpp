// kquant_device.hpp -- device functions shared by the K-quant kernels (HIP sources only).
//
// The per-super-block terms restate the reference kernels' float and integer operations in the
// same order (arasheedu/Kernelcore kernels/llm/matvec_q4k_q8.cu:44-85, matvec_q6k_q8.cu:44-102,
// matmul_q4k_q8kx8.cu, matmul_q6k_q8kx8.cu; mirror llm/llm_reference.cpp:413-596), so a caller
// that adds the terms in super-block order reproduces the reference bit for bit.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kquant.hpp"

namespace kcamd {

constexpr uint32_t kLow4 = 0x0F0F0F0Fu;  // reference: 252645135

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }
__device__ __forceinline__ float f16bits(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (unsigned short)h); }
__device__ __forceinline__ int sbyte(int w, int i) { return (w << (24 - 8 * i)) >> 24; }

// Eight activation words at p: one 16-byte load pair when p is 16-byte aligned (A16), else
// single-word loads.
template <bool A16>
__device__ __forceinline__ void load8(const int* p, int* w) {
    if (A16) {
        const int4 a = reinterpret_cast<const int4*>(p)[0], b = reinterpret_cast<const int4*>(p)[1];
        w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w, w[4] = b.x, w[5] = b.y, w[6] = b.z, w[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = p[i];
    }
}

// Matvec LDS layout (ints), nsbp = padded super-blocks:
//   xs   [nsbp][68]  q8 words of each super-block (64 + pad: 4 lanes groups read 4 different
//                    super-blocks per ds_read_b128 without bank conflicts)
//   dx   [nsbp * 8]  block scales d
//   aux  [nsbp * 8]  Q4_K: d * sum (the reference's xd[2b] * xd[2b+1]); Q6_K: (int) sum of 32
//   s16  [nsbp * 8]  Q6_K: sum of the first 16 values of each block
//   terms[WT][nt][16] per-super-block float terms, nt = nsbp (Q4_K) or 2 * nsbp (Q6_K)
template <bool A16 = true>
__device__ __forceinline__ float q4k_term(const uint32_t* c, const int* xs, const float* dx, const float* dxs) {
    const uint32_t h = c[0];
    const float d = f16bits(h & 0xFFFFu), dmin = f16bits(h >> 16);
    const int s0 = (int)c[1], s1 = (int)c[2], s2 = (int)c[3];
    const int sclo = s0 & 0x3F3F3F3F;
    const int mlo = s1 & 0x3F3F3F3F;
    const int schi = (s2 & 0x0F0F0F0F) | ((s0 >> 2) & 0x30303030);
    const int mhi = ((s2 >> 4) & 0x0F0F0F0F) | ((s1 >> 2) & 0x30303030);
    float fd = 0.0f, fm = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int xaw[8], xbw[8];
        load8<A16>(xs + 16 * j, xaw);
        load8<A16>(xs + 16 * j + 8, xbw);
        int da = 0, db = 0;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint32_t q = c[4 + 8 * j + w];
            da = dot4((int)(q & kLow4), xaw[w], da);
            db = dot4((int)((q >> 4) & kLow4), xbw[w], db);
        }
        const int sh = 16 * (j & 1);
        const int scw = j < 2 ? sclo : schi;
        const int mw = j < 2 ? mlo : mhi;
        const int sca = (scw >> sh) & 255, scb = (scw >> (sh + 8)) & 255;
        const int ma = (mw >> sh) & 255, mb = (mw >> (sh + 8)) & 255;
        fd += (float)(sca * da) * dx[2 * j] + (float)(scb * db) * dx[2 * j + 1];
        fm += (float)ma * dxs[2 * j] + (float)mb * dxs[2 * j + 1];
    }
    return d * fd - dmin * fm;
}

// The two halves of a Q6_K super-block (matvec_q6k_q8.cu:33-105): out[n] = d * (sum_t is_t * dx_t).
template <bool A16 = true>
__device__ __forceinline__ void q6k_terms(const uint32_t* c, uint32_t dbits, const int* xs, const float* dx,
                                          const int* sum32, const int* s16, float* out0, float* out1) {
    const float d = f16bits(dbits);
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        int da[4] = {0, 0, 0, 0}, db[4] = {0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int xw[8];
            load8<A16>(xs + (4 * n + t) * 8, xw);
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                const int qa = (int)c[16 * n + w];
                const int qc = (int)c[16 * n + 8 + w];
                const int h = (int)c[32 + 8 * n + w];
                int q;
                if (t == 0) q = (qa & 0x0F0F0F0F) | ((h << 4) & 0x30303030);
                else if (t == 1) q = (qc & 0x0F0F0F0F) | ((h << 2) & 0x30303030);
                else if (t == 2) q = ((qa >> 4) & 0x0F0F0F0F) | (h & 0x30303030);
                else q = ((qc >> 4) & 0x0F0F0F0F) | ((h >> 2) & 0x30303030);
                if (w < 4) da[t] = dot4(q, xw[w], da[t]);
                else db[t] = dot4(q, xw[w], db[t]);
            }
        }
        const int sw0 = (int)c[48 + 2 * n], sw1 = (int)c[48 + 2 * n + 1];
        int is[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int sw = t < 2 ? sw0 : sw1;
            const int lo = 2 * (t & 1);
            const int sa = s16[4 * n + t];
            const int sb = sum32[4 * n + t] - sa;
            is[t] = sbyte(sw, lo) * (da[t] - 32 * sa) + sbyte(sw, lo + 1) * (db[t] - 32 * sb);
        }
        const float v = d * ((float)is[0] * dx[4 * n] + (float)is[1] * dx[4 * n + 1] + (float)is[2] * dx[4 * n + 2] +
                             (float)is[3] * dx[4 * n + 3]);
        if (n == 0) *out0 = v;
        else *out1 = v;
    }
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// The slabs of one (tile, group) segment held by a lane: its 16-byte piece of every slab (and the
// Q6_K d). NT: non-temporal loads (the weights are read once per matvec).
template <bool Q6, bool NT>
struct Pieces {
    static constexpr int kSlabs = Q6 ? kQ6kSlabs : kQ4kSlabs;
    u32x4 c[kSlabs];
    uint32_t dbits;
    __device__ __forceinline__ void load(const uint8_t* seg, int lane) {
#pragma unroll
        for (int i = 0; i < kSlabs; ++i) {
            const u32x4* p = reinterpret_cast<const u32x4*>(seg + i * 1024 + lane * 16);
            c[i] = NT ? __builtin_nontemporal_load(p) : *p;
        }
        if (Q6) dbits = *reinterpret_cast<const uint16_t*>(seg + kSlabs * 1024 + lane * 2);
    }
};


// ---- per-256 activations (quantize_cols_k slots): one column's term of a super-block ----------

// matmul_q4k_q8kx8 per column (llm/llm_reference.cpp:529-562): xs = slot + s*64, xd = the slot's
// d of super-block s, b16 = its 16 sums of 16 (sums of 32 are pairs of them).
template <bool A16>
__device__ __forceinline__ float q4k_term_k(const uint32_t* c, const int* xs, float xd, const int* b16) {
    const uint32_t h = c[0];
    const float d = f16bits(h & 0xFFFFu), dmin = f16bits(h >> 16);
    const int s0 = (int)c[1], s1 = (int)c[2], s2 = (int)c[3];
    const int sclo = s0 & 0x3F3F3F3F;
    const int mlo = s1 & 0x3F3F3F3F;
    const int schi = (s2 & 0x0F0F0F0F) | ((s0 >> 2) & 0x30303030);
    const int mhi = ((s2 >> 4) & 0x0F0F0F0F) | ((s1 >> 2) & 0x30303030);
    int is = 0, im = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int xaw[8], xbw[8];
        load8<A16>(xs + 16 * j, xaw);
        load8<A16>(xs + 16 * j + 8, xbw);
        int da = 0, db = 0;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint32_t q = c[4 + 8 * j + w];
            da = dot4((int)(q & kLow4), xaw[w], da);
            db = dot4((int)((q >> 4) & kLow4), xbw[w], db);
        }
        const int sh = 16 * (j & 1);
        const int scw = j < 2 ? sclo : schi;
        const int mw = j < 2 ? mlo : mhi;
        is += ((scw >> sh) & 255) * da + ((scw >> (sh + 8)) & 255) * db;
        im += ((mw >> sh) & 255) * (b16[4 * j] + b16[4 * j + 1]) +
              ((mw >> (sh + 8)) & 255) * (b16[4 * j + 2] + b16[4 * j + 3]);
    }
    return (d * xd) * (float)is - (dmin * xd) * (float)im;
}

// matmul_q6k_q8kx8 per column (llm/llm_reference.cpp:564-596).
template <bool A16>
__device__ __forceinline__ float q6k_term_k(const uint32_t* c, uint32_t dbits, const int* xs, float xd,
                                            const int* b16) {
    const float d = f16bits(dbits);
    int is = 0;
#pragma unroll
    for (int n = 0; n < 2; ++n) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int xw[8];
            load8<A16>(xs + (4 * n + t) * 8, xw);
            int da = 0, db = 0;
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                const int qa = (int)c[16 * n + 8 * (t & 1) + w];
                const int h = (int)c[32 + 8 * n + w];
                const int q = ((qa >> (4 * (t >> 1))) & 0x0F0F0F0F) | (((h >> (2 * t)) << 4) & 0x30303030);
                if (w < 4) da = dot4(q, xw[w], da);
                else db = dot4(q, xw[w], db);
            }
            const int sw = (int)c[48 + 2 * n + (t >> 1)];
            const int lo = 2 * (t & 1);
            const int o = (4 * n + t) * 2;
            is += sbyte(sw, lo) * (da - 32 * b16[o]) + sbyte(sw, lo + 1) * (db - 32 * b16[o + 1]);
        }
    }
    return (d * xd) * (float)is;
}

}  // namespace kcamd
