// kmatmul_mfma.hip -- the prefill matmul on CDNA4 matrix cores: Y = W X for Q4_K / Q6_K weights
// and per-256 8-bit activations (matmul_{q4k,q6k}_q8kx{4,8}; reference
// kernels/llm/matmul_q4k_q8kx8.cu, matmul_q6k_q8kx8.cu, mirror llm/llm_reference.cpp:529-596).
//
// Per (row r, column c, super-block s) the reference forms two exact integers,
//   is = sum_j sc_j * dot(q_j, x_j)        (8 sub-blocks of 32, q 4-bit, sc 6-bit)
//   im = sum_j m_j * B_j                   (B_j = sum of the 32 activations of sub-block j)
// and adds (d * xd) * is - (dmin * xd) * im. Here both integers come from
// v_mfma_f32_32x32x16_f16, exactly:
//   - the weight operand is sc_j * q (<= 945: an exact fp16 integer), produced in registers from
//     the stream with a byte permute and one packed fp16 FMA per two weights
//     ((1024 + q) * sc - 1024 * sc, the fp16 exponent trick);
//   - the activation operand is the int8 value as fp16 (exact), staged once per workgroup in LDS;
//   - every product is an integer below 2^17 and the fp32 sums stay exact while below 2^24 in
//     magnitude (256 * 945 * 127 = 3.1e7 bounds them; realistic data stays far below 2^24, and any
//     rounding beyond it is at most 2^-24 relative);
//   - im is one more MFMA with K = 16: [64 * (B >> 6), B & 63] against [m, m] (the reference's
//     byte split of B, so every operand is an exact fp16 integer).
// The float combine is acc += xd * (d * is - dmin * im) with fused multiply-adds: within a few
// ulps of the reference's order, far inside the 1e-3 bar (the tests check both).
//
// Q6_K: is = sum_t sc_t * dot(q_t - 32, x_t) over 16 sub-blocks of 16 (sc int8), no min term.
// sc * (q - 32) reaches 4096 and is not always an fp16 integer, so the scale is split,
// sc = 16 * sh + sl (sh in [-8, 7], sl in [0, 15]), and each K-step of 16 (one sub-block) runs two
// MFMAs into the same accumulator: with (16 sh)(q - 32) and with sl (q - 32), both exact fp16
// integers. acc += (d * xd) * is, as a fused multiply-add.
//
// Tiling: a workgroup of 4 wavefronts computes 128 weight rows x 128 activation columns; each
// wavefront 64 x 64 as 2 x 2 blocks of 32 x 32. The output's lane index runs along weight rows,
// so stores of y (column-major, y + c * rows) are contiguous 128-byte runs.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "internal.hpp"
#include "kquant.hpp"
#include "launch.hpp"

namespace kcamd {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int kBM = 128;         // weight rows per workgroup
constexpr int kBN = 128;         // activation columns per workgroup
constexpr int kXStride = 264;    // halves per staged column (256 + 8: spreads ds_read_b128 over banks)
constexpr int kLds = kBN * kXStride * 2 + kBN * 16 * 2 + kBN * 4;

__device__ __forceinline__ h2 bits_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t h2_bits(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// Four int8 activations -> four fp16 (two packed pairs): (x ^ 0x80) | 0x6400 is 1024 + x + 128.
__device__ __forceinline__ uint2 i8x4_to_h4(uint32_t w) {
    const uint32_t u = w ^ 0x80808080u;
    const h2 off = {(_Float16)(-1152.0f), (_Float16)(-1152.0f)};
    const h2 lo = bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) + off;
    const h2 hi = bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) + off;
    return make_uint2(h2_bits(lo), h2_bits(hi));
}

// Eight 4-bit weights (nibble `hiNib` of 8 bytes) times the sub-block scale, as 8 exact fp16.
__device__ __forceinline__ h8 dequant8(uint2 q, bool hiNib, _Float16 sc) {
    const uint32_t mask = hiNib ? 0xFFF0FFF0u : 0xFF0FFF0Fu;
    const _Float16 mul = hiNib ? sc * (_Float16)0.0625f : sc;
    const _Float16 sub = hiNib ? sc * (_Float16)(-64.0f) : sc * (_Float16)(-1024.0f);
    const h2 m2 = {mul, mul}, s2 = {sub, sub};
    h8 r;
    const uint32_t w[2] = {q.x, q.y};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const h2 a = bits_h2(__builtin_amdgcn_perm(0x64646464u, w[i], 0x04010400u) & mask);
        const h2 b = bits_h2(__builtin_amdgcn_perm(0x64646464u, w[i], 0x04030402u) & mask);
        const h2 ra = __builtin_elementwise_fma(a, m2, s2);
        const h2 rb = __builtin_elementwise_fma(b, m2, s2);
        r[4 * i + 0] = ra[0];
        r[4 * i + 1] = ra[1];
        r[4 * i + 2] = rb[0];
        r[4 * i + 3] = rb[1];
    }
    return r;
}

// One wavefront's view of 32 weight rows for one super-block: lane -> row lane % 32 and k-half
// lane / 32. Rows past the stream (padding of the last 16-row tile and beyond) read as zeros;
// their loads go to the first row instead, so every address stays inside the stream.
struct Rows32 {
    uint2 qs[4][2];  // [j'][u]: qs bytes 32j' + 16u + 8h .. +7
    float d, dmin;
    int scw[2], mw[2];  // scales / mins of sub-blocks 0-3 and 4-7, one byte each
    __device__ __forceinline__ void load(const uint8_t* qw, int row, int rows_stream, int ngroups, int s, int h) {
        const bool live = row < rows_stream;
        const int rr = live ? row : 0;
        const int tile = rr >> 4, r = rr & 15, g = s >> 2, kq = s & 3;
        const uint8_t* piece = qw + ((size_t)tile * ngroups + g) * kQ4kSeg + (kq * 16 + r) * 16;
        uint4 hdr = *reinterpret_cast<const uint4*>(piece);
        if (!live) hdr = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint2 v = *reinterpret_cast<const uint2*>(piece + (1 + 2 * a + u) * 1024 + 8 * h);
                qs[a][u] = live ? v : make_uint2(0, 0);
            }
        d = (float)__builtin_bit_cast(_Float16, (unsigned short)(hdr.x & 0xFFFFu));
        dmin = (float)__builtin_bit_cast(_Float16, (unsigned short)(hdr.x >> 16));
        const int s0 = (int)hdr.y, s1 = (int)hdr.z, s2 = (int)hdr.w;
        scw[0] = s0 & 0x3F3F3F3F;
        mw[0] = s1 & 0x3F3F3F3F;
        scw[1] = (s2 & 0x0F0F0F0F) | ((s0 >> 2) & 0x30303030);
        mw[1] = ((s2 >> 4) & 0x0F0F0F0F) | ((s1 >> 2) & 0x30303030);
    }
    __device__ __forceinline__ _Float16 sc(int j) const { return (_Float16)(float)((scw[j >> 2] >> (8 * (j & 3))) & 255); }
    __device__ __forceinline__ _Float16 m(int j) const { return (_Float16)(float)((mw[j >> 2] >> (8 * (j & 3))) & 255); }
};

// Q6_K rows: lane -> row lane % 32, half h. K-step t (sub-block t = values 16t .. 16t+15) needs
// ql bytes 64n + 32(quad & 1) + 16(t & 1) + 8h .. +7 (nibble quad >> 1) and qh bytes
// 32n + 16(t & 1) + 8h .. +7 (bits 2 quad), n = t / 8, quad = (t / 2) & 3.
struct Rows32Q6 {
    uint2 ql[2][2][2];  // [n][quad & 1][t & 1]
    uint2 qh[2][2];     // [n][t & 1]
    int sw[4];          // the 16 int8 scales
    float d;
    __device__ __forceinline__ void load(const uint8_t* qw, int row, int rows_stream, int ngroups, int s, int h) {
        const bool live = row < rows_stream;
        const int rr = live ? row : 0;
        const int tile = rr >> 4, r = rr & 15, g = s >> 2, kq = s & 3;
        const uint8_t* seg = qw + ((size_t)tile * ngroups + g) * kQ6kSeg;
        const uint8_t* piece = seg + (kq * 16 + r) * 16;
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const uint2 v = *reinterpret_cast<const uint2*>(piece + (4 * n + 2 * a + u) * 1024 + 8 * h);
                    ql[n][a][u] = live ? v : make_uint2(0, 0);
                }
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint2 v = *reinterpret_cast<const uint2*>(piece + (8 + 2 * n + u) * 1024 + 8 * h);
                qh[n][u] = live ? v : make_uint2(0, 0);
            }
        const uint4 sc = *reinterpret_cast<const uint4*>(piece + 12 * 1024);
        sw[0] = live ? (int)sc.x : 0;
        sw[1] = live ? (int)sc.y : 0;
        sw[2] = live ? (int)sc.z : 0;
        sw[3] = live ? (int)sc.w : 0;
        const uint32_t dbits = *reinterpret_cast<const uint16_t*>(seg + kQ6kSlabs * 1024 + (kq * 16 + r) * 2);
        d = live ? (float)__builtin_bit_cast(_Float16, (unsigned short)dbits) : 0.0f;
    }
    // K-step t as two exact fp16 operands: 16 sh (q - 32) and sl (q - 32), sc_t = 16 sh + sl.
    __device__ __forceinline__ void dequant(int t, h8& b1, h8& b2) const {
        const int n = t >> 3, quad = (t >> 1) & 3, u = t & 1;
        const uint2 l = ql[n][quad & 1][u], hb = qh[n][u];
        const int sc = (sw[t >> 2] << (24 - 8 * (t & 3))) >> 24;
        const int sh = sc >> 4, sl = sc & 15;
        const _Float16 fh = (_Float16)(float)sh, fl = (_Float16)(float)sl;
        const h2 mh = {fh, fh}, ml = {fl, fl};
        const h2 ch = {(_Float16)(float)(-1056 * sh), (_Float16)(float)(-1056 * sh)};
        const h2 cl = {(_Float16)(float)(-1056 * sl), (_Float16)(float)(-1056 * sl)};
        const h2 sixteen = {(_Float16)16.0f, (_Float16)16.0f};
        const uint32_t lw[2] = {l.x, l.y}, hw[2] = {hb.x, hb.y};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t q = ((lw[i] >> (4 * (quad >> 1))) & 0x0F0F0F0Fu) | (((hw[i] >> (2 * quad)) & 0x03030303u) << 4);
            const h2 a = bits_h2(__builtin_amdgcn_perm(0x64646464u, q, 0x04010400u));  // 1024 + q
            const h2 b = bits_h2(__builtin_amdgcn_perm(0x64646464u, q, 0x04030402u));
            const h2 a1 = __builtin_elementwise_fma(a, mh, ch) * sixteen, b1v = __builtin_elementwise_fma(b, mh, ch) * sixteen;
            const h2 a2 = __builtin_elementwise_fma(a, ml, cl), b2v = __builtin_elementwise_fma(b, ml, cl);
            b1[4 * i + 0] = a1[0];
            b1[4 * i + 1] = a1[1];
            b1[4 * i + 2] = b1v[0];
            b1[4 * i + 3] = b1v[1];
            b2[4 * i + 0] = a2[0];
            b2[4 * i + 1] = a2[1];
            b2[4 * i + 2] = b2v[0];
            b2[4 * i + 3] = b2v[1];
        }
    }
};

template <bool Q6>
__global__ __launch_bounds__(256) void matmul_kq_mfma_kernel(const uint8_t* __restrict__ qw,
                                                              const int* __restrict__ xq, float* __restrict__ y,
                                                              int rows, int nsb, int ncols) {
    extern __shared__ int4 lds4[];
    _Float16* xa = reinterpret_cast<_Float16*>(lds4);
    _Float16* xm = xa + kBN * kXStride;
    float* xdl = reinterpret_cast<float*>(xm + kBN * 16);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave & 1, wc = wave >> 1;
    const int h = lane >> 5, l32 = lane & 31;
    const int row0 = blockIdx.x * kBM + wr * 64;  // this wavefront's first weight row
    const int col0 = blockIdx.y * kBN;            // this workgroup's first activation column
    const int ngroups = (nsb + kGroupSb - 1) / kGroupSb;
    const int rows_stream = ((rows + kTileRows - 1) / kTileRows) * kTileRows;
    const int slot_ints = nsb * 85;

    f16v acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;
    const f16v zero = acc[0][0];

    // Software pipeline: the global loads of super-block s+1 (this thread's share of the
    // activations, this wavefront's weights) are issued before super-block s is computed, so
    // their latency hides behind the matrix work.
    constexpr int kWordsPerThread = kBN * 64 / 256;
    int xw[kWordsPerThread];
    int xp[4] = {0, 0, 0, 0};
    float xdv = 0.0f;
    auto fetchX = [&](int s) {
#pragma unroll
        for (int i = 0; i < kWordsPerThread; ++i) {
            const int idx = i * 256 + tid;
            const int c = idx >> 6, w = idx & 63;
            xw[i] = col0 + c < ncols ? xq[(size_t)(col0 + c) * slot_ints + s * 64 + w] : 0;
        }
        if (tid < kBN) {
            const bool live = col0 + tid < ncols;
            const int* slot = xq + (size_t)(live ? col0 + tid : 0) * slot_ints;
            xdv = live ? reinterpret_cast<const float*>(slot + nsb * 64)[s] : 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) xp[j] = live ? slot[nsb * 81 + s * 4 + j] : 0;
        }
    };
    using Rows = typename std::conditional<Q6, Rows32Q6, Rows32>::type;
    Rows wnext[2];
    fetchX(0);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) wnext[rb].load(qw, row0 + rb * 32 + l32, rows_stream, ngroups, 0, h);

    for (int s = 0; s < nsb; ++s) {
        // ---- stage super-block s (already in registers) into LDS as fp16
#pragma unroll
        for (int i = 0; i < kWordsPerThread; ++i) {
            const int idx = i * 256 + tid;
            const int c = idx >> 6, w = idx & 63;
            *reinterpret_cast<uint2*>(xa + c * kXStride + 4 * w) = i8x4_to_h4((uint32_t)xw[i]);
        }
        if (!Q6 && tid < kBN) {  // [B>>6 of 0-3 | of 4-7 | B&63 of 0-3 | of 4-7]
            h8 mlo, mhi;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int hb = (xp[j >> 2] << (24 - 8 * (j & 3))) >> 24;  // signed byte
                const int lb = (xp[2 + (j >> 2)] >> (8 * (j & 3))) & 255;
                mlo[j] = (_Float16)(float)(64 * hb);
                mhi[j] = (_Float16)(float)lb;
            }
            *reinterpret_cast<h8*>(xm + tid * 16) = mlo;
            *reinterpret_cast<h8*>(xm + tid * 16 + 8) = mhi;
        }
        if (tid < kBN) xdl[tid] = xdv;
        __syncthreads();
        Rows wrow[2] = {wnext[0], wnext[1]};
        if (s + 1 < nsb) {
            fetchX(s + 1);
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) wnext[rb].load(qw, row0 + rb * 32 + l32, rows_stream, ngroups, s + 1, h);
        }

        f16v is[2][2], im[2][2];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            h8 av[2];
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
                av[cb] = *reinterpret_cast<const h8*>(xa + (wc * 64 + cb * 32 + l32) * kXStride + 16 * t + 8 * h);
            if constexpr (Q6) {
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    h8 b1, b2;
                    wrow[rb].dequant(t, b1, b2);
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) {
                        is[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[cb], b1, t == 0 ? zero : is[rb][cb], 0,
                                                                           0, 0);
                        is[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[cb], b2, is[rb][cb], 0, 0, 0);
                    }
                }
            } else {
                const int j = t >> 1, u = t & 1;
                h8 bw[2];
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) bw[rb] = dequant8(wrow[rb].qs[j >> 1][u], j & 1, wrow[rb].sc(j));
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb)
                        is[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[cb], bw[rb], t == 0 ? zero : is[rb][cb],
                                                                           0, 0, 0);
            }
        }
        if constexpr (!Q6) {
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                const h8 am = *reinterpret_cast<const h8*>(xm + (wc * 64 + cb * 32 + l32) * 16 + 8 * h);
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    h8 bm;
#pragma unroll
                    for (int e = 0; e < 8; ++e) bm[e] = wrow[rb].m(e);
                    im[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, zero, 0, 0, 0);
                }
            }
        }
        // ---- Q4_K: acc += xd * (d * is - dmin * im); Q6_K: acc += (d * xd) * is
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int c = wc * 64 + cb * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
                const float xd = xdl[c];
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    if constexpr (Q6) {
                        acc[rb][cb][i] = __builtin_fmaf(wrow[rb].d * xd, is[rb][cb][i], acc[rb][cb][i]);
                    } else {
                        const float t2 = __builtin_fmaf(-wrow[rb].dmin, im[rb][cb][i], wrow[rb].d * is[rb][cb][i]);
                        acc[rb][cb][i] = __builtin_fmaf(xd, t2, acc[rb][cb][i]);
                    }
                }
            }
        __syncthreads();  // the next super-block overwrites the staged activations
    }

#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const int row = row0 + rb * 32 + l32;
        if (row >= rows) continue;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int c = col0 + wc * 64 + cb * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
                if (c < ncols) y[(size_t)c * rows + row] = acc[rb][cb][i];
            }
    }
}

template <bool Q6>
int runMfma(const kcMatmulKQ8Args& a, hipStream_t s) {
    static const int attr = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(matmul_kq_mfma_kernel<Q6>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
    if (attr != 0) return fromHip(attr, "matmul (MFMA): LDS size");
    const dim3 grid((a.rows + kBM - 1) / kBM, (a.ncols + kBN - 1) / kBN);
    hipLaunchKernelGGL(matmul_kq_mfma_kernel<Q6>, grid, dim3(256), kLds, s, reinterpret_cast<const uint8_t*>(a.qw), a.xq,
                       a.y, a.rows, a.k / 256, a.ncols);
    return fromHip(hipGetLastError(), Q6 ? "matmul_q6k_q8k (MFMA)" : "matmul_q4k_q8k (MFMA)");
}

}  // namespace

int launchMatmulMfma(bool q6k, const kcMatmulKQ8Args& a, hipStream_t s) {
    return q6k ? runMfma<true>(a, s) : runMfma<false>(a, s);
}

}  // namespace kcamd
