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
// The fp16-activation kernels (matmul_kq_mfma_h_kernel) read the activations converted once to
// fp16 as 16 x (exact: |16 x| <= 2032). Their weight operands are scaled to match: sc q / 16
// (Q4_K) and sh (q - 32), sl (q - 32) / 16 (Q6_K), all still exact fp16 values, so every product
// is the same integer as above; the Q6_K operands then need no x16 product, and their constants
// are fp16 products of small integers.
//
// Tiling: a workgroup of 4 wavefronts computes 128 weight rows x 128 activation columns; each
// wavefront 64 x 64 as 2 x 2 blocks of 32 x 32. The output's lane index runs along weight rows,
// so stores of y (column-major, y + c * rows) are contiguous 128-byte runs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>
#include <vector>

#include "internal.hpp"
#include "kquant.hpp"
#include "kmatmul_mfma.hpp"
#include "launch.hpp"

namespace kcamd {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32v4 __attribute__((ext_vector_type(4)));

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

// Four int8 activations -> four fp16 values 16 x (exact): (x ^ 0x80) | 0x6400 is 1024 + x + 128,
// and (1152 + x) * 16 - 18432 = 16 x in one fused multiply-add.
__device__ __forceinline__ uint2 i8x4_to_h4x16(uint32_t w) {
    const uint32_t u = w ^ 0x80808080u;
    const h2 m = {(_Float16)16.0f, (_Float16)16.0f}, c = {(_Float16)(-18432.0f), (_Float16)(-18432.0f)};
    const h2 lo = __builtin_elementwise_fma(bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)), m, c);
    const h2 hi = __builtin_elementwise_fma(bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)), m, c);
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
// lane / 32. Rows past the stream (padding of the last 16-row tile and beyond) read the first
// row instead, so every address stays inside the stream; their outputs are never stored. (No
// select on the loaded values: it would make the prefetch wait for its own loads.)
// load() only issues the loads (nothing reads the loaded words until decode(), so the loads of
// the next super-block stay in flight behind the current one's compute).
struct Rows32 {
    uint2 qs[4][2];  // [j'][u]: qs bytes 32j' + 16u + 8h .. +7
    uint4 hdr;       // d, dmin (fp16) and the 12 packed scale / min bytes
    float d, dmin;
    int scw[2], mw[2];  // scales / mins of sub-blocks 0-3 and 4-7, one byte each
    __device__ __forceinline__ void load(const uint8_t* qw, int row, int rows_stream, int ngroups, int s, int h) {
        const bool live = row < rows_stream;
        const int rr = live ? row : 0;
        const int tile = rr >> 4, r = rr & 15, g = s >> 2, kq = s & 3;
        const uint8_t* piece = qw + ((size_t)tile * ngroups + g) * kQ4kSeg + (kq * 16 + r) * 16;
        hdr = *reinterpret_cast<const uint4*>(piece);
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int u = 0; u < 2; ++u) qs[a][u] = *reinterpret_cast<const uint2*>(piece + (1 + 2 * a + u) * 1024 + 8 * h);
    }
    __device__ __forceinline__ void decode() {
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
    uint32_t dbits;     // d (fp16)
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
                for (int u = 0; u < 2; ++u)
                    ql[n][a][u] = *reinterpret_cast<const uint2*>(piece + (4 * n + 2 * a + u) * 1024 + 8 * h);
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
            for (int u = 0; u < 2; ++u) qh[n][u] = *reinterpret_cast<const uint2*>(piece + (8 + 2 * n + u) * 1024 + 8 * h);
        const uint4 sc = *reinterpret_cast<const uint4*>(piece + 12 * 1024);
        sw[0] = (int)sc.x;
        sw[1] = (int)sc.y;
        sw[2] = (int)sc.z;
        sw[3] = (int)sc.w;
        dbits = *reinterpret_cast<const uint16_t*>(seg + kQ6kSlabs * 1024 + (kq * 16 + r) * 2);
    }
    __device__ __forceinline__ void decode() { d = (float)__builtin_bit_cast(_Float16, (unsigned short)dbits); }
    // K-step t for activations 16 x: sh (q - 32) and sl (q - 32) / 16 (so 16 x times them gives
    // 16 sh (q - 32) x and sl (q - 32) x, sc_t = 16 sh + sl), both exact fp16; the constants sh,
    // -1056 sh, sl / 16 and -66 sl are fp16 products of small integers (exact).
    __device__ __forceinline__ void dequantA16(int t, h8& b1, h8& b2) const {
        const int n = t >> 3, quad = (t >> 1) & 3, u = t & 1;
        const uint2 l = ql[n][quad & 1][u], hb = qh[n][u];
        const int w = sw[t >> 2];
        const int sh = (w << (24 - 8 * (t & 3))) >> 28, sl = (w >> (8 * (t & 3))) & 15;
        const _Float16 fh = (_Float16)(short)sh, fl = (_Float16)(short)sl;
        const h2 mh = {fh, fh}, ml = {fl * (_Float16)0.0625f, fl * (_Float16)0.0625f};
        const h2 ch = {fh * (_Float16)(-1056.0f), fh * (_Float16)(-1056.0f)};
        const h2 cl = {fl * (_Float16)(-66.0f), fl * (_Float16)(-66.0f)};
        const uint32_t lw[2] = {l.x, l.y}, hw[2] = {hb.x, hb.y};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t q = ((lw[i] >> (4 * (quad >> 1))) & 0x0F0F0F0Fu) | (((hw[i] >> (2 * quad)) & 0x03030303u) << 4);
            const h2 a = bits_h2(__builtin_amdgcn_perm(0x64646464u, q, 0x04010400u));  // 1024 + q
            const h2 b = bits_h2(__builtin_amdgcn_perm(0x64646464u, q, 0x04030402u));
            const h2 a1 = __builtin_elementwise_fma(a, mh, ch), b1v = __builtin_elementwise_fma(b, mh, ch);
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
        wrow[0].decode();
        wrow[1].decode();
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

// Row-wavefront variant: the same 128 x 128 tile per workgroup, each wavefront 32 weight rows x
// all 128 columns (four 32 x 32 blocks, so one dequantized weight fragment feeds four MFMAs).
// NG = 2: eight wavefronts, the super-blocks split by parity between wavefronts 0-3 and 4-7
// (two per SIMD, overlapping each other's vector and matrix work); both groups' activations are
// staged per iteration and the two partial sums are added at the end.
constexpr int kLdsGrp = kBN * kXStride * 2 + kBN * 16 * 2 + kBN * 4;

template <bool Q6, int NG>
__global__ __launch_bounds__(256 * NG) void matmul_kq_mfma8_kernel(const uint8_t* __restrict__ qw,
                                                              const int* __restrict__ xq, float* __restrict__ y,
                                                              int rows, int nsb, int ncols) {
    extern __shared__ int4 lds4[];
    _Float16* xa0 = reinterpret_cast<_Float16*>(lds4);             // [NG][kBN][kXStride]
    _Float16* xm0 = xa0 + NG * kBN * kXStride;                       // [NG][kBN][16]
    float* xd0 = reinterpret_cast<float*>(xm0 + NG * kBN * 16);      // [NG][kBN]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int NT = 256 * NG;  // threads
    const int grp = wave >> 2, wr = wave & 3;
    const int h = lane >> 5, l32 = lane & 31;
    const int row = blockIdx.x * kBM + wr * 32 + l32;  // this lane's weight row
    const int col0 = blockIdx.y * kBN;
    const int ngroups = (nsb + kGroupSb - 1) / kGroupSb;
    const int rows_stream = ((rows + kTileRows - 1) / kTileRows) * kTileRows;
    const int slot_ints = nsb * 85;
    const int iters = (nsb + NG - 1) / NG;
    const _Float16* xa = xa0 + grp * kBN * kXStride;
    const _Float16* xm = xm0 + grp * kBN * 16;
    const float* xdl = xd0 + grp * kBN;

    f16v acc[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[cb][i] = 0.0f;
    const f16v zero = acc[0];

    // activations of both super-blocks of an iteration: 32 words per thread, and for 256 threads
    // one column's mins words and scale
    constexpr int kWords = NG * kBN * 64 / NT;
    int xw[kWords];
    int xp[4] = {0, 0, 0, 0};
    float xdv = 0.0f;
    auto fetchX = [&](int it) {
#pragma unroll
        for (int i = 0; i < kWords; ++i) {
            const int idx = i * NT + tid;
            const int sb = idx >> 13, rem = idx & 8191;
            const int c = rem >> 6, w = rem & 63;
            const int sx = NG * it + sb;
            const bool live = col0 + c < ncols && sx < nsb;  // dead columns / super-blocks: never stored
            xw[i] = xq[(size_t)(live ? col0 + c : 0) * slot_ints + (live ? sx : 0) * 64 + w];
        }
        if (tid < NG * kBN) {
            const int sb = tid >> 7, c = tid & 127, sx = NG * it + sb;
            const bool live = col0 + c < ncols && sx < nsb;
            const int* slot = xq + (size_t)(live ? col0 + c : 0) * slot_ints;
            const int sxc = live ? sx : 0;
            xdv = reinterpret_cast<const float*>(slot + nsb * 64)[sxc];
#pragma unroll
            for (int j = 0; j < 4; ++j) xp[j] = slot[nsb * 81 + sxc * 4 + j];
        }
    };
    using Rows = typename std::conditional<Q6, Rows32Q6, Rows32>::type;
    Rows wcur, wnext;
    fetchX(0);
    if (grp < nsb) wnext.load(qw, row, rows_stream, ngroups, grp, h);

    for (int it = 0; it < iters; ++it) {
        // ---- stage this iteration's two super-blocks (in registers) into LDS as fp16
#pragma unroll
        for (int i = 0; i < kWords; ++i) {
            const int idx = i * NT + tid;
            const int sb = idx >> 13, rem = idx & 8191;
            const int c = rem >> 6, w = rem & 63;
            *reinterpret_cast<uint2*>(xa0 + (sb * kBN + c) * kXStride + 4 * w) = i8x4_to_h4((uint32_t)xw[i]);
        }
        if (tid < NG * kBN) {
            const int sb = tid >> 7, c = tid & 127;
            if (!Q6) {  // [B>>6 of 0-3 | of 4-7 | B&63 of 0-3 | of 4-7]
                h8 mlo, mhi;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int hb = (xp[j >> 2] << (24 - 8 * (j & 3))) >> 24;  // signed byte
                    const int lb = (xp[2 + (j >> 2)] >> (8 * (j & 3))) & 255;
                    mlo[j] = (_Float16)(float)(64 * hb);
                    mhi[j] = (_Float16)(float)lb;
                }
                *reinterpret_cast<h8*>(xm0 + (sb * kBN + c) * 16) = mlo;
                *reinterpret_cast<h8*>(xm0 + (sb * kBN + c) * 16 + 8) = mhi;
            }
            xd0[sb * kBN + c] = xdv;
        }
        __syncthreads();
        const int s = NG * it + grp;  // this wavefront's super-block
        const bool active = s < nsb;
        wcur = wnext;
        wcur.decode();
        if (it + 1 < iters) {
            fetchX(it + 1);
            if (s + NG < nsb) wnext.load(qw, row, rows_stream, ngroups, s + NG, h);
        }
        if constexpr (!Q6 && NG == 2) {
          if (active) {
            // Q4_K with two wavefronts per SIMD: the super-block's 16 weight fragments are
            // dequantized first (64 registers), then each column block runs its 16 MFMAs into one
            // accumulator and is combined at once, so only one block's partial sums are live.
            h8 bwa[16];
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int j = t >> 1, u = t & 1;
                bwa[t] = dequant8(wcur.qs[j >> 1][u], j & 1, wcur.sc(j));
            }
            h8 bm;
#pragma unroll
            for (int e = 0; e < 8; ++e) bm[e] = wcur.m(e);
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                f16v isb = zero;
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    const h8 av = *reinterpret_cast<const h8*>(xa + (cb * 32 + l32) * kXStride + 16 * t + 8 * h);
                    isb = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bwa[t], isb, 0, 0, 0);
                }
                const h8 am = *reinterpret_cast<const h8*>(xm + (cb * 32 + l32) * 16 + 8 * h);
                const f16v im = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, zero, 0, 0, 0);
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const float4 xd4 = *reinterpret_cast<const float4*>(xdl + cb * 32 + q4 * 8 + h * 4);
                    const float xdv4[4] = {xd4.x, xd4.y, xd4.z, xd4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int i = 4 * q4 + e;
                        const float t2 = __builtin_fmaf(-wcur.dmin, im[i], wcur.d * isb[i]);
                        acc[cb][i] = __builtin_fmaf(xdv4[e], t2, acc[cb][i]);
                    }
                }
            }
          }
        } else if (active) {
            f16v is[4];
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                h8 av[4];
#pragma unroll
                for (int cb = 0; cb < 4; ++cb)
                    av[cb] = *reinterpret_cast<const h8*>(xa + (cb * 32 + l32) * kXStride + 16 * t + 8 * h);
                if constexpr (Q6) {
                    h8 b1, b2;
                    wcur.dequant(t, b1, b2);
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb) {
                        is[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[cb], b1, t == 0 ? zero : is[cb], 0, 0, 0);
                        is[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[cb], b2, is[cb], 0, 0, 0);
                    }
                } else {
                    const int j = t >> 1, u = t & 1;
                    const h8 bw = dequant8(wcur.qs[j >> 1][u], j & 1, wcur.sc(j));
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb)
                        is[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[cb], bw, t == 0 ? zero : is[cb], 0, 0, 0);
                }
            }
            h8 bm;
            if constexpr (!Q6) {
#pragma unroll
                for (int e = 0; e < 8; ++e) bm[e] = wcur.m(e);
            }
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                f16v im;
                if constexpr (!Q6) {
                    const h8 am = *reinterpret_cast<const h8*>(xm + (cb * 32 + l32) * 16 + 8 * h);
                    im = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, zero, 0, 0, 0);
                }
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const float4 xd4 = *reinterpret_cast<const float4*>(xdl + cb * 32 + q4 * 8 + h * 4);
                    const float xdv4[4] = {xd4.x, xd4.y, xd4.z, xd4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int i = 4 * q4 + e;
                        if constexpr (Q6) {
                            acc[cb][i] = __builtin_fmaf(wcur.d * xdv4[e], is[cb][i], acc[cb][i]);
                        } else {
                            const float t2 = __builtin_fmaf(-wcur.dmin, im[i], wcur.d * is[cb][i]);
                            acc[cb][i] = __builtin_fmaf(xdv4[e], t2, acc[cb][i]);
                        }
                    }
                }
            }
        }
        __syncthreads();  // the next iteration overwrites the staged activations
    }
    // ---- group 1 hands its partial sums to group 0 through LDS (the activations are done)
    float* red = reinterpret_cast<float*>(lds4);
    if (NG == 2 && grp == 1)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i) red[((wr * 64 + lane) * 4 + cb) * 16 + i] = acc[cb][i];
    if (NG == 2) __syncthreads();
    if (grp == 0 && row < rows) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int c = col0 + cb * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
                const float v = NG == 2 ? acc[cb][i] + red[((wr * 64 + lane) * 4 + cb) * 16 + i] : acc[cb][i];
                if (c < ncols) y[(size_t)c * rows + row] = v;
            }
    }
}

template <bool Q6, int NG>
int runMfma8(const kcMatmulKQ8Args& a, hipStream_t s) {
    static const int attr = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(matmul_kq_mfma8_kernel<Q6, NG>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, NG * kLdsGrp);
    if (attr != 0) return fromHip(attr, "matmul (MFMA): LDS size");
    const dim3 grid((a.rows + kBM - 1) / kBM, (a.ncols + kBN - 1) / kBN);
    hipLaunchKernelGGL((matmul_kq_mfma8_kernel<Q6, NG>), grid, dim3(256 * NG), NG * kLdsGrp, s,
                       reinterpret_cast<const uint8_t*>(a.qw), a.xq, a.y, a.rows, a.k / 256, a.ncols);
    return fromHip(hipGetLastError(), Q6 ? "matmul_q6k_q8k (MFMA)" : "matmul_q4k_q8k (MFMA)");
}

// ---------------------------------------------------------------- fp16-activation variant
// The activations are first converted once per matmul to fp16 (act[c][k]; for Q4_K also the mins
// operand of every (column, super-block), act_to_f16_kernel), so the matmul stages them with
// direct global-to-LDS loads (no registers, no per-workgroup conversion) into a double-buffered
// LDS tile: super-block s + 1 streams in while s is computed. A column's 256 values (32 chunks of
// 16 B) sit 528 B apart (one chunk of padding), so the 16 columns read by a quarter-wavefront's
// ds_read_b128 start 16 B apart modulo 256 B (no bank conflicts) and every read of a lane is its
// base plus an immediate offset. One direct load fills 1 KB (64 lanes x 16 B) and each lane picks
// the chunk of that layout it fetches: 66 loads fill a stage (pad chunks re-read chunk 0).
// Each wavefront computes 32 weight rows x 128 columns (four 32 x 32 blocks); the A operands of
// K-step t + 1 are read while K-step t runs.

// act[c][s * 256 ..] = the 256 int8 activations of super-block s of column c, as fp16; for Q4_K,
// mins[c][s][16] = [64 (B_j >> 6) for j < 8 | B_j & 63 for j < 8] (B_j = sum of the 32 values of
// sub-block j, the reference's byte split); xdT[s][c] = the scale of column c's super-block s
// (0 for the padding columns ncols <= c < ncp).
// One thread per 16 activations of a column (four slot words in, 32 bytes out), and per entry of
// xdT and of the min operands; 32-bit indices (the launcher keeps ncols * k * 2 below 2^32).
__global__ void act_to_f16_kernel(const int* __restrict__ xq, uint4* __restrict__ act, h8* __restrict__ mins,
                                  float* __restrict__ xdT, int nsb, unsigned quads, int ncols, int ncp) {
    const unsigned i = blockIdx.x * 256u + threadIdx.x;
    const unsigned per = (unsigned)nsb * 16u;  // 16-value groups per column
    if (i < quads) {
        const unsigned c = i / per, w = (i - c * per) * 4u;
        const int* src = xq + (size_t)c * nsb * 85 + w;
        const uint2 a0 = i8x4_to_h4x16((uint32_t)src[0]), a1 = i8x4_to_h4x16((uint32_t)src[1]);
        const uint2 a2 = i8x4_to_h4x16((uint32_t)src[2]), a3 = i8x4_to_h4x16((uint32_t)src[3]);
        act[2 * (size_t)i] = make_uint4(a0.x, a0.y, a1.x, a1.y);
        act[2 * (size_t)i + 1] = make_uint4(a2.x, a2.y, a3.x, a3.y);
    }
    if (i < (unsigned)nsb * (unsigned)ncp) {
        const unsigned sx = i / (unsigned)ncp, c = i - sx * (unsigned)ncp;
        xdT[i] = (int)c < ncols ? reinterpret_cast<const float*>(xq + (size_t)c * nsb * 85 + nsb * 64)[sx] : 0.0f;
    }
    if (mins && i < (unsigned)ncols * (unsigned)nsb) {
        const unsigned c = i / (unsigned)nsb, sx = i - c * (unsigned)nsb;
        const int* pw = xq + (size_t)c * nsb * 85 + nsb * 81 + sx * 4;
        const int w0 = pw[0], w1 = pw[1], w2 = pw[2], w3 = pw[3];
        h8 lo, hi;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int hb = ((j < 4 ? w0 : w1) << (24 - 8 * (j & 3))) >> 24;
            const int lb = ((j < 4 ? w2 : w3) >> (8 * (j & 3))) & 255;
            lo[j] = (_Float16)(float)(64 * hb);
            hi[j] = (_Float16)(float)lb;
        }
        mins[2 * (size_t)i] = lo;
        mins[2 * (size_t)i + 1] = hi;
    }
}

constexpr int kColB = 528;  // bytes per column in LDS: 32 chunks + 1 pad chunk

// The fp16-activation kernel's view of 32 weight rows for one super-block, loaded in whole 16-byte
// chunks: lane -> row lane % 32 and half h = lane / 32, which takes chunk h of every pair of slabs
// (a wavefront waits about as long for the memory unit to take a 16-byte load as an 8-byte one).
// K-step t then covers, in lane half h, the 8 values at k = 64 (t >> 2) + 32 ((t >> 1) & 1) + 16 h
// + 8 (t & 1) (qs bytes 32 (t >> 2) + 16 h + 8 (t & 1) .., nibble (t >> 1) & 1, sub-block t >> 1):
// the A operand reads the activation chunk at byte 64 (t >> 1) + 32 h + 16 (t & 1) of the column,
// so both operands of a step pair the same k.
struct Rows32W {
    uint4 q16[4];  // [a]: qs bytes 32a + 16h .. +15
    uint4 hdr;     // d, dmin (fp16) and the 12 packed scale / min bytes
    float d, dmin;
    int scw[2], mw[2];
    __device__ __forceinline__ void load(const uint8_t* qw, int row, int rows_stream, int ngroups, int s, int h) {
        const bool live = row < rows_stream;
        const int rr = live ? row : 0;
        const int tile = rr >> 4, r = rr & 15, g = s >> 2, kq = s & 3;
        const uint8_t* piece = qw + ((size_t)tile * ngroups + g) * kQ4kSeg + (kq * 16 + r) * 16;
        hdr = *reinterpret_cast<const uint4*>(piece);
#pragma unroll
        for (int a = 0; a < 4; ++a) q16[a] = *reinterpret_cast<const uint4*>(piece + (1 + 2 * a + h) * 1024);
    }
    __device__ __forceinline__ void decode() {
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
    // the 8 bytes of K-step t
    __device__ __forceinline__ uint2 bytes(int t) const {
        const uint4 q = q16[t >> 2];
        return (t & 1) ? make_uint2(q.z, q.w) : make_uint2(q.x, q.y);
    }
};

// Q6_K rows loaded in whole chunks (see Rows32W): K-step t covers, in lane half h, the 8 values
// k = 128 n + 32 quad + 16 h + 8 p (n = t >> 3, quad = (t >> 1) & 3, p = t & 1): ql bytes
// 64 n + 32 (quad & 1) + 16 h + 8 p .. (nibble quad >> 1), qh bytes 32 n + 16 h + 8 p .. (bits
// 2 quad), scale of sub-block 8 n + 2 quad + h (so the two lane halves of a step scale by different
// sub-blocks); the activation chunk is again at byte 64 (t >> 1) + 32 h + 16 p of the column.
struct Rows32Q6W {
    uint4 ql16[2][2];  // [n][a]: ql bytes 64n + 32a + 16h .. +15
    uint4 qh16[2];     // [n]: qh bytes 32n + 16h .. +15
    int sw[4];         // the 16 int8 scales
    uint32_t dbits;    // d (fp16)
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
            for (int a = 0; a < 2; ++a) ql16[n][a] = *reinterpret_cast<const uint4*>(piece + (4 * n + 2 * a + h) * 1024);
#pragma unroll
        for (int n = 0; n < 2; ++n) qh16[n] = *reinterpret_cast<const uint4*>(piece + (8 + 2 * n + h) * 1024);
        const uint4 sc = *reinterpret_cast<const uint4*>(piece + 12 * 1024);
        sw[0] = (int)sc.x;
        sw[1] = (int)sc.y;
        sw[2] = (int)sc.z;
        sw[3] = (int)sc.w;
        dbits = *reinterpret_cast<const uint16_t*>(seg + kQ6kSlabs * 1024 + (kq * 16 + r) * 2);
    }
    __device__ __forceinline__ void decode() { d = (float)__builtin_bit_cast(_Float16, (unsigned short)dbits); }
    // K-step t for activations 16 x, as Rows32Q6::dequantA16: sh (q - 32) and sl (q - 32) / 16.
    __device__ __forceinline__ void dequantA16(int t, int h, h8& b1, h8& b2) const {
        const int n = t >> 3, quad = (t >> 1) & 3, p = t & 1;
        const uint4 L = ql16[n][quad & 1], H = qh16[n];
        const uint32_t lw[2] = {p ? L.z : L.x, p ? L.w : L.y}, hw[2] = {p ? H.z : H.x, p ? H.w : H.y};
        const int w = sw[2 * n + (quad >> 1)];
        const int bi = 2 * (quad & 1) + h;  // this lane half's sub-block within the scale word
        const int sh = (w << (24 - 8 * bi)) >> 28, sl = (w >> (8 * bi)) & 15;
        const _Float16 fh = (_Float16)(short)sh, fl = (_Float16)(short)sl;
        const h2 mh = {fh, fh}, ml = {fl * (_Float16)0.0625f, fl * (_Float16)0.0625f};
        const h2 ch = {fh * (_Float16)(-1056.0f), fh * (_Float16)(-1056.0f)};
        const h2 cl = {fl * (_Float16)(-66.0f), fl * (_Float16)(-66.0f)};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t q = ((lw[i] >> (4 * (quad >> 1))) & 0x0F0F0F0Fu) | (((hw[i] >> (2 * quad)) & 0x03030303u) << 4);
            const h2 a = bits_h2(__builtin_amdgcn_perm(0x64646464u, q, 0x04010400u));  // 1024 + q
            const h2 b = bits_h2(__builtin_amdgcn_perm(0x64646464u, q, 0x04030402u));
            const h2 a1 = __builtin_elementwise_fma(a, mh, ch), b1v = __builtin_elementwise_fma(b, mh, ch);
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

// LDS geometry of the fp16-activation kernel with CB column blocks of 32 per wavefront and NW
// wavefronts per workgroup (every wavefront of a workgroup covers the same 32 CB columns, each its
// own 32 weight rows, so a workgroup stages each activation tile once for 32 NW rows).
template <int CB, int NW>
struct HGeo {
    static constexpr int kCols = 32 * CB;                   // activation columns per workgroup
    static constexpr int kRows = 32 * NW;                   // weight rows per workgroup
    static constexpr int kActLoads = kCols * 33 / 64;       // direct loads of 1 KB per stage
    static constexpr int kActB = kActLoads * 1024;          // the stage's activation tile
    static constexpr int kPerWave = (kActLoads + NW - 1) / NW;  // loads per wavefront (the last ones repeat)
    static constexpr int kMinB = kCols * 32;                // Q4_K min operands
    static constexpr int kBuf = kActB + kMinB + 1024;       // + column scales (one 1 KB load)
    static constexpr int kLds = 2 * kBuf;
};

// Eight 4-bit weights (nibble hiNib of 8 bytes) times a sub-block scale: m2 / s2 precomputed.
__device__ __forceinline__ h8 dequant8s(uint2 q, bool hiNib, h2 m2, h2 s2) {
    const uint32_t mask = hiNib ? 0xFFF0FFF0u : 0xFF0FFF0Fu;
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

// Buffer resources of the three staged arrays (raw buffers: the hardware checks every offset
// against the byte size and returns zero past it).
typedef __attribute__((address_space(3))) void* LdsPtr;
struct HRes {
    __amdgpu_buffer_rsrc_t act, mins, xd;
};
__device__ __forceinline__ __amdgpu_buffer_rsrc_t bufRes(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Direct loads of super-block s into stage buffer buf: the activation tile (goff = this lane's
// byte offsets of its loads in act at super-block 0), the Q4_K min operands and the column scales.
// They are buffer loads into LDS rather than global_load_lds: the compiler counts the latter as
// possibly LDS-side operations and then waits for every LDS read in flight (lgkmcnt(0)) before
// each use, which serializes the A-operand reads of the K loop with the matrix ops.
// (wave is wavefront-uniform: the loads past the activation tile are issued by single wavefronts.)
template <bool Q6, int CB, int NW>
__device__ __forceinline__ void stageH(char* buf, const HRes& rs, const uint32_t (&goff)[HGeo<CB, NW>::kPerWave],
                                       int s, int wave, int lane, int col0, int ncols, int nsb, int ncp) {
    using G = HGeo<CB, NW>;
#pragma unroll
    for (int r = 0; r < G::kPerWave; ++r) {
        const int g = min(r * NW + wave, G::kActLoads - 1);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.act, (LdsPtr)(buf + g * 1024), 16, goff[r], (uint32_t)s * 512u, 0,
                                                 0);
    }
    if constexpr (!Q6) {  // 32 columns per load, by wavefronts NW - CB .. NW - 1
        const int wq = wave - (NW - CB);
        if (wq >= 0) {
            const int p = wq * 64 + lane, c = p >> 1;
            const int cc = col0 + c < ncols ? col0 + c : 0;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.mins, (LdsPtr)(buf + G::kActB + wq * 1024), 16,
                                                     (uint32_t)(((cc * nsb + s) * 16 + (p & 1) * 8) * 2), 0, 0, 0);
        }
    }
    // the column scales: one wavefront writes the 1 KB (lanes past the tile repeat)
    if (wave == 0)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs.xd, (LdsPtr)(buf + G::kActB + G::kMinB), 16,
                                                 (uint32_t)((s * ncp + col0 + ((lane & 31) % (8 * CB)) * 4) * 4), 0, 0,
                                                 0);
}

// One workgroup's tile: weight rows rowTile * 32 NW .., columns colTile * 32 CB .., super-blocks
// [sb0, sb1) of the nsb (y = the partial sum over that range).
template <bool Q6, int CB, int NW>
__device__ __forceinline__ void hTile(char* lbase, const uint8_t* __restrict__ qw, const _Float16* __restrict__ act,
                                      const _Float16* __restrict__ mins, const float* __restrict__ xdT,
                                      float* __restrict__ y, int rows, int nsb, int ncols, int ncp, int rowTile,
                                      int colTile, int sb0, int sb1) {
    using G = HGeo<CB, NW>;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, l32 = lane & 31;
    const int row = rowTile * G::kRows + wave * 32 + l32;
    const int col0 = colTile * G::kCols;
    const int ngroups = (nsb + kGroupSb - 1) / kGroupSb;
    const int rows_stream = ((rows + kTileRows - 1) / kTileRows) * kTileRows;
    const int k = nsb * 256;
    const HRes rs{bufRes(act, (uint32_t)ncols * (uint32_t)k * 2u), bufRes(mins, (uint32_t)ncols * (uint32_t)nsb * 32u),
                  bufRes(xdT, (uint32_t)nsb * (uint32_t)ncp * 4u)};

    // this lane's byte offset into act of each of its direct loads (super-block 0); columns past
    // ncols read column 0
    uint32_t goff[G::kPerWave];
#pragma unroll
    for (int r = 0; r < G::kPerWave; ++r) {
        const int g = min(r * NW + wave, G::kActLoads - 1);
        const int slot = g * 64 + lane, c = slot / 33, kc = slot - 33 * c;
        const int cc = col0 + c < ncols ? col0 + c : 0;
        goff[r] = (uint32_t)cc * (uint32_t)k * 2u + (uint32_t)(kc == 32 ? 0 : kc) * 16u;
    }

    f16v acc[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[cb][i] = 0.0f;
    const f16v zero = acc[0];
    using Rows = typename std::conditional<Q6, Rows32Q6W, Rows32W>::type;
    Rows wcur, wnext;
    stageH<Q6, CB, NW>(lbase, rs, goff, sb0, wave, lane, col0, ncols, nsb, ncp);
    wnext.load(qw, row, rows_stream, ngroups, sb0, h);
    // this lane's A-operand byte offset in a stage for column block cb (K-step t adds
    // 64 (t >> 1) + 16 (t & 1), the k-order of Rows32W / Rows32Q6W)
    int aoff[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) aoff[cb] = (cb * 32 + l32) * kColB + h * 32;

    // A wavefront waits at each vector-memory instruction until the CU's memory unit takes it (about
    // 20 cycles per instruction and CU, whatever its width), so a burst of loads stalls its issuer.
    // With 8 wavefronts the two of a SIMD (w, w + 4) leave the barrier together: the second one
    // issues its loads at K-step 8 instead, so one of them computes while the other waits.
    const bool late = NW == 8 && wave >= NW / 2;
    for (int s = sb0; s < sb1; ++s) {
        const int b = (s - sb0) & 1;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wavefront's loads of stage s
        __syncthreads();  // everyone's: stage s is complete, stage b ^ 1 is no longer read
        wcur = wnext;
        wcur.decode();
        if (s + 1 < sb1 && !late) {
            stageH<Q6, CB, NW>(lbase + (b ^ 1) * G::kBuf, rs, goff, s + 1, wave, lane, col0, ncols, nsb, ncp);
            wnext.load(qw, row, rows_stream, ngroups, s + 1, h);
        }
        const char* buf = lbase + b * G::kBuf;
        f16v is[CB];
        h2 m2[8], s2[8];  // Q4_K: per sub-block (1024 + q) -> sc * q constants
        if constexpr (!Q6) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // sc q / 16 (the activations are 16 x): (1024 + q) sc / 16 - 64 sc for a low nibble,
                // (1024 + 16 q) sc / 256 - 4 sc for a high one; exact (sc / 256 >= 2^-8, q sc <= 945)
                const _Float16 sc = wcur.sc(j);
                const bool hiNib = j & 1;
                const _Float16 mul = hiNib ? sc * (_Float16)0.00390625f : sc * (_Float16)0.0625f;
                const _Float16 sub = hiNib ? sc * (_Float16)(-4.0f) : sc * (_Float16)(-64.0f);
                m2[j] = h2{mul, mul};
                s2[j] = h2{sub, sub};
            }
        }
        // Software pipeline over the 16 K-steps: step t runs its matrix ops while the B operand of
        // t + 1 is dequantized and the A operand of t + 1 is read from LDS (no dependence between
        // the three, so the scheduler interleaves them; the barrier keeps each step's reads ahead).
        h8 av[CB], an[CB];
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) av[cb] = *reinterpret_cast<const h8*>(buf + aoff[cb]);
        h8 bq, bq2, bn, bn2;  // B operands of steps t and t + 1 (Q6_K: two per step)
        if constexpr (Q6)
            wcur.dequantA16(0, h, bq, bq2);
        else
            bq = dequant8s(wcur.bytes(0), false, m2[0], s2[0]);
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            if (t + 1 < 16) {
                const int tn = t + 1, toff = 64 * (tn >> 1) + 16 * (tn & 1);
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) an[cb] = *reinterpret_cast<const h8*>(buf + aoff[cb] + toff);
                if constexpr (Q6) {
                    wcur.dequantA16(tn, h, bn, bn2);
                } else {
                    const int j = tn >> 1;  // sub-block (nibble j & 1 of the step's bytes)
                    bn = dequant8s(wcur.bytes(tn), j & 1, m2[j], s2[j]);
                }
            }
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                is[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[cb], bq, t == 0 ? zero : is[cb], 0, 0, 0);
                if constexpr (Q6) is[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[cb], bq2, is[cb], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (late && t == 8 && s + 1 < sb1) {
                stageH<Q6, CB, NW>(lbase + (b ^ 1) * G::kBuf, rs, goff, s + 1, wave, lane, col0, ncols, nsb, ncp);
                wnext.load(qw, row, rows_stream, ngroups, s + 1, h);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (t + 1 < 16) {
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) av[cb] = an[cb];
                bq = bn;
                if constexpr (Q6) bq2 = bn2;
            }
        }
        h8 bm;
        if constexpr (!Q6) {
#pragma unroll
            for (int e = 0; e < 8; ++e) bm[e] = wcur.m(e);
        }
        const _Float16* xm = reinterpret_cast<const _Float16*>(buf + G::kActB);
        const char* xdl = buf + G::kActB + G::kMinB;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            f16v im;
            if constexpr (!Q6) {
                const h8 am = *reinterpret_cast<const h8*>(xm + (cb * 32 + l32) * 16 + 8 * h);
                im = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, zero, 0, 0, 0);
            }
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                // (an ext_vector read: HIP's float4 struct here made the compiler wait for the
                // direct loads in flight before this read)
                const h8 xd8 = *reinterpret_cast<const h8*>(xdl + (cb * 32 + q4 * 8 + h * 4) * 4);
                const u32v4 xdw = __builtin_bit_cast(u32v4, xd8);
                float xdv4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t wv = xdw[e];
                    xdv4[e] = __builtin_bit_cast(float, wv);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = 4 * q4 + e;
                    if constexpr (Q6) {
                        acc[cb][i] = __builtin_fmaf(wcur.d * xdv4[e], is[cb][i], acc[cb][i]);
                    } else {
                        const float t2 = __builtin_fmaf(-wcur.dmin, im[i], wcur.d * is[cb][i]);
                        acc[cb][i] = __builtin_fmaf(xdv4[e], t2, acc[cb][i]);
                    }
                }
            }
        }
    }
    if (row < rows) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int c = col0 + cb * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
                if (c < ncols) y[(size_t)c * rows + row] = acc[cb][i];
            }
    }
}

using HPart = MfmaPart;
using HGroup = MfmaGroup;

template <int NW>
__global__ __launch_bounds__(64 * NW) void matmul_kq_mfma_h_kernel(HGroup g, const _Float16* __restrict__ act,
                                                                   const _Float16* __restrict__ mins,
                                                                   const float* __restrict__ xdT, int nsb, int ncols,
                                                                   int ncp) {
    extern __shared__ int4 lds4[];
    char* lbase = reinterpret_cast<char*>(lds4);
    const int bx = blockIdx.x;
    const int pi = (g.nparts > 2 && bx >= g.p[2].tile0) ? 2 : (g.nparts > 1 && bx >= g.p[1].tile0) ? 1 : 0;
    const HPart& p = g.p[pi];
    const int z = blockIdx.z, sb0 = z * nsb / g.ks, sb1 = (z + 1) * nsb / g.ks;
    if (p.q6)
        hTile<true, 2, NW>(lbase, p.qw, act, mins, xdT, p.y[z], p.rows, nsb, ncols, ncp, bx - p.tile0, blockIdx.y, sb0,
                           sb1);
    else
        hTile<false, 2, NW>(lbase, p.qw, act, mins, xdT, p.y[z], p.rows, nsb, ncols, ncp, bx - p.tile0, blockIdx.y, sb0,
                            sb1);
}

// The fp16 activation buffer: ncols * k halves, then (Q4_K) ncols * nsb * 16 halves of mins, then
// nsb * ncp floats of column scales (ncp = ncols rounded up to whole 128-column tiles).
int actCols(int ncols) { return (ncols + 127) / 128 * 128; }
size_t actBytes(int ncols, int k) {
    return (size_t)ncols * k * 2 + (size_t)ncols * (k / 256) * 32 + (size_t)(k / 256) * actCols(ncols) * 4;
}

// Wavefronts per workgroup of the fp16-activation kernel for a grid of wgs8 workgroups of 8
// (option matmul_waves: 4, 8, or 0 = by the grid). 8 wavefronts (256 weight rows, one workgroup
// per CU) stage each activation tile once per CU instead of once per 128 rows and stagger their
// loads; they are taken when their grid fills the CUs in whole rounds or fits in one.
// Whether runMfmaH runs a matrix of this type on the producer-wavefront kernel.
bool wsRuns(bool q6) {
    const int ws = option("matmul_ws"), path = option("matmul_path");
    return ws != 1 && !(ws == 3 && q6) && (path == 0 || path == 2);
}

int hWaves(long long wgs8) {
    const int o = option("matmul_waves");
    if (option("matmul_path") == 7 || o == 4) return 4;
    if (o == 8) return 8;
    const long long cus = cuCount();
    return wgs8 <= cus || wgs8 % cus == 0 ? 8 : 4;
}

// Whether the producer-wavefront kernel splits the Q6_K parts of group g over K (on top of a group
// split of one): a Q4_K part beside a Q6_K one given a second output, at least two super-blocks,
// option matmul_split6 not 1.
bool splitsQ6(const MfmaGroup& g, int nparts, int nsb) {
    bool q4 = false, q6 = false;
    for (int i = 0; i < nparts; ++i) {
        q4 |= !g.p[i].q6;
        q6 |= g.p[i].q6 && g.p[i].y[1];
    }
    return q4 && q6 && nsb >= 2 && option("matmul_split6") != 1;
}

// The fp16-activation kernel over parts[0..nparts) (one conversion of the activations), K split
// into ks ranges.
int runMfmaH(const MmPart* parts, int nparts, const int* xq, int k, int ncols, int ks, void* act, hipStream_t s,
             const ActF16* pre = nullptr, int* part_ks = nullptr) {
    if (part_ks)
        for (int i = 0; i < nparts; ++i) part_ks[i] = ks;
    using G = HGeo<2, 4>;  // (the LDS geometry does not depend on the wavefront count)
    static const int attr4 = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(matmul_kq_mfma_h_kernel<4>),
                                                      hipFuncAttributeMaxDynamicSharedMemorySize, G::kLds);
    static const int attr8 = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(matmul_kq_mfma_h_kernel<8>),
                                                      hipFuncAttributeMaxDynamicSharedMemorySize, G::kLds);
    if (attr4 != 0 || attr8 != 0) return fromHip(attr4 ? attr4 : attr8, "matmul (MFMA): LDS size");
    const int nsb = k / 256;
    long long tiles8 = 0;
    for (int i = 0; i < nparts; ++i) tiles8 += (parts[i].rows + 255) / 256;
    // the producer-wavefront kernel (256-row tiles) unless option matmul_ws = 1 (3: for Q4_K-only
    // groups, a group with a Q6_K matrix on the kernel above)
    bool ws = true;
    for (int i = 0; i < nparts; ++i) ws = ws && wsRuns(parts[i].q6 != 0);
    const int nw = ws ? 8 : hWaves(tiles8 * ((ncols + G::kCols - 1) / G::kCols) * ks);
    const int wg_rows = ws ? mfmaWsRows() : 32 * nw;
    HGroup g{};
    bool any_q4 = false;
    int tiles = 0;
    for (int i = 0; i < nparts; ++i) {
        g.p[i] = HPart{static_cast<const uint8_t*>(parts[i].qw), {parts[i].y[0], parts[i].y[1]}, parts[i].rows,
                       parts[i].q6, tiles};
        tiles += (parts[i].rows + wg_rows - 1) / wg_rows;
        any_q4 |= !parts[i].q6;
    }
    g.nparts = nparts;
    g.ks = ks;
    // slots handed over (no quantizer-written fp16 operands) to Q4_K matrices: the producer
    // wavefronts convert them themselves, unless option matmul_ws = 2 (a conversion launch first,
    // as for the other kernels and for Q6_K)
    bool all_q4 = true;
    for (int i = 0; i < nparts; ++i) all_q4 = all_q4 && !parts[i].q6;
    if (ws && all_q4 && !pre && option("matmul_ws") != 2 && option("matmul_path") != 7 && mfmaWsSlotsFits(nsb) &&
        mfmaWsFits(g, nsb, ncols))
        return launchMfmaWsSlots(g, tiles, xq, nsb, ncols, s);
    const long long words = (long long)ncols * nsb * 64;
    _Float16* mins;
    float* xdT;
    int ncp;
    if (pre) {  // written by the quantizer
        act = pre->act;
        mins = static_cast<_Float16*>(pre->mins);
        xdT = pre->xdT;
        ncp = pre->ncp;
    } else {
        mins = static_cast<_Float16*>(act) + (size_t)ncols * k;
        xdT = reinterpret_cast<float*>(mins + (size_t)ncols * nsb * 16);
        ncp = actCols(ncols);
        const long long quads = words / 4, threads = std::max(quads, (long long)nsb * ncp);
        hipLaunchKernelGGL(act_to_f16_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, xq,
                           static_cast<uint4*>(act), any_q4 ? reinterpret_cast<h8*>(mins) : nullptr, xdT, nsb,
                           (unsigned)quads, ncols, ncp);
    }
    if (option("matmul_path") == 7)  // the wide-tile kernel (every weight dequantized once per workgroup)
        return launchMfmaW(g, tiles, act, mins, xdT, nsb, ncols, ncp, s);
    if (ws && mfmaWsFits(g, nsb, ncols)) {
        // A Q6_K part among Q4_K ones runs twice the matrix ops per super-block (its split scale), so
        // its workgroups would end long after the others': given a second output (y[1]) and a caller
        // that takes per-part splits (part_ks), it runs in two K ranges when the group has one
        // (option matmul_split6 = 1: never).
        // Each part then owns ks x its row tiles of blockIdx.x (no idle workgroups).
        if (part_ks && ks == 1 && splitsQ6(g, nparts, nsb)) {
            tiles = 0;
            for (int i = 0; i < nparts; ++i) {
                g.p[i].ntiles = (parts[i].rows + wg_rows - 1) / wg_rows;
                g.p[i].ks = parts[i].q6 && parts[i].y[1] ? 2 : 1;
                g.p[i].tile0 = tiles;
                tiles += g.p[i].ks * g.p[i].ntiles;
                part_ks[i] = g.p[i].ks;
            }
        }
        return launchMfmaWs(g, tiles, act, mins, xdT, nsb, ncols, ncp, s);
    }
    if (ws) {  // beyond the 32-bit offsets: the 8-wavefront kernel over the same 256-row tiles
        const dim3 grid(tiles, (ncols + G::kCols - 1) / G::kCols, ks);
        hipLaunchKernelGGL(matmul_kq_mfma_h_kernel<8>, grid, dim3(512), G::kLds, s, g,
                           static_cast<const _Float16*>(act), mins, xdT, nsb, ncols, ncp);
        return fromHip(hipGetLastError(), "matmul_q4k/q6k_q8k (MFMA)");
    }
    const dim3 grid(tiles, (ncols + G::kCols - 1) / G::kCols, ks);
    if (nw == 8)
        hipLaunchKernelGGL(matmul_kq_mfma_h_kernel<8>, grid, dim3(512), G::kLds, s, g,
                           static_cast<const _Float16*>(act), mins, xdT, nsb, ncols, ncp);
    else
        hipLaunchKernelGGL(matmul_kq_mfma_h_kernel<4>, grid, dim3(256), G::kLds, s, g,
                           static_cast<const _Float16*>(act), mins, xdT, nsb, ncols, ncp);
    return fromHip(hipGetLastError(), "matmul_q4k/q6k_q8k (MFMA)");
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

// y += p over n floats (the second K half of a split launch): four per thread (both arrays 16-byte
// aligned, as the launcher checks), the last n % 4 one each.
__global__ void add_partial_kernel(float* __restrict__ y, const float* __restrict__ p, long long n) {
    const long long i = blockIdx.x * 256LL + threadIdx.x, i4 = 4 * i;
    if (i4 + 3 < n) {
        float4 a = reinterpret_cast<const float4*>(y)[i];
        const float4 b = reinterpret_cast<const float4*>(p)[i];
        a.x += b.x;
        a.y += b.y;
        a.z += b.z;
        a.w += b.w;
        reinterpret_cast<float4*>(y)[i] = a;
    } else {
        for (long long j = i4; j < n; ++j) y[j] += p[j];
    }
}
// The same one float per thread (y not 16-byte aligned).
__global__ void add_partial1_kernel(float* __restrict__ y, const float* __restrict__ p, long long n) {
    const long long i = blockIdx.x * 256LL + threadIdx.x;
    if (i < n) y[i] += p[i];
}

// A by-name launch on the fp16-activation kernel: a grid under two workgroups of 4 wavefronts per
// CU splits K in two, the second half's partial sums staged after the activations and added into
// y by one more kernel (fl(a + b): the same for either order).
int stagedKs(bool q6k, const kcMatmulKQ8Args& a) { return matmulKs(a.rows, a.k, a.ncols, q6k); }
size_t stagedActBytes(const kcMatmulKQ8Args& a) { return (actBytes(a.ncols, a.k) + 255) & ~size_t(255); }
size_t stagedBytes(const kcMatmulKQ8Args& a, int ks) {
    return stagedActBytes(a) + (ks == 2 ? (size_t)a.rows * a.ncols * 4 : 0);
}
int runStaged(bool q6k, const kcMatmulKQ8Args& a, int ks, void* buf, hipStream_t s) {
    float* partial = ks == 2 ? reinterpret_cast<float*>(static_cast<char*>(buf) + stagedActBytes(a)) : nullptr;
    const MmPart part{a.qw, {a.y, partial}, a.rows, q6k ? 1 : 0};
    if (int st = runMfmaH(&part, 1, a.xq, a.k, a.ncols, ks, buf, s)) return st;
    if (ks == 1) return 0;
    const long long n = (long long)a.rows * a.ncols;
    if (reinterpret_cast<uintptr_t>(a.y) % 16 == 0)  // (the partial sums are 256-byte aligned)
        hipLaunchKernelGGL(add_partial_kernel, dim3((unsigned)((n / 4 + 1 + 255) / 256)), dim3(256), 0, s, a.y, partial,
                           n);
    else
        hipLaunchKernelGGL(add_partial1_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a.y, partial, n);
    return fromHip(hipGetLastError(), "matmul (MFMA, K split): partial sum");
}

// ---- the fixed scratch of kcLaunchMatmulNoAlloc -----------------------------------------------
//
// The fp16 activations of one MFMA launch staged in a file-scope device array instead of the
// runtime's per-stream scratch, for callers that cannot allocate. Each GPU holds its own copy of
// the array until the process ends; its device address is looked up once per device when the
// runtime starts (hipGetSymbolAddress; the array's name is only a host-side stand-in and must never
// be passed to a kernel). Every call on a GPU shares it: calls that overlap on one GPU race. The
// conversion kernel rewrites every byte the matmul reads on each call, so nothing needs clearing.
constexpr size_t kFixedScratchBytes = size_t(16) << 20;
constexpr int kMaxDevices = 16;
static __device__ __align__(256) unsigned char scratch[kFixedScratchBytes];
void* g_fixed_scratch[kMaxDevices] = {};

}  // namespace

// The device's compute units (cached per device).
int cuCount() {
    static int cus[16] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

int fixedScratchInit(int device) {
    if (device < 0 || device >= kMaxDevices) return fromHip(hipErrorInvalidDevice, "fixed scratch: device index");
    void* p = nullptr;
    const hipError_t st = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (st != hipSuccess || !p) {
        g_fixed_scratch[device] = nullptr;
        return fromHip(st != hipSuccess ? st : hipErrorInvalidSymbol, "fixed scratch: hipGetSymbolAddress");
    }
    g_fixed_scratch[device] = p;
    return 0;
}

size_t fixedScratchBytes() { return kFixedScratchBytes; }

int launchMatmulKqNoAlloc(bool q6k, bool per256, const kcMatmulKQ8Args& a, hipStream_t s) {
    const int path = option("matmul_path");
    const bool mfma = per256 && (path >= 2 || (path == 0 && a.ncols >= 64));
    if (!mfma) return launchMatmulCols(q6k, per256, a, s);  // the column kernel stages nothing
    if (path == 3) return q6k ? runMfma<true>(a, s) : runMfma<false>(a, s);
    if (path == 4) return q6k ? runMfma8<true, 2>(a, s) : runMfma8<false, 2>(a, s);
    if (path == 5) return q6k ? runMfma8<true, 1>(a, s) : runMfma8<false, 1>(a, s);
    // the K split of launchMatmulMfma when its partial sums fit too, else one K range
    int ks = stagedKs(q6k, a);
    if (ks == 2 && stagedBytes(a, 2) > kFixedScratchBytes) ks = 1;
    const size_t need = stagedBytes(a, ks);
    if (need > kFixedScratchBytes) {
        setDetail("matmul (no-alloc): %d columns of %d values need %zu bytes of staging, above the fixed %zu "
                  "(ncols * k * 2 + ncols * k / 8 + k / 64 * ncols rounded up to 128)",
                  a.ncols, a.k, need, kFixedScratchBytes);
        return KC_ERROR_INVALID_VALUE;
    }
    int dev = 0;
    if (int e = fromHip(hipGetDevice(&dev), "hipGetDevice")) return e;
    void* p = dev >= 0 && dev < kMaxDevices ? g_fixed_scratch[dev] : nullptr;
    if (!p) {
        setDetail("matmul (no-alloc): the fixed scratch of device %d was not set up (kcInit)", dev);
        return KC_ERROR_NOT_INITIALIZED;
    }
    return runStaged(q6k, a, ks, p, s);
}

// K split in two where one K range leaves compute units idle. The producer-wavefront kernel holds
// one workgroup per CU, so it splits only when twice its workgroups still run at once (a 4096-row
// matrix over 1024 columns, 256 workgroups: 45.7 us in one K range, 51.5 us in two, the partial
// sums' extra pass included); the other kernels split below two 128-row workgroups per CU.
int matmulKs(int rows, int k, int ncols, bool q6) {
    if (k / 256 < 2) return 1;
    const long long ct = (ncols + 63) / 64;
    if (wsRuns(q6)) return 2LL * ((rows + mfmaWsRows() - 1) / mfmaWsRows()) * ct <= cuCount() ? 2 : 1;
    return (long long)((rows + kBM - 1) / kBM) * ct < 2LL * cuCount() ? 2 : 1;
}

bool mfmaHUsable(int ncols, int k) {
    const int path = option("matmul_path");
    return (path == 0 || path == 7) && (size_t)ncols * k * 2 < (1ull << 32);
}


int launchMatmulMfma(bool q6k, const kcMatmulKQ8Args& a, hipStream_t s) {
    const int path = option("matmul_path");
    if (path == 3) return q6k ? runMfma<true>(a, s) : runMfma<false>(a, s);  // 2 x 2 blocks per wavefront
    if (path == 4) return q6k ? runMfma8<true, 2>(a, s) : runMfma8<false, 2>(a, s);
    // fp16 activations staged by direct loads (a per-stream buffer, addressed with 32-bit offsets)
    if (path != 5 && (size_t)a.ncols * a.k * 2 < (1ull << 32)) {
        const int ks = stagedKs(q6k, a);
        if (void* buf = streamScratch(s, stagedBytes(a, ks))) return runStaged(q6k, a, ks, buf, s);
    }
    return q6k ? runMfma8<true, 1>(a, s) : runMfma8<false, 1>(a, s);
}

size_t matmulStagingBytes(int rows, int k, int ncols) {
    const int path = option("matmul_path");
    if (!(path == 0 && ncols >= 64) && !(path >= 2 && path != 3 && path != 4 && path != 5)) return 0;
    if ((size_t)ncols * k * 2 >= (1ull << 32)) return 0;
    const kcMatmulKQ8Args a{nullptr, nullptr, nullptr, nullptr, rows, k, ncols, 8};
    return stagedBytes(a, std::max(stagedKs(false, a), stagedKs(true, a)));  // (either type)
}

bool matmulGroupSplitsQ6(const MmPart* parts, int nparts, int k, int ncols) {
    if (nparts < 1 || nparts > 3 || k % 256 != 0 || ncols < 64 || !mfmaHUsable(ncols, k)) return false;
    if (option("matmul_ws") == 1 || option("matmul_ws") == 3 || (option("matmul_path") != 0 && option("matmul_path") != 2))
        return false;
    MfmaGroup g{};
    for (int i = 0; i < nparts; ++i)
        g.p[i] = MfmaPart{static_cast<const uint8_t*>(parts[i].qw), {parts[i].y[0], parts[i].y[1]}, parts[i].rows,
                          parts[i].q6, 0};
    g.nparts = nparts;
    g.ks = 1;
    return mfmaWsFits(g, k / 256, ncols) && splitsQ6(g, nparts, k / 256);
}

bool matmulGroupReadsActOnly(int ncols, int k) { return ncols >= 64 && mfmaHUsable(ncols, k); }

int launchMatmulGroup(const MmPart* parts, int nparts, const int* xq, int k, int ncols, int ks, int* used_ks,
                      hipStream_t s, const ActF16* pre, int* part_ks) {
    *used_ks = 1;
    if (part_ks)
        for (int i = 0; i < nparts && i < 3; ++i) part_ks[i] = 1;
    if (nparts < 1 || nparts > 3 || ks < 1 || ks > 2 || k % 256 != 0) return fromHip(hipErrorInvalidValue, "matmul group");
    if (matmulGroupReadsActOnly(ncols, k)) {
        if (ks > k / 256) ks = 1;
        if (pre) {
            *used_ks = ks;
            return runMfmaH(parts, nparts, xq, k, ncols, ks, nullptr, s, pre, part_ks);
        }
        if (void* act = streamScratch(s, actBytes(ncols, k))) {
            *used_ks = ks;
            return runMfmaH(parts, nparts, xq, k, ncols, ks, act, s, nullptr, part_ks);
        }
    }
    for (int i = 0; i < nparts; ++i) {  // one matmul per part, no K split
        const kcMatmulKQ8Args a{static_cast<const int*>(parts[i].qw), xq, parts[i].y[0], nullptr, parts[i].rows, k,
                                ncols, 8};
        const int st = launchMatmulKq(parts[i].q6 != 0, true, a, s);
        if (st) return st;
    }
    return 0;
}

}  // namespace kcamd
