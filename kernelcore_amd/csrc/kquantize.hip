// kquantize.hip -- f32 weights -> ggml block_q4_K / block_q6_K on the GPU (gfx950), and a
// counter-based normal generator for synthetic weights.
//
// The reference has no quantizer: its weights come from GGUF files that ggml (llama.cpp, not
// vendored) wrote. These kernels restate the published steps of ggml's reference quantizers,
// quantize_row_q4_K_ref and quantize_row_q6_K_ref, with their scale searches:
//   Q4_K: per sub-block of 32, weights w = sqrt(mean x^2) + |x|; a weighted least-squares fit of a
//         scale and a min (min <= 0) over 21 candidate inverse scales (15 + (-1 + 0.1 i)) / range,
//         keeping the candidate of least weighted squared error; the 8 scales and mins quantized to
//         6 bits against their maxima (d = max scale / 63, dmin = max min / 63, fp16); each value
//         then rounded to the nearest of the 16 grid points d*sc*q - dmin*m.
//   Q6_K: per sub-block of 16, x^2-weighted fit of a scale over 19 candidates -(32 + 0.1 i) / max;
//         the 16 scales quantized to int8 against the one of largest magnitude (d = -max / 128,
//         fp16); each value rounded to the nearest of d*sc*(q - 32), q in 0..63.
// Every float operation is sequential in the order of those loops (the build disables FMA
// contraction; division and square root are IEEE), so the bytes are bit-identical to the CPU
// restatement the tests compare against.
//
// Work split: one thread per sub-block (8 per Q4_K super-block, 16 per Q6_K super-block); the
// per-super-block maxima and the packing of nibbles go through LDS.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "internal.hpp"
#include "kquantize.hpp"

namespace kcamd {
namespace {

__device__ __forceinline__ int nearestEven(float f) { return (int)__builtin_rintf(f); }
__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }
__device__ __forceinline__ float halfToFloat(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}

// IEEE binary16 round to nearest even, overflow to infinity (ggml_fp32_to_fp16).
__device__ uint32_t floatToHalf(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const uint32_t sign = (u >> 16) & 0x8000u, ax = u & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7e00u;
    if (ax >= 0x477ff000u) return sign | 0x7c00u;
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return sign;
        const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int)(ax >> 23);
        uint32_t h = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1))) ++h;
        return sign | h;
    }
    uint32_t h = (ax >> 13) - (112u << 10);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;
    return sign | h;
}

constexpr int kQ4Threads = 256;  // 32 super-blocks x 8 sub-blocks
constexpr int kQ6Threads = 256;  // 16 super-blocks x 16 sub-blocks

__global__ __launch_bounds__(kQ4Threads) void quantize_q4k_kernel(const float* __restrict__ x,
                                                                  uint8_t* __restrict__ out, long long nsb) {
    __shared__ float sh_scale[kQ4Threads], sh_min[kQ4Threads];
    __shared__ uint8_t sh_L[32][256];
    const int tid = threadIdx.x, j = tid & 7, sbl = tid >> 3;
    const long long sb = (long long)blockIdx.x * 32 + sbl;
    const bool live = sb < nsb;
    float xv[32];
    const float* xs = x + (live ? sb : 0) * 256 + 32 * j;
#pragma unroll
    for (int l = 0; l < 32; ++l) xv[l] = live ? xs[l] : 0.0f;
    // the fit of sub-block j
    float sum_x2 = 0.0f;
#pragma unroll
    for (int l = 0; l < 32; ++l) sum_x2 += xv[l] * xv[l];
    const float av = __builtin_sqrtf(sum_x2 / 32.0f);
    float w[32];
#pragma unroll
    for (int l = 0; l < 32; ++l) w[l] = av + __builtin_fabsf(xv[l]);
    uint8_t L[32];
    float lo = xv[0], hi = xv[0], sw = w[0], sx = w[0] * xv[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) {
        if (xv[i] < lo) lo = xv[i];
        if (xv[i] > hi) hi = xv[i];
        sw += w[i];
        sx += w[i] * xv[i];
    }
    if (lo > 0.0f) lo = 0.0f;
    float scale, neg_min;
    if (hi == lo) {
#pragma unroll
        for (int i = 0; i < 32; ++i) L[i] = 0;
        scale = 0.0f;
        neg_min = -lo;
    } else {
        float iscale = 15.0f / (hi - lo);
        scale = 1.0f / iscale;
        float best = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const int l = clampi(nearestEven(iscale * (xv[i] - lo)), 0, 15);
            L[i] = (uint8_t)l;
            const float diff = scale * (float)l + lo - xv[i];
            best += w[i] * (diff * diff);
        }
        for (int step = 0; step <= 20; ++step) {
            iscale = (-1.0f + 0.1f * (float)step + 15.0f) / (hi - lo);
            float sl = 0.0f, sl2 = 0.0f, sxl = 0.0f;
            uint8_t cand[32];
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const int l = clampi(nearestEven(iscale * (xv[i] - lo)), 0, 15);
                cand[i] = (uint8_t)l;
                sl += w[i] * (float)l;
                sl2 += w[i] * (float)l * (float)l;
                sxl += w[i] * (float)l * xv[i];
            }
            const float det = sw * sl2 - sl * sl;
            if (det > 0.0f) {
                float s = (sw * sxl - sx * sl) / det;
                float m = (sl2 * sx - sl * sxl) / det;
                if (m > 0.0f) {
                    m = 0.0f;
                    s = sxl / sl2;
                }
                float err = 0.0f;
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    const float diff = s * (float)cand[i] + m - xv[i];
                    err += w[i] * (diff * diff);
                }
                if (err < best) {
#pragma unroll
                    for (int i = 0; i < 32; ++i) L[i] = cand[i];
                    best = err;
                    scale = s;
                    lo = m;
                }
            }
        }
        neg_min = -lo;
    }
    sh_scale[tid] = scale;
    sh_min[tid] = neg_min;
    __syncthreads();
    float max_scale = 0.0f, max_min = 0.0f;
    for (int i = 0; i < 8; ++i) {
        const float s = sh_scale[sbl * 8 + i], m = sh_min[sbl * 8 + i];
        if (s > max_scale) max_scale = s;
        if (m > max_min) max_min = m;
    }
    const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    uint32_t ls = (uint8_t)nearestEven(inv_scale * scale), lm = (uint8_t)nearestEven(inv_min * neg_min);
    if (ls > 63) ls = 63;
    if (lm > 63) lm = 63;
    const uint32_t d16 = floatToHalf(max_scale / 63.0f), m16 = floatToHalf(max_min / 63.0f);
    // the 6-bit pair this sub-block packs into the block is (ls, lm) itself (the packing is lossless)
    const float d = halfToFloat(d16) * (float)ls;
    if (d != 0.0f) {
        const float dm = halfToFloat(m16) * (float)lm;
#pragma unroll
        for (int i = 0; i < 32; ++i) L[i] = (uint8_t)clampi(nearestEven((xv[i] + dm) / d), 0, 15);
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) sh_L[sbl][32 * j + i] = L[i];
    // ls / lm of every sub-block for the scale bytes (reuse the float arrays as integers)
    __syncthreads();
    reinterpret_cast<uint32_t*>(sh_scale)[tid] = ls;
    reinterpret_cast<uint32_t*>(sh_min)[tid] = lm;
    __syncthreads();
    if (!live) return;
    uint8_t* b = out + sb * 144;
    // thread j writes 16 of the 128 nibble bytes: pair p = j / 2 of sub-blocks (2p, 2p + 1), half j % 2
    {
        const int p = j >> 1, h0 = (j & 1) * 16;
        uint32_t words[4];
#pragma unroll
        for (int wq = 0; wq < 4; ++wq) {
            uint32_t v = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int l = h0 + wq * 4 + e;
                v |= (uint32_t)(sh_L[sbl][64 * p + l] | (sh_L[sbl][64 * p + 32 + l] << 4)) << (8 * e);
            }
            words[wq] = v;
        }
        uint8_t* q = b + 16 + 32 * p + h0;
#pragma unroll
        for (int wq = 0; wq < 4; ++wq)
#pragma unroll
            for (int e = 0; e < 4; ++e) q[wq * 4 + e] = (uint8_t)(words[wq] >> (8 * e));
    }
    if (j == 0) {
        const uint32_t* LS = reinterpret_cast<const uint32_t*>(sh_scale) + sbl * 8;
        const uint32_t* LM = reinterpret_cast<const uint32_t*>(sh_min) + sbl * 8;
        uint8_t sc[12] = {};
        for (int jj = 0; jj < 8; ++jj) {
            if (jj < 4) {
                sc[jj] = (uint8_t)LS[jj];
                sc[jj + 4] = (uint8_t)LM[jj];
            } else {
                sc[jj + 4] = (uint8_t)((LS[jj] & 0xF) | ((LM[jj] & 0xF) << 4));
                sc[jj - 4] |= (uint8_t)((LS[jj] >> 4) << 6);
                sc[jj] |= (uint8_t)((LM[jj] >> 4) << 6);
            }
        }
        b[0] = (uint8_t)d16;
        b[1] = (uint8_t)(d16 >> 8);
        b[2] = (uint8_t)m16;
        b[3] = (uint8_t)(m16 >> 8);
        for (int i = 0; i < 12; ++i) b[4 + i] = sc[i];
    }
}

__global__ __launch_bounds__(kQ6Threads) void quantize_q6k_kernel(const float* __restrict__ x,
                                                                  uint8_t* __restrict__ out, long long nsb) {
    __shared__ float sh_scale[kQ6Threads];
    __shared__ int8_t sh_sc[16][16];
    __shared__ uint8_t sh_L[16][256];
    const int tid = threadIdx.x, g = tid & 15, sbl = tid >> 4;
    const long long sb = (long long)blockIdx.x * 16 + sbl;
    const bool live = sb < nsb;
    float xv[16];
    const float* xs = x + (live ? sb : 0) * 256 + 16 * g;
#pragma unroll
    for (int l = 0; l < 16; ++l) xv[l] = live ? xs[l] : 0.0f;
    uint8_t L[16];
    float mx = 0.0f, amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float ax = __builtin_fabsf(xv[i]);
        if (ax > amax) {
            amax = ax;
            mx = xv[i];
        }
    }
    float scale = 0.0f;
    if (amax < 1e-15f) {
#pragma unroll
        for (int i = 0; i < 16; ++i) L[i] = 0;
    } else {
        float iscale = -32.0f / mx;
        float sumlx = 0.0f, suml2 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int l = clampi(nearestEven(iscale * xv[i]), -32, 31);
            L[i] = (uint8_t)(l + 32);
            const float w = xv[i] * xv[i];
            sumlx += w * xv[i] * (float)l;
            suml2 += w * (float)l * (float)l;
        }
        scale = suml2 != 0.0f ? sumlx / suml2 : 0.0f;
        float best = scale * sumlx;
        for (int step = -9; step <= 9; ++step) {
            if (step == 0) continue;
            iscale = -(32.0f + 0.1f * (float)step) / mx;
            sumlx = suml2 = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int l = clampi(nearestEven(iscale * xv[i]), -32, 31);
                const float w = xv[i] * xv[i];
                sumlx += w * xv[i] * (float)l;
                suml2 += w * (float)l * (float)l;
            }
            if (suml2 > 0.0f && sumlx * sumlx > best * suml2) {
#pragma unroll
                for (int i = 0; i < 16; ++i) L[i] = (uint8_t)(32 + clampi(nearestEven(iscale * xv[i]), -32, 31));
                scale = sumlx / suml2;
                best = scale * sumlx;
            }
        }
    }
    sh_scale[tid] = scale;
    __syncthreads();
    // the scale of largest magnitude, the first one in sub-block order on ties
    float max_scale = 0.0f, max_abs = 0.0f;
    for (int i = 0; i < 16; ++i) {
        const float s = sh_scale[sbl * 16 + i], a = __builtin_fabsf(s);
        if (a > max_abs) {
            max_abs = a;
            max_scale = s;
        }
    }
    const bool zero = max_abs < 1e-15f;
    uint32_t d16 = 0;
    if (!zero) {
        const float iscale = -128.0f / max_scale;
        d16 = floatToHalf(1.0f / iscale);
        const int v = nearestEven(iscale * scale);
        const int sc = v < 127 ? v : 127;
        sh_sc[sbl][g] = (int8_t)sc;
        const float d = halfToFloat(d16) * (float)sc;
        if (d != 0.0f) {
#pragma unroll
            for (int i = 0; i < 16; ++i) L[i] = (uint8_t)(clampi(nearestEven(xv[i] / d), -32, 31) + 32);
        }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sh_L[sbl][16 * g + i] = L[i];
    __syncthreads();
    if (!live) return;
    uint8_t* b = out + sb * 210;
    if (zero) {  // an all-zero block
        for (int i = g; i < 210; i += 16) b[i] = 0;
        return;
    }
    // thread g writes ql bytes [8g, 8g + 8) and qh bytes [4g, 4g + 4)
    const uint8_t* Ls = sh_L[sbl];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int t = 8 * g + e, half = t >> 6, lq = t & 63;  // ql[64 * half + lq]
        const int l = lq & 31, base = 128 * half + (lq >= 32 ? 32 : 0);
        b[t] = (uint8_t)((Ls[base + l] & 0xF) | ((Ls[base + l + 64] & 0xF) << 4));
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int t = 4 * g + e, half = t >> 5, l = t & 31, j = 128 * half;
        b[128 + t] = (uint8_t)((Ls[j + l] >> 4) | ((Ls[j + l + 32] >> 4) << 2) | ((Ls[j + l + 64] >> 4) << 4) |
                               ((Ls[j + l + 96] >> 4) << 6));
    }
    b[192 + g] = (uint8_t)sh_sc[sbl][g];
    if (g == 0) {
        b[208] = (uint8_t)d16;
        b[209] = (uint8_t)(d16 >> 8);
    }
}

// splitmix64 finaliser: a counter-based stream (value i depends on seed and i only).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// y[i] = mean + std * N(0, 1): Box-Muller on two 24-bit uniforms per pair of outputs.
__global__ void fill_normal_kernel(float* __restrict__ y, long long n, uint64_t seed, float mean, float stdev) {
    const long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x;  // pair index
    if (2 * p >= n) return;
    const uint64_t r = mix64(seed + 0x9e3779b97f4a7c15ull * (uint64_t)(p + 1));
    const float u1 = ((float)(uint32_t)(r >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
    const float u2 = (float)(uint32_t)((r >> 16) & 0xffffffu) * (1.0f / 16777216.0f);
    const float rad = __builtin_sqrtf(-2.0f * __logf(u1));
    float sn, cs;
    __sincosf(6.2831853f * u2, &sn, &cs);
    y[2 * p] = mean + stdev * (rad * cs);
    if (2 * p + 1 < n) y[2 * p + 1] = mean + stdev * (rad * sn);
}

}  // namespace

int launchQuantizeKquant(bool q6k, const float* x, void* blocks, long long nsb, hipStream_t s) {
    if (nsb <= 0) return 0;
    auto* out = static_cast<uint8_t*>(blocks);
    if (q6k) hipLaunchKernelGGL(quantize_q6k_kernel, dim3((unsigned)((nsb + 15) / 16)), dim3(kQ6Threads), 0, s, x, out, nsb);
    else hipLaunchKernelGGL(quantize_q4k_kernel, dim3((unsigned)((nsb + 31) / 32)), dim3(kQ4Threads), 0, s, x, out, nsb);
    return fromHip(hipGetLastError(), q6k ? "quantize_kquant (Q6_K)" : "quantize_kquant (Q4_K)");
}

int launchFillNormal(float* y, long long n, unsigned long long seed, float mean, float stdev, hipStream_t s) {
    if (n <= 0) return 0;
    const long long pairs = (n + 1) / 2;
    hipLaunchKernelGGL(fill_normal_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, s, y, n, (uint64_t)seed,
                       mean, stdev);
    return fromHip(hipGetLastError(), "fill_normal_f32");
}

}  // namespace kcamd
