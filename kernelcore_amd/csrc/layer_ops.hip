// layer_ops.hip -- the bandwidth-bound layer kernels around the K-quant matmuls (gfx950):
// residual add + RMS partial sums, RMS norm x weight fused with the 8-bit quantization (per 32 or
// per 256 values), SwiGLU fused with the quantization, ggml RoPE, the fp16 KV-cache SET_ROWS,
// FLASH_ATTN_EXT (the reference's four kernels and a fused single-kernel form), and plain
// rms_norm / mul_rows / silu_mul / vector_add.
//
// Float operations follow the reference kernels in order (arasheedu/Kernelcore
// kernels/llm/add_sumsq_f.cu, sumsq_part.cu, norm_mul_q8_f.cu, norm_mul_q8k_f.cu,
// silu_mul_q8x4f.cu, silu_mul_q8kf.cu, rope_ggml.cu, set_rows_f16.cu, fa_*.cu, rms_norm.cu,
// mul_rows.cu, silu_mul.cu): sums of squares and the row total run sequentially per thread as
// there, so the norms and their quantized bytes are bit-identical; exp2f / sinf / cosf use the
// GPU's own math library, within a few ulps of the CPU's.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "internal.hpp"
#include "launch.hpp"

namespace kcamd {
namespace {

constexpr float kLog2e = 1.44269504f;

__device__ __forceinline__ int q8r(float t) {
    int q;
    if (t >= 0.0f) q = (int)(t + 0.5f);
    else q = (int)(t - 0.5f);
    return q > 127 ? 127 : (q < -127 ? -127 : q);
}

// (ss in LDS, 16-byte aligned: the sums in block order, sixteen read ahead of their adds)
__device__ __forceinline__ float rmsScale(const float* ss, int nb, int n, float eps) {
    float tot = 0.0f;
    const float4* s4 = reinterpret_cast<const float4*>(ss);
    int j = 0;
    for (; j + 16 <= nb; j += 16) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = s4[j / 4 + u];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            tot += v[u].x;
            tot += v[u].y;
            tot += v[u].z;
            tot += v[u].w;
        }
    }
    for (; j < nb; ++j) tot += ss[j];
    return 1.0f / sqrtf(tot / (float)n + eps);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + exp2f(-g * kLog2e)); }

// ---------------------------------------------------------------- wavefront helpers

template <int CTRL>
__device__ __forceinline__ int dppI(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dppF(float v) {
    return __builtin_bit_cast(float, dppI<CTRL>(__builtin_bit_cast(int, v)));
}
__device__ __forceinline__ float laneF(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// The maximum over the wavefront (every lane gets it): within rows of 16 by DPP (pairs, quads,
// mirrored halves), then the four rows' results read back as scalars.
__device__ __forceinline__ float waveMax(float v) {
    v = fmaxf(v, dppF<0xB1>(v));
    v = fmaxf(v, dppF<0x4E>(v));
    v = fmaxf(v, dppF<0x141>(v));
    v = fmaxf(v, dppF<0x140>(v));
    return fmaxf(fmaxf(laneF(v, 0), laneF(v, 16)), fmaxf(laneF(v, 32), laneF(v, 48)));
}

// Block quantization by the 8 lanes of an aligned group (lane j holds values 4j .. 4j + 3 of the
// block): quant32's arithmetic (the block maximum and the integer sum do not depend on the order
// of their terms; every value takes the same rounding), the cross-lane steps as DPP moves inside a
// row of 16 lanes. Returns this lane's word; every lane gets d and the block's sum.
struct Q8L {
    int w, sum;
    float d;
};
__device__ __forceinline__ Q8L quant8(const float (&y)[4]) {
    float m = fmaxf(fmaxf(fmaxf(y[0], 0.0f - y[0]), fmaxf(y[1], 0.0f - y[1])),
                    fmaxf(fmaxf(y[2], 0.0f - y[2]), fmaxf(y[3], 0.0f - y[3])));
    m = fmaxf(m, dppF<0xB1>(m));   // quad_perm [1,0,3,2]
    m = fmaxf(m, dppF<0x4E>(m));   // quad_perm [2,3,0,1]
    m = fmaxf(m, dppF<0x141>(m));  // row_half_mirror: the other quad of the 8
    Q8L o;
    o.d = fmaxf(0.0f, m) / 127.0f;
    float id;
    if (o.d > 0.0f) id = 1.0f / o.d;
    else id = 0.0f;
    const int c0 = q8r(y[0] * id), c1 = q8r(y[1] * id), c2 = q8r(y[2] * id), c3 = q8r(y[3] * id);
    o.w = (c0 & 255) | ((c1 & 255) << 8) | ((c2 & 255) << 16) | ((c3 & 255) << 24);
    int sm = (c0 + c1) + (c2 + c3);
    sm += dppI<0xB1>(sm);
    sm += dppI<0x4E>(sm);
    sm += dppI<0x141>(sm);
    o.sum = sm;
    return o;
}

// The sum of squares of a block of 32 in element order, by the 8 lanes of an aligned group (lane
// j holds values 4j .. 4j + 3): the running sum passes from lane j - 1 to lane j in eight steps
// (step k completes lane k), the same additions as one thread over the 32 values. Lane 7 returns
// the block's sum.
__device__ __forceinline__ float sumsq8(const float (&v)[4], int j) {
    float s = 0.0f, t = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        t = s;
#pragma unroll
        for (int e = 0; e < 4; ++e) t += v[e] * v[e];
        const float left = dppF<0x111>(t);  // row_shr:1: lane i - 1's value
        if (j == k + 1) s = left;
    }
    return t;
}

// The row's RMS scale from its nb per-32 sums of squares, summed in block order (rmsScale); every
// lane of the wavefront gets it.
__device__ __forceinline__ float rmsScaleWave(const float* ss, int nb, int n, float eps) {
    const int lane = threadIdx.x & 63;
    float tot = 0.0f;
    for (int j0 = 0; j0 < nb; j0 += 64) {
        const float v = ss[min(j0 + lane, nb - 1)];
        const int cnt = min(64, nb - j0);
        for (int L = 0; L < cnt; ++L) tot += laneF(v, L);
    }
    return 1.0f / sqrtf(tot / (float)n + eps);
}

// The MFMA layout of one quantized super-block (ActF16): lane L's four codes as fp16, lanes 8i
// (holding the sum B_i of values 32i .. 32i + 31 in b32) the two min operands of sub-block i,
// lane 0 the scale.
__device__ __forceinline__ void actF16Store(const ActF16& ao, int nsb, int s, int col, int lane, int c0, int c1, int c2,
                                            int c3, int b32, float d) {
    const int k = nsb * 256;
    typedef _Float16 hv4 __attribute__((ext_vector_type(4)));
    hv4 hq;
    hq[0] = (_Float16)(float)(16 * c0);  // 16 x: exact, and the matmul's weight operand is then sc q / 16
    hq[1] = (_Float16)(float)(16 * c1);
    hq[2] = (_Float16)(float)(16 * c2);
    hq[3] = (_Float16)(float)(16 * c3);
    *reinterpret_cast<hv4*>(static_cast<_Float16*>(ao.act) + (size_t)col * k + s * 256 + 4 * lane) = hq;
    if ((lane & 7) == 0) {
        _Float16* mn = static_cast<_Float16*>(ao.mins) + ((size_t)col * nsb + s) * 16 + (lane >> 3);
        mn[0] = (_Float16)(float)(64 * (b32 >> 6));
        mn[8] = (_Float16)(float)(b32 & 63);
    }
    if (lane == 0) ao.xdT[(size_t)s * ao.ncp + col] = d;
}

// One super-block of 256 values, four per lane (lane L holds values 4L .. 4L + 3), into a
// per-256 slot of nsb super-blocks (quantize_cols_k.cu / quant256 above): the same values, the
// max and the integer sums taken across lanes (both exact in any order).
// ao (optional): the same codes as fp16, the min operands and the scale in the MFMA matmul's
// layout (ActF16) for column col.
// (ao is taken by value: the address of a kernel argument would put it in scratch memory.)
__device__ __forceinline__ void quant256Wave(float y0, float y1, float y2, float y3, int* qc, int nsb, int s,
                                             ActF16 ao = ActF16{}, bool use_ao = false, int col = 0) {
    const int lane = threadIdx.x & 63;
    float am = fmaxf(fmaxf(fmaxf(y0, 0.0f - y0), fmaxf(y1, 0.0f - y1)), fmaxf(fmaxf(y2, 0.0f - y2), fmaxf(y3, 0.0f - y3)));
    am = waveMax(am);
    const float d = fmaxf(0.0f, am) / 127.0f;
    float id;
    if (d > 0.0f) id = 1.0f / d;
    else id = 0.0f;
    const int c0 = q8r(y0 * id), c1 = q8r(y1 * id), c2 = q8r(y2 * id), c3 = q8r(y3 * id);
    int s16 = c0 + c1 + c2 + c3;
    s16 += dppI<0xB1>(s16);
    s16 += dppI<0x4E>(s16);  // the 16 values of lanes 4g .. 4g + 3
    const int b32 = s16 + __shfl_down(s16, 4);  // lanes 8i: the sum of 32 values 32i .. 32i + 31
    if (qc) {  // the int8 slot (null: a caller whose products read only the MFMA layout)
        qc[s * 64 + lane] = (c0 & 255) | ((c1 & 255) << 8) | ((c2 & 255) << 16) | ((c3 & 255) << 24);
        if ((lane & 3) == 0) qc[nsb * 65 + s * 16 + (lane >> 2)] = s16;
        int pw[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int b = __builtin_amdgcn_readlane(b32, 8 * i);
            pw[i >> 2] |= ((b >> 6) & 255) << (8 * (i & 3));
            pw[2 + (i >> 2)] |= (b & 63) << (8 * (i & 3));
        }
        if (lane < 4) qc[nsb * 81 + s * 4 + lane] = lane == 0 ? pw[0] : (lane == 1 ? pw[1] : (lane == 2 ? pw[2] : pw[3]));
        if (lane == 0) reinterpret_cast<float*>(qc + nsb * 64)[s] = d;
    }
    if (use_ao) actF16Store(ao, nsb, s, col, lane, c0, c1, c2, c3, b32, d);
}

// Four consecutive floats at p (16-byte aligned when A16).
template <bool A16>
__device__ __forceinline__ float4 load4(const float* p) {
    if (A16) return *reinterpret_cast<const float4*>(p);
    return make_float4(p[0], p[1], p[2], p[3]);
}
template <bool A16>
__device__ __forceinline__ void store4(float* p, float4 v) {
    if (A16) *reinterpret_cast<float4*>(p) = v;
    else p[0] = v.x, p[1] = v.y, p[2] = v.z, p[3] = v.w;
}

// ---------------------------------------------------------------- residual add + RMS norm

// out = a + b and per-32 sums of out^2 into the row's slot tail (add_sumsq_f.cu). a may be null:
// then x = b and only the sums are written (sumsq_part.cu). a and out may be the same buffer (the
// residual stream updated in place). Four values per lane, eight lanes per block of 32 (grid: the
// rows, the row's quads by 256); the sums of squares in element order (sumsq8).
template <bool A16>
__global__ __launch_bounds__(256) void add_sumsq_kernel(const float* a, const float* b, const float* b2, float* out,
                                                        int* __restrict__ q, int n, int rows) {
    const int nb = n / 32, nq = n / 4, row = blockIdx.x;
    const int qi = blockIdx.y * 256 + threadIdx.x, qc = min(qi, nq - 1), j = qi & 7;
    const size_t o = (size_t)row * n + 4 * qc;
    const float4 bv = load4<A16>(b + o);
    float v[4] = {bv.x, bv.y, bv.z, bv.w};
    if (b2) {  // a product split in two partial sums
        const float4 bw = load4<A16>(b2 + o);
        v[0] += bw.x, v[1] += bw.y, v[2] += bw.z, v[3] += bw.w;
    }
    if (a) {
        const float4 av = load4<A16>(a + o);
        v[0] = av.x + v[0], v[1] = av.y + v[1], v[2] = av.z + v[2], v[3] = av.w + v[3];
        if (qi < nq) store4<A16>(out + o, make_float4(v[0], v[1], v[2], v[3]));
    }
    const float sq = sumsq8(v, j);
    if (j == 7 && qi < nq) reinterpret_cast<float*>(q + (size_t)row * nb * 11 + nb * 10)[qi >> 3] = sq;
}

// y = x * r * w, quantized per 32 into the row's slot (norm_mul_q8_f.cu). Four values per lane,
// eight lanes per block (quant8); every wavefront takes the row total itself (rmsScaleWave).
template <bool A16>
__global__ __launch_bounds__(256) void norm_mul_q8_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                          float* __restrict__ y, int* __restrict__ q, int n, int rows,
                                                          float eps) {
    const int nb = n / 32, nq = n / 4, row = blockIdx.x;
    const int qi = blockIdx.y * 256 + threadIdx.x, qc = min(qi, nq - 1);
    int* qr = q + (size_t)row * nb * 11;
    const size_t o = (size_t)row * n + 4 * qc;
    const float4 xv = load4<A16>(x + o), wv = load4<A16>(w + 4 * qc);  // in flight while r is summed
    const float r = rmsScaleWave(reinterpret_cast<const float*>(qr + nb * 10), nb, n, eps);
    const float v[4] = {xv.x * r * wv.x, xv.y * r * wv.y, xv.z * r * wv.z, xv.w * r * wv.w};
    const Q8L b = quant8(v);
    if (qi < nq) {
        store4<A16>(y + o, make_float4(v[0], v[1], v[2], v[3]));
        qr[qi] = b.w;  // block qi / 8, word qi % 8
        if ((qi & 7) == 0) {
            float* xd2 = reinterpret_cast<float*>(qr + nb * 8) + (qi >> 3) * 2;
            xd2[0] = b.d;
            xd2[1] = (float)b.sum;
        }
    }
}

// add_sumsq_f / sumsq_part and norm_mul_q8_f in one workgroup per row (NP passes of the block's
// threads over the row's quads): x = a + b (a null: x is read), the per-32 sums of squares
// (sumsq8) into LDS and the slot tail, the row total in block order by the first wavefront, then
// y = x * r * w and quant8 -- the values and bytes of the two kernels.
template <bool A16, int NP>
__global__ __launch_bounds__(1024) void add_norm_q8_kernel(const float* a, const float* b, float* x,
                                                           const float* __restrict__ w, float* y, int* __restrict__ q,
                                                           int n, float eps) {
    __shared__ float ss[8192 / 32 + 1];
    const int nb = n / 32, nq = n / 4, row = blockIdx.x, nth = blockDim.x;
    int* qr = q + (size_t)row * nb * 11;
    float v[NP][4];
    float4 wv[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int qi = threadIdx.x + p * nth, qc = min(qi, nq - 1);
        const size_t o = (size_t)row * n + 4 * qc;
        float4 xv;
        if (a) {
            const float4 bv = load4<A16>(b + o), av = load4<A16>(a + o);
            xv = make_float4(av.x + bv.x, av.y + bv.y, av.z + bv.z, av.w + bv.w);
            if (qi < nq) store4<A16>(x + o, xv);
        } else {
            xv = load4<A16>(x + o);
        }
        v[p][0] = xv.x, v[p][1] = xv.y, v[p][2] = xv.z, v[p][3] = xv.w;
        wv[p] = load4<A16>(w + 4 * qc);
        const float sq = sumsq8(v[p], qi & 7);
        if ((qi & 7) == 7 && qi < nq) {
            ss[qi >> 3] = sq;
            reinterpret_cast<float*>(qr + nb * 10)[qi >> 3] = sq;
        }
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const float r = rmsScaleWave(ss, nb, n, eps);
        if (threadIdx.x == 0) ss[nb] = r;
    }
    __syncthreads();
    const float r = ss[nb];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int qi = threadIdx.x + p * nth;
        const size_t o = (size_t)row * n + 4 * min(qi, nq - 1);
        const float yv[4] = {v[p][0] * r * wv[p].x, v[p][1] * r * wv[p].y, v[p][2] * r * wv[p].z, v[p][3] * r * wv[p].w};
        const Q8L bq = quant8(yv);
        if (qi < nq) {
            store4<A16>(y + o, make_float4(yv[0], yv[1], yv[2], yv[3]));
            qr[qi] = bq.w;
            if ((qi & 7) == 0) {
                float* xd2 = reinterpret_cast<float*>(qr + nb * 8) + (qi >> 3) * 2;
                xd2[0] = bq.d;
                xd2[1] = (float)bq.sum;
            }
        }
    }
}

// The same with per-256 slots (norm_mul_q8k_f.cu): q holds rows slots of nsb*85 ints, then the
// rows per-32 slots whose tails hold the partial sums. One workgroup of four wavefronts per row;
// each wavefront takes super-blocks w, w + 4, ... with four values per lane. The row total is
// summed in block order from values read back lane by lane.
template <bool A16>
__global__ __launch_bounds__(256) void norm_mul_q8k_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           float* __restrict__ y, int* __restrict__ q, int n, int rows,
                                                           float eps) {
    const int nsb = n / 256, nb = n / 32;
    const int row = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* ss = reinterpret_cast<const float*>(q + (size_t)rows * nsb * 85 + (size_t)row * nb * 11 + nb * 10);
    float tot = 0.0f;
    for (int j0 = 0; j0 < nb; j0 += 256) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = ss[min(j0 + 4 * lane + e, nb - 1)];
        const int cnt = min(256, nb - j0) / 4;  // nb is a multiple of 8
        for (int L = 0; L < cnt; ++L)
#pragma unroll
            for (int e = 0; e < 4; ++e) tot += laneF(v[e], L);
    }
    const float r = 1.0f / sqrtf(tot / (float)n + eps);
    int* qr = q + (size_t)row * nsb * 85;
    for (int sb = wave; sb < nsb; sb += 4) {
        const size_t o = (size_t)row * n + sb * 256 + 4 * lane;
        const float4 xv = load4<A16>(x + o), wv = load4<A16>(w + sb * 256 + 4 * lane);
        const float4 yv = make_float4(xv.x * r * wv.x, xv.y * r * wv.y, xv.z * r * wv.z, xv.w * r * wv.w);
        store4<A16>(y + o, yv);
        quant256Wave(yv.x, yv.y, yv.z, yv.w, qr, nsb, sb);
    }
}

// SwiGLU, quantized per 32 (silu_mul_q8x4f.cu) or per 256 (silu_mul_q8kf.cu); columns of n. The
// per-32 form: four values per lane, eight lanes per block (quant8).
template <bool A16>
__global__ __launch_bounds__(256) void silu_mul_q8_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                          float* __restrict__ y, int* __restrict__ q, int n, int cols) {
    const int nb = n / 32, nq = n / 4, c = blockIdx.x;
    const int qi = blockIdx.y * 256 + threadIdx.x, qc = min(qi, nq - 1);
    const size_t o = (size_t)c * n + 4 * qc;
    const float4 gv = load4<A16>(g + o), uv = load4<A16>(u + o);
    const float v[4] = {silu(gv.x) * uv.x, silu(gv.y) * uv.y, silu(gv.z) * uv.z, silu(gv.w) * uv.w};
    const Q8L b = quant8(v);
    if (qi < nq) {
        store4<A16>(y + o, make_float4(v[0], v[1], v[2], v[3]));
        int* qcol = q + (size_t)c * nb * 11;
        qcol[qi] = b.w;
        if ((qi & 7) == 0) {
            float* xd2 = reinterpret_cast<float*>(qcol + nb * 8) + (qi >> 3) * 2;
            xd2[0] = b.d;
            xd2[1] = (float)b.sum;
        }
    }
}

template <bool A16>
__global__ __launch_bounds__(1024) void silu_mul_q8k_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                           float* __restrict__ y, int* __restrict__ q, int n, int cols,
                                                           ActF16 ao, int has_ao) {
    const int nsb = n / 256;
    const int c = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int* qc = q ? q + (size_t)c * nsb * 85 : nullptr;
    const int nw = blockDim.x >> 6;
    for (int sb = wave; sb < nsb; sb += nw) {
        const size_t o = (size_t)c * n + sb * 256 + 4 * lane;
        const float4 gv = load4<A16>(g + o), uv = load4<A16>(u + o);
        const float4 yv = make_float4(silu(gv.x) * uv.x, silu(gv.y) * uv.y, silu(gv.z) * uv.z, silu(gv.w) * uv.w);
        if (y) store4<A16>(y + o, yv);
        quant256Wave(yv.x, yv.y, yv.z, yv.w, qc, nsb, sb, ao, has_ao != 0, c);
    }
}

// ---------------------------------------------------------------- elementwise and row ops

__global__ void vector_add_kernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ out,
                                  int count) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) out[i] = a[i] + b[i];
}

__global__ void mul_rows_kernel(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ y, int n,
                                int count) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) y[i] = x[i] * w[i % n];
}

__global__ void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ out,
                                int count) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) out[i] = silu(g[i]) * u[i];
}

// One thread per row, sequential sums as rms_norm.cu (bit-identical).
__global__ void rms_norm_kernel(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ y, int n,
                                int rows, float eps) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const float* xr = x + (size_t)row * n;
    float ss = 0.0f;
    for (int j = 0; j < n; ++j) ss += xr[j] * xr[j];
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    float* yr = y + (size_t)row * n;
    for (int j = 0; j < n; ++j) yr[j] = xr[j] * r * w[j];
}

// The same per row with one workgroup of 64 lanes (rows up to 16384 values): the row staged in LDS
// by coalesced loads, its sum of squares in element order by one lane (the same additions, so the
// same bits), then y = x r w by every lane. A thread per row leaves the GPU nearly idle and waits
// for each of its row's loads in turn (a Qwen3 layer's per-head q / k norms, 32 and 8 rows of 128).
__global__ __launch_bounds__(64) void rms_norm_row_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                          float* __restrict__ y, int n, float eps) {
    extern __shared__ float xs[];
    __shared__ float rr;
    const int lane = threadIdx.x;
    const float* xr = x + (size_t)blockIdx.x * n;
    for (int j = lane; j < n; j += 64) xs[j] = xr[j];
    __syncthreads();
    if (lane == 0) {
        float ss = 0.0f;
#pragma unroll 8
        for (int j = 0; j < n; ++j) ss += xs[j] * xs[j];
        rr = 1.0f / sqrtf(ss / (float)n + eps);
    }
    __syncthreads();
    const float r = rr;
    float* yr = y + (size_t)blockIdx.x * n;
    for (int j = lane; j < n; j += 64) yr[j] = xs[j] * r * w[j];
}

// The same for short rows (n = 4, 8, .. 128: float4s per row dividing 64; rows 16-byte aligned)
// with one lane per row: a workgroup's 64 rows (contiguous in memory) come into LDS by coalesced
// 16-byte loads (rows padded by 4 floats, so the lanes' row reads hit different banks), each lane
// takes its row's sum of squares in element order (the same additions as the kernels above, so the
// same bits), and the outputs y = x r w leave by coalesced stores (in place is safe: every load
// precedes every store). A Qwen3 prompt's per-head q / k norms are 32768 + 8192 rows of 128 per
// layer at 1024 tokens: a workgroup per row left one lane per 64 working through the row's serial
// sum.
constexpr int kNormLaneMax = 128;
__global__ __launch_bounds__(64) void rms_norm_lane_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           float* __restrict__ y, int n, int rows, float eps) {
    __shared__ float4 xs[64 * (kNormLaneMax / 4 + 1)];
    __shared__ float rr[64];
    const int lane = threadIdx.x, row0 = blockIdx.x * 64;
    const int q = n / 4, stride = q + 1, rstep = 64 / q;  // float4s per row in memory and in LDS
    const int nq = min(64, rows - row0) * q;
    const int r0 = lane / q, c0 = lane - r0 * q;  // this lane's loads: rows r0 + i rstep, float4 c0
    const float4* xb = reinterpret_cast<const float4*>(x + (size_t)row0 * n);
#pragma unroll 8
    for (int i = 0; lane + 64 * i < nq; ++i) xs[(r0 + i * rstep) * stride + c0] = xb[lane + 64 * i];
    __syncthreads();
    if (row0 + lane < rows) {
        const float4* xr = xs + lane * stride;
        float ss = 0.0f;
        for (int i = 0; i < q; ++i) {
            const float4 u = xr[i];
            ss += u.x * u.x;
            ss += u.y * u.y;
            ss += u.z * u.z;
            ss += u.w * u.w;
        }
        rr[lane] = 1.0f / sqrtf(ss / (float)n + eps);
    }
    __syncthreads();
    float4* yb = reinterpret_cast<float4*>(y + (size_t)row0 * n);
    const float4 wv = reinterpret_cast<const float4*>(w)[c0];
#pragma unroll 8
    for (int i = 0; lane + 64 * i < nq; ++i) {
        const int r = r0 + i * rstep;
        const float4 u = xs[r * stride + c0];
        const float rv = rr[r];
        yb[lane + 64 * i] = make_float4(u.x * rv * wv.x, u.y * rv * wv.y, u.z * rv * wv.z, u.w * rv * wv.w);
    }
}

// ggml ROPE (rope_ggml.cu): one thread per (token, head, pair); each thread takes the pair's
// angle itself (the reference's per-(token, pair) value, recomputed per head).
__global__ void rope_kernel(const float* __restrict__ x, float* __restrict__ y, const int* __restrict__ pos,
                            const float* __restrict__ ff, int pairs, int nh, int count, float log2_base, int m1,
                            int m2) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= count) return;
    const int th = idx / pairs, i = idx - th * pairs, t = th / nh;
    const float theta = (float)pos[t] * exp2f(-(float)i / (float)pairs * log2_base) / ff[i];
    const float c = cosf(theta), s = sinf(theta);
    const size_t a = 2 * (size_t)th * pairs + (size_t)i * m1;
    const float x0 = x[a], x1 = x[a + m2];
    y[a] = x0 * c - x1 * s;
    y[a + m2] = x0 * s + x1 * c;
}

// fp32 -> fp16 bits as set_rows_f16.cu: nearest even, |x| >= 65520 -> +-0x7bff, -0 -> +0.
__device__ __forceinline__ uint32_t f2h(float x) {
    if (x == 0.0f) return 0;
    const uint32_t sign = x < 0.0f ? 0x8000u : 0u;
    if (!(fabsf(x) < 65520.0f)) return sign | 0x7bffu;
    return __builtin_bit_cast(unsigned short, (_Float16)x);
}

// ggml SET_ROWS into fp16 (set_rows_f16.cu): one thread per (row, pair) writes one 32-bit word.
__global__ void set_rows_kernel(const float* __restrict__ src, const int* __restrict__ idx, int* __restrict__ dst,
                                int pairs, int rows, int src_row, int dst_row, int dst_rows) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= pairs * rows) return;
    const int r = i / pairs, j = i - r * pairs;
    const int row = idx[2 * r];  // low word of the int64 row number
    if (row < 0 || row >= dst_rows) return;
    const float* sp = src + (size_t)r * src_row + 2 * j;
    dst[(size_t)row * dst_row + j] = (int)(f2h(sp[0]) | (f2h(sp[1]) << 16));
}

// ---------------------------------------------------------------- fused batch kernels (model path)

// RoPE of q (nh heads) and k (nkv heads) of a batch, and the fp16 stores of the roped k and of v
// into the cache rows pos[t] (rope_ggml.cu, set_rows_f16.cu): one thread per (token, group of 4
// heads, pair), which takes theta, its cosine and sine once for its heads (q heads first, then the
// k heads with their v), all its loads issued before the first is used. Rows outside [0, dst_rows)
// are not stored. v2 (may be null): v's product in two K ranges, stored as v + v2.
__global__ void rope_qk_store_kernel(const float* __restrict__ q, float* __restrict__ qr, const float* __restrict__ k,
                                     const float* __restrict__ v, const float* __restrict__ v2,
                                     unsigned short* __restrict__ kc,
                                     unsigned short* __restrict__ vc, const int* __restrict__ pos,
                                     const float* __restrict__ ff, int pairs, int nh, int nkv, int n, float log2_base,
                                     int m1, int m2, int dst_row, int dst_rows) {
    const int ng = (nh + nkv + 3) / 4;
    const long long idx = blockIdx.x * (long long)blockDim.x + threadIdx.x;
    if (idx >= (long long)n * ng * pairs) return;
    const int i = (int)(idx % pairs);
    const long long tg = idx / pairs;
    const int hg = (int)(tg % ng), t = (int)(tg / ng);
    // every load of the thread's four heads first (one memory round trip, not one per head)
    float x0[4], x1[4], va[4], vb[4], wa[4], wb[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int h = hg * 4 + u;
        x0[u] = x1[u] = va[u] = vb[u] = wa[u] = wb[u] = 0.0f;
        if (h < nh) {
            const size_t a = 2 * ((size_t)t * nh + h) * pairs + (size_t)i * m1;
            x0[u] = q[a];
            x1[u] = q[a + m2];
        } else if (h < nh + nkv) {
            const size_t a = 2 * ((size_t)t * nkv + (h - nh)) * pairs + (size_t)i * m1;
            x0[u] = k[a];
            x1[u] = k[a + m2];
            va[u] = v[a];
            vb[u] = v[a + m2];
            if (v2) {
                wa[u] = v2[a];
                wb[u] = v2[a + m2];
            }
        }
    }
    const int p = pos[t];
    const float theta = (float)p * exp2f(-(float)i / (float)pairs * log2_base) / ff[i];
    const float c = cosf(theta), sn = sinf(theta);
    const bool store = p >= 0 && p < dst_rows;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int h = hg * 4 + u;
        if (h < nh) {
            const size_t a = 2 * ((size_t)t * nh + h) * pairs + (size_t)i * m1;
            qr[a] = x0[u] * c - x1[u] * sn;
            qr[a + m2] = x0[u] * sn + x1[u] * c;
        } else if (h < nh + nkv && store) {
            const int hk = h - nh;
            const size_t e = (size_t)p * dst_row * 2 + 2 * (size_t)hk * pairs + (size_t)i * m1;
            kc[e] = (unsigned short)f2h(x0[u] * c - x1[u] * sn);
            kc[e + m2] = (unsigned short)f2h(x0[u] * sn + x1[u] * c);
            const float v0 = v2 ? va[u] + wa[u] : va[u], v1 = v2 ? vb[u] + wb[u] : vb[u];
            vc[e] = (unsigned short)f2h(v0);
            vc[e + m2] = (unsigned short)f2h(v1);
        }
    }
}

// The same for a model with per-head q / k norms (Qwen3), the norms included: RMS_NORM(q) * q_norm
// and RMS_NORM(k) * k_norm per head row of hd = 2 pairs values, then the RoPE and stores above, in
// one launch instead of three. A workgroup of 256 threads takes 64 consecutive head rows (q rows
// [n][nh] in workgroups 0 .. nq_blocks - 1, then the k rows [n][nkv] with their v rows): the rows
// come into LDS by coalesced 16-byte loads (padded by 4 floats), the first wavefront's lanes sum a
// row's squares each in element order and take r (rms_norm_lane_kernel's arithmetic), theta, its
// cosine and sine are taken once per (token, pair) of the workgroup's tokens into LDS
// (rope_qk_store_kernel's arithmetic), and every thread rotates pairs of the normed values x r w:
// thread t always pair t % pairs, of rows 256 / pairs apart. The same floats as the three launches,
// bit for bit. hd 64 or 128 (lp = log2(pairs)), ff (the frequency factors) hd / 2 values.
constexpr int kNormRopeThreads = 256;
// One workgroup's 64 head rows of norm_rope_qk_store_kernel: q rows (ISQ) or k rows with their v.
template <bool ISQ>
__device__ __forceinline__ void normRopeRows(const float* __restrict__ q, float* __restrict__ qr,
                                             const float* __restrict__ k, const float* __restrict__ v,
                                             const float* __restrict__ v2, const float* __restrict__ qw,
                                             const float* __restrict__ kw, unsigned short* __restrict__ kc,
                                             unsigned short* __restrict__ vc, const int* __restrict__ pos,
                                             const float* __restrict__ ff, int lp, int nh, int nkv, int n,
                                             float log2_base, int m1, int m2, int dst_row, int dst_rows, float eps,
                                             int nq_blocks) {
    extern __shared__ float4 nr_lds[];
    const int pairs = 1 << lp, hd = 2 * pairs, lq4 = lp - 1, q4 = hd / 4, stride = q4 + 1;
    float4* xs = nr_lds;                                       // 64 rows, padded
    float* rr = reinterpret_cast<float*>(xs + 64 * stride);    // per row: the norm's scale
    int* tl = reinterpret_cast<int*>(rr + 64);                 // per row: its token - t0
    long long* dst = reinterpret_cast<long long*>(tl + 64);    // per row: q row / cache offset, -1: no store
    float2* cs = reinterpret_cast<float2*>(dst + 64);          // [token - t0][pairs] (cos, sin)
    const int tid = threadIdx.x;
    const int nhd = ISQ ? nh : nkv, rows = n * nhd;
    const int row0 = (ISQ ? (int)blockIdx.x : (int)blockIdx.x - nq_blocks) * 64;
    const int nr = min(64, rows - row0), nqw = nr * q4;
    const float4* xb = reinterpret_cast<const float4*>((ISQ ? q : k) + (size_t)row0 * hd);
    const int t0 = row0 / nhd, ntok = (row0 + nr - 1) / nhd - t0 + 1;
    const int i = tid & (pairs - 1), a = i * m1;  // this thread's pair: values a, a + m2 of a head row
    const int rstep = kNormRopeThreads >> lp;     // the thread's rows: tid / pairs + j rstep
    // Every global load is issued before any is used (one memory round trip): the 64 rows (at most
    // 8 16-byte words per thread), the positions of the first 4 x 256 (token, pair) entries of the
    // cos / sin table, and in a k workgroup the v (+ v2) values that the thread stores.
    float4 xl[8];  // (clamped: past nqw a thread reloads the last word, which it does not store)
#pragma unroll
    for (int j = 0; j < 8; ++j) xl[j] = xb[min(tid + j * kNormRopeThreads, nqw - 1)];
    const float fi = ff[i];  // entry u of the table has pair u % pairs = i (256 is a multiple of pairs)
    const float* w = ISQ ? qw : kw;
    const float wa_ = w[a], wb_ = w[a + m2];
    int pp[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) pp[j] = pos[t0 + min((tid + j * kNormRopeThreads) >> lp, ntok - 1)];
    const int prow = ISQ ? 0 : pos[min((row0 + min(tid, nr - 1)) / nhd, n - 1)];
    constexpr int kVr = 16;  // rows per thread at pairs = 64
    float va[kVr], vb[kVr], wa[kVr], wb[kVr];
    if (!ISQ) {  // (unconditional, clamped loads: a load under a condition is waited for at its end)
        const float* v2p = v2 ? v2 : v;
#pragma unroll
        for (int j = 0; j < kVr; ++j) {
            const size_t av = (size_t)(row0 + min((tid >> lp) + j * rstep, nr - 1)) * hd + a;
            va[j] = v[av];
            vb[j] = v[av + m2];
            wa[j] = v2p[av];
            wb[j] = v2p[av + m2];
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // unconditional (a clamped word is stored again, the same value),
        const int jj = min(tid + j * kNormRopeThreads, nqw - 1);  // so no load sinks into a branch
        xs[(jj >> lq4) * stride + (jj & (q4 - 1))] = xl[j];
    }
    // theta per (token, pair) of this workgroup's tokens t0 .. t0 + ntok - 1
    const float fr = exp2f(-(float)i / (float)pairs * log2_base);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int u = tid + j * kNormRopeThreads;
        if (u < ntok * pairs) {
            const float theta = (float)pp[j] * fr / fi;
            cs[u] = make_float2(cosf(theta), sinf(theta));
        }
    }
    for (int u = tid + 4 * kNormRopeThreads; u < ntok * pairs; u += kNormRopeThreads) {
        const float theta = (float)pos[t0 + (u >> lp)] * fr / fi;
        cs[u] = make_float2(cosf(theta), sinf(theta));
    }
    __syncthreads();
    if (tid < nr) {
        const float4* xr = xs + tid * stride;
        float ss = 0.0f;
        for (int e = 0; e < q4; ++e) {
            const float4 x4 = xr[e];
            ss += x4.x * x4.x;
            ss += x4.y * x4.y;
            ss += x4.z * x4.z;
            ss += x4.w * x4.w;
        }
        rr[tid] = 1.0f / sqrtf(ss / (float)hd + eps);
        const int row = row0 + tid, t = row / nhd, hh = row - t * nhd;
        tl[tid] = t - t0;
        if (ISQ) dst[tid] = (long long)row * hd;
        else dst[tid] = prow >= 0 && prow < dst_rows ? (long long)prow * dst_row * 2 + (long long)hh * hd : -1;
    }
    __syncthreads();
    const float* xf = reinterpret_cast<const float*>(xs);
#pragma unroll
    for (int j = 0; j < kVr; ++j) {
        const int r = (tid >> lp) + j * rstep;
        if (j * rstep >= 64 || r >= nr) break;
        const float rv = rr[r];
        const float x0 = xf[r * 4 * stride + a] * rv * wa_, x1 = xf[r * 4 * stride + a + m2] * rv * wb_;
        const float2 csv = cs[(tl[r] << lp) + i];
        const float y0 = x0 * csv.x - x1 * csv.y, y1 = x0 * csv.y + x1 * csv.x;
        const long long d = dst[r];
        if (ISQ) {
            qr[d + a] = y0;
            qr[d + a + m2] = y1;
        } else if (d >= 0) {
            const size_t e = (size_t)d + a;
            kc[e] = (unsigned short)f2h(y0);
            kc[e + m2] = (unsigned short)f2h(y1);
            const float v0 = v2 ? va[j] + wa[j] : va[j], v1 = v2 ? vb[j] + wb[j] : vb[j];
            vc[e] = (unsigned short)f2h(v0);
            vc[e + m2] = (unsigned short)f2h(v1);
        }
    }
}

__global__ __launch_bounds__(kNormRopeThreads) void norm_rope_qk_store_kernel(
    const float* __restrict__ q, float* __restrict__ qr, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ v2, const float* __restrict__ qw, const float* __restrict__ kw,
    unsigned short* __restrict__ kc, unsigned short* __restrict__ vc, const int* __restrict__ pos,
    const float* __restrict__ ff, int lp, int nh, int nkv, int n, float log2_base, int m1, int m2, int dst_row,
    int dst_rows, float eps, int nq_blocks) {
    if ((int)blockIdx.x < nq_blocks)
        normRopeRows<true>(q, qr, k, v, v2, qw, kw, kc, vc, pos, ff, lp, nh, nkv, n, log2_base, m1, m2, dst_row,
                           dst_rows, eps, nq_blocks);
    else
        normRopeRows<false>(q, qr, k, v, v2, qw, kw, kc, vc, pos, ff, lp, nh, nkv, n, log2_base, m1, m2, dst_row,
                            dst_rows, eps, nq_blocks);
}

// The ggml graph's ROPE(q), ROPE(k), SET_ROWS(k cache, roped k, idx) and SET_ROWS(v cache, v, idx)
// in one launch (rope_ggml.cu, set_rows_f16.cu): one thread per (token, group of 4 heads, pair) as
// rope_qk_store_kernel, which also keeps the roped k in kr and takes the cache rows from idx (int64,
// low words; rows outside [0, dst_rows) are not stored). Sources: q, k contiguous [n][heads][hd];
// v rows src_v floats apart (v2, when given, the second K range of v's product, the same layout:
// v + v2 is stored, and written back into v); cache rows k_row / v_row 32-bit words apart.
__global__ void rope_kv_rows_kernel(const float* __restrict__ q, float* __restrict__ qr, const float* __restrict__ k,
                                    float* __restrict__ kr, float* __restrict__ v, unsigned short* __restrict__ kc,
                                    unsigned short* __restrict__ vc, const int* __restrict__ pos,
                                    const int* __restrict__ idx, const float* __restrict__ ff, int pairs, int nh,
                                    int nkv, int n, float log2_base, int m1, int m2, int src_v, int k_row, int v_row,
                                    int dst_rows, const float* __restrict__ v2) {
    const int ng = (nh + nkv + 3) / 4;
    const long long id = blockIdx.x * (long long)blockDim.x + threadIdx.x;
    if (id >= (long long)n * ng * pairs) return;
    const int i = (int)(id % pairs);
    const long long tg = id / pairs;
    const int hg = (int)(tg % ng), t = (int)(tg / ng);
    // every load of the thread's four heads first (one memory round trip, not one per head); each
    // thread reads and writes only its own elements, so in-place q / k / v stay correct
    float x0[4], x1[4], va[4], vb[4], wa[4], wb[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int h = hg * 4 + u;
        x0[u] = x1[u] = va[u] = vb[u] = wa[u] = wb[u] = 0.0f;
        if (h < nh) {
            const size_t a = 2 * ((size_t)t * nh + h) * pairs + (size_t)i * m1;
            x0[u] = q[a];
            x1[u] = q[a + m2];
        } else if (h < nh + nkv) {
            const int hk = h - nh;
            const size_t a = 2 * ((size_t)t * nkv + hk) * pairs + (size_t)i * m1;
            const size_t av = (size_t)t * src_v + 2 * (size_t)hk * pairs + (size_t)i * m1;
            x0[u] = k[a];
            x1[u] = k[a + m2];
            va[u] = v[av];
            vb[u] = v[av + m2];
            if (v2) {
                wa[u] = v2[av];
                wb[u] = v2[av + m2];
            }
        }
    }
    const float theta = (float)pos[t] * exp2f(-(float)i / (float)pairs * log2_base) / ff[i];
    const float c = cosf(theta), sn = sinf(theta);
    const int row = idx[2 * t];
    const bool store = row >= 0 && row < dst_rows;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int h = hg * 4 + u;
        if (h < nh) {
            const size_t a = 2 * ((size_t)t * nh + h) * pairs + (size_t)i * m1;
            qr[a] = x0[u] * c - x1[u] * sn;
            qr[a + m2] = x0[u] * sn + x1[u] * c;
        } else if (h < nh + nkv) {
            const int hk = h - nh;
            const size_t a = 2 * ((size_t)t * nkv + hk) * pairs + (size_t)i * m1;
            const float y0 = x0[u] * c - x1[u] * sn, y1 = x0[u] * sn + x1[u] * c;
            kr[a] = y0;
            kr[a + m2] = y1;
            const size_t o = 2 * (size_t)hk * pairs + (size_t)i * m1;
            const size_t av = (size_t)t * src_v + o;
            float v0 = va[u], v1 = vb[u];
            if (v2) {  // the whole product, also back into v (stored or not)
                v0 = va[u] + wa[u];
                v1 = vb[u] + wb[u];
                v[av] = v0;
                v[av + m2] = v1;
            }
            if (store) {
                const size_t e = (size_t)row * k_row * 2 + o, f = (size_t)row * v_row * 2 + o;
                kc[e] = (unsigned short)f2h(y0);
                kc[e + m2] = (unsigned short)f2h(y1);
                vc[f] = (unsigned short)f2h(v0);
                vc[f + m2] = (unsigned short)f2h(v1);
            }
        }
    }
}

// Residual add + RMS norm + per-256 quantization of a batch (add_sumsq_f.cu then norm_mul_q8k_f.cu
// in one workgroup per row): x = a + (b [+ b2]) (a null: x = b, not stored), the per-32 sums of
// squares in order, their total in block order, y = x r w quantized per 256 into the row's slot.
// regs (a row of at most four values per thread): each thread keeps its quad and the norm weights
// of it in registers from the first loads on, the per-32 sums chained through the block's 8 lanes
// (sumsq8: the same additions in the same order), and only those sums pass through LDS. Else the
// row is loaded with every thread (coalesced) into LDS, blocks of 32 padded to 36 floats so that
// the per-block sums (one thread each, in order) read different banks.
template <bool A16>
__global__ __launch_bounds__(1024) void add_norm_q8k_kernel(const float* a, const float* b, const float* b2, float* out,
                                                           const float* __restrict__ w, int* __restrict__ q, int n,
                                                           float eps, ActF16 ao, int has_ao, float* __restrict__ y,
                                                           int regs) {
    extern __shared__ float xs[];  // n / 32 blocks of 36 floats, then n / 32 sums of squares
    const int nsb = n / 256, nb = n / 32;
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float* ss = xs + nb * 36;
    const size_t r0 = (size_t)row * n;
    const int nt = blockDim.x;
    if (regs) {  // 4 nt >= n: thread t holds values 4t .. 4t + 3 = super-block t / 64, lane t % 64
        const bool live = wave < nsb;  // wavefront-uniform (n is a multiple of 256)
        const int i = live ? 4 * tid : 0;
        // the four loads unconditional (an absent b2 / a reads b again), all issued before any use
        float4 v = load4<A16>(b + r0 + i);
        const float4 u = load4<A16>((b2 ? b2 : b) + r0 + i);
        const float4 x = load4<A16>((a ? a : b) + r0 + i);
        const float4 wv = load4<A16>(w + i);
        if (b2) v.x += u.x, v.y += u.y, v.z += u.z, v.w += u.w;
        if (a) {
            v = make_float4(x.x + v.x, x.y + v.y, x.z + v.z, x.w + v.w);
            if (live) store4<A16>(out + r0 + i, v);
        }
        const float xv[4] = {v.x, v.y, v.z, v.w};
        const float sq = sumsq8(xv, tid & 7);
        if (live && (tid & 7) == 7) ss[tid >> 3] = sq;
        __syncthreads();
        if (!live) return;
        const float r = rmsScale(ss, nb, n, eps);
        const float4 yv = make_float4(v.x * r * wv.x, v.y * r * wv.y, v.z * r * wv.z, v.w * r * wv.w);
        if (y) store4<A16>(y + r0 + i, yv);
        quant256Wave(yv.x, yv.y, yv.z, yv.w, q ? q + (size_t)row * nsb * 85 : nullptr, nsb, wave, ao, has_ao != 0,
                     row);
        return;
    }
    for (int i = 4 * tid; i < n; i += 4 * nt) {
        float4 v = load4<A16>(b + r0 + i);
        if (b2) {
            const float4 u = load4<A16>(b2 + r0 + i);
            v.x += u.x, v.y += u.y, v.z += u.z, v.w += u.w;
        }
        if (a) {
            const float4 x = load4<A16>(a + r0 + i);
            v = make_float4(x.x + v.x, x.y + v.y, x.z + v.z, x.w + v.w);
            store4<A16>(out + r0 + i, v);
        }
        *reinterpret_cast<float4*>(xs + (i >> 5) * 36 + (i & 31)) = v;
    }
    __syncthreads();
    for (int bl = tid; bl < nb; bl += nt) {
        const float* xb = xs + bl * 36;
        float sq = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float4 v = *reinterpret_cast<const float4*>(xb + 4 * k);
            sq += v.x * v.x;
            sq += v.y * v.y;
            sq += v.z * v.z;
            sq += v.w * v.w;
        }
        ss[bl] = sq;
    }
    __syncthreads();
    const float r = rmsScale(ss, nb, n, eps);
    int* qr = q ? q + (size_t)row * nsb * 85 : nullptr;
    for (int sb = wave; sb < nsb; sb += nt >> 6) {
        const int e = sb * 256 + 4 * lane;
        const float4 xv = *reinterpret_cast<const float4*>(xs + (e >> 5) * 36 + (e & 31));
        const float4 wv = load4<A16>(w + e);
        const float4 yv = make_float4(xv.x * r * wv.x, xv.y * r * wv.y, xv.z * r * wv.z, xv.w * r * wv.w);
        if (y) store4<A16>(y + r0 + e, yv);  // the normed row itself (the input of F16 matrices)
        quant256Wave(yv.x, yv.y, yv.z, yv.w, qr, nsb, sb, ao, has_ao != 0, row);
    }
}

// ---------------------------------------------------------------- FLASH_ATTN_EXT over an fp16 cache

__device__ __forceinline__ float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (unsigned short)h); }

struct Fa {  // kcFaDims, as kernel arguments
    int H, T, D, group, tp, k_row, k_head, v_row, v_head, N, q_tok, q_head, m_row, has_mask, H_kv;
};

__device__ __forceinline__ float maskAt(const int* mask, const Fa& d, int i, int t) {
    if (!d.has_mask) return 0.0f;
    const uint32_t w = (uint32_t)mask[(size_t)i * d.m_row + t / 2];
    return h2f((w >> ((t & 1) * 16)) & 0xFFFFu);
}

// s[(h * N + i) * tp + t] = scale * q.K + mask (fa_scores.cu): one thread per (head, query, t).
__global__ void fa_scores_kernel(const float* __restrict__ q, const int* __restrict__ k, const int* __restrict__ mask,
                                 float* __restrict__ s, Fa d, float scale) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long per = (long long)d.N * d.tp;
    if (idx >= (long long)d.H * per) return;
    const int h = (int)(idx / per);
    const int r = (int)(idx - (long long)h * per);
    const int i = r / d.tp, t = r - i * d.tp;
    if (t >= d.T) return;
    const int kvh = h / d.group;
    const float* qh = q + (size_t)i * d.q_tok + (size_t)h * d.q_head;
    const int* kr = k + (size_t)t * d.k_row + (size_t)kvh * d.k_head;
    float a = 0.0f;
    for (int j = 0; j < d.D / 2; ++j) {
        const uint32_t w = (uint32_t)kr[j];
        a += qh[2 * j] * h2f(w & 0xFFFFu) + qh[2 * j + 1] * h2f(w >> 16);
    }
    s[idx] = scale * a + maskAt(mask, d, i, t);
}

__global__ void fa_max_kernel(const float* __restrict__ s, float* __restrict__ m, Fa d) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= d.H * d.N) return;
    const float* sr = s + (size_t)row * d.tp;
    float mx = sr[0];
    for (int t = 1; t < d.T; ++t) mx = fmaxf(mx, sr[t]);
    m[row] = mx;
}

__global__ void fa_exp_kernel(float* __restrict__ s, const float* __restrict__ m, Fa d) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)d.H * d.N * d.tp) return;
    const int row = (int)(idx / d.tp), t = (int)(idx - (long long)row * d.tp);
    if (t < d.T) s[idx] = exp2f((s[idx] - m[row]) * kLog2e);
}

// out[(i * H + h) * D + dd] = sum_t p * V / sum_t p (fa_values.cu): one thread per (query, head, dd).
__global__ void fa_values_kernel(const float* __restrict__ p, const int* __restrict__ v, float* __restrict__ out,
                                 Fa d) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= d.N * d.H * d.D) return;
    const int i = idx / (d.H * d.D);
    const int r = idx - i * d.H * d.D;
    const int h = r / d.D, dd = r - h * d.D;
    const int kvh = h / d.group;
    const float* pr = p + ((size_t)h * d.N + i) * d.tp;
    const int* vc = v + (size_t)kvh * d.v_head + dd / 2;
    const int sh = (dd & 1) * 16;
    float a = 0.0f, sum = 0.0f;
    for (int t = 0; t < d.T; ++t) {
        const float x = h2f(((uint32_t)vc[(size_t)t * d.v_row] >> sh) & 0xFFFFu);
        a += pr[t] * x;
        sum += pr[t];
    }
    out[idx] = a / sum;
}

// Fused single-kernel attention for decode and short prefills: one workgroup per (query, head).
// Scores go to LDS (T <= kFaMaxT), the softmax uses the row maximum and exp2 as the four-kernel
// path does, and the value sums run over t with the workgroup's threads split over (dd, t-slices).
__global__ __launch_bounds__(256) void flash_attn_kernel(const float* __restrict__ q, const int* __restrict__ k,
                                                         const int* __restrict__ v, const int* __restrict__ mask,
                                                         float* __restrict__ out, Fa d, float scale) {
    extern __shared__ float lds[];
    float* sc = lds;              // [T]
    float* red = lds + d.T;       // [256] reduction scratch
    const int i = blockIdx.x / d.H, h = blockIdx.x - i * d.H;
    const int kvh = h / d.group;
    const int tid = threadIdx.x;
    const float* qh = q + (size_t)i * d.q_tok + (size_t)h * d.q_head;
    // scores: one thread per position, q from L1
    float mx = -INFINITY;
    for (int t = tid; t < d.T; t += 256) {
        const int* kr = k + (size_t)t * d.k_row + (size_t)kvh * d.k_head;
        float a = 0.0f;
        for (int j = 0; j < d.D / 2; ++j) {
            const uint32_t w = (uint32_t)kr[j];
            a += qh[2 * j] * h2f(w & 0xFFFFu) + qh[2 * j + 1] * h2f(w >> 16);
        }
        const float sv = scale * a + maskAt(mask, d, i, t);
        sc[t] = sv;
        mx = fmaxf(mx, sv);
    }
    red[tid] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) red[tid] = fmaxf(red[tid], red[tid + o]);
        __syncthreads();
    }
    const float m = red[0];
    __syncthreads();
    for (int t = tid; t < d.T; t += 256) sc[t] = exp2f((sc[t] - m) * kLog2e);
    __syncthreads();
    // values: threads split as (dd, slice); each slice sums a strided subset of t
    const int slices = 256 / d.D > 0 ? 256 / d.D : 1;
    for (int dd0 = 0; dd0 < d.D; dd0 += 256 / slices) {
        const int dd = dd0 + tid % (256 / slices);
        const int sl = tid / (256 / slices);
        float a = 0.0f, sum = 0.0f;
        if (dd < d.D && sl < slices) {
            const int* vc = v + (size_t)kvh * d.v_head + dd / 2;
            const int sh = (dd & 1) * 16;
            for (int t = sl; t < d.T; t += slices) {
                const float x = h2f(((uint32_t)vc[(size_t)t * d.v_row] >> sh) & 0xFFFFu);
                a += sc[t] * x;
                sum += sc[t];
            }
        }
        red[tid] = a;
        __syncthreads();
        if (sl == 0 && dd < d.D) {
            float at = 0.0f;
            for (int j = 0; j < slices; ++j) at += red[j * (256 / slices) + tid % (256 / slices)];
            red[tid] = at;
        }
        // row sum of p: one more pass over the same slices
        __syncthreads();
        const float at = (sl == 0 && dd < d.D) ? red[tid] : 0.0f;
        __syncthreads();
        red[tid] = sum;
        __syncthreads();
        if (sl == 0 && dd < d.D) {
            float st = 0.0f;
            for (int j = 0; j < slices; ++j) st += red[j * (256 / slices) + tid % (256 / slices)];
            out[((size_t)i * d.H + h) * d.D + dd] = at / st;
        }
        __syncthreads();
    }
}

Fa toFa(const kcFaDims& x) {
    return Fa{x.H, x.T, x.D, x.group, x.tp, x.k_row, x.k_head, x.v_row, x.v_head, x.N, x.q_tok, x.q_head, x.m_row,
              x.has_mask, x.H_kv};
}

unsigned blocksFor(long long threads) { return (unsigned)((threads + 255) / 256); }
// Threads of a workgroup that handles one row of n values per 256 with one wavefront per
// super-block (at most 16 wavefronts, at least 4).
int waveThreads(int n) { return 64 * std::min(16, std::max(4, n / 256)); }

}  // namespace

int launchVectorAdd(const float* a, const float* b, float* out, int count, hipStream_t s) {
    if (count == 0) return 0;
    hipLaunchKernelGGL(vector_add_kernel, dim3(blocksFor(count)), dim3(256), 0, s, a, b, out, count);
    return fromHip(hipGetLastError(), "vector_add");
}

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int launchAddSumsq(const float* a, const float* b, float* out, int* q, int n, int rows, hipStream_t s,
                   const float* b2) {
    if (rows <= 0 || n <= 0) return 0;
    const dim3 grid(rows, blocksFor(n / 4));
    if (al16(b) && (!b2 || al16(b2)) && (!a || (al16(a) && al16(out))))
        hipLaunchKernelGGL(add_sumsq_kernel<true>, grid, dim3(256), 0, s, a, b, b2, out, q, n, rows);
    else
        hipLaunchKernelGGL(add_sumsq_kernel<false>, grid, dim3(256), 0, s, a, b, b2, out, q, n, rows);
    return fromHip(hipGetLastError(), a ? "add_sumsq_f" : "sumsq_part");
}

int launchNormMulQ8(bool per256, const kcNormMulQ8Args& a, hipStream_t s) {
    if (per256 && a.rows > 0) {
        if (al16(a.x) && al16(a.w) && al16(a.y))
            hipLaunchKernelGGL(norm_mul_q8k_kernel<true>, dim3(a.rows), dim3(256), 0, s, a.x, a.w, a.y, a.q, a.n,
                               a.rows, a.eps);
        else
            hipLaunchKernelGGL(norm_mul_q8k_kernel<false>, dim3(a.rows), dim3(256), 0, s, a.x, a.w, a.y, a.q, a.n,
                               a.rows, a.eps);
    } else if (!per256 && a.rows > 0 && a.n > 0) {
        const dim3 grid(a.rows, blocksFor(a.n / 4));
        if (al16(a.x) && al16(a.w) && al16(a.y))
            hipLaunchKernelGGL(norm_mul_q8_kernel<true>, grid, dim3(256), 0, s, a.x, a.w, a.y, a.q, a.n, a.rows, a.eps);
        else
            hipLaunchKernelGGL(norm_mul_q8_kernel<false>, grid, dim3(256), 0, s, a.x, a.w, a.y, a.q, a.n, a.rows, a.eps);
    }
    return fromHip(hipGetLastError(), per256 ? "norm_mul_q8k_f" : "norm_mul_q8_f");
}

int launchAddNormQ8(const float* a, const float* b, float* x, const float* w, float* y, int* q, int n, int rows,
                    float eps, hipStream_t s) {
    if (rows <= 0) return 0;
    if (n <= 0 || n % 256 || n > 8192) return fromHip(hipErrorInvalidValue, "add_norm_q8: row length");
    const int nq = n / 4, nth = std::min(1024, nq);
    const bool a16 = (!a || (al16(a) && al16(b))) && al16(x) && al16(w) && al16(y);
    if (nq <= 1024) {
        if (a16) hipLaunchKernelGGL((add_norm_q8_kernel<true, 1>), dim3(rows), dim3(nth), 0, s, a, b, x, w, y, q, n, eps);
        else hipLaunchKernelGGL((add_norm_q8_kernel<false, 1>), dim3(rows), dim3(nth), 0, s, a, b, x, w, y, q, n, eps);
    } else {
        if (a16) hipLaunchKernelGGL((add_norm_q8_kernel<true, 2>), dim3(rows), dim3(nth), 0, s, a, b, x, w, y, q, n, eps);
        else hipLaunchKernelGGL((add_norm_q8_kernel<false, 2>), dim3(rows), dim3(nth), 0, s, a, b, x, w, y, q, n, eps);
    }
    return fromHip(hipGetLastError(), "add_norm_q8_f");
}

int launchSiluMulQ8(bool per256, const kcSiluMulQ8FArgs& a, hipStream_t s) {
    if (per256 && a.cols > 0) {
        if (al16(a.g) && al16(a.u) && al16(a.y))
            hipLaunchKernelGGL(silu_mul_q8k_kernel<true>, dim3(a.cols), dim3(256), 0, s, a.g, a.u, a.y, a.q, a.n, a.cols,
                               ActF16{}, 0);
        else
            hipLaunchKernelGGL(silu_mul_q8k_kernel<false>, dim3(a.cols), dim3(256), 0, s, a.g, a.u, a.y, a.q, a.n, a.cols,
                               ActF16{}, 0);
    } else if (!per256 && a.cols > 0 && a.n > 0) {
        const dim3 grid(a.cols, blocksFor(a.n / 4));
        if (al16(a.g) && al16(a.u) && al16(a.y))
            hipLaunchKernelGGL(silu_mul_q8_kernel<true>, grid, dim3(256), 0, s, a.g, a.u, a.y, a.q, a.n, a.cols);
        else
            hipLaunchKernelGGL(silu_mul_q8_kernel<false>, grid, dim3(256), 0, s, a.g, a.u, a.y, a.q, a.n, a.cols);
    }
    return fromHip(hipGetLastError(), per256 ? "silu_mul_q8kf" : "silu_mul_q8x4f");
}

int launchSiluMulQ8KAct(const kcSiluMulQ8FArgs& a, const ActF16* ao, hipStream_t s) {
    if (a.cols <= 0) return 0;
    if (!a.q && !ao) return fromHip(hipErrorInvalidValue, "silu_mul_q8kf: no quantized output");
    if (al16(a.g) && al16(a.u) && (!a.y || al16(a.y)))
        hipLaunchKernelGGL(silu_mul_q8k_kernel<true>, dim3(a.cols), dim3(waveThreads(a.n)), 0, s, a.g, a.u, a.y, a.q,
                           a.n, a.cols, ao ? *ao : ActF16{}, ao ? 1 : 0);
    else
        hipLaunchKernelGGL(silu_mul_q8k_kernel<false>, dim3(a.cols), dim3(waveThreads(a.n)), 0, s, a.g, a.u, a.y, a.q,
                           a.n, a.cols, ao ? *ao : ActF16{}, ao ? 1 : 0);
    return fromHip(hipGetLastError(), "silu_mul_q8kf");
}

int launchMulRows(const kcMulRowsArgs& a, hipStream_t s) {
    if (a.count == 0) return 0;
    hipLaunchKernelGGL(mul_rows_kernel, dim3(blocksFor(a.count)), dim3(256), 0, s, a.x, a.w, a.y, a.n, a.count);
    return fromHip(hipGetLastError(), "mul_rows");
}

int launchSiluMul(const kcSiluMulArgs& a, hipStream_t s) {
    if (a.count == 0) return 0;
    hipLaunchKernelGGL(silu_mul_kernel, dim3(blocksFor(a.count)), dim3(256), 0, s, a.g, a.u, a.out, a.count);
    return fromHip(hipGetLastError(), "silu_mul");
}

int launchRmsNorm(const kcRmsNormArgs& a, hipStream_t s) {
    if (a.rows == 0) return 0;
    const bool a16 = (reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.y) |
                      reinterpret_cast<uintptr_t>(a.w)) % 16 == 0;
    if (a.n > 0 && a.n <= kNormLaneMax && a.n % 4 == 0 && 64 % (a.n / 4) == 0 && a16)
        hipLaunchKernelGGL(rms_norm_lane_kernel, dim3((unsigned)((a.rows + 63) / 64)), dim3(64), 0, s, a.x, a.w, a.y,
                           a.n, a.rows, a.eps);
    else if (a.n > 0 && a.n <= 16384)
        hipLaunchKernelGGL(rms_norm_row_kernel, dim3(a.rows), dim3(64), (size_t)a.n * 4, s, a.x, a.w, a.y, a.n, a.eps);
    else
        hipLaunchKernelGGL(rms_norm_kernel, dim3(blocksFor(a.rows)), dim3(256), 0, s, a.x, a.w, a.y, a.n, a.rows,
                           a.eps);
    return fromHip(hipGetLastError(), "rms_norm");
}

int launchRope(const kcRopeGgmlArgs& a, hipStream_t s) {
    const int pairs = a.head_dim / 2;
    const long long count = (long long)pairs * a.n_head * a.n_tokens;
    if (count <= 0) return 0;
    if (count > INT32_MAX) return fromHip(hipErrorInvalidValue, "rope_ggml: more than 2^31 pairs");
    hipLaunchKernelGGL(rope_kernel, dim3(blocksFor(count)), dim3(256), 0, s, a.x, a.y, a.pos, a.ff, pairs, a.n_head,
                       (int)count, a.log2_base, a.neox ? 1 : 2, a.neox ? pairs : 1);
    return fromHip(hipGetLastError(), "rope_ggml");
}

int launchNormRopeQKStore(const float* q, float* qr, const float* k, const float* v, const float* qw, const float* kw,
                          int* kcache, int* vcache, const int* pos, const float* ff, int head_dim, int nh, int nkv,
                          int n, float log2_base, int neox, int dst_row, int dst_rows, float eps, hipStream_t s,
                          const float* v2) {
    const int pairs = head_dim / 2;
    if (n <= 0) return 0;
    if ((head_dim != 64 && head_dim != 128) || nh <= 0 || nkv <= 0 || !al16(q) || !al16(k))
        return fromHip(hipErrorInvalidValue, "q / k norm + rope + kv store: shape");
    const long long nqb = ((long long)n * nh + 63) / 64, nkb = ((long long)n * nkv + 63) / 64;
    if (nqb + nkb > INT32_MAX) return fromHip(hipErrorInvalidValue, "q / k norm + rope + kv store: rows");
    const int max_tok = 64 / std::min(nh, nkv) + 2;  // tokens one workgroup's 64 rows can span
    const size_t lds = sizeof(float) * (64 * (head_dim + 4) + 64 + 64 + 128) + sizeof(float) * 2 * (size_t)max_tok * pairs;
    hipLaunchKernelGGL(norm_rope_qk_store_kernel, dim3((unsigned)(nqb + nkb)), dim3(kNormRopeThreads), lds, s, q, qr, k,
                       v, v2, qw, kw, reinterpret_cast<unsigned short*>(kcache), reinterpret_cast<unsigned short*>(vcache),
                       pos, ff, pairs == 64 ? 6 : 5, nh, nkv, n, log2_base, neox ? 1 : 2, neox ? pairs : 1, dst_row,
                       dst_rows, eps, (int)nqb);
    return fromHip(hipGetLastError(), "q / k norm + rope + kv store");
}

int launchRopeQKStore(const float* q, float* qr, const float* k, const float* v, int* kcache, int* vcache,
                      const int* pos, const float* ff, int head_dim, int nh, int nkv, int n, float log2_base, int neox,
                      int dst_row, int dst_rows, hipStream_t s, const float* v2) {
    const int pairs = head_dim / 2;
    const long long threads = (long long)n * ((nh + nkv + 3) / 4) * pairs;
    hipLaunchKernelGGL(rope_qk_store_kernel, dim3(blocksFor(threads)), dim3(256), 0, s, q, qr, k, v, v2,
                       reinterpret_cast<unsigned short*>(kcache), reinterpret_cast<unsigned short*>(vcache), pos, ff,
                       pairs, nh, nkv, n, log2_base, neox ? 1 : 2, neox ? pairs : 1, dst_row, dst_rows);
    return fromHip(hipGetLastError(), "rope + kv store");
}

int launchRopeKvRows(const RopeKvRows& r, hipStream_t s) {
    const int pairs = r.head_dim / 2;
    const long long threads = (long long)r.n * ((r.nh + r.nkv + 3) / 4) * pairs;
    if (threads <= 0) return 0;
    hipLaunchKernelGGL(rope_kv_rows_kernel, dim3(blocksFor(threads)), dim3(256), 0, s, r.q, r.qr, r.k, r.kr,
                       const_cast<float*>(r.v),
                       reinterpret_cast<unsigned short*>(r.kcache), reinterpret_cast<unsigned short*>(r.vcache), r.pos,
                       r.idx, r.ff, pairs, r.nh, r.nkv, r.n, r.log2_base, r.neox ? 1 : 2, r.neox ? pairs : 1, r.src_v,
                       r.k_row, r.v_row, r.dst_rows, r.v2);
    return fromHip(hipGetLastError(), "rope + set_rows");
}

int launchAddNormQ8K(const float* a, const float* b, const float* b2, float* out, const float* w, int* q, int n,
                     int rows, float eps, hipStream_t s, const ActF16* ao, float* y) {
    if (rows <= 0) return 0;
    if (!q && !ao) return fromHip(hipErrorInvalidValue, "add + norm: no quantized output");
    const size_t lds = sizeof(float) * ((size_t)n / 32 * 37);
    if (n % 256 || lds > 65536) return fromHip(hipErrorInvalidValue, "add + norm: row length");
    // the register form wherever a row is at most four values per thread (option addnorm_lds = 1:
    // the LDS form always)
    const int nth = waveThreads(n), regs = 4 * nth >= n && option("addnorm_lds") != 1;
    if (al16(b) && (!b2 || al16(b2)) && (!a || (al16(a) && al16(out))) && al16(w) && (!y || al16(y)))
        hipLaunchKernelGGL(add_norm_q8k_kernel<true>, dim3(rows), dim3(nth), lds, s, a, b, b2, out, w, q, n, eps,
                           ao ? *ao : ActF16{}, ao ? 1 : 0, y, regs);
    else
        hipLaunchKernelGGL(add_norm_q8k_kernel<false>, dim3(rows), dim3(nth), lds, s, a, b, b2, out, w, q, n, eps,
                           ao ? *ao : ActF16{}, ao ? 1 : 0, y, regs);
    return fromHip(hipGetLastError(), "add + norm");
}

int launchSetRows(const kcSetRowsF16Args& a, hipStream_t s) {
    hipLaunchKernelGGL(set_rows_kernel, dim3(blocksFor((long long)a.pairs * a.rows)), dim3(256), 0, s, a.src, a.idx,
                       a.dst, a.pairs, a.rows, a.src_row, a.dst_row, a.dst_rows);
    return fromHip(hipGetLastError(), "set_rows_f16");
}

int launchFaScores(const kcFaScoresArgs& a, hipStream_t s) {
    const Fa d = toFa(a.d);
    hipLaunchKernelGGL(fa_scores_kernel, dim3(blocksFor((long long)d.H * d.N * d.tp)), dim3(256), 0, s, a.q, a.k,
                       a.mask, a.s, d, a.scale);
    return fromHip(hipGetLastError(), "fa_scores");
}

int launchFaMax(const kcFaMaxArgs& a, hipStream_t s) {
    const Fa d = toFa(a.d);
    hipLaunchKernelGGL(fa_max_kernel, dim3(blocksFor((long long)d.H * d.N)), dim3(256), 0, s, a.s, a.m, d);
    return fromHip(hipGetLastError(), "fa_max");
}

int launchFaExp(const kcFaExpArgs& a, hipStream_t s) {
    const Fa d = toFa(a.d);
    hipLaunchKernelGGL(fa_exp_kernel, dim3(blocksFor((long long)d.H * d.N * d.tp)), dim3(256), 0, s, a.s, a.m, d);
    return fromHip(hipGetLastError(), "fa_exp");
}

int launchFaValues(const kcFaValuesArgs& a, hipStream_t s) {
    const Fa d = toFa(a.d);
    hipLaunchKernelGGL(fa_values_kernel, dim3(blocksFor((long long)d.N * d.H * d.D)), dim3(256), 0, s, a.p, a.v,
                       a.out, d);
    return fromHip(hipGetLastError(), "fa_values");
}

int launchFlashAttn(const kcFlashAttnArgs& a, hipStream_t s) {
    const Fa d = toFa(a.d);
    const size_t lds = sizeof(float) * ((size_t)d.T + 256);
    static const int attr = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(flash_attn_kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != 0) return fromHip(attr, "flash_attn_f16: LDS size");
    hipLaunchKernelGGL(flash_attn_kernel, dim3(d.N * d.H), dim3(256), lds, s, a.q, a.k, a.v, a.mask, a.out, d,
                       a.scale);
    return fromHip(hipGetLastError(), "flash_attn_f16");
}

}  // namespace kcamd
