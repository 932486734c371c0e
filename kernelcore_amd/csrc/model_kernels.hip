// model_kernels.hip -- kernels the decode driver needs beyond the reference's kernel set (gfx950):
// token-embedding rows from a K-quant stream, attention whose context length and positions are
// read from device memory (so one captured hipGraph serves every decode step), the greedy argmax
// with its bookkeeping, and the per-step position update.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "internal.hpp"
#include "kquant.hpp"
#include "model_kernels.hpp"

namespace kcamd {
namespace {

__device__ __forceinline__ float f16v(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (unsigned short)h); }

// y[i][:] = dequantized row tok[i] of a Q4_K / Q6_K stream (ggml dequantize_row_q4_K / q6_K with
// the reference's operation order, llm/llm_reference.cpp:342-383). One thread per (token, 16 values).
template <bool Q6>
__global__ void get_rows_kernel(const uint8_t* __restrict__ qw, const int* __restrict__ tok, float* __restrict__ y,
                                int n, int k) {
    const int nsb = k / 256, ngroups = (nsb + kGroupSb - 1) / kGroupSb;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)n * (k / 16)) return;
    const int i = (int)(idx / (k / 16));
    const int part = (int)(idx - (long long)i * (k / 16));  // 16 values
    const int s = part / 16, v0 = (part % 16) * 16;
    const int row = tok[i];
    const int tile = row >> 4, r = row & 15, g = s >> 2, kq = s & 3;
    const uint8_t* seg = qw + ((size_t)tile * ngroups + g) * (Q6 ? kQ6kSeg : kQ4kSeg);
    const uint8_t* piece = seg + (kq * 16 + r) * 16;  // byte b of the block: slab b / 16, offset b % 16
    auto at = [&](int b) -> uint32_t { return piece[(b >> 4) * 1024 + (b & 15)]; };
    float* out = y + (size_t)i * k + s * 256 + v0;
    if (!Q6) {
        const float d = f16v(at(0) | (at(1) << 8)), dmin = f16v(at(2) | (at(3) << 8));
        const int jj = v0 / 64, hi = (v0 % 64) / 32, l0 = v0 % 32;  // 64 values per qs group of 32 bytes
        const int j = 2 * jj + hi;                                   // sub-block of 32
        int sc, m;
        if (j < 4) {
            sc = at(4 + j) & 63;
            m = at(8 + j) & 63;
        } else {
            sc = (at(12 + j - 4) & 0xF) | ((at(4 + j - 4) >> 6) << 4);
            m = (at(12 + j - 4) >> 4) | ((at(4 + j) >> 6) << 4);
        }
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        for (int l = 0; l < 16; ++l) {
            const uint32_t b = at(16 + 32 * jj + l0 + l);
            out[l] = d1 * (float)(hi ? (b >> 4) : (b & 0xF)) - m1;
        }
    } else {
        const float d = f16v(*reinterpret_cast<const uint16_t*>(seg + kQ6kSlabs * 1024 + (kq * 16 + r) * 2));
        const int nh = v0 / 128, quad = (v0 % 128) / 32, l0 = v0 % 32;
        const int scv = (int)(int8_t)at(192 + 8 * nh + l0 / 16 + 2 * quad);
        for (int l = 0; l < 16; ++l) {
            const int ll = l0 + l;
            const uint32_t qlb = at(64 * nh + ll + ((quad & 1) ? 32 : 0));
            const uint32_t qhb = at(128 + 32 * nh + ll);
            const int q = (int)(((quad >> 1) ? (qlb >> 4) : (qlb & 0xF)) | (((qhb >> (2 * quad)) & 3) << 4)) - 32;
            out[l] = d * (float)scv * (float)q;
        }
    }
}

// Attention over an fp16 KV cache for the decode driver. One workgroup per (query i, head h).
// Context: T = *n_ctx positions (read on the device); causal: query i sees t <= T - n + i.
// Same math as FLASH_ATTN_EXT (fa_scores / fa_exp / fa_values): s = scale * q.K, p = exp2((s - max)
// * log2 e), out = sum p V / sum p. Scores live in LDS (T <= max_t). 16 lanes per position:
// each lane holds 8 of the 128 query values and the dot product is reduced across the 16.
constexpr float kLog2e = 1.44269504f;
__global__ __launch_bounds__(256) void attn_kernel(const float* __restrict__ q, const int* __restrict__ kc_,
                                                   const int* __restrict__ vc, float* __restrict__ out,
                                                   const int* __restrict__ n_ctx, AttnShape a) {
    extern __shared__ float lds[];
    float* sc = lds;            // [max_t]
    float* red = lds + a.max_t; // [256 + 64]
    const int i = blockIdx.x / a.H, h = blockIdx.x - i * a.H;
    const int kvh = h / (a.H / a.H_kv);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int T_all = *n_ctx;
    const int T = a.causal ? T_all - a.N + i + 1 : T_all;
    const float* qh = q + (size_t)i * a.q_tok + (size_t)h * a.D;
    // scores: 16 lanes per position, 16 positions per workgroup step
    const int sub = lane >> 4, l16 = lane & 15;  // position slot within the wave, lane within it
    const int dpl = a.D / 16;                    // values per lane (D <= 256)
    float qv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) qv[e] = e < dpl ? qh[l16 * dpl + e] : 0.0f;
    float mx = -INFINITY;
    for (int t0 = 0; t0 < T; t0 += 16) {
        const int t = t0 + wave * 4 + sub;
        float a2 = 0.0f;
        if (t < T) {
            const int* kr = kc_ + (size_t)t * a.kv_row + (size_t)kvh * (a.D / 2) + l16 * (dpl / 2);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (2 * e < dpl) {
                    const uint32_t w = (uint32_t)kr[e];
                    a2 += qv[2 * e] * f16v(w & 0xFFFFu) + qv[2 * e + 1] * f16v(w >> 16);
                }
            }
        }
        a2 += __shfl_xor(a2, 1, 16);
        a2 += __shfl_xor(a2, 2, 16);
        a2 += __shfl_xor(a2, 4, 16);
        a2 += __shfl_xor(a2, 8, 16);
        if (t < T && l16 == 0) {
            const float s = a.scale * a2;
            sc[t] = s;
            mx = fmaxf(mx, s);
        }
    }
    red[tid] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) red[tid] = fmaxf(red[tid], red[tid + o]);
        __syncthreads();
    }
    const float m = red[0];
    __syncthreads();
    for (int t = tid; t < T; t += 256) sc[t] = exp2f((sc[t] - m) * kLog2e);
    __syncthreads();
    // values: lane pairs per dd (dd = tid % D), the positions split over 256 / D slices
    const int slices = 256 / a.D;
    const int dd = tid % a.D, sl = tid / a.D;
    float acc = 0.0f, sum = 0.0f;
    const int* vcol = vc + (size_t)kvh * (a.D / 2) + dd / 2;
    const int sh = (dd & 1) * 16;
    for (int t = sl; t < T; t += slices) {
        const float p = sc[t];
        acc += p * f16v(((uint32_t)vcol[(size_t)t * a.kv_row] >> sh) & 0xFFFFu);
        sum += p;
    }
    red[tid] = acc;
    red[256 + (tid & 63)] = 0.0f;
    __syncthreads();
    float at = 0.0f;
    if (sl == 0)
        for (int j = 0; j < slices; ++j) at += red[j * a.D + dd];
    __syncthreads();
    red[tid] = sum;
    __syncthreads();
    if (sl == 0) {
        float st = 0.0f;
        for (int j = 0; j < slices; ++j) st += red[j * a.D + dd];
        out[((size_t)i * a.H + h) * a.D + dd] = at / st;
    }
}

// Greedy step: token = argmax(logits) (lowest index on ties); tokens[0] = token; gen[*step] =
// token; ++*step; ++*n_past. One workgroup of 1024 threads.
__global__ __launch_bounds__(1024) void argmax_step_kernel(const float* __restrict__ logits, int n, int* tokens,
                                                           int* gen, int* step, int* n_past, int max_gen) {
    __shared__ float bv[1024];
    __shared__ int bi[1024];
    const int tid = threadIdx.x;
    float best = -INFINITY;
    int besti = 0x7fffffff;
    for (int j = tid; j < n; j += 1024) {
        const float v = logits[j];
        if (v > best || (v == best && j < besti)) {
            best = v;
            besti = j;
        }
    }
    bv[tid] = best;
    bi[tid] = besti;
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
        if (tid < o) {
            const float v = bv[tid + o];
            const int j = bi[tid + o];
            if (v > bv[tid] || (v == bv[tid] && j < bi[tid])) {
                bv[tid] = v;
                bi[tid] = j;
            }
        }
        __syncthreads();
    }
    if (tid == 0) {
        const int tokn = bi[0] == 0x7fffffff ? 0 : bi[0];
        tokens[0] = tokn;
        const int st = *step;
        if (st < max_gen) gen[st] = tokn;
        *step = st + 1;
        if (n_past) *n_past = *n_past + 1;
    }
}

// Positions of the n tokens of a step: pos[i] = *n_past + i, idx[i] (int64) the same, and the
// context length the step attends over, n_ctx = *n_past + n.
__global__ void positions_kernel(const int* __restrict__ n_past, int n, int* pos, long long* idx, int* n_ctx) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int p0 = *n_past;
    if (i < n) {
        pos[i] = p0 + i;
        idx[i] = p0 + i;
    }
    if (i == 0) *n_ctx = p0 + n;
}

}  // namespace

int launchGetRows(bool q6k, const void* qw, const int* tok, float* y, int n, int k, hipStream_t s) {
    const long long threads = (long long)n * (k / 16);
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (q6k) hipLaunchKernelGGL(get_rows_kernel<true>, grid, dim3(256), 0, s, (const uint8_t*)qw, tok, y, n, k);
    else hipLaunchKernelGGL(get_rows_kernel<false>, grid, dim3(256), 0, s, (const uint8_t*)qw, tok, y, n, k);
    return fromHip(hipGetLastError(), "get_rows");
}

int launchAttn(const float* q, const int* k, const int* v, float* out, const int* n_ctx, const AttnShape& a,
               hipStream_t s) {
    const size_t lds = sizeof(float) * ((size_t)a.max_t + 256 + 64);
    static const int attr = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(attn_kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != 0) return fromHip(attr, "attn: LDS size");
    hipLaunchKernelGGL(attn_kernel, dim3(a.N * a.H), dim3(256), lds, s, q, k, v, out, n_ctx, a);
    return fromHip(hipGetLastError(), "attn");
}

int launchArgmaxStep(const float* logits, int n, int* tokens, int* gen, int* step, int* n_past, int max_gen,
                     hipStream_t s) {
    hipLaunchKernelGGL(argmax_step_kernel, dim3(1), dim3(1024), 0, s, logits, n, tokens, gen, step, n_past, max_gen);
    return fromHip(hipGetLastError(), "argmax");
}

int launchPositions(const int* n_past, int n, int* pos, long long* idx, int* n_ctx, hipStream_t s) {
    hipLaunchKernelGGL(positions_kernel, dim3((n + 255) / 256), dim3(256), 0, s, n_past, n, pos, idx, n_ctx);
    return fromHip(hipGetLastError(), "positions");
}

}  // namespace kcamd
