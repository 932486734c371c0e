// model_kernels.hip -- kernels the decode driver needs beyond the reference's kernel set (gfx950):
// token-embedding rows from a K-quant stream, attention whose context length and positions are
// read from device memory (so one captured hipGraph serves every decode step), the greedy argmax
// with its bookkeeping, and the per-step position update.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "internal.hpp"
#include "kquant.hpp"
#include "model_kernels.hpp"

namespace kcamd {
namespace {

__device__ __forceinline__ float f16v(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (unsigned short)h); }

// y[i][:] = dequantized row tok[i] of a Q4_K / Q6_K stream (ggml dequantize_row_q4_K / q6_K with
// the reference's operation order, llm/llm_reference.cpp:342-383). One thread per (token, 16 values).
// A row id outside [0, rows) (the ids are device data no host check has seen) yields zeros.
template <bool Q6>
__global__ void get_rows_kernel(const uint8_t* __restrict__ qw, const int* __restrict__ tok, float* __restrict__ y,
                                int n, int k, int rows) {
    const int nsb = k / 256, ngroups = (nsb + kGroupSb - 1) / kGroupSb;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)n * (k / 16)) return;
    const int i = (int)(idx / (k / 16));
    const int part = (int)(idx - (long long)i * (k / 16));  // 16 values
    const int s = part / 16, v0 = (part % 16) * 16;
    const int row = tok[i];
    if (row < 0 || row >= rows) {
        float* out = y + (size_t)i * k + part * 16;
        for (int l = 0; l < 16; ++l) out[l] = 0.0f;
        return;
    }
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


typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4* LdsS4;

// Causal attention of a batch of N queries (positions p0 .. p0 + N - 1, p0 = T - N, T = *n_ctx)
// on the matrix cores, v_mfma_f32_32x32x16_f16, in one pass over the keys per (query tile of 32,
// query head) workgroup of W wavefronts. k and v are fp16 in the cache; q and p are each split
// into two fp16 operands, hi = fp16(x) and lo = fp16(x - hi), and every product runs as two MFMAs,
// which keeps them within about 2^-22 of fp32 (one fp16 rounding of q or p would be 2^-11: enough
// to flip the 8-bit quantization of the attention output downstream). p is scaled by 2^10 before
// the split so that lo stays in fp16's normal range; the sum is divided back. Scores are computed
// transposed, S^T = K Q^T (A = K rows from the cache, B = q), which leaves each lane one query and
// 16 of the 32 keys of a block: lane (j, h) holds keys 8a + 4h + b (value 4a + b). Those registers
// are directly the A operand of P V when the MFMA's k index runs over the keys in that order,
// kappa(k) = {0,1,2,3,8,9,10,11 | 4,5,6,7,12,13,14,15} (+16 for the second half of the block).
// Wavefront w of the workgroup: wavefront w takes the key blocks kb = w, w + W, .. and keeps its own
// running maximum m and sum l per query (FLASH_ATTN_EXT's online softmax, ggml-cpu/ops.cpp), its
// output accumulators rescaled by exp(m_old - m_new) before each block's P V; at the end the
// partial results are merged, o = sum_w o_w exp(m_w - M) over l = sum_w l_w exp(m_w - M). Each
// wavefront loads the K fragments and V rows of its next block into registers while it computes
// the current one; V goes to the wavefront's own LDS buffer row-major (rows padded by 16 halves)
// and each lane takes its B operand, V[keys kappa(k)][d], from there by transposed reads. Query
// tiles are dispatched longest first.
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// MASKED: FLASH_ATTN_EXT's form for the ggml backend -- the N queries attend over T = t_host keys
// with ggml's f16 mask (row i of m_row2 halves: dot * scale + mask[i][key], the oracle's order)
// instead of the causal positions. msum holds the tile's mask summary (mask_summary_kernel): only
// its key blocks lo .. hi are read, and only blocks mlo .. mhi load and add the mask's values (the
// others hold 0 for every query of the tile); a block among those whose mask is -inf for every query
// of the tile is skipped (it would add nothing).
template <int D, int W, bool MASKED = false>
__global__ __launch_bounds__(64 * W) void attn_prefill_kernel(const float* __restrict__ q, const int* __restrict__ kc,
                                                               const int* __restrict__ vc, float* __restrict__ out,
                                                               const int* __restrict__ n_ctx, AttnShape a,
                                                               const unsigned short* __restrict__ mask = nullptr,
                                                               int m_row2 = 0, int t_host = 0,
                                                               const int* __restrict__ msum = nullptr) {
    constexpr int KS = D / 16, DB = D / 32;
    constexpr int VR = D + 16;       // halves per V row in LDS (8 dwords mod 32 banks: the four rows of a
                                     // transposed read's 16 lanes on different banks)
    constexpr int CPR = D / 8;       // 16-byte chunks per V row
    constexpr int RPL = 64 / CPR;    // V rows per wavefront load
    constexpr int VL = 32 / RPL;     // loads per V block
    // the V buffers, reused by the merge for the partial outputs of wavefronts 1 .. (rows of D + 4
    // floats: the lanes' 16-byte stores of different queries on different banks)
    constexpr int OR = D + 4;
    constexpr int kLdsHalves = W * 32 * VR > (W - 1) * 32 * OR * 2 ? W * 32 * VR : (W - 1) * 32 * OR * 2;
    __shared__ __attribute__((aligned(16))) _Float16 vsall[kLdsHalves];
    __shared__ __attribute__((aligned(16))) float qx[W][4][32];
    const int T = MASKED ? t_host : *n_ctx, N = a.N, p0 = T - N;
    const int tiles = (N + 31) / 32;
    const int i0 = (tiles - 1 - (int)blockIdx.x) * 32;
    const int head = blockIdx.y, kvh = head / (a.H / a.H_kv);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
    _Float16* vs = vsall + wave * 32 * VR;
    // this lane's row for the transposed V reads: group g = lane / 16 (lane half h = g / 2, d 16 (g % 2)
    // on), lane L = lane % 16 of it: key 4 h + L / 4, d 16 (g % 2) + 4 (L % 4)
    const int vlane = (4 * h + ((lane & 15) >> 2)) * VR + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const int* kb0 = kc + (size_t)kvh * (D / 2);
    const int* vb0 = vc + (size_t)kvh * (D / 2);
    h8 qb[KS], ql[KS];
    {
        const bool live = i0 + j < N;
        const float* qp = q + (size_t)min(i0 + j, N - 1) * a.q_tok + (size_t)head * D + 8 * h;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const float4 lo = *reinterpret_cast<const float4*>(qp + 16 * ks);
            const float4 hi = *reinterpret_cast<const float4*>(qp + 16 * ks + 4);
            const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = live ? v[e] : 0.0f;
                const _Float16 hq = (_Float16)x;
                qb[ks][e] = hq;
                ql[ks][e] = (_Float16)(x - (float)hq);
            }
        }
    }
    const int qpos = p0 + i0 + j;
    // key blocks bk0 .. bkend - 1 (causal: up to the tile's last query), those of mlo .. mhi with the
    // mask's values
    int bk0 = 0, bkend = min(p0 + i0 + 31, T - 1) / 32 + 1, mlo = 0, mhi = -1;
    if constexpr (MASKED) {
        const int* ms = msum + 4 * (i0 / 32);
        const int lo = ms[0], hi = ms[1];
        bk0 = lo <= hi ? lo : 0;
        bkend = lo <= hi ? hi + 1 : 0;
        mlo = ms[2];
        mhi = ms[3];
    }
    auto mixed = [&](int kb) { return MASKED && kb >= mlo && kb <= mhi; };
    // MASKED: this lane's 16 mask values of a key block (keys 32 kb + 8 g + 4 h + 0..3) as 8 words,
    // read inside the query's row (keys past it are dropped by key < T)
    const unsigned short* mrow = MASKED ? mask + (size_t)min(i0 + j, N - 1) * m_row2 : nullptr;
    uint32_t mk[8], mkn[8];
    auto loadM = [&](int kb, uint32_t* dst) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int w2 = 0; w2 < 2; ++w2) {
                const int key = min(kb * 32 + 8 * g + 4 * h + 2 * w2, m_row2 - 2);
                dst[2 * g + w2] = *reinterpret_cast<const uint32_t*>(mrow + key);
            }
    };
    f32x16 zero;
#pragma unroll
    for (int v = 0; v < 16; ++v) zero[v] = 0.0f;
    h8 ka[KS], kn[KS];
    u32x4v vr[VL];
    auto loadK = [&](int kb, h8* dst) {
        const int* kr = kb0 + (size_t)min(kb * 32 + j, T - 1) * a.kv_row + 4 * h;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) dst[ks] = *reinterpret_cast<const h8*>(kr + 8 * ks);
    };
    auto loadV = [&](int kb) {
#pragma unroll
        for (int r = 0; r < VL; ++r) {
            const int key = min(kb * 32 + r * RPL + lane / CPR, T - 1);
            vr[r] = *reinterpret_cast<const u32x4v*>(vb0 + (size_t)key * a.kv_row + (lane % CPR) * 4);
        }
    };
    // LDS ordering among the lanes of this wavefront (its own buffers; waves run different counts)
    auto waveSync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    if (bk0 + wave < bkend) {
        loadK(bk0 + wave, ka);
        loadV(bk0 + wave);
        if (mixed(bk0 + wave)) loadM(bk0 + wave, mk);
    }
    f32x16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = zero;
    float m = -INFINITY, l = 0.0f;
    for (int kb = bk0 + wave; kb < bkend; kb += W) {
        waveSync();  // the previous block's LDS reads are done
#pragma unroll
        for (int r = 0; r < VL; ++r)
            *reinterpret_cast<u32x4v*>(vs + (r * RPL + lane / CPR) * VR + (lane % CPR) * 8) = vr[r];
        const bool mx = mixed(kb), mxn = kb + W < bkend && mixed(kb + W);
        if (kb + W < bkend) {
            loadK(kb + W, kn);
            loadV(kb + W);
            if (mxn) loadM(kb + W, mkn);
        }
        float mval[16];
        if (!mx) {  // (the block's mask is 0 for every query of the tile)
#pragma unroll
            for (int v = 0; v < 16; ++v) mval[v] = 0.0f;
        } else {
            bool any = false;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t w2 = mk[v >> 1];
                mval[v] = (float)__builtin_bit_cast(_Float16, (unsigned short)((v & 1) ? (w2 >> 16) : (w2 & 0xFFFFu)));
                const int key_abs = kb * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                any |= key_abs < T && mval[v] != -INFINITY;
            }
            if (__ballot(any) == 0) {  // every score of the block masked: nothing to add
                if (kb + W < bkend) {
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) ka[ks] = kn[ks];
                    if (mxn)
#pragma unroll
                        for (int e = 0; e < 8; ++e) mk[e] = mkn[e];
                }
                continue;
            }
        }
        f32x16 sh = zero, sl = zero;  // two independent chains (q hi, q lo)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            sh = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[ks], qb[ks], sh, 0, 0, 0);
            sl = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[ks], ql[ks], sl, 0, 0, 0);
        }
        // the causal limit (MASKED: the mask's values) and the end of the context only in the blocks
        // that reach them (a uniform branch)
        f32x16 sacc;
        float bm = -INFINITY;
        if ((MASKED ? mx : kb * 32 + 31 > p0 + i0) || kb * 32 + 31 >= T) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int key_abs = kb * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                if constexpr (MASKED)
                    sacc[v] = key_abs < T ? a.scale * (sh[v] + sl[v]) + mval[v] : -INFINITY;
                else
                    sacc[v] = key_abs <= qpos && key_abs < T ? a.scale * (sh[v] + sl[v]) : -INFINITY;
                bm = fmaxf(bm, sacc[v]);
            }
        } else {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                sacc[v] = a.scale * (sh[v] + sl[v]);
                bm = fmaxf(bm, sacc[v]);
            }
        }
        bm = fmaxf(bm, __shfl_xor(bm, 32));
        const float mn = fmaxf(m, bm);
        // exp2 on the transcendental unit (v_exp_f32: exp2f's result for arguments from -126 up, 0
        // below, where p and alpha are absorbed by the sums they join); masked scores (-inf) give 0
        // without a branch, and so does alpha for a first block (m = -inf); a query with every score
        // so far masked (mn = -inf) subtracts 0 instead
        const float msafe = mn == -INFINITY ? 0.0f : mn;
        const float alpha = __builtin_amdgcn_exp2f((m - msafe) * kLog2e);
        m = mn;
        h8 pa[2], pl[2];
        float ls = 0.0f;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const float pv = __builtin_amdgcn_exp2f((sacc[v] - msafe) * kLog2e);
            ls += pv;
            const float ps = pv * 1024.0f;
            const _Float16 hp = (_Float16)ps;
            pa[v >> 3][v & 7] = hp;
            pl[v >> 3][v & 7] = (_Float16)(ps - (float)hp);
        }
        l = l * alpha + ls;
        waveSync();  // V block staged
        // rescale: O^T, so this lane's accumulators all hold its own query j
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[db][v] *= alpha;
#pragma unroll
        for (int mm = 0; mm < 2; ++mm)
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                // O^T += V^T P^T: the A operand V^T[32 db + j][keys 16 mm + 8 (e / 4) + 4 h + e % 4],
                // e = 0..7, by two transposed reads (ds_read_b64_tr_b16: in each group of 16 lanes,
                // lane i receives element i % 4 of the four halves lanes 4 e + i / 4 address; lane L
                // addresses V[key + L / 4][d0 + 4 (L % 4)]); the B operand P^T, the lane's query j
                const _Float16* vp = vs + vlane + 16 * mm * VR + 32 * db;
                const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LdsS4)vp);
                const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LdsS4)(vp + 8 * VR));
                const h8 vbv = __builtin_bit_cast(h8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vbv, pa[mm], o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vbv, pl[mm], o[db], 0, 0, 0);
            }
        if (kb + W < bkend) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) ka[ks] = kn[ks];
            if (mxn)
#pragma unroll
                for (int e = 0; e < 8; ++e) mk[e] = mkn[e];
        }
    }
    // ---- merge: wavefronts 1.. hand (m, l, o) to wavefront 0 through LDS
    l += __shfl_xor(l, 32);
    __syncthreads();  // every wavefront is done with its V buffer
    if (h == 0) {
        qx[wave][1][j] = m;
        qx[wave][2][j] = l;
    }
    // lane (j, h) holds O^T[d][j] for d = 32 db + 8 (v / 4) + 4 h + v % 4: query j's row, four
    // consecutive d per group of four v
    float* ob = reinterpret_cast<float*>(vsall);  // [W - 1][32 queries][OR]
    if (wave > 0) {
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4)
                *reinterpret_cast<float4*>(ob + ((wave - 1) * 32 + j) * OR + 32 * db + 8 * g4 + 4 * h) =
                    make_float4(o[db][4 * g4], o[db][4 * g4 + 1], o[db][4 * g4 + 2], o[db][4 * g4 + 3]);
    }
    __syncthreads();
    if (wave != 0) return;
    if (h == 0) {  // per query: the merged maximum, each wavefront's factor and the merged sum
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, qx[w][1][j]);
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float mw = qx[w][1][j];
            const float c = mw == -INFINITY ? 0.0f : exp2f((mw - M) * kLog2e);
            qx[w][3][j] = c;
            L += qx[w][2][j] * c;
        }
        qx[0][0][j] = L;
    }
    waveSync();
    if (i0 + j < N) {
        const float inv = 1.0f / (qx[0][0][j] * 1024.0f);
        const float c0 = qx[0][3][j];
        float* orow = out + (size_t)(i0 + j) * a.q_tok + (size_t)head * D;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d = 32 * db + 8 * g4 + 4 * h;
                float r[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float acc = o[db][4 * g4 + e] * c0;
#pragma unroll
                    for (int w = 1; w < W; ++w) acc += ob[((w - 1) * 32 + j) * OR + d + e] * qx[w][3][j];
                    r[e] = acc * inv;
                }
                *reinterpret_cast<float4*>(orow + d) = make_float4(r[0], r[1], r[2], r[3]);
            }
    }
}

}  // namespace

// ggml's f16 mask summarised per tile of 32 query rows (rows from N on read row N - 1) for the
// masked attention kernels: {lo, hi, mlo, mhi} = the first and last 32-key block holding a value
// other than -inf (keys below T; lo > hi when there is none), and the first and last block of lo ..
// hi holding a value other than +-0 (-inf included; mlo > mhi when there is none), so that blocks of
// lo .. hi outside mlo .. mhi hold 0 for every query of the tile: adding their values changes no
// score. A causal mask gives lo = 0 and mlo = mhi = hi, the diagonal block. One workgroup of 16
// wavefronts per tile, a wavefront per key block at a time: lane l reads row l / 2, keys 16 (l % 2) ..
// + 15, in 4-byte pairs inside the row (rows of m_row2 >= T halves, 4-byte aligned). Past
// kMaskBlocks blocks the flags do not fit in LDS and mlo .. mhi = lo .. hi (every block with values).
constexpr int kMaskBlocks = 8192;
constexpr int kMaskWaves = 16;

__global__ __launch_bounds__(64 * kMaskWaves) void mask_summary_kernel(const unsigned short* __restrict__ mask,
                                                                       int m_row2, int N, int T,
                                                                       int* __restrict__ sum) {
    __shared__ uint8_t nz[kMaskBlocks];  // per block: a value other than +-0
    __shared__ int red[2 * kMaskWaves];
    const int tile = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nkb = (T + 31) / 32;
    const unsigned short* mr = mask + (size_t)min(tile * 32 + lane / 2, N - 1) * m_row2;
    int lo = INT_MAX, hi = -1;
    for (int b = wave; b < nkb; b += kMaskWaves) {
        bool live = false, nonzero = false;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // keys k, k + 1; past T the load is clamped into the row and counts for nothing
            // (unconditional: a load under a branch is waited for alone)
            const int k = b * 32 + 16 * (lane & 1) + 2 * e;
            const int k0 = min(k, m_row2 - 2);  // (T = m_row2 odd: the row's last pair, key k at its end)
            const uint32_t w = *reinterpret_cast<const uint32_t*>(mr + k0);
#pragma unroll
            for (int x = 0; x < 2; ++x) {
                const int key = k0 + x;
                const uint32_t hv = x ? w >> 16 : w & 0xFFFFu;
                if (key >= k && key < T) {
                    live |= hv != 0xFC00u;
                    nonzero |= (hv & 0x7FFFu) != 0;
                }
            }
        }
        const bool bl = __ballot(live) != 0, bn = __ballot(nonzero) != 0;
        if (bl) {
            lo = min(lo, b);
            hi = max(hi, b);
        }
        if (lane == 0 && b < kMaskBlocks) nz[b] = bn ? 1 : 0;
    }
    if (lane == 0) {
        red[2 * wave] = lo;
        red[2 * wave + 1] = hi;
    }
    __syncthreads();
    for (int w = 0; w < kMaskWaves; ++w) {
        lo = min(lo, red[2 * w]);
        hi = max(hi, red[2 * w + 1]);
    }
    int ml = INT_MAX, mh = -1;
    if (nkb > kMaskBlocks) {
        ml = lo;
        mh = hi;
    } else {
        for (int b = max(lo, 0) + (int)threadIdx.x; b <= hi; b += 64 * kMaskWaves)
            if (nz[b]) {
                ml = min(ml, b);
                mh = max(mh, b);
            }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        ml = min(ml, __shfl_xor(ml, o));
        mh = max(mh, __shfl_xor(mh, o));
    }
    __syncthreads();  // red read by every thread
    if (lane == 0) {
        red[2 * wave] = ml;
        red[2 * wave + 1] = mh;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 0; w < kMaskWaves; ++w) {
            ml = min(ml, red[2 * w]);
            mh = max(mh, red[2 * w + 1]);
        }
        int* o = sum + 4 * tile;
        o[0] = lo;
        o[1] = hi;
        o[2] = ml;
        o[3] = mh;
    }
}

int launchGetRows(bool q6k, const void* qw, const int* tok, float* y, int n, int k, int rows, hipStream_t s) {
    const long long threads = (long long)n * (k / 16);
    if (threads == 0) return 0;
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (q6k) hipLaunchKernelGGL(get_rows_kernel<true>, grid, dim3(256), 0, s, (const uint8_t*)qw, tok, y, n, k, rows);
    else hipLaunchKernelGGL(get_rows_kernel<false>, grid, dim3(256), 0, s, (const uint8_t*)qw, tok, y, n, k, rows);
    return fromHip(hipGetLastError(), "get_rows");
}

// The query heads of a KV head in one workgroup (kattn_prefill.hip) when its grid of (query tile, KV
// head) workgroups fills the GPU; else one query head per workgroup, whose grid is G times larger
// (option attn_path = 3: always the former, 2: always the latter).
static bool useGqa(const AttnShape& a) {
    const int ap = option("attn_path");
    if (ap == 2 || !attnGqaSupports(a)) return false;
    return ap == 3 || (long long)((a.N + 31) / 32) * a.H_kv >= cuCount();
}

template <int D>
static int runPrefill(const float* q, const int* k, const int* v, float* out, const int* n_ctx, const AttnShape& a,
                       hipStream_t s) {
    if (useGqa(a)) return launchAttnGqa(q, k, v, out, n_ctx, a, nullptr, 0, 0, a.max_t, nullptr, s);
    const dim3 grid((a.N + 31) / 32, a.H);
    // key blocks split over 2 wavefronts for D = 128 (registers: one wavefront per SIMD), over 4
    // for D = 64 (two per SIMD)
    if (D == 128)
        hipLaunchKernelGGL((attn_prefill_kernel<D, 2>), grid, dim3(128), 0, s, q, k, v, out, n_ctx, a);
    else
        hipLaunchKernelGGL((attn_prefill_kernel<D, 4>), grid, dim3(256), 0, s, q, k, v, out, n_ctx, a);
    return fromHip(hipGetLastError(), "attn (prefill)");
}

bool attnMaskedSupports(const AttnShape& a) { return a.D == 64 || a.D == 128; }

int launchAttnMasked(const float* q, const int* k, const int* v, const unsigned short* mask, int m_row2, int T,
                     float* out, const AttnShape& a, const int* msum, hipStream_t s) {
    if (!attnMaskedSupports(a) || m_row2 < 2 || m_row2 % 2 || T <= 0 || T > m_row2 || a.N <= 0 || !msum)
        return fromHip(hipErrorInvalidValue, "attn (masked): shape");
    if (useGqa(a)) return launchAttnGqa(q, k, v, out, nullptr, a, mask, m_row2, T, T, msum, s);
    const dim3 grid((a.N + 31) / 32, a.H);
    if (a.D == 128)
        hipLaunchKernelGGL((attn_prefill_kernel<128, 2, true>), grid, dim3(128), 0, s, q, k, v, out, nullptr, a, mask,
                           m_row2, T, msum);
    else
        hipLaunchKernelGGL((attn_prefill_kernel<64, 4, true>), grid, dim3(256), 0, s, q, k, v, out, nullptr, a, mask,
                           m_row2, T, msum);
    return fromHip(hipGetLastError(), "attn (masked)");
}

int maskSummaryInts(int N) { return 4 * ((N + 31) / 32); }

int launchMaskSummary(const unsigned short* mask, int m_row2, int N, int T, int* sum, hipStream_t s) {
    if (m_row2 < 2 || m_row2 % 2 || T <= 0 || T > m_row2 || N <= 0 || !mask || !sum)
        return fromHip(hipErrorInvalidValue, "mask summary: shape");
    hipLaunchKernelGGL(mask_summary_kernel, dim3((N + 31) / 32), dim3(64 * kMaskWaves), 0, s, mask, m_row2, N, T, sum);
    return fromHip(hipGetLastError(), "mask summary");
}

int launchAttn(const float* q, const int* k, const int* v, float* out, const int* n_ctx, const AttnShape& a,
               hipStream_t s) {
    const int ap = option("attn_path");
    if (a.N > 1 && a.causal && ap != 1 && (a.D == 64 || a.D == 128)) {  // matrix cores, one pass
        return a.D == 128 ? runPrefill<128>(q, k, v, out, n_ctx, a, s) : runPrefill<64>(q, k, v, out, n_ctx, a, s);
    }
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
