// kdecode.hip -- the single-token decode kernels of the model driver (gfx950).
//
// One token is latency-bound: every launch costs a few microseconds whatever it moves, so the
// layer is cut into six kernels instead of the reference graph's sixteen nodes:
//   1. dmv (norm prologue): RMS norm x weight + per-32 quantization of the residual row, done by
//      every workgroup into its own LDS, then the q / k / v matvecs in one grid;
//   2. attn_decode: per-head q / k RMS norm (Qwen3), RoPE, k and v into the fp16 cache, and the
//      attention split over the context in chunks of 64 positions;
//   3. attn_merge_wave: the merge of the partial softmaxes and the per-32 quantization of the
//      output, one wavefront per 64 outputs;
//   4. dmv (slot prologue, residual epilogue): attention output projection, x += o;
//   5. dmv (norm prologue, SwiGLU epilogue): FFN norm, gate and up matvecs, silu(g) * u and its
//      per-32 quantization;
//   6. dmv (slot prologue, residual epilogue): down projection, x += down.
// The matvec terms, norms, sums of squares and quantizations repeat the operations of the
// reference kernels they replace (kernels/llm/add_sumsq_f.cu, sumsq_part.cu, norm_mul_q8_f.cu,
// matvec_q4k_q8.cu, matvec_q6k_q8.cu, silu_mul_q8x4f.cu, rope_ggml.cu, set_rows_f16.cu in
// arasheedu/Kernelcore) in the same order, so the residual stream matches the unfused kernels
// bit for bit; the split softmax changes only the attention's rounding.
#include <hip/hip_runtime.h>

#include <type_traits>

#include <algorithm>

#include <cstdint>

#include "internal.hpp"
#include "kdecode.hpp"
#include "kquant_device.hpp"

namespace kcamd {
namespace {

constexpr int kXs = 68;  // LDS ints per super-block of activations (64 + 4 pad)
constexpr float kLog2e = 1.44269504f;
constexpr int kChunk = 64;  // attention positions per workgroup
constexpr int kMaxGroup = 8;  // query heads per KV head
// One (chunk, query head) row of the attention partials: D unnormalized output sums, then the
// running max and the sum of exponentials.
__host__ __device__ constexpr int partRow(int D) { return D + 2; }

// Round half away from zero and clamp to [-127, 127] (quantize_q8x4.cu): t + copysign(0.5, t) is
// t + 0.5 for t >= 0 and t - 0.5 below; for t = -0 it is -0.5, which truncates to the same 0.
__device__ __forceinline__ int q8r(float t) {
    const int q = (int)(t + __builtin_copysignf(0.5f, t));
    return q > 127 ? 127 : (q < -127 ? -127 : q);
}

// The low bytes of a, b, c, d as one word (a in the low byte): three byte permutes.
__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x0c0c0400u);
    return (int)__builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + exp2f(-g * kLog2e)); }

// fp32 -> fp16 bits as set_rows_f16.cu: nearest even, |x| >= 65520 -> +-0x7bff, -0 -> +0.
__device__ __forceinline__ uint32_t f2h(float x) {
    if (x == 0.0f) return 0;
    const uint32_t sign = x < 0.0f ? 0x8000u : 0u;
    if (!(fabsf(x) < 65520.0f)) return sign | 0x7bffu;
    return __builtin_bit_cast(unsigned short, (_Float16)x);
}

__device__ __forceinline__ float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (unsigned short)h); }

// Quantization of one block of 32 values by one thread (quantize_q8x4.cu:15-40, the reference's
// order): amax, d = amax / 127, q = round(v / d) packed four to a word; also the block's sum of q
// and the sum of its first 16 values. One thread per block keeps the work free of cross-lane
// traffic, whose latency would otherwise dominate these small kernels.
struct Q32 {
    int w[8];
    int sum, s16;
    float d;
};
__device__ __forceinline__ Q32 quant32Seq(const float* y) {
    // max and integer sums as balanced trees: both are exact, so the order does not matter and
    // the dependency chains stay short
    // (|y| here and max(y, 0 - y) in the reference differ only in the sign of a zero maximum,
    // which d = max(0, m) / 127 maps to the same 0)
    float m[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) m[i] = fmaxf(fabsf(y[i]), fabsf(y[i + 16]));
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) m[i] = fmaxf(m[i], m[i + w]);
    Q32 o;
    o.d = fmaxf(0.0f, m[0]) / 127.0f;
    float id;
    if (o.d > 0.0f) id = 1.0f / o.d;
    else id = 0.0f;
    int q[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) q[i] = q8r(y[i] * id);
#pragma unroll
    for (int k = 0; k < 8; ++k) o.w[k] = pack4(q[4 * k], q[4 * k + 1], q[4 * k + 2], q[4 * k + 3]);
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) {
            q[i] += q[i + w];
            q[16 + i] += q[16 + i + w];
        }
    o.s16 = q[0];
    o.sum = q[0] + q[16];
    return o;
}

// Block b of a quantized row into a per-32 slot: words at b * 8, (d, sum) at nb * 8 + 2b.
__device__ __forceinline__ void storeQ32(int* slot, int nb, int b, const Q32& q) {
    int4* w = reinterpret_cast<int4*>(slot + b * 8);
    w[0] = make_int4(q.w[0], q.w[1], q.w[2], q.w[3]);
    w[1] = make_int4(q.w[4], q.w[5], q.w[6], q.w[7]);
    *reinterpret_cast<float2*>(slot + nb * 8 + 2 * b) = make_float2(q.d, (float)q.sum);
}

// ---------------------------------------------------------------- fused decode matvec

// Activations in LDS, the matvec layout: xs[nsbp][kXs] words, per block of 32 its d, d * sum
// (Q4_K), sum (Q6_K) and the sum of its first 16 values (Q6_K).
struct Act {
    int* xs;
    float* dx;
    float* dsum;
    int* isum;
    int* s16;
    __device__ Act(int* base, int nsbp) {
        xs = base;
        dx = reinterpret_cast<float*>(xs + nsbp * kXs);
        dsum = dx + nsbp * 8;
        isum = reinterpret_cast<int*>(dsum + nsbp * 8);
        s16 = isum + nsbp * 8;
    }
    static constexpr int ints(int nsbp) { return nsbp * (kXs + 32); }
};

// Staging is split in two: the global loads into registers (issued before the weights' loads,
// so that waiting for them does not wait for the weights: the load counter drains in order),
// then the LDS work. Up to four 16-byte words per thread per array; the launchers check the fit.
// Loads are unconditional (clamped index): on this GPU a load under a branch gets a wait of its
// own, and each wait costs a memory round trip of about a microsecond.
typedef int i32x4 __attribute__((ext_vector_type(4)));  // (HIP's int4 struct copies through the stack)
struct StageRegs {
    i32x4 v[4];
    i32x4 u[4];
};

// The norm prologue holds block b = threadIdx.x (32 values of x and of w) in registers; the
// launchers keep n / 32 <= threads.
struct NormRegs {
    i32x4 x[8], w[8];
};
__device__ __forceinline__ void loadNorm(NormRegs& r, const float* x, const float* w, int n) {
    const int b = min((int)threadIdx.x, n / 32 - 1);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        r.x[k] = reinterpret_cast<const i32x4*>(x)[b * 8 + k];
        r.w[k] = reinterpret_cast<const i32x4*>(w)[b * 8 + k];
    }
}

// A per-32 slot: nsb * 16 int4 of words, nsb * 4 int4 of (d, sum) pairs.
__device__ __forceinline__ void loadSlot(StageRegs& r, const int* xq, const float* xd, int nsb) {
    const int tid = threadIdx.x, nth = blockDim.x, n4 = nsb * 16;
#pragma unroll
    for (int u = 0; u < 4; ++u) r.v[u] = reinterpret_cast<const i32x4*>(xq)[min(u * nth + tid, n4 - 1)];
    r.u[0] = reinterpret_cast<const i32x4*>(xd)[min(tid, nsb * 4 - 1)];
    r.u[1] = r.u[2] = r.u[3] = i32x4{0, 0, 0, 0};
}

// From a per-32 slot (xq words, xd = d, sum pairs). raw: LDS scratch of nsb * 16 floats and a
// dummy 16-byte word after them, the target of out-of-range stores: the stores are unconditional
// so that the compiler keeps their loads together at the top.
__device__ __forceinline__ void stageSlot(const Act& A, float* raw, const StageRegs& r, int nsb, int nsbp) {
    const int tid = threadIdx.x, nth = blockDim.x, n4 = nsb * 16;
    i32x4* dummy = reinterpret_cast<i32x4*>(raw + nsb * 16);
#pragma unroll
    for (int u = 0; u < 4; ++u) {  // xs rows are kXs = 68 ints apart: 16 words of 16 B per super-block
        const int i = u * nth + tid;
        i32x4* dst = i < n4 ? reinterpret_cast<i32x4*>(A.xs + (i >> 4) * kXs + (i & 15) * 4) : dummy;
        *dst = r.v[u];
    }
    *(tid < nsb * 4 ? reinterpret_cast<i32x4*>(raw) + tid : dummy) = r.u[0];
    for (int i = nsb * 64 + tid; i < nsbp * 64; i += nth) A.xs[(i >> 6) * kXs + (i & 63)] = 0;
    __syncthreads();
    for (int b = tid; b < nsbp * 8; b += nth) {
        float d = 0.0f, sm = 0.0f;
        int a = 0;
        if (b < nsb * 8) {
            d = raw[2 * b];
            sm = raw[2 * b + 1];
            const int* xw = A.xs + (b >> 3) * kXs + (b & 7) * 8;
            for (int w = 0; w < 4; ++w) a = dot4(0x01010101, xw[w], a);
        }
        A.dx[b] = d;
        A.dsum[b] = d * sm;
        A.isum[b] = (int)sm;
        A.s16[b] = a;
    }
}

// From the residual row x: per-32 sums of squares in order (sumsq_part.cu / add_sumsq_f.cu),
// their total in order, r = 1 / sqrt(total / n + eps), y = x * r * w and its per-32
// quantization (norm_mul_q8_f.cu), thread b on block b from registers. ss: LDS scratch of
// nsbp * 8 floats (16-byte aligned); the blocks' sums of squares are also returned there.
__device__ __forceinline__ void stageNorm(const Act& A, float* ss, const NormRegs& st, int n, float eps, int nsbp) {
    const int tid = threadIdx.x, nth = blockDim.x;
    const int nb = n / 32;
    float xv[32];
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int v = st.x[k][e];  // (copied out: bit_cast of a vector element reads element 0)
            xv[4 * k + e] = __builtin_bit_cast(float, v);
        }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) s += xv[i] * xv[i];
    if (tid < nb) ss[tid] = s;
    for (int b = nb + tid; b < nsbp * 8; b += nth) ss[b] = 0.0f;
    __syncthreads();
    // the total in block order; 16-byte reads, all issued before the adds. ss is zero from nb
    // to the next multiple of 32 (inside nsbp * 8), and tot + 0 = tot (tot >= 0).
    float tot = 0.0f;
    for (int j0 = 0; j0 < nb; j0 += 32) {
        float4 q[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) q[k] = reinterpret_cast<const float4*>(ss + j0)[k];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            tot += q[k].x;
            tot += q[k].y;
            tot += q[k].z;
            tot += q[k].w;
        }
    }
    const float r = 1.0f / sqrtf(tot / (float)n + eps);
    if (tid < nb) {
        float y[32];
#pragma unroll
        for (int k = 0; k < 8; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int wv = st.w[k][e];
                y[4 * k + e] = xv[4 * k + e] * r * __builtin_bit_cast(float, wv);
            }
        const Q32 q = quant32Seq(y);
        const int b = tid;
        i32x4* xw = reinterpret_cast<i32x4*>(A.xs + (b >> 3) * kXs + (b & 7) * 8);
        xw[0] = i32x4{q.w[0], q.w[1], q.w[2], q.w[3]};
        xw[1] = i32x4{q.w[4], q.w[5], q.w[6], q.w[7]};
        A.dx[b] = q.d;
        A.dsum[b] = q.d * (float)q.sum;
        A.isum[b] = q.sum;
        A.s16[b] = q.s16;
    }
    for (int b = nb + tid; b < nsbp * 8; b += nth) {  // padding blocks of the last group
        i32x4* xw = reinterpret_cast<i32x4*>(A.xs + (b >> 3) * kXs + (b & 7) * 8);
        xw[0] = xw[1] = i32x4{0, 0, 0, 0};
        A.dx[b] = 0.0f;
        A.dsum[b] = 0.0f;
        A.isum[b] = 0;
        A.s16[b] = 0;
    }
}

// Block quantization by the 8 lanes of an aligned group (lane j holds values 4j .. 4j+3 of the
// block): the same arithmetic as quant32Seq (the block maximum and the integer sums do not depend
// on the order of their terms; every value takes the same rounding), with the cross-lane steps as
// DPP moves inside a row of 16 lanes. Returns this lane's word (values 4j .. 4j+3); every lane gets
// d, the block's sum of q and the sum of its first 16 values.
struct Q8L {
    int w, sum, s16;
    float d;
};
template <int CTRL>
__device__ __forceinline__ int dppMovI(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dppMovF(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ Q8L quant8(const float (&y)[4]) {
    float m = fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3])));
    m = fmaxf(m, dppMovF<0xB1>(m));   // quad_perm [1,0,3,2]
    m = fmaxf(m, dppMovF<0x4E>(m));   // quad_perm [2,3,0,1]
    m = fmaxf(m, dppMovF<0x141>(m));  // row_half_mirror: the other quad of the 8
    Q8L o;
    o.d = fmaxf(0.0f, m) / 127.0f;
    float id;
    if (o.d > 0.0f) id = 1.0f / o.d;
    else id = 0.0f;
    const int q0 = q8r(y[0] * id), q1 = q8r(y[1] * id), q2 = q8r(y[2] * id), q3 = q8r(y[3] * id);
    o.w = pack4(q0, q1, q2, q3);
    int s = (q0 + q1) + (q2 + q3);
    s += dppMovI<0xB1>(s);
    s += dppMovI<0x4E>(s);  // every lane of the quad: the quad's sum (lanes 0-3: values 0-15)
    o.s16 = s;  // lane 0 (the lane that stores the block's scalars): the sum of values 0-15
    s += dppMovI<0x141>(s);
    o.sum = s;
    return o;
}

// The norm prologue with 8 lanes per block (thread t: block t / 8, values 4 (t % 8) .. +3; at most
// four passes of the workgroup): the per-32 sums of squares in element order as a chain through
// the 8 lanes (each lane continues the running sum it receives from its left neighbour: the same
// additions as one thread over 32 values), their total in block order, r, y = x * r * w and the
// 8-lane quantization. The x / w words of every pass are loaded first (NormRegs8).
typedef float f32x4v __attribute__((ext_vector_type(4)));
template <int NP>
struct NormRegs8 {
    i32x4 x[NP], w[NP];
};
template <int NP>
__device__ __forceinline__ void loadNorm8(NormRegs8<NP>& r, const float* x, const float* w, int n) {
    const int nth = blockDim.x, last = n / 4 - 1;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int t = min((int)threadIdx.x + p * nth, last);
        r.x[p] = reinterpret_cast<const i32x4*>(x)[t];
        r.w[p] = reinterpret_cast<const i32x4*>(w)[t];
    }
}
template <int NP>
__device__ __forceinline__ void stageNorm8(const Act& A, float* ss, const NormRegs8<NP>& st, int n, float eps,
                                           int nsbp) {
    const int tid = threadIdx.x, nth = blockDim.x, nb = n / 32, nq = n / 4;
    const int j = tid & 7;
    const int np = (nq + nth - 1) / nth;  // passes (<= NP: the launchers check)
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        if (p >= np) break;
        float xv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int v = st.x[p][e];
            xv[e] = __builtin_bit_cast(float, v);
        }
        // the running sum passes from lane j - 1 to lane j, eight steps; step k completes lane k
        float s = 0.0f, t = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            t = s;
#pragma unroll
            for (int e = 0; e < 4; ++e) t += xv[e] * xv[e];
            const float left = dppMovF<0x111>(t);  // row_shr:1: lane i - 1's value
            if (j == k + 1) s = left;
        }
        const int q = tid + p * nth;
        if (j == 7 && q < nq) ss[q >> 3] = t;
    }
    for (int b = nb + tid; b < nsbp * 8; b += nth) ss[b] = 0.0f;
    __syncthreads();
    // the total in block order; every 16-byte read issued before the adds (ss is zero past nb up
    // to a multiple of 32 inside nsbp * 8, and tot + 0 = tot)
    float tot = 0.0f;
    for (int j0 = 0; j0 < nb; j0 += 48) {
        f32x4v q[12];
#pragma unroll
        for (int k = 0; k < 12; ++k) q[k] = reinterpret_cast<const f32x4v*>(ss + j0)[min(k, (nsbp * 8 - j0) / 4 - 1)];
#pragma unroll
        for (int k = 0; k < 12; ++k) {
            if (j0 + 4 * k < nb) {
                tot += q[k][0];
                tot += q[k][1];
                tot += q[k][2];
                tot += q[k][3];
            }
        }
    }
    const float r = 1.0f / sqrtf(tot / (float)n + eps);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        if (p >= np) break;
        const int q = tid + p * nth;
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int xv = st.x[p][e], wv = st.w[p][e];
            y[e] = __builtin_bit_cast(float, xv) * r * __builtin_bit_cast(float, wv);
        }
        const Q8L o = quant8(y);
        if (q < nq) {
            const int b = q >> 3;
            A.xs[(b >> 3) * kXs + (b & 7) * 8 + j] = o.w;
            if (j == 0) {
                A.dx[b] = o.d;
                A.dsum[b] = o.d * (float)o.sum;
                A.isum[b] = o.sum;
                A.s16[b] = o.s16;
            }
        }
    }
    for (int b = nb + tid; b < nsbp * 8; b += nth) {  // padding blocks of the last group
        i32x4* xw = reinterpret_cast<i32x4*>(A.xs + (b >> 3) * kXs + (b & 7) * 8);
        xw[0] = xw[1] = i32x4{0, 0, 0, 0};
        A.dx[b] = 0.0f;
        A.dsum[b] = 0.0f;
        A.isum[b] = 0;
        A.s16[b] = 0;
    }
}

// LDS floats the staging needs beyond Act: stageNorm ss, stageSlot raw (+ its dummy word).
__host__ __device__ constexpr int stageFloats(int pro, int nsbp) {
    return pro == kProNorm ? nsbp * 8 : nsbp * 16 + 4;
}

// The workgroup's tile slots: for a plain matvec TPW tiles of one part; for SwiGLU TPW tiles of
// the gate (part 0) then the same TPW tiles of the up projection (part 1).
struct Slot {
    const uint8_t* qw;
    int tile, live;
};

template <int EPI>
__device__ __forceinline__ Slot slotOf(const DmvArgs& a, int part, int j) {
    Slot s;
    if (EPI == kEpiSwiglu) {
        const bool up = j >= a.tpw;
        s.qw = static_cast<const uint8_t*>(up ? a.p1.qw : a.p0.qw);
        s.tile = blockIdx.x * a.tpw + (up ? j - a.tpw : j);
        s.live = s.tile < a.p0.tiles;
    } else {
        const DmvPart& p = part == 2 ? a.p2 : (part == 1 ? a.p1 : a.p0);
        s.qw = static_cast<const uint8_t*>(p.qw);
        s.tile = (blockIdx.x - p.wg0) * a.tpw + j;
        s.live = s.tile < p.tiles;
    }
    return s;
}

// Items of the workgroup: (slot j, group g), item i -> j = i % NS, g = i / NS; wave w takes
// items w, w + nw, ...; each writes its lanes' per-super-block terms to LDS in super-block order.
template <bool Q6, int EPI>
__device__ __forceinline__ void dmvItems(const DmvArgs& a, int part, const Act& A, float* terms, int ns,
                                         Pieces<Q6, true>& first, bool first_live) {
    constexpr int kSeg = Q6 ? kQ6kSeg : kQ4kSeg;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int kq = lane >> 4, r = lane & 15;
    const int ngroups = a.ngroups, ntmax = 2 * ngroups * kGroupSb;
    const int nitems = ns * ngroups;
    Pieces<Q6, true> cur = first;
    bool cur_live = first_live;
    for (int i = wave; i < nitems; i += nw) {
        const int in = i + nw;
        Pieces<Q6, true> nxt;
        bool nxt_live = false;
        if (in < nitems) {
            const Slot sn = slotOf<EPI>(a, part, in % ns);
            nxt_live = sn.live;
            if (nxt_live) nxt.load(sn.qw + ((size_t)sn.tile * ngroups + in / ns) * kSeg, lane);
        }
        if (cur_live) {
            const int j = i % ns, g = i / ns;
            const int s = g * kGroupSb + kq;
            const uint32_t* c = reinterpret_cast<const uint32_t*>(cur.c);
            float* tt = terms + (j * 16 + r) * (ntmax + 4);  // one row's terms, contiguous
            if (Q6) {
                float t0, t1;
                q6k_terms(c, cur.dbits, A.xs + s * kXs, A.dx + 8 * s, A.isum + 8 * s, A.s16 + 8 * s, &t0, &t1);
                tt[2 * s] = t0;
                tt[2 * s + 1] = t1;
            } else {
                tt[s] = q4k_term(c, A.xs + s * kXs, A.dx + 8 * s, A.dsum + 8 * s);
            }
        }
        cur = nxt;
        cur_live = nxt_live;
    }
}

// N8: the norm prologue with 8 lanes per block of 32 (stageNorm8, at most two passes of the
// workgroup), else one thread per block (stageNorm).
template <int PRO, int EPI, bool N8, int PRE = 0>
__global__ __launch_bounds__(EPI == kEpiSwiglu ? 768 : 512) void dmv_kernel(DmvArgs a) {
    extern __shared__ int4 lds4[];
    int* lds = reinterpret_cast<int*>(lds4);
    const int nsbp = a.ngroups * kGroupSb;
    const int ntmax = 2 * nsbp;
    const int ns = EPI == kEpiSwiglu ? 2 * a.tpw : a.tpw;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    Act A(lds, nsbp);
    float* terms = reinterpret_cast<float*>(lds + Act::ints(nsbp));
    float* extra = terms + ns * 16 * (ntmax + 4);  // norm scratch, or the SwiGLU row values
    int part = 0;
    if (EPI != kEpiSwiglu) {
        if (a.nparts > 2 && (int)blockIdx.x >= a.p2.wg0) part = 2;
        else if (a.nparts > 1 && (int)blockIdx.x >= a.p1.wg0) part = 1;
    }
    const DmvPart& P = part == 2 ? a.p2 : (part == 1 ? a.p1 : a.p0);
    const bool q6 = P.q6 != 0;

    // Loads in order: the residual row value, the activations, then the first item's weights.
    bool row_ok = false;
    int row = 0;
    float y_old = 0.0f;
    if (EPI != kEpiSwiglu && tid < ns * 16) {
        const Slot s = slotOf<EPI>(a, part, tid >> 4);
        row = s.tile * kTileRows + (tid & 15);
        row_ok = s.live && row < P.rows;
        if (EPI == kEpiResid) y_old = (a.r ? a.r : P.y)[row_ok ? row : 0];
    }
    // The norm prologue: with 8 lanes per block in the wide SwiGLU workgroups (at most two passes:
    // the launcher checks n / 4 <= 2 * threads), one thread per block in the others (where 8 lanes
    // per block would take up to four passes of their serial steps).
    StageRegs st;
    NormRegs8<2> nr8;
    NormRegs nr;
    if (PRO == kProNorm && N8) loadNorm8(nr8, a.x, a.nw, a.k);
    else if (PRO == kProNorm) loadNorm(nr, a.x, a.nw, a.k);
    else loadSlot(st, a.xq, a.xd, a.k / 256);
    // The first item (wave < nw <= items always): 13 slabs and a Q6_K d read for either type
    // with no branch (a Q4_K segment rereads its last slab, and its d address is slab 0). A dead
    // tile reads tile 0. Issued before the staging, so that the item's weights stream in while
    // the activations are staged (the staging waits for its own loads only) -- except in the
    // SwiGLU workgroups, whose 28 MB of weights issued all at once queue the activations' small
    // loads behind them: there the weights are issued once the activations are staged.
    Pieces<true, true> f6;
    Pieces<false, true> f4;
    bool first_live = false;
    // slabs [LO, HI) of the first item (SwiGLU: PRE of them before the staging, the rest after)
    const Slot s0 = slotOf<EPI>(a, part, wave % ns);
    const int seg = q6 ? kQ6kSeg : kQ4kSeg, nsl = q6 ? kQ6kSlabs : kQ4kSlabs;
    const uint8_t* p0 = s0.qw + ((size_t)(s0.live ? s0.tile : 0) * a.ngroups + wave / ns) * seg;
    first_live = s0.live;
    auto loadFirst = [&](auto lo, auto hi) {
#pragma unroll
        for (int i = decltype(lo)::value; i < decltype(hi)::value; ++i)
            f6.c[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p0 + min(i, nsl - 1) * 1024 + lane * 16));
        if constexpr (decltype(hi)::value == kQ6kSlabs)
            f6.dbits = *reinterpret_cast<const uint16_t*>(p0 + (q6 ? kQ6kSlabs * 1024 + lane * 2 : 0));
    };
    using Lo = std::integral_constant<int, 0>;
    using Pre = std::integral_constant<int, (EPI == kEpiSwiglu ? PRE : kQ6kSlabs)>;
    using Hi = std::integral_constant<int, kQ6kSlabs>;
    loadFirst(Lo{}, Pre{});
    __builtin_amdgcn_sched_barrier(0);
    if (PRO == kProNorm && N8) stageNorm8(A, extra, nr8, a.k, a.eps, nsbp);
    else if (PRO == kProNorm) stageNorm(A, extra, nr, a.k, a.eps, nsbp);
    else stageSlot(A, extra, st, a.k / 256, nsbp);
    __syncthreads();
    if constexpr (EPI == kEpiSwiglu) loadFirst(Pre{}, Hi{});
#pragma unroll
    for (int i = 0; i < kQ4kSlabs; ++i) f4.c[i] = f6.c[i];
    if (q6) dmvItems<true, EPI>(a, part, A, terms, ns, f6, first_live);
    else dmvItems<false, EPI>(a, part, A, terms, ns, f4, first_live);
    __syncthreads();

    const int nreal = q6 ? 2 * (a.k / 256) : a.k / 256;
    if (tid < ns * 16) {  // one thread per output row (the launcher keeps ns * 16 <= threads)
        // the row's terms in super-block order; 16-byte reads, eight issued before their adds
        const float4* tt = reinterpret_cast<const float4*>(terms + tid * (ntmax + 4));
        const int n4 = ntmax / 4;
        float acc = 0.0f;
        for (int u0 = 0; u0 < nreal; u0 += 32) {
            float4 q[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) q[k] = tt[min(u0 / 4 + k, n4 - 1)];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int u = u0 + 4 * k;
                if (u < nreal) acc += q[k].x;
                if (u + 1 < nreal) acc += q[k].y;
                if (u + 2 < nreal) acc += q[k].z;
                if (u + 3 < nreal) acc += q[k].w;
            }
        }
        if (EPI == kEpiSwiglu) {
            extra[tid] = acc;
        } else if (row_ok) {
            if (EPI == kEpiResid) P.y[row] = y_old + acc;
            else P.y[row] = acc;
        }
    }
    if (EPI == kEpiSwiglu) {
        // silu(gate) * up for the workgroup's TPW * 16 rows (one lane each), then one thread per
        // block of 32 quantizes it (silu_mul_q8x4f.cu).
        __syncthreads();
        const int nrow = a.tpw * kTileRows;
        float* vb = extra + 2 * nrow;  // blocks of 32 values, 33 floats apart
        if (tid < nrow) vb[(tid >> 5) * 33 + (tid & 31)] = silu(extra[tid]) * extra[nrow + tid];
        __syncthreads();
        // eight lanes per block of 32 (quant8: the same bytes, scale and sum as quant32Seq)
        if (tid < nrow / 4) {
            const int b = tid >> 3, j = tid & 7, bg = blockIdx.x * (nrow / 32) + b, nbo = a.p0.rows / 32;
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = vb[b * 33 + 4 * j + e];
            const Q8L o = quant8(y);
            if (bg < nbo) {
                a.qout[bg * 8 + j] = o.w;
                if (j == 0) *reinterpret_cast<float2*>(a.qout + nbo * 8 + 2 * bg) = make_float2(o.d, (float)o.sum);
            }
        }
    }
}

// ---------------------------------------------------------------- standalone norm + quantization

// add_sumsq (sums only) + norm_mul_q8 of one row into a per-32 slot [nb*8 words | nb*2 floats |
// nb floats: the sums of squares].
__global__ __launch_bounds__(512) void rms_q8_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                     int* __restrict__ slot, int n, float eps) {
    extern __shared__ int4 lds4[];
    int* lds = reinterpret_cast<int*>(lds4);
    const int nsbp = (n / 256 + kGroupSb - 1) / kGroupSb * kGroupSb;
    Act A(lds, nsbp);
    float* ss = reinterpret_cast<float*>(lds + Act::ints(nsbp));
    NormRegs st;
    loadNorm(st, x, w, n);
    stageNorm(A, ss, st, n, eps, nsbp);
    __syncthreads();
    const int nb = n / 32;
    for (int i = threadIdx.x; i < nb * 8; i += blockDim.x) slot[i] = A.xs[(i >> 6) * kXs + (i & 63)];
    float* xd = reinterpret_cast<float*>(slot + nb * 8);
    for (int b = threadIdx.x; b < nb; b += blockDim.x) {
        xd[2 * b] = A.dx[b];
        xd[2 * b + 1] = (float)A.isum[b];
        xd[2 * nb + b] = ss[b];
    }
}

// ---------------------------------------------------------------- split-context attention

// Sums over the 16 (or 8) lanes of a DPP row group with row-local DPP moves (no LDS traffic):
// pairs, quads, mirrored halves of 8, mirrored halves of 16; every lane ends with the total.
template <int CTRL>
__device__ __forceinline__ float dppMove(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int LANES>
__device__ __forceinline__ float dppSum(float v) {
    v += dppMove<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v += dppMove<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v += dppMove<0x141>(v);  // row_half_mirror
    if (LANES == 16) v += dppMove<0x140>(v);  // row_mirror
    return v;
}

// Maximum / sum over the 64 lanes of a wavefront: row-local DPP moves, then the four row results
// read back with readlane (scalar), so no LDS permutes.
__device__ __forceinline__ float waveMax64(float v) {
    v = fmaxf(v, dppMove<0xB1>(v));
    v = fmaxf(v, dppMove<0x4E>(v));
    v = fmaxf(v, dppMove<0x141>(v));
    v = fmaxf(v, dppMove<0x140>(v));
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
__device__ __forceinline__ float waveSum64(float v) {
    v = dppSum<16>(v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Workgroup (chunk c, KV head g) of 256 threads: the attention of one token at position p = pos[0]
// against positions [64c, 64c + 64) of the context T = p + 1 (FLASH_ATTN_EXT: s = scale q.k,
// softmax, sum p v) for the G = H / Hkv query heads of g. Each workgroup first normalizes
// (Qwen3, rms_norm.cu) and ropes (rope_ggml.cu) its query heads; the workgroup of the last chunk
// does the same for k, stores k and v as fp16 into cache row p (set_rows_f16.cu) and takes
// position p from LDS, the others read positions below p from the cache. Partial results (max,
// sum of exp, unnormalized output) go to part, which attn_merge_kernel combines. (Merging in the
// workgroup that arrives last, counted with a device-scope atomic, was slower here: the release
// fence each workgroup needs writes the XCD's L2 back.)
// LP lanes hold one position's D values, 8 each (D = 8 LP).
template <int D, int G>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnDecodeArgs a) {
    constexpr int LP = D / 8;           // lanes per position
    constexpr int PPI = 64 / LP;        // positions per wave instruction
    constexpr int NI = (kChunk / 4) / PPI;  // instructions per wave (16 positions per wave)
    constexpr int pairs = D / 2;
    __shared__ float sc[G][kChunk];
    __shared__ float red[16][G * D];  // [wave * 4 + row of 16 lanes][head * D + d]
    __shared__ float mg[G], lg[G];
    __shared__ float qs[G * D];
    __shared__ float raw[(G + 2) * D];
    __shared__ float nwl[2 * D];
    __shared__ float kn[D], vn[D], rn[G + 1], ffl[D / 2];
    const QkPostArgs& q = a.qp;
    const int p = q.pos[0], T = p + 1;
    const int nch = (T + kChunk - 1) / kChunk;
    const int c = blockIdx.x, kvh = blockIdx.y;
    if (c >= nch) return;
    const bool last = c == nch - 1;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = lane / LP, l = lane % LP;
    const int t0 = c * kChunk + wave * 16;
    // Every global load first, unconditional (clamped rows; position p and rows past it are
    // replaced or masked below): a load under a branch gets a wait of its own.
    // The token's q, k, v (NR words per thread), the q / k norm weights and the RoPE frequency
    // factors first, then the cache rows: waiting for the small loads (the load counter drains
    // in order) leaves the cache rows in flight behind the RoPE work.
    constexpr int NR = ((G + 2) * D + 255) / 256;
    float rv[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int i = min(tid + r * 256, (G + 2) * D - 1);
        const float* src = i < G * D ? q.q + (size_t)kvh * G * D + i
                                     : (i < (G + 1) * D ? q.k + (size_t)kvh * D + (i - G * D)
                                                        : q.v + (size_t)kvh * D + (i - (G + 1) * D));
        rv[r] = *src;
    }
    const int tn = tid % (2 * D);
    const float nwv = *(q.qk_norm ? (tn < D ? q.q_norm + tn : q.k_norm + tn - D) : q.q + (tn % D));
    const float ffv = q.ff[tid % pairs];
    const int tmax = max(p - 1, 0);
    u32x4 kp[NI], vp[NI];
#pragma unroll
    for (int n = 0; n < NI; ++n) {
        const size_t row = (size_t)min(t0 + n * PPI + sub, tmax) * q.kv_row + (size_t)kvh * pairs + l * 4;
        kp[n] = *reinterpret_cast<const u32x4*>(q.kcache + row);
        vp[n] = *reinterpret_cast<const u32x4*>(q.vcache + row);
    }
#pragma unroll
    for (int r = 0; r < NR; ++r)
        if (tid + r * 256 < (G + 2) * D) raw[tid + r * 256] = rv[r];
    if (tid < 2 * D) nwl[tid] = nwv;
    if (tid < pairs) ffl[tid] = ffv;
    __syncthreads();
    if (q.qk_norm) {
        if (tid <= G) {  // heads 0..G-1: q, head G: k; sequential sums as rms_norm.cu
            float ss = 0.0f;
            for (int j = 0; j < D; ++j) ss += raw[tid * D + j] * raw[tid * D + j];
            rn[tid] = 1.0f / sqrtf(ss / (float)D + q.eps);
        }
        __syncthreads();
        for (int i = tid; i < (G + 1) * D; i += 256) {
            const int h = i / D, e = i % D;
            raw[i] = raw[i] * rn[h] * nwl[(h < G ? 0 : D) + e];
        }
        __syncthreads();
    }
    const int m1 = q.neox ? 1 : 2, m2 = q.neox ? pairs : 1;
    for (int i = tid; i < (G + 1) * pairs; i += 256) {
        const int h = i / pairs, j = i % pairs;
        const float theta = (float)p * exp2f(-(float)j / (float)pairs * q.log2_base) / ffl[j];
        float sn, cs;
        sincosf(theta, &sn, &cs);  // one shared argument reduction for both
        const int o = j * m1;
        const float x0 = raw[h * D + o], x1 = raw[h * D + o + m2];
        const float y0 = x0 * cs - x1 * sn, y1 = x0 * sn + x1 * cs;
        if (h < G) {
            qs[h * D + o] = y0;
            qs[h * D + o + m2] = y1;
        } else {
            kn[o] = h2f(f2h(y0));
            kn[o + m2] = h2f(f2h(y1));
        }
    }
    for (int e = tid; e < D; e += 256) vn[e] = h2f(f2h(raw[(G + 1) * D + e]));
    __syncthreads();
    if (last)
        for (int j = tid; j < pairs; j += 256) {
            const size_t w = (size_t)p * q.kv_row + (size_t)kvh * pairs + j;
            q.kcache[w] = (int)(f2h(kn[2 * j]) | (f2h(kn[2 * j + 1]) << 16));
            q.vcache[w] = (int)(f2h(vn[2 * j]) | (f2h(vn[2 * j + 1]) << 16));
        }
    float qv[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[g][e] = qs[g * D + l * 8 + e];
    // this lane's 8 values of the token's k and v as the fp16 words the cache row p holds
    // (kn = h2f(f2h(.)), so f2h(kn) gives back the stored bits): position p takes them with a
    // select instead of a branch per value
    u32x4 knw, vnw;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        knw[e] = f2h(kn[l * 8 + 2 * e]) | (f2h(kn[l * 8 + 2 * e + 1]) << 16);
        vnw[e] = f2h(vn[l * 8 + 2 * e]) | (f2h(vn[l * 8 + 2 * e + 1]) << 16);
    }
#pragma unroll
    for (int n = 0; n < NI; ++n) {
        const int tl = wave * 16 + n * PPI + sub, t = c * kChunk + tl;
        const u32x4 kw = t == p ? knw : kp[n];
        float kf[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            kf[2 * e] = h2f(kw[e] & 0xFFFFu);
            kf[2 * e + 1] = h2f(kw[e] >> 16);
        }
        // the G dot products, then their row sums step by step across the heads (independent
        // cross-lane moves back to back instead of one head's dependent chain at a time)
        float sg[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) s += qv[g][e] * kf[e];
            sg[g] = s;
        }
#pragma unroll
        for (int g = 0; g < G; ++g) sg[g] += dppMove<0xB1>(sg[g]);
#pragma unroll
        for (int g = 0; g < G; ++g) sg[g] += dppMove<0x4E>(sg[g]);
#pragma unroll
        for (int g = 0; g < G; ++g) sg[g] += dppMove<0x141>(sg[g]);
        if (LP == 16)
#pragma unroll
            for (int g = 0; g < G; ++g) sg[g] += dppMove<0x140>(sg[g]);
        if (l == 0)
#pragma unroll
            for (int g = 0; g < G; ++g) sc[g][tl] = t < T ? a.scale * sg[g] : -INFINITY;
    }
    __syncthreads();
    for (int g = wave; g < G; g += 4) {  // one wavefront per head: lane = position
        const float s = sc[g][lane];
        const float m = waveMax64(s);
        const float pr = s == -INFINITY ? 0.0f : exp2f((s - m) * kLog2e);
        const float sum = waveSum64(pr);
        sc[g][lane] = pr;
        if (lane == 0) {
            mg[g] = m;
            lg[g] = sum;
        }
    }
    __syncthreads();
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
#pragma unroll
    for (int n = 0; n < NI; ++n) {
        const int tl = wave * 16 + n * PPI + sub, t = c * kChunk + tl;
        const u32x4 vw = t == p ? vnw : vp[n];
        float vf[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            vf[2 * e] = h2f(vw[e] & 0xFFFFu);
            vf[2 * e + 1] = h2f(vw[e] >> 16);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float pr = sc[g][tl];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] += pr * vf[e];
        }
    }
    // the position slots through LDS, one row of 16 lanes per LDS row (for D = 64 the two slots of
    // a row are added first, lane l + 8 into lane l), summed in row order
    static_assert(LP == 8 || LP == 16, "lanes per position");
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float v = acc[g][e];
                if (LP == 8) v += dppMove<0x128>(v);  // row_ror:8
                if (LP == 16 || (lane & 8) == 0) red[wave * 4 + (lane >> 4)][g * D + l * 8 + e] = v;
            }
    __syncthreads();
    float* pp = a.part + ((size_t)kvh * a.max_chunks + c) * kMaxGroup * partRow(D);
    for (int i = tid; i < G * D; i += 256) {
        float v = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) v += red[r][i];
        pp[(i / D) * partRow(D) + i % D] = v;
    }
    if (tid < G) {
        pp[tid * partRow(D) + D] = mg[tid];
        pp[tid * partRow(D) + D + 1] = lg[tid];
    }
}

// Merge of the chunk partials of KV head blockIdx.x (its G query heads), in chunk order with a
// running max and rescaled sums, and the per-32 quantization of the outputs into the slot.
template <int D>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnDecodeArgs a) {
    __shared__ float vb[kMaxGroup * D / 32 * 33];
    const int T = a.qp.pos[0] + 1;
    const int nch = (T + kChunk - 1) / kChunk;
    const int kvh = blockIdx.x, G = a.G, tid = threadIdx.x;
    const float* base = a.part + (size_t)kvh * a.max_chunks * kMaxGroup * partRow(D);
    for (int i = tid; i < G * D; i += 256) {
        const int g = i / D, d = i % D;
        float M = -INFINITY, L = 0.0f, O = 0.0f;
        for (int c0 = 0; c0 < nch; c0 += 16) {
            float mv[16], lv[16], ov[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {  // unconditional loads (chunks past nch reread the last)
                const float* pc = base + ((size_t)min(c0 + u, nch - 1) * kMaxGroup + g) * partRow(D);
                mv[u] = pc[D];
                lv[u] = pc[D + 1];
                ov[u] = pc[d];
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                if (c0 + u < nch) {
                    if (mv[u] > M) {
                        const float f = exp2f((M - mv[u]) * kLog2e);
                        L *= f;
                        O *= f;
                        M = mv[u];
                    }
                    const float f = exp2f((mv[u] - M) * kLog2e);
                    L += lv[u] * f;
                    O += ov[u] * f;
                }
            }
        }
        vb[(i >> 5) * 33 + (i & 31)] = O / L;
    }
    __syncthreads();
    const int nbl = G * D / 32;
    if (tid < nbl) storeQ32(a.slot, a.nq, kvh * nbl + tid, quant32Seq(vb + tid * 33));
}

template <int CTRL>
__device__ __forceinline__ int dppMoveI(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}

// The same merge with one wavefront per 64 consecutive outputs of one query head (blockIdx.x =
// h * (D / 64) + j): each lane runs attn_merge_kernel's chunk-order recurrence for one output,
// with every load of a group of 16 chunks issued before the arithmetic, and the wavefront then
// quantizes its two blocks of 32 (lanes 0-31, 32-63) with cross-lane moves. The block maximum
// and the integer sums do not depend on the order of their terms, so the bytes, scales and sums
// equal quant32Seq's: the slot is bit-identical to attn_merge_kernel's, from 2-4 times as many
// workgroups and without the per-thread loops.
template <int D>
__global__ __launch_bounds__(64) void attn_merge_wave_kernel(AttnDecodeArgs a) {
    const int T = a.qp.pos[0] + 1;
    const int nch = (T + kChunk - 1) / kChunk;
    const int lane = threadIdx.x, h = blockIdx.x / (D / 64), d0 = (blockIdx.x % (D / 64)) * 64;
    const size_t row = (size_t)kMaxGroup * partRow(D);  // floats per (KV head, chunk)
    const float* base = a.part + (size_t)(h / a.G) * a.max_chunks * row + (h % a.G) * partRow(D);
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += 16) {
        float ov[16], mv[16], lv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {  // unconditional loads (chunks past nch reread the last)
            const float* pc = base + (size_t)min(c0 + u, nch - 1) * row;
            ov[u] = pc[d0 + lane];
            mv[u] = pc[D];
            lv[u] = pc[D + 1];
        }
        // Branch-free, so that no load moves under a branch (and waits alone there): a chunk
        // past nch rereads the last one, whose max is already M (no rescale), and gets weight 0,
        // which adds +0 to L and O: unchanged (the sign of a zero O does not reach the bytes).
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            if (mv[u] > M) {
                const float f = exp2f((M - mv[u]) * kLog2e);
                L *= f;
                O *= f;
                M = mv[u];
            }
            float f = exp2f((mv[u] - M) * kLog2e);
            if (c0 + u >= nch) f = 0.0f;
            L += lv[u] * f;
            O += ov[u] * f;
        }
    }
    const float v = O / L;
    // block maximum of |v| over 32 lanes: the 16-lane row by DPP, then the row pair
    float m = fabsf(v);
    m = fmaxf(m, dppMove<0xB1>(m));
    m = fmaxf(m, dppMove<0x4E>(m));
    m = fmaxf(m, dppMove<0x141>(m));
    m = fmaxf(m, dppMove<0x140>(m));
    m = fmaxf(m, __shfl_xor(m, 16));
    const float dq = fmaxf(0.0f, m) / 127.0f;
    float id;
    if (dq > 0.0f) id = 1.0f / dq;
    else id = 0.0f;
    const int q = q8r(v * id);
    // the block's sum of q, the same way
    int sq = q;
    sq += dppMoveI<0xB1>(sq);
    sq += dppMoveI<0x4E>(sq);
    sq += dppMoveI<0x141>(sq);
    sq += dppMoveI<0x140>(sq);
    sq += __shfl_xor(sq, 16);
    // the four bytes of a word from the lanes of a quad (quad_perm [1,1,1,1], [2,...], [3,...])
    const int q1 = dppMoveI<0x55>(q), q2 = dppMoveI<0xAA>(q), q3 = dppMoveI<0xFF>(q);
    const int b = (h * D + d0) / 32 + (lane >> 5);
    if ((lane & 3) == 0)
        a.slot[b * 8 + ((lane & 31) >> 2)] = pack4(q, q1, q2, q3);
    if ((lane & 31) == 0) *reinterpret_cast<float2*>(a.slot + a.nq * 8 + 2 * b) = make_float2(dq, (float)sq);
}

// ---------------------------------------------------------------- split-context FLASH_ATTN_EXT

// flash_decode_f16: FLASH_ATTN_EXT (fa_scores / fa_max / fa_exp / fa_values: s = scale q.k + mask,
// softmax over the context, sum p v) for a few query tokens over a long context, split over
// 64-position chunks so that the whole GPU takes part (the one-kernel flash_attn_f16 runs one
// workgroup per (token, head)). Workgroup (chunk c, KV head g, token i) of 256 threads computes the
// G query heads of g against positions [64c, 64c + 64) with the layout of attn_decode_kernel (LP
// lanes per position, 8 values each); it writes the chunk's maximum, sum of exponentials and
// unnormalized output to part; flash_merge_kernel combines the chunks in order with a running
// maximum. A chunk whose positions are all masked contributes nothing.
// RP: the ROPE / SET_ROWS prologue (FdRope; one query token): the raw q of the G heads and k, v of
// KV head g into LDS, RoPE as rope_kv_rows_kernel computes it (the same expressions, so the same
// bits), the roped q and k written by the workgroups of chunk 0 (where rp.qr / rp.kr are given:
// the other chunks read the raw q and k meanwhile, so these outputs must not overlap them), the fp16
// cache row of head g
// stored by the workgroup whose chunk holds it (chunk 0's when the view does not hold it), and
// that row read from registers by the workgroup that holds it: no workgroup reads a row another
// one writes.
template <int D, int G, bool RP>
__global__ __launch_bounds__(256) void flash_decode_kernel(const float* __restrict__ q, const int* __restrict__ k,
                                                           const int* __restrict__ v, const int* __restrict__ mask,
                                                           float* __restrict__ part, kcFaDims d, float scale, int nch,
                                                           FdRope rp) {
    constexpr int LP = D / 8;      // lanes per position
    constexpr int PPI = 64 / LP;   // positions per wave instruction
    constexpr int NI = 16 / PPI;   // instructions per wave (16 positions per wave)
    constexpr int pairs = D / 2;
    __shared__ float sc[G][kChunk];
    __shared__ float red[16][G * D];
    __shared__ float mg[G], lg[G];
    const int c = blockIdx.x, kvh = blockIdx.y, i = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = lane / LP, l = lane % LP;
    const int t0 = c * kChunk + wave * 16, tmax = d.T - 1;
    // every load first, unconditional (rows past the context are clamped and masked below)
    u32x4 kp[NI], vp[NI];
    float mk[NI];
#pragma unroll
    for (int n = 0; n < NI; ++n) {
        const int t = min(t0 + n * PPI + sub, tmax);
        kp[n] = *reinterpret_cast<const u32x4*>(k + (size_t)t * d.k_row + (size_t)kvh * d.k_head + l * 4);
        vp[n] = *reinterpret_cast<const u32x4*>(v + (size_t)t * d.v_row + (size_t)kvh * d.v_head + l * 4);
        const uint32_t w = d.has_mask ? (uint32_t)mask[(size_t)i * d.m_row + t / 2] : 0u;
        mk[n] = h2f((w >> ((t & 1) * 16)) & 0xFFFFu);
    }
    float qv[G][8];
    int tnew = -1;     // RP: the view row of the new cache row (-1: none)
    u32x4 knw, vnw;    // RP: this lane's 8 values of that row, as the fp16 words the cache holds
    if constexpr (RP) {
        __shared__ float raw[(G + 2) * D];
        __shared__ float qs[G * D];
        __shared__ float kn[D];
        __shared__ float ffl[pairs];
        __shared__ float nwl[2 * D], rn[G + 1];
        constexpr int NR = ((G + 2) * D + 255) / 256;
        float rv[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int x = min(tid + r * 256, (G + 2) * D - 1);
            rv[r] = x < G * D ? rp.q[(size_t)kvh * G * D + x]
                              : (x < (G + 1) * D ? rp.k[(size_t)kvh * D + (x - G * D)]
                                                 : rp.v[(size_t)kvh * D + (x - (G + 1) * D)]);
        }
        const float ffv = rp.ff[tid % pairs];
        const int tn = tid % (2 * D);
        const float nwv = rp.qk_norm ? (tn < D ? rp.q_norm[tn] : rp.k_norm[tn - D]) : 0.0f;
        const int p = rp.pos[0], row = rp.idx[0];
        const bool stored = row >= 0 && row < rp.dst_rows;
        const int tv = row - rp.row0;
        tnew = stored && tv >= 0 && tv < d.T ? tv : -1;
        const int cstore = tnew >= 0 ? tnew / kChunk : 0;
#pragma unroll
        for (int r = 0; r < NR; ++r)
            if (tid + r * 256 < (G + 2) * D) raw[tid + r * 256] = rv[r];
        if (tid < pairs) ffl[tid] = ffv;
        if (tid < 2 * D) nwl[tid] = nwv;
        __syncthreads();
        if (rp.qk_norm) {  // rms_norm + MUL of each head (q heads 0 .. G - 1, k head G): sequential sums
            if (tid <= G) {
                float ss = 0.0f;
                for (int j = 0; j < D; ++j) ss += raw[tid * D + j] * raw[tid * D + j];
                rn[tid] = 1.0f / sqrtf(ss / (float)D + rp.eps);
            }
            __syncthreads();
            for (int x = tid; x < (G + 1) * D; x += 256) {
                const int h = x / D, e = x % D;
                const float y = raw[x] * rn[h] * nwl[(h < G ? 0 : D) + e];
                raw[x] = y;
                if (c == 0) {
                    if (h < G) {
                        if (rp.qn) rp.qn[(size_t)(kvh * G + h) * D + e] = y;
                    } else if (rp.kn) {
                        rp.kn[(size_t)kvh * D + e] = y;
                    }
                }
            }
            __syncthreads();
        }
        const int m1 = rp.neox ? 1 : 2, m2 = rp.neox ? pairs : 1;
        for (int x = tid; x < (G + 1) * pairs; x += 256) {
            const int h = x / pairs, j = x % pairs;
            const float theta = (float)p * exp2f(-(float)j / (float)pairs * rp.log2_base) / ffl[j];
            const float cs = cosf(theta), sn = sinf(theta);
            const int o = j * m1;
            const float x0 = raw[h * D + o], x1 = raw[h * D + o + m2];
            const float y0 = x0 * cs - x1 * sn, y1 = x0 * sn + x1 * cs;
            if (h < G) {
                qs[h * D + o] = y0;
                qs[h * D + o + m2] = y1;
                if (c == 0 && rp.qr) {
                    rp.qr[(size_t)(kvh * G + h) * D + o] = y0;
                    rp.qr[(size_t)(kvh * G + h) * D + o + m2] = y1;
                }
            } else {
                kn[o] = y0;
                kn[o + m2] = y1;
                if (c == 0 && rp.kr) {
                    rp.kr[(size_t)kvh * D + o] = y0;
                    rp.kr[(size_t)kvh * D + o + m2] = y1;
                }
                if (stored && c == cstore) {
                    unsigned short* kc = reinterpret_cast<unsigned short*>(rp.kc);
                    unsigned short* vc = reinterpret_cast<unsigned short*>(rp.vc);
                    const size_t e = (size_t)row * rp.k_row * 2 + (size_t)kvh * D + o;
                    const size_t f = (size_t)row * rp.v_row * 2 + (size_t)kvh * D + o;
                    kc[e] = (unsigned short)f2h(y0);
                    kc[e + m2] = (unsigned short)f2h(y1);
                    vc[f] = (unsigned short)f2h(raw[(G + 1) * D + o]);
                    vc[f + m2] = (unsigned short)f2h(raw[(G + 1) * D + o + m2]);
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) qv[g][e] = qs[g * D + l * 8 + e];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            knw[e] = f2h(kn[l * 8 + 2 * e]) | (f2h(kn[l * 8 + 2 * e + 1]) << 16);
            vnw[e] = f2h(raw[(G + 1) * D + l * 8 + 2 * e]) | (f2h(raw[(G + 1) * D + l * 8 + 2 * e + 1]) << 16);
        }
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float4* qh =
                reinterpret_cast<const float4*>(q + (size_t)i * d.q_tok + (size_t)(kvh * G + g) * d.q_head + l * 8);
            const float4 a = qh[0], b = qh[1];
            qv[g][0] = a.x, qv[g][1] = a.y, qv[g][2] = a.z, qv[g][3] = a.w;
            qv[g][4] = b.x, qv[g][5] = b.y, qv[g][6] = b.z, qv[g][7] = b.w;
        }
    }
#pragma unroll
    for (int n = 0; n < NI; ++n) {
        const int tl = wave * 16 + n * PPI + sub, t = c * kChunk + tl;
        const u32x4 kw = RP && t == tnew ? knw : kp[n];
        float kf[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            kf[2 * e] = h2f(kw[e] & 0xFFFFu);
            kf[2 * e + 1] = h2f(kw[e] >> 16);
        }
        float sg[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float sv = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) sv += qv[g][e] * kf[e];
            sg[g] = dppSum<LP>(sv);
        }
        if (l == 0)
#pragma unroll
            for (int g = 0; g < G; ++g) sc[g][tl] = t < d.T ? scale * sg[g] + mk[n] : -INFINITY;
    }
    __syncthreads();
    for (int g = wave; g < G; g += 4) {  // one wavefront per head: lane = position
        const float sv = sc[g][lane];
        const float m = waveMax64(sv);
        const float pr = sv == -INFINITY ? 0.0f : exp2f((sv - m) * kLog2e);
        const float sum = waveSum64(pr);
        sc[g][lane] = pr;
        if (lane == 0) {
            mg[g] = m;
            lg[g] = sum;
        }
    }
    __syncthreads();
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
#pragma unroll
    for (int n = 0; n < NI; ++n) {
        const int tl = wave * 16 + n * PPI + sub;
        const u32x4 vw = RP && c * kChunk + tl == tnew ? vnw : vp[n];
        float vf[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            vf[2 * e] = h2f(vw[e] & 0xFFFFu);
            vf[2 * e + 1] = h2f(vw[e] >> 16);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float pr = sc[g][tl];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] += pr * vf[e];
        }
    }
    // the position slots through LDS, one row of 16 lanes per LDS row (for D = 64 the two slots of
    // a row are added first), summed in row order
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float a = acc[g][e];
            if (LP == 8) a += dppMove<0x128>(a);  // row_ror:8
            if (LP == 16 || (lane & 8) == 0) red[wave * 4 + (lane >> 4)][g * D + l * 8 + e] = a;
        }
    __syncthreads();
    for (int x = tid; x < G * D; x += 256) {
        float a = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) a += red[r][x];
        const int g = x / D, h = kvh * G + g;
        part[(((size_t)i * d.H + h) * nch + c) * (D + 2) + x % D] = a;
    }
    if (tid < G) {
        float* pc = part + (((size_t)i * d.H + kvh * G + tid) * nch + c) * (D + 2);
        pc[D] = mg[tid];
        pc[D + 1] = lg[tid];
    }
}

// out[i][h][:] of the chunk partials of (token i, head h) = blockIdx.x, in chunk order. The
// partials of 16 chunks are loaded before they are merged (one memory round trip per 16 chunks).
// slot (optional, one token): the head's D outputs also quantized per 32 into the per-32 slot of
// the token's nb = H * D / 32 blocks (quantize_q8x4.cu: codes and d / sum pairs; quant8).
template <int D>
__global__ __launch_bounds__(128) void flash_merge_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                          int nch, int* __restrict__ slot, int nb) {
    __shared__ float ov[D];
    const float* base = part + (size_t)blockIdx.x * nch * (D + 2);
    for (int e = threadIdx.x; e < D; e += 128) {
        float M = -INFINITY, L = 0.0f, O = 0.0f;
        for (int c0 = 0; c0 < nch; c0 += 16) {
            float mc[16], lc[16], oc[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const float* pc = base + (size_t)min(c0 + u, nch - 1) * (D + 2);
                mc[u] = pc[D];
                lc[u] = pc[D + 1];
                oc[u] = pc[e];
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                if (c0 + u >= nch) break;
                const float m = mc[u];
                if (m == -INFINITY) continue;  // every position of the chunk masked
                if (m > M) {
                    const float f = exp2f((M - m) * kLog2e);
                    L *= f;
                    O *= f;
                    M = m;
                }
                const float f = exp2f((m - M) * kLog2e);
                L += lc[u] * f;
                O += oc[u] * f;
            }
        }
        out[(size_t)blockIdx.x * D + e] = O / L;
        ov[e] = O / L;
    }
    if (slot) {
        __syncthreads();
        const int t = threadIdx.x;
        if (t < D / 4) {  // eight lanes per block of 32, four values each
            const float y[4] = {ov[4 * t], ov[4 * t + 1], ov[4 * t + 2], ov[4 * t + 3]};
            const Q8L o = quant8(y);
            const int b = blockIdx.x * (D / 32) + (t >> 3), j = t & 7;
            slot[b * 8 + j] = o.w;
            if (j == 0) *reinterpret_cast<float2*>(slot + nb * 8 + 2 * b) = make_float2(o.d, (float)o.sum);
        }
    }
}

}  // namespace

// ---------------------------------------------------------------- launchers

size_t dmvLds(int pro, int epi, int k, int tpw) {
    const int nsbp = (k / 256 + kGroupSb - 1) / kGroupSb * kGroupSb;
    const int ns = epi == kEpiSwiglu ? 2 * tpw : tpw;
    size_t ints = (size_t)Act::ints(nsbp) + (size_t)ns * 16 * (2 * nsbp + 4);
    size_t extra = stageFloats(pro, nsbp);
    const size_t swi = (size_t)ns * kTileRows + (size_t)tpw * kTileRows / 32 * 33 + 33;
    if (epi == kEpiSwiglu && extra < swi) extra = swi;
    return 4 * (ints + extra);
}

DmvPlan planDecodeMatvec(int pro, int epi, int k, int tpw) {
    DmvPlan p;
    if (k <= 0 || k % 256 || tpw < 1) {
        p.why = "decode matvec: k must be a positive multiple of 256 and tpw >= 1";
        return p;
    }
    const int ngroups = (k / 256 + kGroupSb - 1) / kGroupSb, nsb = k / 256;
    const int ns = epi == kEpiSwiglu ? 2 * tpw : tpw;
    if (ns > 8 || (epi == kEpiSwiglu && tpw % 2)) {
        p.why = "decode matvec: tiles per workgroup";
        return p;
    }
    // whether nw wavefronts hold the tiles' row sums and stage the activations
    auto fits = [&](int nw, bool* n8) {
        const int nth = 64 * nw;
        *n8 = pro == kProNorm && (epi == kEpiSwiglu || k / 4 <= 2 * nth);
        if (ns * kTileRows > 64 * nw) return false;
        if (pro == kProNorm && (*n8 ? k / 4 > 2 * nth : k / 32 > nth)) return false;
        if (pro == kProSlot && (nsb * 16 > 4 * nth || nsb * 4 > nth)) return false;
        return true;
    };
    // At most 12 (SwiGLU) or 8 wavefronts. Beyond that, a divisor of the items (from half the cap
    // up) gives every wavefront the same number of them; where no divisor fits, the cap (the item
    // loop strides by the wavefront count, so uneven shares are correct, only less balanced).
    const int items = ns * ngroups, cap = epi == kEpiSwiglu ? 12 : 8;
    int nw = items <= cap ? items : 0;
    bool n8 = false;
    if (!nw)
        for (int d = cap; d >= (cap + 1) / 2 && !nw; --d)
            if (items % d == 0 && fits(d, &n8)) nw = d;
    if (!nw) nw = std::min(items, cap);
    if (!fits(nw, &n8)) {
        p.why = "decode matvec: activations exceed the staging registers";
        return p;
    }
    const size_t lds = dmvLds(pro, epi, k, tpw);
    if (lds > 65536) {
        p.why = "decode matvec: activations exceed LDS";
        return p;
    }
    p.nw = nw;
    p.n8 = n8;
    p.lds = lds;
    return p;
}

int launchDecodeMatvec(int pro, int epi, DmvArgs a, hipStream_t s) {
    const DmvPlan plan = planDecodeMatvec(pro, epi, a.k, a.tpw);
    if (!plan.nw) return fromHip(hipErrorInvalidValue, plan.why);
    a.ngroups = (a.k / 256 + kGroupSb - 1) / kGroupSb;
    int wgs = 0;
    if (epi == kEpiSwiglu) {
        a.p0.tiles = tilesOf(a.p0.rows);
        wgs = (a.p0.tiles + a.tpw - 1) / a.tpw;
    } else {
        DmvPart* ps[3] = {&a.p0, &a.p1, &a.p2};
        for (int i = 0; i < a.nparts; ++i) {
            ps[i]->tiles = tilesOf(ps[i]->rows);
            ps[i]->wg0 = wgs;
            wgs += (ps[i]->tiles + a.tpw - 1) / a.tpw;
        }
    }
    const int nw = plan.nw;
    const bool n8 = plan.n8;
    const size_t lds = plan.lds;
    const dim3 grid(wgs), block(64 * nw);
#define KC_DMV(P, Q)                                                                                         \
    if (pro == P && epi == Q && n8 == (P == kProNorm && Q == kEpiSwiglu))                                    \
        hipLaunchKernelGGL((dmv_kernel<P, Q, P == kProNorm && Q == kEpiSwiglu>), grid, block, lds, s, a);     \
    if (pro == P && epi == Q && n8 && P == kProNorm && Q != kEpiSwiglu)                                        \
        hipLaunchKernelGGL((dmv_kernel<P, Q, true>), grid, block, lds, s, a);
    // The SwiGLU workgroups issue 9 of the 13 slab loads of each wavefront's weights before the
    // activations are staged and the rest after (config 4 decode, measured: 812 tok/s with all
    // after, 819 with 3 or 6 before, 821 with 9, 803 with all 13: their 28 MB in flight then delay
    // the activation loads). Option "swiglu_pre": 1-13 that many before, 14 none.
    const int po = option("swiglu_pre");
    const int pre = epi != kEpiSwiglu ? 0 : (po == 0 ? 9 : (po >= 14 ? 0 : po));
    if (pre > 0 && pro == kProNorm && epi == kEpiSwiglu && n8) {
        if (pre <= 3) hipLaunchKernelGGL((dmv_kernel<kProNorm, kEpiSwiglu, true, 3>), grid, block, lds, s, a);
        else if (pre <= 6) hipLaunchKernelGGL((dmv_kernel<kProNorm, kEpiSwiglu, true, 6>), grid, block, lds, s, a);
        else if (pre <= 9) hipLaunchKernelGGL((dmv_kernel<kProNorm, kEpiSwiglu, true, 9>), grid, block, lds, s, a);
        else hipLaunchKernelGGL((dmv_kernel<kProNorm, kEpiSwiglu, true, 13>), grid, block, lds, s, a);
        return fromHip(hipGetLastError(), "decode matvec");
    }
    KC_DMV(kProSlot, kEpiStore)
    KC_DMV(kProSlot, kEpiResid)
    KC_DMV(kProNorm, kEpiStore)
    KC_DMV(kProNorm, kEpiResid)
    KC_DMV(kProNorm, kEpiSwiglu)
    KC_DMV(kProSlot, kEpiSwiglu)
#undef KC_DMV
    return fromHip(hipGetLastError(), "decode matvec");
}

bool rmsQ8Supports(int n) {
    const int nsbp = (n / 256 + kGroupSb - 1) / kGroupSb * kGroupSb;
    const size_t lds = 4 * ((size_t)Act::ints(nsbp) + stageFloats(kProNorm, nsbp));
    return n > 0 && n % 256 == 0 && lds <= 65536 && n / 32 <= (n <= 8192 ? 256 : 512);
}

int launchRmsQ8(const float* x, const float* w, int* slot, int n, float eps, hipStream_t s) {
    const int nsbp = (n / 256 + kGroupSb - 1) / kGroupSb * kGroupSb;
    const size_t lds = 4 * ((size_t)Act::ints(nsbp) + stageFloats(kProNorm, nsbp));
    const int threads = n <= 8192 ? 256 : 512;
    if (!rmsQ8Supports(n)) return fromHip(hipErrorInvalidValue, "rms_q8: row too long");
    hipLaunchKernelGGL(rms_q8_kernel, dim3(1), dim3(threads), lds, s, x, w, slot, n, eps);
    return fromHip(hipGetLastError(), "rms_q8");
}

bool attnDecodeSupports(int D, int G) { return (D == 64 || D == 128) && G >= 1 && G <= kMaxGroup; }

size_t attnDecodePartFloats(int Hkv, int max_ctx, int D) {
    return (size_t)Hkv * ((max_ctx + kChunk - 1) / kChunk) * kMaxGroup * partRow(D);
}

int launchAttnDecode(AttnDecodeArgs a, int D, int Hkv, int max_ctx, hipStream_t s, bool seq_merge) {
    if (!attnDecodeSupports(D, a.G)) return fromHip(hipErrorInvalidValue, "attn_decode: shape");
    a.max_chunks = (max_ctx + kChunk - 1) / kChunk;
    const dim3 grid(a.max_chunks, Hkv);
#define KC_AD(DD, GG) \
    if (D == DD && a.G == GG) hipLaunchKernelGGL((attn_decode_kernel<DD, GG>), grid, dim3(256), 0, s, a);
    KC_AD(128, 1) KC_AD(128, 2) KC_AD(128, 3) KC_AD(128, 4) KC_AD(128, 5) KC_AD(128, 6) KC_AD(128, 7) KC_AD(128, 8)
    KC_AD(64, 1) KC_AD(64, 2) KC_AD(64, 3) KC_AD(64, 4) KC_AD(64, 5) KC_AD(64, 6) KC_AD(64, 7) KC_AD(64, 8)
#undef KC_AD
    if (seq_merge) {
        if (D == 128) hipLaunchKernelGGL(attn_merge_kernel<128>, dim3(Hkv), dim3(256), 0, s, a);
        else hipLaunchKernelGGL(attn_merge_kernel<64>, dim3(Hkv), dim3(256), 0, s, a);
    } else {
        const dim3 grid(Hkv * a.G * D / 64);
        if (D == 128) hipLaunchKernelGGL(attn_merge_wave_kernel<128>, grid, dim3(64), 0, s, a);
        else hipLaunchKernelGGL(attn_merge_wave_kernel<64>, grid, dim3(64), 0, s, a);
    }
    return fromHip(hipGetLastError(), "attn_decode");
}

bool flashDecodeSupports(int D, int G) { return (D == 64 || D == 128) && G >= 1 && G <= kMaxGroup; }
size_t flashDecodePartFloats(const kcFaDims& d) {
    return (size_t)d.N * d.H * ((d.T + kChunk - 1) / kChunk) * (d.D + 2);
}

int launchFlashDecode(const kcFlashDecodeArgs& a, hipStream_t s, int* slot, const FdRope* rope) {
    const kcFaDims& d = a.d;
    if (!flashDecodeSupports(d.D, d.group)) return fromHip(hipErrorInvalidValue, "flash_decode_f16: shape");
    if (rope && (d.N != 1 || d.H != d.H_kv * d.group))
        return fromHip(hipErrorInvalidValue, "flash_decode_f16: the RoPE prologue takes one query token");
    const int nch = (d.T + kChunk - 1) / kChunk;
    const dim3 grid(nch, d.H_kv, d.N);
    const FdRope rp = rope ? *rope : FdRope{};
#define KC_FD(DD, GG)                                                                                              \
    if (d.D == DD && d.group == GG) {                                                                              \
        if (rope)                                                                                                  \
            hipLaunchKernelGGL((flash_decode_kernel<DD, GG, true>), grid, dim3(256), 0, s, a.q, a.k, a.v, a.mask,  \
                               a.part, d, a.scale, nch, rp);                                                      \
        else                                                                                                       \
            hipLaunchKernelGGL((flash_decode_kernel<DD, GG, false>), grid, dim3(256), 0, s, a.q, a.k, a.v, a.mask, \
                               a.part, d, a.scale, nch, rp);                                                      \
    }
    KC_FD(128, 1) KC_FD(128, 2) KC_FD(128, 3) KC_FD(128, 4) KC_FD(128, 5) KC_FD(128, 6) KC_FD(128, 7) KC_FD(128, 8)
    KC_FD(64, 1) KC_FD(64, 2) KC_FD(64, 3) KC_FD(64, 4) KC_FD(64, 5) KC_FD(64, 6) KC_FD(64, 7) KC_FD(64, 8)
#undef KC_FD
    if (int e = fromHip(hipGetLastError(), "flash_decode_f16")) return e;
    if (slot && (d.N != 1 || (d.H * d.D) % 32)) return fromHip(hipErrorInvalidValue, "flash_decode_f16: slot of one token");
    const int nb = d.H * d.D / 32;
    if (d.D == 128)
        hipLaunchKernelGGL(flash_merge_kernel<128>, dim3(d.N * d.H), dim3(128), 0, s, a.part, a.out, nch, slot, nb);
    else
        hipLaunchKernelGGL(flash_merge_kernel<64>, dim3(d.N * d.H), dim3(128), 0, s, a.part, a.out, nch, slot, nb);
    return fromHip(hipGetLastError(), "flash_decode_f16: merge");
}

}  // namespace kcamd
