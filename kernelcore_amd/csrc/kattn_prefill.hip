// kattn_prefill.hip -- attention of a batch of queries on the matrix cores (gfx950), one workgroup
// per (query tile of 32, KV head): FLASH_ATTN_EXT (ggml-cpu/ops.cpp's online softmax; the reference's
// fa_scores / fa_max / fa_exp / fa_values, kernels/llm/flash_attn_f16.cu) for a causal prompt (the
// decode driver's prefill) or with ggml's f16 mask (the backend's batch FLASH_ATTN_EXT).
//
// The G = H / H_kv query heads of a KV head read the same keys and values, so they share one
// workgroup: wavefront w takes query head g G + w % G and key-block split w / G (S = 2 splits take
// alternate blocks of 32 keys). Each split's G wavefronts share its key block in LDS: K and V rows
// (and ggml's mask for the tile's 32 queries) arrive by buffer-to-LDS loads (rows padded by 16 B:
// the lanes of a read hit different banks) into a ring of three blocks, so two blocks' loads are in
// flight while one is computed (a memory round trip under this load outlasts a block's work).
// A causal prompt's tile reads the key blocks up to its last query. A masked one reads those its
// mask summary (mask_summary_kernel) names, lo .. hi, and loads the mask's values only for blocks
// mlo .. mhi (the others hold 0 for all 32 queries: the causal mask's blocks below the diagonal).
//
// Per wavefront (32 queries of one head, lane (j, h) = query j, lane half h):
//   S^T = K Q^T: v_mfma_f32_32x32x16_f16 with A = K rows (LDS), B = q split into fp16 hi = fp16(x)
//   and lo = fp16(x - hi) (registers; two chains, within about 2^-22 of f32 products). Lane (j, h)
//   then holds keys 8 (v / 4) + 4 h + v % 4 (v = 0..15) of query j.
//   Online softmax per query: the block maximum over both lane halves, alpha = exp(m_old - m_new),
//   p = exp(s - m_new) (masked scores -inf -> p = 0), the running sum per lane half.
//   O^T += V^T P^T: A = V^T, each lane's eight values gathered from eight V rows of LDS (16-bit
//   reads: the 32 lanes of a half read 32 consecutive d of one row); B = p scaled by 2^10 and split
//   into hi / lo fp16 the same way: with the MFMA's k index running over the keys in the order
//   kappa = {0-3, 8-11 | 4-7, 12-15} (+16), the score registers are directly the B operand.
//   Lane (j, h) holds O^T[d][j] for d = 32 t + 8 (v / 4) + 4 h + v % 4: its own query, so the
//   rescale by alpha needs no exchange between lanes.
// The two splits merge at the end through LDS (o = sum o_w exp(m_w - M) / sum l_w exp(m_w - M), the
// order of the one-head kernel before this one), and the output rows are written as float4.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "internal.hpp"
#include "model_kernels.hpp"

namespace kcamd {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4* LdsS4;
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* LdsPtr;

constexpr float kLog2e = 1.44269504f;
constexpr int kSplits = 2;
constexpr int kRing = 3;  // blocks per split in LDS

__device__ __forceinline__ __amdgpu_buffer_rsrc_t bufRes(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// LDS geometry for head size D.
template <int D>
struct AttnGeo {
    static constexpr int kCpr = D / 8;                  // 16-byte chunks per K / V row
    static constexpr int kKRow = 2 * D + 16;            // LDS bytes per K row (one pad chunk)
    // LDS bytes per V row (two pad chunks: 8 dwords mod 32 banks, so the four rows of a transposed
    // read's 16 lanes fall on different banks; K's one pad chunk keeps its 16-byte row reads apart)
    static constexpr int kVRow = 2 * D + 32;
    static constexpr int kKLoads = (32 * (kCpr + 1) + 63) / 64;  // 1 KiB direct loads per K or V block
    static constexpr int kKBytes = kKLoads * 1024;
    static_assert(32 * (kCpr + 2) <= kKLoads * 64, "V rows with two pad chunks in K's load count");
    static constexpr int kMRow = 20;                    // mask tile: dwords per row (16 + 4 pad)
    static constexpr int kMLoads = 32 * kMRow / 64;     // 256-byte direct loads of the mask tile
    static constexpr int kBuf = 2 * kKBytes + kMLoads * 256;  // one block of one split: K, V, mask
    static constexpr int kLoop = kRing * kSplits * kBuf;
    static constexpr int kORow = D / 2 + 4;             // merge: floats per lane (o, m, l, pad)
    static constexpr int kMerge(int G) { return G * 64 * kORow * 4; }
};

// MASKED: ggml's mask rows (m_row2 halves each) over t_host keys instead of the causal positions,
// msum the mask's summary per query tile ({lo, hi, mlo, mhi}).
template <int D, bool MASKED>
__global__ __launch_bounds__(512) void attn_prefill_gqa_kernel(const float* __restrict__ q, const int* __restrict__ kc,
                                                               const int* __restrict__ vc, float* __restrict__ out,
                                                               const int* __restrict__ n_ctx, AttnShape a,
                                                               const unsigned short* __restrict__ mask, int m_row2,
                                                               int t_host, int cache_rows,
                                                               const int* __restrict__ msum) {
    using Geo = AttnGeo<D>;
    constexpr int KS = D / 16, DB = D / 32;
    extern __shared__ int4 lds4[];
    char* lds = reinterpret_cast<char*>(lds4);
    const int G = a.H / a.H_kv;
    const int T = MASKED ? t_host : *n_ctx, N = a.N, p0 = T - N;
    const int tiles = (N + 31) / 32;
    const int i0 = (tiles - 1 - (int)blockIdx.x) * 32;  // longest query tiles first
    const int kvh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gw = wave % G, sp = wave / G;  // head within the group, split
    const int head = kvh * G + gw;
    const int j = lane & 31, h = lane >> 5;
    const int qpos = p0 + i0 + j;
    // key blocks kb0 .. kend - 1 (causal: up to the tile's last query), those of mlo .. mhi with the
    // mask's values
    int kb0 = 0, kend = min(p0 + i0 + 31, T - 1) / 32 + 1, mlo = 0, mhi = -1;
    if constexpr (MASKED) {
        const int* ms = msum + 4 * (i0 / 32);
        const int lo = ms[0], hi = ms[1];
        kb0 = lo <= hi ? lo : 0;
        kend = lo <= hi ? hi + 1 : 0;
        mlo = ms[2];
        mhi = ms[3];
    }
    auto mixed = [&](int kb) { return MASKED && kb >= mlo && kb <= mhi; };
    const int nit = (kend - kb0 + kSplits - 1) / kSplits;
    char* sbuf = lds + sp * kRing * Geo::kBuf;  // this split's ring

    // q of this lane's query as the B operand: hi / lo fp16 of values 16 ks + 8 h .. + 8
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

    // K and V rows by direct loads: slot L 64 + lane of a block's kKLoads loads holds key slot /
    // cpr, chunk slot % cpr, cpr = kCpr + 1 for K and kCpr + 2 for V (pad chunks and slots past 32
    // keys reread chunk 0 / key 31). Keys from T on read row T - 1: cache rows past the context are not written yet and may
    // hold any bits, and an Inf there times p = 0 would still make NaN (their scores are replaced
    // by -inf anyway). MASKED: the tile's 32 mask rows (queries past N read row N - 1), 32 keys each,
    // in dword loads (mask rows need only 4-byte alignment), kMRow dwords per LDS row; keys past the
    // mask's rows read the next row or zero (past the buffer), scores past T are replaced anyway.
    // Every wavefront issues the same count per block (the last load repeated: the same bytes to the
    // same place), so the waits below count loads.
    const uint32_t span = (uint32_t)((size_t)cache_rows * a.kv_row * 4 - (size_t)kvh * D * 2);
    const __amdgpu_buffer_rsrc_t rk = bufRes(kc + (size_t)kvh * (D / 2), span);
    const __amdgpu_buffer_rsrc_t rv = bufRes(vc + (size_t)kvh * (D / 2), span);
    const __amdgpu_buffer_rsrc_t rm = bufRes(mask, MASKED ? (uint32_t)((size_t)N * m_row2 * 2) : 0u);
    // loads per wavefront of block kb (with the mask's values or without)
    auto loadsOf = [&](int kb) { return (2 * Geo::kKLoads + (mixed(kb) ? Geo::kMLoads : 0) + G - 1) / G; };
    auto issue = [&](int kb, char* buf) {
        const int nl = 2 * Geo::kKLoads + (mixed(kb) ? Geo::kMLoads : 0), per = (nl + G - 1) / G;
        for (int i = 0; i < per; ++i) {
            const int L = min(gw + G * i, nl - 1);
            if (L < 2 * Geo::kKLoads) {
                const int LL = L < Geo::kKLoads ? L : L - Geo::kKLoads, cpr = L < Geo::kKLoads ? Geo::kCpr + 1 : Geo::kCpr + 2;
                const int slot = LL * 64 + lane, key = min(slot / cpr, 31), c = slot % cpr;
                const int row = min(kb * 32 + key, T - 1);
                const uint32_t voff = (uint32_t)row * (uint32_t)a.kv_row * 4u + (uint32_t)(c >= Geo::kCpr ? 0 : c) * 16u;
                if (L < Geo::kKLoads)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (LdsPtr)(buf + L * 1024), 16, voff, 0, 0, 0);
                else
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (LdsPtr)(buf + L * 1024), 16, voff, 0, 0, 0);
            } else if constexpr (MASKED) {
                const int LM = L - 2 * Geo::kKLoads;
                const int slot = LM * 64 + lane, r = slot / Geo::kMRow, c = slot % Geo::kMRow;
                const uint32_t voff = (uint32_t)min(i0 + r, N - 1) * (uint32_t)m_row2 * 2u +
                                      (uint32_t)(kb * 32 + 2 * (c < 16 ? c : 0)) * 2u;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (LdsPtr)(buf + 2 * Geo::kKBytes + LM * 256), 4, voff, 0,
                                                         0, 0);
            }
        }
    };
    // wait for all but this wavefront's last n loads
    auto waitBut = [&](int n) {
        switch (n) {
#define KC_VMCNT(x) \
    case x: asm volatile("s_waitcnt vmcnt(" #x ")" ::: "memory"); break;
            KC_VMCNT(1) KC_VMCNT(2) KC_VMCNT(3) KC_VMCNT(4) KC_VMCNT(5) KC_VMCNT(6) KC_VMCNT(7) KC_VMCNT(8)
            KC_VMCNT(9) KC_VMCNT(10) KC_VMCNT(11) KC_VMCNT(12) KC_VMCNT(13) KC_VMCNT(14) KC_VMCNT(15)
            KC_VMCNT(16) KC_VMCNT(17) KC_VMCNT(18) KC_VMCNT(19) KC_VMCNT(20) KC_VMCNT(21) KC_VMCNT(22)
            KC_VMCNT(23) KC_VMCNT(24) KC_VMCNT(25) KC_VMCNT(26) KC_VMCNT(27) KC_VMCNT(28) KC_VMCNT(29)
            KC_VMCNT(30) KC_VMCNT(31) KC_VMCNT(32) KC_VMCNT(33) KC_VMCNT(34) KC_VMCNT(35) KC_VMCNT(36)
            KC_VMCNT(37) KC_VMCNT(38) KC_VMCNT(39) KC_VMCNT(40) KC_VMCNT(41) KC_VMCNT(42) KC_VMCNT(43)
            KC_VMCNT(44) KC_VMCNT(45) KC_VMCNT(46) KC_VMCNT(47) KC_VMCNT(48) KC_VMCNT(49) KC_VMCNT(50)
#undef KC_VMCNT
            default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
        }
    };

    f32x16 zero;
#pragma unroll
    for (int v = 0; v < 16; ++v) zero[v] = 0.0f;
    f32x16 o[DB];
#pragma unroll
    for (int t = 0; t < DB; ++t) o[t] = zero;
    float m = -INFINITY, l = 0.0f;

    // block it of this split: kb = kSplits it + sp, in ring slot it % kRing
    if (kb0 + sp < kend) issue(kb0 + sp, sbuf);
    if (kb0 + sp + kSplits < kend) {
        issue(kb0 + sp + kSplits, sbuf + Geo::kBuf);
        waitBut(loadsOf(kb0 + sp + kSplits));
    } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    const int koff = j * Geo::kKRow + 16 * h;  // this lane's K row (A operand), half h
    const _Float16* vcol = nullptr;
    // this lane's row for the transposed V reads: group g = lane / 16 (lane half h = g / 2, d 16 (g % 2)
    // on), lane L = lane % 16 of it: key 4 h + L / 4, d 16 (g % 2) + 4 (L % 4)
    const int vlane = (4 * (lane >> 5) + ((lane & 15) >> 2)) * (Geo::kVRow / 2) + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    int rc = 0, rn = 2;  // ring slots of block it and of block it + 2
    for (int it = 0; it < nit; ++it) {
        const int kb = kb0 + kSplits * it + sp, kbn = kb + 2 * kSplits;
        char* cur = sbuf + rc * Geo::kBuf;
        if (kbn < kend) issue(kbn, sbuf + rn * Geo::kBuf);  // (its slot held block it - 1)
        bool work = kb < kend;
        float mval[16];
        if (!mixed(kb)) {  // (the block's mask is 0 for every query of the tile)
#pragma unroll
            for (int v = 0; v < 16; ++v) mval[v] = 0.0f;
        } else {  // a block whose mask is -inf for every query of the tile adds nothing
            uint32_t mk[8];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint2 w2 = *reinterpret_cast<const uint2*>(cur + 2 * Geo::kKBytes + j * Geo::kMRow * 4 +
                                                                 (8 * g + 4 * h) * 2);
                mk[2 * g] = w2.x;
                mk[2 * g + 1] = w2.y;
            }
            bool any = false;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t w2 = mk[v >> 1];
                mval[v] = (float)__builtin_bit_cast(_Float16, (unsigned short)((v & 1) ? (w2 >> 16) : (w2 & 0xFFFFu)));
                const int key = kb * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                any |= key < T && mval[v] != -INFINITY;
            }
            work = work && __ballot(any) != 0;
        }
        if (work) {
            // S^T = K Q^T, two chains (q hi, q lo)
            f32x16 sh = zero, sl = zero;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const h8 ka = *reinterpret_cast<const h8*>(cur + koff + 32 * ks);
                sh = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qb[ks], sh, 0, 0, 0);
                sl = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, ql[ks], sl, 0, 0, 0);
            }
            // scores of the lane's 16 keys; the causal limit (MASKED: the mask's values) and the end of
            // the context only in the blocks that reach them (a uniform branch)
            float sc[16];
            if ((MASKED ? mixed(kb) : kb * 32 + 31 > p0 + i0) || kb * 32 + 31 >= T) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int key = kb * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                    if constexpr (MASKED) sc[v] = key < T ? a.scale * (sh[v] + sl[v]) + mval[v] : -INFINITY;
                    else sc[v] = key <= qpos && key < T ? a.scale * (sh[v] + sl[v]) : -INFINITY;
                }
            } else {
#pragma unroll
                for (int v = 0; v < 16; ++v) sc[v] = a.scale * (sh[v] + sl[v]);
            }
            float bm = sc[0];
#pragma unroll
            for (int v = 1; v < 16; ++v) bm = fmaxf(bm, sc[v]);
            bm = fmaxf(bm, __shfl_xor(bm, 32));
            const float mn = fmaxf(m, bm);
            // exp2 on the transcendental unit (v_exp_f32: exp2f's result for arguments from -126 up,
            // 0 below, where p and alpha are absorbed by the sums they join); masked scores (-inf)
            // give 0 without a branch, and so does alpha for a first block (m = -inf); a query with
            // every score so far masked (mn = -inf) subtracts 0 instead
            const float msafe = mn == -INFINITY ? 0.0f : mn;
            const float alpha = __builtin_amdgcn_exp2f((m - msafe) * kLog2e);
            m = mn;
            h8 pa[2], pl[2];
            float ls = 0.0f;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float pv = __builtin_amdgcn_exp2f((sc[v] - msafe) * kLog2e);
                ls += pv;
                const float ps = pv * 1024.0f;
                const _Float16 hp = (_Float16)ps;
                pa[v >> 3][v & 7] = hp;
                pl[v >> 3][v & 7] = (_Float16)(ps - (float)hp);
            }
            l = l * alpha + ls;
#pragma unroll
            for (int t = 0; t < DB; ++t)
#pragma unroll
                for (int v = 0; v < 16; ++v) o[t][v] *= alpha;
            // O^T += V^T P^T: for half mm of the block's keys in kappa order, lane (j, h) needs
            // V[16 mm + 8 (e / 4) + 4 h + e % 4][32 t + j] for e = 0..7: two transposed reads
            // (ds_read_b64_tr_b16: in each group of 16 lanes, lane i receives element i % 4 of the
            // rows lanes 4 e + i / 4 address, e = 0..3; lane L here addresses V[key + L / 4][d0 +
            // 4 (L % 4)], so lane i receives V[key + e][d0 + i])
            vcol = reinterpret_cast<const _Float16*>(cur + Geo::kKBytes) + vlane;
#pragma unroll
            for (int mm = 0; mm < 2; ++mm)
#pragma unroll
                for (int t = 0; t < DB; ++t) {
                    const _Float16* vp = vcol + 16 * mm * (Geo::kVRow / 2) + 32 * t;
                    const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LdsS4)vp);
                    const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LdsS4)(vp + 8 * (Geo::kVRow / 2)));
                    const h8 va = __builtin_bit_cast(h8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                    o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pa[mm], o[t], 0, 0, 0);
                    o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pl[mm], o[t], 0, 0, 0);
                }
        }
        if (kbn < kend) waitBut(loadsOf(kbn));  // block it + 1 landed (block it + 2 may still be in flight)
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();  // block it read by every wavefront; block it + 1 staged
        rc = rc == kRing - 1 ? 0 : rc + 1;
        rn = rn == kRing - 1 ? 0 : rn + 1;
    }

    // ---- merge: split 1 hands (o, m, l) to split 0 through LDS (the loop's buffers)
    l += __shfl_xor(l, 32);
    float* mg = reinterpret_cast<float*>(lds) + (size_t)(gw * 64 + lane) * Geo::kORow;
    if (sp == 1) {
#pragma unroll
        for (int t = 0; t < DB; ++t)
#pragma unroll
            for (int v4 = 0; v4 < 4; ++v4)
                *reinterpret_cast<float4*>(mg + 16 * t + 4 * v4) =
                    make_float4(o[t][4 * v4], o[t][4 * v4 + 1], o[t][4 * v4 + 2], o[t][4 * v4 + 3]);
        mg[D / 2] = m;
        mg[D / 2 + 1] = l;
    }
    __syncthreads();
    if (sp == 1 || i0 + j >= N) return;
    const float m1 = mg[D / 2], l1 = mg[D / 2 + 1];
    const float M = fmaxf(m, m1);
    const float c0 = m == -INFINITY ? 0.0f : exp2f((m - M) * kLog2e);
    const float c1 = m1 == -INFINITY ? 0.0f : exp2f((m1 - M) * kLog2e);
    const float inv = 1.0f / ((l * c0 + l1 * c1) * 1024.0f);
    float* orow = out + (size_t)(i0 + j) * a.q_tok + (size_t)head * D + 4 * h;
#pragma unroll
    for (int t = 0; t < DB; ++t)
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
            const float4 o1 = *reinterpret_cast<const float4*>(mg + 16 * t + 4 * v4);
            float4 r;
            r.x = (o[t][4 * v4] * c0 + o1.x * c1) * inv;
            r.y = (o[t][4 * v4 + 1] * c0 + o1.y * c1) * inv;
            r.z = (o[t][4 * v4 + 2] * c0 + o1.z * c1) * inv;
            r.w = (o[t][4 * v4 + 3] * c0 + o1.w * c1) * inv;
            *reinterpret_cast<float4*>(orow + 32 * t + 8 * v4) = r;
        }
}

template <int D, bool MASKED>
int launchGqa(const float* q, const int* k, const int* v, float* out, const int* n_ctx, const AttnShape& a,
              const unsigned short* mask, int m_row2, int t_host, int cache_rows, const int* msum, hipStream_t s) {
    using Geo = AttnGeo<D>;
    const int G = a.H / a.H_kv;
    const int lds = std::max(Geo::kLoop, Geo::kMerge(G));
    static const int attr = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(attn_prefill_gqa_kernel<D, MASKED>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != 0) return fromHip(attr, "attn (prefill, GQA): LDS size");
    const dim3 grid((a.N + 31) / 32, a.H_kv);
    hipLaunchKernelGGL((attn_prefill_gqa_kernel<D, MASKED>), grid, dim3(64 * G * kSplits), lds, s, q, k, v, out,
                       n_ctx, a, mask, m_row2, t_host, cache_rows, msum);
    return fromHip(hipGetLastError(), MASKED ? "attn (masked, GQA)" : "attn (prefill, GQA)");
}

}  // namespace

bool attnGqaSupports(const AttnShape& a) {
    if (a.H_kv <= 0 || a.H % a.H_kv != 0) return false;
    const int G = a.H / a.H_kv;
    return (a.D == 64 || a.D == 128) && G >= 1 && G <= 4 && a.N > 0;
}

int launchAttnGqa(const float* q, const int* k, const int* v, float* out, const int* n_ctx, const AttnShape& a,
                  const unsigned short* mask, int m_row2, int t_host, int cache_rows, const int* msum, hipStream_t s) {
    if (!attnGqaSupports(a) || cache_rows <= 0 || (mask && !msum))
        return fromHip(hipErrorInvalidValue, "attn (GQA): shape");
    const bool masked = mask != nullptr;
    if (a.D == 128)
        return masked ? launchGqa<128, true>(q, k, v, out, n_ctx, a, mask, m_row2, t_host, cache_rows, msum, s)
                      : launchGqa<128, false>(q, k, v, out, n_ctx, a, mask, m_row2, t_host, cache_rows, msum, s);
    return masked ? launchGqa<64, true>(q, k, v, out, n_ctx, a, mask, m_row2, t_host, cache_rows, msum, s)
                  : launchGqa<64, false>(q, k, v, out, n_ctx, a, mask, m_row2, t_host, cache_rows, msum, s);
}

}  // namespace kcamd
