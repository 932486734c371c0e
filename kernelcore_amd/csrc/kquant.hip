// kquant.hip -- K-quant weight streams, activation quantizers and the decode matvecs (gfx950).
//
// Arithmetic follows the reference kernels operation by operation (arasheedu/Kernelcore
// kernels/llm/quantize_q8x4.cu, quantize_cols.cu, quantize_cols_k.cu, matvec_q4k_q8.cu,
// matvec_q6k_q8.cu; C++ mirror llm/llm_reference.cpp:79-104, 413-527). The library is built with
// -ffp-contract=off so no multiply-add is fused: quantized bytes, scales and matvec outputs are
// bit-identical to the reference. Only the work distribution is new:
//   - quantizers: 8 lanes per block of 32 (per-32) or one wavefront per 256 (per-256), with the
//     max and the sums reduced across lanes (both are order-independent: max and integer sums);
//   - matvecs: one lane per (row, super-block), 16 rows x 4 super-blocks per wavefront, weights
//     streamed from the slab layout of kquant.hpp with one coalesced dwordx4 load per slab.
//     Each lane writes its super-block's float term (d*fd - dmin*fm, or the two Q6_K halves)
//     to LDS; the row sums are then added in super-block order, the reference's order.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "internal.hpp"
#include "kquant.hpp"
#include "kquant_device.hpp"
#include "launch.hpp"

namespace kcamd {
namespace {

constexpr int kXsStride = 68;  // LDS ints per super-block of activations (64 + 4 pad)

// ---------------------------------------------------------------- weight streams

// One thread per 16-byte piece of the stream. Q6_K segments end with 8 pieces holding the
// 64 fp16 d values.
template <bool Q6>
__global__ void repack_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int rows, int nsb,
                              int ngroups, long long pieces, bool unpack) {
    const long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= pieces) return;
    constexpr int kSlabs = Q6 ? kQ6kSlabs : kQ4kSlabs;
    constexpr int kPer = kSlabs * 64 + (Q6 ? 8 : 0);
    constexpr int kBlock = Q6 ? kQ6kBlock : kQ4kBlock;
    constexpr int kSeg = Q6 ? kQ6kSeg : kQ4kSeg;
    const long long seg = p / kPer;
    const int q = (int)(p - seg * kPer);
    const int tile = (int)(seg / ngroups);
    const int g = (int)(seg - (long long)tile * ngroups);
    uint8_t* out = dst + seg * kSeg;
    if (q < kSlabs * 64) {
        const int c = q >> 6, lane = q & 63;
        const int row = tile * kTileRows + (lane & 15), s = g * kGroupSb + (lane >> 4);
        uint8_t* piece = out + c * 1024 + lane * 16;
        const bool real = row < rows && s < nsb;
        const size_t boff = ((size_t)row * nsb + s) * kBlock + 16 * c;
        if (!unpack) {
            for (int i = 0; i < 16; ++i) piece[i] = real ? src[boff + i] : 0;
        } else if (real) {
            const uint8_t* in = src + seg * kSeg + c * 1024 + lane * 16;
            for (int i = 0; i < 16; ++i) dst[boff + i] = in[i];
        }
        if (unpack) return;
    } else {  // Q6_K d plane: 8 lanes per piece
        const int j = q - kSlabs * 64;
        for (int i = 0; i < 8; ++i) {
            const int lane = j * 8 + i;
            const int row = tile * kTileRows + (lane & 15), s = g * kGroupSb + (lane >> 4);
            const bool real = row < rows && s < nsb;
            const size_t boff = ((size_t)row * nsb + s) * kBlock + 208;
            if (!unpack) {
                uint8_t* d = out + kSlabs * 1024 + lane * 2;
                d[0] = real ? src[boff] : 0;
                d[1] = real ? src[boff + 1] : 0;
            } else if (real) {
                const uint8_t* in = src + seg * kSeg + kSlabs * 1024 + lane * 2;
                dst[boff] = in[0];
                dst[boff + 1] = in[1];
            }
        }
    }
}

// ---------------------------------------------------------------- activation quantizers

// q = x * id rounded half away from zero, clamped to +-127 (quantize_q8x4.cu:22-33).
__device__ __forceinline__ int q8round(float v, float id) {
    const float t = v * id;
    int q;
    if (t >= 0.0f) q = (int)(t + 0.5f);
    else q = (int)(t - 0.5f);
    return q > 127 ? 127 : (q < -127 ? -127 : q);
}
__device__ __forceinline__ float absmax4(float4 v) {
    float a = fmaxf(0.0f, fmaxf(v.x, 0.0f - v.x));
    a = fmaxf(a, fmaxf(v.y, 0.0f - v.y));
    a = fmaxf(a, fmaxf(v.z, 0.0f - v.z));
    return fmaxf(a, fmaxf(v.w, 0.0f - v.w));
}
__device__ __forceinline__ int pack4(float4 v, float id, int* sum) {
    const int a = q8round(v.x, id), b = q8round(v.y, id), c = q8round(v.z, id), d = q8round(v.w, id);
    *sum = a + b + c + d;
    return (a & 255) | ((b & 255) << 8) | ((c & 255) << 16) | ((d & 255) << 24);
}

// Per-32 blocks: 8 lanes per block, lane w packs word w. Column c of `ncols` (k values each)
// writes its slot (xq at q + c * slot, xd after the nb * 8 words); count = nb * ncols.
// With slot == 0 the blocks are contiguous (quantize_q8x4: xq, xd separate arrays).
__device__ __forceinline__ float4 load4(const float* p, bool vec) {
    if (vec) return *reinterpret_cast<const float4*>(p);
    return make_float4(p[0], p[1], p[2], p[3]);
}

template <bool Vec>  // Vec: x is 16-byte aligned, one dwordx4 load per lane
__global__ void quantize_q8_kernel(const float* __restrict__ x, int* __restrict__ xq, float* __restrict__ xd,
                                   int count, int nb, int slot) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int b = t >> 3, w = t & 7;
    const bool live = b < count;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) v = load4(x + ((size_t)b * 8 + w) * 4, Vec);
    float amax = absmax4(v);
    amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
    const float d = amax / 127.0f;
    float id;
    if (d > 0.0f) id = 1.0f / d;
    else id = 0.0f;
    int sum;
    const int word = pack4(v, id, &sum);
    sum += __shfl_xor(sum, 1, 8);
    sum += __shfl_xor(sum, 2, 8);
    sum += __shfl_xor(sum, 4, 8);
    if (!live) return;
    int* wq;
    float* wd;
    if (slot) {
        const int c = b / nb, bl = b - c * nb;
        int* base = xq + (size_t)c * slot;
        wq = base + bl * 8;
        wd = reinterpret_cast<float*>(base + nb * 8) + bl * 2;
    } else {
        wq = xq + (size_t)b * 8;
        wd = xd + (size_t)b * 2;
    }
    wq[w] = word;
    if (w == 0) {
        wd[0] = d;
        wd[1] = (float)sum;
    }
}

// Per-256 slots (quantize_cols_k.cu:20-74): one wavefront per (column, super-block); lane L packs
// word L (values 4L..4L+3), sums of 16 come from lanes 4g..4g+3, sums of 32 from lanes 8i..8i+7.
// ao (has_ao): the same codes also in the MFMA matmul's layout (ActF16): fp16 codes, the min
// operands 64 (B_i >> 6) and B_i & 63 from lanes 8i, the scale from lane 0.
template <bool Vec>
__global__ void quantize_k_kernel(const float* __restrict__ x, int* __restrict__ q, int nsb, int count, ActF16 ao,
                                  int has_ao) {
    const int wid = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wid >= count) return;  // whole wavefronts
    const int c = wid / nsb, s = wid - c * nsb;
    const float4 v = load4(x + (size_t)c * nsb * 256 + (size_t)s * 256 + lane * 4, Vec);
    float amax = absmax4(v);
    for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    const float d = amax / 127.0f;
    float id;
    if (d > 0.0f) id = 1.0f / d;
    else id = 0.0f;
    int s4;
    const int word = pack4(v, id, &s4);
    int s16 = s4 + __shfl_xor(s4, 1);
    s16 += __shfl_xor(s16, 2);
    int s32 = s16 + __shfl_xor(s16, 4);
    if (q) {  // the int8 slot (null: a caller whose products read only the MFMA layout)
        int* qc = q + (size_t)c * nsb * 85;
        qc[s * 64 + lane] = word;
        if ((lane & 3) == 0) qc[nsb * 65 + s * 16 + (lane >> 2)] = s16;
        // Lane 0 gathers B_i (lanes 8i): words [B>>6 of sums 0-3 | of 4-7 | B&63 of 0-3 | of 4-7].
        int pw[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int b = __shfl(s32, 8 * i);
            const int sh = 8 * (i & 3);
            pw[i >> 2] |= ((b >> 6) & 255) << sh;
            pw[2 + (i >> 2)] |= (b & 63) << sh;
        }
        if (lane == 0) {
            for (int i = 0; i < 4; ++i) qc[nsb * 81 + s * 4 + i] = pw[i];
            reinterpret_cast<float*>(qc + nsb * 64)[s] = d;
        }
    }
    if (has_ao) {
        const int k = nsb * 256;
        typedef _Float16 hv4 __attribute__((ext_vector_type(4)));
        hv4 hq;
#pragma unroll
        for (int e = 0; e < 4; ++e) hq[e] = (_Float16)(float)(16 * ((word << (24 - 8 * e)) >> 24));  // 16 x
        *reinterpret_cast<hv4*>(static_cast<_Float16*>(ao.act) + (size_t)c * k + s * 256 + 4 * lane) = hq;
        if ((lane & 7) == 0) {
            _Float16* mn = static_cast<_Float16*>(ao.mins) + ((size_t)c * nsb + s) * 16 + (lane >> 3);
            mn[0] = (_Float16)(float)(64 * (s32 >> 6));
            mn[8] = (_Float16)(float)(s32 & 63);
        }
        if (lane == 0) ao.xdT[(size_t)s * ao.ncp + c] = d;
    }
}

// ---------------------------------------------------------------- decode matvecs

// AF (k <= 4096: at most four activation words and one (d, sum) pair per thread): the activations
// are loaded into registers before the first segment's weights, so the staging waits for them alone
// (a wave's vector loads complete in issue order); else the weights go out first and the staging's
// loads after them.
template <bool Q6, int WT, bool PIPE, bool NT, bool AF>
__global__ __launch_bounds__(256) void matvec_kq_kernel(const uint8_t* __restrict__ qw, const int* __restrict__ xq,
                                                        const float* __restrict__ xd, float* __restrict__ y, int rows,
                                                        int nsb, int ntiles) {
    constexpr int WK = 4 / WT;  // waves of one tile splitting its super-block groups
    constexpr int kSeg = Q6 ? kQ6kSeg : kQ4kSeg;
    extern __shared__ int4 lds4[];
    int* lds = reinterpret_cast<int*>(lds4);
    const int ngroups = (nsb + kGroupSb - 1) / kGroupSb;
    const int nsbp = ngroups * kGroupSb;
    const int nt = Q6 ? 2 * nsbp : nsbp;
    int* xs = lds;
    float* dx = reinterpret_cast<float*>(xs + nsbp * kXsStride);
    float* aux = dx + nsbp * 8;
    int* s16 = reinterpret_cast<int*>(aux + nsbp * 8);
    float* terms = reinterpret_cast<float*>(s16 + nsbp * 8);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wt = wave % WT, wk = wave / WT;
    const int tile = blockIdx.x * WT + wt;
    const int kq = lane >> 4, r = lane & 15;
    const bool live = tile < ntiles;
    const uint8_t* seg0 = qw + (size_t)(live ? tile : 0) * ngroups * kSeg;

    Pieces<Q6, NT> cur;
    int g = wk;
    if constexpr (AF) {
        // unconditional, clamped 4-byte loads (xq needs no 16-byte alignment), then the weights
        const int nw = nsb * 64, nbk = nsb * 8;
        int xw[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) xw[u] = xq[min(u * 256 + tid, nw - 1)];
        const float d0 = xd[2 * min(tid, nbk - 1)], s0 = xd[2 * min(tid, nbk - 1) + 1];
        if (live && g < ngroups) cur.load(seg0 + (size_t)g * kSeg, lane);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = u * 256 + tid;
            if (i < nsbp * 64) xs[(i >> 6) * kXsStride + (i & 63)] = i < nw ? xw[u] : 0;
        }
        if (tid < nsbp * 8) {
            const float d = tid < nbk ? d0 : 0.0f, sm = tid < nbk ? s0 : 0.0f;
            dx[tid] = d;
            if (Q6) reinterpret_cast<int*>(aux)[tid] = (int)sm;
            else aux[tid] = d * sm;
        }
        if (Q6) {  // the sums of the blocks' first 16 values, from the staged words
            __syncthreads();
            if (tid < nsbp * 8) {
                int a = 0;
                if (tid < nbk)
                    for (int w = 0; w < 4; ++w) a = dot4(0x01010101, xs[(tid >> 3) * kXsStride + (tid & 7) * 8 + w], a);
                s16[tid] = a;
            }
        }
    } else {
        // The first segment's loads go out before the activations are staged, so both latencies overlap.
        if (live && g < ngroups) cur.load(seg0 + (size_t)g * kSeg, lane);
        for (int i = tid; i < nsbp * 64; i += 256) {  // 4-byte loads: xq needs no 16-byte alignment
            const int s = i >> 6, w = i & 63;
            xs[s * kXsStride + w] = s < nsb ? xq[i] : 0;
        }
        for (int b = tid; b < nsbp * 8; b += 256) {
            float d = 0.0f, sm = 0.0f;
            if (b < nsb * 8) {
                d = xd[2 * b];
                sm = xd[2 * b + 1];
            }
            dx[b] = d;
            if (Q6) {
                reinterpret_cast<int*>(aux)[b] = (int)sm;
                int a = 0;
                if (b < nsb * 8)
                    for (int w = 0; w < 4; ++w) a = dot4(0x01010101, xq[b * 8 + w], a);
                s16[b] = a;
            } else {
                aux[b] = d * sm;
            }
        }
    }
    __syncthreads();

    float* tterms = terms + wt * nt * 16;
    if (live) {
        while (g < ngroups) {
            const int gn = g + WK;
            Pieces<Q6, NT> nxt;
            if (PIPE && gn < ngroups) nxt.load(seg0 + (size_t)gn * kSeg, lane);
            const uint32_t* c = reinterpret_cast<const uint32_t*>(cur.c);
            const int s = g * kGroupSb + kq;
            if (Q6) {
                float t0, t1;
                q6k_terms(c, cur.dbits, xs + s * kXsStride, dx + 8 * s, reinterpret_cast<const int*>(aux) + 8 * s,
                          s16 + 8 * s, &t0, &t1);
                tterms[(2 * s) * 16 + r] = t0;
                tterms[(2 * s + 1) * 16 + r] = t1;
            } else {
                tterms[s * 16 + r] = q4k_term(c, xs + s * kXsStride, dx + 8 * s, aux + 8 * s);
            }
            if (PIPE) cur = nxt;
            else if (gn < ngroups) cur.load(seg0 + (size_t)gn * kSeg, lane);
            g = gn;
        }
    }
    __syncthreads();
    if (live && wk == 0 && kq == 0) {
        const int row = tile * kTileRows + r;
        const int nreal = Q6 ? 2 * nsb : nsb;
        float acc = 0.0f;
        for (int t = 0; t < nreal; ++t) acc += tterms[t * 16 + r];
        if (row < rows) y[row] = acc;
    }
}

constexpr size_t kMatvecMaxLds = 65536;

size_t matvecLds(bool q6, int nsb, int wt) {
    const int nsbp = groupsOf(nsb) * kGroupSb;
    const int nt = q6 ? 2 * nsbp : nsbp;
    return sizeof(int) * (size_t(nsbp) * (kXsStride + 24) + size_t(wt) * nt * 16);
}

template <bool Q6, int WT, bool PIPE, bool NT>
int runMatvec(const kcMatvecQ4Q8Args& a, hipStream_t s) {
    const int nsb = a.k / 256;
    const int ntiles = tilesOf(a.rows);
    const size_t lds = matvecLds(Q6, nsb, WT);
    const int blocks = (ntiles + WT - 1) / WT;
    const auto* qw = reinterpret_cast<const uint8_t*>(a.qw);
    // Activations first for a small matrix (one tile per workgroup), where they fit four words per
    // thread: config 1 (3072 x 3072) 3.97 -> 3.74 us per matvec in a replayed graph. A large one
    // starts its weight stream first (config 2: 48.2 against 49.5 us). Option matvec_af = 1: weights
    // first always, 2: activations first wherever they fit.
    const int af = option("matvec_af");
    if (groupsOf(nsb) * kGroupSb * 64 <= 4 * 256 && af != 1 && (WT == 1 || af == 2))
        hipLaunchKernelGGL((matvec_kq_kernel<Q6, WT, PIPE, NT, true>), dim3(blocks), dim3(256), lds, s, qw, a.xq, a.xd,
                           a.y, a.rows, nsb, ntiles);
    else
        hipLaunchKernelGGL((matvec_kq_kernel<Q6, WT, PIPE, NT, false>), dim3(blocks), dim3(256), lds, s, qw, a.xq, a.xd,
                           a.y, a.rows, nsb, ntiles);
    return fromHip(hipGetLastError(), Q6 ? "matvec_q6k_q8" : "matvec_q4k_q8");
}

template <bool Q6, int WT>
int pickVariant(const kcMatvecQ4Q8Args& a, bool pipe, bool nt, hipStream_t s) {
    if (pipe) return nt ? runMatvec<Q6, WT, true, true>(a, s) : runMatvec<Q6, WT, true, false>(a, s);
    return nt ? runMatvec<Q6, WT, false, true>(a, s) : runMatvec<Q6, WT, false, false>(a, s);
}

template <bool Q6>
int pickShape(const kcMatvecQ4Q8Args& a, int wt, bool pipe, bool nt, hipStream_t s) {
    if (wt == 4) return pickVariant<Q6, 4>(a, pipe, nt, s);
    if (wt == 2) return pickVariant<Q6, 2>(a, pipe, nt, s);
    return pickVariant<Q6, 1>(a, pipe, nt, s);
}

}  // namespace

// ---------------------------------------------------------------- launchers

int launchRepack(const kcKquantRepackArgs& a, bool unpack, hipStream_t s) {
    const bool q6 = a.qtype == KC_QTYPE_Q6_K;
    const int nsb = a.k / 256;
    const int ngroups = groupsOf(nsb);
    const long long segs = (long long)tilesOf(a.rows) * ngroups;
    const long long pieces = segs * (q6 ? kQ6kSlabs * 64 + 8 : kQ4kSlabs * 64);
    const unsigned blocks = (unsigned)((pieces + 255) / 256);
    if (pieces == 0) return 0;
    const uint8_t* src = static_cast<const uint8_t*>(a.src);
    uint8_t* dst = static_cast<uint8_t*>(a.dst);
    if (q6)
        hipLaunchKernelGGL(repack_kernel<true>, dim3(blocks), dim3(256), 0, s, src, dst, a.rows, nsb, ngroups, pieces,
                           unpack);
    else
        hipLaunchKernelGGL(repack_kernel<false>, dim3(blocks), dim3(256), 0, s, src, dst, a.rows, nsb, ngroups, pieces,
                           unpack);
    return fromHip(hipGetLastError(), unpack ? "unpack_kquant" : "repack_kquant");
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static void quantizeQ8(const float* x, int* xq, float* xd, int count, int nb, int slot, hipStream_t s) {
    const long long threads = (long long)count * 8;
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (aligned16(x)) hipLaunchKernelGGL(quantize_q8_kernel<true>, grid, dim3(256), 0, s, x, xq, xd, count, nb, slot);
    else hipLaunchKernelGGL(quantize_q8_kernel<false>, grid, dim3(256), 0, s, x, xq, xd, count, nb, slot);
}

int launchQuantizeQ8x4(const float* x, int* xq, float* xd, int count, hipStream_t s) {
    if (count == 0) return 0;
    quantizeQ8(x, xq, xd, count, 0, 0, s);
    return fromHip(hipGetLastError(), "quantize_q8x4");
}

int launchQuantizeCols(const float* x, int* q, int k, int ncols, hipStream_t s) {
    const int nb = k / 32;
    quantizeQ8(x, q, nullptr, nb * ncols, nb, nb * 11, s);
    return fromHip(hipGetLastError(), "quantize_cols");
}

int launchQuantizeColsK(const float* x, int* q, int k, int ncols, hipStream_t s, const ActF16* ao) {
    if (!q && !ao) return fromHip(hipErrorInvalidValue, "quantize_cols_k: no output");
    const int nsb = k / 256;
    const long long waves = (long long)nsb * ncols;
    const dim3 grid((unsigned)((waves + 3) / 4));
    const ActF16 a = ao ? *ao : ActF16{};
    if (aligned16(x))
        hipLaunchKernelGGL(quantize_k_kernel<true>, grid, dim3(256), 0, s, x, q, nsb, (int)waves, a, ao ? 1 : 0);
    else hipLaunchKernelGGL(quantize_k_kernel<false>, grid, dim3(256), 0, s, x, q, nsb, (int)waves, a, ao ? 1 : 0);
    return fromHip(hipGetLastError(), "quantize_cols_k");
}

int launchMatvecKq(bool q6k, const kcMatvecQ4Q8Args& a, hipStream_t s) {
    if (a.rows == 0) return 0;
    // Tiles per workgroup: 4 when there are enough tiles to fill the GPU several times over,
    // else fewer, with the remaining waves splitting the super-block groups of one tile
    // (measured on MI355X: 128256 rows best at 4, 1024-16384 rows best at 1).
    const int ntiles = tilesOf(a.rows);
    int wt = option("matvec_waves");  // forced tiles per workgroup (1, 2 or 4)
    if (wt != 1 && wt != 2 && wt != 4) wt = ntiles >= 4096 ? 4 : (ntiles >= 2048 ? 2 : 1);
    while (wt > 1 && matvecLds(q6k, a.k / 256, wt) > kMatvecMaxLds) wt /= 2;
    // 0 = default, 1 = off, 2 = on. Defaults: non-temporal weight loads (about 10% faster at
    // config 2), no software pipelining (it costs occupancy and measured slower).
    const int po = option("matvec_pipe"), no = option("matvec_nt");
    const bool pipe = po == 2;
    const bool nt = no != 1;
    return q6k ? pickShape<true>(a, wt, pipe, nt, s) : pickShape<false>(a, wt, pipe, nt, s);
}

}  // namespace kcamd
