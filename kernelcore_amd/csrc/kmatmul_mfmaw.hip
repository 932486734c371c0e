// kmatmul_mfmaw.hip -- the prefill matmul's wide-tile MFMA kernel (gfx950): Y = W X for Q4_K / Q6_K
// weights and per-256 8-bit activations, the arithmetic of kmatmul_mfma.hip (exact integer sums per
// super-block on v_mfma_f32_32x32x16_f16, the reference's combine per super-block; reference
// kernels/llm/matmul_q4k_q8kx8.cu, matmul_q6k_q8kx8.cu, mirror llm/llm_reference.cpp:529-596) with
// a tiling that dequantizes every weight once per workgroup instead of once per wavefront.
// Selected by the option matmul_path = 7; not the default (measured below).
//
// A workgroup of 4 wavefronts owns 128 weight rows x 128 activation columns; wavefront w computes
// rows 64 (w & 1) .. +64 and columns 64 (w >> 1) .. +64 as 2 x 2 blocks of 32 x 32, so every A
// (activation) fragment it reads from LDS feeds two matrix ops and every B (weight) fragment two.
// K advances in stages of a quarter super-block (64 values):
//   - the activations of a stage (already fp16, 16 x, from act_to_f16 or the quantizers) arrive by
//     direct buffer-to-LDS loads, three stages ahead, into a ring of four tiles; 144 bytes per
//     column (64 halves + 16 B of padding: the eight lanes of one LDS read phase hit distinct banks);
//   - the weights of a stage are dequantized by all 256 threads (thread t: row t % 128, half t / 128,
//     32 weights) from the stream into the MFMA operand form (Q4_K: sc q / 16; Q6_K: sh (q - 32) and
//     sl (q - 32) / 16, sc = 16 sh + sl) and written to one of two LDS tiles with the same pitch, a
//     quarter between each K-step's matrix ops of the stage before; their raw bytes are loaded two
//     dequantizations ahead;
//   - the fragments of K-step t + 1 are read from LDS while K-step t runs its matrix ops.
// After a super-block's fourth stage: the Q4_K min term (one more matrix op per block against the
// staged [64 (B >> 6), B & 63] operands) and the combine acc += xd (d is - dmin im) (Q6_K:
// acc += (d xd) is), as in kmatmul_mfma.hip.
//
// Measured on MI355X (gate 8192 x 3072 x 512, Q4_K, the kernel alone after a clock warm-up): 43.6 us
// against about 40 us for kmatmul_mfma.hip's kernel. At one wavefront per SIMD (the LDS of the ring
// and 364 registers per lane) nothing hides the barrier per stage and the exposed LDS and memory
// latencies: without the dequantization and the combine the same pipeline still takes 28 us.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "internal.hpp"
#include "kmatmul_mfma.hpp"
#include "kquant.hpp"

namespace kcamd {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32v4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* LdsPtr;

constexpr int kWRows = 128;  // weight rows per workgroup
constexpr int kPitch = 144;  // LDS bytes per row / column of a stage: 64 halves + 16 B

__device__ __forceinline__ h2 bits_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }

template <bool Q6, int CB>
struct WGeo {
    static constexpr int kCols = 64 * CB;                 // activation columns per workgroup
    static constexpr int kAB = kCols * kPitch;            // activation tile of a stage
    static constexpr int kALoads = kAB / 1024;            // its direct 1 KB loads
    static constexpr int kAPerWave = (kALoads + 3) / 4;   // per wavefront (the last ones repeat)
    static constexpr int kBB = kWRows * kPitch;           // one weight operand tile of a stage
    static constexpr int kBS = (Q6 ? 2 : 1) * kBB;        // the weight operands of a stage
    static constexpr int kMinsB = Q6 ? 0 : kCols * 32;    // Q4_K min operands of a super-block
    static constexpr int kScB = 1024;                     // column scales of a super-block (<= 256 columns)
    static constexpr int kSb = kMinsB + kScB;
    // LDS: a ring of four activation tiles (stage st in tile st % 4), two weight tiles (st % 2),
    // two super-block regions (min operands and column scales, by super-block parity)
    static constexpr int kBOff = 4 * kAB;
    static constexpr int kSbOff = kBOff + 2 * kBS;
    static constexpr int kLds = kSbOff + 2 * kSb;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t bufRes(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Eight 4-bit weights (nibble `hiNib` of 8 bytes) -> sc q / 16 as fp16 (exact): (1024 + q) m + c.
__device__ __forceinline__ h8 nib8(uint32_t w0, uint32_t w1, bool hiNib, h2 m2, h2 c2) {
    const uint32_t mask = hiNib ? 0xFFF0FFF0u : 0xFF0FFF0Fu;
    h8 r;
    const uint32_t w[2] = {w0, w1};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const h2 a = bits_h2(__builtin_amdgcn_perm(0x64646464u, w[i], 0x04010400u) & mask);
        const h2 b = bits_h2(__builtin_amdgcn_perm(0x64646464u, w[i], 0x04030402u) & mask);
        const h2 ra = __builtin_elementwise_fma(a, m2, c2), rb = __builtin_elementwise_fma(b, m2, c2);
        r[4 * i + 0] = ra[0];
        r[4 * i + 1] = ra[1];
        r[4 * i + 2] = rb[0];
        r[4 * i + 3] = rb[1];
    }
    return r;
}

// Q6_K: eight 6-bit weights (bytes q, each 0..63) -> sh (q - 32) and sl (q - 32) / 16 (exact fp16).
__device__ __forceinline__ void six8(uint32_t q0, uint32_t q1, h2 mh, h2 ch, h2 ml, h2 cl, h8& hi, h8& lo) {
    const uint32_t q[2] = {q0, q1};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const h2 a = bits_h2(__builtin_amdgcn_perm(0x64646464u, q[i], 0x04010400u));  // 1024 + q
        const h2 b = bits_h2(__builtin_amdgcn_perm(0x64646464u, q[i], 0x04030402u));
        const h2 ah = __builtin_elementwise_fma(a, mh, ch), bh = __builtin_elementwise_fma(b, mh, ch);
        const h2 al = __builtin_elementwise_fma(a, ml, cl), bl = __builtin_elementwise_fma(b, ml, cl);
        hi[4 * i + 0] = ah[0];
        hi[4 * i + 1] = ah[1];
        hi[4 * i + 2] = bh[0];
        hi[4 * i + 3] = bh[1];
        lo[4 * i + 0] = al[0];
        lo[4 * i + 1] = al[1];
        lo[4 * i + 2] = bl[0];
        lo[4 * i + 3] = bl[1];
    }
}

// The raw weight bytes one thread dequantizes per stage (row t / 2, half t % 2 of the 64 values).
// Q4_K: 16 bytes of qs (32 nibbles: sub-blocks 2q and 2q + 1, positions 16 h .. +16).
// Q6_K: 32 ql bytes and 32 qh bytes (one (n, quad) run of 32 values).
template <bool Q6>
struct RawW;
template <>
struct RawW<false> {
    uint4 qs;
};
template <>
struct RawW<true> {
    uint4 ql[2], qh[2];
};

template <bool Q6, int CB>
struct WTile {
    using G = WGeo<Q6, CB>;
    // thread roles
    int tid, lane, wave, wr, wc, l32, h;
    // dequantization: this thread's stream row (clamped into the stream) and half
    const uint8_t* qw;
    int drow, drl, dh, ngroups;  // drl: the row within the tile
    // stream addressing of a (row, super-block) piece: segment base + piece offset
    __device__ __forceinline__ const uint8_t* piece(int row, int s) const {
        const int tile = row >> 4, r = row & 15, g = s >> 2, kq = s & 3;
        return qw + ((size_t)tile * ngroups + g) * (Q6 ? kQ6kSeg : kQ4kSeg) + (kq * 16 + r) * 16;
    }
    // Q4_K: the raw bytes of stage q; Q6_K: of stages 2n and 2n + 1 (the same bytes: the two
    // stages take the low / high nibbles and qh bits 2 quad with quad = 2 (q & 1) + dh)
    __device__ __forceinline__ void loadRaw(RawW<Q6>& r, int s, int qn) const {
        const uint8_t* p = piece(drow, s);
        if constexpr (!Q6) {
            r.qs = *reinterpret_cast<const uint4*>(p + (1 + 2 * qn + dh) * 1024);
        } else {
            const int n = qn;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                r.ql[u] = *reinterpret_cast<const uint4*>(p + (4 * n + 2 * dh + u) * 1024);
                r.qh[u] = *reinterpret_cast<const uint4*>(p + (8 + 2 * n + u) * 1024);
            }
        }
    }
    // Q4_K header (d, dmin, 12 scale bytes) / Q6_K 16 scale bytes, of this thread's dequant row
    __device__ __forceinline__ uint4 loadHdrD(int s) const {
        const uint8_t* p = piece(drow, s);
        return *reinterpret_cast<const uint4*>(p + (Q6 ? 12 * 1024 : 0));
    }
    // The per-stage constants of the dequantization of stage q (super-block header / scales hd):
    // Q4_K: the (1024 + q) -> sc q / 16 multipliers and offsets of sub-blocks 2q (low nibbles)
    // and 2q + 1 (high); Q6_K: sh (q - 32) and sl (q - 32) / 16 ones of this thread's two
    // sub-blocks of 16.
    struct DqC {
        h2 m[2], c[2], ml[2], cl[2];
    };
    __device__ __forceinline__ DqC dqPrep(uint4 hd, int q) const {
        DqC k;
        if constexpr (!Q6) {
            const int s0 = (int)hd.y, s2 = (int)hd.w;
            const int scw0 = s0 & 0x3F3F3F3F;
            const int scw1 = (s2 & 0x0F0F0F0F) | ((s0 >> 2) & 0x30303030);
            const int j0 = 2 * q, j1 = 2 * q + 1;
            const int sc0 = ((j0 < 4 ? scw0 : scw1) >> (8 * (j0 & 3))) & 255;
            const int sc1 = ((j1 < 4 ? scw0 : scw1) >> (8 * (j1 & 3))) & 255;
            const _Float16 f0 = (_Float16)(float)sc0, f1 = (_Float16)(float)sc1;
            // low nibble: (1024 + q) sc / 16 - 64 sc; high nibble: (1024 + 16 q) sc / 256 - 4 sc
            const _Float16 m0 = f0 * (_Float16)0.0625f, c0 = f0 * (_Float16)(-64.0f);
            const _Float16 m1 = f1 * (_Float16)0.00390625f, c1 = f1 * (_Float16)(-4.0f);
            k.m[0] = h2{m0, m0};
            k.c[0] = h2{c0, c0};
            k.m[1] = h2{m1, m1};
            k.c[1] = h2{c1, c1};
        } else {
            const uint32_t sw[4] = {hd.x, hd.y, hd.z, hd.w};
#pragma unroll
            for (int g2 = 0; g2 < 2; ++g2) {  // scale 4q + 2 dh + g2 (values 16 g2 .. of this half)
                const int gi = 4 * q + 2 * dh + g2;
                const int sc = ((int)(sw[gi >> 2] << (24 - 8 * (gi & 3)))) >> 24;
                const int sh = sc >> 4, sl = sc & 15;
                const _Float16 fh = (_Float16)(float)sh, fl = (_Float16)(float)sl;
                const _Float16 ch = fh * (_Float16)(-1056.0f), mlv = fl * (_Float16)0.0625f, clv = fl * (_Float16)(-66.0f);
                k.m[g2] = h2{fh, fh};
                k.c[g2] = h2{ch, ch};
                k.ml[g2] = h2{mlv, mlv};
                k.cl[g2] = h2{clv, clv};
            }
        }
        return k;
    }
    // Part P (0..3) of the dequantization of stage q into LDS buffer buf: eight of this thread's
    // 32 values (Q4_K: low nibbles 0-7, 8-15, then high nibbles 0-7, 8-15; Q6_K: values 8P ..
    // 8P + 7 of its 32, both operand halves).
    template <int P>
    __device__ __forceinline__ void dqPart(const RawW<Q6>& r, const DqC& k, int q, char* bbuf) const {
        char* brow = bbuf + (size_t)drl * kPitch;
        if constexpr (!Q6) {
            constexpr bool hi = P >= 2;
            const uint32_t w0 = (P & 1) ? r.qs.z : r.qs.x, w1 = (P & 1) ? r.qs.w : r.qs.y;
            const h8 v = nib8(w0, w1, hi, k.m[hi], k.c[hi]);
            // stage layout: sub-block 2q at 0..31, 2q + 1 at 32..63; this thread's half at 16 dh
            *reinterpret_cast<h8*>(brow + (hi ? 64 : 0) + 32 * dh + 16 * (P & 1)) = v;
        } else {
            constexpr int g2 = P >> 1, hv = P & 1;
            const int quad = 2 * (q & 1) + dh, nsel = q & 1;
            const uint4 L = r.ql[g2], H = r.qh[g2];
            const uint32_t l0 = hv ? L.z : L.x, l1 = hv ? L.w : L.y, h0 = hv ? H.z : H.x, h1 = hv ? H.w : H.y;
            const uint32_t q0 = ((l0 >> (4 * nsel)) & 0x0F0F0F0Fu) | (((h0 >> (2 * quad)) & 0x03030303u) << 4);
            const uint32_t q1 = ((l1 >> (4 * nsel)) & 0x0F0F0F0Fu) | (((h1 >> (2 * quad)) & 0x03030303u) << 4);
            h8 hiv, lov;
            six8(q0, q1, k.m[g2], k.c[g2], k.ml[g2], k.cl[g2], hiv, lov);
            // this thread's 32 values at 32 dh; sub-block g2 at 16 g2
            *reinterpret_cast<h8*>(brow + 64 * dh + 32 * g2 + 16 * hv) = hiv;
            *reinterpret_cast<h8*>(brow + G::kBB + 64 * dh + 32 * g2 + 16 * hv) = lov;
        }
    }
    __device__ __forceinline__ void dequant(const RawW<Q6>& r, uint4 hd, int q, char* bbuf) const {
        const DqC k = dqPrep(hd, q);
        dqPart<0>(r, k, q, bbuf);
        dqPart<1>(r, k, q, bbuf);
        dqPart<2>(r, k, q, bbuf);
        dqPart<3>(r, k, q, bbuf);
    }
};

// One workgroup's tile: weight rows rowTile * 128 .., columns colTile * 64 CB .., super-blocks
// [sb0, sb1) (y = the partial sum over that range).
template <bool Q6, int CB>
__device__ __forceinline__ void wTile(char* lds, const uint8_t* __restrict__ qw, const _Float16* __restrict__ act,
                                      const _Float16* __restrict__ mins, const float* __restrict__ xdT,
                                      float* __restrict__ y, int rows, int nsb, int ncols, int ncp, int rowTile,
                                      int colTile, int sb0, int sb1) {
    using G = WGeo<Q6, CB>;
    WTile<Q6, CB> T;
    T.tid = threadIdx.x;
    T.lane = T.tid & 63;
    T.wave = T.tid >> 6;
    T.wr = T.wave & 1;
    T.wc = T.wave >> 1;
    T.l32 = T.lane & 31;
    T.h = T.lane >> 5;
    T.qw = qw;
    T.ngroups = (nsb + kGroupSb - 1) / kGroupSb;
    const int rows_stream = ((rows + kTileRows - 1) / kTileRows) * kTileRows;
    const int R0 = rowTile * kWRows, C0 = colTile * G::kCols;
    {
        // thread t: row t % 128, half t / 128 (the eight lanes of one LDS write phase store to
        // eight rows, 144 B apart: distinct banks)
        T.drl = T.tid & (kWRows - 1);
        T.dh = T.tid >> 7;
        const int dr = R0 + T.drl;
        T.drow = dr < rows_stream ? dr : 0;
    }
    const int k = nsb * 256;
    const __amdgpu_buffer_rsrc_t ract = bufRes(act, (uint32_t)ncols * (uint32_t)k * 2u);
    const __amdgpu_buffer_rsrc_t rmin = bufRes(mins, Q6 ? 0u : (uint32_t)ncols * (uint32_t)nsb * 32u);
    const __amdgpu_buffer_rsrc_t rxd = bufRes(xdT, (uint32_t)nsb * (uint32_t)ncp * 4u);

    // this lane's byte offsets (super-block 0, stage 0) of its direct activation loads: LDS chunk
    // g = 64 load + lane holds column g / 9, piece g % 9 (pieces 0-7: 8 halves each; 8 = padding)
    uint32_t aoff[G::kAPerWave];
#pragma unroll
    for (int r = 0; r < G::kAPerWave; ++r) {
        const int ld = min(r * 4 + T.wave, G::kALoads - 1);
        const int g = ld * 64 + T.lane, c = g / 9, pc = g - 9 * c;
        const int cc = C0 + c < ncols ? C0 + c : 0;
        aoff[r] = (uint32_t)cc * (uint32_t)k * 2u + (uint32_t)(pc == 8 ? 0 : pc) * 16u;
    }
    // the activations of stage st = 4 (s - sb0) + q into buffer st & 1
    auto loadA = [&](int s, int q, char* buf) {
#pragma unroll
        for (int r = 0; r < G::kAPerWave; ++r) {
            const int ld = min(r * 4 + T.wave, G::kALoads - 1);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ract, (LdsPtr)(buf + ld * 1024), 16, aoff[r],
                                                     (uint32_t)s * 512u + (uint32_t)q * 128u, 0, 0);
        }
    };
    // the super-block's Q4_K min operands ([col][16] halves) and column scales into region sbuf
    auto loadSb = [&](int s, char* sbuf) {
        if constexpr (!Q6) {
            // kCols * 32 B = (kCols / 32) loads of 1 KB: lane -> column p / 2, half p & 1
#pragma unroll
            for (int r = 0; r < (G::kCols / 32 + 3) / 4; ++r) {
                const int ld = min(r * 4 + T.wave, G::kCols / 32 - 1);
                const int p = ld * 64 + T.lane, c = p >> 1;
                const int cc = C0 + c < ncols ? C0 + c : 0;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rmin, (LdsPtr)(sbuf + ld * 1024), 16,
                                                         (uint32_t)(((cc * nsb + s) * 16 + (p & 1) * 8) * 2), 0, 0, 0);
            }
        }
        // scales: kCols floats (<= 1 KB); lanes past them repeat
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rxd, (LdsPtr)(sbuf + G::kMinsB), 16,
                                                 (uint32_t)((s * ncp + C0 + (T.lane % (G::kCols / 4)) * 4) * 4), 0, 0,
                                                 0);
    };

    // the MFMA rows' headers (d, dmin, mins) per row block
    const int mrow[2] = {R0 + 64 * T.wr + T.l32, R0 + 64 * T.wr + 32 + T.l32};
    const int mrowc[2] = {mrow[0] < rows_stream ? mrow[0] : 0, mrow[1] < rows_stream ? mrow[1] : 0};
    auto loadHdrM = [&](int s, uint4 (&hm)[2]) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            const uint8_t* p = T.piece(mrowc[rb], s);
            if constexpr (!Q6) {
                hm[rb] = *reinterpret_cast<const uint4*>(p);
            } else {
                const int tile = mrowc[rb] >> 4, r = mrowc[rb] & 15, g = s >> 2, kq = s & 3;
                const uint8_t* seg = qw + ((size_t)tile * T.ngroups + g) * kQ6kSeg;
                hm[rb] = make_uint4(*reinterpret_cast<const uint16_t*>(seg + kQ6kSlabs * 1024 + (kq * 16 + r) * 2), 0, 0, 0);
            }
        }
    };

    f16v acc[2][CB], is[2][CB];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[rb][cb][i] = 0.0f;
    const f16v zero = acc[0][0];

    // this lane's fragment offsets within an activation / weight tile
    int aof[CB], bof[2];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) aof[cb] = (T.wc * 32 * CB + cb * 32 + T.l32) * kPitch + T.h * 16;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) bof[rb] = (64 * T.wr + 32 * rb + T.l32) * kPitch + T.h * 16;

    char* const bufB = lds + G::kBOff;
    char* const sbufs = lds + G::kSbOff;
    // Pipeline (stage st = 4 (s - sb0) + q, nst stages): at stage st every wavefront issues, in
    // this order, the raw weights two dequantizations ahead (Q4_K: stage st + 3, a ring of four
    // register sets; Q6_K, at odd stages: the pair of stages (st + 3) / 2, a ring of two), at q == 0
    // the next super-block's headers, min operands and column scales, and the activations of stage
    // st + 3 (a ring of four LDS tiles); then runs stage st's matrix ops with a quarter of stage
    // st + 1's dequantization between them, and after a super-block's last stage its combine. Past
    // the last stage the loads repeat the last one (their data is never read), so every stage
    // issues the same loads and the counted waits are constants.
    constexpr int kNRaw = Q6 ? 4 : 1;                                  // loads of one raw set
    constexpr int kNH = (Q6 ? 1 : (G::kCols / 32 + 3) / 4 + 1) + 3;    // headers, min operands, scales
    constexpr int kNA = G::kAPerWave;
    // loads issued after stage st's activations, at the start of stage st (stages st - 2, st - 1)
    constexpr int kWait0 = 2 * kNA + (Q6 ? 1 : 2) * kNRaw;            // q == 0, 3
    constexpr int kWait12 = kWait0 + kNH;                              // q == 1, 2
    const int nst = 4 * (sb1 - sb0);
    const int npair = 2 * (sb1 - sb0);

    uint4 hdD[2], hm[2][2];  // by super-block parity: the dequant row's header, the MFMA rows' headers
    RawW<Q6> raw[Q6 ? 2 : 4];
    typename WTile<Q6, CB>::DqC dqk;
    // super-block s's scales, min operands and headers into the registers / region of parity par
    auto loadH = [&](int s, int par) {
        loadSb(s, sbufs + par * G::kSb);
        hdD[par] = T.loadHdrD(s);
        loadHdrM(s, hm[par]);
    };
    auto loadAst = [&](int st, char* abuf) {
        st = min(st, nst - 1);
        loadA(sb0 + (st >> 2), st & 3, abuf);
    };
    auto loadRawSt = [&](int st, RawW<Q6>& r) {  // Q4_K: stage st; Q6_K: pair st
        if constexpr (!Q6) {
            st = min(st, nst - 1);
            T.loadRaw(r, sb0 + (st >> 2), st & 3);
        } else {
            st = min(st, npair - 1);
            T.loadRaw(r, sb0 + (st >> 1), st & 1);
        }
    };

    // prologue: super-block sb0's headers and scales, the raw weights of stages 0-2 (Q6_K: pairs
    // 0 and 1), the activations of stages 0-2; stage 0 dequantized now
    loadH(sb0, 0);
    if constexpr (!Q6) {
        loadRawSt(0, raw[0]);
        loadRawSt(1, raw[1]);
        loadRawSt(2, raw[2]);
    } else {
        loadRawSt(0, raw[0]);
        loadRawSt(1, raw[1]);
    }
    __builtin_amdgcn_sched_barrier(0);
    loadAst(0, lds);
    loadAst(1, lds + G::kAB);
    loadAst(2, lds + 2 * G::kAB);
    __builtin_amdgcn_sched_barrier(0);
    T.dequant(raw[0], hdD[0], 0, bufB);

    // The combine of a super-block (parity pc of its headers and scales), one 32 x 32 block at a
    // time (block b: rows 64 wr + 32 (b / CB), columns 32 CB wc + 32 (b % CB)): Q4_K
    // acc += xd (d is - dmin im), the min term im one more matrix op against the staged
    // [64 (B >> 6), B & 63] operands; Q6_K acc += (d xd) is.
    struct CombBlk {
        float d, dmin;
        f16v im;
    };
    auto combPrep = [&](int pc, int b) {
        const int rb = b / CB, cb = b % CB;
        const uint4& hmr = hm[pc][rb];
        CombBlk c;
        c.d = (float)__builtin_bit_cast(_Float16, (unsigned short)(hmr.x & 0xFFFFu));
        if constexpr (!Q6) {
            c.dmin = (float)__builtin_bit_cast(_Float16, (unsigned short)(hmr.x >> 16));
            const int s1w = (int)hmr.z, s2 = (int)hmr.w;
            const int mw0 = s1w & 0x3F3F3F3F, mw1 = ((s2 >> 4) & 0x0F0F0F0F) | ((s1w >> 2) & 0x30303030);
            h8 bm;
#pragma unroll
            for (int e = 0; e < 8; ++e) bm[e] = (_Float16)(float)(((e < 4 ? mw0 : mw1) >> (8 * (e & 3))) & 255);
            const char* sb = sbufs + pc * G::kSb;
            const h8 am = *reinterpret_cast<const h8*>(sb + (T.wc * 32 * CB + cb * 32 + T.l32) * 32 + 16 * T.h);
            c.im = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, zero, 0, 0, 0);
        } else {
            c.dmin = 0.0f;
        }
        return c;
    };
    auto combPart = [&](int pc, int b, int t, const CombBlk& c) {
        const int rb = b / CB, cb = b % CB;
        const char* sb = sbufs + pc * G::kSb;
        // the column scales of elements 4t .. 4t + 3: columns 8t + 4h .. + 3 of the block
        const u32v4 w4 = *reinterpret_cast<const u32v4*>(sb + G::kMinsB + (T.wc * 32 * CB + cb * 32 + t * 8 + T.h * 4) * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // (through a scalar: a bit_cast of the element expression w4[e] itself reads element 0
            // whatever e is)
            const uint32_t wv = w4[e];
            const float xd = __builtin_bit_cast(float, wv);
            const int i = 4 * t + e;
            if constexpr (!Q6) {
                const float t2 = __builtin_fmaf(-c.dmin, c.im[i], c.d * is[rb][cb][i]);
                acc[rb][cb][i] = __builtin_fmaf(xd, t2, acc[rb][cb][i]);
            } else {
                acc[rb][cb][i] = __builtin_fmaf(c.d * xd, is[rb][cb][i], acc[rb][cb][i]);
            }
        }
    };

    auto stage = [&](auto qc, auto oc, int s) {
        constexpr int Q = decltype(qc)::value;
        constexpr int par = decltype(oc)::value ? 1 : 0;  // parity of s - sb0
        const int st = 4 * (s - sb0) + Q;
        const char* abuf = lds + Q * G::kAB;
        const char* bbuf = bufB + (Q & 1) * G::kBS;
        char* nbbuf = bufB + ((Q + 1) & 1) * G::kBS;
        // Stage st's activations (this wavefront's loads) and every LDS write, then everyone's.
        if constexpr (Q == 0) {
            if (s == sb0) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(2 * kNA) : "memory");
            else asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kWait0) : "memory");
        } else if constexpr (Q == 1) {
            if (s == sb0) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kWait12 - kNRaw) : "memory");
            else asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kWait12) : "memory");
        } else if constexpr (Q == 2) {
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kWait12) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kWait0) : "memory");
        }
        // a bare barrier: these waits are the ones this stage needs (__syncthreads' fence would
        // drain every load in flight, the prefetches included)
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (!Q6) loadRawSt(st + 3, raw[(Q + 3) & 3]);
        else if constexpr (Q & 1) loadRawSt(2 * (s - sb0) + (Q >> 1) + 2, raw[(Q >> 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (Q == 0) loadH(min(s + 1, sb1 - 1), par ^ 1);
        __builtin_amdgcn_sched_barrier(0);
        loadAst(st + 3, lds + ((Q + 3) & 3) * G::kAB);
        __builtin_amdgcn_sched_barrier(0);
        // stage st + 1's raw weights and its super-block's header (past the last stage: repeats)
        const RawW<Q6>& rw = Q6 ? raw[((Q + 1) >> 1) & 1] : raw[(Q + 1) & 3];
        dqk = T.dqPrep(Q == 3 ? hdD[par ^ 1] : hdD[par], (Q + 1) & 3);
        // K-steps t = 0..3 of 16 values; the fragments of step t + 1 are read from LDS while step t
        // runs its matrix ops (one wavefront per SIMD: nothing else hides the LDS latency)
        struct Frag {
            h8 a[CB], b[2], b2[2];
        };
        auto readFrag = [&](int t, Frag& f) {
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) f.a[cb] = *reinterpret_cast<const h8*>(abuf + aof[cb] + 32 * t);
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                f.b[rb] = *reinterpret_cast<const h8*>(bbuf + bof[rb] + 32 * t);
                if constexpr (Q6) f.b2[rb] = *reinterpret_cast<const h8*>(bbuf + bof[rb] + G::kBB + 32 * t);
            }
        };
        Frag fr[2];
        readFrag(0, fr[0]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if (t < 3) readFrag(t + 1, fr[(t + 1) & 1]);
            const Frag& f = fr[t & 1];
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    is[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[cb], f.b[rb], (Q == 0 && t == 0) ? zero : is[rb][cb], 0, 0, 0);
                    if constexpr (Q6) is[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[cb], f.b2[rb], is[rb][cb], 0, 0, 0);
                }
            // a quarter of stage st + 1's dequantization
            if (t == 0) T.template dqPart<0>(rw, dqk, (Q + 1) & 3, nbbuf);
            if (t == 1) T.template dqPart<1>(rw, dqk, (Q + 1) & 3, nbbuf);
            if (t == 2) T.template dqPart<2>(rw, dqk, (Q + 1) & 3, nbbuf);
            if (t == 3) T.template dqPart<3>(rw, dqk, (Q + 1) & 3, nbbuf);
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (Q == 3) {  // the super-block's combine
#pragma unroll
            for (int b = 0; b < 2 * CB; ++b) {
                const CombBlk c = combPrep(par, b);
#pragma unroll
                for (int t = 0; t < 4; ++t) combPart(par, b, t, c);
            }
        }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using Ev = std::integral_constant<bool, false>;
    using Od = std::integral_constant<bool, true>;
    for (int s = sb0; s < sb1; s += 2) {
        stage(I0{}, Ev{}, s);
        stage(I1{}, Ev{}, s);
        stage(I2{}, Ev{}, s);
        stage(I3{}, Ev{}, s);
        if (s + 1 < sb1) {
            stage(I0{}, Od{}, s + 1);
            stage(I1{}, Od{}, s + 1);
            stage(I2{}, Od{}, s + 1);
            stage(I3{}, Od{}, s + 1);
        }
    }
    // every wavefront's direct loads have landed before the workgroup ends (the repeated loads
    // past the last stage write LDS the next workgroup on this CU may own)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        if (mrow[rb] >= rows) continue;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int c = C0 + T.wc * 32 * CB + cb * 32 + (i >> 2) * 8 + T.h * 4 + (i & 3);
                if (c < ncols) y[(size_t)c * rows + mrow[rb]] = acc[rb][cb][i];
            }
    }
}

template <int CB>
__global__ __launch_bounds__(256, 1) void matmul_kq_mfma_w_kernel(MfmaGroup g, const _Float16* __restrict__ act,
                                                                  const _Float16* __restrict__ mins,
                                                                  const float* __restrict__ xdT, int nsb, int ncols,
                                                                  int ncp) {
    extern __shared__ int4 lds4[];
    char* lds = reinterpret_cast<char*>(lds4);
    const int bx = blockIdx.x;
    const int pi = (g.nparts > 2 && bx >= g.p[2].tile0) ? 2 : (g.nparts > 1 && bx >= g.p[1].tile0) ? 1 : 0;
    const MfmaPart& p = g.p[pi];
    const int z = blockIdx.z, sb0 = z * nsb / g.ks, sb1 = (z + 1) * nsb / g.ks;
    if (p.q6)
        wTile<true, CB>(lds, p.qw, act, mins, xdT, p.y[z], p.rows, nsb, ncols, ncp, bx - p.tile0, blockIdx.y, sb0, sb1);
    else
        wTile<false, CB>(lds, p.qw, act, mins, xdT, p.y[z], p.rows, nsb, ncols, ncp, bx - p.tile0, blockIdx.y, sb0, sb1);
}

template <int CB>
int launchW(const MfmaGroup& g, int tiles, const _Float16* act, const _Float16* mins, const float* xdT, int nsb,
            int ncols, int ncp, hipStream_t s) {
    constexpr int lds = WGeo<true, CB>::kLds > WGeo<false, CB>::kLds ? WGeo<true, CB>::kLds : WGeo<false, CB>::kLds;
    static const int attr = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(matmul_kq_mfma_w_kernel<CB>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != 0) return fromHip(attr, "matmul (MFMA, wide tiles): LDS size");
    const dim3 grid(tiles, (ncols + 64 * CB - 1) / (64 * CB), g.ks);
    hipLaunchKernelGGL(matmul_kq_mfma_w_kernel<CB>, grid, dim3(256), lds, s, g, act, mins, xdT, nsb, ncols, ncp);
    return fromHip(hipGetLastError(), "matmul_q4k/q6k_q8k (MFMA, wide tiles)");
}

}  // namespace

int launchMfmaW(const MfmaGroup& g, int tiles, const void* act, const void* mins, const float* xdT, int nsb, int ncols,
                int ncp, hipStream_t s) {
    return launchW<2>(g, tiles, static_cast<const _Float16*>(act), static_cast<const _Float16*>(mins), xdT, nsb, ncols,
                      ncp, s);
}

}  // namespace kcamd
