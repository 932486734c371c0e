// kmatmul_mfmaws.hip -- the prefill matmul with producer and consumer wavefronts (gfx950): Y = W X
// for Q4_K / Q6_K weights and per-256 8-bit activations, the arithmetic of kmatmul_mfma.hip (exact
// integer sums per super-block on v_mfma_f32_32x32x16_f16, the reference's combine per super-block;
// reference kernels/llm/matmul_q4k_q8kx8.cu, matmul_q6k_q8kx8.cu, mirror
// llm/llm_reference.cpp:529-596).
//
// A wavefront stalls at each vector-memory instruction until the CU's memory unit takes it (about
// 20 cycles per instruction), and a wavefront that stalls issues neither matrix ops nor the VALU
// dequantization that feeds them. So the loads get wavefronts of their own: a workgroup of 12
// wavefronts owns 256 weight rows x 64 activation columns,
//   - 8 consumer wavefronts (two per SIMD), each 32 weight rows x 64 columns as two 32 x 32 blocks:
//     they only read LDS, dequantize and issue matrix ops (the K-step pipeline of
//     kmatmul_mfma.hip's hTile, with the weights read from LDS instead of memory);
//   - 4 producer wavefronts (one per SIMD) issue every load of a stage, straight into LDS with
//     buffer-to-LDS loads: the activation tile (fp16, 16 x, as act_to_f16 or the quantizers write
//     it), the column scales, and the weights of the 256 rows; for Q4_K also the min operands.
// Two LDS stages: while the consumers compute one, the producers fill the other and wait for their
// loads; one barrier per stage hands it over. A Q4_K stage is a super-block (72 KiB: each 16-row
// tile's header slab and eight qs slabs), a Q6_K stage half of one (47 KiB, below). One launch may
// mix Q4_K and Q6_K matrices (q / k / v with a Q6_K v); each workgroup takes its matrix's path.
// Slot mode (Q4_K callers that hand over int8 slots, kcLaunchKernel's matmul_q4k_q8k*): the
// producers read the per-256 slots themselves, convert them to the same fp16 operands in registers
// and write them to the stage, in place of a conversion launch before the matmul.
#include <hip/hip_runtime.h>

#include <cstdint>

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

constexpr int kCons = 8;                       // consumer wavefronts
constexpr int kProd = 4;                       // producer wavefronts
constexpr int kThreads = 64 * (kCons + kProd);
constexpr int kRows = 32 * kCons;              // weight rows per workgroup
constexpr int kCols = 64;                      // activation columns per workgroup
constexpr int kColB = 528;                     // LDS bytes per column: 32 chunks of 16 B + 1 pad chunk
constexpr int kActLoads = kCols * 33 / 64;     // 1 KiB direct loads of the activation tile
constexpr int kMinOff = kActLoads * 1024;      // Q4_K min operands: 32 B per column
constexpr int kXdOff = kMinOff + kCols * 32;   // column scales (one 1 KiB load, 256 B used)
constexpr int kWOff = kXdOff + 1024;           // weights: [tile][slab][16 rows x 16 B]
constexpr int kTiles = kRows / kTileRows;      // 16-row tiles per workgroup
constexpr int kWLoads = kTiles * kQ4kSlabs / 4;  // each load: four (tile, slab) chunks of 256 B
constexpr int kStage = kWOff + kTiles * kQ4kSlabs * 256;
constexpr int kLdsBytes = 2 * kStage;
constexpr int kLoads = kActLoads + 2 + 1 + kWLoads;  // per super-block
constexpr int kPerProd = kLoads / kProd;
static_assert(kLoads % kProd == 0 && kWLoads * 4 == kTiles * kQ4kSlabs, "load split");
static_assert(kLdsBytes <= 160 * 1024, "LDS");

__device__ __forceinline__ h2 bits_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t h2_bits(h2 v) { return __builtin_bit_cast(uint32_t, v); }
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Four int8 activations -> four fp16 values 16 x (exact): (x ^ 0x80) | 0x6400 is 1024 + x + 128,
// and (1152 + x) * 16 - 18432 = 16 x in one fused multiply-add (act_to_f16's conversion).
__device__ __forceinline__ uint2 i8x4_to_h4x16(uint32_t w) {
    const uint32_t u = w ^ 0x80808080u;
    const h2 m = {(_Float16)16.0f, (_Float16)16.0f}, c = {(_Float16)(-18432.0f), (_Float16)(-18432.0f)};
    const h2 lo = __builtin_elementwise_fma(bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)), m, c);
    const h2 hi = __builtin_elementwise_fma(bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)), m, c);
    return make_uint2(h2_bits(lo), h2_bits(hi));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t bufRes(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Eight 4-bit weights (nibble hiNib of 8 bytes) times a sub-block scale, as exact fp16 (the
// operand of kmatmul_mfma.hip's dequant8s: (1024 + q) m2 + s2).
__device__ __forceinline__ h8 nib8(uint2 q, bool hiNib, h2 m2, h2 s2) {
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

struct WsArgs {
    const _Float16* act;  // fp16 mode: act_to_f16's (or a quantizer's) operands
    const _Float16* mins;
    const float* xdT;
    const int* xq;        // slot mode: the per-256 slots (nsb * 85 ints per column)
    int nsb, ncols, ncp;
};

constexpr int kWPerProd = kWLoads / kProd;  // slot mode: each producer's weight loads
static_assert(kWLoads % kProd == 0, "weight load split");

// Q6_K: a stage holds half a super-block (128 values): per 16-row tile the row pieces ql 4n ..
// 4n + 3, qh 8 + 2n, 9 + 2n and the scales (piece 12) of half n, the activation half (16 chunks of
// 16 B per column + 1 pad chunk), the tiles' d values and the column scales. Two stages of 47 KiB;
// each holds the same matrix-op work as a Q4_K stage (two ops per K-step, Q6_K's split scale).
constexpr int kQ6Pieces = 7;
constexpr int kQ6ColB = 272;                              // LDS bytes per column and half
constexpr int kQ6ActLoads = kCols * 17 / 64;              // 1 KiB direct loads of the activation half
constexpr int kQ6WOff = kQ6ActLoads * 1024;               // weights: [tile][piece][16 rows x 16 B]
constexpr int kQ6WLoads = kTiles * kQ6Pieces / 4;         // each load: four (tile, piece) chunks of 256 B
constexpr int kQ6DOff = kQ6WOff + kQ6WLoads * 1024;       // d: [tile][16 rows] fp16 (512 B used)
constexpr int kQ6XdOff = kQ6DOff + 1024;                  // column scales (256 B used)
constexpr int kQ6Stage = kQ6XdOff + 1024;
constexpr int kQ6Loads = kQ6ActLoads + kQ6WLoads + 2;     // per half super-block
constexpr int kQ6PerProd = (kQ6Loads + kProd - 1) / kProd;
static_assert(kCols * 17 % 64 == 0 && kTiles * kQ6Pieces % 4 == 0, "Q6_K load split");
static_assert(2 * kQ6Stage <= kLdsBytes, "Q6_K LDS");

// Slot mode: this producer lane's part of super-block s. Lane L = 64 p + lane of the 256 takes
// column L / 4's activation words 16 (L % 4) .. +15 (64 int8); producer 0's lanes also the column
// scale of column col0 + lane, producer 1's the four words of its min bytes. Columns past ncols read
// column 0 (never stored). The launcher keeps nsb % 4 == 0: every read is 16-byte aligned.
struct SlotRegs {
    i32x4 a[4];
    i32x4 m;
    float d;
};
__device__ __forceinline__ void loadSlots(SlotRegs& r, const int* __restrict__ xq, int p, int lane, int col0,
                                          int ncols, int nsb, int s) {
    const int L = p * 64 + lane, c = L >> 2, qq = L & 3;
    const int cc = col0 + c < ncols ? col0 + c : 0;
    const i32x4* src = reinterpret_cast<const i32x4*>(xq + (size_t)cc * nsb * 85 + s * 64 + qq * 16);
#pragma unroll
    for (int u = 0; u < 4; ++u) r.a[u] = src[u];
    const int cl = col0 + lane < ncols ? col0 + lane : 0;
    const int* colp = xq + (size_t)cl * nsb * 85;
    if (p == 0) r.d = reinterpret_cast<const float*>(colp + nsb * 64)[s];
    if (p == 1) r.m = *reinterpret_cast<const i32x4*>(colp + nsb * 81 + s * 4);
}
// ... converted and written to the stage: the activation chunks, the scales, the min operands
// [64 (B_j >> 6) for j < 8 | B_j & 63 for j < 8] (the reference's byte split of the sub-block sums).
__device__ __forceinline__ void writeSlots(char* buf, const SlotRegs& r, int p, int lane) {
    const int L = p * 64 + lane, c = L >> 2, qq = L & 3;
    char* dst = buf + c * kColB + qq * 128;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const i32x4 w = r.a[u];
        const int w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3];  // (scalar copies before use)
        const uint2 h0 = i8x4_to_h4x16((uint32_t)w0), h1 = i8x4_to_h4x16((uint32_t)w1);
        const uint2 h2v = i8x4_to_h4x16((uint32_t)w2), h3 = i8x4_to_h4x16((uint32_t)w3);
        *reinterpret_cast<uint4*>(dst + u * 32) = make_uint4(h0.x, h0.y, h1.x, h1.y);
        *reinterpret_cast<uint4*>(dst + u * 32 + 16) = make_uint4(h2v.x, h2v.y, h3.x, h3.y);
    }
    if (p == 0) reinterpret_cast<float*>(buf + kXdOff)[lane] = r.d;
    if (p == 1) {
        const int m0 = r.m[0], m1 = r.m[1], m2 = r.m[2], m3 = r.m[3];
        h8 lo, hi;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int hb = ((j < 4 ? m0 : m1) << (24 - 8 * (j & 3))) >> 24;
            const int lb = ((j < 4 ? m2 : m3) >> (8 * (j & 3))) & 255;
            lo[j] = (_Float16)(float)(64 * hb);
            hi[j] = (_Float16)(float)lb;
        }
        *reinterpret_cast<h8*>(buf + kMinOff + lane * 32) = lo;
        *reinterpret_cast<h8*>(buf + kMinOff + lane * 32 + 16) = hi;
    }
}

// The producers' loads of super-block s into stage buf. Load L = kProd r + p of the kLoads:
// activation chunks, then the min operands, the column scales, the weight chunks; voff[r] is this
// lane's byte offset of load r at super-block 0 of the array it reads (the super-block's part is
// the uniform soffset).
__device__ __forceinline__ void produce(char* buf, int p, int lane, const uint32_t (&voff)[kPerProd],
                                        __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rm,
                                        __amdgpu_buffer_rsrc_t rx, __amdgpu_buffer_rsrc_t rw, int s, int ncp) {
    (void)lane;
#pragma unroll
    for (int r = 0; r < kPerProd; ++r) {
        const int L = kProd * r + p;
        if (L < kActLoads) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (LdsPtr)(buf + L * 1024), 16, voff[r], (uint32_t)s * 512u, 0, 0);
        } else if (L < kActLoads + 2) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (LdsPtr)(buf + kMinOff + (L - kActLoads) * 1024), 16, voff[r],
                                                     (uint32_t)s * 32u, 0, 0);
        } else if (L == kActLoads + 2) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (LdsPtr)(buf + kXdOff), 16, voff[r], (uint32_t)(s * ncp) * 4u, 0,
                                                     0);
        } else {
            const int wl = L - (kActLoads + 3);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (LdsPtr)(buf + kWOff + wl * 1024), 16, voff[r],
                                                     (uint32_t)((s >> 2) * kQ4kSeg + (s & 3) * 256), 0, 0);
        }
    }
}

// One workgroup: rows rowTile * 256 .., columns colTile * 64 .., super-blocks [sb0, sb1).
template <bool SLOTS>
__device__ __forceinline__ void wsTile(char* lbase, const uint8_t* __restrict__ qw, const WsArgs& a,
                                       float* __restrict__ y, int rows, int rowTile, int colTile, int sb0, int sb1) {
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nsb = a.nsb, ncols = a.ncols, k = nsb * 256;
    const int col0 = colTile * kCols;
    const int ngroups = (nsb + kGroupSb - 1) / kGroupSb;
    const int tiles_stream = (rows + kTileRows - 1) / kTileRows;
    const bool prod = wave >= kCons;

    if (SLOTS && prod) {
        const int p = wave - kCons;
        const __amdgpu_buffer_rsrc_t rw = bufRes(qw, (uint32_t)tiles_stream * (uint32_t)ngroups * (uint32_t)kQ4kSeg);
        uint32_t voff[kWPerProd];
#pragma unroll
        for (int r = 0; r < kWPerProd; ++r) {  // tiles past the stream read tile 0 (their rows are never stored)
            const int q = (kProd * r + p) * 4 + (lane >> 4), t = q / kQ4kSlabs, j = q - kQ4kSlabs * t;
            int tg = rowTile * kTiles + t;
            if (tg >= tiles_stream) tg = 0;
            voff[r] = (uint32_t)tg * (uint32_t)ngroups * (uint32_t)kQ4kSeg + (uint32_t)(j * 1024 + (lane & 15) * 16);
        }
        auto weights = [&](char* buf, int s) {
#pragma unroll
            for (int r = 0; r < kWPerProd; ++r)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (LdsPtr)(buf + kWOff + (kProd * r + p) * 1024), 16, voff[r],
                                                         (uint32_t)((s >> 2) * kQ4kSeg + (s & 3) * 256), 0, 0);
        };
        SlotRegs sr;
        weights(lbase, sb0);
        loadSlots(sr, a.xq, p, lane, col0, ncols, nsb, sb0);
        writeSlots(lbase, sr, p, lane);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        for (int s = sb0; s < sb1; ++s) {
            const int b = (s - sb0) & 1;
            if (s + 1 < sb1) {
                weights(lbase + (b ^ 1) * kStage, s + 1);
                loadSlots(sr, a.xq, p, lane, col0, ncols, nsb, s + 1);
                writeSlots(lbase + (b ^ 1) * kStage, sr, p, lane);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        }
        return;
    }
    if (!SLOTS && prod) {
        const int p = wave - kCons;
        const __amdgpu_buffer_rsrc_t ra = bufRes(a.act, (uint32_t)ncols * (uint32_t)k * 2u);
        const __amdgpu_buffer_rsrc_t rm = bufRes(a.mins, (uint32_t)ncols * (uint32_t)nsb * 32u);
        const __amdgpu_buffer_rsrc_t rx = bufRes(a.xdT, (uint32_t)nsb * (uint32_t)a.ncp * 4u);
        const __amdgpu_buffer_rsrc_t rw = bufRes(qw, (uint32_t)tiles_stream * (uint32_t)ngroups * (uint32_t)kQ4kSeg);
        uint32_t voff[kPerProd];
#pragma unroll
        for (int r = 0; r < kPerProd; ++r) {
            const int L = kProd * r + p;
            if (L < kActLoads) {  // columns past ncols read column 0 (never stored)
                const int slot = L * 64 + lane, c = slot / 33, kc = slot - 33 * c;
                const int cc = col0 + c < ncols ? col0 + c : 0;
                voff[r] = (uint32_t)cc * (uint32_t)k * 2u + (uint32_t)(kc == 32 ? 0 : kc) * 16u;
            } else if (L < kActLoads + 2) {
                const int p2 = (L - kActLoads) * 64 + lane, c = p2 >> 1;
                const int cc = col0 + c < ncols ? col0 + c : 0;
                voff[r] = (uint32_t)((cc * nsb * 16 + (p2 & 1) * 8) * 2);
            } else if (L == kActLoads + 2) {
                voff[r] = (uint32_t)((col0 + (lane & 15) * 4) * 4);
            } else {  // tiles past the stream read tile 0 (their rows are never stored)
                const int q = (L - (kActLoads + 3)) * 4 + (lane >> 4), t = q / kQ4kSlabs, j = q - kQ4kSlabs * t;
                int tg = rowTile * kTiles + t;
                if (tg >= tiles_stream) tg = 0;
                voff[r] = (uint32_t)tg * (uint32_t)ngroups * (uint32_t)kQ4kSeg + (uint32_t)(j * 1024 + (lane & 15) * 16);
            }
        }
        produce(lbase, p, lane, voff, ra, rm, rx, rw, sb0, a.ncp);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        for (int s = sb0; s < sb1; ++s) {
            const int b = (s - sb0) & 1;
            if (s + 1 < sb1) produce(lbase + (b ^ 1) * kStage, p, lane, voff, ra, rm, rx, rw, s + 1, a.ncp);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        }
        return;
    }

    // consumer wavefront: rows rowTile * 256 + wave * 32 + lane % 32, lane half h
    const int h = lane >> 5, l32 = lane & 31;
    const int row = rowTile * kRows + wave * 32 + l32;
    const int woff = kWOff + (wave * 2 + (l32 >> 4)) * kQ4kSlabs * 256 + (l32 & 15) * 16;
    int aoff[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) aoff[cb] = (cb * 32 + l32) * kColB + h * 32;
    f16v acc[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[cb][i] = 0.0f;
    const f16v zero = acc[0];
    __syncthreads();  // stage 0 loaded
    for (int s = sb0; s < sb1; ++s) {
        const char* buf = lbase + ((s - sb0) & 1) * kStage;
        // the row's super-block: header (d, dmin, 12 scale / min bytes) and the qs chunks of this half
        const uint4 hdr = *reinterpret_cast<const uint4*>(buf + woff);
        uint4 q16[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) q16[j] = *reinterpret_cast<const uint4*>(buf + woff + (1 + 2 * j + h) * 256);
        h8 av[2], an[2];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) av[cb] = *reinterpret_cast<const h8*>(buf + aoff[cb]);
        const float d = (float)__builtin_bit_cast(_Float16, (unsigned short)(hdr.x & 0xFFFFu));
        const float dmin = (float)__builtin_bit_cast(_Float16, (unsigned short)(hdr.x >> 16));
        const int s0 = (int)hdr.y, s1 = (int)hdr.z, s2 = (int)hdr.w;
        const int scw[2] = {s0 & 0x3F3F3F3F, (s2 & 0x0F0F0F0F) | ((s0 >> 2) & 0x30303030)};
        const int mw[2] = {s1 & 0x3F3F3F3F, ((s2 >> 4) & 0x0F0F0F0F) | ((s1 >> 2) & 0x30303030)};
        h2 m2[8], c2[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // sc q / 16 (the activations are 16 x): (1024 + q) sc / 16 - 64 sc for a low nibble,
            // (1024 + 16 q) sc / 256 - 4 sc for a high one; exact (sc / 256 >= 2^-8, q sc <= 945).
            // sc splat as {1024 + sc, 1024 + sc} by a byte permute, then m = (1024 + sc) f - 1024 f
            // = sc f in one fused op (both products exact) and c = -1024 m (-64 sc, -4 sc)
            const int b = j & 3;
            const h2 t = bits_h2(__builtin_amdgcn_perm(0x64646464u, (uint32_t)scw[j >> 2], 0x04000400u | (b << 16) | b));
            const _Float16 f = (j & 1) ? (_Float16)0.00390625f : (_Float16)0.0625f;
            m2[j] = __builtin_elementwise_fma(t, h2{f, f}, h2{(_Float16)-1024.0f * f, (_Float16)-1024.0f * f});
            c2[j] = m2[j] * h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
        }
        // K-step t covers, in lane half h, k = 64 (t >> 2) + 32 ((t >> 1) & 1) + 16 h + 8 (t & 1):
        // qs bytes 32 (t >> 2) + 16 h + 8 (t & 1) (chunk t >> 2, nibble (t >> 1) & 1), activation
        // chunk at byte 64 (t >> 1) + 32 h + 16 (t & 1) of the column; step t + 1's operands are
        // read and dequantized while step t runs its matrix ops
        auto bytes = [&](int t) {
            const uint4 q = q16[t >> 2];
            return (t & 1) ? make_uint2(q.z, q.w) : make_uint2(q.x, q.y);
        };
        f16v is[2];
        h8 bq = nib8(bytes(0), false, m2[0], c2[0]), bn;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            if (t + 1 < 16) {
                const int tn = t + 1, toff = 64 * (tn >> 1) + 16 * (tn & 1), j = tn >> 1;
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) an[cb] = *reinterpret_cast<const h8*>(buf + aoff[cb] + toff);
                bn = nib8(bytes(tn), j & 1, m2[j], c2[j]);
            }
            // (scheduling fences: the next step's reads and dequantization stay ahead of this
            // step's matrix ops instead of being sunk to just before their use)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
                is[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[cb], bq, t == 0 ? zero : is[cb], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (t + 1 < 16) {
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) av[cb] = an[cb];
                bq = bn;
            }
        }
        // the min term (one matrix op per block against [64 (B >> 6) | B & 63]) and the combine
        h8 bm;  // the eight min bytes as fp16: {1024 + m, 1024 + m'} by byte permutes, less 1024
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
            const uint32_t w = (uint32_t)mw[e2 >> 1];
            const h2 t = bits_h2(__builtin_amdgcn_perm(0x64646464u, w, (e2 & 1) ? 0x04030402u : 0x04010400u)) -
                         h2{(_Float16)1024.0f, (_Float16)1024.0f};
            bm[2 * e2] = t[0];
            bm[2 * e2 + 1] = t[1];
        }
        const _Float16* xm = reinterpret_cast<const _Float16*>(buf + kMinOff);
        const char* xdl = buf + kXdOff;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const h8 am = *reinterpret_cast<const h8*>(xm + (cb * 32 + l32) * 16 + 8 * h);
            const f16v im = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, zero, 0, 0, 0);
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                // (each element copied to a scalar before its bit cast: a bit cast of the vector
                // element itself compiles to element 0 for all four)
                const u32v4 xdw = *reinterpret_cast<const u32v4*>(xdl + (cb * 32 + q4 * 8 + h * 4) * 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = 4 * q4 + e;
                    const uint32_t wv = xdw[e];
                    const float t2 = __builtin_fmaf(-dmin, im[i], d * is[cb][i]);
                    acc[cb][i] = __builtin_fmaf(__builtin_bit_cast(float, wv), t2, acc[cb][i]);
                }
            }
        }
        __syncthreads();  // stage read: the producers may refill it; the next stage is loaded
    }
    if (row < rows) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int c = col0 + cb * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
                if (c < ncols) y[(size_t)c * rows + row] = acc[cb][i];
            }
    }
}

// Q6_K K-step t (0..7) of a half super-block n for activations 16 x: in lane half h the 8 values
// k = 128 n + 32 quad + 16 h + 8 p (quad = t >> 1, p = t & 1): ql bytes 64 n + 32 (quad & 1) + 16 h
// + 8 p (nibble quad >> 1; ql[a] holds bytes 64 n + 32 a + 16 h ..), qh bytes 32 n + 16 h + 8 p
// (bits 2 quad), the int8 scale of sub-block 8 n + 2 quad + h (byte 2 (quad & 1) + h of word
// quad >> 1 of sw, the half's eight scales) split as sc = 16 sh + sl: b1 = sh (q - 32) and
// b2 = sl (q - 32) / 16, exact fp16 values (kmatmul_mfma.hip's Q6_K operands, in its K-step order).
__device__ __forceinline__ void dq6(const uint4 (&ql)[2], uint4 qh, uint2 sw, int t, int h, h8& b1, h8& b2) {
    const int quad = t >> 1, p = t & 1;
    const uint4 L = ql[quad & 1];
    const uint32_t lw[2] = {p ? L.z : L.x, p ? L.w : L.y}, hw[2] = {p ? qh.z : qh.x, p ? qh.w : qh.y};
    const int w = (quad >> 1) ? (int)sw.y : (int)sw.x;
    const int bi = 2 * (quad & 1) + h;
    const int sh = (w << (24 - 8 * bi)) >> 28, sl = (w >> (8 * bi)) & 15;
    const _Float16 fh = (_Float16)(short)sh, fl = (_Float16)(short)sl;
    const h2 mh = {fh, fh}, ml = {fl * (_Float16)0.0625f, fl * (_Float16)0.0625f};
    const h2 ch = {fh * (_Float16)(-1056.0f), fh * (_Float16)(-1056.0f)};
    const h2 cl = {fl * (_Float16)(-66.0f), fl * (_Float16)(-66.0f)};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        // q (0..63) per byte, then 1024 + q as fp16 (high byte 0x64)
        const uint32_t q = ((lw[i] >> (4 * (quad >> 1))) & 0x0F0F0F0Fu) | (((hw[i] >> (2 * quad)) & 0x03030303u) << 4);
        const h2 x0 = bits_h2(__builtin_amdgcn_perm(0x64646464u, q, 0x04010400u));
        const h2 x1 = bits_h2(__builtin_amdgcn_perm(0x64646464u, q, 0x04030402u));
        const h2 a1 = __builtin_elementwise_fma(x0, mh, ch), c1 = __builtin_elementwise_fma(x1, mh, ch);
        const h2 a2 = __builtin_elementwise_fma(x0, ml, cl), c2 = __builtin_elementwise_fma(x1, ml, cl);
        b1[4 * i + 0] = a1[0];
        b1[4 * i + 1] = a1[1];
        b1[4 * i + 2] = c1[0];
        b1[4 * i + 3] = c1[1];
        b2[4 * i + 0] = a2[0];
        b2[4 * i + 1] = a2[1];
        b2[4 * i + 2] = c2[0];
        b2[4 * i + 3] = c2[1];
    }
}

// One Q6_K workgroup: rows rowTile * 256 .., columns colTile * 64 .., super-blocks [sb0, sb1), in
// stages of half a super-block (stage 2 (s - sb0) + n in buffer n), fp16 activations as act_to_f16
// or the quantizers write them. The consumers run kmatmul_mfma.hip's Q6_K K-steps in its order
// (bit-identical sums) and combine once per super-block: acc += (d xd) is.
__device__ __forceinline__ void wsTileQ6(char* lbase, const uint8_t* __restrict__ qw, const WsArgs& a,
                                         float* __restrict__ y, int rows, int rowTile, int colTile, int sb0, int sb1) {
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nsb = a.nsb, ncols = a.ncols, k = nsb * 256;
    const int col0 = colTile * kCols;
    const int ngroups = (nsb + kGroupSb - 1) / kGroupSb;
    const int tiles_stream = (rows + kTileRows - 1) / kTileRows;
    const int nst = 2 * (sb1 - sb0);

    if (wave >= kCons) {
        const int p = wave - kCons;
        const __amdgpu_buffer_rsrc_t ra = bufRes(a.act, (uint32_t)ncols * (uint32_t)k * 2u);
        const __amdgpu_buffer_rsrc_t rx = bufRes(a.xdT, (uint32_t)nsb * (uint32_t)a.ncp * 4u);
        const __amdgpu_buffer_rsrc_t rw = bufRes(qw, (uint32_t)tiles_stream * (uint32_t)ngroups * (uint32_t)kQ6kSeg);
        // this lane's byte offset of each of its loads at super-block 0, half 0; a weight piece of
        // half 1 lies dn further (ql pieces 4 on, qh pieces 2 on, the scales the same)
        uint32_t voff[kQ6PerProd], dn[kQ6PerProd];
#pragma unroll
        for (int r = 0; r < kQ6PerProd; ++r) {
            const int L = kProd * r + p;
            dn[r] = 0;
            if (L < kQ6ActLoads) {  // columns past ncols read column 0 (never stored)
                const int slot = L * 64 + lane, c = slot / 17, kc = slot - 17 * c;
                const int cc = col0 + c < ncols ? col0 + c : 0;
                voff[r] = (uint32_t)cc * (uint32_t)k * 2u + (uint32_t)(kc == 16 ? 0 : kc) * 16u;
            } else if (L < kQ6ActLoads + kQ6WLoads) {  // tiles past the stream read tile 0
                const int q = (L - kQ6ActLoads) * 4 + (lane >> 4), t = q / kQ6Pieces, jj = q - kQ6Pieces * t;
                int tg = rowTile * kTiles + t;
                if (tg >= tiles_stream) tg = 0;
                const int piece = jj < 4 ? jj : (jj < 6 ? 4 + jj : 12);
                dn[r] = jj < 4 ? 4096u : (jj < 6 ? 2048u : 0u);
                voff[r] = (uint32_t)tg * (uint32_t)ngroups * (uint32_t)kQ6kSeg + (uint32_t)(piece * 1024 + (lane & 15) * 16);
            } else if (L == kQ6ActLoads + kQ6WLoads) {  // d: lane (tile, 8-row half); lanes 32.. repeat
                int tg = rowTile * kTiles + ((lane >> 1) & 15);
                if (tg >= tiles_stream) tg = 0;
                voff[r] = (uint32_t)tg * (uint32_t)ngroups * (uint32_t)kQ6kSeg + (uint32_t)(kQ6kSlabs * 1024 + (lane & 1) * 16);
            } else {  // the column scales
                voff[r] = (uint32_t)((col0 + (lane & 15) * 4) * 4);
            }
        }
        auto produce = [&](char* buf, int st) {
            const int s = sb0 + (st >> 1), n = st & 1;
            const uint32_t sw = (uint32_t)((s >> 2) * kQ6kSeg);
#pragma unroll
            for (int r = 0; r < kQ6PerProd; ++r) {
                const int L = kProd * r + p;
                if (L < kQ6ActLoads)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (LdsPtr)(buf + L * 1024), 16, voff[r],
                                                             (uint32_t)(s * 512 + n * 256), 0, 0);
                else if (L < kQ6ActLoads + kQ6WLoads)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (LdsPtr)(buf + kQ6WOff + (L - kQ6ActLoads) * 1024), 16,
                                                             voff[r] + (n ? dn[r] : 0u), sw + (uint32_t)((s & 3) * 256),
                                                             0, 0);
                else if (L == kQ6ActLoads + kQ6WLoads)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (LdsPtr)(buf + kQ6DOff), 16, voff[r],
                                                             sw + (uint32_t)((s & 3) * 32), 0, 0);
                else if (L < kQ6Loads)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (LdsPtr)(buf + kQ6XdOff), 16, voff[r],
                                                             (uint32_t)(s * a.ncp) * 4u, 0, 0);
            }
        };
        produce(lbase, 0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        for (int st = 0; st < nst; ++st) {
            if (st + 1 < nst) produce(lbase + ((st + 1) & 1) * kQ6Stage, st + 1);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        }
        return;
    }

    // consumer wavefront: rows rowTile * 256 + wave * 32 + lane % 32, lane half h
    const int h = lane >> 5, l32 = lane & 31;
    const int row = rowTile * kRows + wave * 32 + l32;
    const int t16 = wave * 2 + (l32 >> 4);
    const int woff = kQ6WOff + t16 * kQ6Pieces * 256 + (l32 & 15) * 16;
    const int doff = kQ6DOff + t16 * 32 + (l32 & 15) * 2;
    int aoff[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) aoff[cb] = (cb * 32 + l32) * kQ6ColB + h * 32;
    f16v acc[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[cb][i] = 0.0f;
    const f16v zero = acc[0];
    f16v is[2];
    __syncthreads();  // stage 0 loaded
    for (int s = sb0; s < sb1; ++s) {
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            const char* buf = lbase + n * kQ6Stage;
            uint4 ql[2];
#pragma unroll
            for (int a2 = 0; a2 < 2; ++a2) ql[a2] = *reinterpret_cast<const uint4*>(buf + woff + (2 * a2 + h) * 256);
            const uint4 qh = *reinterpret_cast<const uint4*>(buf + woff + (4 + h) * 256);
            const uint2 sw = *reinterpret_cast<const uint2*>(buf + woff + 6 * 256 + 8 * n);
            h8 av[2], an[2];
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) av[cb] = *reinterpret_cast<const h8*>(buf + aoff[cb]);
            h8 bq, bq2, bn, bn2;
            dq6(ql, qh, sw, 0, h, bq, bq2);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                if (t + 1 < 8) {
                    const int tn = t + 1, toff = 64 * (tn >> 1) + 16 * (tn & 1);
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) an[cb] = *reinterpret_cast<const h8*>(buf + aoff[cb] + toff);
                    dq6(ql, qh, sw, tn, h, bn, bn2);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) {
                    is[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[cb], bq, n == 0 && t == 0 ? zero : is[cb], 0, 0, 0);
                    is[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[cb], bq2, is[cb], 0, 0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
                if (t + 1 < 8) {
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) av[cb] = an[cb];
                    bq = bn;
                    bq2 = bn2;
                }
            }
            if (n == 1) {  // the super-block's combine: acc += (d xd) is
                const float d = (float)__builtin_bit_cast(_Float16, *reinterpret_cast<const unsigned short*>(buf + doff));
                const char* xdl = buf + kQ6XdOff;
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) {
                        const u32v4 xdw = *reinterpret_cast<const u32v4*>(xdl + (cb * 32 + q4 * 8 + h * 4) * 4);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int i = 4 * q4 + e;
                            const uint32_t wv = xdw[e];  // (a scalar copy before the bit cast)
                            acc[cb][i] = __builtin_fmaf(d * __builtin_bit_cast(float, wv), is[cb][i], acc[cb][i]);
                        }
                    }
            }
            __syncthreads();  // stage read: the producers may refill it; the next stage is loaded
        }
    }
    if (row < rows) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int c = col0 + cb * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
                if (c < ncols) y[(size_t)c * rows + row] = acc[cb][i];
            }
    }
}

// A workgroup finds its part from its row tile and its K range from blockIdx.z and the part's split;
// Q6_K parts (never in slot mode) take wsTileQ6 on a uniform branch.
template <bool SLOTS>
__global__ __launch_bounds__(kThreads) void matmul_kq_mfma_ws_kernel(MfmaGroup g, WsArgs a) {
    extern __shared__ int4 lds4[];
    char* lbase = reinterpret_cast<char*>(lds4);
    const int bx = blockIdx.x;
    const int pi = (g.nparts > 2 && bx >= g.p[2].tile0) ? 2 : (g.nparts > 1 && bx >= g.p[1].tile0) ? 1 : 0;
    const MfmaPart& p = g.p[pi];
    int z = blockIdx.z, ks = g.ks, rt = bx - p.tile0;
    if (p.ks) {  // the part's own split over its workgroups
        ks = p.ks;
        z = rt / p.ntiles;
        rt -= z * p.ntiles;
    }
    const int sb0 = z * a.nsb / ks, sb1 = (z + 1) * a.nsb / ks;
    if (!SLOTS && p.q6)
        wsTileQ6(lbase, p.qw, a, p.y[z], p.rows, rt, blockIdx.y, sb0, sb1);
    else
        wsTile<SLOTS>(lbase, p.qw, a, p.y[z], p.rows, rt, blockIdx.y, sb0, sb1);
}

}  // namespace

int mfmaWsRows() { return kRows; }

bool mfmaWsFits(const MfmaGroup& g, int nsb, int ncols) {
    for (int i = 0; i < g.nparts; ++i) {
        const unsigned long long wbytes = (unsigned long long)tilesOf(g.p[i].rows) * (unsigned long long)groupsOf(nsb) *
                                          (g.p[i].q6 ? kQ6kSeg : kQ4kSeg);
        if (wbytes >= (1ull << 32)) return false;
    }
    return (unsigned long long)ncols * nsb * 512ull < (1ull << 32);
}

int launchMfmaWs(const MfmaGroup& g, int tiles, const void* act, const void* mins, const float* xdT, int nsb, int ncols,
                 int ncp, hipStream_t s) {
    static const int attr = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(matmul_kq_mfma_ws_kernel<false>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (attr != 0) return fromHip(attr, "matmul (MFMA, producer wavefronts): LDS size");
    bool any_q4 = false;
    for (int i = 0; i < g.nparts; ++i) any_q4 |= !g.p[i].q6;
    const WsArgs a{static_cast<const _Float16*>(act), static_cast<const _Float16*>(mins), xdT, nullptr, nsb, ncols, ncp};
    const dim3 grid(tiles, (ncols + kCols - 1) / kCols, g.ks);
    hipLaunchKernelGGL(matmul_kq_mfma_ws_kernel<false>, grid, dim3(kThreads), any_q4 ? kLdsBytes : 2 * kQ6Stage, s, g,
                       a);
    return fromHip(hipGetLastError(), "matmul_q4k/q6k_q8k (MFMA, producer wavefronts)");
}

bool mfmaWsSlotsFits(int nsb) { return nsb % 4 == 0; }

int launchMfmaWsSlots(const MfmaGroup& g, int tiles, const int* xq, int nsb, int ncols, hipStream_t s) {
    static const int attr = (int)hipFuncSetAttribute(reinterpret_cast<const void*>(matmul_kq_mfma_ws_kernel<true>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (attr != 0) return fromHip(attr, "matmul (MFMA, producer wavefronts, slots): LDS size");
    if (!mfmaWsSlotsFits(nsb)) return fromHip(hipErrorInvalidValue, "matmul (MFMA, slots): k not a multiple of 1024");
    const WsArgs a{nullptr, nullptr, nullptr, xq, nsb, ncols, 0};
    const dim3 grid(tiles, (ncols + kCols - 1) / kCols, g.ks);
    for (int i = 0; i < g.nparts; ++i)
        if (g.p[i].q6) return fromHip(hipErrorInvalidValue, "matmul (MFMA, slots): Q6_K part");
    hipLaunchKernelGGL(matmul_kq_mfma_ws_kernel<true>, grid, dim3(kThreads), kLdsBytes, s, g, a);
    return fromHip(hipGetLastError(), "matmul_q4k_q8k (MFMA, producer wavefronts, slots)");
}

}  // namespace kcamd
