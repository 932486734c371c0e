/*
 * llm_kernels.h -- typed arguments of the built-in LLM kernels, launched by name through
 * kcLaunchKernel / kcLaunchKernelChunked (kc.h).
 *
 * The structs keep the field order, types and defaults of the reference's
 * llm/llm_kernels.hpp (arasheedu/Kernelcore), so its callers fill them unchanged; in C++ they
 * are also reachable as llm::<Name> (e.g. llm::MatvecQ4Q8Args). Differences on this device:
 *   - `dims` (a device int array the reference's CPU marshal reads back, llm_kernels.cpp:85-90)
 *     may be NULL: sizes travel as kernel arguments. When non-NULL it must be a live
 *     allocation of the stated length, and if the runtime holds a host copy of it (the bytes
 *     were written with kcMemcpy/kcMemset), its values must match the sizes, as in the
 *     reference (InvalidValue otherwise).
 *   - K-quant weights (`qw`) are this library's weight stream, written by the repack kernels
 *     below from raw ggml blocks (reference: llm::ref::repackQ4K/Q6K, llm_reference.cpp:385-411,
 *     which writes a CPU-oriented 8-row word interleave). kcKquantStreamBytes gives its size.
 */
#ifndef KERNELCORE_LLM_KERNELS_H
#define KERNELCORE_LLM_KERNELS_H

#include "kc.h"

#if defined(__cplusplus)
#define KC_INIT(v) = v
#else
#define KC_INIT(v)
#endif

/* ---- slot layouts of quantized activations (llm/llm_kernels.hpp:79-89) --------------------------
 * per 32 values:  [nb * 8 packed int8 words | nb * 2 floats {d, sum q} | nb floats (RMS partial sums)]
 * per 256 values: [nsb * 64 words | nsb float d | nsb * 16 int sums of 16 | nsb * 4 words: the sums
 *                  of 32 as bytes, B >> 6 for sums 0-3 and 4-7, then B & 63] */
static inline int kcScratchInts(int nb) { return nb * 11; }
static inline int kcScratchKInts(int nsb) { return nsb * 85; }

/* kernels/vector_add.cu via include/kernelcore/kernels.hpp:10-15: out = a + b. Chunkable. */
typedef struct kcVectorAddArgs {
    const float* a;
    const float* b;
    float* out;
    int count;
} kcVectorAddArgs;

/* quantize_q8x4 (llm_kernels.hpp:52-58): count blocks of 32 -> xq[count][8], xd[count][2]. */
typedef struct kcQuantizeArgs {
    const float* x;
    int* xq;
    float* xd;
    int count;
} kcQuantizeArgs;

/* matvec_q4k_q8 / matvec_q6k_q8 (llm_kernels.hpp:62-70): y[rows] = W x. rows % 8 == 0,
 * k % 256 == 0, qw: kcKquantStreamBytes bytes, xq: k/32*8 ints, xd: k/32*2 floats. */
typedef struct kcMatvecQ4Q8Args {
    const int* qw;
    const int* xq;
    const float* xd;
    float* y;
    const int* dims;
    int rows;
    int k;
} kcMatvecQ4Q8Args;

/* matmul_{q4k,q6k}_q8x{4,8} (per-32 slots) and matmul_{q4k,q6k}_q8kx{4,8} (per-256 slots),
 * llm_kernels.hpp:262-271: Y = W X, column c from slot xq + c * slot_ints, written to y + c * rows.
 * On the GPU the x4 / x8 names are the same kernels (a column-tiled kernel, bit-exact per column,
 * and for Q4_K with per-256 slots and >= 32 columns the MFMA kernel); row_block is validated
 * (> 0) and otherwise unused. */
typedef struct kcMatmulKQ8Args {
    const int* qw;
    const int* xq;
    float* y;
    const int* dims;
    int rows;
    int k;
    int ncols;
    int row_block KC_INIT(8);
} kcMatmulKQ8Args;

/* matmul_f16 (llm_kernels.hpp:285-296): Y = W X for fp16 weights and fp32 activations. qw: the
 * weights in ggml's row-major F16 layout (rows x k halves, two per 32-bit word; the reference's
 * load-time 8-row interleave, llm_reference.cpp:740-746, has no counterpart here); x: ncols columns
 * of k floats; y: ncols columns of rows floats. rows % 8 == 0, k even; dims may be NULL, else
 * {rows, k, ncols}. From 9 columns (k % 16 == 0) the products run on the matrix cores with each
 * activation split into two fp16 parts: activations must then stay below 65504 in magnitude. */
typedef struct kcMatmulF16Args {
    const int* qw;
    const float* x;
    float* y;
    const int* dims;
    int rows;
    int k;
    int ncols;
} kcMatmulF16Args;

/* quantize_cols / quantize_cols_k (llm_kernels.hpp:277-283). k % 256 == 0. */
typedef struct kcQuantizeColsArgs {
    const float* x;
    int* q;
    const int* dims;
    int k;
    int ncols;
} kcQuantizeColsArgs;

/* rms_norm (llm_kernels.hpp:134-141): one row of n per row. */
typedef struct kcRmsNormArgs {
    const float* x;
    const float* w;
    float* y;
    int n;
    int rows;
    float eps;
} kcRmsNormArgs;

/* mul_rows (llm_kernels.hpp:161-168): y[i] = x[i] * w[i % n]. */
typedef struct kcMulRowsArgs {
    const float* x;
    const float* w;
    float* y;
    int n;
    int count;
} kcMulRowsArgs;

/* rope_ggml (llm_kernels.hpp:173-185): NORM (pairs 2i, 2i+1) or NEOX (i, i + head_dim/2). */
typedef struct kcRopeGgmlArgs {
    const float* x;
    float* y;
    const int* pos;
    const float* ff;
    const int* dims;
    int head_dim;
    int n_head;
    int n_tokens;
    float log2_base;
    bool neox KC_INIT(false);
} kcRopeGgmlArgs;

/* add_sumsq_f / sumsq_part / norm_mul_q8_f (+ norm_mul_q8k_f) / silu_mul_q8x4f (+ silu_mul_q8kf),
 * llm_kernels.hpp:187-215. Rows of n values, n % 256 == 0. */
typedef struct kcAddSumsqFArgs {
    const float* a;
    const float* b;
    float* out;
    int* q;
    const int* dims;
    int n;
    int rows;
} kcAddSumsqFArgs;
typedef struct kcSumsqPartArgs {
    const float* x;
    int* q;
    const int* dims;
    int n;
    int rows;
} kcSumsqPartArgs;
typedef struct kcNormMulQ8Args {
    const float* x;
    const float* w;
    float* y;
    int* q;
    const int* dims;
    int n;
    int rows;
    float eps;
} kcNormMulQ8Args;
/* add_norm_q8_f (no reference counterpart: add_sumsq_f, or sumsq_part when a and b are null,
 * followed by norm_mul_q8_f, in one launch with one workgroup per row, for rows of 256 .. 8192
 * values): x = a + b (else x is read), the per-32 sums of squares into the slot tails, then
 * y = x * r * w and the per-32 slot q -- the same bytes as the two launches. dims: [n / 32, n, rows]. */
typedef struct kcAddNormQ8FArgs {
    const float* a;
    const float* b;
    float* x;
    const float* w;
    float* y;
    int* q;
    const int* dims;
    int n;
    int rows;
    float eps;
} kcAddNormQ8FArgs;
typedef struct kcSiluMulQ8FArgs {
    const float* g;
    const float* u;
    float* y;
    int* q;
    const int* dims;
    int n;
    int cols;
} kcSiluMulQ8FArgs;

/* silu_mul (llm_kernels.hpp:255-260): out = silu(g) * u. */
typedef struct kcSiluMulArgs {
    const float* g;
    const float* u;
    float* out;
    int count;
} kcSiluMulArgs;

/* set_rows_f16 (llm_kernels.hpp:295-308): dst row idx[r] (int64) = fp16(src row r). */
typedef struct kcSetRowsF16Args {
    const float* src;
    const int* idx;
    int* dst;
    const int* dims;
    int pairs;
    int rows;
    int src_row;
    int dst_row;
    int dst_rows;
} kcSetRowsF16Args;

/* FLASH_ATTN_EXT over an fp16 KV cache (llm_kernels.hpp:313-366). */
typedef struct kcFaDims {
    int H KC_INIT(0);
    int T KC_INIT(0);
    int D KC_INIT(0);
    int group KC_INIT(0);
    int tp KC_INIT(0);
    int k_row KC_INIT(0);
    int k_head KC_INIT(0);
    int v_row KC_INIT(0);
    int v_head KC_INIT(0);
    int N KC_INIT(0);
    int q_tok KC_INIT(0);
    int q_head KC_INIT(0);
    int m_row KC_INIT(0);
    int has_mask KC_INIT(0);
    int H_kv KC_INIT(0);
} kcFaDims;
typedef struct kcFaScoresArgs {
    const float* q;
    const int* k;
    const int* mask;
    float* s;
    const int* dims;
    kcFaDims d;
    float scale;
} kcFaScoresArgs;
typedef struct kcFaMaxArgs {
    const float* s;
    float* m;
    const int* dims;
    kcFaDims d;
} kcFaMaxArgs;
typedef struct kcFaExpArgs {
    float* s;
    const float* m;
    const int* dims;
    kcFaDims d;
} kcFaExpArgs;
typedef struct kcFaValuesArgs {
    const float* p;
    const int* v;
    float* out;
    const int* dims;
    kcFaDims d;
} kcFaValuesArgs;

/* flash_attn_f16 (no reference counterpart beyond the four fa_* kernels it fuses): the same
 * FLASH_ATTN_EXT result, out[N][H][D], in one kernel; d.T <= 16384. */
typedef struct kcFlashAttnArgs {
    const float* q;
    const int* k;
    const int* v;
    const int* mask;
    float* out;
    const int* dims;
    kcFaDims d;
    float scale;
} kcFlashAttnArgs;

/* flash_decode_f16 (no reference counterpart: the same FLASH_ATTN_EXT result for a few query tokens
 * over a long context): split over 64-position chunks, each chunk's maximum, sum of exponentials
 * and unnormalized output in part (N * H * ceil(T / 64) * (D + 2) floats), then merged in chunk
 * order into out[N][H][D]. D is 64 or 128 and the group (query heads per KV head) at most 8;
 * within 2e-6 of the four fa_* kernels (another summation order). */
typedef struct kcFlashDecodeArgs {
    const float* q;
    const int* k;
    const int* v;
    const int* mask;
    float* out;
    float* part;
    const int* dims;
    kcFaDims d;
    float scale;
} kcFlashDecodeArgs;

/* ---- K-quant weight streams (this device's layout; no reference counterpart beyond
 * llm::ref::repackQ4K/Q6K and the ggml backend's unpack_stream, ggml-kernelcore.cpp:124-154) ----
 * Rows are grouped in tiles of 16 and super-blocks in groups of 4 (padding rows and super-blocks
 * are zero blocks). For tile t and group g the 64 (super-block, row) pairs are the 64 lanes of a
 * wavefront (lane = kq * 16 + r), and their ggml blocks are stored as 1 KiB slabs: slab c holds
 * bytes [16c, 16c + 16) of the 64 blocks in lane order, so one 16-byte load per lane reads a
 * whole slab. Q4_K: 9 slabs (144 B per block). Q6_K: 13 slabs (bytes 0..207) then the 64 fp16
 * `d` values (128 B). The stream must be 16-byte aligned. */
#define KC_QTYPE_Q4_K 12 /* ggml type ids */
#define KC_QTYPE_Q6_K 14
typedef struct kcKquantRepackArgs {
    const void* src; /* repack: ggml blocks (rows * k/256 blocks); unpack: the stream */
    void* dst;       /* repack: the stream; unpack: ggml blocks */
    int qtype;       /* KC_QTYPE_Q4_K or KC_QTYPE_Q6_K */
    int rows;
    int k;
} kcKquantRepackArgs;
/* get_rows_kquant: y[i][0..k) = the dequantized row ids[i] of a Q4_K / Q6_K weight stream, n rows.
 * The block formula and float order of ggml's dequantize_row_q4_K / q6_K as the reference restates
 * them (llm/llm_reference.cpp:342-383: d1 = d*sc, m1 = dmin*m, y = d1*q - m1; y = (d*sc)*q), so
 * the values are bit-identical to it; the reference calls it for the token embedding
 * (llm/gguf_model.cpp:96-104), ggml as GET_ROWS. ids are device ints; an id outside [0, rows)
 * yields a row of zeros. */
typedef struct kcGetRowsKquantArgs {
    const void* qw;  /* the weight stream (repack_kquant) */
    const int* ids;  /* n row ids */
    float* y;        /* n x k floats */
    int qtype;       /* KC_QTYPE_Q4_K or KC_QTYPE_Q6_K */
    int rows;
    int k;
    int n;
} kcGetRowsKquantArgs;
/* kcLaunchMatmulNoAlloc: the matmul names matmul_{q4k,q6k}_q8{,k}x{4,8} with kcMatmulKQ8Args, the same
 * validation, kernels and results as kcLaunchKernel, but allocating nothing: no hipMalloc, hipFree or
 * allocating library routine on any call. It has no counterpart in the reference; it is for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Where kcLaunchKernel stages a batch's fp16 activations (per-256 slots, 64 columns and
 * more) in the runtime's per-stream scratch, this stages them in a fixed 16 MiB device array that
 * each GPU holds until the process ends: ncols * k * 2 + ncols * k / 8 + (k / 256) * 4 * ncols
 * rounded up to 128 must be at most 16 MiB (e.g. 512 columns of 12288 values), else InvalidValue
 * with the sizes in the detail text. Every call on a GPU shares that array, so calls that overlap
 * on one GPU (concurrent streams, a graph replayed while another call runs) race; inside a
 * concurrent group it returns UnsupportedOperation. */
KC_API kcError_t kcLaunchMatmulNoAlloc(const char* name, const kcMatmulKQ8Args* args, kcStream_t stream) KC_NOEXCEPT;
/* quantize_kquant: rows x k f32 values (row-major, k % 256 == 0) -> rows * k/256 ggml blocks
 * (block_q4_K, 144 bytes, or block_q6_K, 210 bytes), as ggml's reference quantizers
 * quantize_row_q4_K_ref / quantize_row_q6_K_ref compute them (third-party: the reference itself
 * has no quantizer; its weights come from GGUF files written by ggml). For making the synthetic
 * K-quant weights of the BASELINE configurations on the device. */
typedef struct kcQuantizeKquantArgs {
    const float* x;
    void* blocks;
    int qtype; /* KC_QTYPE_Q4_K or KC_QTYPE_Q6_K */
    int rows;
    int k;
} kcQuantizeKquantArgs;
/* fill_normal_f32: y[i] = mean + stdev * N(0, 1) for i < n, a deterministic function of (seed, i)
 * (splitmix64 counter stream, Box-Muller): synthetic weights and activations of a given seed. */
typedef struct kcFillNormalArgs {
    float* y;
    long long n;
    unsigned long long seed;
    float mean;
    float stdev;
} kcFillNormalArgs;
/* Bytes of the weight stream of a rows x k matrix (buft_get_alloc_size, ggml-kernelcore.cpp:116-118). */
KC_API kcError_t kcKquantStreamBytes(int qtype, int rows, int k, size_t* bytes) KC_NOEXCEPT;

#ifdef __cplusplus
namespace kc::kernels {
typedef ::kcVectorAddArgs VectorAddArgs;
}
namespace llm {
typedef ::kcQuantizeArgs QuantizeArgs;
typedef ::kcMatvecQ4Q8Args MatvecQ4Q8Args;
typedef ::kcMatmulKQ8Args MatmulKQ8Args;
typedef ::kcMatmulF16Args MatmulF16Args;
typedef ::kcQuantizeColsArgs QuantizeColsArgs;
typedef ::kcRmsNormArgs RmsNormArgs;
typedef ::kcMulRowsArgs MulRowsArgs;
typedef ::kcRopeGgmlArgs RopeGgmlArgs;
typedef ::kcAddSumsqFArgs AddSumsqFArgs;
typedef ::kcSumsqPartArgs SumsqPartArgs;
typedef ::kcNormMulQ8Args NormMulQ8Args;
typedef ::kcAddNormQ8FArgs AddNormQ8FArgs;
typedef ::kcSiluMulQ8FArgs SiluMulQ8FArgs;
typedef ::kcSiluMulArgs SiluMulArgs;
typedef ::kcSetRowsF16Args SetRowsF16Args;
typedef ::kcFaDims FaDims;
typedef ::kcFaScoresArgs FaScoresArgs;
typedef ::kcFaMaxArgs FaMaxArgs;
typedef ::kcFaExpArgs FaExpArgs;
typedef ::kcFaValuesArgs FaValuesArgs;
typedef ::kcKquantRepackArgs KquantRepackArgs;
typedef ::kcGetRowsKquantArgs GetRowsKquantArgs;
typedef ::kcQuantizeKquantArgs QuantizeKquantArgs;
typedef ::kcFillNormalArgs FillNormalArgs;
typedef ::kcFlashAttnArgs FlashAttnArgs;
inline int scratchInts(int nb) { return nb * 11; }
inline float* scratchScales(int* q, int nb) { return reinterpret_cast<float*>(q + nb * 8); }
inline int scratchKInts(int nsb) { return nsb * 85; }
inline int padTo8(int n) { return (n + 7) / 8 * 8; }
constexpr int kFaDims = 15;
inline void faDimsInts(const FaDims& d, int* out) {
    const int v[kFaDims] = {d.H,      d.T,  d.D,     d.group,  d.tp,    d.k_row,    d.k_head, d.v_row,
                            d.v_head, d.N,  d.q_tok, d.q_head, d.m_row, d.has_mask, d.H_kv};
    for (int i = 0; i < kFaDims; ++i) out[i] = v[i];
}
/* llm_kernels.hpp:370: every built-in kernel is registered by kcInit on this device. */
inline kc::Error registerKernels() noexcept { return kc::Error::Success; }
}  // namespace llm
#endif

#endif /* KERNELCORE_LLM_KERNELS_H */
