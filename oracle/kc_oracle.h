/*
 * kc_oracle.h -- CPU restatement of Kernelcore's K-quant LLM hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This oracle is the checker for the HIP path: only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py may load it. The product
 * library (kernelcore_amd/libkernelcore.so) never links or calls it.
 *
 * Every function restates the reference's C++ mirror (llm/llm_reference.cpp) or its kernel
 * (kernels/llm/*.cu) with the same float operations in the same order, so results are
 * bit-identical to the reference's own Kernelcore path. Weights are taken as raw ggml blocks
 * (block_q4_K: 144 bytes, block_q6_K: 210 bytes per 256 weights, rows back to back) instead
 * of the reference's 8-row word-interleaved stream: the interleave only moves bytes
 * (llm/llm_reference.cpp:385-411), the arithmetic per row is unchanged.
 *
 * Pinning (each function is checked in tests/test_oracle.py):
 *   - against the reference's own llm_reference.cpp compiled into oracle/_ref (bit-exact),
 *     and against the committed fixtures in tests/golden/ made from it;
 *   - against closed forms: IEEE binary16 decode over all 65536 patterns (numpy),
 *     quantizer invariants, double-precision dequantized dot products (3e-2, the
 *     reference's own bound, tests/test_llm_kernels.cpp:232-242).
 */
#ifndef KC_ORACLE_H
#define KC_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml_fp16_to_fp32 as llm/llm_reference.cpp:284-309 (IEEE binary16, exact). */
float kco_f16_to_f32(uint16_t h);
/* fp32 -> fp16 as set_rows_f16 converts (llm/llm_reference.cpp:735-744): round to nearest
 * even, |x| >= 65520 -> 0x7bff with sign, -0 -> +0. */
uint16_t kco_f32_to_f16(float x);

/* IEEE binary16 round to nearest even, overflow to infinity (ggml_fp32_to_fp16). */
uint16_t kco_f32_to_f16_rne(float x);
/* ggml's reference weight quantizers f32 -> block_q4_K / block_q6_K (quantize_row_q4_K_ref /
 * quantize_row_q6_K_ref, third-party, restated; see kc_oracle.c). k % 256 == 0. */
void kco_quantize_row_q4k(const float* x, uint8_t* blocks, int k);
void kco_quantize_row_q6k(const float* x, uint8_t* blocks, int k);
void kco_quantize_q4k_mt(const float* x, uint8_t* blocks, int rows, int k, int nthreads);
void kco_quantize_q6k_mt(const float* x, uint8_t* blocks, int rows, int k, int nthreads);

/* ggml dequantize_row_q4_K / q6_K (llm/llm_reference.cpp:342-383). k % 256 == 0. */
void kco_dequant_row_q4k(const uint8_t* blocks, int k, float* out);
void kco_dequant_row_q6k(const uint8_t* blocks, int k, float* out);

/* Per-32 activations (kernels/llm/quantize_q8x4.cu, llm/llm_reference.cpp:79-104):
 * xq[count][8] packed int8 words, xd[count][2] = {d, (float) sum q}. */
void kco_quantize_q8x4(const float* x, int32_t* xq, float* xd, int count);
/* quantize_cols (kernels/llm/quantize_cols.cu): ncols columns of k into slots of
 * (k/32)*11 ints; the partial-sum tail of each slot is left untouched. */
void kco_quantize_cols(const float* x, int32_t* q, int k, int ncols);
/* Per-256 activations (llm/llm_reference.cpp:491-527): one slot of nsb*85 ints. */
void kco_quantize_q8k(const float* x, int32_t* q, int nsb);
/* quantize_cols_k (kernels/llm/quantize_cols_k.cu): ncols slots of (k/256)*85 ints. */
void kco_quantize_cols_k(const float* x, int32_t* q, int k, int ncols);

/* y[rows] = W x, W as ggml blocks (rows x k/256 blocks), x as per-32 q8 activations.
 * matvec_q4k_q8: llm/llm_reference.cpp:413-445; matvec_q6k_q8: :447-489. */
void kco_matvec_q4k_q8(const uint8_t* w, const int32_t* xq, const float* xd, float* y, int rows, int k);
void kco_matvec_q6k_q8(const uint8_t* w, const int32_t* xq, const float* xd, float* y, int rows, int k);
/* Y = W X for fp16 weights and fp32 activations (llm/llm_reference.cpp:756-764, the mirror of
 * kernels/llm/matmul_f16.cu): w row-major ggml F16 [rows][k], x ncols columns of k floats, y ncols
 * columns of rows floats; per output a += (w0 x0 + w1 x1) over the value pairs in order. k even. */
void kco_matmul_f16(const uint16_t* w, const float* x, float* y, int rows, int k, int ncols);
/* One column with per-256 activations (a quantize_cols_k slot), llm/llm_reference.cpp:529-596:
 * the per-column result of matmul_{q4k,q6k}_q8kx{4,8}. */
void kco_matvec_q4k_q8k(const uint8_t* w, const int32_t* slot, float* y, int rows, int k);
void kco_matvec_q6k_q8k(const uint8_t* w, const int32_t* slot, float* y, int rows, int k);
/* Y = W X, column c of X as slot q + c*slot_ints, Y column c at y + c*rows.
 * per-32 slots (matmul_*_q8x{4,8}: bit-identical per column to the matvec) or per-256 slots. */
void kco_matmul_q4k_q8(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols);
void kco_matmul_q6k_q8(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols);
void kco_matmul_q4k_q8k(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols);
void kco_matmul_q6k_q8k(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols);

/* ---- layer ops around the matvecs (llm/llm_reference.cpp:141-153, 600-727, 773-798) ---- */
void kco_rms_norm(const float* x, const float* w, float* y, int n, int rows, float eps);
void kco_mul_rows(const float* x, const float* w, float* y, int n, int count);
void kco_silu_mul(const float* g, const float* u, float* out, int count);
void kco_add(const float* a, const float* b, float* out, int count);
/* ggml ROPE (NORM pairs (2i, 2i+1) or NEOX pairs (i, i + head_dim/2)), out of place.
 * Follows the GPU kernel (kernels/llm/rope_ggml.cu:21-44): cosf/sinf of theta directly. */
void kco_rope_ggml(const float* x, float* y, const int32_t* pos, const float* ff, int head_dim, int n_head,
                   int n_tokens, float log2_base, int neox);
/* The reference mirror's variant (llm/llm_reference.cpp:620-635): sin/cos of (theta/2pi)*2pi. */
void kco_rope_ggml_turns(const float* x, float* y, const int32_t* pos, const float* ff, int head_dim, int n_head,
                         int n_tokens, float log2_base, int neox);
/* Fused producers of per-32 slots (q: rows slots of (n/32)*11 ints). */
void kco_add_sumsq_f(const float* a, const float* b, float* out, int32_t* q, int n, int rows);
void kco_sumsq_part(const float* x, int32_t* q, int n, int rows);
void kco_norm_mul_q8(const float* x, const float* w, float* y, int32_t* q, int n, int rows, float eps);
void kco_silu_mul_q8f(const float* g, const float* u, float* y, int32_t* q, int n, int cols);
/* Per-256 variants: q holds rows slots of (n/256)*85 ints; sq the per-32 slots with the sums. */
void kco_norm_mul_q8k(const float* x, const float* w, float* y, int32_t* q, const int32_t* sq, int n, int rows,
                      float eps);
void kco_silu_mul_q8k(const float* g, const float* u, float* y, int32_t* q, int n, int cols);

/* ggml SET_ROWS into fp16 (llm/llm_reference.cpp:766-772). dst strides in fp16 pairs. */
void kco_set_rows_f16(const float* src, const int64_t* idx, uint16_t* dst, int pairs, int rows, int src_row,
                      int dst_row, int dst_rows);

/* FLASH_ATTN_EXT over an fp16 KV cache (llm/llm_reference.cpp:773-798), FaDims order of
 * llm/llm_kernels.hpp:316-332. */
typedef struct kco_fa_dims {
    int H, T, D, group, tp, k_row, k_head, v_row, v_head, N, q_tok, q_head, m_row, has_mask, H_kv;
} kco_fa_dims;
void kco_flash_attn_f16(const float* q, const uint16_t* k, const uint16_t* v, const uint16_t* mask, float* out,
                        const kco_fa_dims* d, float scale);

/* ---- CPU baseline: the same row arithmetic, rows split over nthreads OpenMP threads ---- */
void kco_matvec_q4k_q8_mt(const uint8_t* w, const int32_t* xq, const float* xd, float* y, int rows, int k,
                          int nthreads);
void kco_matvec_q6k_q8_mt(const uint8_t* w, const int32_t* xq, const float* xd, float* y, int rows, int k,
                          int nthreads);
void kco_matmul_q4k_q8k_mt(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols, int nthreads);
int  kco_max_threads(void);

/* ---- vectorised, threaded forms (kc_oracle_simd.c), bit-identical to the scalar ones above -- */
/* 2: AVX-512 VNNI, 1: AVX2, 0: scalar integer dots (the environment's KCO_SIMD caps it). */
int kco_simd_level(void);
int kco_simd_cap(int cap); /* caps the level for this process; returns the level in use */
void kco_matmul_q4k_q8k_simd(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols, int nthreads);
void kco_matmul_q6k_q8k_simd(const uint8_t* w, const int32_t* q, float* y, int rows, int k, int ncols, int nthreads);
void kco_matvec_q4k_q8_simd(const uint8_t* w, const int32_t* xq, const float* xd, float* y, int rows, int k,
                            int nthreads);
void kco_matvec_q6k_q8_simd(const uint8_t* w, const int32_t* xq, const float* xd, float* y, int rows, int k,
                            int nthreads);
void kco_flash_attn_f16_mt(const float* q, const uint16_t* k, const uint16_t* v, const uint16_t* mask, float* out,
                           const kco_fa_dims* d, float scale, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
