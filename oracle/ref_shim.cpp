// ref_shim.cpp -- C bindings over the reference's own C++ mirror (llm/llm_reference.cpp),
// compiled from /root/reference by oracle/Makefile into oracle/_ref/libkcref.so.
// TEST INFRASTRUCTURE ONLY: it pins the C restatement in kc_oracle.c; nothing in the product
// loads it. Weights are taken as raw ggml blocks and repacked with the reference's own
// repackQ4K/repackQ6K (llm/llm_reference.cpp:385-411) before its matvecs run.
#include "llm_reference.hpp"

#include <cstdint>
#include <vector>

using namespace llm::ref;

extern "C" {

float kcref_f16_to_f32(uint16_t h) { return f16ToF32(h); }
uint16_t kcref_f32_to_f16(float x) { return f32ToF16(x); }
void kcref_dequant_row_q4k(const uint8_t* src, int k, float* out) { dequantRowQ4K(src, k, out); }
void kcref_dequant_row_q6k(const uint8_t* src, int k, float* out) { dequantRowQ6K(src, k, out); }
void kcref_quantize_q8x4(const float* x, int* xq, float* xd, int count) { quantizeQ8x4(x, xq, xd, count); }
void kcref_quantize_q8k(const float* x, int* q, int nsb) { quantizeQ8K(x, q, nsb); }

// rows % 8 == 0 (the reference's stream groups rows by 8)
void kcref_matvec_q4k_q8(const uint8_t* w, const int* xq, const float* xd, float* y, int rows, int k) {
    std::vector<int> qw(size_t(rows) * (k / 256) * 37);
    repackQ4K(w, rows, k, qw.data());
    matvecQ4KQ8(qw.data(), xq, xd, y, rows, k);
}
void kcref_matvec_q6k_q8(const uint8_t* w, const int* xq, const float* xd, float* y, int rows, int k) {
    std::vector<int> qw(size_t(rows) * (k / 256) * 53);
    repackQ6K(w, rows, k, qw.data());
    matvecQ6KQ8(qw.data(), xq, xd, y, rows, k);
}
void kcref_matvec_q4k_q8k(const uint8_t* w, const int* slot, float* y, int rows, int k) {
    std::vector<int> qw(size_t(rows) * (k / 256) * 37);
    repackQ4K(w, rows, k, qw.data());
    matvecQ4KQ8K(qw.data(), slot, y, rows, k);
}
void kcref_matvec_q6k_q8k(const uint8_t* w, const int* slot, float* y, int rows, int k) {
    std::vector<int> qw(size_t(rows) * (k / 256) * 53);
    repackQ6K(w, rows, k, qw.data());
    matvecQ6KQ8K(qw.data(), slot, y, rows, k);
}
// rows % 8 == 0; w row-major ggml F16, repacked by the reference's repackF16 for its own stream
// round trip (unpackF16) before matmulF16 runs on the row-major values it returns.
void kcref_matmul_f16(const uint16_t* w, const float* x, float* y, int rows, int k, int ncols) {
    std::vector<int> qw(size_t(rows) * (k / 2));
    repackF16(w, rows, k, qw.data());
    std::vector<uint16_t> back(size_t(rows) * k);
    unpackF16(qw.data(), rows, k, back.data());
    matmulF16(back.data(), x, y, rows, k, ncols);
}
// The reference's stream itself, for layout tests.
void kcref_repack_q4k(const uint8_t* w, int rows, int k, int* qw) { repackQ4K(w, rows, k, qw); }
void kcref_repack_q6k(const uint8_t* w, int rows, int k, int* qw) { repackQ6K(w, rows, k, qw); }

void kcref_rms_norm(const float* x, const float* w, float* y, int n, int rows, float eps) { rmsNorm(x, w, y, n, rows, eps); }
void kcref_mul_rows(const float* x, const float* w, float* y, int n, int count) { mulRows(x, w, y, n, count); }
void kcref_silu_mul(const float* g, const float* u, float* out, int count) { siluMul(g, u, out, count); }
void kcref_rope_ggml(const float* x, float* y, const int* pos, const float* ff, int head_dim, int n_head, int n_tokens,
                     float log2_base, int neox) {
    ropeGgml(x, y, pos, ff, head_dim, n_head, n_tokens, log2_base, neox != 0);
}
void kcref_add_sumsq_f(const float* a, const float* b, float* out, int* q, int n, int rows) { addSumsqF(a, b, out, q, n, rows); }
void kcref_sumsq_part(const float* x, int* q, int n, int rows) { sumsqPart(x, q, n, rows); }
void kcref_norm_mul_q8(const float* x, const float* w, float* y, int* q, int n, int rows, float eps) {
    normMulQ8(x, w, y, q, n, rows, eps);
}
void kcref_norm_mul_q8k(const float* x, const float* w, float* y, int* q, const int* sq, int n, int rows, float eps) {
    normMulQ8K(x, w, y, q, sq, n, rows, eps);
}
void kcref_silu_mul_q8f(const float* g, const float* u, float* y, int* q, int n, int cols) { siluMulQ8F(g, u, y, q, n, cols); }
void kcref_silu_mul_q8k(const float* g, const float* u, float* y, int* q, int n, int cols) { siluMulQ8K(g, u, y, q, n, cols); }
void kcref_set_rows_f16(const float* src, const int64_t* idx, uint16_t* dst, int pairs, int rows, int src_row,
                        int dst_row, int dst_rows) {
    setRowsF16(src, idx, dst, pairs, rows, src_row, dst_row, dst_rows);
}
// d: the 15 FaDims ints in llm/llm_kernels.hpp order
void kcref_flash_attn_f16(const float* q, const uint16_t* k, const uint16_t* v, const uint16_t* mask, float* out,
                          const int* d, float scale) {
    llm::FaDims fd;
    fd.H = d[0]; fd.T = d[1]; fd.D = d[2]; fd.group = d[3]; fd.tp = d[4]; fd.k_row = d[5]; fd.k_head = d[6];
    fd.v_row = d[7]; fd.v_head = d[8]; fd.N = d[9]; fd.q_tok = d[10]; fd.q_head = d[11]; fd.m_row = d[12];
    fd.has_mask = d[13]; fd.H_kv = d[14];
    flashAttnF16(q, k, v, mask, out, fd, scale);
}

}  // extern "C"
