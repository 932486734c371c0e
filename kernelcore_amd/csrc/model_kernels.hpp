// model_kernels.hpp -- launchers of the decode driver's own kernels (model_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace kcamd {

// Attention shape for attn_kernel: q is [N][H][D] (q_tok floats per token), the fp16 caches are
// [t][H_kv][D] as 32-bit words (kv_row words per position); T comes from device memory.
struct AttnShape {
    int N, H, H_kv, D, q_tok, kv_row, max_t, causal;
    float scale;
};

int launchGetRows(bool q6k, const void* qw, const int* tok, float* y, int n, int k, int rows, hipStream_t s);
int launchAttn(const float* q, const int* k, const int* v, float* out, const int* n_ctx, const AttnShape& a,
               hipStream_t s);
// FLASH_ATTN_EXT on the matrix cores with ggml's f16 mask (rows of m_row2 halves, 4-byte aligned)
// over T <= m_row2 keys: q rows a.q_tok floats apart (heads D apart), K / V rows a.kv_row words
// apart (heads D / 2 words apart), out[N][H][D] rows a.q_tok apart; D 64 or 128. msum: the mask's
// summary (launchMaskSummary over the same mask, N and T, earlier on the stream).
bool attnMaskedSupports(const AttnShape& a);
int launchAttnMasked(const float* q, const int* k, const int* v, const unsigned short* mask, int m_row2, int T,
                     float* out, const AttnShape& a, const int* msum, hipStream_t s);
// The mask's summary for launchAttnMasked: maskSummaryInts(N) ints, four per tile of 32 query rows.
int maskSummaryInts(int N);
int launchMaskSummary(const unsigned short* mask, int m_row2, int N, int T, int* sum, hipStream_t s);
// The same attention with the G = H / H_kv query heads of a KV head in one workgroup (kattn_prefill.hip,
// G <= 4, D 64 or 128): mask null = causal over T = *n_ctx, else ggml's mask (m_row2 halves per
// row) over t_host keys with its summary msum; cache_rows = the rows K and V hold.
bool attnGqaSupports(const AttnShape& a);
int launchAttnGqa(const float* q, const int* k, const int* v, float* out, const int* n_ctx, const AttnShape& a,
                  const unsigned short* mask, int m_row2, int t_host, int cache_rows, const int* msum, hipStream_t s);
int launchArgmaxStep(const float* logits, int n, int* tokens, int* gen, int* step, int* n_past, int max_gen,
                     hipStream_t s);
int launchPositions(const int* n_past, int n, int* pos, long long* idx, int* n_ctx, hipStream_t s);

}  // namespace kcamd
