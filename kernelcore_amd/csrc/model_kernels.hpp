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
int launchArgmaxStep(const float* logits, int n, int* tokens, int* gen, int* step, int* n_past, int max_gen,
                     hipStream_t s);
int launchPositions(const int* n_past, int n, int* pos, long long* idx, int* n_ctx, hipStream_t s);

}  // namespace kcamd
