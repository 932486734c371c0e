// kdecode.hpp -- launchers of the fused single-token decode kernels (kdecode.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

#include "kernelcore/llm_kernels.h"

namespace kcamd {

// Prologue: where the matvec's activations come from.
constexpr int kProSlot = 0;  // a per-32 slot (xq words, xd = d / sum pairs)
constexpr int kProNorm = 1;  // RMS norm x weight of the residual row x, quantized per 32 in LDS
// Epilogue: what happens to each output row.
constexpr int kEpiStore = 0;   // y[row] = acc
constexpr int kEpiResid = 1;   // y[row] += acc (the residual stream)
constexpr int kEpiSwiglu = 2;  // part 0 = gate, part 1 = up: silu(g) * u quantized per 32 into qout

// One weight matrix of a grouped matvec (device stream of kcamd::streamBytes layout).
struct DmvPart {
    const void* qw;
    float* y;
    int rows;
    int q6;     // Q6_K (else Q4_K)
    int tiles;  // set by the launcher
    int wg0;    // first workgroup (set by the launcher)
};

struct DmvArgs {
    DmvPart p0, p1, p2;
    int nparts;
    int k;        // input length, a multiple of 256, shared by the parts
    int tpw;      // 16-row tiles per workgroup (per part for SwiGLU: 2 for whole blocks of 32)
    int ngroups;  // set by the launcher
    const float* x;   // kProNorm: residual row
    const float* nw;  // kProNorm: norm weight
    float eps;
    const int* xq;    // kProSlot
    const float* xd;  // kProSlot
    int* qout;        // kEpiSwiglu: per-32 slot of p0.rows values
    const float* r;   // kEpiResid: the residual read (y = r + acc); null: y itself, updated in place
};

struct QkPostArgs {
    const float *q, *k, *v;  // one token: [H * D], [Hkv * D], [Hkv * D]
    float* qr;               // (unused by the fused attention)
    int *kcache, *vcache;    // fp16 pairs, kv_row words per position
    const int* pos;          // pos[0]: the token's position (device)
    const float* ff;         // RoPE frequency factors [D / 2]
    const float *q_norm, *k_norm;
    int H, Hkv, D, kv_row, qk_norm, neox;
    float log2_base, eps;
};

struct AttnDecodeArgs {
    QkPostArgs qp;  // the token's q, k, v (before RoPE), caches, position, RoPE / norm parameters
    float* part;    // partial results, attnDecodePartFloats floats
    int* slot;      // per-32 slot of the H * D outputs
    int G, max_chunks, nq;
    float scale;
};

size_t dmvLds(int pro, int epi, int k, int tpw);

// The launch shape of a decode matvec (host only, no HIP call): wavefronts per workgroup, the
// 8-lane norm prologue, LDS bytes; nw == 0 when no shape fits (`why` says which limit).
struct DmvPlan {
    int nw = 0;
    bool n8 = false;
    size_t lds = 0;
    const char* why = nullptr;
};
DmvPlan planDecodeMatvec(int pro, int epi, int k, int tpw);
// rms_q8 (the output norm before the head) handles rows up to this many values.
bool rmsQ8Supports(int n);

int launchDecodeMatvec(int pro, int epi, DmvArgs a, hipStream_t s);
int launchRmsQ8(const float* x, const float* w, int* slot, int n, float eps, hipStream_t s);
bool attnDecodeSupports(int D, int G);
size_t attnDecodePartFloats(int Hkv, int max_ctx, int D);
// seq_merge: the merge in one workgroup per KV head with one thread per block quantizing (the
// first form, kept as a diagnostic); else one wavefront per 64 outputs (same results, bit for bit).
int launchAttnDecode(AttnDecodeArgs a, int D, int Hkv, int max_ctx, hipStream_t s, bool seq_merge = false);
// The ROPE / SET_ROWS prologue of a one-token flash_decode (the ggml graph's ROPE(q), ROPE(k),
// SET_ROWS(k cache), SET_ROWS(v cache) before FLASH_ATTN_EXT): every workgroup ropes its heads'
// q and k itself, the new cache row is stored by one workgroup and taken from registers by the one
// whose chunk holds it, and the roped q and k are written as the ROPE nodes' outputs.
struct FdRope {
    const float *q, *k, *v;  // one token, before RoPE: q [H][D], k [Hkv][D] contiguous; v [Hkv][D]
    float *qr, *kr;          // the ROPE outputs (same layouts as q, k); null: not written. The
                             // workgroups of chunk 0 write them while others still read q, k, v,
                             // so they must not overlap those (qn, kn below likewise)
    int *kc, *vc;            // the caches (SET_ROWS destinations): fp16 rows k_row / v_row words apart
    const int* pos;          // ROPE positions (int32; pos[0])
    const int* idx;          // SET_ROWS row (int64; its low word)
    const float* ff;         // RoPE frequency factors [D / 2]
    float log2_base;
    int neox;
    int k_row, v_row;  // cache row strides (32-bit words)
    int dst_rows;      // cache rows: a row index outside [0, dst_rows) is not stored
    int row0;          // the cache row of the attention's K / V view row 0 (the same for both)
    // Qwen3's per-head RMS norms of q and k before RoPE (q, k above are then their inputs): weights
    // [D], the normed q and k written as the MUL nodes' outputs (qn, kn; same layouts as q, k; null:
    // not written)
    const float *q_norm, *k_norm;
    float *qn, *kn;
    float eps;
    int qk_norm;
};
// flash_decode_f16 (kcFlashDecodeArgs): the split-context FLASH_ATTN_EXT for D 64 / 128, group <= 8.
bool flashDecodeSupports(int D, int G);
size_t flashDecodePartFloats(const kcFaDims& d);
// slot (optional, one query token): the output also quantized into a per-32 slot of H * D values.
// rope (optional, one query token): the ROPE / SET_ROWS prologue above (a.q is then unused).
int launchFlashDecode(const kcFlashDecodeArgs& a, hipStream_t s, int* slot = nullptr, const FdRope* rope = nullptr);

}  // namespace kcamd
