/*
 * model.h -- the decode driver: a Llama / Qwen3-architecture transformer with K-quant weights
 * running on the kc* runtime and the built-in kernels (C ABI).
 *
 * It replaces the reference's standalone driver (llm/llm_model.hpp:195 decodeToken,
 * llm/llm_model.cpp:287-360) and follows the op order of the reference's ggml backend graph
 * (docs/cuda_cpu_poc_plan.md:1158): RMS_NORM+MUL (fused with the 8-bit quantization), MUL_MAT q/k/v,
 * [per-head q/k RMS_NORM for Qwen3], ROPE q/k, SET_ROWS k/v into an fp16 cache, FLASH_ATTN_EXT,
 * MUL_MAT o, ADD, RMS_NORM+MUL, MUL_MAT gate/up, SWIGLU (fused with the quantization), MUL_MAT
 * down, ADD; then the output norm and head. As in the reference backend, a single token uses
 * per-32 activations and the matvecs; a batch uses per-256 activations and the matmuls.
 *
 * Weights arrive as raw ggml blocks (kcModelSetTensor) and are repacked on the GPU; the KV cache
 * is fp16 in HBM. kcModelGenerate runs greedy decode as replays of one captured hipGraph: the
 * next token, the position and the context length stay on the GPU between steps.
 */
#ifndef KERNELCORE_MODEL_H
#define KERNELCORE_MODEL_H

#include "kc.h"

typedef struct kcModelConfig {
    int n_layer;
    int n_embd;
    int n_head;
    int n_head_kv;
    int head_dim;
    int n_ff;
    int n_vocab;
    float norm_eps;
    float rope_theta;
    int rope_neox;  /* 0: NORM pairs (2i, 2i+1), Llama; 1: NEOX pairs (i, i + head_dim/2), Qwen3 */
    int qk_norm;    /* per-head RMS norm of q and k before RoPE (Qwen3) */
    int max_ctx;    /* KV-cache capacity in positions (<= 16384) */
    int max_batch;  /* largest n_tokens of one kcModelForward */
} kcModelConfig;

typedef struct kcModel_st* kcModel_t;

/* tensor ids for kcModelSetTensor / kcModelTensorInfo; per-layer ids take a layer index */
#define KC_TENSOR_TOKEN_EMBD 0  /* Q4_K, n_vocab x n_embd */
#define KC_TENSOR_OUTPUT_NORM 1 /* f32 [n_embd] */
#define KC_TENSOR_OUTPUT 2      /* Q6_K, n_vocab x n_embd */
#define KC_TENSOR_ATTN_NORM 3   /* f32 [n_embd] */
#define KC_TENSOR_WQ 4          /* Q4_K, n_head*head_dim x n_embd */
#define KC_TENSOR_WK 5          /* Q4_K, n_head_kv*head_dim x n_embd */
#define KC_TENSOR_WV 6          /* Q6_K, n_head_kv*head_dim x n_embd */
#define KC_TENSOR_WO 7          /* Q4_K, n_embd x n_head*head_dim */
#define KC_TENSOR_FFN_NORM 8    /* f32 [n_embd] */
#define KC_TENSOR_W_GATE 9      /* Q4_K, n_ff x n_embd */
#define KC_TENSOR_W_UP 10       /* Q4_K, n_ff x n_embd */
#define KC_TENSOR_W_DOWN 11     /* Q6_K, n_embd x n_ff */
#define KC_TENSOR_Q_NORM 12     /* f32 [head_dim] (qk_norm only) */
#define KC_TENSOR_K_NORM 13     /* f32 [head_dim] (qk_norm only) */
#define KC_TENSOR_ROPE_FREQS 14 /* f32 [head_dim / 2], optional: RoPE frequency factors (theta_i / ff[i]) */
#define KC_TENSOR_COUNT 15
#define KC_QTYPE_F32 0
#define KC_QTYPE_F16 1 /* ggml F16: row-major fp16 values (per-layer matrices only; matmul_f16) */

KC_API kcError_t kcModelCreate(const kcModelConfig* cfg, kcModel_t* model) KC_NOEXCEPT;
KC_API kcError_t kcModelDestroy(kcModel_t model) KC_NOEXCEPT;
/* Host-only check of a config (no device work, callable before kcInit): InvalidValue for widths the
 * driver does not handle, else *fused = 1 when single tokens run the six fused kernels per layer
 * and 0 when they run one kernel per op (both give the same results to the parity bars). A model
 * with an F16 matrix, or gate and up matrices of different types, also takes the unfused path. */
KC_API kcError_t kcModelPlanDecode(const kcModelConfig* cfg, int* fused) KC_NOEXCEPT;
/* What a tensor holds: qtype (KC_QTYPE_F32, KC_QTYPE_F16, KC_QTYPE_Q4_K, KC_QTYPE_Q6_K), rows and k
 * (f32 vectors: rows = 1), and the bytes kcModelSetTensor expects (ggml blocks, halves or floats). */
KC_API kcError_t kcModelTensorInfo(kcModel_t model, int tensor, int layer, int* qtype, int* rows, int* k,
                                   size_t* bytes) KC_NOEXCEPT;
KC_API kcError_t kcModelSetTensor(kcModel_t model, int tensor, int layer, const void* host, size_t bytes) KC_NOEXCEPT;
/* The same with the weight type given: any matrix tensor takes KC_QTYPE_Q4_K or KC_QTYPE_Q6_K
 * (a GGUF "Q4_K_M" file mixes them per layer), the per-layer matrices also KC_QTYPE_F16 (ggml F16,
 * e.g. a Qwen3 attn_v; multiplied by the f32 activations, as the reference's ggml backend does), the
 * f32 vectors KC_QTYPE_F32. (A model with an F16 matrix, or a layer whose gate and up matrices differ
 * in type, decodes single tokens with the unfused kernels.) */
KC_API kcError_t kcModelSetTensorTyped(kcModel_t model, int tensor, int layer, int qtype, const void* host,
                                       size_t bytes) KC_NOEXCEPT;
/* Creates a model from a GGUF file (general.architecture "llama" or "qwen3"; Q4_K / Q6_K matrices,
 * F16 per-layer matrices, f32 norms; output.weight absent = tied to token_embd; rope_freqs.weight
 * optional): the
 * hyperparameters come from the file's metadata, max_ctx and max_batch from the caller. Errors
 * (unreadable file, unsupported architecture or tensor type, shape mismatch) return InvalidValue
 * with the reason in kcGetLastErrorDetail. The file is read once; the model does not keep it. */
KC_API kcError_t kcModelLoadGguf(const char* path, int max_ctx, int max_batch, kcModel_t* model) KC_NOEXCEPT;
/* Appends n_tokens (host ids) at the current position and returns the last token's logits
 * (host, n_vocab floats; may be NULL). n_tokens == 1: the decode path; more: the batch path. */
KC_API kcError_t kcModelForward(kcModel_t model, const int* tokens, int n_tokens, float* logits) KC_NOEXCEPT;
/* Greedy decode: starts from the argmax of the last forward's logits and generates `steps`
 * tokens (written to tokens_out, host), each one graph replay. */
KC_API kcError_t kcModelGenerate(kcModel_t model, int steps, int* tokens_out) KC_NOEXCEPT;
/* Current position (tokens in the KV cache); kcModelReset empties the cache. */
KC_API kcError_t kcModelPosition(kcModel_t model, int* pos) KC_NOEXCEPT;
KC_API kcError_t kcModelReset(kcModel_t model) KC_NOEXCEPT;
/* Copies positions [pos0, pos0 + n) of a layer's fp16 KV cache (which: 0 k, 1 v) to host memory:
 * n * n_head_kv * head_dim halves, in the ggml set_rows layout (a position's heads back to back). For
 * checks and inspection; it waits for the model's queued work. */
KC_API kcError_t kcModelReadCache(kcModel_t model, int layer, int which, int pos0, int n, void* host) KC_NOEXCEPT;
/* The model's stream (its work is ordered on it), for timing with kcEventRecord. */
KC_API kcError_t kcModelStream(kcModel_t model, kcStream_t* stream) KC_NOEXCEPT;

#endif /* KERNELCORE_MODEL_H */
