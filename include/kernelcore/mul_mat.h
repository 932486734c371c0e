/*
 * mul_mat.h -- the MUL_MAT dispatch of the reference's ggml backend, as a C ABI over the kc*
 * runtime: the host half of a ggml backend on MI355X, with no ggml header.
 *
 * A ggml MUL_MAT node dst = mul_mat(w, x) (w: rows x k, x: ncols columns of k f32 values,
 * dst: ncols x rows) becomes the same launches the reference records
 * (integrations/llama.cpp/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp):
 *   - F16 weights: matmul_f16 on the f32 columns as they are (:561-567);
 *   - K-quant weights: the input quantized once per recording (quantized_input, :471-497) --
 *     per-256 slots by quantize_cols_k for a batch when batch_k256 holds (:424: ncols > 1, not
 *     matvec_cols, q8k) and the columns are contiguous; else per-32 slots, by quantize_cols for
 *     contiguous columns of a batch, by one quantize_q8x4 per column otherwise -- then, for a batch
 *     without matvec_cols, one matmul_{q4k,q6k}_q8[k]x{4,8} (x8 when tile == 8 and ncols > 4), else
 *     one matvec_{q4k,q6k}_q8 per column into dst + c * rows (mul_mat_impl, :555-589).
 * A recording keeps the quantized inputs it made (keyed by input pointer, ncols, k and slot kind),
 * so matrices that read the same input (q, k, v; gate, up) quantize it once; kcMulMatRecordingReset
 * starts a new recording. The reference keys its per-recording cache by ggml tensor (:323); a caller
 * here names an input by its pointer, so one that writes new values to an input within a recording
 * (or reuses an input's memory for another tensor) resets the recording first. The ggml backend
 * (ggml_backend.h) keys the same cache by tensor.
 *
 * Weights are what a backend buffer holds after its set_tensor: K-quant as the repacked stream
 * (repack_kquant, kcKquantStreamBytes bytes), F16 as ggml's row-major halves. Launches go to the
 * recording's stream in order; nothing is synchronized unless the recording's scratch grows
 * (then the stream is synchronized before the old scratch is freed, and cached inputs are
 * dropped: the reference's flush-and-grow, scratch_take :431-449).
 */
#ifndef KERNELCORE_MUL_MAT_H
#define KERNELCORE_MUL_MAT_H

#include "kc.h"

/* The backend's switches (ggml-kernelcore.cpp:46-53) and their environment variables (:81-86):
 * GGML_KERNELCORE_MATVEC_COLS=1 -> matvec_cols = 1 (default 0); GGML_KERNELCORE_Q8K=0 -> q8k = 0
 * (default 1); GGML_KERNELCORE_TILE=4 -> tile = 4 (any other value: 8, the default);
 * GGML_KERNELCORE_ROW_BLOCK=n -> row_block = max(1, n) (default 8; passed on in the matmul
 * arguments, a CPU cache-blocking factor the GPU kernels accept and ignore). */
typedef struct kcMulMatConfig {
    int matvec_cols;
    int q8k;
    int tile;
    int row_block;
} kcMulMatConfig;

/* One MUL_MAT node. wtype: KC_QTYPE_Q4_K (12), KC_QTYPE_Q6_K (14) or KC_QTYPE_F16 (1).
 * K-quant: rows % 8 == 0, k % 256 == 0; F16: rows % 8 == 0, k even, x contiguous.
 * x_col_bytes: bytes from one input column to the next (ggml nb[1]), >= 4 k, a multiple of 4. */
typedef struct kcMulMatNode {
    int wtype;
    const void* w;
    int rows;
    int k;
    const float* x;
    long long ncols;
    size_t x_col_bytes;
    float* y;
} kcMulMatNode;

/* What a node recorded (for tests and profiling): the kernel that quantized its input ("" when
 * the recording's slots were reused, or for F16), whether they were reused, the product kernel,
 * the number of launches and whether the slots are per 256 values. */
typedef struct kcMulMatPlan {
    char quantizer[24];
    int input_reused;
    char kernel[24];
    int launches;
    int k256;
} kcMulMatPlan;

typedef struct kcMulMatRecording_st* kcMulMatRecording_t;

/* The reference's defaults, overridden by the GGML_KERNELCORE_* variables above. */
KC_API void kcMulMatConfigFromEnv(kcMulMatConfig* cfg) KC_NOEXCEPT;
/* cfg NULL: kcMulMatConfigFromEnv. stream: where every launch of the recording goes. */
KC_API kcError_t kcMulMatRecordingCreate(kcMulMatRecording_t* rec, const kcMulMatConfig* cfg,
                                         kcStream_t stream) KC_NOEXCEPT;
KC_API kcError_t kcMulMatRecordingReset(kcMulMatRecording_t rec) KC_NOEXCEPT;
KC_API kcError_t kcMulMatRecordingDestroy(kcMulMatRecording_t rec) KC_NOEXCEPT;
/* Records (launches) one node; plan may be NULL. InvalidValue for shapes or types the node's
 * kernels do not take, with the reason in kcGetLastErrorDetail. */
KC_API kcError_t kcMulMat(kcMulMatRecording_t rec, const kcMulMatNode* node, kcMulMatPlan* plan) KC_NOEXCEPT;

/* ADD (optional) + RMS_NORM + MUL by the norm weight, with the result also quantized for the
 * MUL_MATs that read it (fused_norm, ggml-kernelcore.cpp:502-530): with a and b given, x = a + b
 * (add_sumsq_f writes x and the per-32 partial sums of squares), else sumsq_part reads x; then
 * y = x / rms(x) * w (norm_mul_q8k_f for a batch under batch_k256, else norm_mul_q8_f), whose
 * 8-bit slots are registered under y: a kcMulMat of the same recording reading y (ncols = rows,
 * k = n, contiguous) takes them without quantizing again. n % 256 == 0, n * rows < 2^24. */
typedef struct kcMulMatNormNode {
    const float* a; /* NULL: no ADD */
    const float* b;
    float* x;       /* the norm's input (with ADD: written, a + b) */
    const float* w; /* the norm weight, n values */
    float* y;
    int n;
    int rows;
    float eps;
} kcMulMatNormNode;
/* plan: quantizer = the partial-sums kernel, kernel = the norm kernel. */
KC_API kcError_t kcMulMatFusedNorm(kcMulMatRecording_t rec, const kcMulMatNormNode* node,
                                   kcMulMatPlan* plan) KC_NOEXCEPT;

/* SWIGLU (y = silu(g) * u over cols rows of n) with the result also quantized and registered under
 * y as above (fused_swiglu, ggml-kernelcore.cpp:533-545: silu_mul_q8kf for a batch under
 * batch_k256, else silu_mul_q8x4f). n % 256 == 0, n * cols < 2^24. */
typedef struct kcMulMatSwigluNode {
    const float* g;
    const float* u;
    float* y;
    int n;
    int cols;
} kcMulMatSwigluNode;
KC_API kcError_t kcMulMatFusedSwiglu(kcMulMatRecording_t rec, const kcMulMatSwigluNode* node,
                                     kcMulMatPlan* plan) KC_NOEXCEPT;

#endif /* KERNELCORE_MUL_MAT_H */
