/*
 * ggml_backend.h -- the compute side of the reference's ggml backend on MI355X, as a C ABI over
 * tensor descriptors, with no ggml header: which ops the backend claims and how it runs a graph of
 * them (integrations/llama.cpp/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp: dev_supports_op_impl
 * :902-957 with weight_shape_ok :103-109 and flash_attn_ok :873-891; backend_graph_compute
 * :706-792 with its op launchers :591-699 and fusions :502-545; the switches :42-57, :75-89).
 *
 * The ggml glue is the only part that needs llama.cpp: its supports_op and graph_compute
 * callbacks fill one kcGgmlTensor per ggml_tensor (the node and every src it reads) and call
 * kcGgmlSupportsOp / kcGgmlGraphCompute; its buffer callbacks are kcWeight* (weights.h).
 *
 * kcGgmlGraphCompute walks the nodes as the reference does -- nodes without the compute flag and
 * empty nodes skipped; consecutive MUL_MATs of one input as one step; [ADD +] RMS_NORM + MUL by a
 * row vector fused into add_sumsq_f / sumsq_part + norm_mul_q8[k]_f, whose 8-bit output the next
 * MUL_MATs take; RMS_NORM + MUL otherwise one rms_norm with the weight; SWIGLU with n % 256 == 0
 * fused into silu_mul_q8[k]f -- and launches the same kernels (kcLaunchKernel names) on the
 * backend's stream, except that FLASH_ATTN_EXT runs split over the context for up to 8 query tokens
 * (flash_decode_f16) and as one flash_attn_f16 kernel for larger batches (the four fa_* kernels
 * beyond 16384 positions), and that a fused norm or SwiGLU whose n * rows reaches 2^24 (beyond the
 * fused kernels) runs unfused. It returns once the stream has run them.
 *
 * Graphs (switch on): the launches of a call are captured into a HIP graph and launched; the graph
 * is kept, and a later call with the same nodes (ops, types, shapes, strides, data pointers,
 * parameters, flags and the same src links) launches it again without recording. Off: the
 * launches go to the stream one by one. Either way the scratch (8-bit activations) is sized by a
 * planning pass before anything is launched, so it never grows while a graph is recorded.
 */
#ifndef KERNELCORE_GGML_BACKEND_H
#define KERNELCORE_GGML_BACKEND_H

#include "kc.h"
#include "mul_mat.h"

/* ggml ops the backend knows (the glue maps ggml_op onto these; any other op is KC_GGML_OP_OTHER) */
#define KC_GGML_OP_NONE 0
#define KC_GGML_OP_RESHAPE 1
#define KC_GGML_OP_VIEW 2
#define KC_GGML_OP_PERMUTE 3
#define KC_GGML_OP_TRANSPOSE 4
#define KC_GGML_OP_MUL_MAT 5
#define KC_GGML_OP_ADD 6
#define KC_GGML_OP_RMS_NORM 7
#define KC_GGML_OP_MUL 8
#define KC_GGML_OP_ROPE 9
#define KC_GGML_OP_GLU 10
#define KC_GGML_OP_SET_ROWS 11
#define KC_GGML_OP_FLASH_ATTN_EXT 12
#define KC_GGML_OP_OTHER 13

/* ggml type ids (ggml.h's enum ggml_type, the GGUF numbering); other types never match a rule */
#define KC_GGML_TYPE_F32 0
#define KC_GGML_TYPE_F16 1
#define KC_GGML_TYPE_Q4_K 12
#define KC_GGML_TYPE_Q6_K 14
#define KC_GGML_TYPE_I32 26
#define KC_GGML_TYPE_I64 27

/* ggml.h's values, read from op_params as the glue copies them: ROPE op_params[2] mode bit, GLU
 * op_params[0] */
#define KC_GGML_ROPE_TYPE_NEOX 2
#define KC_GGML_GLU_OP_SWIGLU 2

/* Where a tensor (a view: its view_src) lives: the backend's weight buffer type (kcWeight*), its
 * KV-cache buffer type (the reference's kc_host_buffer_type: device memory here), or elsewhere. */
#define KC_GGML_BUFFER_OTHER 0
#define KC_GGML_BUFFER_WEIGHTS 1
#define KC_GGML_BUFFER_KV 2

typedef struct kcGgmlTensor {
    int op;                          /* KC_GGML_OP_* */
    int type;                        /* KC_GGML_TYPE_* */
    int64_t ne[4];                   /* ggml_tensor ne, nb, data */
    size_t nb[4];
    void* data;
    const struct kcGgmlTensor* src[5]; /* ggml_tensor src[0..4]; NULL where ggml's is NULL */
    int32_t op_params[16];           /* ggml_tensor op_params, copied as they are */
    int buffer;                      /* KC_GGML_BUFFER_* */
    int compute;                     /* flags & GGML_TENSOR_FLAG_COMPUTE */
    int output;                      /* flags & GGML_TENSOR_FLAG_OUTPUT */
    int view;                        /* view_src != NULL */
    int uses;                        /* the graph's use count of the node (ggml_cgraph use_counts) */
} kcGgmlTensor;

/* The backend's switches and their environment variables (ggml-kernelcore.cpp:42-57, :75-89). */
typedef struct kcGgmlConfig {
    kcMulMatConfig mul_mat; /* GGML_KERNELCORE_MATVEC_COLS, _Q8K, _TILE, _ROW_BLOCK (mul_mat.h) */
    int disabled;           /* GGML_KERNELCORE_DISABLE=1: claim nothing (default 0) */
    int matmul_only;        /* GGML_KERNELCORE_MATMUL_ONLY=1: only MUL_MAT (default 0) */
    int attn;               /* GGML_KERNELCORE_ATTN=0: no SET_ROWS / FLASH_ATTN_EXT, no KV buffers (default 1) */
    int attn_tokens;        /* GGML_KERNELCORE_ATTN_TOKENS=n: largest batch whose attention runs here (default 8) */
    int concurrent;         /* GGML_KERNELCORE_CONCURRENT=0: MUL_MATs of one input not grouped (default 1) */
    int graphs;             /* GGML_KERNELCORE_GRAPHS=0: no graph recording (default 1) */
    int profile;            /* GGML_KERNELCORE_PROFILE=1: time each call's recording and run; =2: also
                               every launch (default 0; ggml-kernelcore.cpp:331-346, 1033-1035) */
} kcGgmlConfig;

/* The times are host wall clock over the calls that succeeded, kept only with profile >= 1
 * (BackendCtx t_compute / t_record / t_run, ggml-kernelcore.cpp:331-346): compute_ms the whole
 * kcGgmlGraphCompute call; record_ms the planning pass and the walk that records the graph (or,
 * graphs off, issues the launches); run_ms the graph launch (a kept graph's too) and the wait for
 * the stream (graphs off: the wait). */
typedef struct kcGgmlStats {
    long long computes;       /* kcGgmlGraphCompute calls that succeeded */
    long long graphs_recorded; /* calls that recorded (and launched) a new graph */
    long long graphs_reused;   /* calls that launched the kept graph again */
    long long launches;        /* kernel launches recorded or made (a reused graph's count again) */
    double compute_ms;
    double record_ms;
    double run_ms;
} kcGgmlStats;

/* profile = 2: every launch timed on the device (HIP events on the backend's stream around it; the
 * call's launches are then made one by one, as the reference times them only with graphs off,
 * :400-415), summed per kernel name; launches made for a MUL_MAT node or a group of them carry the
 * first weight's shape ("matvec_q4k_q8 3072x3072": rows x k), as GGML_KERNELCORE_PROFILE=2 does. */
typedef struct kcGgmlProfileEntry {
    char name[64];
    long long launches;
    double ms;
} kcGgmlProfileEntry;

typedef struct kcGgmlBackend_st* kcGgmlBackend_t;

/* The reference's defaults overridden by the variables above. */
KC_API void kcGgmlConfigFromEnv(kcGgmlConfig* cfg) KC_NOEXCEPT;

/* supports_op: 1 when the backend runs op (with its srcs as described), else 0; cfg NULL: from the
 * environment. Host logic only: no device is touched. */
KC_API int kcGgmlSupportsOp(const kcGgmlConfig* cfg, const kcGgmlTensor* op) KC_NOEXCEPT;
/* get_host_buffer_type: 1 when the backend offers its KV-cache buffer type (not disabled, not
 * matmul_only, attn on), else 0. */
KC_API int kcGgmlOffersKvBuffer(const kcGgmlConfig* cfg) KC_NOEXCEPT;

/* The launch sequence kcGgmlGraphCompute would make for nodes[0..n_nodes), as kernel names
 * separated by spaces ("[" and "]" around a concurrent group), without a device: written to names
 * (size bytes, NUL-terminated) when it fits; *needed (optional) is the size it takes. The scratch
 * ints the call would take go to *scratch_ints (optional). UnsupportedOperation names the first
 * compute node the backend does not run. */
KC_API kcError_t kcGgmlGraphPlan(const kcGgmlConfig* cfg, const kcGgmlTensor* const* nodes, int n_nodes, char* names,
                                 size_t size, size_t* needed, size_t* scratch_ints) KC_NOEXCEPT;

/* init: a backend on stream (NULL: the default stream) with cfg (NULL: from the environment).
 * Needs kcInit; fails with UnsupportedOperation when cfg disables the backend. */
KC_API kcError_t kcGgmlBackendCreate(kcGgmlBackend_t* backend, const kcGgmlConfig* cfg,
                                     kcStream_t stream) KC_NOEXCEPT;
KC_API kcError_t kcGgmlBackendDestroy(kcGgmlBackend_t backend) KC_NOEXCEPT;
/* graph_compute over nodes[0..n_nodes) (the graph's nodes in order). */
KC_API kcError_t kcGgmlGraphCompute(kcGgmlBackend_t backend, const kcGgmlTensor* const* nodes,
                                    int n_nodes) KC_NOEXCEPT;
KC_API kcError_t kcGgmlBackendGetStats(kcGgmlBackend_t backend, kcGgmlStats* stats) KC_NOEXCEPT;
/* The per-launch times of profile = 2, in name order: the first min(capacity, *count) entries are
 * written; *count is how many there are. */
KC_API kcError_t kcGgmlBackendGetProfile(kcGgmlBackend_t backend, kcGgmlProfileEntry* entries, int capacity,
                                         int* count) KC_NOEXCEPT;

#endif /* KERNELCORE_GGML_BACKEND_H */
