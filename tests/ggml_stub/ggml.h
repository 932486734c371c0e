// Test-only stand-in for the part of ggml's public API (ggml.h) that the Kernelcore ggml glue
// (kernelcore_amd/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp) uses, written from ggml's documented
// interface so the glue can be compiled and run here without llama.cpp. It is not ggml: enum values
// other than the GGUF type ids, and the struct layouts, are this stand-in's own; a real build uses
// ggml's headers.
#pragma once

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#define GGML_API __attribute__((visibility("default")))
#define GGML_BACKEND_API __attribute__((visibility("default")))
#define GGML_NORETURN __attribute__((noreturn))

#define GGML_MAX_DIMS 4
#define GGML_MAX_SRC 10
#define GGML_MAX_OP_PARAMS 64
#define GGML_MAX_NAME 64

#ifdef __cplusplus
extern "C" {
#endif

// the GGUF type ids (ggml_type's values)
enum ggml_type {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_Q4_0 = 2,
    GGML_TYPE_Q8_0 = 8,
    GGML_TYPE_Q4_K = 12,
    GGML_TYPE_Q5_K = 13,
    GGML_TYPE_Q6_K = 14,
    GGML_TYPE_I32 = 26,
    GGML_TYPE_I64 = 27,
    GGML_TYPE_COUNT = 40,
};

enum ggml_op {
    GGML_OP_NONE = 0,
    GGML_OP_ADD,
    GGML_OP_MUL,
    GGML_OP_RMS_NORM,
    GGML_OP_MUL_MAT,
    GGML_OP_RESHAPE,
    GGML_OP_VIEW,
    GGML_OP_PERMUTE,
    GGML_OP_TRANSPOSE,
    GGML_OP_GET_ROWS,
    GGML_OP_SET_ROWS,
    GGML_OP_SOFT_MAX,
    GGML_OP_ROPE,
    GGML_OP_FLASH_ATTN_EXT,
    GGML_OP_GLU,
    GGML_OP_COUNT,
};

enum ggml_tensor_flag {
    GGML_TENSOR_FLAG_INPUT = 1,
    GGML_TENSOR_FLAG_OUTPUT = 2,
    GGML_TENSOR_FLAG_PARAM = 4,
    GGML_TENSOR_FLAG_LOSS = 8,
    GGML_TENSOR_FLAG_COMPUTE = 16,
};

enum ggml_status {
    GGML_STATUS_ALLOC_FAILED = -2,
    GGML_STATUS_FAILED = -1,
    GGML_STATUS_SUCCESS = 0,
    GGML_STATUS_ABORTED = 1,
};

struct ggml_backend_buffer;

struct ggml_tensor {
    enum ggml_type type;
    struct ggml_backend_buffer * buffer;
    int64_t ne[GGML_MAX_DIMS];
    size_t nb[GGML_MAX_DIMS];
    enum ggml_op op;
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    int32_t flags;
    struct ggml_tensor * src[GGML_MAX_SRC];
    struct ggml_tensor * view_src;
    size_t view_offs;
    void * data;
    char name[GGML_MAX_NAME];
    void * extra;
};

struct ggml_cgraph;

typedef uint8_t ggml_guid[16];
typedef ggml_guid * ggml_guid_t;

GGML_API bool ggml_guid_matches(ggml_guid_t guid_a, ggml_guid_t guid_b);
GGML_API size_t ggml_nbytes(const struct ggml_tensor * tensor);
GGML_API int64_t ggml_nelements(const struct ggml_tensor * tensor);
GGML_API bool ggml_is_contiguous(const struct ggml_tensor * tensor);
GGML_API const char * ggml_op_desc(const struct ggml_tensor * t);
GGML_API GGML_NORETURN void ggml_abort(const char * file, int line, const char * fmt, ...);

#define GGML_ABORT(...) ggml_abort(__FILE__, __LINE__, __VA_ARGS__)
#define GGML_ASSERT(x) \
    do { \
        if (!(x)) GGML_ABORT("GGML_ASSERT(%s) failed", #x); \
    } while (0)

#ifdef __cplusplus
}
#endif
