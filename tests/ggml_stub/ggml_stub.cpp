// Test-only bodies of the ggml functions the Kernelcore glue calls (see ggml.h here), restated from
// their definitions in ggml: byte size and contiguity of a tensor by its type's block size, guid
// comparison, the buffer object a buffer type hands out.
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "ggml-backend-impl.h"
#include "ggml-impl.h"

namespace {
void blocks(ggml_type t, int64_t* blck, size_t* size) {
    *blck = 1;
    switch (t) {
        case GGML_TYPE_F16: *size = 2; return;
        case GGML_TYPE_Q4_K: *blck = 256; *size = 144; return;
        case GGML_TYPE_Q6_K: *blck = 256; *size = 210; return;
        case GGML_TYPE_I64: *size = 8; return;
        default: *size = 4; return;
    }
}
}  // namespace

extern "C" {

bool ggml_guid_matches(ggml_guid_t a, ggml_guid_t b) { return std::memcmp(a, b, sizeof(ggml_guid)) == 0; }

int64_t ggml_nelements(const ggml_tensor* t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }

size_t ggml_nbytes(const ggml_tensor* t) {
    for (int i = 0; i < GGML_MAX_DIMS; ++i)
        if (t->ne[i] <= 0) return 0;
    int64_t blck;
    size_t size;
    blocks(t->type, &blck, &size);
    size_t n = blck == 1 ? size : size_t(t->ne[0]) * t->nb[0] / size_t(blck);
    if (blck == 1) n += size_t(t->ne[0] - 1) * t->nb[0];
    for (int i = 1; i < GGML_MAX_DIMS; ++i) n += size_t(t->ne[i] - 1) * t->nb[i];
    return n;
}

bool ggml_is_contiguous(const ggml_tensor* t) {
    int64_t blck;
    size_t next;
    blocks(t->type, &blck, &next);
    if (t->ne[0] != blck && t->nb[0] != next) return false;
    next *= size_t(t->ne[0] / blck);
    for (int i = 1; i < GGML_MAX_DIMS; ++i)
        if (t->ne[i] != 1) {
            if (t->nb[i] != next) return false;
            next *= size_t(t->ne[i]);
        }
    return true;
}

const char* ggml_op_desc(const ggml_tensor* t) {
    static const char* names[GGML_OP_COUNT] = {"NONE", "ADD", "MUL", "RMS_NORM", "MUL_MAT", "RESHAPE", "VIEW", "PERMUTE",
                                               "TRANSPOSE", "GET_ROWS", "SET_ROWS", "SOFT_MAX", "ROPE", "FLASH_ATTN_EXT",
                                               "GLU"};
    return t->op >= 0 && t->op < GGML_OP_COUNT ? names[t->op] : "?";
}

void ggml_abort(const char* file, int line, const char* fmt, ...) {
    std::fprintf(stderr, "%s:%d: ", file, line);
    va_list ap;
    va_start(ap, fmt);
    std::vfprintf(stderr, fmt, ap);
    va_end(ap);
    std::fprintf(stderr, "\n");
    std::abort();
}

void ggml_log_internal(int, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vfprintf(stderr, fmt, ap);
    va_end(ap);
}

ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft, ggml_backend_buffer_i iface, void* context,
                                               size_t size) {
    return new ggml_backend_buffer{iface, buft, context, size, GGML_BACKEND_BUFFER_USAGE_ANY};
}

ggml_backend_buffer_type_t ggml_backend_buffer_get_type(ggml_backend_buffer_t buffer) { return buffer->buft; }

}  // extern "C"
