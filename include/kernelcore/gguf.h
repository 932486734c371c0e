/*
 * gguf.h -- a read-only GGUF file reader (C ABI): the metadata and the tensor directory of a
 * llama.cpp / Ollama model file, the file mapped read-only.
 *
 * It restates the reference's minimal reader (llm/gguf.hpp:12-60, llm/gguf.cpp) behind C
 * linkage: open, look up numbers / strings / tensors, close. GGUF versions 2 and 3 are read;
 * every length, count and offset is checked against the file size, so a truncated or corrupt file
 * is an InvalidValue error with the reason in kcGetLastErrorDetail, never a read past the map.
 * These calls touch no GPU and need no kcInit. kcModelLoadGguf (model.h) builds a model from a
 * file through the same reader.
 */
#ifndef KERNELCORE_GGUF_H
#define KERNELCORE_GGUF_H

#include <stdint.h>

#include "kc.h"

typedef struct kcGguf_st* kcGguf_t;

/* ggml tensor type ids of the types this reader knows the block size of */
#define KC_GGML_F32 0
#define KC_GGML_F16 1
#define KC_GGML_Q4_0 2
#define KC_GGML_Q4_1 3
#define KC_GGML_Q5_0 6
#define KC_GGML_Q5_1 7
#define KC_GGML_Q8_0 8
#define KC_GGML_Q2_K 10
#define KC_GGML_Q3_K 11
#define KC_GGML_Q4_K 12
#define KC_GGML_Q5_K 13
#define KC_GGML_Q6_K 14
#define KC_GGML_Q8_K 15
#define KC_GGML_BF16 30

KC_API kcError_t kcGgufOpen(const char* path, kcGguf_t* file) KC_NOEXCEPT;
KC_API kcError_t kcGgufClose(kcGguf_t file) KC_NOEXCEPT;
/* GGUF version (2 or 3) and the data section's alignment */
KC_API kcError_t kcGgufVersion(kcGguf_t file, int* version, int* alignment) KC_NOEXCEPT;
/* A numeric scalar (any integer, float or bool type) as a double; InvalidValue if the key is
 * missing or not numeric. */
KC_API kcError_t kcGgufGetNum(kcGguf_t file, const char* key, double* value) KC_NOEXCEPT;
/* A string scalar; the pointer and length stay valid until kcGgufClose (not NUL-terminated). */
KC_API kcError_t kcGgufGetStr(kcGguf_t file, const char* key, const char** str, size_t* len) KC_NOEXCEPT;
/* An array's element count and GGUF element type (0 UINT8 ... 12 FLOAT64, 8 STRING) */
KC_API kcError_t kcGgufGetArray(kcGguf_t file, const char* key, int64_t* count, int* elem_type) KC_NOEXCEPT;
KC_API kcError_t kcGgufTensorCount(kcGguf_t file, int* count) KC_NOEXCEPT;
/* The i-th tensor's name (directory order; NUL-terminated, valid until kcGgufClose) */
KC_API kcError_t kcGgufTensorName(kcGguf_t file, int i, const char** name) KC_NOEXCEPT;
/* A tensor by name: ggml type, dimensions (ne[0] = values per row), its bytes and a pointer to
 * them in the mapped file (valid until kcGgufClose). InvalidValue if the name is absent. */
KC_API kcError_t kcGgufTensorInfo(kcGguf_t file, const char* name, int* type, int* n_dims, int64_t ne[4],
                                  size_t* bytes, const void** data) KC_NOEXCEPT;

#endif /* KERNELCORE_GGUF_H */
