#pragma once

#include "ggml.h"
#include "ggml-backend.h"

// Kernelcore backend on AMD Instinct MI355X (gfx950): GGUF K-quant (Q4_K, Q6_K) matrix products,
// RMS norm, RoPE, SwiGLU, the fp16 KV cache and flash attention as HIP kernels in HBM, through
// libkernelcore_amd (kernelcore_amd/ in this repository). The three entry points of the reference
// backend's header (integrations/llama.cpp/ggml/include/ggml-kernelcore.h:15-17).

#ifdef __cplusplus
extern "C" {
#endif

GGML_BACKEND_API ggml_backend_t     ggml_backend_kernelcore_init(void);
GGML_BACKEND_API bool               ggml_backend_is_kc(ggml_backend_t backend);
GGML_BACKEND_API ggml_backend_reg_t ggml_backend_kernelcore_reg(void);

#ifdef __cplusplus
}
#endif
