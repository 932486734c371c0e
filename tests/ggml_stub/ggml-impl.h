// Test-only stand-in for ggml-impl.h (see ggml.h here): logging and the graph with its use counts.
#pragma once

#include "ggml.h"

#ifdef __cplusplus
extern "C" {
#endif

GGML_API void ggml_log_internal(int level, const char * format, ...);
#define GGML_LOG_INFO(...) ggml_log_internal(2, __VA_ARGS__)
#define GGML_LOG_WARN(...) ggml_log_internal(3, __VA_ARGS__)
#define GGML_LOG_ERROR(...) ggml_log_internal(4, __VA_ARGS__)

// The stand-in's graph keeps one use count per node (ggml keeps them in its visited hash set).
struct ggml_cgraph {
    int size;
    int n_nodes;
    int n_leafs;
    struct ggml_tensor ** nodes;
    struct ggml_tensor ** leafs;
    int32_t * use_counts;
};

static inline int ggml_node_get_use_count(const struct ggml_cgraph * cgraph, int node_idx) {
    return cgraph->use_counts[node_idx];
}

#ifdef __cplusplus
}
#endif
