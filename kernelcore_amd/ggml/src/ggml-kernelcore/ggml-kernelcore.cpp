// ggml-kernelcore.cpp -- the ggml backend "Kernelcore" on AMD Instinct MI355X (gfx950): the vtables
// llama.cpp's scheduler calls, each mapped onto libkernelcore_amd's C ABI (include/kernelcore/*.h).
// It takes the place of the reference's integrations/llama.cpp/ggml/src/ggml-kernelcore/
// ggml-kernelcore.cpp and exports what that file exports (ggml_backend_kernelcore_init / _is_kc / _reg
// and GGML_BACKEND_DL_IMPL, :1025-1054); it builds only inside a llama.cpp tree (ggml's headers).
//
// - Device: ACCEL, as the reference's (:830-847), so llama.cpp offers this backend's buffer type
//   for every weight; supports_op and graph_compute are kcGgmlSupportsOp / kcGgmlGraphCompute over
//   one kcGgmlTensor descriptor per ggml tensor (ggml_backend.h holds the rules and the node walk).
// - Buffer type "Kernelcore": HBM (kcMalloc). A 2-D K-quant weight is held in the kernels' stream
//   layout (kcWeightSetTensor repacks it on the GPU; get_tensor unpacks; memset_tensor sets ggml
//   bytes of it); every other tensor is a plain device copy. Not a host buffer.
// - Buffer type "Kernelcore_Host": the KV caches (the reference's host buffer type, :285-310, which
//   llama.cpp's hook places CPU layers' caches in). Here it is HBM too, so it is not a host buffer:
//   where the CPU backend reads a cache (attention this backend does not claim), ggml's scheduler
//   copies it, instead of every attention of the GPU reading its cache over PCIe.
// - Compute: each call runs on the backend's own HIP stream and returns once the stream has run
//   the launches; a HIP graph of a call is kept and launched again by a later call with the same
//   nodes (kcGgmlGraphCompute). GGML_KERNELCORE_PROFILE=1|2 times calls (and launches) and prints
//   the sums when the backend is freed, as the reference does (:331-346).

#include "ggml-kernelcore.h"

#include "ggml-backend-impl.h"
#include "ggml-impl.h"

#include <kernelcore/ggml_backend.h>
#include <kernelcore/kc.h>
#include <kernelcore/weights.h>

#include <algorithm>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <unordered_map>
#include <vector>

namespace {

// ---- the runtime (process-wide) ----------------------------------------------------------------------

struct KcRuntime {
    bool ok = false;
    kcGgmlConfig cfg{};  // the GGML_KERNELCORE_* switches (kcGgmlConfigFromEnv)
    char device[192] = "Kernelcore";
};

KcRuntime & runtime() {
    static KcRuntime rt = [] {
        KcRuntime r;
        kcGgmlConfigFromEnv(&r.cfg);
        if (kcInit() != kc::Error::Success) {
            GGML_LOG_ERROR("Kernelcore: kcInit failed: %s\n", kcGetLastErrorDetail());
            return r;
        }
        kcDeviceProperties p{};
        if (kcGetDeviceProperties(&p, 0) == kc::Error::Success)
            std::snprintf(r.device, sizeof r.device, "Kernelcore on %s: K-quant LLM kernels in HBM", p.name);
        r.ok = true;
        GGML_LOG_INFO("Kernelcore: %s, graphs %s\n", r.device, r.cfg.graphs ? "on" : "off");
        return r;
    }();
    return rt;
}

// ---- weights --------------------------------------------------------------------------------------

bool is_kquant(ggml_type t) { return t == GGML_TYPE_Q4_K || t == GGML_TYPE_Q6_K; }

// A tensor the weight buffers hold in the kernels' stream layout: a 2-D K-quant matrix of whole
// super-blocks and 8-row groups (the reference's weight_shape_ok for K-quants, :103-109).
bool stream_weight(const ggml_tensor * t) {
    return is_kquant(t->type) && t->ne[0] % 256 == 0 && t->ne[1] % 8 == 0 && t->ne[2] == 1 && t->ne[3] == 1 &&
           t->ne[0] <= INT_MAX && t->ne[1] <= INT_MAX && ggml_is_contiguous(t);
}

[[noreturn]] void fail(const char * what) {
    GGML_ABORT("Kernelcore: %s failed: %s", what, kcGetLastErrorDetail());
}

// ---- buffers ------------------------------------------------------------------------------------------

struct BufferCtx {
    void * base = nullptr;
    size_t size = 0;
};

void buffer_free(ggml_backend_buffer_t buffer) {
    auto * ctx = static_cast<BufferCtx *>(buffer->context);
    (void) kcFree(ctx->base);
    delete ctx;
}

void * buffer_get_base(ggml_backend_buffer_t buffer) { return static_cast<BufferCtx *>(buffer->context)->base; }

void buffer_memset_tensor(ggml_backend_buffer_t, ggml_tensor * tensor, uint8_t value, size_t offset, size_t size) {
    const kc::Error e = stream_weight(tensor)
                            ? kcWeightMemsetTensor(tensor->type, int(tensor->ne[1]), int(tensor->ne[0]), tensor->data,
                                                   value, offset, size, nullptr)
                            : kcMemset(static_cast<char *>(tensor->data) + offset, value, size);
    if (e != kc::Error::Success) fail("memset_tensor");
}

void buffer_set_tensor(ggml_backend_buffer_t, ggml_tensor * tensor, const void * data, size_t offset, size_t size) {
    if (stream_weight(tensor)) {
        GGML_ASSERT(offset == 0 && size == ggml_nbytes(tensor) && "Kernelcore: K-quant weights are uploaded whole");
        if (kcWeightSetTensor(tensor->type, int(tensor->ne[1]), int(tensor->ne[0]), tensor->data, data, 0, size,
                              nullptr) != kc::Error::Success)
            fail("set_tensor (repack)");
        return;
    }
    if (kcMemcpy(static_cast<char *>(tensor->data) + offset, data, size, kc::CopyKind::HostToDevice) != kc::Error::Success)
        fail("set_tensor");
}

void buffer_get_tensor(ggml_backend_buffer_t, const ggml_tensor * tensor, void * data, size_t offset, size_t size) {
    const kc::Error e =
        stream_weight(tensor)
            ? kcWeightGetTensor(tensor->type, int(tensor->ne[1]), int(tensor->ne[0]), tensor->data, data, offset, size,
                                nullptr)
            : kcMemcpy(data, static_cast<const char *>(tensor->data) + offset, size, kc::CopyKind::DeviceToHost);
    if (e != kc::Error::Success) fail("get_tensor");
}

ggml_backend_buffer_type_t kc_buffer_type();
ggml_backend_buffer_type_t kc_host_buffer_type();

bool own_buffer(ggml_backend_buffer_t b) {
    return b && (ggml_backend_buffer_get_type(b) == kc_buffer_type() || ggml_backend_buffer_get_type(b) == kc_host_buffer_type());
}

// Between tensors in this backend's buffers a copy stays on the device (no reference counterpart:
// there, host memory made ggml's fallback through the host as cheap). A weight's stream is not its
// ggml bytes, so weights take the fallback.
bool buffer_cpy_tensor(ggml_backend_buffer_t, const ggml_tensor * src, ggml_tensor * dst) {
    const ggml_backend_buffer_t sb = src->view_src ? src->view_src->buffer : src->buffer;
    if (!own_buffer(sb) || stream_weight(src) || stream_weight(dst) || ggml_nbytes(src) != ggml_nbytes(dst)) return false;
    return kcMemcpy(dst->data, src->data, ggml_nbytes(src), kc::CopyKind::DeviceToDevice) == kc::Error::Success;
}

void buffer_clear(ggml_backend_buffer_t buffer, uint8_t value) {
    auto * ctx = static_cast<BufferCtx *>(buffer->context);
    if (kcMemset(ctx->base, value, ctx->size) != kc::Error::Success) fail("clear");
}

const ggml_backend_buffer_i buffer_i = {
    /* .free_buffer   = */ buffer_free,
    /* .get_base      = */ buffer_get_base,
    /* .init_tensor   = */ nullptr,
    /* .memset_tensor = */ buffer_memset_tensor,
    /* .set_tensor    = */ buffer_set_tensor,
    /* .get_tensor    = */ buffer_get_tensor,
    /* .set_tensor_2d = */ nullptr,
    /* .get_tensor_2d = */ nullptr,
    /* .cpy_tensor    = */ buffer_cpy_tensor,
    /* .clear         = */ buffer_clear,
    /* .reset         = */ nullptr,
};

// The KV caches: fp16 rows in ggml's layout, plain copies (nothing is repacked).
void kv_buffer_memset_tensor(ggml_backend_buffer_t, ggml_tensor * tensor, uint8_t value, size_t offset, size_t size) {
    if (kcMemset(static_cast<char *>(tensor->data) + offset, value, size) != kc::Error::Success) fail("memset_tensor");
}
void kv_buffer_set_tensor(ggml_backend_buffer_t, ggml_tensor * tensor, const void * data, size_t offset, size_t size) {
    if (kcMemcpy(static_cast<char *>(tensor->data) + offset, data, size, kc::CopyKind::HostToDevice) != kc::Error::Success)
        fail("set_tensor");
}
void kv_buffer_get_tensor(ggml_backend_buffer_t, const ggml_tensor * tensor, void * data, size_t offset, size_t size) {
    if (kcMemcpy(data, static_cast<const char *>(tensor->data) + offset, size, kc::CopyKind::DeviceToHost) != kc::Error::Success)
        fail("get_tensor");
}

const ggml_backend_buffer_i kv_buffer_i = {
    /* .free_buffer   = */ buffer_free,
    /* .get_base      = */ buffer_get_base,
    /* .init_tensor   = */ nullptr,
    /* .memset_tensor = */ kv_buffer_memset_tensor,
    /* .set_tensor    = */ kv_buffer_set_tensor,
    /* .get_tensor    = */ kv_buffer_get_tensor,
    /* .set_tensor_2d = */ nullptr,
    /* .get_tensor_2d = */ nullptr,
    /* .cpy_tensor    = */ buffer_cpy_tensor,
    /* .clear         = */ buffer_clear,
    /* .reset         = */ nullptr,
};

// ---- buffer types -------------------------------------------------------------------------------------

ggml_backend_buffer_t alloc_buffer(ggml_backend_buffer_type_t buft, const ggml_backend_buffer_i & iface, size_t size) {
    if (!runtime().ok) return nullptr;
    void * p = nullptr;
    const size_t bytes = size ? size : 64;  // llama.cpp probes with empty buffers
    if (kcMalloc(&p, bytes) != kc::Error::Success) {
        GGML_LOG_ERROR("Kernelcore: allocating %zu bytes failed: %s\n", bytes, kcGetLastErrorDetail());
        return nullptr;
    }
    return ggml_backend_buffer_init(buft, iface, new BufferCtx{p, bytes}, size);
}

const char * buft_get_name(ggml_backend_buffer_type_t) { return "Kernelcore"; }
ggml_backend_buffer_t buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) { return alloc_buffer(buft, buffer_i, size); }
size_t buft_get_alignment(ggml_backend_buffer_type_t) { return 64; }  // the streams and the 16-byte loads need 16

size_t buft_get_alloc_size(ggml_backend_buffer_type_t, const ggml_tensor * tensor) {
    size_t stream = 0;
    if (stream_weight(tensor) &&
        kcWeightAllocSize(tensor->type, int(tensor->ne[1]), int(tensor->ne[0]), &stream) == kc::Error::Success)
        return std::max(stream, ggml_nbytes(tensor));
    return ggml_nbytes(tensor);
}

bool buft_is_host(ggml_backend_buffer_type_t) { return false; }  // HBM, and weights are not in ggml layout

const ggml_backend_buffer_type_i buft_i = {
    /* .get_name         = */ buft_get_name,
    /* .alloc_buffer     = */ buft_alloc_buffer,
    /* .alloc_buffer_n   = */ nullptr,
    /* .get_alignment    = */ buft_get_alignment,
    /* .get_max_size     = */ nullptr,
    /* .get_alloc_size   = */ buft_get_alloc_size,
    /* .get_alloc_size_n = */ nullptr,
    /* .is_host          = */ buft_is_host,
};

const char * kv_buft_get_name(ggml_backend_buffer_type_t) { return "Kernelcore_Host"; }
ggml_backend_buffer_t kv_buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) { return alloc_buffer(buft, kv_buffer_i, size); }
size_t kv_buft_get_alloc_size(ggml_backend_buffer_type_t, const ggml_tensor * tensor) { return ggml_nbytes(tensor); }
bool   kv_buft_is_host(ggml_backend_buffer_type_t) { return false; }  // HBM: the CPU backend gets copies

const ggml_backend_buffer_type_i kv_buft_i = {
    /* .get_name         = */ kv_buft_get_name,
    /* .alloc_buffer     = */ kv_buft_alloc_buffer,
    /* .alloc_buffer_n   = */ nullptr,
    /* .get_alignment    = */ buft_get_alignment,
    /* .get_max_size     = */ nullptr,
    /* .get_alloc_size   = */ kv_buft_get_alloc_size,
    /* .get_alloc_size_n = */ nullptr,
    /* .is_host          = */ kv_buft_is_host,
};

// ---- tensor descriptors -----------------------------------------------------------------------------------

int kc_op(ggml_op op) {
    switch (op) {
        case GGML_OP_NONE: return KC_GGML_OP_NONE;
        case GGML_OP_RESHAPE: return KC_GGML_OP_RESHAPE;
        case GGML_OP_VIEW: return KC_GGML_OP_VIEW;
        case GGML_OP_PERMUTE: return KC_GGML_OP_PERMUTE;
        case GGML_OP_TRANSPOSE: return KC_GGML_OP_TRANSPOSE;
        case GGML_OP_MUL_MAT: return KC_GGML_OP_MUL_MAT;
        case GGML_OP_ADD: return KC_GGML_OP_ADD;
        case GGML_OP_RMS_NORM: return KC_GGML_OP_RMS_NORM;
        case GGML_OP_MUL: return KC_GGML_OP_MUL;
        case GGML_OP_ROPE: return KC_GGML_OP_ROPE;
        case GGML_OP_GLU: return KC_GGML_OP_GLU;
        case GGML_OP_SET_ROWS: return KC_GGML_OP_SET_ROWS;
        case GGML_OP_FLASH_ATTN_EXT: return KC_GGML_OP_FLASH_ATTN_EXT;
        default: return KC_GGML_OP_OTHER;
    }
}

// Where a tensor lives (a view: where its view_src lives).
int kc_buffer(const ggml_tensor * t) {
    const ggml_backend_buffer_t b = t->view_src ? t->view_src->buffer : t->buffer;
    if (!b) return KC_GGML_BUFFER_OTHER;
    const ggml_backend_buffer_type_t bt = ggml_backend_buffer_get_type(b);
    return bt == kc_buffer_type() ? KC_GGML_BUFFER_WEIGHTS : bt == kc_host_buffer_type() ? KC_GGML_BUFFER_KV : KC_GGML_BUFFER_OTHER;
}

// One kcGgmlTensor per ggml tensor (elements of an unordered_map keep their addresses): a graph's
// nodes first, each with its use count, then every src they read linked to its own descriptor
// (tensors outside the node list -- weights, inputs, views -- carry no uses). `depth` bounds how far
// srcs are linked (supports_op reads the op's srcs, not theirs).
struct Descs {
    std::unordered_map<const ggml_tensor *, kcGgmlTensor> d;

    kcGgmlTensor * put(const ggml_tensor * t, int uses) {
        auto [it, fresh] = d.try_emplace(t);
        kcGgmlTensor & k = it->second;
        if (!fresh) return &k;
        std::memset(&k, 0, sizeof k);
        k.op = kc_op(t->op);
        k.type = int(t->type);
        for (int i = 0; i < 4; ++i) {
            k.ne[i] = t->ne[i];
            k.nb[i] = t->nb[i];
        }
        k.data = t->data;
        static_assert(sizeof k.op_params <= sizeof t->op_params, "op_params");
        std::memcpy(k.op_params, t->op_params, sizeof k.op_params);
        k.buffer = kc_buffer(t);
        k.compute = (t->flags & GGML_TENSOR_FLAG_COMPUTE) != 0;
        k.output = (t->flags & GGML_TENSOR_FLAG_OUTPUT) != 0;
        k.view = t->view_src != nullptr;
        k.uses = uses;
        return &k;
    }
    void link(const ggml_tensor * t, int depth) {
        kcGgmlTensor & k = d.at(t);
        for (int i = 0; i < 5; ++i) {
            if (!t->src[i] || k.src[i]) continue;
            const bool fresh = !d.count(t->src[i]);
            k.src[i] = put(t->src[i], 0);
            if (fresh && depth > 1) link(t->src[i], depth - 1);
        }
    }
    const kcGgmlTensor * op(const ggml_tensor * t) {  // an op and its srcs (supports_op)
        const kcGgmlTensor * k = put(t, 0);
        link(t, 1);
        return k;
    }
};

// ---- backend ----------------------------------------------------------------------------------------------

struct BackendCtx {
    kcStream_t      stream = nullptr;   // the backend's own HIP stream (launches are asynchronous on it)
    kcGgmlBackend_t core = nullptr;     // kcGgmlGraphCompute's state: scratch, the kept graph, stats
    int             profile = 0;

    ~BackendCtx() {
        if (profile && core) print_profile();
        if (core) (void) kcGgmlBackendDestroy(core);
        if (stream) (void) kcStreamDestroy(stream);
    }
    void print_profile() const {
        kcGgmlStats s{};
        if (kcGgmlBackendGetStats(core, &s) != kc::Error::Success || !s.computes) return;
        std::fprintf(stderr, "Kernelcore profile: %lld graph_compute calls, %lld launches; compute %.1f ms, recording %.1f ms, "
                             "kernel runs %.1f ms\n", s.computes, s.launches, s.compute_ms, s.record_ms, s.run_ms);
        int n = 0;
        if (kcGgmlBackendGetProfile(core, nullptr, 0, &n) != kc::Error::Success || n == 0) return;
        std::vector<kcGgmlProfileEntry> e(static_cast<size_t>(n));
        if (kcGgmlBackendGetProfile(core, e.data(), n, &n) != kc::Error::Success) return;
        for (const auto & k : e)
            std::fprintf(stderr, "  %-40s %8lld launches %9.1f ms %7.1f us each\n", k.name, k.launches, k.ms,
                         k.ms * 1e3 / double(k.launches));
    }
};

const char * backend_get_name(ggml_backend_t) { return "Kernelcore"; }

void backend_free(ggml_backend_t backend) {
    delete static_cast<BackendCtx *>(backend->context);
    delete backend;
}

ggml_status backend_graph_compute(ggml_backend_t backend, ggml_cgraph * cgraph) {
    auto & ctx = *static_cast<BackendCtx *>(backend->context);
    Descs ds;
    std::vector<const kcGgmlTensor *> nodes(size_t(std::max(cgraph->n_nodes, 0)));
    for (int i = 0; i < cgraph->n_nodes; ++i) nodes[size_t(i)] = ds.put(cgraph->nodes[i], ggml_node_get_use_count(cgraph, i));
    for (int i = 0; i < cgraph->n_nodes; ++i) ds.link(cgraph->nodes[i], INT_MAX);
    const kc::Error e = kcGgmlGraphCompute(ctx.core, nodes.data(), cgraph->n_nodes);
    if (e == kc::Error::Success) return GGML_STATUS_SUCCESS;
    if (e == kc::Error::UnsupportedOperation)  // nothing was launched; the scheduler gave an unclaimed node
        GGML_ABORT("%s: %s\n", __func__, kcGetLastErrorDetail());
    GGML_LOG_ERROR("Kernelcore: graph_compute failed: %s\n", kcGetLastErrorDetail());
    return GGML_STATUS_FAILED;
}

const ggml_backend_i backend_i = {
    /* .get_name            = */ backend_get_name,
    /* .free                = */ backend_free,
    /* .set_tensor_async    = */ nullptr,
    /* .get_tensor_async    = */ nullptr,
    /* .set_tensor_2d_async = */ nullptr,
    /* .get_tensor_2d_async = */ nullptr,
    /* .cpy_tensor_async    = */ nullptr,
    /* .synchronize         = */ nullptr,
    /* .graph_plan_create   = */ nullptr,
    /* .graph_plan_free     = */ nullptr,
    /* .graph_plan_update   = */ nullptr,
    /* .graph_plan_compute  = */ nullptr,
    /* .graph_compute       = */ backend_graph_compute,
    /* .event_record        = */ nullptr,
    /* .event_wait          = */ nullptr,
    /* .graph_optimize      = */ nullptr,
};

ggml_guid_t backend_guid() {
    static ggml_guid guid = {0x6b, 0x63, 0x2d, 0x6d, 0x69, 0x33, 0x35, 0x35, 0x78, 0x2d, 0x67, 0x66, 0x78, 0x39, 0x35, 0x30};
    return &guid;
}

// ---- device -------------------------------------------------------------------------------------------------

const char * dev_get_name(ggml_backend_dev_t) { return "Kernelcore"; }
const char * dev_get_description(ggml_backend_dev_t) { return runtime().device; }

void dev_get_memory(ggml_backend_dev_t, size_t * free, size_t * total) {
    *free = *total = 0;
    if (runtime().ok && kcDeviceGetMemoryInfo(free, total) != kc::Error::Success) *free = *total = 0;
}

enum ggml_backend_dev_type dev_get_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_ACCEL; }

void dev_get_props(ggml_backend_dev_t dev, ggml_backend_dev_props * props) {
    props->name = dev_get_name(dev);
    props->description = dev_get_description(dev);
    props->type = dev_get_type(dev);
    dev_get_memory(dev, &props->memory_free, &props->memory_total);
    // Weights are copied into HBM, so a memory-mapped model file would stay resident as a second
    // copy: ask llama.cpp's auto load mode to read the file instead (not when nothing is claimed).
    const KcRuntime & rt = runtime();
    const bool claims_weights = rt.ok && !rt.cfg.disabled;
    props->caps = {
        /* .async                = */ false,
        /* .host_buffer          = */ false,
        /* .buffer_from_host_ptr = */ false,
        /* .events               = */ false,
        /* .mmap_support         = */ !claims_weights,
    };
}

ggml_backend_t dev_init_backend(ggml_backend_dev_t, const char *) { return ggml_backend_kernelcore_init(); }

ggml_backend_buffer_type_t dev_get_buffer_type(ggml_backend_dev_t) { return kc_buffer_type(); }

// llama.cpp's hook places the KV caches of CPU layers in this buffer type, so that attention runs here.
ggml_backend_buffer_type_t dev_get_host_buffer_type(ggml_backend_dev_t) {
    const KcRuntime & rt = runtime();
    return rt.ok && kcGgmlOffersKvBuffer(&rt.cfg) ? kc_host_buffer_type() : nullptr;
}

bool dev_supports_op(ggml_backend_dev_t, const ggml_tensor * op) {
    const KcRuntime & rt = runtime();
    if (!rt.ok) return false;
    Descs ds;
    const bool r = kcGgmlSupportsOp(&rt.cfg, ds.op(op)) != 0;
    static const bool dbg = std::getenv("GGML_KERNELCORE_DEBUG") != nullptr;
    if (dbg && op->op != GGML_OP_NONE && op->op != GGML_OP_VIEW && op->op != GGML_OP_RESHAPE && op->op != GGML_OP_PERMUTE)
        std::fprintf(stderr, "Kernelcore supports_op %s %s: %d\n", ggml_op_desc(op), op->name, r ? 1 : 0);
    return r;
}

// The kernels read HBM: inputs in other buffers (host memory) are copied here by the scheduler.
bool dev_supports_buft(ggml_backend_dev_t, ggml_backend_buffer_type_t buft) {
    return buft == kc_buffer_type() || buft == kc_host_buffer_type();
}

const ggml_backend_device_i device_i = {
    /* .get_name             = */ dev_get_name,
    /* .get_description      = */ dev_get_description,
    /* .get_memory           = */ dev_get_memory,
    /* .get_type             = */ dev_get_type,
    /* .get_props            = */ dev_get_props,
    /* .init_backend         = */ dev_init_backend,
    /* .get_buffer_type      = */ dev_get_buffer_type,
    /* .get_host_buffer_type = */ dev_get_host_buffer_type,
    /* .buffer_from_host_ptr = */ nullptr,
    /* .supports_op          = */ dev_supports_op,
    /* .supports_buft        = */ dev_supports_buft,
    /* .offload_op           = */ nullptr,
    /* .event_new            = */ nullptr,
    /* .event_free           = */ nullptr,
    /* .event_synchronize    = */ nullptr,
};

// ---- registry -----------------------------------------------------------------------------------------------

const char * reg_get_name(ggml_backend_reg_t) { return "Kernelcore"; }
size_t       reg_get_device_count(ggml_backend_reg_t) { return 1; }

ggml_backend_dev_t reg_get_device(ggml_backend_reg_t reg, size_t index) {
    GGML_ASSERT(index == 0);
    static ggml_backend_device device = {
        /* .iface   = */ device_i,
        /* .reg     = */ reg,
        /* .context = */ nullptr,
    };
    return &device;
}

void * reg_get_proc_address(ggml_backend_reg_t, const char *) { return nullptr; }

const ggml_backend_reg_i reg_i = {
    /* .get_name         = */ reg_get_name,
    /* .get_device_count = */ reg_get_device_count,
    /* .get_device       = */ reg_get_device,
    /* .get_proc_address = */ reg_get_proc_address,
};

ggml_backend_buffer_type_t kc_buffer_type() {
    static ggml_backend_buffer_type buft = {
        /* .iface   = */ buft_i,
        /* .device  = */ reg_get_device(ggml_backend_kernelcore_reg(), 0),
        /* .context = */ nullptr,
    };
    return &buft;
}

ggml_backend_buffer_type_t kc_host_buffer_type() {
    static ggml_backend_buffer_type buft = {
        /* .iface   = */ kv_buft_i,
        /* .device  = */ reg_get_device(ggml_backend_kernelcore_reg(), 0),
        /* .context = */ nullptr,
    };
    return &buft;
}

} // namespace

ggml_backend_t ggml_backend_kernelcore_init(void) {
    const KcRuntime & rt = runtime();
    if (!rt.ok) return nullptr;
    auto * ctx = new BackendCtx;
    ctx->profile = rt.cfg.profile;
    if (kcStreamCreate(&ctx->stream) != kc::Error::Success || kcGgmlBackendCreate(&ctx->core, &rt.cfg, ctx->stream) != kc::Error::Success) {
        GGML_LOG_ERROR("Kernelcore: backend init failed: %s\n", kcGetLastErrorDetail());
        delete ctx;
        return nullptr;
    }
    return new ggml_backend{
        /* .guid    = */ backend_guid(),
        /* .iface   = */ backend_i,
        /* .device  = */ reg_get_device(ggml_backend_kernelcore_reg(), 0),
        /* .context = */ ctx,
    };
}

bool ggml_backend_is_kc(ggml_backend_t backend) {
    return backend != nullptr && ggml_guid_matches(backend->guid, backend_guid());
}

ggml_backend_reg_t ggml_backend_kernelcore_reg(void) {
    static ggml_backend_reg reg = {
        /* .api_version = */ GGML_BACKEND_API_VERSION,
        /* .iface       = */ reg_i,
        /* .context     = */ nullptr,
    };
    return &reg;
}

GGML_BACKEND_DL_IMPL(ggml_backend_kernelcore_reg)
