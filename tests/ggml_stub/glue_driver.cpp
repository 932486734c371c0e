// Test entry points over the Kernelcore ggml glue (kernelcore_amd/ggml/src/ggml-kernelcore/), built
// with the ggml stand-in of this directory into libkcggml_glue_test.so and called from
// tests/test_ggml_glue.py and tests/test_gpu_ggml_glue.py through ctypes. Each drives the glue
// through its vtables, as ggml's scheduler and llama.cpp would: registry -> device -> buffer types,
// buffers and the backend.
#include <cstdio>
#include <cstring>
#include <unordered_map>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-impl.h"
#include "ggml-kernelcore.h"

#include <kernelcore/ggml_backend.h>

namespace {
ggml_backend_dev_t device() {
    ggml_backend_reg_t reg = ggml_backend_kernelcore_reg();
    return reg->iface.get_device(reg, 0);
}
ggml_backend_buffer_type_t buft(int kind) {  // 0: the weights' buffer type, 1: the KV caches'
    ggml_backend_dev_t dev = device();
    return kind == 0 ? dev->iface.get_buffer_type(dev) : dev->iface.get_host_buffer_type(dev);
}
void copy(char* dst, int n, const char* src) { std::snprintf(dst, size_t(n), "%s", src ? src : ""); }
ggml_tensor tensor2d(ggml_type type, int64_t ne0, int64_t ne1) {
    ggml_tensor t{};
    t.type = type;
    t.ne[0] = ne0, t.ne[1] = ne1, t.ne[2] = t.ne[3] = 1;
    const bool kq = type == GGML_TYPE_Q4_K || type == GGML_TYPE_Q6_K;
    t.nb[0] = kq ? (type == GGML_TYPE_Q4_K ? 144 : 210) : (type == GGML_TYPE_F16 ? 2 : 4);
    t.nb[1] = kq ? t.nb[0] * size_t(ne0 / 256) : t.nb[0] * size_t(ne0);
    t.nb[2] = t.nb[3] = t.nb[1] * size_t(ne1);
    return t;
}
ggml_op stub_op(int kc) {
    switch (kc) {
        case KC_GGML_OP_NONE: return GGML_OP_NONE;
        case KC_GGML_OP_RESHAPE: return GGML_OP_RESHAPE;
        case KC_GGML_OP_VIEW: return GGML_OP_VIEW;
        case KC_GGML_OP_PERMUTE: return GGML_OP_PERMUTE;
        case KC_GGML_OP_TRANSPOSE: return GGML_OP_TRANSPOSE;
        case KC_GGML_OP_MUL_MAT: return GGML_OP_MUL_MAT;
        case KC_GGML_OP_ADD: return GGML_OP_ADD;
        case KC_GGML_OP_RMS_NORM: return GGML_OP_RMS_NORM;
        case KC_GGML_OP_MUL: return GGML_OP_MUL;
        case KC_GGML_OP_ROPE: return GGML_OP_ROPE;
        case KC_GGML_OP_GLU: return GGML_OP_GLU;
        case KC_GGML_OP_SET_ROWS: return GGML_OP_SET_ROWS;
        case KC_GGML_OP_FLASH_ATTN_EXT: return GGML_OP_FLASH_ATTN_EXT;
        default: return GGML_OP_SOFT_MAX;
    }
}
}  // namespace

extern "C" {

// The registry and its device as llama.cpp reads them.
int kcgt_info(char* reg_name, char* dev_name, char* desc, int n, int* dev_count, int* dev_type, size_t* mem_free,
              size_t* mem_total, int* mmap_support, int* api_version, int* dl_reg) {
    ggml_backend_reg_t reg = ggml_backend_kernelcore_reg();
    copy(reg_name, n, reg->iface.get_name(reg));
    *dev_count = int(reg->iface.get_device_count(reg));
    ggml_backend_dev_t dev = device();
    ggml_backend_dev_props p{};
    dev->iface.get_props(dev, &p);
    copy(dev_name, n, p.name);
    copy(desc, n, p.description);
    *dev_type = int(p.type);
    *mem_free = p.memory_free;
    *mem_total = p.memory_total;
    *mmap_support = p.caps.mmap_support;
    *api_version = reg->api_version;
    extern ggml_backend_reg_t ggml_backend_init(void);
    *dl_reg = ggml_backend_init() == reg && dev->reg == reg;
    return 0;
}

// A buffer type (kind 0 weights, 1 KV): 0 when the device offers none.
int kcgt_buft(int kind, char* name, int n, size_t* alignment, int* is_host, int* supported) {
    ggml_backend_buffer_type_t b = buft(kind);
    if (!b) return 0;
    copy(name, n, b->iface.get_name(b));
    *alignment = b->iface.get_alignment(b);
    *is_host = b->iface.is_host(b);
    ggml_backend_dev_t dev = device();
    *supported = dev->iface.supports_buft(dev, b) && b->device == dev;
    return 1;
}

size_t kcgt_alloc_size(int kind, int type, int64_t ne0, int64_t ne1) {
    ggml_backend_buffer_type_t b = buft(kind);
    const ggml_tensor t = tensor2d(ggml_type(type), ne0, ne1);
    return b->iface.get_alloc_size(b, &t);
}

// supports_op of out = mul_mat(w, x): w (wtype, k x rows) in a buffer of kind wkind (-1: no buffer),
// x f32 k x ncols; out f32 rows x ncols.
int kcgt_supports_mul_mat(int wtype, int64_t k, int64_t rows, int64_t ncols, int wkind) {
    ggml_backend_buffer b{};
    b.buft = wkind >= 0 ? buft(wkind) : nullptr;
    ggml_tensor w = tensor2d(ggml_type(wtype), k, rows), x = tensor2d(GGML_TYPE_F32, k, ncols),
                y = tensor2d(GGML_TYPE_F32, rows, ncols);
    w.buffer = wkind >= 0 ? &b : nullptr;
    y.op = GGML_OP_MUL_MAT;
    y.src[0] = &w, y.src[1] = &x;
    ggml_backend_dev_t dev = device();
    return dev->iface.supports_op(dev, &y);
}

// One tensor (type, ne0 x ne1) at the start of a fresh buffer of kind: set_tensor(data, whole), read
// back; memset_tensor(value, off, size), read back; clear(clear_value), read back; then a device copy
// (cpy_tensor) into a second tensor of the same buffer, read back. Returns 0, or -1 when the buffer
// could not be allocated, -2 when cpy_tensor declined.
int kcgt_buffer_ops(int kind, int type, int64_t ne0, int64_t ne1, const void* data, void* after_set, int value,
                    size_t off, size_t size, void* after_memset, int clear_value, void* after_clear, void* after_cpy) {
    ggml_backend_buffer_type_t b = buft(kind);
    ggml_tensor t = tensor2d(ggml_type(type), ne0, ne1), u = t;
    const size_t nbytes = ggml_nbytes(&t), alloc = b->iface.get_alloc_size(b, &t);
    const size_t align = b->iface.get_alignment(b), second = (alloc + align - 1) / align * align;
    ggml_backend_buffer_t buf = b->iface.alloc_buffer(b, second + alloc);
    if (!buf) return -1;
    char* base = static_cast<char*>(buf->iface.get_base(buf));
    t.buffer = u.buffer = buf;
    t.data = base;
    u.data = base + second;
    buf->iface.set_tensor(buf, &t, data, 0, nbytes);
    buf->iface.get_tensor(buf, &t, after_set, 0, nbytes);
    buf->iface.memset_tensor(buf, &t, uint8_t(value), off, size);
    buf->iface.get_tensor(buf, &t, after_memset, 0, nbytes);
    buf->iface.set_tensor(buf, &t, data, 0, nbytes);
    int rc = 0;
    if (buf->iface.cpy_tensor(buf, &t, &u)) buf->iface.get_tensor(buf, &u, after_cpy, 0, nbytes);
    else rc = -2;
    buf->iface.clear(buf, uint8_t(clear_value));
    buf->iface.get_tensor(buf, &t, after_clear, 0, nbytes);
    buf->iface.free_buffer(buf);
    delete buf;
    return rc;
}

// graph_compute of nodes[0..n_nodes) given as kcGgmlTensor descriptors (kernelcore_amd/ggml_graph.py),
// each turned into a ggml tensor: the same data, shapes, op_params, flags; tensors in the weights / KV
// buffers placed in a buffer of the glue's buffer types; view_base[i] (parallel to tensors[]) the
// descriptor a view views. tensors[0..n_tensors) must hold every node and every src they read. Then
// ggml_backend_kernelcore_init() and graph_compute through the backend's vtable, as ggml's scheduler
// calls it. Returns the ggml_status, or -10 when no backend could be made.
int kcgt_graph_compute(const kcGgmlTensor* const* tensors, const kcGgmlTensor* const* view_base, int n_tensors,
                       const kcGgmlTensor* const* nodes, int n_nodes, int repeat) {
    ggml_backend_buffer weights{}, kv{};
    weights.buft = buft(0);
    kv.buft = buft(1);
    std::vector<ggml_tensor> ts(static_cast<size_t>(n_tensors));
    std::unordered_map<const kcGgmlTensor*, ggml_tensor*> map;
    for (int i = 0; i < n_tensors; ++i) map[tensors[i]] = &ts[size_t(i)];
    for (int i = 0; i < n_tensors; ++i) {
        const kcGgmlTensor& k = *tensors[i];
        ggml_tensor& t = ts[size_t(i)];
        t = ggml_tensor{};
        t.type = ggml_type(k.type);
        t.op = stub_op(k.op);
        for (int d = 0; d < 4; ++d) t.ne[d] = k.ne[d], t.nb[d] = k.nb[d];
        std::memcpy(t.op_params, k.op_params, sizeof k.op_params);
        t.data = k.data;
        t.flags = (k.compute ? GGML_TENSOR_FLAG_COMPUTE : 0) | (k.output ? GGML_TENSOR_FLAG_OUTPUT : 0);
        t.buffer = k.buffer == KC_GGML_BUFFER_WEIGHTS ? &weights : k.buffer == KC_GGML_BUFFER_KV ? &kv : nullptr;
        for (int s = 0; s < 5; ++s)
            if (k.src[s]) {
                auto it = map.find(k.src[s]);
                if (it == map.end()) return -11;
                t.src[s] = it->second;
            }
        if (view_base[i]) {
            auto it = map.find(view_base[i]);
            if (it == map.end()) return -12;
            t.view_src = it->second;
            t.view_offs = size_t(static_cast<const char*>(k.data) - static_cast<const char*>(view_base[i]->data));
        }
    }
    std::vector<ggml_tensor*> gn(static_cast<size_t>(n_nodes));
    std::vector<int32_t> uses(static_cast<size_t>(n_nodes));
    for (int i = 0; i < n_nodes; ++i) {
        gn[size_t(i)] = map.at(nodes[i]);
        uses[size_t(i)] = nodes[i]->uses;
    }
    ggml_cgraph g{n_nodes, n_nodes, 0, gn.data(), nullptr, uses.data()};
    ggml_backend_t be = ggml_backend_kernelcore_init();
    if (!be || !ggml_backend_is_kc(be)) return -10;
    int st = GGML_STATUS_SUCCESS;
    for (int r = 0; r < repeat && st == GGML_STATUS_SUCCESS; ++r) st = be->iface.graph_compute(be, &g);
    be->iface.free(be);
    return st;
}

}  // extern "C"
