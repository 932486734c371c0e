// ggml_backend.cpp -- the compute side of the reference's ggml backend over kcGgmlTensor
// descriptors (integrations/llama.cpp/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp):
//   - kcGgmlSupportsOp restates dev_supports_op_impl (:902-957) with weight_shape_ok (:103-109),
//     in_kv_buffer / f16_rows / flash_attn_ok (:865-891);
//   - kcGgmlGraphCompute restates backend_graph_compute (:706-792) -- the node walk and its fusion
//     patterns -- and the op launchers rms_norm / mul / add / rope / swiglu / set_rows / flash_attn
//     (:597-699), over the MUL_MAT recording of mul_mat.cpp (mul_mat_impl, quantized_input,
//     fused_norm, fused_swiglu), on a HIP stream.
// The rules and the kernels each op launches are the reference's (they are the backend's
// behaviour); the recording is this device's: a planning pass sizes the scratch and names the
// launches first, then the launches are made eagerly or captured once into a HIP graph that later
// calls with the same nodes launch again.
//
// ggml's own helpers that the reference calls (ggml_is_contiguous, ggml_nrows, ggml_nelements,
// ggml_are_same_shape, ggml_is_empty, ggml_can_fuse) belong to ggml, which the reference tree does
// not hold; they are restated below from their definitions in ggml (ggml.c: ggml_is_contiguous_n;
// ggml-impl.h: ggml_can_fuse_ext, ggml_node_has_n_uses).
#include <algorithm>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iterator>
#include <map>
#include <new>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "internal.hpp"
#include "kdecode.hpp"
#include "kernelcore/ggml_backend.h"
#include "kernelcore/llm_kernels.h"
#include "launch.hpp"
#include "model_kernels.hpp"
#include "mul_mat_internal.hpp"

using T = kcGgmlTensor;

namespace kcamd::ggml {
// The structure of a node list as its signature reads it (each src slot a node index, a leaf -- a
// tensor outside the list, numbered in first-seen order -- or none), kept while the same node array
// with the same src links comes back, so that a call that launches the kept graph again spends its
// host time on the fields alone.
struct SigShape {
    std::vector<const kcGgmlTensor*> nodes;
    std::vector<const kcGgmlTensor*> srcs;  // per node, its 5 src links
    std::vector<int64_t> ref;               // per node and src slot: index >= 0, -1 none, -2 - leaf id
    std::vector<const kcGgmlTensor*> leaves;
};
}  // namespace kcamd::ggml

struct kcGgmlBackend_st {
    kcGgmlConfig cfg{};
    kcStream_t stream = nullptr;
    kcMulMatRecording_st rec;
    std::map<int, float*> ones;  // device float[n] of 1.0f: rms_norm without a weight, rope without factors
    kcGraph_t graph = nullptr;   // the kept graph, the signature of its nodes, the scratch it points into
    std::vector<uint64_t> sig;
    kcamd::ggml::SigShape shape;     // the last call's node structure, and its signature
    std::vector<uint64_t> sig_now;
    unsigned graph_gen = 0;
    unsigned graph_options = 0;  // the kernel options' generation the graph was recorded under
    long long graph_launches = 0;
    kcGgmlStats stats{};
    // profile = 2: the launch timer of the calls and the device times summed per launch name
    kcamd::LaunchTimer timer;
    std::map<std::string, std::pair<long long, double>> per_kernel;
};

namespace {

using E = kcError_t;
constexpr E ok = kc::Error::Success;

E bad(const char* why) {
    kcamd::setDetail("ggml backend: %s", why);
    return kc::Error::InvalidValue;
}

// ---- ggml's tensor predicates ----------------------------------------------------------------

// Bytes per block and values per block of the types the rules meet; 0 bytes for any other type.
size_t typeSize(int type, int64_t* blck) {
    *blck = 1;
    switch (type) {
        case KC_GGML_TYPE_F32: return 4;
        case KC_GGML_TYPE_F16: return 2;
        case KC_GGML_TYPE_I32: return 4;
        case KC_GGML_TYPE_I64: return 8;
        case KC_GGML_TYPE_Q4_K: *blck = 256; return 144;
        case KC_GGML_TYPE_Q6_K: *blck = 256; return 210;
        default: return 0;
    }
}

// ggml_is_contiguous: elements packed in each row, then every dimension of more than one element
// packed after the previous ones (dimensions of one element take any stride).
bool contiguous(const T* t) {
    int64_t blck = 1;
    size_t next = typeSize(t->type, &blck);
    if (!next) return false;
    if (t->ne[0] != blck && t->nb[0] != next) return false;
    next *= size_t(t->ne[0] / blck);
    for (int i = 1; i < 4; ++i)
        if (t->ne[i] != 1) {
            if (t->nb[i] != next) return false;
            next *= size_t(t->ne[i]);
        }
    return true;
}

int64_t nrows(const T* t) { return t->ne[1] * t->ne[2] * t->ne[3]; }
int64_t nelements(const T* t) { return t->ne[0] * nrows(t); }
bool sameShape(const T* a, const T* b) {
    for (int i = 0; i < 4; ++i)
        if (a->ne[i] != b->ne[i]) return false;
    return true;
}
bool empty(const T* t) {
    for (int i = 0; i < 4; ++i)
        if (t->ne[i] == 0) return true;
    return false;
}
float paramF32(const T* t, int i) {
    float v;
    std::memcpy(&v, &t->op_params[i], sizeof v);
    return v;
}
bool f32c(const T* t) { return t && t->type == KC_GGML_TYPE_F32 && contiguous(t); }
// v is one contiguous f32 row as long as x's rows (a norm weight)
bool rowVectorOf(const T* v, const T* x) {
    return v && v->type == KC_GGML_TYPE_F32 && contiguous(v) && v->ne[0] == x->ne[0] && nrows(v) == 1;
}

// ggml_can_fuse: nodes[i..i+n) carry ops[0..n) in order; each but the last has exactly one use and
// is neither a view nor a graph output; each after the first reads the one before it and has its
// shape.
bool canFuse(const T* const* nodes, int n_nodes, int i, const int* ops, int n) {
    for (int j = 0; j < n; ++j) {
        if (i + j >= n_nodes) return false;
        const T* node = nodes[i + j];
        if (node->op != ops[j]) return false;
        if (j < n - 1 && (node->uses != 1 || node->view || node->output)) return false;
        if (j > 0) {
            const T* prev = nodes[i + j - 1];
            if (node->src[0] != prev && node->src[1] != prev) return false;
            if (!sameShape(node, prev)) return false;
        }
    }
    return true;
}

// ---- supports_op -----------------------------------------------------------------------------

bool weightShapeOk(const T* w) {  // K-quants (super-blocks of 256) and fp16, in 8-row groups
    const bool kq = (w->type == KC_GGML_TYPE_Q4_K || w->type == KC_GGML_TYPE_Q6_K) && w->ne[0] % 256 == 0;
    const bool f16 = w->type == KC_GGML_TYPE_F16 && w->ne[0] % 2 == 0;
    return (kq || f16) && w->ne[2] == 1 && w->ne[3] == 1 && w->ne[1] % 8 == 0 && w->ne[0] <= INT32_MAX &&
           w->ne[1] <= INT32_MAX && contiguous(w);
}

bool inKv(const T* t) { return t->buffer == KC_GGML_BUFFER_KV; }
bool f16Rows(const T* t) {  // fp16, rows and heads at 32-bit word strides
    return t->type == KC_GGML_TYPE_F16 && t->nb[0] == 2 && t->nb[1] % 4 == 0 && t->nb[2] % 4 == 0 && t->ne[3] == 1 &&
           t->nb[1] / 4 <= INT32_MAX && t->nb[2] / 4 <= INT32_MAX;
}

// flash_attn_ok, and the size limits of the attention kernels (beyond them the reference's kernels
// refuse the launch; here the op is not claimed, so the scheduler places it elsewhere).
// A batch attention flashAttn runs on the matrix cores, reading ggml's mask (no score matrix in
// scratch, so the 2^24-value limit below does not apply): a mask, more than 8 query tokens, the
// decoder caches' layout (heads D / 2 words apart in K and V rows of one stride, q and out
// [N][H][D]) and a shape the kernel takes.
bool maskedAttn(const T* op) {
    const T *q = op->src[0], *k = op->src[1], *v = op->src[2], *mask = op->src[3];
    if (!mask || q->ne[1] <= 8 || k->ne[0] > INT32_MAX || k->ne[1] > INT32_MAX || q->ne[1] > INT32_MAX) return false;
    const int D = int(k->ne[0]), H = int(q->ne[2]), Hkv = int(k->ne[2]), N = int(q->ne[1]), T = int(k->ne[1]);
    const kcamd::AttnShape as{N, H, Hkv, D, int(q->nb[1] / 4), int(k->nb[1] / 4), T, 0, paramF32(op, 0)};
    return kcamd::attnMaskedSupports(as) && q->nb[2] / 4 == uint64_t(D) && q->nb[1] / 4 == uint64_t(H) * D &&
           k->nb[2] / 4 == uint64_t(D / 2) && v->nb[2] / 4 == uint64_t(D / 2) && v->nb[1] == k->nb[1] &&
           mask->nb[1] / 4 > 0;
}

bool flashAttnOk(const kcGgmlConfig& c, const T* op) {
    const T* q = op->src[0];
    const T* k = op->src[1];
    const T* v = op->src[2];
    const T* mask = op->src[3];
    if (!q || !k || !v) return false;
    if (op->src[4] || q->ne[1] > c.attn_tokens) return false;  // no sinks
    if (paramF32(op, 1) != 0.0f || paramF32(op, 2) != 0.0f) return false;  // no ALiBi, no softcap
    if (!inKv(k) || !inKv(v) || !f16Rows(k) || !f16Rows(v)) return false;
    const int64_t D = k->ne[0];
    if (v->ne[0] != D || q->ne[0] != D || D % 8 || k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2] || k->ne[2] <= 0 ||
        q->ne[2] % k->ne[2] || q->ne[3] != 1 || k->ne[1] <= 0 || k->ne[1] > INT32_MAX)
        return false;
    if (q->type != KC_GGML_TYPE_F32 || q->nb[0] != 4 || q->nb[1] % 4 || q->nb[2] % 4) return false;
    if (!f32c(op) || op->ne[0] != D || op->ne[1] != q->ne[2] || op->ne[2] != q->ne[1] || op->ne[3] != 1) return false;
    if (mask && (mask->type != KC_GGML_TYPE_F16 || mask->nb[0] != 2 || mask->nb[1] % 4 || mask->ne[0] < k->ne[1] ||
                 mask->ne[1] < q->ne[1] || mask->ne[2] != 1 || mask->ne[3] != 1))
        return false;
    const int64_t tp = (k->ne[1] + 7) / 8 * 8, rows = q->ne[2] * q->ne[1];
    if (rows * D >= (int64_t(1) << 24) || q->nb[2] / 4 < uint64_t(D)) return false;
    return rows * tp < (int64_t(1) << 24) || maskedAttn(op);
}

bool supports(const kcGgmlConfig& c, const T* op) {
    if (!op || c.disabled) return false;
    const T* s0 = op->src[0];
    const T* s1 = op->src[1];
    switch (op->op) {
        case KC_GGML_OP_NONE:
        case KC_GGML_OP_RESHAPE:
        case KC_GGML_OP_VIEW:
        case KC_GGML_OP_PERMUTE:
        case KC_GGML_OP_TRANSPOSE:
            return true;
        case KC_GGML_OP_MUL_MAT:  // the weight in this backend's buffers (repacked), any batch size
            return s0 && s1 && s0->buffer == KC_GGML_BUFFER_WEIGHTS && weightShapeOk(s0) && f32c(s1) &&
                   s1->ne[0] == s0->ne[0] && f32c(op) && op->ne[0] == s0->ne[1] && nrows(op) == nrows(s1);
        default:
            break;
    }
    if (c.matmul_only) return false;
    switch (op->op) {
        case KC_GGML_OP_RMS_NORM:
            return f32c(s0) && f32c(op) && sameShape(s0, op);
        case KC_GGML_OP_ADD:
            return f32c(s0) && f32c(s1) && f32c(op) && sameShape(s0, s1) && sameShape(s0, op);
        case KC_GGML_OP_MUL:  // s1 broadcast over the rows of s0 (rows a multiple of 8 wide), or same-shape
            return f32c(s0) && f32c(s1) && f32c(op) && sameShape(s0, op) &&
                   ((rowVectorOf(s1, s0) && s0->ne[0] % 8 == 0) || (sameShape(s0, s1) && nelements(s0) % 8 == 0));
        case KC_GGML_OP_ROPE: {
            const int32_t* p = op->op_params;
            const T* ff = op->src[2];
            return s0 && (p[2] == 0 /* NORM */ || p[2] == KC_GGML_ROPE_TYPE_NEOX) && p[1] == s0->ne[0] &&
                   paramF32(op, 6) == 1.0f && paramF32(op, 7) == 0.0f && paramF32(op, 8) == 1.0f && p[15] == 0 &&
                   f32c(s0) && f32c(op) && sameShape(s0, op) && s0->ne[0] % 16 == 0 && s0->ne[3] == 1 && s1 &&
                   s1->type == KC_GGML_TYPE_I32 && contiguous(s1) && s1->ne[0] == s0->ne[2] &&
                   (!ff || (f32c(ff) && ff->ne[0] >= s0->ne[0] / 2));
        }
        case KC_GGML_OP_SET_ROWS:  // f32 rows stored as fp16 at i64 row indices of a KV-buffer tensor
            return c.attn && s0 && s1 && inKv(op) && op->type == KC_GGML_TYPE_F16 && op->nb[0] == 2 &&
                   op->nb[1] % 4 == 0 && op->ne[2] == 1 && op->ne[3] == 1 && op->ne[1] <= INT32_MAX &&
                   s0->type == KC_GGML_TYPE_F32 && s0->nb[0] == 4 && s0->nb[1] % 4 == 0 && s0->ne[0] == op->ne[0] &&
                   s0->ne[0] % 16 == 0 && s0->ne[2] == 1 && s0->ne[3] == 1 && s1->type == KC_GGML_TYPE_I64 &&
                   contiguous(s1) && s1->ne[0] == s0->ne[1] && s1->ne[1] == 1 && s1->ne[2] == 1 && s1->ne[3] == 1;
        case KC_GGML_OP_FLASH_ATTN_EXT:
            return c.attn && flashAttnOk(c, op);
        case KC_GGML_OP_GLU:
            return op->op_params[0] == KC_GGML_GLU_OP_SWIGLU && op->op_params[1] == 0 && f32c(s0) && f32c(s1) &&
                   f32c(op) && sameShape(s0, s1) && sameShape(s0, op);
        default:
            return false;
    }
}

// ---- the graph walk ---------------------------------------------------------------------------

// One pass over a graph's nodes: a plan (dry recording, no backend) or the launches.
struct Pass {
    const kcGgmlConfig& cfg;
    kcMulMatRecording_st& rec;
    kcGgmlBackend_st* be;            // null in a plan
    std::vector<int>* ones_wanted;   // a plan: the lengths of the 1.0f arrays the launches read
    bool capturing;                  // launches recorded into a graph (MUL_MAT groups run concurrently)
    // Batch products whose second K half (partial sums) is not yet added: the ADD that reads one adds
    // it inside its fused norm; any other reader, and the end of the walk, adds it first. A product
    // marked views (a Q6_K matrix split beside Q4_K ones) keeps its half past the views of it: the
    // fused RoPE / cache store takes v's along, any other reader adds it to the whole product.
    struct Pending {
        const T* t;
        const float* h;
        bool views;
    };
    std::vector<Pending> pending{};
    // The summaries the pass's masked attention launches read (mask_summary_kernel), one per mask
    // tensor: every layer's attention reads the same mask, whose values stay as they are while a
    // later node still reads it (ggml reuses a tensor's memory only after its last reader). An entry
    // holds while the scratch it lies in does (gen).
    struct MaskSum {
        const T* mask;
        int N, T_keys;
        unsigned gen;
        int* sum;
    };
    std::vector<MaskSum> masks{};
};

const float* onesOf(Pass& p, int n) {
    if (!p.be) {
        p.ones_wanted->push_back(n);
        return reinterpret_cast<const float*>(uintptr_t(256));  // a plan never dereferences it
    }
    const auto it = p.be->ones.find(n);
    return it == p.be->ones.end() ? nullptr : it->second;
}

E launch(Pass& p, const char* kernel, const void* args) { return kcamd::mulmat::launch(p.rec, kernel, args); }

E marker(Pass& p, const char* m) {
    if (p.rec.trace) {
        try {
            p.rec.trace->push_back(m);
        } catch (...) {
            return kc::Error::OutOfMemory;
        }
    }
    return ok;
}

const float* f32(const T* t) { return static_cast<const float*>(t->data); }
float* f32w(const T* t) { return static_cast<float*>(t->data); }

// The tensor whose values t holds as a MUL_MAT reads them: t, or through RESHAPE / VIEW nodes that
// keep its memory and its elements packed, the tensor they view. The quantized inputs are cached by
// this key, as the reference caches them by tensor (:323): ggml's allocator gives a tensor's memory to
// a later tensor once the first is dead, so a data pointer does not name one tensor's values.
const T* keyOf(const T* t) {
    while (t && (t->op == KC_GGML_OP_RESHAPE || t->op == KC_GGML_OP_VIEW) && t->src[0] &&
           t->data == t->src[0]->data && nelements(t) == nelements(t->src[0]) && contiguous(t) &&
           contiguous(t->src[0]))
        t = t->src[0];
    return t;
}

kcMulMatNode mulMatNode(const T* dst) {
    const T* w = dst->src[0];
    const T* x = dst->src[1];
    return kcMulMatNode{w->type, w->data, int(w->ne[1]), int(w->ne[0]), f32(x), (long long)nrows(x), x->nb[1], f32w(dst)};
}

E mulMat(Pass& p, const T* dst) {
    kcMulMatPlan plan{};
    return kcamd::mulmat::mulMat(p.rec, mulMatNode(dst), plan, keyOf(dst->src[1]));
}

E mulMatInput(Pass& p, const T* dst) {
    kcMulMatPlan plan{};
    return kcamd::mulmat::mulMatInput(p.rec, mulMatNode(dst), plan, keyOf(dst->src[1]));
}

// RMS_NORM, with the weight of a following MUL when given (rms_norm, :597-606)
E rmsNorm(Pass& p, const T* norm, const float* weight, const T* out) {
    const T* x = norm->src[0];
    const int n = int(x->ne[0]), rows = int(nrows(x));
    const float* w = weight ? weight : onesOf(p, n);
    if (!w) return kc::Error::InternalError;
    const kcRmsNormArgs a{f32(x), w, f32w(out), n, rows, paramF32(norm, 0)};
    return launch(p, "rms_norm", &a);
}

E mul(Pass& p, const T* dst) {  // by a row vector (broadcast) or elementwise (:612-619)
    const T* a = dst->src[0];
    const T* b = dst->src[1];
    const int count = int(nelements(a));
    const int n = rowVectorOf(b, a) ? int(a->ne[0]) : count;
    const kcMulRowsArgs m{f32(a), f32(b), f32w(dst), n, count};
    return launch(p, "mul_rows", &m);
}

E add(Pass& p, const T* dst) {  // :621-626
    const kcVectorAddArgs a{f32(dst->src[0]), f32(dst->src[1]), f32w(dst), int(nelements(dst))};
    return launch(p, "vector_add", &a);
}

E rope(Pass& p, const T* dst) {  // :628-639
    const T* x = dst->src[0];
    const int hd = int(x->ne[0]), nh = int(x->ne[1]), nt = int(x->ne[2]), pairs = hd / 2;
    const float* ff = dst->src[2] ? f32(dst->src[2]) : onesOf(p, pairs);
    if (!ff) return kc::Error::InternalError;
    const bool neox = (dst->op_params[2] & KC_GGML_ROPE_TYPE_NEOX) != 0;
    const kcRopeGgmlArgs a{f32(x), f32w(dst), static_cast<const int*>(dst->src[1]->data), ff, nullptr, hd, nh, nt,
                           std::log2(paramF32(dst, 5)), neox};
    return launch(p, "rope_ggml", &a);
}

E swiglu(Pass& p, const T* dst) {  // :641-646
    const kcSiluMulArgs a{f32(dst->src[0]), f32(dst->src[1]), f32w(dst), int(nelements(dst))};
    return launch(p, "silu_mul", &a);
}

// The pending second K half of product t (null if none), now the caller's to add.
const float* takePending(Pass& p, const T* t) {
    for (auto it = p.pending.begin(); it != p.pending.end(); ++it)
        if (it->t == t) {
            const float* h = it->h;
            p.pending.erase(it);
            return h;
        }
    return nullptr;
}
bool viewOp(int op) {
    return op == KC_GGML_OP_RESHAPE || op == KC_GGML_OP_VIEW || op == KC_GGML_OP_PERMUTE ||
           op == KC_GGML_OP_TRANSPOSE;
}
// The tensor a chain of views of t looks into (t itself when t is no view).
const T* viewBase(const T* t) {
    while (t && t->view && viewOp(t->op) && t->src[0]) t = t->src[0];
    return t;
}
// The pending half of the product a view t (or t itself) looks into, when that product keeps its
// half past views; *base = the product.
const float* takeViewPending(Pass& p, const T* t, const T** base) {
    const T* b = viewBase(t);
    for (auto it = p.pending.begin(); it != p.pending.end(); ++it)
        if (it->t == t || (it->views && it->t == b)) {
            const float* h = it->h;
            *base = it->t;
            p.pending.erase(it);
            return h;
        }
    return nullptr;
}
// t += h (the product's two K halves, fl(y1 + y2) as the by-name launch's add)
E addHalf(Pass& p, const T* t, const float* h) {
    const kcVectorAddArgs a{f32(t), h, f32w(t), int(nelements(t))};
    return launch(p, "vector_add", &a);
}
// Adds the pending half of t, if any, before something reads t (a view node, which reads no data,
// leaves the halves that are kept past views; another reader of a view of such a product adds the
// half to the whole product).
E settle(Pass& p, const T* t, bool view_node = false) {
    if (!t || p.pending.empty()) return ok;
    for (auto it = p.pending.begin(); it != p.pending.end(); ++it)
        if (it->t == t && !(view_node && it->views)) {
            const float* h = it->h;
            p.pending.erase(it);
            return addHalf(p, t, h);
        }
    if (view_node) return ok;
    const T* base = nullptr;
    if (const float* h = takeViewPending(p, t, &base)) return addHalf(p, base, h);
    return ok;
}

// [ADD +] RMS_NORM + MUL, the result also quantized for the MUL_MATs that read it (:502-530).
// Beyond the fused kernels' 2^24 values: the ADD and a weighted rms_norm.
E fusedNorm(Pass& p, const T* addNode, const T* norm, const T* mulNode) {
    const T* x = norm->src[0];
    const int64_t n = x->ne[0], rows = nrows(x);
    // an ADD operand with a pending second K half: it becomes b, its half b2 (x = a + (b + b2))
    const T* a = addNode ? addNode->src[0] : nullptr;
    const T* b = addNode ? addNode->src[1] : nullptr;
    const float* b2 = nullptr;
    if (addNode && a == b) {  // x + x: both operands need the half, so it is added first
        if (E e = settle(p, a); e != ok) return e;
    } else if (addNode) {
        if (const float* h = takePending(p, a)) {
            std::swap(a, b);
            b2 = h;
        } else {
            b2 = takePending(p, b);
        }
        if (E e = settle(p, a); e != ok) return e;  // (both operands pending: one is added first)
        if (b2 && (n * rows >= (int64_t(1) << 24) || !kcamd::mulmat::fusesHalf(p.rec, int(n)))) {
            if (E e = addHalf(p, b, b2); e != ok) return e;
            b2 = nullptr;
        }
    }
    if (n * rows >= (int64_t(1) << 24)) {
        if (addNode)
            if (E e = add(p, addNode); e != ok) return e;
        return rmsNorm(p, norm, f32(mulNode->src[1]), mulNode);
    }
    const kcMulMatNormNode nn{addNode ? f32(a) : nullptr, addNode ? f32(b) : nullptr, f32w(x), f32(mulNode->src[1]),
                              f32w(mulNode), int(n), int(rows), paramF32(norm, 0)};
    kcMulMatPlan plan{};
    return kcamd::mulmat::fusedNorm(p.rec, nn, plan, b2, mulNode);
}

// SWIGLU with the result also quantized for the down projection (:533-545); n % 256 == 0.
E fusedSwiglu(Pass& p, const T* dst) {
    const int64_t n = dst->ne[0], cols = nrows(dst);
    if (n * cols >= (int64_t(1) << 24)) return swiglu(p, dst);
    const kcMulMatSwigluNode sn{f32(dst->src[0]), f32(dst->src[1]), f32w(dst), int(n), int(cols)};
    kcMulMatPlan plan{};
    return kcamd::mulmat::fusedSwiglu(p.rec, sn, plan, dst);
}

// ---- fusions beyond the reference's --------------------------------------------------------------
// No reference counterpart (option ggml_extra_fusions = 1 keeps the reference's launches): where the
// reference launches one matvec per MUL_MAT, 2-3 MUL_MATs of one input column run as one launch
// whose rows each take the reference matvec's sum, from the same per-32 slot; gate and up followed
// by SWIGLU also apply silu(gate) * up and quantize it per 32 into the slot the down MUL_MAT reads;
// ROPE of q and k and the two SET_ROWS into the caches run as one launch; a MUL_MAT whose one use is
// an ADD writes the ADD's result (residual + each row's sum); RMS_NORM + MUL whose one use is a
// group of MUL_MATs (q / k / v, gate / up + SWIGLU) is computed in the group's launch (the norm as
// add_norm_q8_f's, per workgroup).

// A launch of this build's own kernels (no by-name entry), named in the trace like the others.
template <class F>
E direct(Pass& p, const char* name, F&& fn) {
    if (E e = marker(p, name); e != ok) return e;
    if (p.rec.dry) return ok;
    return kcamd::mulmat::timed(p.rec, name, fn);
}

// While it lives, launches are timed under the weight shape of MUL_MAT mm ("rows x k"), as
// GGML_KERNELCORE_PROFILE=2 names them (ggml-kernelcore.cpp:549-553).
struct ShapeTag {
    kcamd::LaunchTimer* t;
    ShapeTag(const Pass& p, const T* mm) : t(p.rec.timer) {
        if (t) t->tag = std::to_string(mm->src[0]->ne[1]) + "x" + std::to_string(mm->src[0]->ne[0]);
    }
    ~ShapeTag() {
        if (t) t->tag.clear();
    }
};

bool kquant(const T* w) { return w->type == KC_GGML_TYPE_Q4_K || w->type == KC_GGML_TYPE_Q6_K; }
bool computed(const T* t) { return t->compute && !empty(t); }
bool noop(const T* t) {
    return t->op == KC_GGML_OP_NONE || t->op == KC_GGML_OP_RESHAPE || t->op == KC_GGML_OP_VIEW ||
           t->op == KC_GGML_OP_PERMUTE || t->op == KC_GGML_OP_TRANSPOSE;
}
int nextWork(const T* const* nodes, int n, int j) {  // the next node with work after no-op nodes
    while (j < n && noop(nodes[j])) ++j;
    return j;
}

// The bytes from t's data pointer to the end of its last element (0 when it has none).
size_t spanBytes(const T* t) {
    int64_t blck = 1;
    const size_t es = typeSize(t->type, &blck);
    if (!es || empty(t)) return 0;
    size_t end = es + size_t(t->ne[0] / blck - 1) * t->nb[0];
    for (int d = 1; d < 4; ++d) end += size_t(t->ne[d] - 1) * t->nb[d];
    return end;
}
bool overlaps(const T* a, const T* b) {
    if (!a || !b) return false;
    const char* pa = static_cast<const char*>(a->data);
    const char* pb = static_cast<const char*>(b->data);
    const size_t na = spanBytes(a), nb = spanBytes(b);
    return na && nb && pa < pb + nb && pb < pa + na;
}
// Whether anything outside fused[0..nf) needs t's values: t is a graph output, or a node reads it
// (itself or through no-op views of t) that is not one of them.
bool readBeyond(const T* t, const T* const* nodes, int n, const T* const* fused, int nf) {
    if (t->output) return true;
    for (int j = 0; j < n; ++j) {
        const T* r = nodes[j];
        if (std::find(std::begin(r->src), std::end(r->src), t) == std::end(r->src)) continue;
        if (std::find(fused, fused + nf, r) != fused + nf) continue;
        if (noop(r) && !readBeyond(r, nodes, n, fused, nf)) continue;
        return true;
    }
    return false;
}

// MUL_MATs mm[0..g) of the one-column input x through one decode matvec with epilogue epi
// (prologue pro: the input's per-32 slot, or the norm of the row the input is the norm of)
bool decodeMatvecOk(const T* x, const T* const* mm, int g, int epi, int tpw, int pro = kcamd::kProSlot) {
    if (g < 1 || g > 3 || !f32c(x) || nrows(x) != 1 || x->ne[0] % 256 || x->ne[0] > INT_MAX) return false;
    for (int j = 0; j < g; ++j)
        if (!kquant(mm[j]->src[0]) || mm[j]->src[0]->ne[0] != x->ne[0] || !f32c(mm[j])) return false;
    return kcamd::planDecodeMatvec(pro, epi, int(x->ne[0]), tpw).nw > 0;
}

// The per-32 slot of the group's input (the fused norm's, or quantized now) as DmvArgs.
E slotArgs(Pass& p, const T* mm0, kcamd::DmvArgs& a) {
    const T* x = mm0->src[1];
    const int k = int(x->ne[0]);
    if (E e = mulMatInput(p, mm0); e != ok) return e;
    int* q = kcamd::mulmat::inputSlot(p.rec, keyOf(x), 1, k, false);
    if (!q) return kc::Error::InternalError;
    a.k = k;
    a.xq = q;
    a.xd = reinterpret_cast<const float*>(q + k / 32 * 8);
    return ok;
}

kcamd::DmvPart dmvPart(const T* mm, float* y) {
    const T* w = mm->src[0];
    return kcamd::DmvPart{w->data, y, int(w->ne[1]), w->type == KC_GGML_TYPE_Q6_K ? 1 : 0, 0, 0};
}

// nodes[i] = a one-column K-quant MUL_MAT (one use, not a view or an output) and the next node with
// work the ADD of it and a residual of its shape: *add = that ADD's index.
bool matvecAddOk(const T* const* nodes, int n, int i, int* add) {
    const T* mm = nodes[i];
    if (mm->uses != 1 || mm->view || mm->output) return false;
    const int j = nextWork(nodes, n, i + 1);
    if (j >= n || nodes[j]->op != KC_GGML_OP_ADD || !computed(nodes[j])) return false;
    const T* ad = nodes[j];
    const T* r = ad->src[0] == mm ? ad->src[1] : (ad->src[1] == mm ? ad->src[0] : nullptr);
    if (!r || r == mm || !f32c(r) || !sameShape(r, mm) || !f32c(ad)) return false;
    if (!decodeMatvecOk(mm->src[1], &mm, 1, kcamd::kEpiResid, 1)) return false;
    *add = j;
    return true;
}

E decodeMatvecAdd(Pass& p, const T* mm, const T* ad) {
    kcamd::DmvArgs a{};
    if (E e = slotArgs(p, mm, a); e != ok) return e;
    a.p0 = dmvPart(mm, f32w(ad));
    a.nparts = 1;
    a.tpw = 1;
    a.r = f32(ad->src[0] == mm ? ad->src[1] : ad->src[0]);
    return direct(p, "decode_matvec_add", [&](hipStream_t s) {
        return kcamd::launchDecodeMatvec(kcamd::kProSlot, kcamd::kEpiResid, a, s);
    });
}

E decodeGroup(Pass& p, const T* const* mm, int g) {
    kcamd::DmvArgs a{};
    if (E e = slotArgs(p, mm[0], a); e != ok) return e;
    kcamd::DmvPart* ps[3] = {&a.p0, &a.p1, &a.p2};
    for (int j = 0; j < g; ++j) *ps[j] = dmvPart(mm[j], f32w(mm[j]));
    a.nparts = g;
    a.tpw = 1;
    return direct(p, "decode_matvec", [&](hipStream_t s) {
        return kcamd::launchDecodeMatvec(kcamd::kProSlot, kcamd::kEpiStore, a, s);
    });
}

// nodes[i], nodes[i + 1] = gate, up of one input column and nodes[i + 2] their SWIGLU, whose one
// use is a K-quant MUL_MAT (which reads the slot, not the f32 result); gate's and up's one use is
// the GLU. None of the three is a view or a graph output.
bool decodeSwigluOk(const T* const* nodes, int n, int i, int pro = kcamd::kProSlot) {
    if (i + 2 >= n) return false;
    const T *ga = nodes[i], *up = nodes[i + 1], *glu = nodes[i + 2];
    if (glu->op != KC_GGML_OP_GLU || glu->src[0] != ga || glu->src[1] != up || !computed(glu) ||
        glu->op_params[0] != KC_GGML_GLU_OP_SWIGLU || glu->op_params[1] != 0 || !f32c(glu))
        return false;
    for (const T* t : {ga, up, glu})
        if (t->uses != 1 || t->view || t->output) return false;
    if (ga->src[0]->ne[1] != up->src[0]->ne[1] || glu->ne[0] != ga->ne[0]) return false;
    const T* user = nullptr;
    for (int j = i + 3; j < n && !user; ++j)
        for (int s = 0; s < 5; ++s)
            if (nodes[j]->src[s] == glu) user = nodes[j];
    if (!user || user->op != KC_GGML_OP_MUL_MAT || user->src[1] != glu || !kquant(user->src[0])) return false;
    const T* mm[2] = {ga, up};
    return decodeMatvecOk(ga->src[1], mm, 2, kcamd::kEpiSwiglu, 2, pro);
}

// nodes[i] = RMS_NORM of one row and nodes[i + 1] its MUL by the norm weight (ggml_can_fuse), whose
// only uses are 2-3 MUL_MATs after it (not a view or an output): g.first, g.n = that group;
// g.glu: the group is gate / up followed by their SWIGLU (decodeSwigluOk).
struct NormGroup {
    int first = 0, n = 0;
    bool glu = false;
};
bool normGroupOk(const T* const* nodes, int n, int i, NormGroup& g) {
    static const int kNormMul[2] = {KC_GGML_OP_RMS_NORM, KC_GGML_OP_MUL};
    if (i + 1 >= n || !canFuse(nodes, n, i, kNormMul, 2)) return false;
    const T *norm = nodes[i], *mul = nodes[i + 1];
    if (mul->src[0] != norm || !rowVectorOf(mul->src[1], norm) || mul->view || mul->output) return false;
    const int j = nextWork(nodes, n, i + 2);
    int c = 0;
    while (j + c < n && c < 3 && nodes[j + c]->op == KC_GGML_OP_MUL_MAT && nodes[j + c]->src[1] == mul &&
           computed(nodes[j + c]))
        ++c;
    if (c < 2 || mul->uses != c) return false;
    g.first = j, g.n = c;
    g.glu = c == 2 && decodeSwigluOk(nodes, n, j, kcamd::kProNorm);
    return g.glu || decodeMatvecOk(mul, nodes + j, c, kcamd::kEpiStore, 2, kcamd::kProNorm);
}

E decodeNormGroup(Pass& p, const T* norm, const T* mul, const T* const* mm, const NormGroup& g) {
    kcamd::DmvArgs a{};
    a.k = int(norm->src[0]->ne[0]);
    a.x = f32(norm->src[0]);
    a.nw = f32(mul->src[1]);
    a.eps = paramF32(norm, 0);
    a.tpw = 2;
    if (g.glu) {
        a.p0 = dmvPart(mm[0], nullptr);
        a.p1 = dmvPart(mm[1], nullptr);
        a.nparts = 2;
        if (E e = kcamd::mulmat::outputSlot(p.rec, mm[2], a.p0.rows, 1, false, &a.qout); e != ok) return e;
        return direct(p, "decode_norm_swiglu", [&](hipStream_t s) {
            return kcamd::launchDecodeMatvec(kcamd::kProNorm, kcamd::kEpiSwiglu, a, s);
        });
    }
    kcamd::DmvPart* ps[3] = {&a.p0, &a.p1, &a.p2};
    for (int j = 0; j < g.n; ++j) *ps[j] = dmvPart(mm[j], f32w(mm[j]));
    a.nparts = g.n;
    return direct(p, "decode_norm_matvec", [&](hipStream_t s) {
        return kcamd::launchDecodeMatvec(kcamd::kProNorm, kcamd::kEpiStore, a, s);
    });
}

E decodeSwiglu(Pass& p, const T* ga, const T* up, const T* glu) {
    kcamd::DmvArgs a{};
    if (E e = slotArgs(p, ga, a); e != ok) return e;
    a.p0 = dmvPart(ga, nullptr);
    a.p1 = dmvPart(up, nullptr);
    a.nparts = 2;
    a.tpw = 2;
    if (E e = kcamd::mulmat::outputSlot(p.rec, glu, a.p0.rows, 1, false, &a.qout); e != ok) return e;
    return direct(p, "decode_swiglu", [&](hipStream_t s) {
        return kcamd::launchDecodeMatvec(kcamd::kProSlot, kcamd::kEpiSwiglu, a, s);
    });
}


// nodes[i] = ROPE(q), then (past no-op nodes) ROPE(k) of the same positions, factors and
// parameters, SET_ROWS(k cache, the roped k) and SET_ROWS(v cache, v) of the same row indices:
// at[0..3) their indices.
bool ropeKvOk(const T* const* nodes, int n, int i, int (&at)[3]) {
    const T* rq = nodes[i];
    const int a = nextWork(nodes, n, i + 1), b = a < n ? nextWork(nodes, n, a + 1) : n,
              c = b < n ? nextWork(nodes, n, b + 1) : n;
    if (c >= n) return false;
    const T *rk = nodes[a], *sk = nodes[b], *sv = nodes[c];
    if (rk->op != KC_GGML_OP_ROPE || sk->op != KC_GGML_OP_SET_ROWS || sv->op != KC_GGML_OP_SET_ROWS) return false;
    if (!computed(rk) || !computed(sk) || !computed(sv)) return false;
    if (rk->src[1] != rq->src[1] || rk->src[2] != rq->src[2] ||
        std::memcmp(rk->op_params, rq->op_params, sizeof rq->op_params) != 0)
        return false;
    const int64_t hd = rq->ne[0], nt = rq->ne[2], kv = rk->ne[1] * hd;
    if (rk->ne[0] != hd || rk->ne[2] != nt) return false;
    const T *ks = sk->src[0], *vs = sv->src[0];
    if (ks->data != rk->data || ks->ne[0] != kv || ks->ne[1] != nt || ks->nb[1] != size_t(kv) * 4) return false;
    if (sv->src[1] != sk->src[1] || vs->ne[0] != kv || vs->ne[1] != nt || vs->nb[1] / 4 > INT32_MAX) return false;
    if (vs->data == rq->data || vs->data == rk->data || sk->ne[1] != sv->ne[1]) return false;
    at[0] = a, at[1] = b, at[2] = c;
    return true;
}

E ropeKv(Pass& p, const T* rq, const T* rk, const T* sk, const T* sv) {
    const int hd = int(rq->ne[0]);
    const float* ff = rq->src[2] ? f32(rq->src[2]) : onesOf(p, hd / 2);
    if (!ff) return kc::Error::InternalError;
    // v's product split over K: its pending half, at the view's offset, stored with it
    const T* vbase = nullptr;
    const float* v2 = takeViewPending(p, sv->src[0], &vbase);
    if (v2) v2 += (static_cast<const char*>(sv->src[0]->data) - static_cast<const char*>(vbase->data)) / 4;
    const kcamd::RopeKvRows r{f32(rq->src[0]), f32w(rq), f32(rk->src[0]), f32w(rk), f32(sv->src[0]),
                              static_cast<int*>(sk->data), static_cast<int*>(sv->data),
                              static_cast<const int*>(rq->src[1]->data), static_cast<const int*>(sk->src[1]->data), ff,
                              hd, int(rq->ne[1]), int(rk->ne[1]), int(rq->ne[2]), std::log2(paramF32(rq, 5)),
                              (rq->op_params[2] & KC_GGML_ROPE_TYPE_NEOX) != 0, int(sv->src[0]->nb[1] / 4),
                              int(sk->nb[1] / 4), int(sv->nb[1] / 4), int(sk->ne[1]), v2};
    return direct(p, "rope_set_rows", [&](hipStream_t s) { return kcamd::launchRopeKvRows(r, s); });
}

// (No reference counterpart.) After ropeKvOk's four nodes, the next node with work: the
// FLASH_ATTN_EXT of one token on the roped q, whose K and V are views of the two caches the
// SET_ROWS write (rows as the caches' rows from one common row, heads D halves apart), taken by the
// split-context kernel with its per-32 slot: then the four nodes run as that kernel's prologue.
// fa: the attention node's index.
// The fused attention's intermediate outputs that it writes (the ROPE results; Qwen3's per-head
// norm MUL results): those something outside the fused nodes reads.
struct FaWrites {
    bool qr = false, kr = false, qn = false, kn = false;
};
// norms (Qwen3): RMS_NORM q, MUL q, RMS_NORM k, MUL k before the ROPEs (their MUL results are what
// the ROPEs read). The kernel's chunk-0 workgroups write the outputs of *w while the others still
// read the raw q, k and v; ggml's allocator runs ROPE, RMS_NORM and MUL in place, so a written output
// that overlaps one of those sources refuses the fusion.
bool ropeFaOk(const T* const* nodes, int n, int i, const int (&at)[3], int* fa, FaWrites* w,
              const T* const* norms = nullptr) {
    const T *rq = nodes[i], *rk = nodes[at[0]], *sk = nodes[at[1]], *sv = nodes[at[2]];
    const int f = nextWork(nodes, n, at[2] + 1);
    if (f >= n) return false;
    const T* node = nodes[f];
    if (node->op != KC_GGML_OP_FLASH_ATTN_EXT || !computed(node)) return false;
    const T *q = node->src[0], *k = node->src[1], *v = node->src[2];
    const int64_t hd = rq->ne[0], nh = rq->ne[1], nkv = rk->ne[1];
    if (!q || !k || !v || q->data != rq->data || rq->ne[2] != 1 || q->ne[1] != 1 || q->ne[2] != nh) return false;
    if (k->ne[0] != hd || k->ne[2] != nkv || v->ne[0] != hd || v->ne[2] != nkv || nh % nkv) return false;
    if (q->nb[2] != size_t(hd) * 4 || k->nb[2] != size_t(hd) * 2 || v->nb[2] != size_t(hd) * 2) return false;
    // the raw sources: contiguous heads
    const T *q0 = rq->src[0], *k0 = rk->src[0], *v0 = sv->src[0];
    if (q0->nb[0] != 4 || q0->nb[1] != size_t(hd) * 4 || k0->nb[0] != 4 || k0->nb[1] != size_t(hd) * 4 ||
        v0->nb[0] != 4)
        return false;
    // K and V: views of the caches from the same row, with the caches' row strides
    if (k->nb[1] != sk->nb[1] || v->nb[1] != sv->nb[1] || sk->nb[1] % 4 || sv->nb[1] % 4) return false;
    const auto off = [](const T* view, const T* base) {
        return static_cast<const char*>(view->data) - static_cast<const char*>(base->data);
    };
    const ptrdiff_t ok_ = off(k, sk), ov = off(v, sv);
    if (ok_ < 0 || ov < 0 || ok_ % ptrdiff_t(sk->nb[1]) || ov % ptrdiff_t(sv->nb[1])) return false;
    if (ok_ / ptrdiff_t(sk->nb[1]) != ov / ptrdiff_t(sv->nb[1]) || ok_ / ptrdiff_t(sk->nb[1]) > INT32_MAX) return false;
    // what flashAttn takes for one token with its slot
    const int D = int(hd), G = int(nh / nkv);
    if (!kcamd::flashDecodeSupports(D, G) || (nh * hd) % 256 || q->nb[1] % 16) return false;
    const T* fused[9] = {rq, rk, sk, sv, node};
    int nf = 5;
    if (norms)
        for (int j = 0; j < 4; ++j) fused[nf++] = norms[j];
    const T* srcs[3] = {norms ? norms[0]->src[0] : q0, norms ? norms[2]->src[0] : k0, v0};
    FaWrites wr;
    wr.qr = readBeyond(rq, nodes, n, fused, nf);
    wr.kr = readBeyond(rk, nodes, n, fused, nf);
    if (norms) {
        wr.qn = readBeyond(norms[1], nodes, n, fused, nf);
        wr.kn = readBeyond(norms[3], nodes, n, fused, nf);
    }
    const std::pair<bool, const T*> outs[4] = {{wr.qr, rq}, {wr.kr, rk}, {wr.qn, norms ? norms[1] : nullptr},
                                               {wr.kn, norms ? norms[3] : nullptr}};
    for (const auto& [written, o] : outs)
        if (written)
            for (const T* src : srcs)
                if (overlaps(o, src)) return false;
    *fa = f;
    *w = wr;
    return true;
}

// (No reference counterpart.) nodes[i] = RMS_NORM of q's heads and its MUL by a D-value weight, the
// same for k (Qwen3), each norm read by its MUL alone, then ROPE of those two MUL results, the cache
// SET_ROWS and the one-token FLASH_ATTN_EXT as ropeFaOk takes them: the norms run in the attention's
// prologue too (the MUL results still written). jr: the ROPE(q) index.
bool normRopeFaOk(const T* const* nodes, int n, int i, int* jr, int (&at)[3], int* fa, FaWrites* w) {
    static const int kNormMul[2] = {KC_GGML_OP_RMS_NORM, KC_GGML_OP_MUL};
    if (i + 3 >= n || !canFuse(nodes, n, i, kNormMul, 2) || !canFuse(nodes, n, i + 2, kNormMul, 2)) return false;
    const T *nq = nodes[i], *mq = nodes[i + 1], *nk = nodes[i + 2], *mk = nodes[i + 3];
    if (mq->src[0] != nq || mk->src[0] != nk || !rowVectorOf(mq->src[1], nq) || !rowVectorOf(mk->src[1], nk)) return false;
    const T *q0 = nq->src[0], *k0 = nk->src[0];
    if (nk->ne[0] != nq->ne[0] || paramF32(nq, 0) != paramF32(nk, 0) || !f32c(q0) || !f32c(k0) || !f32c(mq) || !f32c(mk))
        return false;
    const int j = nextWork(nodes, n, i + 4);
    if (j >= n || nodes[j]->op != KC_GGML_OP_ROPE || !computed(nodes[j]) || nodes[j]->src[0] != mq) return false;
    if (!ropeKvOk(nodes, n, j, at) || nodes[at[0]]->src[0] != mk || !ropeFaOk(nodes, n, j, at, fa, w, nodes + i))
        return false;
    *jr = j;
    return true;
}

E ropeFlashAttn(Pass& p, const T* rq, const T* rk, const T* sk, const T* sv, const T* dst, const FaWrites& w,
                const T* const* norms = nullptr) {
    const T* q = dst->src[0];
    const T* k = dst->src[1];
    const T* v = dst->src[2];
    const T* mask = dst->src[3];
    kcFaDims d{};
    d.D = int(k->ne[0]);
    d.T = int(k->ne[1]);
    d.H_kv = int(k->ne[2]);
    d.H = int(q->ne[2]);
    d.N = 1;
    d.group = d.H / d.H_kv;
    d.tp = (d.T + 7) / 8 * 8;
    d.k_row = int(k->nb[1] / 4), d.k_head = int(k->nb[2] / 4);
    d.v_row = int(v->nb[1] / 4), d.v_head = int(v->nb[2] / 4);
    d.q_tok = int(q->nb[1] / 4), d.q_head = int(q->nb[2] / 4);
    d.m_row = mask ? int(mask->nb[1] / 4) : 0;
    d.has_mask = mask ? 1 : 0;
    const int hd = int(rq->ne[0]);
    const float* ff = rq->src[2] ? f32(rq->src[2]) : onesOf(p, hd / 2);
    if (!ff) return kc::Error::InternalError;
    int* part = nullptr;
    if (E e = kcamd::mulmat::take(p.rec, kcamd::flashDecodePartFloats(d), &part); e != ok) return e;
    int* slot = nullptr;
    if (E e = kcamd::mulmat::outputSlot(p.rec, dst, d.H * d.D, 1, false, &slot); e != ok) return e;
    const kcFlashDecodeArgs a{f32(q), static_cast<const int*>(k->data), static_cast<const int*>(v->data),
                              mask ? static_cast<const int*>(mask->data) : nullptr, f32w(dst),
                              reinterpret_cast<float*>(part), nullptr, d, paramF32(dst, 0)};
    const ptrdiff_t row0 = (static_cast<const char*>(k->data) - static_cast<const char*>(sk->data)) / ptrdiff_t(sk->nb[1]);
    const kcamd::FdRope r{f32(rq->src[0]), f32(rk->src[0]), f32(sv->src[0]), w.qr ? f32w(rq) : nullptr,
                          w.kr ? f32w(rk) : nullptr,
                          static_cast<int*>(sk->data), static_cast<int*>(sv->data),
                          static_cast<const int*>(rq->src[1]->data), static_cast<const int*>(sk->src[1]->data), ff,
                          std::log2(paramF32(rq, 5)), (rq->op_params[2] & KC_GGML_ROPE_TYPE_NEOX) != 0,
                          int(sk->nb[1] / 4), int(sv->nb[1] / 4), int(sk->ne[1]), int(row0)};
    if (norms) {  // nodes: RMS_NORM q, MUL q, RMS_NORM k, MUL k
        kcamd::FdRope rn = r;
        rn.q = f32(norms[0]->src[0]);
        rn.k = f32(norms[2]->src[0]);
        rn.q_norm = f32(norms[1]->src[1]);
        rn.k_norm = f32(norms[3]->src[1]);
        rn.qn = w.qn ? f32w(norms[1]) : nullptr;
        rn.kn = w.kn ? f32w(norms[3]) : nullptr;
        rn.eps = paramF32(norms[0], 0);
        rn.qk_norm = 1;
        return direct(p, "norm_rope_flash_decode_q8",
                      [&](hipStream_t s) { return kcamd::launchFlashDecode(a, s, slot, &rn); });
    }
    return direct(p, "rope_flash_decode_q8", [&](hipStream_t s) { return kcamd::launchFlashDecode(a, s, slot, &r); });
}

E setRows(Pass& p, const T* dst) {  // dst rows src1[r] (int64) = fp16(src0 row r) (:650-661)
    const T* src = dst->src[0];
    const T* idx = dst->src[1];
    const kcSetRowsF16Args a{f32(src), static_cast<const int*>(idx->data), static_cast<int*>(dst->data), nullptr,
                             int(src->ne[0] / 2), int(src->ne[1]), int(src->nb[1] / 4), int(dst->nb[1] / 4),
                             int(dst->ne[1])};
    return launch(p, "set_rows_f16", &a);
}

// FLASH_ATTN_EXT (:663-699): the dimensions as the reference derives them. Up to 8 query tokens
// (decode) the context is split over 64-position chunks (flash_decode_f16, the chunk partials in the
// scratch); larger batches take one flash_attn_f16 kernel, or beyond its 16384 positions the four
// fa_* kernels with their scores in the scratch.
E flashAttn(Pass& p, const T* dst) {
    const T* q = dst->src[0];
    const T* k = dst->src[1];
    const T* v = dst->src[2];
    const T* mask = dst->src[3];
    kcFaDims d{};
    d.D = int(k->ne[0]);
    d.T = int(k->ne[1]);
    d.H_kv = int(k->ne[2]);
    d.H = int(q->ne[2]);
    d.N = int(q->ne[1]);
    d.group = d.H / d.H_kv;
    d.tp = (d.T + 7) / 8 * 8;
    d.k_row = int(k->nb[1] / 4), d.k_head = int(k->nb[2] / 4);
    d.v_row = int(v->nb[1] / 4), d.v_head = int(v->nb[2] / 4);
    d.q_tok = int(q->nb[1] / 4), d.q_head = int(q->nb[2] / 4);
    d.m_row = mask ? int(mask->nb[1] / 4) : 0;
    d.has_mask = mask ? 1 : 0;
    const float scale = paramF32(dst, 0);
    const int* kd = static_cast<const int*>(k->data);
    const int* vd = static_cast<const int*>(v->data);
    const int* md = mask ? static_cast<const int*>(mask->data) : nullptr;
    if (d.N <= 8 && kcamd::flashDecodeSupports(d.D, d.group) && d.q_tok % 4 == 0 && d.q_head % 4 == 0) {
        int* part = nullptr;
        if (E e = kcamd::mulmat::take(p.rec, kcamd::flashDecodePartFloats(d), &part); e != ok) return e;
        const kcFlashDecodeArgs a{f32(q), kd, vd, md, f32w(dst), reinterpret_cast<float*>(part), nullptr, d, scale};
        if (d.N == 1 && (d.H * d.D) % 256 == 0 && kcamd::option("ggml_extra_fusions") != 1) {
            // one token: the output's per-32 slot too, for the MUL_MAT that reads it (the o projection)
            int* slot = nullptr;
            if (E e = kcamd::mulmat::outputSlot(p.rec, dst, d.H * d.D, 1, false, &slot); e != ok) return e;
            return direct(p, "flash_decode_q8", [&](hipStream_t s) { return kcamd::launchFlashDecode(a, s, slot); });
        }
        return launch(p, "flash_decode_f16", &a);
    }
    // a batch with a mask, in the layout of the decoder's caches (heads D / 2 words apart in K and V
    // rows of one stride, q and out [N][H][D]): on the matrix cores, masked key blocks skipped
    const kcamd::AttnShape as{d.N, d.H, d.H_kv, d.D, d.q_tok, d.k_row, d.T, 0, scale};
    if (maskedAttn(dst)) {
        const auto* mh = static_cast<const unsigned short*>(mask->data);
        // the mask's summary per query tile: computed by the first masked attention that reads it
        int* sum = nullptr;
        bool fresh = true;
        for (const auto& m : p.masks)
            if (m.mask == mask && m.N == d.N && m.T_keys == d.T && m.gen == p.rec.gen) {
                sum = m.sum;
                fresh = false;
            }
        if (fresh) {
            if (E e = kcamd::mulmat::take(p.rec, size_t(kcamd::maskSummaryInts(d.N)), &sum); e != ok) return e;
            try {
                p.masks.push_back({mask, d.N, d.T, p.rec.gen, sum});
            } catch (...) {
                return kc::Error::OutOfMemory;
            }
        }
        return direct(p, "attn_masked", [&](hipStream_t s) {
            if (fresh)
                if (int st = kcamd::launchMaskSummary(mh, 2 * d.m_row, d.N, d.T, sum, s)) return st;
            return kcamd::launchAttnMasked(f32(q), kd, vd, mh, 2 * d.m_row, d.T, f32w(dst), as, sum, s);
        });
    }
    if (d.T <= 16384) {
        const kcFlashAttnArgs a{f32(q), kd, vd, md, f32w(dst), nullptr, d, scale};
        return launch(p, "flash_attn_f16", &a);
    }
    const size_t rows = size_t(d.H) * size_t(d.N);
    int* sc = nullptr;
    if (E e = kcamd::mulmat::take(p.rec, rows * size_t(d.tp) + rows, &sc); e != ok) return e;
    float* s = reinterpret_cast<float*>(sc);
    float* m = s + rows * size_t(d.tp);
    const kcFaScoresArgs sa{f32(q), kd, md, s, nullptr, d, scale};
    const kcFaMaxArgs ma{s, m, nullptr, d};
    const kcFaExpArgs ea{s, m, nullptr, d};
    const kcFaValuesArgs va{s, vd, f32w(dst), nullptr, d};
    if (E e = launch(p, "fa_scores", &sa); e != ok) return e;
    if (E e = launch(p, "fa_max", &ma); e != ok) return e;
    if (E e = launch(p, "fa_exp", &ea); e != ok) return e;
    return launch(p, "fa_values", &va);
}

// (No reference counterpart.) mm[0..g) = 1-3 batch MUL_MATs of one input (q / k / v; gate / up; o;
// down) that all run on the per-256 MFMA matmul: K-quant weights of one k, contiguous f32 input
// columns and outputs, at least 64 columns. They run as one grouped launch over their rows (the
// decode driver's prefill does the same), from the fp16 form the input's producer wrote with its
// slots (else converted once), instead of one by-name matmul each that converts its input itself.
// One MUL_MAT takes the by-name launch's K split (matmulKs), its second half added afterwards.
bool batchGroupOk(const Pass& p, const T* const* mm, int g) {
    if (g < 1 || g > 3 || !p.rec.cfg.q8k || p.rec.cfg.matvec_cols) return false;
    const T* x = mm[0]->src[1];
    const int64_t k = mm[0]->src[0]->ne[0], ncols = nrows(x);
    if (ncols < 64 || ncols > INT32_MAX || k % 256 || k > INT32_MAX || !f32c(x) || x->nb[1] != size_t(k) * 4)
        return false;
    if (!kcamd::mfmaHUsable(int(ncols), int(k))) return false;
    for (int j = 0; j < g; ++j) {
        const T* w = mm[j]->src[0];
        if (mm[j]->src[1] != x || !kquant(w) || w->ne[0] != k || w->ne[1] % 8 || w->ne[1] * ncols > INT32_MAX ||
            !f32c(mm[j]) || mm[j]->ne[0] != w->ne[1] || nrows(mm[j]) != ncols)
            return false;
    }
    return true;
}

E batchGroup(Pass& p, const T* const* mm, int g) {
    if (E e = mulMatInput(p, mm[0]); e != ok) return e;  // quantize_cols_k, once per input
    const T* x = mm[0]->src[1];
    const int k = int(mm[0]->src[0]->ne[0]), ncols = int(nrows(x));
    const int* q = p.rec.dry ? nullptr : kcamd::mulmat::inputSlot(p.rec, keyOf(x), ncols, k, true);
    if (!p.rec.dry && !q) return kc::Error::InternalError;
    const kcamd::ActF16* pre = kcamd::mulmat::inputAct(p.rec, keyOf(x), ncols, k);
    kcamd::MmPart parts[3];
    for (int j = 0; j < g; ++j) {
        const T* w = mm[j]->src[0];
        parts[j] = kcamd::MmPart{w->data, {f32w(mm[j]), nullptr}, int(w->ne[1]), w->type == KC_GGML_TYPE_Q6_K ? 1 : 0};
    }
    const int rows0 = parts[0].rows;
    const int ks = g == 1 ? kcamd::matmulKs(rows0, k, ncols, parts[0].q6 != 0) : 1;
    if (ks == 2) {  // the second K half's partial sums
        int* part = nullptr;
        if (E e = kcamd::mulmat::take(p.rec, size_t(rows0) * size_t(ncols), &part); e != ok) return e;
        parts[0].y[1] = reinterpret_cast<float*>(part);
    }
    // a Q6_K matrix beside Q4_K ones (a Q6_K v in q / k / v) may run in two K ranges of its own
    // (matmulGroupSplitsQ6): its second half goes to scratch and stays pending past the views of it
    bool split6 = false;
    if (g > 1) {
        kcamd::MmPart probe[3];
        for (int j = 0; j < g; ++j) {
            probe[j] = parts[j];
            if (probe[j].q6) probe[j].y[1] = reinterpret_cast<float*>(uintptr_t(256));  // (not dereferenced)
        }
        split6 = kcamd::matmulGroupSplitsQ6(probe, g, k, ncols);
        for (int j = 0; split6 && j < g; ++j)
            if (parts[j].q6) {
                int* part = nullptr;
                if (E e = kcamd::mulmat::take(p.rec, size_t(parts[j].rows) * size_t(ncols), &part); e != ok) return e;
                parts[j].y[1] = reinterpret_cast<float*>(part);
            }
    }
    const E e = direct(p, "matmul_group", [&](hipStream_t s) {
        int used = 1, pks[3] = {1, 1, 1};
        if (int st = kcamd::launchMatmulGroup(parts, g, q, k, ncols, ks, &used, s, pre, split6 ? pks : nullptr))
            return st;
        bool as_planned = used == ks;  // (the launcher runs the MFMA kernel whenever batchGroupOk holds)
        for (int j = 0; split6 && j < g; ++j) as_planned = as_planned && pks[j] == (parts[j].q6 ? 2 : 1);
        if (!as_planned) {
            kcamd::setDetail("ggml backend: the grouped matmul took another K split than planned");
            return int(kc::Error::InternalError);
        }
        return 0;
    });
    if (e != ok) return e;
    for (int j = 0; split6 && j < g; ++j) {
        if (!parts[j].q6) continue;
        const T* y = mm[j];
        if (y->uses == 1 && !y->view && !y->output) p.pending.push_back({y, parts[j].y[1], true});
        else if (E e2 = addHalf(p, y, parts[j].y[1]); e2 != ok) return e2;
    }
    if (ks != 2) return ok;
    // the half is added by whatever reads the product next (the ADD's fused norm takes it along)
    // unless the product is a view, an output or read twice: then now
    const T* y = mm[0];
    if (y->uses == 1 && !y->view && !y->output) {
        p.pending.push_back({y, parts[0].y[1], false});
        return ok;
    }
    return addHalf(p, y, parts[0].y[1]);
}

E concurrent(Pass& p, bool begin) {
    if (E e = marker(p, begin ? "[" : "]"); e != ok) return e;
    if (p.rec.dry) return ok;
    return begin ? kcStreamConcurrentBegin(p.rec.stream) : kcStreamConcurrentEnd(p.rec.stream);
}

// backend_graph_compute's walk (:712-788)
E walk(Pass& p, const T* const* nodes, int n) {
    static const int kNormMul[2] = {KC_GGML_OP_RMS_NORM, KC_GGML_OP_MUL};
    for (int i = 0; i < n; ++i) {
        const T* node = nodes[i];
        // a reader of a product with a pending K half (views included) adds it first; an ADD decides
        // below (its fused norm takes it along)
        if (!p.pending.empty() && node->op != KC_GGML_OP_ADD)
            for (int s = 0; s < 5; ++s)
                if (E e = settle(p, node->src[s], viewOp(node->op)); e != ok) return e;
        // nothing to compute (e.g. a prompt's earlier batches select no output rows); fused
        // partners of an empty node are empty too
        if (!computed(node)) continue;
        E e = ok;
        switch (node->op) {
            case KC_GGML_OP_MUL_MAT: {
                const ShapeTag tag(p, node);
                if (kcamd::option("ggml_extra_fusions") != 1) {  // one input column: the fused decode matvec
                    int ga = 1;
                    while (i + ga < n && ga < 3 && nodes[i + ga]->op == KC_GGML_OP_MUL_MAT &&
                           nodes[i + ga]->src[1] == node->src[1] && computed(nodes[i + ga]))
                        ++ga;
                    if (ga == 2 && decodeSwigluOk(nodes, n, i)) {
                        e = decodeSwiglu(p, nodes[i], nodes[i + 1], nodes[i + 2]);
                        i += 2;
                        break;
                    }
                    if (ga >= 2 && decodeMatvecOk(node->src[1], nodes + i, ga, kcamd::kEpiStore, 1)) {
                        e = decodeGroup(p, nodes + i, ga);
                        i += ga - 1;
                        break;
                    }
                    int add = 0;
                    if (ga == 1 && matvecAddOk(nodes, n, i, &add)) {
                        e = decodeMatvecAdd(p, node, nodes[add]);
                        i = add;
                        break;
                    }
                }
                if (kcamd::option("ggml_extra_fusions") != 1) {  // a batch group on the matrix cores: one launch
                    int gb = 1;
                    while (i + gb < n && gb < 3 && nodes[i + gb]->op == KC_GGML_OP_MUL_MAT &&
                           nodes[i + gb]->src[1] == node->src[1] && computed(nodes[i + gb]))
                        ++gb;
                    if (batchGroupOk(p, nodes + i, gb)) {
                        e = batchGroup(p, nodes + i, gb);
                        i += gb - 1;
                        break;
                    }
                }
                // consecutive MUL_MATs of one input (q, k, v; gate, up) as one step
                int g = 1;
                while (p.cfg.concurrent && p.capturing && i + g < n && nodes[i + g]->op == KC_GGML_OP_MUL_MAT &&
                       nodes[i + g]->src[1] == node->src[1] && computed(nodes[i + g]))
                    ++g;
                if (g == 1) {
                    e = mulMat(p, node);
                    break;
                }
                e = mulMatInput(p, node);  // the shared input quantized first (its own step)
                if (e == ok) e = concurrent(p, true);
                if (e != ok) break;
                for (int j = 0; e == ok && j < g; ++j) e = mulMat(p, nodes[i + j]);
                const E f = concurrent(p, false);
                if (e == ok) e = f;
                i += g - 1;
                break;
            }
            case KC_GGML_OP_ADD:
            case KC_GGML_OP_RMS_NORM: {
                int jr = 0, at4[3], fa4 = 0;
                FaWrites w4;
                if (node->op == KC_GGML_OP_RMS_NORM && kcamd::option("ggml_extra_fusions") != 1 &&
                    normRopeFaOk(nodes, n, i, &jr, at4, &fa4, &w4)) {  // per-head norms into the attention's launch
                    e = ropeFlashAttn(p, nodes[jr], nodes[at4[0]], nodes[at4[1]], nodes[at4[2]], nodes[fa4], w4,
                                      nodes + i);
                    i = fa4;
                    break;
                }
                NormGroup ng;
                if (node->op == KC_GGML_OP_RMS_NORM && kcamd::option("ggml_extra_fusions") != 1 &&
                    normGroupOk(nodes, n, i, ng)) {  // the norm in the group's launch
                    const ShapeTag tag(p, nodes[ng.first]);
                    e = decodeNormGroup(p, node, nodes[i + 1], nodes + ng.first, ng);
                    i = ng.first + ng.n - 1 + (ng.glu ? 1 : 0);
                    break;
                }
                // [ADD +] RMS_NORM + MUL by a row vector (the norm weight): the fused producer
                // (n % 256 == 0), else vector_add or a one-pass rms_norm
                const int ni = node->op == KC_GGML_OP_ADD ? i + 1 : i;  // the RMS_NORM node
                const T* norm = ni < n ? nodes[ni] : nullptr;
                const T* mulNode = ni + 1 < n ? nodes[ni + 1] : nullptr;
                const bool pattern = norm && mulNode && norm->op == KC_GGML_OP_RMS_NORM &&
                                     canFuse(nodes, n, ni, kNormMul, 2) && mulNode->src[0] == norm &&
                                     rowVectorOf(mulNode->src[1], norm) && norm->src[0]->ne[0] % 256 == 0 &&
                                     contiguous(norm->src[0]) &&
                                     (node->op == KC_GGML_OP_RMS_NORM || norm->src[0] == node);
                if (pattern) {
                    e = fusedNorm(p, node->op == KC_GGML_OP_ADD ? node : nullptr, norm, mulNode);
                    i = ni + 1;
                } else if (node->op == KC_GGML_OP_ADD) {
                    e = settle(p, node->src[0]);
                    if (e == ok) e = settle(p, node->src[1]);
                    if (e == ok) e = add(p, node);
                } else {
                    const T* next = i + 1 < n ? nodes[i + 1] : nullptr;
                    if (next && canFuse(nodes, n, i, kNormMul, 2) && next->src[0] == node &&
                        rowVectorOf(next->src[1], node)) {
                        e = rmsNorm(p, node, f32(next->src[1]), next);
                        ++i;
                    } else {
                        e = rmsNorm(p, node, nullptr, node);
                    }
                }
                break;
            }
            case KC_GGML_OP_MUL: e = mul(p, node); break;
            case KC_GGML_OP_ROPE: {
                int at[3];
                int fa = 0;
                FaWrites w;
                if (kcamd::option("ggml_extra_fusions") != 1 && ropeKvOk(nodes, n, i, at)) {
                    if (ropeFaOk(nodes, n, i, at, &fa, &w)) {  // and the attention they feed: one launch
                        e = ropeFlashAttn(p, node, nodes[at[0]], nodes[at[1]], nodes[at[2]], nodes[fa], w);
                        i = fa;
                    } else {
                        e = ropeKv(p, node, nodes[at[0]], nodes[at[1]], nodes[at[2]]);
                        i = at[2];
                    }
                } else {
                    e = rope(p, node);
                }
                break;
            }
            case KC_GGML_OP_GLU: e = node->ne[0] % 256 == 0 ? fusedSwiglu(p, node) : swiglu(p, node); break;
            case KC_GGML_OP_SET_ROWS: e = setRows(p, node); break;
            case KC_GGML_OP_FLASH_ATTN_EXT: e = flashAttn(p, node); break;
            case KC_GGML_OP_NONE:
            case KC_GGML_OP_RESHAPE:
            case KC_GGML_OP_VIEW:
            case KC_GGML_OP_PERMUTE:
            case KC_GGML_OP_TRANSPOSE:
                break;
            default:
                kcamd::setDetail("ggml backend: node %d: op %d is not one this backend runs", i, node->op);
                return kc::Error::UnsupportedOperation;
        }
        if (e != ok) return e;
    }
    while (!p.pending.empty()) {  // products nothing in the list read: whole for the caller
        const T* t = p.pending.front().t;
        if (E e = settle(p, t); e != ok) return e;
    }
    return ok;
}

// Every node present, and every node with work one this backend claims (the scheduler only hands
// it such nodes; anything else is refused before a launch).
E checkNodes(const kcGgmlConfig& c, const T* const* nodes, int n) {
    if (n < 0 || (n > 0 && !nodes)) return bad("null node list or negative count");
    for (int i = 0; i < n; ++i) {
        if (!nodes[i]) {
            kcamd::setDetail("ggml backend: node %d is null", i);
            return kc::Error::InvalidValue;
        }
        if (computed(nodes[i]) && !supports(c, nodes[i])) {
            kcamd::setDetail("ggml backend: node %d (op %d) is not one this backend runs with these operands", i,
                             nodes[i]->op);
            return kc::Error::UnsupportedOperation;
        }
    }
    return ok;
}

// A plan of the walk: its launch names, the scratch it takes and the 1.0f arrays it reads.
struct Plan {
    std::vector<const char*> trace;
    std::vector<int> ones;
    size_t scratch = 0;
    size_t staging = 0;  // the largest per-stream fp16 staging of a by-name MFMA matmul
    long long launches = 0;
};

E plan(const kcGgmlConfig& c, const T* const* nodes, int n, Plan& out) {
    if (E e = checkNodes(c, nodes, n); e != ok) return e;
    kcMulMatRecording_st dry;
    dry.cfg = c.mul_mat;
    dry.act_f16 = true;
    dry.dry = true;
    dry.trace = &out.trace;
    Pass p{c, dry, nullptr, &out.ones, c.graphs != 0};
    if (E e = walk(p, nodes, n); e != ok) return e;
    out.scratch = dry.peak;
    for (const char* t : out.trace)
        if (t[0] != '[' && t[0] != ']') ++out.launches;
    for (int i = 0; i < n; ++i) {  // the MFMA matmuls' staging (a graph records the buffer it finds)
        const T* t = nodes[i];
        if (t->op == KC_GGML_OP_MUL_MAT && computed(t) && kquant(t->src[0]))
            out.staging = std::max(out.staging, kcamd::matmulStagingBytes(int(t->src[0]->ne[1]), int(t->src[0]->ne[0]),
                                                                          int(nrows(t->src[1]))));
    }
    return ok;
}

// The nodes as a graph would be recorded from them: every field a launch or a fusion decision reads,
// src links as node indices (or, for tensors outside the list, their first-seen order and fields).
// In two parts: the structure (sigShape, kept while the node array and its src links are the same)
// and the fields in that order (sigValues).
using kcamd::ggml::SigShape;
constexpr int kSrcs = 5;

bool sameShape(const SigShape& sh, const T* const* nodes, int n) {
    if (sh.nodes.size() != size_t(n) || !std::equal(nodes, nodes + n, sh.nodes.begin())) return false;
    for (int i = 0; i < n; ++i)
        if (!std::equal(nodes[i]->src, nodes[i]->src + kSrcs, sh.srcs.begin() + size_t(i) * kSrcs)) return false;
    return true;
}

void sigShape(const T* const* nodes, int n, SigShape& sh) {
    sh.nodes.assign(nodes, nodes + n);
    sh.srcs.clear();
    sh.ref.clear();
    sh.leaves.clear();
    std::unordered_map<const T*, int64_t> id;
    id.reserve(size_t(n) * 2);
    for (int i = 0; i < n; ++i) id.emplace(nodes[i], i);
    std::unordered_map<const T*, int64_t> leaf;
    for (int i = 0; i < n; ++i)
        for (const T* src : nodes[i]->src) {
            sh.srcs.push_back(src);
            if (!src) {
                sh.ref.push_back(-1);
                continue;
            }
            const auto it = id.find(src);
            if (it != id.end()) {
                sh.ref.push_back(it->second);
                continue;
            }
            const auto [lt, fresh] = leaf.emplace(src, int64_t(leaf.size()));
            if (fresh) sh.leaves.push_back(src);
            sh.ref.push_back(-2 - lt->second);
        }
}

void sigValues(const SigShape& sh, std::vector<uint64_t>& s) {
    const auto put = [&s](const T* t) {
        s.push_back(uint64_t(uint32_t(t->op)) | uint64_t(uint32_t(t->type)) << 32);
        for (int d = 0; d < 4; ++d) s.push_back(uint64_t(t->ne[d]));
        for (int d = 0; d < 4; ++d) s.push_back(uint64_t(t->nb[d]));
        s.push_back(uint64_t(reinterpret_cast<uintptr_t>(t->data)));
        for (int j = 0; j < 16; j += 2) s.push_back(uint64_t(uint32_t(t->op_params[j])) | uint64_t(uint32_t(t->op_params[j + 1])) << 32);
        s.push_back(uint64_t(uint32_t(t->buffer)) | uint64_t(t->compute != 0) << 32 | uint64_t(t->output != 0) << 33 |
                    uint64_t(t->view != 0) << 34);
        s.push_back(uint64_t(uint32_t(t->uses)));
    };
    s.clear();
    s.push_back(uint64_t(sh.nodes.size()));
    size_t r = 0;
    int64_t next = 0;  // leaves put so far (a leaf's fields follow its first reference)
    for (const T* node : sh.nodes) {
        put(node);
        for (int k = 0; k < kSrcs; ++k) {
            const int64_t v = sh.ref[r++];
            if (v == -1) {
                s.push_back(~uint64_t(0));
            } else if (v >= 0) {
                s.push_back(uint64_t(v));
            } else {
                const int64_t lid = -2 - v;
                s.push_back(uint64_t(1) << 62 | uint64_t(lid));
                if (lid == next) {
                    put(sh.leaves[size_t(lid)]);
                    ++next;
                }
            }
        }
    }
}

E makeOnes(kcGgmlBackend_st& be, const std::vector<int>& lengths) {
    for (const int n : lengths) {
        if (n <= 0) return bad("a 1.0f array of no length");
        if (be.ones.count(n)) continue;
        void* d = nullptr;
        if (E e = kcMalloc(&d, size_t(n) * sizeof(float)); e != ok) return e;
        const std::vector<float> v(size_t(n), 1.0f);
        if (E e = kcMemcpy(d, v.data(), v.size() * sizeof(float), kc::CopyKind::HostToDevice); e != ok) {
            (void)kcFree(d);
            return e;
        }
        be.ones.emplace(n, static_cast<float*>(d));
    }
    return ok;
}

void dropGraph(kcGgmlBackend_st& be) {
    if (be.graph) (void)kcGraphDestroy(be.graph);
    be.graph = nullptr;
    be.sig.clear();
}

double msSince(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

// profile = 2: the device time of every timed launch of the call, summed per name (the stream has run them)
E collectTimes(kcGgmlBackend_st& be) {
    for (const auto& m : be.timer.marks) {
        float ms = 0.0f;
        if (int e = kcamd::fromHip(hipEventElapsedTime(&ms, m.a, m.b), "hipEventElapsedTime")) return E(e);
        auto& [count, total] = be.per_kernel[m.name];
        ++count;
        total += ms;
    }
    be.timer.marks.clear();
    be.timer.used = 0;
    return ok;
}

E compute(kcGgmlBackend_st& be, const T* const* nodes, int n) {
    if (n < 0 || (n > 0 && !nodes)) return bad("null node list or negative count");
    for (int i = 0; i < n; ++i)
        if (!nodes[i]) {
            kcamd::setDetail("ggml backend: node %d is null", i);
            return kc::Error::InvalidValue;
        }
    const auto t0 = std::chrono::steady_clock::now();
    const bool prof = be.cfg.profile >= 1, each = be.cfg.profile >= 2;
    const bool graphs = be.cfg.graphs != 0 && !each;  // launches timed one by one: no graph
    const unsigned options = kcamd::optionsGeneration();  // read before the walk reads any option
    if (graphs) {
        if (!sameShape(be.shape, nodes, n)) sigShape(nodes, n, be.shape);
        sigValues(be.shape, be.sig_now);
        // the kept graph again: the same fields as when it was recorded (and checked) -- what the
        // checks read is in the signature
        if (be.graph && be.graph_gen == be.rec.gen && be.graph_options == options && be.sig_now == be.sig) {
            const auto tr = std::chrono::steady_clock::now();
            if (E e = kcGraphLaunch(be.graph, be.stream); e != ok) return e;
            if (E e = kcStreamSynchronize(be.stream); e != ok) return e;
            ++be.stats.computes;
            ++be.stats.graphs_reused;
            be.stats.launches += be.graph_launches;
            if (prof) {
                be.stats.run_ms += msSince(tr);
                be.stats.compute_ms += msSince(t0);
            }
            return ok;
        }
    }
    Plan pl;  // (checks the nodes first)
    if (E e = plan(be.cfg, nodes, n, pl); e != ok) return e;
    if (E e = makeOnes(be, pl.ones); e != ok) return e;
    kcamd::mulmat::reset(be.rec);
    if (pl.scratch > be.rec.cap) {  // replaced before anything is recorded into it
        dropGraph(be);
        if (E e = kcamd::mulmat::reserve(be.rec, pl.scratch); e != ok) return e;
    }
    Pass p{be.cfg, be.rec, &be, nullptr, graphs};
    double record = 0, run = 0;
    if (!graphs) {
        be.rec.timer = each ? &be.timer : nullptr;
        const E e = walk(p, nodes, n);
        be.rec.timer = nullptr;
        record = msSince(t0);
        const auto tr = std::chrono::steady_clock::now();
        const E s = kcStreamSynchronize(be.stream);
        run = msSince(tr);
        if (each) {
            const E c = e == ok && s == ok ? collectTimes(be) : ok;
            be.timer.marks.clear();
            be.timer.used = 0;
            if (c != ok) return c;
        }
        if (e != ok) return e;
        if (s != ok) return s;
    } else {
        dropGraph(be);
        if (pl.staging) {  // grown now: inside the capture it could not grow, and the MFMA matmuls would
                           // take their unstaged kernels
            void* hs = nullptr;
            if (E e = kcStreamGetNative(be.stream, &hs); e != ok) return e;
            if (!kcamd::streamScratch(hs, pl.staging)) return kc::Error::OutOfMemory;
        }
        if (E e = kcStreamBeginCapture(be.stream); e != ok) return e;
        const E e = walk(p, nodes, n);
        kcGraph_t g = nullptr;
        const E c = kcStreamEndCapture(be.stream, &g);
        if (e != ok || c != ok) {
            if (g) (void)kcGraphDestroy(g);
            return e != ok ? e : c;
        }
        record = msSince(t0);
        const auto tr = std::chrono::steady_clock::now();
        if (E l = kcGraphLaunch(g, be.stream); l != ok) {
            (void)kcGraphDestroy(g);
            return l;
        }
        be.graph = g;
        be.sig = be.sig_now;
        be.graph_gen = be.rec.gen;
        be.graph_options = options;
        be.graph_launches = pl.launches;
        ++be.stats.graphs_recorded;
        if (E s = kcStreamSynchronize(be.stream); s != ok) return s;
        run = msSince(tr);
    }
    ++be.stats.computes;
    be.stats.launches += pl.launches;
    if (prof) {
        be.stats.record_ms += record;
        be.stats.run_ms += run;
        be.stats.compute_ms += msSince(t0);
    }
    return ok;
}

kcGgmlConfig configOrEnv(const kcGgmlConfig* cfg) {
    kcGgmlConfig c;
    if (cfg) c = *cfg;
    else kcGgmlConfigFromEnv(&c);
    return c;
}

bool envIs(const char* name, const char* value) {
    const char* v = std::getenv(name);
    return v && std::strcmp(v, value) == 0;
}

}  // namespace

KC_API void kcGgmlConfigFromEnv(kcGgmlConfig* cfg) noexcept {
    if (!cfg) return;
    kcMulMatConfigFromEnv(&cfg->mul_mat);
    cfg->disabled = envIs("GGML_KERNELCORE_DISABLE", "1");
    cfg->matmul_only = envIs("GGML_KERNELCORE_MATMUL_ONLY", "1");
    cfg->attn = !envIs("GGML_KERNELCORE_ATTN", "0");
    cfg->attn_tokens = 8;
    if (const char* an = std::getenv("GGML_KERNELCORE_ATTN_TOKENS")) cfg->attn_tokens = std::max(0, std::atoi(an));
    cfg->concurrent = !envIs("GGML_KERNELCORE_CONCURRENT", "0");
    cfg->graphs = !envIs("GGML_KERNELCORE_GRAPHS", "0");
    cfg->profile = envIs("GGML_KERNELCORE_PROFILE", "1") ? 1 : envIs("GGML_KERNELCORE_PROFILE", "2") ? 2 : 0;
}

KC_API int kcGgmlSupportsOp(const kcGgmlConfig* cfg, const kcGgmlTensor* op) noexcept {
    return supports(configOrEnv(cfg), op) ? 1 : 0;
}

KC_API int kcGgmlOffersKvBuffer(const kcGgmlConfig* cfg) noexcept {
    const kcGgmlConfig c = configOrEnv(cfg);
    return !c.disabled && !c.matmul_only && c.attn ? 1 : 0;
}

KC_API kcError_t kcGgmlGraphPlan(const kcGgmlConfig* cfg, const kcGgmlTensor* const* nodes, int n_nodes, char* names,
                                 size_t size, size_t* needed, size_t* scratch_ints) noexcept {
    try {
        kcGgmlConfig c = configOrEnv(cfg);
        if (E e = kcamd::mulmat::checkConfig(c.mul_mat); e != ok) return e;
        Plan pl;
        if (E e = plan(c, nodes, n_nodes, pl); e != ok) return e;
        std::string s;
        for (const char* t : pl.trace) {
            if (!s.empty()) s += ' ';
            s += t;
        }
        if (needed) *needed = s.size() + 1;
        if (scratch_ints) *scratch_ints = pl.scratch;
        if (names && size >= s.size() + 1) std::memcpy(names, s.c_str(), s.size() + 1);
        else if (names && size) names[0] = '\0';
        return ok;
    } catch (...) {
        return kc::Error::OutOfMemory;
    }
}

KC_API kcError_t kcGgmlBackendCreate(kcGgmlBackend_t* backend, const kcGgmlConfig* cfg, kcStream_t stream) noexcept {
    if (!backend) return bad("null backend pointer");
    *backend = nullptr;
    kcGgmlConfig c = configOrEnv(cfg);
    if (E e = kcamd::mulmat::checkConfig(c.mul_mat); e != ok) return e;
    if (c.disabled) {
        kcamd::setDetail("ggml backend: disabled (GGML_KERNELCORE_DISABLE=1)");
        return kc::Error::UnsupportedOperation;
    }
    int dev = 0;
    if (E e = kcGetDevice(&dev); e != ok) return e;  // the runtime is up
    auto* be = new (std::nothrow) kcGgmlBackend_st;
    if (!be) return kc::Error::OutOfMemory;
    be->cfg = c;
    be->stream = stream;
    be->rec.cfg = c.mul_mat;
    be->rec.act_f16 = true;  // the batch producers write the MFMA matmul's fp16 form (batchGroup reads it)
    be->rec.stream = stream;
    *backend = be;
    return ok;
}

KC_API kcError_t kcGgmlBackendDestroy(kcGgmlBackend_t backend) noexcept {
    if (!backend) return ok;
    E e = kcStreamSynchronize(backend->stream);  // nothing in flight reads what is freed below
    dropGraph(*backend);
    for (hipEvent_t ev : backend->timer.pool) (void)hipEventDestroy(ev);
    for (auto& [n, ptr] : backend->ones)
        if (E f = kcFree(ptr); e == ok) e = f;
    if (backend->rec.scratch)
        if (E f = kcFree(backend->rec.scratch); e == ok) e = f;
    delete backend;
    return e;
}

KC_API kcError_t kcGgmlGraphCompute(kcGgmlBackend_t backend, const kcGgmlTensor* const* nodes, int n_nodes) noexcept {
    if (!backend) return kc::Error::InvalidResourceHandle;
    try {
        return compute(*backend, nodes, n_nodes);
    } catch (...) {
        return kc::Error::OutOfMemory;
    }
}

KC_API kcError_t kcGgmlBackendGetStats(kcGgmlBackend_t backend, kcGgmlStats* stats) noexcept {
    if (!backend) return kc::Error::InvalidResourceHandle;
    if (!stats) return bad("null stats pointer");
    *stats = backend->stats;
    return ok;
}

KC_API kcError_t kcGgmlBackendGetProfile(kcGgmlBackend_t backend, kcGgmlProfileEntry* entries, int capacity,
                                         int* count) noexcept {
    if (!backend) return kc::Error::InvalidResourceHandle;
    if (!count || capacity < 0 || (capacity > 0 && !entries)) return bad("null count, or capacity without entries");
    *count = int(backend->per_kernel.size());
    int i = 0;
    for (const auto& [name, tc] : backend->per_kernel) {
        if (i == capacity) break;
        kcGgmlProfileEntry& e = entries[i++];
        std::snprintf(e.name, sizeof e.name, "%s", name.c_str());
        e.launches = tc.first;
        e.ms = tc.second;
    }
    return ok;
}
