// gguf_model.cpp -- kcModelLoadGguf: a model from a GGUF file (llama.cpp's tensor names and
// metadata keys), through the reader of gguf.cpp and the public model calls.
//
// Follows the reference loader (llm/gguf_model.cpp:51-106): hyperparameters from
// "<arch>.embedding_length", ".feed_forward_length", ".block_count", ".attention.head_count",
// ".attention.head_count_kv" (default: head_count), ".attention.key_length" (default:
// embedding_length / head_count), ".attention.layer_norm_rms_epsilon" (default 1e-5),
// ".rope.freq_base" (default 10000); the vocabulary from token_embd's rows; output.weight absent
// means the head is token_embd (tied embeddings); rope_freqs.weight, when present, gives the RoPE
// frequency factors. The reference reads "llama" files only; "qwen3" is read here too (NEOX RoPE
// pairs and the per-head attn_q_norm / attn_k_norm), the architecture of BASELINE config 5.
// Matrices may be Q4_K or Q6_K each (a Q4_K_M file mixes them); norms are f32.
#include <cstring>
#include <climits>
#include <cmath>
#include <string>

#include "internal.hpp"
#include "kernelcore/gguf.h"
#include "kernelcore/model.h"

namespace {

using E = kcError_t;
constexpr E ok = kc::Error::Success;

struct Closer {
    kcGguf_t g;
    ~Closer() { (void)kcGgufClose(g); }
};

E fail(const std::string& why) {
    kcamd::setDetail("gguf model: %s", why.c_str());
    return kc::Error::InvalidValue;
}

// The file's type id as the model's qtype (KC_QTYPE_*), or -1.
int qtypeOfGgml(int t) {
    switch (t) {
        case KC_GGML_F32: return KC_QTYPE_F32;
        case KC_GGML_F16: return KC_QTYPE_F16;
        case KC_GGML_Q4_K: return KC_QTYPE_Q4_K;
        case KC_GGML_Q6_K: return KC_QTYPE_Q6_K;
        default: return -1;
    }
}

// Uploads tensor `name` of the file as model tensor `id` (layer `layer`), checking its type and
// shape against what the model expects.
E setFrom(kcGguf_t g, kcModel_t m, const std::string& name, int id, int layer) {
    int type = 0, nd = 0;
    int64_t ne[4] = {};
    size_t bytes = 0;
    const void* data = nullptr;
    if (kcGgufTensorInfo(g, name.c_str(), &type, &nd, ne, &bytes, &data) != ok) return fail("missing tensor " + name);
    const int qt = qtypeOfGgml(type);
    if (qt < 0) return fail("tensor " + name + ": ggml type " + std::to_string(type) + " not supported (Q4_K, Q6_K, F16, F32)");
    int want_qt = 0, rows = 0, k = 0;
    if (E e = kcModelTensorInfo(m, id, layer, &want_qt, &rows, &k, nullptr); e != ok) return e;
    const bool vec = want_qt == KC_QTYPE_F32;
    if (vec != (qt == KC_QTYPE_F32)) return fail("tensor " + name + ": f32 where a matrix is expected, or the reverse");
    const int64_t f_rows = nd > 1 ? ne[1] : 1;
    if (ne[0] != k || f_rows != rows || (nd > 2 && ne[2] != 1) || (nd > 3 && ne[3] != 1))
        return fail("tensor " + name + ": shape " + std::to_string(ne[0]) + " x " + std::to_string(f_rows) +
                    ", expected " + std::to_string(k) + " x " + std::to_string(rows));
    return kcModelSetTensorTyped(m, id, layer, qt, data, bytes);
}

}  // namespace

kcError_t kcModelLoadGguf(const char* path, int max_ctx, int max_batch, kcModel_t* out) noexcept {
    if (!out) return kc::Error::InvalidValue;
    *out = nullptr;
    kcGguf_t g = nullptr;
    if (E e = kcGgufOpen(path, &g); e != ok) return e;
    Closer closer{g};
    try {
        const char* as = nullptr;
        size_t an = 0;
        if (kcGgufGetStr(g, "general.architecture", &as, &an) != ok) return fail("no general.architecture");
        const std::string arch(as, an);
        if (arch != "llama" && arch != "qwen3") return fail("architecture " + arch + " not supported (llama, qwen3)");
        auto num = [&](const char* key, double fallback, bool required, double* v) -> bool {
            if (kcGgufGetNum(g, (arch + "." + key).c_str(), v) == ok) return true;
            *v = fallback;
            return !required;
        };
        double n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim, eps, theta, rope_dims;
        if (!num("block_count", 0, true, &n_layer) || !num("embedding_length", 0, true, &n_embd) ||
            !num("feed_forward_length", 0, true, &n_ff) || !num("attention.head_count", 0, true, &n_head))
            return fail("missing hyperparameters (block_count, embedding_length, feed_forward_length, "
                        "attention.head_count)");
        num("attention.head_count_kv", n_head, false, &n_head_kv);
        num("attention.key_length", n_head > 0 ? n_embd / n_head : 0, false, &head_dim);
        num("attention.layer_norm_rms_epsilon", 1e-5, false, &eps);
        num("rope.freq_base", 10000.0, false, &theta);
        num("rope.dimension_count", head_dim, false, &rope_dims);
        // every count must be a whole number in [1, INT_MAX] before it becomes an int
        const struct {
            const char* key;
            double v;
        } counts[] = {{"block_count", n_layer},
                      {"embedding_length", n_embd},
                      {"feed_forward_length", n_ff},
                      {"attention.head_count", n_head},
                      {"attention.head_count_kv", n_head_kv},
                      {"attention.key_length", head_dim},
                      {"rope.dimension_count", rope_dims}};
        for (const auto& k : counts)
            if (!std::isfinite(k.v) || k.v < 1.0 || k.v > double(INT_MAX) || k.v != std::floor(k.v))
                return fail(arch + "." + k.key + " is not a whole number in [1, 2^31 - 1]");
        if (!std::isfinite(eps) || !(eps > 0.0) || !std::isfinite(theta) || !(theta > 0.0) || theta > 3.0e38)
            return fail("rms epsilon and rope.freq_base must be positive finite numbers");
        if (rope_dims != head_dim) return fail("partial rotary embeddings (rope.dimension_count) not supported");
        int type = 0, nd = 0;
        int64_t ne[4] = {};
        if (kcGgufTensorInfo(g, "token_embd.weight", &type, &nd, ne, nullptr, nullptr) != ok)
            return fail("missing tensor token_embd.weight");
        kcModelConfig c{};
        c.n_layer = int(n_layer);
        c.n_embd = int(n_embd);
        c.n_head = int(n_head);
        c.n_head_kv = int(n_head_kv);
        c.head_dim = int(head_dim);
        c.n_ff = int(n_ff);
        c.n_vocab = int(nd > 1 ? ne[1] : 0);
        c.norm_eps = float(eps);
        c.rope_theta = float(theta);
        c.rope_neox = arch == "qwen3";
        c.qk_norm = arch == "qwen3";
        c.max_ctx = max_ctx;
        c.max_batch = max_batch;
        kcModel_t m = nullptr;
        if (E e = kcModelCreate(&c, &m); e != ok) return e;
        auto set = [&](const std::string& name, int id, int layer) { return setFrom(g, m, name, id, layer); };
        E e = set("token_embd.weight", KC_TENSOR_TOKEN_EMBD, 0);
        if (e == ok) e = set("output_norm.weight", KC_TENSOR_OUTPUT_NORM, 0);
        if (e == ok) {  // tied embeddings: no output.weight, the head is token_embd
            int t2 = 0;
            const bool has_out = kcGgufTensorInfo(g, "output.weight", &t2, nullptr, nullptr, nullptr, nullptr) == ok;
            e = set(has_out ? "output.weight" : "token_embd.weight", KC_TENSOR_OUTPUT, 0);
        }
        if (e == ok && kcGgufTensorInfo(g, "rope_freqs.weight", &type, nullptr, nullptr, nullptr, nullptr) == ok)
            e = set("rope_freqs.weight", KC_TENSOR_ROPE_FREQS, 0);
        static const struct {
            const char* name;
            int id;
        } per_layer[] = {{"attn_norm", KC_TENSOR_ATTN_NORM}, {"attn_q", KC_TENSOR_WQ},
                         {"attn_k", KC_TENSOR_WK},           {"attn_v", KC_TENSOR_WV},
                         {"attn_output", KC_TENSOR_WO},      {"ffn_norm", KC_TENSOR_FFN_NORM},
                         {"ffn_gate", KC_TENSOR_W_GATE},     {"ffn_up", KC_TENSOR_W_UP},
                         {"ffn_down", KC_TENSOR_W_DOWN},     {"attn_q_norm", KC_TENSOR_Q_NORM},
                         {"attn_k_norm", KC_TENSOR_K_NORM}};
        for (int l = 0; e == ok && l < c.n_layer; ++l)
            for (const auto& t : per_layer) {
                if ((t.id == KC_TENSOR_Q_NORM || t.id == KC_TENSOR_K_NORM) && !c.qk_norm) continue;
                e = set("blk." + std::to_string(l) + "." + t.name + ".weight", t.id, l);
                if (e != ok) break;
            }
        if (e != ok) {  // (the runtime calls of the cleanup clear the detail text: keep it)
            const char* d = kcGetLastErrorDetail();
            const std::string why = d ? d : "";
            (void)kcModelDestroy(m);
            if (!why.empty()) kcamd::setDetail("%s", why.c_str());
            return e;
        }
        *out = m;
        return ok;
    } catch (const std::bad_alloc&) {
        kcamd::setDetail("gguf model: out of host memory");
        return kc::Error::OutOfMemory;
    } catch (...) {
        kcamd::setDetail("gguf model: internal error");
        return kc::Error::InternalError;
    }
}
