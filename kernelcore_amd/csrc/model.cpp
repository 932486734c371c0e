// model.cpp -- the decode driver (include/kernelcore/model.h): a Llama / Qwen3-architecture
// transformer with K-quant weights on the kc* runtime and the built-in kernels.
//
// Op order follows the reference's ggml backend graph for one layer (docs/cuda_cpu_poc_plan.md:1158
// in arasheedu/Kernelcore; backend dispatch ggml-kernelcore.cpp:555-589, fusions :743-769):
// single tokens take per-32 activation slots and the matvecs (mul_mat_impl with ncols == 1),
// batches take per-256 slots and the matmuls (batch_k256). As llama.cpp does for a prompt, the
// last layer continues after the attention output projection with the last token only, so
// its FFN, the output norm and the head run on one row (the decode kernels).
#include <hip/hip_runtime.h>
#include <kernelcore/model.h>

#include <array>
#include <cmath>
#include <cstring>
#include <memory>
#include <new>
#include <vector>

#include "internal.hpp"
#include "kdecode.hpp"
#include "kquant.hpp"
#include "launch.hpp"
#include "model_kernels.hpp"

namespace {

struct Layer {
    void *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr, *wg = nullptr, *wu = nullptr, *wd = nullptr;
    float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    int *kcache = nullptr, *vcache = nullptr;
    int q6[KC_TENSOR_COUNT] = {};   // per matrix: 1 if its weights are Q6_K (set with the tensor)
    int f16[KC_TENSOR_COUNT] = {};  // per matrix: 1 if its weights are F16 (row-major, matmul_f16)
};

// The type a tensor takes by default (kcModelSetTensor); kcModelSetTensorTyped may choose the
// other K-quant for any matrix.
int qtypeOf(int tensor) {
    switch (tensor) {
        case KC_TENSOR_OUTPUT_NORM:
        case KC_TENSOR_ATTN_NORM:
        case KC_TENSOR_FFN_NORM:
        case KC_TENSOR_Q_NORM:
        case KC_TENSOR_K_NORM:
        case KC_TENSOR_ROPE_FREQS: return KC_QTYPE_F32;
        case KC_TENSOR_OUTPUT:
        case KC_TENSOR_WV:
        case KC_TENSOR_W_DOWN: return KC_QTYPE_Q6_K;
        default: return KC_QTYPE_Q4_K;
    }
}

bool perLayer(int tensor) { return tensor >= KC_TENSOR_ATTN_NORM && tensor != KC_TENSOR_ROPE_FREQS; }

}  // namespace

struct kcModel_st {
    kcModelConfig c{};
    kcStream_t ks = nullptr;
    hipStream_t s = nullptr;
    std::vector<Layer> L;
    void *tok_embd = nullptr, *output = nullptr;
    int q6_tok = 0, q6_out = 1;  // 1 if the embedding / head matrix is Q6_K
    float* out_norm = nullptr;
    float* ones = nullptr;  // RoPE frequency factors: ones unless KC_TENSOR_ROPE_FREQS is set
    bool rope_freqs_set = false;
    // activations, sized for max_batch tokens
    float *x = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *qr = nullptr, *kr = nullptr;
    float *att = nullptr, *o = nullptr, *gate = nullptr, *up = nullptr, *sw = nullptr, *down = nullptr;
    // second K-range partial sums of the batch's o / down products, and of v's (a Q6_K v among Q4_K
    // q and k: the grouped launch may split it alone)
    float *o2 = nullptr, *down2 = nullptr, *v2 = nullptr;
    // the batch's quantized activations in the MFMA matmul's layout (kcamd::ActF16), for inputs of
    // n_embd, n_head * head_dim and n_ff values
    char *actE = nullptr, *actQ = nullptr, *actF = nullptr;
    float* logits = nullptr;
    int *slotE32 = nullptr, *slotEK = nullptr, *slotQ32 = nullptr, *slotQK = nullptr, *slotF32 = nullptr,
        *slotFK = nullptr;
    int *tokens = nullptr, *pos = nullptr, *n_past = nullptr, *n_ctx = nullptr, *gen = nullptr, *step = nullptr;
    float* attn_part = nullptr;  // split-context attention partials (fused decode)
    long long* idx = nullptr;
    int max_gen = 4096;
    int pos_host = 0;
    kcGraph_t step_graph = nullptr;
    std::vector<void*> allocs;
};

namespace {

using E = kcError_t;
constexpr E ok = kc::Error::Success;
inline E err(int c) { return static_cast<E>(c); }

#define KM_TRY(expr)                    \
    do {                                \
        if (int e_ = (expr)) return err(e_); \
    } while (0)
#define KI_TRY(expr)                    \
    do {                                \
        if (int e_ = (expr)) return e_; \
    } while (0)
#define KM_TRYE(expr)                   \
    do {                                \
        if (E e_ = (expr); e_ != ok) return e_; \
    } while (0)

E alloc(kcModel_st* m, void** p, size_t bytes) {
    KM_TRYE(kcMalloc(p, bytes));
    m->allocs.push_back(*p);
    return ok;
}
template <class T>
E allocT(kcModel_st* m, T** p, size_t count) {
    void* v = nullptr;
    KM_TRYE(alloc(m, &v, count * sizeof(T)));
    *p = static_cast<T*>(v);
    return ok;
}

void shapeOf(const kcModelConfig& c, int tensor, int* rows, int* k) {
    const int Q = c.n_head * c.head_dim, KV = c.n_head_kv * c.head_dim;
    switch (tensor) {
        case KC_TENSOR_TOKEN_EMBD:
        case KC_TENSOR_OUTPUT: *rows = c.n_vocab, *k = c.n_embd; return;
        case KC_TENSOR_OUTPUT_NORM:
        case KC_TENSOR_ATTN_NORM:
        case KC_TENSOR_FFN_NORM: *rows = 1, *k = c.n_embd; return;
        case KC_TENSOR_Q_NORM:
        case KC_TENSOR_K_NORM: *rows = 1, *k = c.head_dim; return;
        case KC_TENSOR_ROPE_FREQS: *rows = 1, *k = c.head_dim / 2; return;
        case KC_TENSOR_WQ: *rows = Q, *k = c.n_embd; return;
        case KC_TENSOR_WK:
        case KC_TENSOR_WV: *rows = KV, *k = c.n_embd; return;
        case KC_TENSOR_WO: *rows = c.n_embd, *k = Q; return;
        case KC_TENSOR_W_GATE:
        case KC_TENSOR_W_UP: *rows = c.n_ff, *k = c.n_embd; return;
        case KC_TENSOR_W_DOWN: *rows = c.n_embd, *k = c.n_ff; return;
        default: *rows = *k = 0;
    }
}

size_t ggmlBytes(int qtype, int rows, int k) {
    if (qtype == KC_QTYPE_F32) return size_t(rows) * k * 4;
    if (qtype == KC_QTYPE_F16) return size_t(rows) * k * 2;
    return size_t(rows) * (k / 256) * (qtype == KC_QTYPE_Q6_K ? 210 : 144);
}

// ---- one decode step (one token, per-32 slots, matvecs) -----------------------------------

int matvec(bool q6, const void* w, const int* slot, float* y, int rows, int k, hipStream_t s) {
    kcMatvecQ4Q8Args a{static_cast<const int*>(w), slot, reinterpret_cast<const float*>(slot + k / 32 * 8), y, nullptr,
                       rows, k};
    return kcamd::launchMatvecKq(q6, a, s);
}

// Layer matrix t times one token: a K-quant matvec of the per-32 slot, or for F16 weights
// matmul_f16 of the same activations in f32 (xf), as the reference's MUL_MAT dispatch does
// (ggml-kernelcore.cpp:559-566).
int proj(const Layer& l, int t, const void* w, const int* slot, const float* xf, float* y, int rows, int k,
         hipStream_t s) {
    if (l.f16[t]) return kcamd::launchMatmulF16(w, xf, y, rows, k, 1, s);
    return matvec(l.q6[t], w, slot, y, rows, k, s);
}

bool anyF16(const kcModel_st* m) {
    for (const auto& l : m->L)
        for (int t = 0; t < KC_TENSOR_COUNT; ++t)
            if (l.f16[t]) return true;
    return false;
}

int normQ8(const float* x, const float* w, float* y, int* slot, int n, float eps, hipStream_t s) {
    kcNormMulQ8Args a{x, w, y, slot, nullptr, n, 1, eps};
    return kcamd::launchNormMulQ8(false, a, s);
}

// FFN of one token (row x of the residual stream, whose per-32 partial sums are in slotE32):
// norm, gate/up, SwiGLU + quantization, down. Leaves the result in m->down (1 row).
int ffnOne(kcModel_st* m, const Layer& l, float* x, hipStream_t s) {
    const auto& c = m->c;
    KI_TRY(normQ8(x, l.ffn_norm, m->xn, m->slotE32, c.n_embd, c.norm_eps, s));
    KI_TRY(proj(l, KC_TENSOR_W_GATE, l.wg, m->slotE32, m->xn, m->gate, c.n_ff, c.n_embd, s));
    KI_TRY(proj(l, KC_TENSOR_W_UP, l.wu, m->slotE32, m->xn, m->up, c.n_ff, c.n_embd, s));
    kcSiluMulQ8FArgs sa{m->gate, m->up, m->sw, m->slotF32, nullptr, c.n_ff, 1};
    KI_TRY(kcamd::launchSiluMulQ8(false, sa, s));
    return proj(l, KC_TENSOR_W_DOWN, l.wd, m->slotF32, m->sw, m->down, c.n_embd, c.n_ff, s);
}

// Output norm + head for the row x (partial sums in slotE32) into m->logits.
int headOne(kcModel_st* m, float* x, hipStream_t s) {
    const auto& c = m->c;
    KI_TRY(normQ8(x, m->out_norm, m->xn, m->slotE32, c.n_embd, c.norm_eps, s));
    return matvec(m->q6_out, m->output, m->slotE32, m->logits, c.n_vocab, c.n_embd, s);
}

// RoPE of q and k (after the optional per-head norm) into m->qr / m->kr.
int ropeQK(kcModel_st* m, int n, hipStream_t s) {
    const auto& c = m->c;
    const float l2b = std::log2(c.rope_theta);
    const float* qin = c.qk_norm ? m->att : m->q;  // the normed q lives in m->att until attention
    const float* kin = c.qk_norm ? m->kr : m->k;
    float* kout = c.qk_norm ? m->k : m->kr;
    kcRopeGgmlArgs rq{qin, m->qr, m->pos, m->ones, nullptr, c.head_dim, c.n_head, n, l2b, c.rope_neox != 0};
    KI_TRY(kcamd::launchRope(rq, s));
    kcRopeGgmlArgs rk{kin, kout, m->pos, m->ones, nullptr, c.head_dim, c.n_head_kv, n, l2b, c.rope_neox != 0};
    return kcamd::launchRope(rk, s);
}

// Qwen3: per-head RMS norm of q (into m->att, free until the attention) and k (into m->kr).
int qkNorm(kcModel_st* m, const Layer& l, int n, hipStream_t s) {
    const auto& c = m->c;
    if (!c.qk_norm) return 0;
    kcRmsNormArgs qa{m->q, l.q_norm, m->att, c.head_dim, c.n_head * n, c.norm_eps};
    KI_TRY(kcamd::launchRmsNorm(qa, s));
    kcRmsNormArgs ka{m->k, l.k_norm, m->kr, c.head_dim, c.n_head_kv * n, c.norm_eps};
    return kcamd::launchRmsNorm(ka, s);
}

// The roped k of this step: m->kr, or m->k when the per-head norm used m->kr.
const float* ropedK(const kcModel_st* m) { return m->c.qk_norm ? m->k : m->kr; }

int kvStore(kcModel_st* m, const Layer& l, int n, hipStream_t s) {
    const auto& c = m->c;
    const int KV = c.n_head_kv * c.head_dim;
    kcSetRowsF16Args ka{ropedK(m), reinterpret_cast<const int*>(m->idx), l.kcache, nullptr, KV / 2, n, KV, KV / 2,
                        c.max_ctx};
    KI_TRY(kcamd::launchSetRows(ka, s));
    kcSetRowsF16Args va{m->v, reinterpret_cast<const int*>(m->idx), l.vcache, nullptr, KV / 2, n, KV, KV / 2,
                        c.max_ctx};
    return kcamd::launchSetRows(va, s);
}

int attention(kcModel_st* m, const Layer& l, int n, hipStream_t s) {
    const auto& c = m->c;
    kcamd::AttnShape a{n, c.n_head, c.n_head_kv, c.head_dim, c.n_head * c.head_dim, c.n_head_kv * c.head_dim / 2,
                       c.max_ctx, n > 1 ? 1 : 0, 1.0f / std::sqrt((float)c.head_dim)};
    return kcamd::launchAttn(m->qr, l.kcache, l.vcache, m->att, m->n_ctx, a, s);
}

// The kernels of one token at position *n_past, reading its id from m->tokens[0]; leaves the
// logits in m->logits.
int decodeStep(kcModel_st* m, hipStream_t s) {
    const auto& c = m->c;
    const int Q = c.n_head * c.head_dim, KV = c.n_head_kv * c.head_dim;
    KI_TRY(kcamd::launchPositions(m->n_past, 1, m->pos, m->idx, m->n_ctx, s));
    KI_TRY(kcamd::launchGetRows(m->q6_tok, m->tok_embd, m->tokens, m->x, 1, c.n_embd, c.n_vocab, s));
    for (int li = 0; li < c.n_layer; ++li) {
        const Layer& l = m->L[li];
        if (li == 0) KI_TRY(kcamd::launchAddSumsq(nullptr, m->x, nullptr, m->slotE32, c.n_embd, 1, s));
        else KI_TRY(kcamd::launchAddSumsq(m->x, m->down, m->x, m->slotE32, c.n_embd, 1, s));
        KI_TRY(normQ8(m->x, l.attn_norm, m->xn, m->slotE32, c.n_embd, c.norm_eps, s));
        KI_TRY(proj(l, KC_TENSOR_WQ, l.wq, m->slotE32, m->xn, m->q, Q, c.n_embd, s));
        KI_TRY(proj(l, KC_TENSOR_WK, l.wk, m->slotE32, m->xn, m->k, KV, c.n_embd, s));
        KI_TRY(proj(l, KC_TENSOR_WV, l.wv, m->slotE32, m->xn, m->v, KV, c.n_embd, s));
        KI_TRY(qkNorm(m, l, 1, s));
        KI_TRY(ropeQK(m, 1, s));
        KI_TRY(kvStore(m, l, 1, s));
        KI_TRY(attention(m, l, 1, s));
        KI_TRY(kcamd::launchQuantizeQ8x4(m->att, m->slotQ32, reinterpret_cast<float*>(m->slotQ32 + Q / 32 * 8), Q / 32, s));
        KI_TRY(proj(l, KC_TENSOR_WO, l.wo, m->slotQ32, m->att, m->o, c.n_embd, Q, s));
        KI_TRY(kcamd::launchAddSumsq(m->x, m->o, m->x, m->slotE32, c.n_embd, 1, s));
        KI_TRY(ffnOne(m, l, m->x, s));
    }
    KI_TRY(kcamd::launchAddSumsq(m->x, m->down, m->x, m->slotE32, c.n_embd, 1, s));
    return headOne(m, m->x, s);
}

// The same step in six launches per layer (kdecode.hip): norm + q/k/v matvecs; q/k norm + RoPE +
// cache store + split-context attention; its merge + quantization; output projection + residual;
// norm + gate/up + SwiGLU + quantization; down projection + residual. decode_path 3 runs the
// merge's first form (one workgroup per KV head), bit-identical.
int qkvTiles() { return kcamd::option("qkv_tiles") > 0 ? kcamd::option("qkv_tiles") : 2; }  // 2: the 8-lane norm prologue

// Whether the six fused kernels have a launch shape for these widths (host only).
bool fusedShapesFit(const kcModelConfig& c, int qkv_tiles) {
    const int Q = c.n_head * c.head_dim;
    return kcamd::planDecodeMatvec(kcamd::kProNorm, kcamd::kEpiStore, c.n_embd, qkv_tiles).nw &&
           kcamd::planDecodeMatvec(kcamd::kProSlot, kcamd::kEpiResid, Q, 1).nw &&
           kcamd::planDecodeMatvec(kcamd::kProNorm, kcamd::kEpiSwiglu, c.n_embd, 2).nw &&
           kcamd::planDecodeMatvec(kcamd::kProSlot, kcamd::kEpiResid, c.n_ff, 1).nw && kcamd::rmsQ8Supports(c.n_embd) &&
           kcamd::attnDecodeSupports(c.head_dim, c.n_head / c.n_head_kv);
}

bool fusedDecode(const kcModel_st* m) {
    for (const auto& l : m->L)  // the SwiGLU matvec runs gate and up as one type
        if (l.q6[KC_TENSOR_W_GATE] != l.q6[KC_TENSOR_W_UP]) return false;
    if (anyF16(m)) return false;  // the fused matvecs take K-quant weights only
    return kcamd::option("decode_path") != 1 && fusedShapesFit(m->c, qkvTiles());
}

int decodeStepFused(kcModel_st* m, hipStream_t s) {
    const auto& c = m->c;
    const int E_ = c.n_embd, Q = c.n_head * c.head_dim, KV = c.n_head_kv * c.head_dim, F = c.n_ff;
    KI_TRY(kcamd::launchPositions(m->n_past, 1, m->pos, m->idx, m->n_ctx, s));
    KI_TRY(kcamd::launchGetRows(m->q6_tok, m->tok_embd, m->tokens, m->x, 1, E_, c.n_vocab, s));
    for (int li = 0; li < c.n_layer; ++li) {
        const Layer& l = m->L[li];
        kcamd::DmvArgs qa{};
        qa.p0 = {l.wq, m->q, Q, l.q6[KC_TENSOR_WQ], 0, 0};
        qa.p1 = {l.wk, m->k, KV, l.q6[KC_TENSOR_WK], 0, 0};
        qa.p2 = {l.wv, m->v, KV, l.q6[KC_TENSOR_WV], 0, 0};
        qa.nparts = 3;
        qa.k = E_;
        qa.tpw = qkvTiles();
        qa.x = m->x;
        qa.nw = l.attn_norm;
        qa.eps = c.norm_eps;
        KI_TRY(kcamd::launchDecodeMatvec(kcamd::kProNorm, kcamd::kEpiStore, qa, s));
        if (kcamd::option("decode_path") == 2) {  // diagnostic: the unfused attention kernels
            KI_TRY(qkNorm(m, l, 1, s));
            KI_TRY(ropeQK(m, 1, s));
            KI_TRY(kvStore(m, l, 1, s));
            KI_TRY(attention(m, l, 1, s));
            KI_TRY(kcamd::launchQuantizeQ8x4(m->att, m->slotQ32, reinterpret_cast<float*>(m->slotQ32 + Q / 32 * 8),
                                             Q / 32, s));
        } else {
        kcamd::QkPostArgs pa{m->q, m->k, m->v, m->qr, l.kcache, l.vcache, m->pos, m->ones, l.q_norm, l.k_norm,
                             c.n_head, c.n_head_kv, c.head_dim, KV / 2, c.qk_norm, c.rope_neox,
                             std::log2(c.rope_theta), c.norm_eps};
        kcamd::AttnDecodeArgs aa{pa, m->attn_part, m->slotQ32, c.n_head / c.n_head_kv, 0, Q / 32,
                                 1.0f / std::sqrt((float)c.head_dim)};
        KI_TRY(kcamd::launchAttnDecode(aa, c.head_dim, c.n_head_kv, c.max_ctx, s, kcamd::option("decode_path") == 3));
        }
        kcamd::DmvArgs oa{};
        oa.p0 = {l.wo, m->x, E_, l.q6[KC_TENSOR_WO], 0, 0};
        oa.nparts = 1;
        oa.k = Q;
        oa.tpw = 1;
        oa.xq = m->slotQ32;
        oa.xd = reinterpret_cast<const float*>(m->slotQ32 + Q / 32 * 8);
        KI_TRY(kcamd::launchDecodeMatvec(kcamd::kProSlot, kcamd::kEpiResid, oa, s));
        kcamd::DmvArgs fa{};
        fa.p0 = {l.wg, nullptr, F, l.q6[KC_TENSOR_W_GATE], 0, 0};
        fa.p1 = {l.wu, nullptr, F, l.q6[KC_TENSOR_W_UP], 0, 0};
        fa.nparts = 2;
        fa.k = E_;
        fa.tpw = 2;
        fa.x = m->x;
        fa.nw = l.ffn_norm;
        fa.eps = c.norm_eps;
        fa.qout = m->slotF32;
        KI_TRY(kcamd::launchDecodeMatvec(kcamd::kProNorm, kcamd::kEpiSwiglu, fa, s));
        kcamd::DmvArgs da{};
        da.p0 = {l.wd, m->x, E_, l.q6[KC_TENSOR_W_DOWN], 0, 0};
        da.nparts = 1;
        da.k = F;
        da.tpw = 1;
        da.xq = m->slotF32;
        da.xd = reinterpret_cast<const float*>(m->slotF32 + F / 32 * 8);
        KI_TRY(kcamd::launchDecodeMatvec(kcamd::kProSlot, kcamd::kEpiResid, da, s));
    }
    KI_TRY(kcamd::launchRmsQ8(m->x, m->out_norm, m->slotE32, E_, c.norm_eps, s));
    return matvec(m->q6_out, m->output, m->slotE32, m->logits, c.n_vocab, E_, s);
}

int decodeAny(kcModel_st* m, hipStream_t s) { return fusedDecode(m) ? decodeStepFused(m, s) : decodeStep(m, s); }

// The matrices t[0..nm) of a layer that read the same batch activations: the K-quant ones in one
// grouped MFMA launch on the per-256 slots, each F16 one as matmul_f16 of the f32 rows xf. A matrix
// with a second output y2[i] may be split over K (*split)[i]: its product is then y[i] + y2[i].
int batchProj(const Layer& l, std::array<int, 3> t, std::array<const void*, 3> w,
              std::array<float*, 3> y, std::array<int, 3> rows, int nm, const int* slot, const float* xf, int k, int n,
              hipStream_t s, const kcamd::ActF16* act, std::array<float*, 3> y2 = {},
              std::array<bool, 3>* split = nullptr) {
    kcamd::MmPart parts[3];
    int at[3], np = 0;
    for (int i = 0; i < nm; ++i) {
        if (split) (*split)[i] = false;
        if (l.f16[t[i]]) {
            KI_TRY(kcamd::launchMatmulF16(w[i], xf, y[i], rows[i], k, n, s));
        } else {
            at[np] = i;
            parts[np++] = kcamd::MmPart{w[i], {y[i], split ? y2[i] : nullptr}, rows[i], l.q6[t[i]]};
        }
    }
    if (!np) return 0;
    int ks = 1, pks[3] = {1, 1, 1};
    KI_TRY(kcamd::launchMatmulGroup(parts, np, slot, k, n, 1, &ks, s, act, split ? pks : nullptr));
    if (split)
        for (int j = 0; j < np; ++j) (*split)[at[j]] = pks[j] == 2;
    return 0;
}

// n > 1 tokens (m->tokens[0..n)) at positions *n_past ..: per-256 slots and the matmuls.
int batchStep(kcModel_st* m, int n, hipStream_t s) {
    const auto& c = m->c;
    const int Q = c.n_head * c.head_dim, KV = c.n_head_kv * c.head_dim;
    const int E_ = c.n_embd;
    KI_TRY(kcamd::launchPositions(m->n_past, n, m->pos, m->idx, m->n_ctx, s));
    KI_TRY(kcamd::launchGetRows(m->q6_tok, m->tok_embd, m->tokens, m->x, n, E_, c.n_vocab, s));
    float* x_last = m->x + (size_t)(n - 1) * E_;
    // the products that read the same activations share one launch; o and down split K in two where
    // one K range would leave CUs idle (the two partial sums are added in the residual add that
    // consumes them)
    const float* down2 = nullptr;
    int ks = 1;
    // the quantizers also write the MFMA layout, so the matmuls launch no conversion
    const int B = c.max_batch;
    const kcamd::ActF16 vE = kcamd::actF16View(m->actE, B, E_, n), vQ = kcamd::actF16View(m->actQ, B, Q, n),
                        vF = kcamd::actF16View(m->actF, B, c.n_ff, n);
    const bool pre = kcamd::option("prefill_act") == 0;  // 1: the matmuls convert the slots themselves
    const kcamd::ActF16 *aE = pre ? &vE : nullptr, *aQ = pre ? &vQ : nullptr, *aF = pre ? &vF : nullptr;
    // the int8 slots only where a product reads them (given the MFMA layout, the grouped matmul reads
    // only that): the quantizers then write about 40% fewer bytes
    int* sE = pre && kcamd::matmulGroupReadsActOnly(n, E_) ? nullptr : m->slotEK;
    int* sQ = pre && kcamd::matmulGroupReadsActOnly(n, Q) ? nullptr : m->slotQK;
    int* sF = pre && kcamd::matmulGroupReadsActOnly(n, c.n_ff) ? nullptr : m->slotFK;
    for (int li = 0; li < c.n_layer; ++li) {
        const Layer& l = m->L[li];
        // residual add (layer 0: the embeddings) + RMS norm + per-256 quantization in one kernel
        // (also the normed rows in f32 when an F16 matrix reads them)
        const bool f16_qkv = l.f16[KC_TENSOR_WQ] || l.f16[KC_TENSOR_WK] || l.f16[KC_TENSOR_WV];
        float* yq = f16_qkv ? m->xn : nullptr;
        if (li == 0) KI_TRY(kcamd::launchAddNormQ8K(nullptr, m->x, nullptr, nullptr, l.attn_norm, sE, E_, n,
                                                    c.norm_eps, s, aE, yq));
        else KI_TRY(kcamd::launchAddNormQ8K(m->x, m->down, down2, m->x, l.attn_norm, sE, E_, n, c.norm_eps, s,
                                            aE, yq));
        std::array<bool, 3> split{};  // (v may run in two K ranges: stored as v + v2)
        KI_TRY(batchProj(l, {KC_TENSOR_WQ, KC_TENSOR_WK, KC_TENSOR_WV}, {l.wq, l.wk, l.wv}, {m->q, m->k, m->v},
                         {Q, KV, KV}, 3, m->slotEK, m->xn, E_, n, s, aE, {nullptr, nullptr, m->v2}, &split));
        // RoPE of q and k with the fp16 cache stores of k and v in one kernel, Qwen3's per-head q / k
        // norms in the same launch (option qk_fuse = 1: the norms as launches of their own)
        const bool fuse = c.qk_norm && kcamd::option("qk_fuse") != 1 && (c.head_dim == 64 || c.head_dim == 128);
        if (fuse) {
            KI_TRY(kcamd::launchNormRopeQKStore(m->q, m->qr, m->k, m->v, l.q_norm, l.k_norm, l.kcache, l.vcache, m->pos,
                                                m->ones, c.head_dim, c.n_head, c.n_head_kv, n, std::log2(c.rope_theta),
                                                c.rope_neox, KV / 2, c.max_ctx, c.norm_eps, s,
                                                split[2] ? m->v2 : nullptr));
        } else {
            KI_TRY(qkNorm(m, l, n, s));
            KI_TRY(kcamd::launchRopeQKStore(c.qk_norm ? m->att : m->q, m->qr, c.qk_norm ? m->kr : m->k, m->v, l.kcache,
                                            l.vcache, m->pos, m->ones, c.head_dim, c.n_head, c.n_head_kv, n,
                                            std::log2(c.rope_theta), c.rope_neox, KV / 2, c.max_ctx, s,
                                            split[2] ? m->v2 : nullptr));
        }
        KI_TRY(attention(m, l, n, s));
        const float* o2 = nullptr;
        if (l.f16[KC_TENSOR_WO]) {
            KI_TRY(kcamd::launchMatmulF16(l.wo, m->att, m->o, E_, Q, n, s));
        } else {
            KI_TRY(kcamd::launchQuantizeColsK(m->att, sQ, Q, n, s, aQ));
            const kcamd::MmPart op{l.wo, {m->o, m->o2}, E_, l.q6[KC_TENSOR_WO]};
            KI_TRY(kcamd::launchMatmulGroup(&op, 1, m->slotQK, Q, n, kcamd::matmulKs(E_, Q, n, op.q6 != 0), &ks, s,
                                            aQ));
            o2 = ks == 2 ? m->o2 : nullptr;
        }
        if (li + 1 < c.n_layer) {
            const bool f16_gu = l.f16[KC_TENSOR_W_GATE] || l.f16[KC_TENSOR_W_UP];
            KI_TRY(kcamd::launchAddNormQ8K(m->x, m->o, o2, m->x, l.ffn_norm, sE, E_, n, c.norm_eps, s, aE,
                                           f16_gu ? m->xn : nullptr));
            KI_TRY(batchProj(l, {KC_TENSOR_W_GATE, KC_TENSOR_W_UP, 0}, {l.wg, l.wu, nullptr},
                             {m->gate, m->up, nullptr}, {c.n_ff, c.n_ff, 0}, 2, m->slotEK, m->xn, E_, n, s, aE));
            // SwiGLU straight into the quantized form (and into f32 when the down matrix is F16)
            const bool f16_d = l.f16[KC_TENSOR_W_DOWN];
            kcSiluMulQ8FArgs sa{m->gate, m->up, f16_d ? m->sw : nullptr, sF, nullptr, c.n_ff, n};
            KI_TRY(kcamd::launchSiluMulQ8KAct(sa, aF, s));
            if (f16_d) {
                KI_TRY(kcamd::launchMatmulF16(l.wd, m->sw, m->down, E_, c.n_ff, n, s));
                down2 = nullptr;
            } else {
                const kcamd::MmPart dp{l.wd, {m->down, m->down2}, E_, l.q6[KC_TENSOR_W_DOWN]};
                KI_TRY(kcamd::launchMatmulGroup(&dp, 1, m->slotFK, c.n_ff, n, kcamd::matmulKs(E_, c.n_ff, n, dp.q6 != 0),
                                                &ks, s, aF));
                down2 = ks == 2 ? m->down2 : nullptr;
            }
        } else {  // the last layer continues with the last token only
            KI_TRY(kcamd::launchAddSumsq(x_last, m->o + (size_t)(n - 1) * E_, x_last, m->slotE32, E_, 1, s,
                                         o2 ? o2 + (size_t)(n - 1) * E_ : nullptr));
            KI_TRY(ffnOne(m, l, x_last, s));
        }
    }
    KI_TRY(kcamd::launchAddSumsq(x_last, m->down, x_last, m->slotE32, E_, 1, s));
    return headOne(m, x_last, s);
}

E checkModel(kcModel_t m) {
    if (!m) {
        kcamd::setDetail("model is null");
        return kc::Error::InvalidValue;
    }
    return ok;
}

E syncModel(kcModel_t m) { return kcStreamSynchronize(m->ks); }

// The widths every kernel of the driver handles. head_dim: 32, 64, 128 or 256 (the batch attention
// kernel's lanes split a head row in 16 parts of at least 2 values).
E checkConfig(const kcModelConfig& c) {
    if (c.n_layer <= 0 || c.n_embd <= 0 || c.n_embd % 256 || c.n_head <= 0 || c.n_head_kv <= 0 ||
        c.n_head % c.n_head_kv || c.head_dim <= 0 || c.head_dim % 16 || c.head_dim > 256 ||
        (c.n_head * c.head_dim) % 256 || (c.n_head_kv * c.head_dim) % 16 || c.n_ff <= 0 || c.n_ff % 256 ||
        c.n_vocab <= 0 || c.n_vocab % 8 || c.max_ctx <= 0 || c.max_ctx > 16384 || c.max_batch <= 0 ||
        c.max_batch > c.max_ctx || !(c.rope_theta > 0.0f)) {
        kcamd::setDetail("model config out of range (dims multiples of 256, head_dim a multiple of 16, max_ctx <= 16384)");
        return kc::Error::InvalidValue;
    }
    if (c.head_dim < 32 || 256 % c.head_dim) {
        kcamd::setDetail("head_dim must be 32, 64, 128 or 256");
        return kc::Error::InvalidValue;
    }
    return ok;
}

}  // namespace

kcError_t kcModelCreate(const kcModelConfig* cfg, kcModel_t* out) noexcept {
    if (!cfg || !out) return kc::Error::InvalidValue;
    *out = nullptr;
    const kcModelConfig& c = *cfg;
    if (E e = checkConfig(c); e != ok) return e;
    auto m = std::unique_ptr<kcModel_st>(new (std::nothrow) kcModel_st);
    if (!m) return kc::Error::OutOfMemory;
    m->c = c;
    auto fail = [&](E e) {
        for (void* p : m->allocs) (void)kcFree(p);
        if (m->ks) (void)kcStreamDestroy(m->ks);
        return e;
    };
    if (E e = kcStreamCreate(&m->ks); e != ok) return e;
    void* hs = nullptr;
    if (E e = kcStreamGetNative(m->ks, &hs); e != ok) return fail(e);
    m->s = static_cast<hipStream_t>(hs);
    const int B = c.max_batch, E_ = c.n_embd, Q = c.n_head * c.head_dim, KV = c.n_head_kv * c.head_dim, F = c.n_ff;
    m->L.resize(c.n_layer);
    for (auto& l : m->L)
        for (int t = 0; t < KC_TENSOR_COUNT; ++t) l.q6[t] = qtypeOf(t) == KC_QTYPE_Q6_K;
#define KM_A(ptr, count) \
    if (E e = allocT(m.get(), &(ptr), (size_t)(count)); e != ok) return fail(e)
    KM_A(m->x, (size_t)B * E_);
    KM_A(m->xn, (size_t)B * E_);
    KM_A(m->q, (size_t)B * Q);
    KM_A(m->qr, (size_t)B * Q);
    KM_A(m->k, (size_t)B * KV);
    KM_A(m->kr, (size_t)B * KV);
    KM_A(m->v, (size_t)B * KV);
    KM_A(m->v2, (size_t)B * KV);
    KM_A(m->att, (size_t)B * Q);
    KM_A(m->o, (size_t)B * E_);
    KM_A(m->o2, (size_t)B * E_);
    KM_A(m->gate, (size_t)B * F);
    KM_A(m->up, (size_t)B * F);
    KM_A(m->sw, (size_t)B * F);
    KM_A(m->down, (size_t)B * E_);
    KM_A(m->down2, (size_t)B * E_);
    KM_A(m->actE, kcamd::actF16Bytes(B, E_));
    KM_A(m->actQ, kcamd::actF16Bytes(B, Q));
    KM_A(m->actF, kcamd::actF16Bytes(B, F));
    KM_A(m->logits, (size_t)c.n_vocab);
    KM_A(m->slotE32, (size_t)E_ / 32 * 11);
    KM_A(m->slotEK, (size_t)B * (E_ / 256 * 85 + E_ / 32 * 11));
    KM_A(m->slotQ32, (size_t)Q / 32 * 11);
    KM_A(m->slotQK, (size_t)B * Q / 256 * 85);
    KM_A(m->slotF32, (size_t)F / 32 * 11);
    KM_A(m->slotFK, (size_t)B * F / 256 * 85);
    KM_A(m->tokens, (size_t)B);
    KM_A(m->pos, (size_t)B);
    KM_A(m->idx, (size_t)B);
    KM_A(m->n_past, 1);
    KM_A(m->n_ctx, 1);
    KM_A(m->gen, (size_t)m->max_gen);
    KM_A(m->step, 1);
    KM_A(m->ones, (size_t)c.head_dim / 2);
    KM_A(m->attn_part, kcamd::attnDecodePartFloats(c.n_head_kv, c.max_ctx, c.head_dim));
    for (auto& l : m->L) {
        KM_A(l.kcache, (size_t)c.max_ctx * KV / 2);
        KM_A(l.vcache, (size_t)c.max_ctx * KV / 2);
    }
#undef KM_A
    std::vector<float> ones(c.head_dim / 2, 1.0f);
    if (E e = kcMemcpy(m->ones, ones.data(), ones.size() * 4, kc::CopyKind::HostToDevice); e != ok) return fail(e);
    const int zero = 0;
    if (E e = kcMemcpy(m->n_past, &zero, 4, kc::CopyKind::HostToDevice); e != ok) return fail(e);
    for (auto [p, k] : {std::pair<void*, int>{m->actE, E_}, {m->actQ, Q}, {m->actF, F}})
        if (E e = kcMemset(p, 0, kcamd::actF16Bytes(B, k)); e != ok) return fail(e);
    *out = m.release();
    return ok;
}

kcError_t kcModelPlanDecode(const kcModelConfig* cfg, int* fused) noexcept {
    if (!cfg || !fused) return kc::Error::InvalidValue;
    if (E e = checkConfig(*cfg); e != ok) return e;
    *fused = fusedShapesFit(*cfg, qkvTiles()) ? 1 : 0;
    return ok;
}

kcError_t kcModelDestroy(kcModel_t m) noexcept {
    if (!m) return kc::Error::Success;
    (void)kcStreamSynchronize(m->ks);
    if (m->step_graph) (void)kcGraphDestroy(m->step_graph);
    for (void* p : m->allocs) (void)kcFree(p);
    (void)kcStreamDestroy(m->ks);
    delete m;
    return kc::Error::Success;
}

kcError_t kcModelTensorInfo(kcModel_t m, int tensor, int layer, int* qtype, int* rows, int* k,
                            size_t* bytes) noexcept {
    if (E e = checkModel(m); e != ok) return e;
    if (tensor < 0 || tensor >= KC_TENSOR_COUNT || (perLayer(tensor) && (layer < 0 || layer >= m->c.n_layer)))
        return kc::Error::InvalidValue;
    int r = 0, kk = 0;
    shapeOf(m->c, tensor, &r, &kk);
    int qt = qtypeOf(tensor);  // the default, or the type the tensor was set with
    if (qt != KC_QTYPE_F32) {
        const int q6 = tensor == KC_TENSOR_TOKEN_EMBD ? m->q6_tok
                       : tensor == KC_TENSOR_OUTPUT   ? m->q6_out
                                                      : m->L[layer].q6[tensor];
        qt = q6 ? KC_QTYPE_Q6_K : KC_QTYPE_Q4_K;
        if (perLayer(tensor) && m->L[layer].f16[tensor]) qt = KC_QTYPE_F16;
    }
    if (qtype) *qtype = qt;
    if (rows) *rows = r;
    if (k) *k = kk;
    if (bytes) *bytes = ggmlBytes(qt, r, kk);
    return ok;
}

kcError_t kcModelSetTensor(kcModel_t m, int tensor, int layer, const void* host, size_t bytes) noexcept {
    if (tensor < 0 || tensor >= KC_TENSOR_COUNT) return kc::Error::InvalidValue;
    return kcModelSetTensorTyped(m, tensor, layer, qtypeOf(tensor), host, bytes);
}

kcError_t kcModelSetTensorTyped(kcModel_t m, int tensor, int layer, int qt, const void* host, size_t bytes) noexcept {
    if (E e = checkModel(m); e != ok) return e;
    int r = 0, kk = 0;
    if (E e = kcModelTensorInfo(m, tensor, layer, nullptr, &r, &kk, nullptr); e != ok) return e;
    const bool vec = qtypeOf(tensor) == KC_QTYPE_F32;
    const bool f16_ok = !vec && perLayer(tensor);  // F16: the per-layer matrices
    if (vec ? qt != KC_QTYPE_F32
            : (qt != KC_QTYPE_Q4_K && qt != KC_QTYPE_Q6_K && !(f16_ok && qt == KC_QTYPE_F16))) {
        kcamd::setDetail("tensor %d: type %d not accepted (%s)", tensor, qt,
                         vec ? "f32 only" : (f16_ok ? "Q4_K, Q6_K or F16" : "Q4_K or Q6_K"));
        return kc::Error::InvalidValue;
    }
    const size_t want = ggmlBytes(qt, r, kk);
    if (!host || bytes != want) {
        kcamd::setDetail("tensor %d: expected %zu bytes", tensor, want);
        return kc::Error::InvalidValue;
    }
    if ((tensor == KC_TENSOR_Q_NORM || tensor == KC_TENSOR_K_NORM) && !m->c.qk_norm) return kc::Error::InvalidValue;
    if (tensor == KC_TENSOR_ROPE_FREQS) {  // into the factors the kernels read (ones by default)
        if (m->rope_freqs_set) return kc::Error::InvalidValue;
        KM_TRYE(kcMemcpy(m->ones, host, bytes, kc::CopyKind::HostToDevice));
        m->rope_freqs_set = true;
        return ok;
    }
    Layer* l = perLayer(tensor) ? &m->L[layer] : nullptr;
    void** slot = nullptr;
    switch (tensor) {
        case KC_TENSOR_TOKEN_EMBD: slot = &m->tok_embd; break;
        case KC_TENSOR_OUTPUT: slot = &m->output; break;
        case KC_TENSOR_OUTPUT_NORM: slot = reinterpret_cast<void**>(&m->out_norm); break;
        case KC_TENSOR_ATTN_NORM: slot = reinterpret_cast<void**>(&l->attn_norm); break;
        case KC_TENSOR_FFN_NORM: slot = reinterpret_cast<void**>(&l->ffn_norm); break;
        case KC_TENSOR_Q_NORM: slot = reinterpret_cast<void**>(&l->q_norm); break;
        case KC_TENSOR_K_NORM: slot = reinterpret_cast<void**>(&l->k_norm); break;
        case KC_TENSOR_WQ: slot = &l->wq; break;
        case KC_TENSOR_WK: slot = &l->wk; break;
        case KC_TENSOR_WV: slot = &l->wv; break;
        case KC_TENSOR_WO: slot = &l->wo; break;
        case KC_TENSOR_W_GATE: slot = &l->wg; break;
        case KC_TENSOR_W_UP: slot = &l->wu; break;
        case KC_TENSOR_W_DOWN: slot = &l->wd; break;
        default: return kc::Error::InvalidValue;
    }
    if (*slot) return kc::Error::InvalidValue;  // each tensor is set once
    const int q6 = qt == KC_QTYPE_Q6_K;
    if (tensor == KC_TENSOR_TOKEN_EMBD) m->q6_tok = q6;
    else if (tensor == KC_TENSOR_OUTPUT) m->q6_out = q6;
    else if (l) {
        l->q6[tensor] = q6;
        l->f16[tensor] = qt == KC_QTYPE_F16;
    }
    if (qt == KC_QTYPE_F32 || qt == KC_QTYPE_F16) {  // uploaded as they are (F16: row-major halves)
        KM_TRYE(alloc(m, slot, bytes));
        return kcMemcpy(*slot, host, bytes, kc::CopyKind::HostToDevice);
    }
    size_t sb = 0;
    KM_TRYE(kcKquantStreamBytes(qt, r, kk, &sb));
    void* raw = nullptr;
    KM_TRYE(kcMalloc(&raw, bytes));
    E e = kcMemcpy(raw, host, bytes, kc::CopyKind::HostToDevice);
    if (e == ok) e = alloc(m, slot, sb);
    if (e == ok) {
        kcKquantRepackArgs ra{raw, *slot, qt, r, kk};
        e = kcLaunchKernel("repack_kquant", &ra, m->ks);
        if (e == ok) e = syncModel(m);
    }
    (void)kcFree(raw);
    return e;
}

static E checkLoaded(kcModel_t m) {
    bool okw = m->tok_embd && m->output && m->out_norm;
    for (const auto& l : m->L)
        okw = okw && l.wq && l.wk && l.wv && l.wo && l.wg && l.wu && l.wd && l.attn_norm && l.ffn_norm &&
              (!m->c.qk_norm || (l.q_norm && l.k_norm));
    if (!okw) {
        kcamd::setDetail("not every tensor has been set");
        return kc::Error::InvalidValue;
    }
    return ok;
}

kcError_t kcModelForward(kcModel_t m, const int* tokens, int n, float* logits) noexcept {
    if (E e = checkModel(m); e != ok) return e;
    if (E e = checkLoaded(m); e != ok) return e;
    if (!tokens || n <= 0 || n > m->c.max_batch || m->pos_host + n > m->c.max_ctx) {
        kcamd::setDetail("n_tokens must be in [1, max_batch] and fit the cache");
        return kc::Error::InvalidValue;
    }
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= m->c.n_vocab) return kc::Error::InvalidValue;
    KM_TRYE(syncModel(m));
    KM_TRYE(kcMemcpy(m->tokens, tokens, sizeof(int) * n, kc::CopyKind::HostToDevice));
    KM_TRYE(kcMemcpy(m->n_past, &m->pos_host, sizeof(int), kc::CopyKind::HostToDevice));
    KM_TRY(n == 1 ? decodeAny(m, m->s) : batchStep(m, n, m->s));
    KM_TRYE(syncModel(m));
    m->pos_host += n;
    if (logits) KM_TRYE(kcMemcpy(logits, m->logits, sizeof(float) * m->c.n_vocab, kc::CopyKind::DeviceToHost));
    return ok;
}

kcError_t kcModelGenerate(kcModel_t m, int steps, int* tokens_out) noexcept {
    if (E e = checkModel(m); e != ok) return e;
    if (E e = checkLoaded(m); e != ok) return e;
    if (steps <= 0 || steps > m->max_gen || m->pos_host == 0 || m->pos_host + steps - 1 > m->c.max_ctx) {
        kcamd::setDetail("steps must be in [1, 4096], after a forward, and fit the cache");
        return kc::Error::InvalidValue;
    }
    KM_TRYE(syncModel(m));
    const int zero = 0;
    KM_TRYE(kcMemcpy(m->step, &zero, sizeof(int), kc::CopyKind::HostToDevice));
    KM_TRYE(kcMemcpy(m->n_past, &m->pos_host, sizeof(int), kc::CopyKind::HostToDevice));
    // the first token: argmax of the last forward's logits (no position consumed)
    KM_TRY(kcamd::launchArgmaxStep(m->logits, m->c.n_vocab, m->tokens, m->gen, m->step, nullptr, m->max_gen, m->s));
    if (!m->step_graph) {
        KM_TRYE(kcStreamBeginCapture(m->ks));
        int e1 = decodeAny(m, m->s);
        if (!e1)
            e1 = kcamd::launchArgmaxStep(m->logits, m->c.n_vocab, m->tokens, m->gen, m->step, m->n_past, m->max_gen,
                                         m->s);
        kcGraph_t g = nullptr;
        const E e2 = kcStreamEndCapture(m->ks, &g);
        if (e1) {
            if (g) (void)kcGraphDestroy(g);
            return err(e1);
        }
        if (e2 != ok) return e2;
        m->step_graph = g;
    }
    for (int i = 1; i < steps; ++i) KM_TRYE(kcGraphLaunch(m->step_graph, m->ks));
    KM_TRYE(syncModel(m));
    m->pos_host += steps - 1;
    if (tokens_out) KM_TRYE(kcMemcpy(tokens_out, m->gen, sizeof(int) * steps, kc::CopyKind::DeviceToHost));
    return ok;
}

kcError_t kcModelPosition(kcModel_t m, int* pos) noexcept {
    if (E e = checkModel(m); e != ok) return e;
    if (!pos) return kc::Error::InvalidValue;
    *pos = m->pos_host;
    return ok;
}

kcError_t kcModelReadCache(kcModel_t m, int layer, int which, int pos0, int n, void* host) noexcept {
    if (E e = checkModel(m); e != ok) return e;
    const auto& c = m->c;
    if (layer < 0 || layer >= c.n_layer || (which != 0 && which != 1) || pos0 < 0 || n < 0 || pos0 + n > c.max_ctx ||
        (n > 0 && !host)) {
        kcamd::setDetail("kcModelReadCache: layer, which (0 k, 1 v) or position range out of bounds");
        return kc::Error::InvalidValue;
    }
    if (n == 0) return ok;
    KM_TRYE(syncModel(m));
    const size_t row = (size_t)c.n_head_kv * c.head_dim * 2;  // bytes per position
    const int* base = which ? m->L[layer].vcache : m->L[layer].kcache;
    return kcMemcpy(host, reinterpret_cast<const char*>(base) + (size_t)pos0 * row, (size_t)n * row,
                    kc::CopyKind::DeviceToHost);
}

kcError_t kcModelReset(kcModel_t m) noexcept {
    if (E e = checkModel(m); e != ok) return e;
    KM_TRYE(syncModel(m));
    m->pos_host = 0;
    return ok;
}

kcError_t kcModelStream(kcModel_t m, kcStream_t* stream) noexcept {
    if (E e = checkModel(m); e != ok) return e;
    if (!stream) return kc::Error::InvalidValue;
    *stream = m->ks;
    return ok;
}
