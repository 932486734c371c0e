// mul_mat.cpp -- kcMulMat: the MUL_MAT dispatch of the reference's ggml backend over the public
// kc* calls (integrations/llama.cpp/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp: switches
// :46-53 and :81-86, batch_k256 :424, scratch_take :431-449, quantized_input :471-497,
// fused_norm :502-530, fused_swiglu :533-545, mul_mat_impl :555-589). The branch structure, the kernels each branch launches and their
// arguments are the reference's (they are the interface a backend drives); the scratch, the input
// cache and the validation are written for a GPU stream: launches are asynchronous, so growing the
// scratch waits for the stream before the old buffer goes.
#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include "internal.hpp"
#include "kernelcore/llm_kernels.h"
#include "kernelcore/model.h"
#include "kernelcore/mul_mat.h"
#include "mul_mat_internal.hpp"

namespace {

using E = kcError_t;
constexpr E ok = kc::Error::Success;

E bad(const char* why) {
    kcamd::setDetail("mul_mat: %s", why);
    return kc::Error::InvalidValue;
}

// Slot ints of one column: per 32 values nb * 11 (8 words of bytes, then d and the sum per block);
// per 256 values nsb * 85 (the reference's scratchInts / scratchKInts, llm/llm_kernels.hpp:84-89).
size_t slotInts(int k, bool k256) { return k256 ? size_t(k / 256) * 85 : size_t(k / 32) * 11; }

// Replaces the scratch by one of `ints` ints: the stream finishes the launches that read the old
// buffer, which is freed, and the cached inputs (in it) are dropped.
E regrow(kcMulMatRecording_st& r, size_t ints) {
    if (r.scratch) {
        if (E e = kcStreamSynchronize(r.stream); e != ok) return e;
        if (E e = kcFree(r.scratch); e != ok) return e;
        r.scratch = nullptr;
    }
    r.cap = r.used = 0;
    r.inputs.clear();
    ++r.gen;
    void* p = nullptr;
    if (E e = kcMalloc(&p, ints * sizeof(int)); e != ok) return e;
    r.scratch = static_cast<int*>(p);
    r.cap = ints;
    return ok;
}

void name(char (&dst)[24], const char* src) {
    std::strncpy(dst, src, sizeof dst - 1);
    dst[sizeof dst - 1] = '\0';
}

E launch(kcMulMatRecording_st& r, const char* kernel, const void* args, kcMulMatPlan& plan) {
    const E e = kcamd::mulmat::launch(r, kernel, args);
    if (e == ok) ++plan.launches;
    return e;
}

// A launch of one of this build's launchers (no by-name entry) on the recording's stream, named and
// counted like launch().
template <class F>
E direct(kcMulMatRecording_st& r, const char* kernel, F&& fn, kcMulMatPlan& plan) {
    if (r.trace) r.trace->push_back(kernel);
    ++plan.launches;
    if (r.dry) return ok;
    return kcamd::mulmat::timed(r, kernel, fn);
}

// Whether a per-256 producer of ncols columns of k values also writes the fp16 MFMA form (act_f16),
// and that form's buffer in the recording's scratch.
// Both are the ggml backend's own (act_f16 recordings; kernel option ggml_extra_fusions = 1 keeps the
// reference's launches), as is the per-256 norm in one workgroup per row.
bool ownFusions(const kcMulMatRecording_st& r) { return r.act_f16 && kcamd::option("ggml_extra_fusions") != 1; }
bool wantAct(const kcMulMatRecording_st& r, long long ncols, int k, bool k256) {
    return ownFusions(r) && k256 && ncols >= 64 && ncols <= INT_MAX && kcamd::mfmaHUsable(int(ncols), k);
}
// The fp16 form sits in the same take as the slots it mirrors (a later take may replace the scratch):
// `ints` of slots, padded to 64 bytes, then the form.
size_t actOffset(size_t ints) { return (ints + 15) / 16 * 16; }
size_t actInts(int ncols, int k) { return (kcamd::actF16Bytes(ncols, k) + 3) / 4; }

// The 8-bit form of the node's input, made once per recording (found again by key).
E quantizedInput(kcMulMatRecording_st& r, const kcMulMatNode& n, bool k256, int** q, kcMulMatPlan& plan,
                 const void* key) {
    for (const auto& in : r.inputs)
        if (in.key == key && in.ncols == n.ncols && in.k == n.k && in.k256 == k256) {
            *q = in.q;
            plan.input_reused = 1;
            return ok;
        }
    const int nb = n.k / 32;
    const size_t slot = slotInts(n.k, k256);
    const bool act = wantAct(r, n.ncols, n.k, k256);
    const size_t ints = slot * size_t(n.ncols);
    int* base = nullptr;
    if (E e = kcamd::mulmat::take(r, act ? actOffset(ints) + actInts(int(n.ncols), n.k) : ints, &base); e != ok)
        return e;
    const bool contiguous = n.x_col_bytes == size_t(n.k) * sizeof(float);
    if (act) {  // the slots and their fp16 form in one launch
        const kcamd::ActF16 ao = kcamd::actF16View(base + actOffset(ints), int(n.ncols), n.k, int(n.ncols));
        name(plan.quantizer, "quantize_cols_k");
        if (E e = direct(r, "quantize_cols_k", [&](hipStream_t s) {
                return kcamd::launchQuantizeColsK(n.x, base, n.k, int(n.ncols), s, &ao);
            }, plan); e != ok)
            return e;
        r.inputs.push_back({key, n.ncols, n.k, k256, base, ao, true});
        *q = base;
        return ok;
    }
    if (k256) {
        const kcQuantizeColsArgs a{n.x, base, nullptr, n.k, int(n.ncols)};
        name(plan.quantizer, "quantize_cols_k");
        if (E e = launch(r, "quantize_cols_k", &a, plan); e != ok) return e;
    } else if (n.ncols > 1 && contiguous) {  // contiguous columns: one launch
        const kcQuantizeColsArgs a{n.x, base, nullptr, n.k, int(n.ncols)};
        name(plan.quantizer, "quantize_cols");
        if (E e = launch(r, "quantize_cols", &a, plan); e != ok) return e;
    } else {
        name(plan.quantizer, "quantize_q8x4");
        for (long long c = 0; c < n.ncols; ++c) {
            int* qc = base + size_t(c) * slot;
            const float* xc = reinterpret_cast<const float*>(reinterpret_cast<const char*>(n.x) + size_t(c) * n.x_col_bytes);
            const kcQuantizeArgs a{xc, qc, reinterpret_cast<float*>(qc + nb * 8), nb};
            if (E e = launch(r, "quantize_q8x4", &a, plan); e != ok) return e;
        }
    }
    r.inputs.push_back({key, n.ncols, n.k, k256, base});
    *q = base;
    return ok;
}

// batch_k256: batches read activations scaled per 256 values unless matvec_cols or q8k = 0
bool batchK256(const kcMulMatRecording_st& r, long long ncols) { return ncols > 1 && !r.cfg.matvec_cols && r.cfg.q8k; }

// Slots for the 8-bit form of an output (ncols columns of k values) plus `extra` ints, registered
// under its key so that the MUL_MATs reading it find them (quantized_slots, :451-467).
E registeredSlots(kcMulMatRecording_st& r, const void* key, int k, long long ncols, bool k256, size_t extra,
                  int** q) {
    if (E e = kcamd::mulmat::take(r, slotInts(k, k256) * size_t(ncols) + extra, q); e != ok) return e;
    for (auto it = r.inputs.begin(); it != r.inputs.end(); ++it)  // rewritten: older slots of it are stale
        if (it->key == key && it->ncols == ncols && it->k == k && it->k256 == k256) {
            r.inputs.erase(it);
            break;
        }
    r.inputs.push_back({key, ncols, k, k256, *q});
    return ok;
}

E fusedNormImpl(kcMulMatRecording_st& r, const kcMulMatNormNode& n, kcMulMatPlan& plan, const float* b2,
                const void* key) {
    if (!n.x || !n.w || !n.y || (n.a != nullptr) != (n.b != nullptr)) return bad("norm: null x, w or y, or one of a / b");
    if (n.n <= 0 || n.n % 256 || n.rows <= 0 || (long long)n.n * n.rows >= (1 << 24))
        return bad("norm: n must be a positive multiple of 256, rows positive, n * rows < 2^24");
    const bool k256 = batchK256(r, n.rows);
    plan.k256 = k256;
    // per 256: the rows' slots, then the per-32 partial sums of squares; per 32: in the slots' tails
    const size_t off = k256 ? size_t(n.rows) * slotInts(n.n, true) : 0;
    const size_t sums = k256 ? size_t(n.rows) * slotInts(n.n, false) : 0;
    const bool one = k256 && n.n <= 8192 && ownFusions(r);  // add_norm_q8k_f
    if (b2 && (!one || !n.a)) return bad("norm: a second K half needs an ADD and the one-kernel per-256 norm");
    const bool act = one && wantAct(r, n.rows, n.n, k256);
    int* qk = nullptr;
    if (E e = registeredSlots(r, key ? key : n.y, n.n, n.rows, k256,
                              act ? actOffset(off + sums) - off + actInts(n.rows, n.n) : sums, &qk);
        e != ok)
        return e;
    int* q = qk + off;
    if (one) {  // per 256: both steps in one workgroup per row (the same bytes)
        kcamd::ActF16 ao{};
        if (act) {
            ao = kcamd::actF16View(qk + actOffset(off + sums), n.rows, n.n, n.rows);
            auto& in = r.inputs.back();  // registeredSlots' entry for y
            in.act = ao;
            in.has_act = true;
        }
        name(plan.kernel, "add_norm_q8k_f");
        return direct(r, "add_norm_q8k_f", [&](hipStream_t s) {
            return kcamd::launchAddNormQ8K(n.a, n.a ? n.b : n.x, n.a ? b2 : nullptr, n.a ? n.x : nullptr, n.w, qk, n.n,
                                           n.rows, n.eps, s, act ? &ao : nullptr, n.y);
        }, plan);
    }
    if (!k256 && n.n <= 8192) {  // both steps in one workgroup per row (the same bytes)
        const kcAddNormQ8FArgs a{n.a, n.b, n.x, n.w, n.y, q, nullptr, n.n, n.rows, n.eps};
        name(plan.kernel, "add_norm_q8_f");
        return launch(r, "add_norm_q8_f", &a, plan);
    }
    if (n.a) {
        const kcAddSumsqFArgs a{n.a, n.b, n.x, q, nullptr, n.n, n.rows};
        name(plan.quantizer, "add_sumsq_f");
        if (E e = launch(r, "add_sumsq_f", &a, plan); e != ok) return e;
    } else {
        const kcSumsqPartArgs a{n.x, q, nullptr, n.n, n.rows};
        name(plan.quantizer, "sumsq_part");
        if (E e = launch(r, "sumsq_part", &a, plan); e != ok) return e;
    }
    const kcNormMulQ8Args a{n.x, n.w, n.y, qk, nullptr, n.n, n.rows, n.eps};
    const char* kernel = k256 ? "norm_mul_q8k_f" : "norm_mul_q8_f";
    name(plan.kernel, kernel);
    return launch(r, kernel, &a, plan);
}

E fusedSwigluImpl(kcMulMatRecording_st& r, const kcMulMatSwigluNode& n, kcMulMatPlan& plan, const void* key) {
    if (!n.g || !n.u || !n.y) return bad("swiglu: null g, u or y");
    if (n.n <= 0 || n.n % 256 || n.cols <= 0 || (long long)n.n * n.cols >= (1 << 24))
        return bad("swiglu: n must be a positive multiple of 256, cols positive, n * cols < 2^24");
    const bool k256 = batchK256(r, n.cols);
    plan.k256 = k256;
    int* q = nullptr;
    const bool act = wantAct(r, n.cols, n.n, k256);
    const size_t ints = slotInts(n.n, k256) * size_t(n.cols);
    if (E e = registeredSlots(r, key ? key : n.y, n.n, n.cols, k256,
                              act ? actOffset(ints) - ints + actInts(n.cols, n.n) : 0, &q);
        e != ok)
        return e;
    const kcSiluMulQ8FArgs a{n.g, n.u, n.y, q, nullptr, n.n, n.cols};
    if (act) {  // the slots and their fp16 form in one launch
        const kcamd::ActF16 ao = kcamd::actF16View(q + actOffset(ints), n.cols, n.n, n.cols);
        auto& in = r.inputs.back();
        in.act = ao;
        in.has_act = true;
        name(plan.kernel, "silu_mul_q8kf");
        return direct(r, "silu_mul_q8kf", [&](hipStream_t s) { return kcamd::launchSiluMulQ8KAct(a, &ao, s); }, plan);
    }
    const char* kernel = k256 ? "silu_mul_q8kf" : "silu_mul_q8x4f";
    name(plan.kernel, kernel);
    return launch(r, kernel, &a, plan);
}

E validate(const kcMulMatNode& n) {
    const bool f16 = n.wtype == KC_QTYPE_F16;
    if (!f16 && n.wtype != KC_QTYPE_Q4_K && n.wtype != KC_QTYPE_Q6_K)
        return bad("weight type must be Q4_K (12), Q6_K (14) or F16 (1)");
    if (!n.w || !n.x || !n.y) return bad("null weight, input or output pointer");
    if (n.rows <= 0 || n.rows % 8) return bad("rows must be a positive multiple of 8");
    if (n.k <= 0 || (f16 ? n.k % 2 : n.k % 256)) return bad("k must be a positive multiple of 256 (F16: even)");
    if (n.ncols < 1 || n.ncols > INT_MAX) return bad("ncols must be in [1, INT_MAX]");
    if (n.x_col_bytes < size_t(n.k) * sizeof(float) || n.x_col_bytes % sizeof(float))
        return bad("x_col_bytes must be at least 4 k and a multiple of 4");
    if (f16 && n.x_col_bytes != size_t(n.k) * sizeof(float)) return bad("F16 weights take contiguous input columns");
    return ok;
}

E mulMatImpl(kcMulMatRecording_st& r, const kcMulMatNode& n, kcMulMatPlan& plan, const void* key) {
    if (E e = validate(n); e != ok) return e;
    const int ncols = int(n.ncols);
    if (n.wtype == KC_QTYPE_F16) {  // f32 activations as they are
        const kcMatmulF16Args a{static_cast<const int*>(n.w), n.x, n.y, nullptr, n.rows, n.k, ncols};
        name(plan.kernel, "matmul_f16");
        return launch(r, "matmul_f16", &a, plan);
    }
    const bool q4 = n.wtype == KC_QTYPE_Q4_K;
    const bool contiguous = n.x_col_bytes == size_t(n.k) * sizeof(float);
    const bool k256 = batchK256(r, n.ncols) && contiguous;
    plan.k256 = k256;
    int* base = nullptr;
    if (E e = quantizedInput(r, n, k256, &base, plan, key ? key : n.x); e != ok) return e;
    if (n.ncols > 1 && !r.cfg.matvec_cols) {  // a batch: one matmul (weights read once per 4 or 8 columns)
        const bool x8 = r.cfg.tile == 8 && n.ncols > 4;
        const char* kernel = k256 ? (x8 ? (q4 ? "matmul_q4k_q8kx8" : "matmul_q6k_q8kx8")
                                        : (q4 ? "matmul_q4k_q8kx4" : "matmul_q6k_q8kx4"))
                                  : (x8 ? (q4 ? "matmul_q4k_q8x8" : "matmul_q6k_q8x8")
                                        : (q4 ? "matmul_q4k_q8x4" : "matmul_q6k_q8x4"));
        const kcMatmulKQ8Args a{static_cast<const int*>(n.w), base, n.y, nullptr, n.rows, n.k, ncols, r.cfg.row_block};
        name(plan.kernel, kernel);
        return launch(r, kernel, &a, plan);
    }
    const char* kernel = q4 ? "matvec_q4k_q8" : "matvec_q6k_q8";  // one matvec per column
    name(plan.kernel, kernel);
    const int nb = n.k / 32;
    const size_t slot = slotInts(n.k, false);
    for (int c = 0; c < ncols; ++c) {
        const int* q = base + size_t(c) * slot;
        const kcMatvecQ4Q8Args a{static_cast<const int*>(n.w), q, reinterpret_cast<const float*>(q + nb * 8),
                                 n.y + size_t(c) * n.rows, nullptr, n.rows, n.k};
        if (E e = launch(r, kernel, &a, plan); e != ok) return e;
    }
    return ok;
}

}  // namespace

hipEvent_t kcamd::LaunchTimer::next() {
    if (used == pool.size()) {
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        try {
            pool.push_back(e);
        } catch (...) {
            (void)hipEventDestroy(e);
            return nullptr;
        }
    }
    return pool[used++];
}

namespace kcamd::mulmat {

kcError_t checkConfig(kcMulMatConfig& c) noexcept {
    if (c.tile != 4 && c.tile != 8) return bad("tile must be 4 or 8");
    if (c.row_block < 1) return bad("row_block must be at least 1");
    c.matvec_cols = c.matvec_cols != 0;
    c.q8k = c.q8k != 0;
    return ok;
}

void reset(kcMulMatRecording_st& r) noexcept {
    r.inputs.clear();
    r.used = r.peak = 0;  // same stream: the next recording's launches run after the last one's
}

kcError_t reserve(kcMulMatRecording_st& r, size_t ints) noexcept {
    ints = (ints + 15) / 16 * 16;
    if (r.dry || ints <= r.cap) return ok;
    return regrow(r, ints);
}

kcError_t take(kcMulMatRecording_st& r, size_t ints, int** out) noexcept {
    ints = (ints + 15) / 16 * 16;
    if (r.dry) {  // an offset only, never dereferenced
        *out = reinterpret_cast<int*>(uintptr_t(256) + r.used * sizeof(int));
        r.used += ints;
        r.peak = std::max(r.peak, r.used);
        return ok;
    }
    if (r.used + ints > r.cap)
        if (E e = regrow(r, std::max(ints * 4, r.cap * 2)); e != ok) return e;
    *out = r.scratch + r.used;
    r.used += ints;
    r.peak = std::max(r.peak, r.used);
    return ok;
}

int* inputSlot(const kcMulMatRecording_st& r, const void* key, long long ncols, int k, bool k256) noexcept {
    for (const auto& in : r.inputs)
        if (in.key == key && in.ncols == ncols && in.k == k && in.k256 == k256) return in.q;
    return nullptr;
}

const kcamd::ActF16* inputAct(const kcMulMatRecording_st& r, const void* key, long long ncols, int k) noexcept {
    for (const auto& in : r.inputs)
        if (in.key == key && in.ncols == ncols && in.k == k && in.k256) return in.has_act ? &in.act : nullptr;
    return nullptr;
}

kcError_t outputSlot(kcMulMatRecording_st& r, const void* key, int k, long long ncols, bool k256, int** q) noexcept {
    try {
        return registeredSlots(r, key, k, ncols, k256, 0, q);
    } catch (...) {
        return kc::Error::OutOfMemory;
    }
}

kcError_t launch(kcMulMatRecording_st& r, const char* kernel, const void* args) noexcept {
    if (r.trace) {
        try {
            r.trace->push_back(kernel);
        } catch (...) {
            return kc::Error::OutOfMemory;
        }
    }
    if (r.dry) return ok;
    if (!r.timer) return kcLaunchKernel(kernel, args, r.stream);
    return timed(r, kernel, [&](hipStream_t) { return int(kcLaunchKernel(kernel, args, r.stream)); });
}

kcError_t mulMat(kcMulMatRecording_st& r, const kcMulMatNode& n, kcMulMatPlan& plan, const void* key) noexcept {
    try {
        return mulMatImpl(r, n, plan, key);
    } catch (...) {
        return kc::Error::OutOfMemory;
    }
}

kcError_t mulMatInput(kcMulMatRecording_st& r, const kcMulMatNode& n, kcMulMatPlan& plan, const void* key) noexcept {
    if (E e = validate(n); e != ok) return e;
    if (n.wtype == KC_QTYPE_F16) return ok;
    const bool k256 = batchK256(r, n.ncols) && n.x_col_bytes == size_t(n.k) * sizeof(float);
    int* q = nullptr;
    try {
        return quantizedInput(r, n, k256, &q, plan, key ? key : n.x);
    } catch (...) {
        return kc::Error::OutOfMemory;
    }
}

bool fusesHalf(const kcMulMatRecording_st& r, int n) noexcept {
    return n > 0 && n % 256 == 0 && n <= 8192 && batchK256(r, 2) && ownFusions(r);
}

kcError_t fusedNorm(kcMulMatRecording_st& r, const kcMulMatNormNode& n, kcMulMatPlan& plan, const float* b2,
                    const void* key) noexcept {
    try {
        return fusedNormImpl(r, n, plan, b2, key);
    } catch (...) {
        return kc::Error::OutOfMemory;
    }
}

kcError_t fusedSwiglu(kcMulMatRecording_st& r, const kcMulMatSwigluNode& n, kcMulMatPlan& plan,
                      const void* key) noexcept {
    try {
        return fusedSwigluImpl(r, n, plan, key);
    } catch (...) {
        return kc::Error::OutOfMemory;
    }
}

}  // namespace kcamd::mulmat

KC_API void kcMulMatConfigFromEnv(kcMulMatConfig* cfg) noexcept {
    if (!cfg) return;
    *cfg = kcMulMatConfig{0, 1, 8, 8};
    if (const char* mc = std::getenv("GGML_KERNELCORE_MATVEC_COLS")) cfg->matvec_cols = std::strcmp(mc, "1") == 0;
    if (const char* rb = std::getenv("GGML_KERNELCORE_ROW_BLOCK")) cfg->row_block = std::max(1, std::atoi(rb));
    if (const char* qk = std::getenv("GGML_KERNELCORE_Q8K")) cfg->q8k = std::strcmp(qk, "0") != 0;
    if (const char* tl = std::getenv("GGML_KERNELCORE_TILE")) cfg->tile = std::atoi(tl) == 4 ? 4 : 8;
}

KC_API kcError_t kcMulMatRecordingCreate(kcMulMatRecording_t* rec, const kcMulMatConfig* cfg,
                                         kcStream_t stream) noexcept {
    if (!rec) return bad("null recording pointer");
    *rec = nullptr;
    kcMulMatConfig c;
    if (cfg) c = *cfg;
    else kcMulMatConfigFromEnv(&c);
    if (E e = kcamd::mulmat::checkConfig(c); e != ok) return e;
    auto* r = new (std::nothrow) kcMulMatRecording_st;
    if (!r) return kc::Error::OutOfMemory;
    r->cfg = c;
    r->stream = stream;
    *rec = r;
    return ok;
}

KC_API kcError_t kcMulMatRecordingReset(kcMulMatRecording_t rec) noexcept {
    if (!rec) return kc::Error::InvalidResourceHandle;
    kcamd::mulmat::reset(*rec);
    return ok;
}

KC_API kcError_t kcMulMatRecordingDestroy(kcMulMatRecording_t rec) noexcept {
    if (!rec) return ok;
    E e = ok;
    if (rec->scratch) {  // launches in flight may still read it
        e = kcStreamSynchronize(rec->stream);
        const E f = kcFree(rec->scratch);
        if (e == ok) e = f;
    }
    delete rec;
    return e;
}

KC_API kcError_t kcMulMat(kcMulMatRecording_t rec, const kcMulMatNode* node, kcMulMatPlan* plan) noexcept {
    if (!rec) return kc::Error::InvalidResourceHandle;
    if (!node) return bad("null node");
    kcMulMatPlan p{};
    const E e = kcamd::mulmat::mulMat(*rec, *node, p);
    if (plan) *plan = p;
    return e;
}

KC_API kcError_t kcMulMatFusedNorm(kcMulMatRecording_t rec, const kcMulMatNormNode* node, kcMulMatPlan* plan) noexcept {
    if (!rec) return kc::Error::InvalidResourceHandle;
    if (!node) return bad("null node");
    kcMulMatPlan p{};
    const E e = kcamd::mulmat::fusedNorm(*rec, *node, p);
    if (plan) *plan = p;
    return e;
}

KC_API kcError_t kcMulMatFusedSwiglu(kcMulMatRecording_t rec, const kcMulMatSwigluNode* node,
                                     kcMulMatPlan* plan) noexcept {
    if (!rec) return kc::Error::InvalidResourceHandle;
    if (!node) return bad("null node");
    kcMulMatPlan p{};
    const E e = kcamd::mulmat::fusedSwiglu(*rec, *node, p);
    if (plan) *plan = p;
    return e;
}
