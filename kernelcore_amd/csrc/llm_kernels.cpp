// llm_kernels.cpp -- the built-in kernel table: argument validation and launch per kernel name.
//
// Validation keeps the reference's rules (arasheedu/Kernelcore llm/llm_kernels.cpp): sizes must
// be positive and fit int32 indexing, every buffer must lie inside one live allocation, and the
// shape rules of each kernel (rows % 8, k % 256, ...) hold. A rejected launch returns
// InvalidValue or InvalidPointer with a detail text, as there. The System V marshalling, chunk
// planning and CPU executor are replaced by one HIP grid per launch (launch.hpp).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>

#include "internal.hpp"
#include "kquant.hpp"
#include "launch.hpp"
#include "kquantize.hpp"
#include "kdecode.hpp"
#include "model_kernels.hpp"

namespace {

using kcamd::checkRange;
using kcamd::setDetail;

constexpr int64_t kMaxIndex = INT32_MAX;

bool fitsIndex(int64_t a, int64_t b = 1) { return a >= 0 && b >= 0 && (b == 0 || a <= kMaxIndex / b); }
size_t f32Bytes(int64_t n) { return static_cast<size_t>(n) * sizeof(float); }
size_t i32Bytes(int64_t n) { return static_cast<size_t>(n) * sizeof(int); }

#define KC_TRY(expr)                 \
    do {                             \
        if (int e_ = (expr)) return e_; \
    } while (0)

int invalid(const char* what) {
    setDetail("%s", what);
    return KC_ERROR_INVALID_VALUE;
}

// Optional device dims array: a live allocation of n ints whose known host copy matches `want`.
int checkDims(const int* dims, const int* want, int n) {
    if (!dims) return 0;
    KC_TRY(checkRange(dims, i32Bytes(n), "dims"));
    if (!kcamd::dimsAgree(dims, want, n)) return KC_ERROR_INVALID_VALUE;
    return 0;
}

hipStream_t hs(void* s) { return static_cast<hipStream_t>(s); }

// ---- vector_add (adapters/vector_add_adapter.cpp:14-24)

int vectorAddValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcVectorAddArgs*>(p);
    if (a.count < 0) return invalid("count < 0");
    const size_t bytes = f32Bytes(a.count);
    KC_TRY(checkRange(a.a, bytes, "a"));
    KC_TRY(checkRange(a.b, bytes, "b"));
    KC_TRY(checkRange(a.out, bytes, "out"));
    return 0;
}
int vectorAddLaunch(const void* p, void* s) {
    const auto& a = *static_cast<const kcVectorAddArgs*>(p);
    return kcamd::launchVectorAdd(a.a, a.b, a.out, a.count, hs(s));
}

// ---- quantize_q8x4 (llm_kernels.cpp:180-189)

int quantValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcQuantizeArgs*>(p);
    if (a.count < 0 || !fitsIndex(a.count, 32)) return invalid("count out of range");
    KC_TRY(checkRange(a.x, f32Bytes(int64_t(a.count) * 32), "x"));
    KC_TRY(checkRange(a.xq, i32Bytes(int64_t(a.count) * 8), "xq"));
    KC_TRY(checkRange(a.xd, f32Bytes(int64_t(a.count) * 2), "xd"));
    return 0;
}
int quantLaunch(const void* p, void* s) {
    const auto& a = *static_cast<const kcQuantizeArgs*>(p);
    return kcamd::launchQuantizeQ8x4(a.x, a.xq, a.xd, a.count, hs(s));
}

// ---- matvec_q4k_q8 / matvec_q6k_q8 (llm_kernels.cpp:264-279: kquantMarshal)

template <bool Q6>
int kquantValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcMatvecQ4Q8Args*>(p);
    if (a.rows < 0 || a.rows % 8 != 0 || a.k <= 0 || a.k % 256 != 0 || !fitsIndex(a.rows, a.k))
        return invalid("rows must be a non-negative multiple of 8 and k a positive multiple of 256");
    if (a.k > kcamd::kMatvecMaxK) return invalid("k exceeds the matvec's activation staging (32768)");
    const int64_t nb = a.k / 32;
    if (reinterpret_cast<uintptr_t>(a.qw) % 16) return invalid("qw (a weight stream) must be 16-byte aligned");
    KC_TRY(checkRange(a.qw, kcamd::streamBytes(Q6, a.rows, a.k), "qw"));
    KC_TRY(checkRange(a.xq, i32Bytes(nb * 8), "xq"));
    KC_TRY(checkRange(a.xd, f32Bytes(nb * 2), "xd"));
    KC_TRY(checkRange(a.y, f32Bytes(a.rows), "y"));
    const int want[2] = {a.rows, a.k};
    return checkDims(a.dims, want, 2);
}
template <bool Q6>
int kquantLaunch(const void* p, void* s) {
    return kcamd::launchMatvecKq(Q6, *static_cast<const kcMatvecQ4Q8Args*>(p), hs(s));
}

// ---- matmul_{q4k,q6k}_q8{,k}x{4,8} (llm_kernels.cpp:290-312: matmulKMarshal)

template <bool Q6, bool K8>
int matmulValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcMatmulKQ8Args*>(p);
    if (a.rows <= 0 || a.rows % 8 != 0 || a.k <= 0 || a.k % 256 != 0 || a.ncols <= 0 || a.row_block <= 0 ||
        !fitsIndex(a.rows, a.k))
        return invalid("rows must be a positive multiple of 8, k a positive multiple of 256, ncols and row_block > 0");
    const int64_t slot = K8 ? int64_t(a.k / 256) * 85 : int64_t(a.k / 32) * 11;
    if (!fitsIndex(slot, a.ncols) || !fitsIndex(a.rows, a.ncols) || a.ncols > 65535 * 8)
        return invalid("ncols out of range");
    if (reinterpret_cast<uintptr_t>(a.qw) % 16) return invalid("qw (a weight stream) must be 16-byte aligned");
    KC_TRY(checkRange(a.qw, kcamd::streamBytes(Q6, a.rows, a.k), "qw"));
    KC_TRY(checkRange(a.xq, i32Bytes(slot * a.ncols), "xq"));
    KC_TRY(checkRange(a.y, f32Bytes(int64_t(a.rows) * a.ncols), "y"));
    const int want[4] = {a.rows, a.k, a.ncols, a.row_block};
    return checkDims(a.dims, want, 4);
}
template <bool Q6, bool K8>
int matmulLaunch(const void* p, void* s) {
    return kcamd::launchMatmulKq(Q6, K8, *static_cast<const kcMatmulKQ8Args*>(p), hs(s));
}

// ---- matmul_f16 (llm_kernels.cpp:834-847: matmulF16Marshal). The reference's thread-count
// limit (rows x column tiles of 4 below 2^24, a CPU chunking bound) is kept so that the same
// launches are accepted.

int matmulF16Validate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcMatmulF16Args*>(p);
    if (a.rows <= 0 || a.rows % 8 || a.k <= 0 || a.k % 2 || a.ncols <= 0 || !fitsIndex(a.rows, a.k) ||
        !fitsIndex(a.ncols, std::max(a.rows, a.k)) || int64_t(a.rows) * ((a.ncols + 3) / 4) >= (int64_t(1) << 24))
        return invalid("rows must be a positive multiple of 8, k positive and even, ncols positive");
    if (reinterpret_cast<uintptr_t>(a.qw) % 4 || reinterpret_cast<uintptr_t>(a.x) % 4 ||
        reinterpret_cast<uintptr_t>(a.y) % 4)
        return invalid("qw, x and y must be 4-byte aligned");
    KC_TRY(checkRange(a.qw, i32Bytes(int64_t(a.rows) * (a.k / 2)), "qw"));
    KC_TRY(checkRange(a.x, f32Bytes(int64_t(a.ncols) * a.k), "x"));
    KC_TRY(checkRange(a.y, f32Bytes(int64_t(a.ncols) * a.rows), "y"));
    const int want[3] = {a.rows, a.k, a.ncols};
    return checkDims(a.dims, want, 3);
}
int matmulF16Launch(const void* p, void* s) {
    const auto& a = *static_cast<const kcMatmulF16Args*>(p);
    return kcamd::launchMatmulF16(a.qw, a.x, a.y, a.rows, a.k, a.ncols, hs(s));
}

// ---- quantize_cols / quantize_cols_k (llm_kernels.cpp:331-345: quantColsMarshal)

template <int kBlock>
int quantColsValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcQuantizeColsArgs*>(p);
    const int64_t slot = kBlock == 32 ? int64_t(a.k / 32) * 11 : int64_t(a.k / 256) * 85;
    if (a.k <= 0 || a.k % 256 != 0 || a.ncols <= 0 || !fitsIndex(a.k, a.ncols) || !fitsIndex(slot, a.ncols))
        return invalid("k must be a positive multiple of 256 and ncols positive");
    KC_TRY(checkRange(a.x, f32Bytes(int64_t(a.k) * a.ncols), "x"));
    KC_TRY(checkRange(a.q, i32Bytes(slot * a.ncols), "q"));
    const int want[2] = {a.k / kBlock, a.ncols};
    return checkDims(a.dims, want, 2);
}
template <int kBlock>
int quantColsLaunch(const void* p, void* s) {
    const auto& a = *static_cast<const kcQuantizeColsArgs*>(p);
    if (kBlock == 32) return kcamd::launchQuantizeCols(a.x, a.q, a.k, a.ncols, hs(s));
    return kcamd::launchQuantizeColsK(a.x, a.q, a.k, a.ncols, hs(s));
}

// ---- ggml layer fusions (llm_kernels.cpp:402-570: checkRowsQ, normDimsOk and the marshals)

int checkRowsQ(int n, int rows, const int* q) {
    if (n <= 0 || n % 256 || rows <= 0 || !fitsIndex(n, rows) || int64_t(n) * rows >= (1 << 24))
        return invalid("n must be a positive multiple of 256, rows positive, n * rows < 2^24");
    return checkRange(q, i32Bytes(int64_t(rows) * (n / 32) * 11), "q");
}

int addSumsqValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcAddSumsqFArgs*>(p);
    KC_TRY(checkRowsQ(a.n, a.rows, a.q));
    const size_t bytes = f32Bytes(int64_t(a.n) * a.rows);
    KC_TRY(checkRange(a.a, bytes, "a"));
    KC_TRY(checkRange(a.b, bytes, "b"));
    KC_TRY(checkRange(a.out, bytes, "out"));
    const int want[3] = {a.n / 32, a.n, a.rows};
    return checkDims(a.dims, want, 3);
}
int addSumsqLaunch(const void* p, void* s) {
    const auto& a = *static_cast<const kcAddSumsqFArgs*>(p);
    return kcamd::launchAddSumsq(a.a, a.b, a.out, a.q, a.n, a.rows, hs(s));
}

int sumsqValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcSumsqPartArgs*>(p);
    KC_TRY(checkRowsQ(a.n, a.rows, a.q));
    KC_TRY(checkRange(a.x, f32Bytes(int64_t(a.n) * a.rows), "x"));
    const int want[3] = {a.n / 32, a.n, a.rows};
    return checkDims(a.dims, want, 3);
}
int sumsqLaunch(const void* p, void* s) {
    const auto& a = *static_cast<const kcSumsqPartArgs*>(p);
    return kcamd::launchAddSumsq(nullptr, a.x, nullptr, a.q, a.n, a.rows, hs(s));
}

template <bool K8>
int normMulValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcNormMulQ8Args*>(p);
    if (K8) {
        if (a.n <= 0 || a.n % 256 || a.rows <= 0 || int64_t(a.n) * a.rows >= (1 << 24))
            return invalid("n must be a positive multiple of 256, rows positive, n * rows < 2^24");
        KC_TRY(checkRange(a.q, i32Bytes(int64_t(a.rows) * (a.n / 256 * 85 + a.n / 32 * 11)), "q"));
    } else {
        KC_TRY(checkRowsQ(a.n, a.rows, a.q));
    }
    const size_t bytes = f32Bytes(int64_t(a.n) * a.rows);
    KC_TRY(checkRange(a.x, bytes, "x"));
    KC_TRY(checkRange(a.w, f32Bytes(a.n), "w"));
    KC_TRY(checkRange(a.y, bytes, "y"));
    if (K8) {
        const int want[4] = {a.n / 256, a.n, a.rows, a.rows * (a.n / 256 * 85)};
        return checkDims(a.dims, want, 4);
    }
    const int want[3] = {a.n / 32, a.n, a.rows};
    return checkDims(a.dims, want, 3);
}
template <bool K8>
int normMulLaunch(const void* p, void* s) {
    return kcamd::launchNormMulQ8(K8, *static_cast<const kcNormMulQ8Args*>(p), hs(s));
}

int addNormValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcAddNormQ8FArgs*>(p);
    KC_TRY(checkRowsQ(a.n, a.rows, a.q));
    if (a.n > 8192) return invalid("add_norm_q8_f: rows of at most 8192 values");
    if ((a.a != nullptr) != (a.b != nullptr)) return invalid("a and b are both given or both null");
    const size_t bytes = f32Bytes(int64_t(a.n) * a.rows);
    if (a.a) {
        KC_TRY(checkRange(a.a, bytes, "a"));
        KC_TRY(checkRange(a.b, bytes, "b"));
    }
    KC_TRY(checkRange(a.x, bytes, "x"));
    KC_TRY(checkRange(a.w, f32Bytes(a.n), "w"));
    KC_TRY(checkRange(a.y, bytes, "y"));
    const int want[3] = {a.n / 32, a.n, a.rows};
    return checkDims(a.dims, want, 3);
}
int addNormLaunch(const void* p, void* s) {
    const auto& a = *static_cast<const kcAddNormQ8FArgs*>(p);
    return kcamd::launchAddNormQ8(a.a, a.b, a.x, a.w, a.y, a.q, a.n, a.rows, a.eps, hs(s));
}

template <bool K8>
int siluQValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcSiluMulQ8FArgs*>(p);
    if (a.n <= 0 || a.n % 256 || a.cols <= 0 || int64_t(a.n) * a.cols >= (1 << 24))
        return invalid("n must be a positive multiple of 256, cols positive, n * cols < 2^24");
    KC_TRY(checkRange(a.q, i32Bytes(int64_t(a.cols) * (K8 ? a.n / 256 * 85 : a.n / 32 * 11)), "q"));
    const size_t bytes = f32Bytes(int64_t(a.n) * a.cols);
    KC_TRY(checkRange(a.g, bytes, "g"));
    KC_TRY(checkRange(a.u, bytes, "u"));
    KC_TRY(checkRange(a.y, bytes, "y"));
    const int want[2] = {a.n, a.cols};
    return checkDims(a.dims, want, 2);
}
template <bool K8>
int siluQLaunch(const void* p, void* s) {
    return kcamd::launchSiluMulQ8(K8, *static_cast<const kcSiluMulQ8FArgs*>(p), hs(s));
}

// ---- rms_norm, mul_rows, silu_mul, rope_ggml, set_rows_f16 (llm_kernels.cpp:386-400, 616-631, 944-972)

int rmsValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcRmsNormArgs*>(p);
    if (a.n <= 0 || a.rows < 0 || !fitsIndex(a.rows, a.n)) return invalid("n must be positive, rows >= 0");
    const size_t bytes = f32Bytes(int64_t(a.rows) * a.n);
    KC_TRY(checkRange(a.x, bytes, "x"));
    KC_TRY(checkRange(a.w, f32Bytes(a.n), "w"));
    return checkRange(a.y, bytes, "y");
}
int rmsLaunch(const void* p, void* s) { return kcamd::launchRmsNorm(*static_cast<const kcRmsNormArgs*>(p), hs(s)); }

int mulRowsValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcMulRowsArgs*>(p);
    if (a.n <= 0 || a.n % 8 || a.count < 0 || a.count % a.n) return invalid("n must be a positive multiple of 8 dividing count");
    KC_TRY(checkRange(a.x, f32Bytes(a.count), "x"));
    KC_TRY(checkRange(a.w, f32Bytes(a.n), "w"));
    return checkRange(a.y, f32Bytes(a.count), "y");
}
int mulRowsLaunch(const void* p, void* s) { return kcamd::launchMulRows(*static_cast<const kcMulRowsArgs*>(p), hs(s)); }

int siluValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcSiluMulArgs*>(p);
    if (a.count < 0) return invalid("count < 0");
    const size_t bytes = f32Bytes(a.count);
    KC_TRY(checkRange(a.g, bytes, "g"));
    KC_TRY(checkRange(a.u, bytes, "u"));
    return checkRange(a.out, bytes, "out");
}
int siluLaunch(const void* p, void* s) { return kcamd::launchSiluMul(*static_cast<const kcSiluMulArgs*>(p), hs(s)); }

int ropeValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcRopeGgmlArgs*>(p);
    if (a.head_dim <= 0 || a.head_dim % 16 || a.n_head <= 0 || a.n_tokens < 0)
        return invalid("head_dim must be a positive multiple of 16, n_head positive, n_tokens >= 0");
    const int64_t pairs = a.head_dim / 2, count = pairs * a.n_head * a.n_tokens;
    if (!fitsIndex(count, 2)) return invalid("too many values");
    KC_TRY(checkRange(a.x, f32Bytes(count * 2), "x"));
    KC_TRY(checkRange(a.y, f32Bytes(count * 2), "y"));
    KC_TRY(checkRange(a.pos, i32Bytes(a.n_tokens), "pos"));
    KC_TRY(checkRange(a.ff, f32Bytes(pairs), "ff"));
    const int want[5] = {(int)pairs, a.n_head, (int)(pairs * a.n_tokens), a.neox ? 1 : 2, a.neox ? (int)pairs : 1};
    return checkDims(a.dims, want, 5);
}
int ropeLaunch(const void* p, void* s) { return kcamd::launchRope(*static_cast<const kcRopeGgmlArgs*>(p), hs(s)); }

int setRowsValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcSetRowsF16Args*>(p);
    if (a.pairs <= 0 || a.pairs % 8 || a.rows <= 0 || a.dst_rows <= 0 || a.src_row < 2 * a.pairs ||
        a.dst_row < a.pairs || int64_t(a.pairs) * a.rows >= (1 << 24) || !fitsIndex(a.rows, a.src_row) ||
        !fitsIndex(a.dst_rows, a.dst_row))
        return invalid("set_rows_f16 shape");
    KC_TRY(checkRange(a.src, f32Bytes(int64_t(a.rows - 1) * a.src_row + 2 * a.pairs), "src"));
    KC_TRY(checkRange(a.idx, i32Bytes(int64_t(a.rows) * 2), "idx"));
    KC_TRY(checkRange(a.dst, i32Bytes(int64_t(a.dst_rows) * a.dst_row), "dst"));
    const int want[5] = {a.pairs, a.rows, a.src_row, a.dst_row, a.dst_rows};
    return checkDims(a.dims, want, 5);
}
int setRowsLaunch(const void* p, void* s) { return kcamd::launchSetRows(*static_cast<const kcSetRowsF16Args*>(p), hs(s)); }

// ---- FLASH_ATTN_EXT: fa_scores, fa_max, fa_exp, fa_values (llm_kernels.cpp:972-1013) and the fused form

int faShape(const kcFaDims& d, const int* dims) {
    if (d.H <= 0 || d.T <= 0 || d.D <= 0 || d.D % 8 || d.H_kv <= 0 || d.group <= 0 || d.H != d.H_kv * d.group ||
        d.N <= 0 || d.tp % 8 || d.tp < d.T || d.k_row < 0 || d.k_head < 0 || d.v_row < 0 || d.v_head < 0 ||
        d.q_tok < 0 || d.q_head < d.D || d.m_row < 0 || (d.has_mask != 0 && d.has_mask != 1))
        return invalid("FaDims out of range");
    const int64_t cap = 1 << 24;
    if (!fitsIndex(int64_t(d.H) * d.N, d.tp) || int64_t(d.H) * d.N * d.tp >= cap || int64_t(d.N) * d.H * d.D >= cap ||
        !fitsIndex(d.T, std::max(d.k_row, d.v_row)) || !fitsIndex(d.N, std::max(d.q_tok, d.m_row)) ||
        !fitsIndex(d.H, d.q_head))
        return invalid("FaDims too large");
    const int want[15] = {d.H, d.T, d.D, d.group, d.tp, d.k_row, d.k_head, d.v_row, d.v_head, d.N, d.q_tok, d.q_head,
                          d.m_row, d.has_mask, d.H_kv};
    return checkDims(dims, want, 15);
}
size_t faScoreBytes(const kcFaDims& d) { return f32Bytes(int64_t(d.H) * d.N * d.tp); }
size_t faCacheBytes(const kcFaDims& d, int row, int head) {
    return (size_t(d.T - 1) * size_t(row) + size_t(d.H_kv - 1) * size_t(head) + size_t(d.D / 2)) * sizeof(int);
}
int faQMask(const kcFaDims& d, const float* q, const int* mask) {
    KC_TRY(checkRange(q, f32Bytes(int64_t(d.N - 1) * d.q_tok + int64_t(d.H - 1) * d.q_head + d.D), "q"));
    if (d.has_mask) return checkRange(mask, (size_t(d.N - 1) * size_t(d.m_row) + size_t(d.T + 1) / 2) * sizeof(int), "mask");
    return 0;
}

int faScoresValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcFaScoresArgs*>(p);
    KC_TRY(faShape(a.d, a.dims));
    KC_TRY(faQMask(a.d, a.q, a.mask));
    KC_TRY(checkRange(a.k, faCacheBytes(a.d, a.d.k_row, a.d.k_head), "k"));
    return checkRange(a.s, faScoreBytes(a.d), "s");
}
int faScoresLaunch(const void* p, void* s) { return kcamd::launchFaScores(*static_cast<const kcFaScoresArgs*>(p), hs(s)); }

int faMaxValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcFaMaxArgs*>(p);
    KC_TRY(faShape(a.d, a.dims));
    KC_TRY(checkRange(a.s, faScoreBytes(a.d), "s"));
    return checkRange(a.m, f32Bytes(int64_t(a.d.H) * a.d.N), "m");
}
int faMaxLaunch(const void* p, void* s) { return kcamd::launchFaMax(*static_cast<const kcFaMaxArgs*>(p), hs(s)); }

int faExpValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcFaExpArgs*>(p);
    KC_TRY(faShape(a.d, a.dims));
    KC_TRY(checkRange(a.s, faScoreBytes(a.d), "s"));
    return checkRange(a.m, f32Bytes(int64_t(a.d.H) * a.d.N), "m");
}
int faExpLaunch(const void* p, void* s) { return kcamd::launchFaExp(*static_cast<const kcFaExpArgs*>(p), hs(s)); }

int faValuesValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcFaValuesArgs*>(p);
    KC_TRY(faShape(a.d, a.dims));
    KC_TRY(checkRange(a.p, faScoreBytes(a.d), "p"));
    KC_TRY(checkRange(a.v, faCacheBytes(a.d, a.d.v_row, a.d.v_head), "v"));
    return checkRange(a.out, f32Bytes(int64_t(a.d.N) * a.d.H * a.d.D), "out");
}
int faValuesLaunch(const void* p, void* s) { return kcamd::launchFaValues(*static_cast<const kcFaValuesArgs*>(p), hs(s)); }

int flashValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcFlashAttnArgs*>(p);
    KC_TRY(faShape(a.d, a.dims));
    if (a.d.T > kcamd::kFlashAttnMaxT) return invalid("flash_attn_f16: T exceeds 16384 (use the fa_* kernels)");
    KC_TRY(faQMask(a.d, a.q, a.mask));
    KC_TRY(checkRange(a.k, faCacheBytes(a.d, a.d.k_row, a.d.k_head), "k"));
    KC_TRY(checkRange(a.v, faCacheBytes(a.d, a.d.v_row, a.d.v_head), "v"));
    return checkRange(a.out, f32Bytes(int64_t(a.d.N) * a.d.H * a.d.D), "out");
}
int flashLaunch(const void* p, void* s) { return kcamd::launchFlashAttn(*static_cast<const kcFlashAttnArgs*>(p), hs(s)); }

int flashDecodeValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcFlashDecodeArgs*>(p);
    KC_TRY(faShape(a.d, a.dims));
    if (!kcamd::flashDecodeSupports(a.d.D, a.d.group)) return invalid("flash_decode_f16: D must be 64 or 128, group at most 8");
    if (a.d.q_head % 4 || a.d.q_tok % 4) return invalid("flash_decode_f16: q rows and heads at 16-byte strides");
    KC_TRY(faQMask(a.d, a.q, a.mask));
    KC_TRY(checkRange(a.k, faCacheBytes(a.d, a.d.k_row, a.d.k_head), "k"));
    KC_TRY(checkRange(a.v, faCacheBytes(a.d, a.d.v_row, a.d.v_head), "v"));
    KC_TRY(checkRange(a.part, kcamd::flashDecodePartFloats(a.d) * sizeof(float), "part"));
    return checkRange(a.out, f32Bytes(int64_t(a.d.N) * a.d.H * a.d.D), "out");
}
int flashDecodeLaunch(const void* p, void* s) {
    return kcamd::launchFlashDecode(*static_cast<const kcFlashDecodeArgs*>(p), hs(s));
}

// ---- repack_kquant / unpack_kquant: ggml blocks <-> this device's weight stream

template <bool Unpack>
int repackValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcKquantRepackArgs*>(p);
    if (a.qtype != KC_QTYPE_Q4_K && a.qtype != KC_QTYPE_Q6_K) return invalid("qtype must be Q4_K (12) or Q6_K (14)");
    if (a.rows < 0 || a.k <= 0 || a.k % 256 != 0 || !fitsIndex(a.rows, a.k))
        return invalid("rows must be non-negative and k a positive multiple of 256");
    const bool q6 = a.qtype == KC_QTYPE_Q6_K;
    const size_t ggml = size_t(a.rows) * size_t(a.k / 256) * (q6 ? kcamd::kQ6kBlock : kcamd::kQ4kBlock);
    const size_t stream = kcamd::streamBytes(q6, a.rows, a.k);
    KC_TRY(checkRange(a.src, Unpack ? stream : ggml, "src"));
    KC_TRY(checkRange(a.dst, Unpack ? ggml : stream, "dst"));
    return 0;
}
template <bool Unpack>
int repackLaunch(const void* p, void* s) {
    return kcamd::launchRepack(*static_cast<const kcKquantRepackArgs*>(p), Unpack, hs(s));
}

// ---- get_rows_kquant (llm/llm_reference.cpp:342-383, used by llm/gguf_model.cpp:96-104)

int getRowsValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcGetRowsKquantArgs*>(p);
    if (a.qtype != KC_QTYPE_Q4_K && a.qtype != KC_QTYPE_Q6_K) return invalid("qtype must be Q4_K (12) or Q6_K (14)");
    if (a.rows < 0 || a.n < 0 || a.k <= 0 || a.k % 256 != 0 || !fitsIndex(a.rows, a.k) || !fitsIndex(a.n, a.k))
        return invalid("rows and n must be non-negative and k a positive multiple of 256");
    KC_TRY(checkRange(a.qw, kcamd::streamBytes(a.qtype == KC_QTYPE_Q6_K, a.rows, a.k), "qw"));
    KC_TRY(checkRange(a.ids, i32Bytes(a.n), "ids"));
    return checkRange(a.y, f32Bytes(int64_t(a.n) * a.k), "y");
}
int getRowsLaunch(const void* p, void* s) {
    const auto& a = *static_cast<const kcGetRowsKquantArgs*>(p);
    return kcamd::launchGetRows(a.qtype == KC_QTYPE_Q6_K, a.qw, a.ids, a.y, a.n, a.k, a.rows, hs(s));
}

// ---- quantize_kquant / fill_normal_f32 (synthetic weights; no reference kernel)

int quantKquantValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcQuantizeKquantArgs*>(p);
    if (a.qtype != KC_QTYPE_Q4_K && a.qtype != KC_QTYPE_Q6_K) return invalid("qtype must be Q4_K (12) or Q6_K (14)");
    if (a.rows < 0 || a.k <= 0 || a.k % 256 != 0 || !fitsIndex(a.rows, a.k / 256))
        return invalid("rows must be non-negative and k a positive multiple of 256");
    const size_t n = size_t(a.rows) * size_t(a.k);
    KC_TRY(checkRange(a.x, n * sizeof(float), "x"));
    return checkRange(a.blocks, n / 256 * (a.qtype == KC_QTYPE_Q6_K ? kcamd::kQ6kBlock : kcamd::kQ4kBlock), "blocks");
}
int quantKquantLaunch(const void* p, void* s) {
    const auto& a = *static_cast<const kcQuantizeKquantArgs*>(p);
    return kcamd::launchQuantizeKquant(a.qtype == KC_QTYPE_Q6_K, a.x, a.blocks, (long long)a.rows * (a.k / 256), hs(s));
}

int fillNormalValidate(const void* p, const kcLaunchContext*) {
    const auto& a = *static_cast<const kcFillNormalArgs*>(p);
    if (a.n < 0) return invalid("n < 0");
    return checkRange(a.y, size_t(a.n) * sizeof(float), "y");
}
int fillNormalLaunch(const void* p, void* s) {
    const auto& a = *static_cast<const kcFillNormalArgs*>(p);
    return kcamd::launchFillNormal(a.y, a.n, a.seed, a.mean, a.stdev, hs(s));
}

const kcKernelEntry kTable[] = {
    {"vector_add", vectorAddValidate, vectorAddLaunch, 1},
    {"quantize_q8x4", quantValidate, quantLaunch, 1},
    {"quantize_cols", quantColsValidate<32>, quantColsLaunch<32>, 1},
    {"quantize_cols_k", quantColsValidate<256>, quantColsLaunch<256>, 1},
    {"matvec_q4k_q8", kquantValidate<false>, kquantLaunch<false>, 1},
    {"matvec_q6k_q8", kquantValidate<true>, kquantLaunch<true>, 1},
    {"matmul_q4k_q8x4", matmulValidate<false, false>, matmulLaunch<false, false>, 1},
    {"matmul_q4k_q8x8", matmulValidate<false, false>, matmulLaunch<false, false>, 1},
    {"matmul_q6k_q8x4", matmulValidate<true, false>, matmulLaunch<true, false>, 1},
    {"matmul_q6k_q8x8", matmulValidate<true, false>, matmulLaunch<true, false>, 1},
    {"matmul_q4k_q8kx4", matmulValidate<false, true>, matmulLaunch<false, true>, 1},
    {"matmul_q4k_q8kx8", matmulValidate<false, true>, matmulLaunch<false, true>, 1},
    {"matmul_q6k_q8kx4", matmulValidate<true, true>, matmulLaunch<true, true>, 1},
    {"matmul_q6k_q8kx8", matmulValidate<true, true>, matmulLaunch<true, true>, 1},
    {"matmul_f16", matmulF16Validate, matmulF16Launch, 1},
    {"add_sumsq_f", addSumsqValidate, addSumsqLaunch, 1},
    {"sumsq_part", sumsqValidate, sumsqLaunch, 1},
    {"norm_mul_q8_f", normMulValidate<false>, normMulLaunch<false>, 1},
    {"norm_mul_q8k_f", normMulValidate<true>, normMulLaunch<true>, 1},
    {"add_norm_q8_f", addNormValidate, addNormLaunch, 1},
    {"silu_mul_q8x4f", siluQValidate<false>, siluQLaunch<false>, 1},
    {"silu_mul_q8kf", siluQValidate<true>, siluQLaunch<true>, 1},
    {"rms_norm", rmsValidate, rmsLaunch, 1},
    {"mul_rows", mulRowsValidate, mulRowsLaunch, 0},
    {"silu_mul", siluValidate, siluLaunch, 1},
    {"rope_ggml", ropeValidate, ropeLaunch, 0},
    {"set_rows_f16", setRowsValidate, setRowsLaunch, 1},
    {"fa_scores", faScoresValidate, faScoresLaunch, 1},
    {"fa_max", faMaxValidate, faMaxLaunch, 1},
    {"fa_exp", faExpValidate, faExpLaunch, 1},
    {"fa_values", faValuesValidate, faValuesLaunch, 1},
    {"flash_attn_f16", flashValidate, flashLaunch, 0},
    {"flash_decode_f16", flashDecodeValidate, flashDecodeLaunch, 0},
    {"repack_kquant", repackValidate<false>, repackLaunch<false>, 0},
    {"unpack_kquant", repackValidate<true>, repackLaunch<true>, 0},
    {"get_rows_kquant", getRowsValidate, getRowsLaunch, 0},
    {"quantize_kquant", quantKquantValidate, quantKquantLaunch, 0},
    {"fill_normal_f32", fillNormalValidate, fillNormalLaunch, 0},
};

}  // namespace

const kcKernelEntry* kcamd::builtinKernels(size_t* count) {
    *count = sizeof kTable / sizeof kTable[0];
    return kTable;
}

kcError_t kcKquantStreamBytes(int qtype, int rows, int k, size_t* bytes) noexcept {
    if (!bytes || (qtype != KC_QTYPE_Q4_K && qtype != KC_QTYPE_Q6_K) || rows < 0 || k <= 0 || k % 256 != 0)
        return kc::Error::InvalidValue;
    *bytes = kcamd::streamBytes(qtype == KC_QTYPE_Q6_K, rows, k);
    return kc::Error::Success;
}
