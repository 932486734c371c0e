// llm_kernels.cpp -- the built-in kernel table: argument validation and launch per kernel name.
//
// Validation keeps the reference's rules (arasheedu/Kernelcore llm/llm_kernels.cpp): sizes must
// be positive and fit int32 indexing, every buffer must lie inside one live allocation, and the
// shape rules of each kernel (rows % 8, k % 256, ...) hold. A rejected launch returns
// InvalidValue or InvalidPointer with a detail text, as there. The System V marshalling, chunk
// planning and CPU executor are replaced by one HIP grid per launch (launch.hpp).
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "internal.hpp"
#include "kquant.hpp"
#include "launch.hpp"

namespace kcamd {
int launchVectorAdd(const float* a, const float* b, float* out, int count, hipStream_t s);
}

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
    {"repack_kquant", repackValidate<false>, repackLaunch<false>, 0},
    {"unpack_kquant", repackValidate<true>, repackLaunch<true>, 0},
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
