// weights.cpp -- kcWeightAllocSize / kcWeightSetTensor / kcWeightGetTensor: the backend buffer's
// tensor uploads and reads (integrations/llama.cpp/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp:
// weight_shape_ok :103-109, buffer_set_tensor :175-191, buffer_get_tensor :193-206,
// buft get_alloc_size :259-266) over the public kc* calls: a K-quant weight is staged on the
// device as ggml blocks and repacked there (repack_kquant) into the stream; reads unpack it
// (unpack_kquant) and copy the asked range back.
#include <cstdint>

#include "internal.hpp"
#include "kernelcore/llm_kernels.h"
#include "kernelcore/model.h"
#include "kernelcore/weights.h"

namespace {

using E = kcError_t;
constexpr E ok = kc::Error::Success;

E bad(const char* why) {
    kcamd::setDetail("weights: %s", why);
    return kc::Error::InvalidValue;
}

bool kquant(int qtype) { return qtype == KC_QTYPE_Q4_K || qtype == KC_QTYPE_Q6_K; }

// The tensor's ggml bytes, after the shape checks (K-quant: rows % 8, k % 256 -- the kernels' and
// weight_shape_ok's rule; fp16 weights: k even).
E ggmlBytes(int qtype, int rows, int k, size_t* bytes) {
    if (rows <= 0 || k <= 0) return bad("rows and k must be positive");
    switch (qtype) {
        case KC_QTYPE_F32: *bytes = size_t(rows) * size_t(k) * 4; return ok;
        case KC_QTYPE_F16:
            if (k % 2) return bad("fp16 weights need an even k");
            *bytes = size_t(rows) * size_t(k) * 2;
            return ok;
        case KC_QTYPE_Q4_K:
        case KC_QTYPE_Q6_K:
            if (rows % 8 || k % 256) return bad("K-quant weights need rows % 8 == 0 and k % 256 == 0");
            *bytes = size_t(rows) * size_t(k / 256) * (qtype == KC_QTYPE_Q4_K ? 144 : 210);
            return ok;
        default: return bad("qtype must be F32 (0), F16 (1), Q4_K (12) or Q6_K (14)");
    }
}

E range(int qtype, int rows, int k, const void* dev, const void* host, size_t offset, size_t size, size_t* total) {
    if (E e = ggmlBytes(qtype, rows, k, total); e != ok) return e;
    if (offset > *total || size > *total - offset) return bad("offset + size beyond the tensor");
    if (size && (!dev || !host)) return bad("null device or host pointer");
    return ok;
}

// A device staging buffer freed on every path.
struct Staging {
    void* p = nullptr;
    ~Staging() {
        if (p) (void)kcFree(p);
    }
};

}  // namespace

KC_API kcError_t kcWeightAllocSize(int qtype, int rows, int k, size_t* bytes) noexcept {
    if (!bytes) return bad("null result pointer");
    if (E e = ggmlBytes(qtype, rows, k, bytes); e != ok) return e;
    if (kquant(qtype)) return kcKquantStreamBytes(qtype, rows, k, bytes);
    return ok;
}

KC_API kcError_t kcWeightSetTensor(int qtype, int rows, int k, void* dst, const void* host, size_t offset, size_t size,
                                   kcStream_t stream) noexcept {
    size_t total = 0;
    if (E e = range(qtype, rows, k, dst, host, offset, size, &total); e != ok) return e;
    if (E e = kcStreamSynchronize(stream); e != ok) return e;  // after the stream's earlier reads of dst
    if (!kquant(qtype)) return size ? kcMemcpy(static_cast<char*>(dst) + offset, host, size, kc::CopyKind::HostToDevice) : ok;
    if (offset != 0 || size != total) return bad("K-quant weights are uploaded whole (offset 0, every byte)");
    Staging st;
    if (E e = kcMalloc(&st.p, total); e != ok) return e;
    if (E e = kcMemcpy(st.p, host, total, kc::CopyKind::HostToDevice); e != ok) return e;
    const kcKquantRepackArgs a{st.p, dst, qtype, rows, k};
    if (E e = kcLaunchKernel("repack_kquant", &a, stream); e != ok) return e;
    return kcStreamSynchronize(stream);
}

KC_API kcError_t kcWeightMemsetTensor(int qtype, int rows, int k, void* dst, int value, size_t offset, size_t size,
                                      kcStream_t stream) noexcept {
    size_t total = 0;
    if (E e = range(qtype, rows, k, dst, dst, offset, size, &total); e != ok) return e;
    if (E e = kcStreamSynchronize(stream); e != ok) return e;  // after the stream's earlier use of dst
    if (!size) return ok;
    if (!kquant(qtype)) return kcMemset(static_cast<char*>(dst) + offset, value, size);
    Staging st;  // the ggml blocks: unpacked, the range set, repacked
    if (E e = kcMalloc(&st.p, total); e != ok) return e;
    const kcKquantRepackArgs un{dst, st.p, qtype, rows, k};
    if (E e = kcLaunchKernel("unpack_kquant", &un, stream); e != ok) return e;
    if (E e = kcStreamSynchronize(stream); e != ok) return e;
    if (E e = kcMemset(static_cast<char*>(st.p) + offset, value, size); e != ok) return e;
    const kcKquantRepackArgs re{st.p, dst, qtype, rows, k};
    if (E e = kcLaunchKernel("repack_kquant", &re, stream); e != ok) return e;
    return kcStreamSynchronize(stream);
}

KC_API kcError_t kcWeightGetTensor(int qtype, int rows, int k, const void* src, void* host, size_t offset, size_t size,
                                   kcStream_t stream) noexcept {
    size_t total = 0;
    if (E e = range(qtype, rows, k, src, host, offset, size, &total); e != ok) return e;
    if (E e = kcStreamSynchronize(stream); e != ok) return e;  // after the stream's writes of src
    if (!size) return ok;
    if (!kquant(qtype))
        return kcMemcpy(host, static_cast<const char*>(src) + offset, size, kc::CopyKind::DeviceToHost);
    Staging st;
    if (E e = kcMalloc(&st.p, total); e != ok) return e;
    const kcKquantRepackArgs a{src, st.p, qtype, rows, k};
    if (E e = kcLaunchKernel("unpack_kquant", &a, stream); e != ok) return e;
    if (E e = kcStreamSynchronize(stream); e != ok) return e;
    return kcMemcpy(host, static_cast<const char*>(st.p) + offset, size, kc::CopyKind::DeviceToHost);
}
