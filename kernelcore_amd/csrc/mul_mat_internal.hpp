// mul_mat_internal.hpp -- the MUL_MAT recording shared by kcMulMat* (mul_mat.cpp) and the ggml
// backend core (ggml_backend.cpp): its scratch, its cache of quantized inputs and the dispatch
// functions behind the public calls.
#pragma once

#include <cstddef>
#include <string>
#include <vector>

#include "kernelcore/mul_mat.h"
#include "launch.hpp"

namespace kcamd {
// Device times of launches (the ggml backend's profile = 2): an event pair on the recording's stream
// around each launch, named by its kernel and the weight shape of the MUL_MAT it serves.
struct LaunchTimer {
    std::string tag;  // "rows x k" of the MUL_MAT (group) being launched, else empty
    struct Mark {
        std::string name;
        hipEvent_t a, b;
    };
    std::vector<Mark> marks;
    std::vector<hipEvent_t> pool;  // created once, reused by every call
    size_t used = 0;
    hipEvent_t next();  // nullptr when HIP cannot create one
};
}  // namespace kcamd

struct kcMulMatRecording_st {
    kcMulMatConfig cfg{};
    kcStream_t stream = nullptr;
    int* scratch = nullptr;
    size_t cap = 0;   // ints
    size_t used = 0;  // ints taken by this recording
    size_t peak = 0;  // the most ints taken since the last reset (a dry recording's requirement)
    unsigned gen = 0; // bumped whenever the scratch buffer is replaced
    // A dry recording plans: it takes scratch offsets and names its kernels without allocating or
    // launching anything (no device is needed); pointers it hands out are never dereferenced.
    bool dry = false;
    std::vector<const char*>* trace = nullptr;  // when set: every kernel name, in launch order
    // A cached input is found by its key: the input's data pointer for kcMulMat* callers, the tensor's
    // identity for the ggml backend (whose allocator hands a freed tensor's memory to a later one).
    struct Input {
        const void* key;
        long long ncols;
        int k;
        bool k256;
        int* q;
        kcamd::ActF16 act{};  // the fp16 MFMA form of the slots, when has_act
        bool has_act = false;
    };
    std::vector<Input> inputs;  // the recording's quantized inputs
    // The ggml backend's recordings: per-256 producers of at least 64 columns that the MFMA matmul
    // takes also write the fp16 form it reads, so the matmuls convert nothing (kcMulMat* leave it off).
    bool act_f16 = false;
    kcamd::LaunchTimer* timer = nullptr;  // when set (never with a dry or capturing recording): each launch timed
};

namespace kcamd::mulmat {

// tile 4 or 8, row_block >= 1; the flags normalised to 0 / 1
kcError_t checkConfig(kcMulMatConfig& c) noexcept;
// a new recording: the cached inputs dropped, the scratch reused from its start
void reset(kcMulMatRecording_st& r) noexcept;
// the scratch holds at least `ints` ints (replacing it waits for the stream and drops the cache)
kcError_t reserve(kcMulMatRecording_st& r, size_t ints) noexcept;
// `ints` ints of the recording's scratch (64-byte multiples), growing it if needed
kcError_t take(kcMulMatRecording_st& r, size_t ints, int** out) noexcept;
// one launch on the recording's stream (dry: named only)
kcError_t launch(kcMulMatRecording_st& r, const char* kernel, const void* args) noexcept;
// fn(hip stream) -> kc code: one launch of a launcher of this build, on the recording's stream,
// timed when the recording has a timer
template <class F>
kcError_t timed(kcMulMatRecording_st& r, const char* kernel, F&& fn) noexcept {
    void* hs = nullptr;
    if (kcError_t e = kcStreamGetNative(r.stream, &hs); e != kc::Error::Success) return e;
    const auto s = static_cast<hipStream_t>(hs);
    hipEvent_t a = r.timer ? r.timer->next() : nullptr, b = r.timer ? r.timer->next() : nullptr;
    if (a && b) (void)hipEventRecord(a, s);
    const auto e = static_cast<kcError_t>(fn(s));
    if (a && b) {
        (void)hipEventRecord(b, s);
        try {
            r.timer->marks.push_back({r.timer->tag.empty() ? std::string(kernel) : std::string(kernel) + " " + r.timer->tag,
                                      a, b});
        } catch (...) {
            return kc::Error::OutOfMemory;
        }
    }
    return e;
}
// Keys: where a function takes `key`, nullptr means the data pointer (the input's x, the output's y).
// the recording's 8-bit slots of the input with this key (nullptr when it made none)
int* inputSlot(const kcMulMatRecording_st& r, const void* key, long long ncols, int k, bool k256) noexcept;
// the fp16 MFMA form of that input's per-256 slots (nullptr when no producer wrote it)
const kcamd::ActF16* inputAct(const kcMulMatRecording_st& r, const void* key, long long ncols, int k) noexcept;
// slots for the 8-bit form of an output registered under key, for a producer that writes them itself
// (the MUL_MATs that read that output then take them)
kcError_t outputSlot(kcMulMatRecording_st& r, const void* key, int k, long long ncols, bool k256, int** q) noexcept;

kcError_t mulMat(kcMulMatRecording_st& r, const kcMulMatNode& n, kcMulMatPlan& plan,
                 const void* key = nullptr) noexcept;
// the node's 8-bit input made now (the reference's mul_mat_input; nothing for F16 weights)
kcError_t mulMatInput(kcMulMatRecording_st& r, const kcMulMatNode& n, kcMulMatPlan& plan,
                      const void* key = nullptr) noexcept;
// b2 (with an ADD, only where fusesHalf): x = a + (b + b2), the second K half of the product b;
// the slots are registered under key (nullptr: n.y)
kcError_t fusedNorm(kcMulMatRecording_st& r, const kcMulMatNormNode& n, kcMulMatPlan& plan,
                    const float* b2 = nullptr, const void* key = nullptr) noexcept;
// whether fusedNorm of rows of n values takes a b2 (the per-256 norm in one workgroup per row)
bool fusesHalf(const kcMulMatRecording_st& r, int n) noexcept;
kcError_t fusedSwiglu(kcMulMatRecording_st& r, const kcMulMatSwigluNode& n, kcMulMatPlan& plan,
                      const void* key = nullptr) noexcept;

}  // namespace kcamd::mulmat
