// runtime.cpp -- the kc* runtime surface (include/kernelcore/kc.h) over HIP on MI355X.
//
// Semantics follow the reference runtime (arasheedu/Kernelcore src/runtime.cpp): every call is
// noexcept and returns a fixed error code; detail text is thread-local and reset per call
// (runtime.cpp:209-228); calls before kcInit return NotInitialized; a kernel fault poisons the
// context until kcDeviceReset (:238-252); copies, memsets, frees and device syncs are refused
// while any stream captures (:449-455). The CPU executor, worker pool and chunk planner are
// gone: a launch is one HIP grid, a stream is a hipStream_t, a graph is a hipGraphExec_t.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <new>
#include <shared_mutex>
#include <string>
#include <vector>

#include "internal.hpp"
#include "launch.hpp"

namespace {

constexpr size_t kShadowMax = 256;   // allocations up to this size keep a host copy (dims checks)
constexpr int kMaxSideStreams = 16;  // parallel branches of one concurrent group

struct Allocation {
    size_t bytes = 0;
    std::vector<uint8_t> shadow;  // host copy of small allocations
    std::vector<uint8_t> known;   // per byte: the shadow holds the device value
};

thread_local std::string t_detail;
thread_local bool t_in_host_func = false;

}  // namespace

struct kcStream_st {
    hipStream_t s = nullptr;
    bool capturing = false;
    bool concurrent = false;           // a kcStreamConcurrentBegin group is open
    hipEvent_t fork = nullptr;         // recorded on `s` when the group opened
    std::vector<hipStream_t> side;     // side streams of concurrent groups
    std::vector<hipEvent_t> side_done; // recorded on side[i] after its launch
    size_t side_used = 0;              // side streams used by the open group
};
struct kcEvent_st {
    hipEvent_t ev = nullptr;
    bool timed = false;
};
struct kcGraph_st {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace {

struct Runtime {
    std::shared_mutex lifecycle;
    bool initialized = false;
    std::atomic<bool> poisoned{false};
    int device = 0;
    std::unique_ptr<kcStream_st> default_stream;

    std::mutex objects_mutex;
    std::map<kcStream_t, std::unique_ptr<kcStream_st>> streams;
    std::map<kcEvent_t, std::unique_ptr<kcEvent_st>> events;
    std::map<kcGraph_t, std::unique_ptr<kcGraph_st>> graphs;

    std::shared_mutex alloc_mutex;
    std::map<uintptr_t, Allocation> allocs;

    std::mutex kernels_mutex;
    std::map<std::string, const kcKernelEntry*> kernels;

    std::mutex capture_mutex;  // capture / concurrent-group state of every stream
    std::atomic<int> capture_count{0};

    std::mutex fault_mutex;
    kcFaultInfo last_fault{};
    bool has_fault = false;

    std::atomic<int> codegen{KC_CODEGEN_AUTO};
    std::mutex options_mutex;
    std::map<std::string, int> options;
    std::atomic<unsigned> options_gen{0};  // bumped by every kcSetKernelOption

    // Device scratch of kernels that stage operands (kcamd::streamScratch), one buffer per HIP
    // stream. A buffer handed out while its stream was capturing may be baked into a graph, so it
    // is never freed before the device stops: when it is replaced or its stream goes away it moves
    // to `retired_scratch`.
    struct Scratch {
        void* p = nullptr;
        size_t bytes = 0;
        bool in_graph = false;
    };
    std::mutex scratch_mutex;
    std::map<hipStream_t, Scratch> scratch;
    std::vector<void*> retired_scratch;
};

// Intentionally leaked: no HIP call may run from a static destructor after the runtime unloads.
Runtime& R() {
    static Runtime* r = new Runtime();
    return *r;
}

using E = kcError_t;
constexpr E ok = kc::Error::Success;
inline E err(int code) { return static_cast<E>(code); }
inline int code(E e) { return static_cast<int>(e); }

// What an entry point needs of the runtime: nothing, an initialized runtime, or one that is also
// not poisoned by a kernel fault.
enum class Need { Nothing, Init, Live };

E stateError(const Runtime& r, Need need) {
    if (need == Need::Nothing) return ok;
    if (!r.initialized) {
        kcamd::setDetail("the runtime is not running: kcInit has not been called, or kcShutdown ended it");
        return kc::Error::NotInitialized;
    }
    if (need == Need::Live && r.poisoned.load()) {
        kcamd::setDetail("a kernel fault poisoned the context; only kcDeviceReset clears it");
        return kc::Error::ContextPoisoned;
    }
    return ok;
}

// The error code for the exception being handled (called only from inside a catch block).
E codeOfCurrentException(const char* fn) noexcept {
    try {
        throw;
    } catch (const std::bad_alloc&) {
        kcamd::setDetail("%s: host memory exhausted", fn);
        return kc::Error::OutOfMemory;
    } catch (const std::exception& e) {
        kcamd::setDetail("%s: internal error (%s)", fn, e.what());
        return kc::Error::InternalError;
    } catch (...) {
        kcamd::setDetail("%s: internal error (non-standard exception)", fn);
        return kc::Error::InternalError;
    }
}

// Every entry point runs its body through one of these two gates. A gate starts the call's detail
// text empty, refuses calls made from a host function running on a stream (that thread belongs to
// HIP), holds the lifecycle lock (shared here, exclusive for init / shutdown / reset) for the whole
// body, checks the state `N` the body needs, and lets no exception out.
bool refuseFromHostFunc(const char* fn) {
    if (!t_in_host_func) return false;
    kcamd::setDetail("%s: a host function enqueued with kcLaunchHostFunc may not call the runtime", fn);
    return true;
}

template <Need N, class Body>
E gated(const char* fn, Body&& body) noexcept {
    t_detail.clear();
    if (refuseFromHostFunc(fn)) return kc::Error::UnsupportedOperation;
    try {
        Runtime& r = R();
        if constexpr (N == Need::Nothing) {
            return body(r);
        } else {
            std::shared_lock life(r.lifecycle);
            if (E e = stateError(r, N); e != ok) return e;
            return body(r);
        }
    } catch (...) {
        return codeOfCurrentException(fn);
    }
}

template <class Body>
E exclusive(const char* fn, Body&& body) noexcept {
    t_detail.clear();
    if (refuseFromHostFunc(fn)) return kc::Error::UnsupportedOperation;
    try {
        Runtime& r = R();
        std::unique_lock life(r.lifecycle);
        return body(r);
    } catch (...) {
        return codeOfCurrentException(fn);
    }
}

E rejectDuringCapture(Runtime& r, const char* what) {
    if (r.capture_count.load() == 0) return ok;
    kcamd::setDetail("%s is not allowed while a stream is capturing (end the capture first)", what);
    return kc::Error::UnsupportedOperation;
}

E findStream(Runtime& r, kcStream_t h, kcStream_st** out) {
    if (!h) {
        *out = r.default_stream.get();
        return ok;
    }
    std::lock_guard lk(r.objects_mutex);
    if (!r.streams.count(h)) {
        kcamd::setDetail("unknown stream handle");
        return kc::Error::InvalidResourceHandle;
    }
    *out = h;
    return ok;
}

E findEvent(Runtime& r, kcEvent_t h, kcEvent_st** out) {
    std::lock_guard lk(r.objects_mutex);
    if (!h || !r.events.count(h)) {
        kcamd::setDetail("unknown event handle");
        return kc::Error::InvalidResourceHandle;
    }
    *out = h;
    return ok;
}

void recordFault(Runtime& r, int hip_status, const char* what) {
    std::lock_guard lk(r.fault_mutex);
    r.last_fault = kcFaultInfo{};
    r.last_fault.code = static_cast<uint32_t>(hip_status);
    std::snprintf(r.last_fault.kernel, sizeof r.last_fault.kernel, "%s", what ? what : "");
    r.has_fault = true;
    r.poisoned.store(true);
}

bool isFault(hipError_t s) {
    return s == hipErrorIllegalAddress || s == hipErrorLaunchFailure || s == hipErrorIllegalState ||
           s == hipErrorAssert || s == hipErrorLaunchTimeOut || s == hipErrorECCNotCorrectable;
}

// Every stream idle; the first error is returned.
E waitAllIdle(Runtime& r, const char* what) {
    std::vector<hipStream_t> snap;
    if (r.default_stream) snap.push_back(r.default_stream->s);
    {
        std::lock_guard lk(r.objects_mutex);
        for (auto& [h, s] : r.streams) snap.push_back(s->s);
    }
    E first = ok;
    for (hipStream_t s : snap) {
        const int e = kcamd::fromHip(hipStreamSynchronize(s), what);
        if (first == ok && e != 0) first = err(e);
    }
    return first;
}

E createStream(kcStream_st* st) {
    if (int e = kcamd::fromHip(hipStreamCreateWithFlags(&st->s, hipStreamNonBlocking), "hipStreamCreate"))
        return err(e);
    return ok;
}

// Gives back the scratch of a drained stream (kept until the device stops if a graph may use it).
void releaseScratch(Runtime& r, hipStream_t s) {
    std::lock_guard lk(r.scratch_mutex);
    auto it = r.scratch.find(s);
    if (it == r.scratch.end()) return;
    if (it->second.in_graph) r.retired_scratch.push_back(it->second.p);
    else (void)hipFree(it->second.p);
    r.scratch.erase(it);
}

void freeAllScratch(Runtime& r) {
    std::lock_guard lk(r.scratch_mutex);
    for (auto& [s, sc] : r.scratch) (void)hipFree(sc.p);
    for (void* p : r.retired_scratch) (void)hipFree(p);
    r.scratch.clear();
    r.retired_scratch.clear();
}

void destroyStream(kcStream_st* st) {
    if (st->s) (void)hipStreamSynchronize(st->s);
    for (hipStream_t s : st->side) {
        (void)hipStreamSynchronize(s);
        releaseScratch(R(), s);
    }
    if (st->s) releaseScratch(R(), st->s);
    for (hipStream_t s : st->side) (void)hipStreamDestroy(s);
    for (hipEvent_t e : st->side_done) (void)hipEventDestroy(e);
    if (st->fork) (void)hipEventDestroy(st->fork);
    if (st->s) (void)hipStreamDestroy(st->s);
    st->side.clear();
    st->side_done.clear();
    st->fork = nullptr;
    st->s = nullptr;
}

void registerBuiltins(Runtime& r) {
    size_t n = 0;
    const kcKernelEntry* table = kcamd::builtinKernels(&n);
    std::lock_guard lk(r.kernels_mutex);
    for (size_t i = 0; i < n; ++i) r.kernels[table[i].name] = &table[i];
}

E startDevice(Runtime& r) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        kcamd::setDetail("no HIP device is visible");
        return kc::Error::InvalidDevice;
    }
    if (int e = kcamd::fromHip(hipSetDevice(0), "hipSetDevice")) return err(e);
    r.device = 0;
    r.default_stream = std::make_unique<kcStream_st>();
    if (E e = createStream(r.default_stream.get()); e != ok) return e;
    // the fixed scratch of kcLaunchMatmulNoAlloc: its device address, looked up once per device
    // (a failure leaves that entry point refusing calls; everything else works)
    (void)kcamd::fixedScratchInit(r.device);
    r.poisoned.store(false);
    {
        std::lock_guard lk(r.fault_mutex);
        r.has_fault = false;
        r.last_fault = kcFaultInfo{};
    }
    registerBuiltins(r);
    return ok;
}

// Frees every object and allocation; returns how many allocations were still live.
size_t stopDevice(Runtime& r) {
    if (r.default_stream) (void)hipStreamSynchronize(r.default_stream->s);
    std::lock_guard lk(r.objects_mutex);
    for (auto& [h, s] : r.streams) destroyStream(s.get());
    r.streams.clear();
    for (auto& [h, g] : r.graphs) {
        if (g->exec) (void)hipGraphExecDestroy(g->exec);
        if (g->graph) (void)hipGraphDestroy(g->graph);
    }
    r.graphs.clear();
    for (auto& [h, e] : r.events) (void)hipEventDestroy(e->ev);
    r.events.clear();
    if (r.default_stream) destroyStream(r.default_stream.get());
    r.default_stream.reset();
    freeAllScratch(r);
    std::unique_lock alk(r.alloc_mutex);
    const size_t leaked = r.allocs.size();
    for (auto& [base, a] : r.allocs) (void)hipFree(reinterpret_cast<void*>(base));
    r.allocs.clear();
    r.capture_count.store(0);
    return leaked;
}

// Host copy bookkeeping for small allocations. `src` null: the bytes become unknown.
void shadowWrite(Runtime& r, void* dst, const void* src, int fill, size_t bytes) {
    std::unique_lock lk(r.alloc_mutex);
    const auto key = reinterpret_cast<uintptr_t>(dst);
    auto it = r.allocs.upper_bound(key);
    if (it == r.allocs.begin()) return;
    --it;
    Allocation& a = it->second;
    if (a.shadow.empty()) return;
    const size_t off = key - it->first;
    if (off >= a.bytes) return;
    const size_t n = std::min(bytes, a.bytes - off);
    if (src == reinterpret_cast<const void*>(1)) {  // memset
        std::memset(a.shadow.data() + off, fill, n);
        std::memset(a.known.data() + off, 1, n);
    } else if (src) {
        std::memcpy(a.shadow.data() + off, src, n);
        std::memset(a.known.data() + off, 1, n);
    } else {
        std::memset(a.known.data() + off, 0, n);
    }
}

// Called through gated<Need::Live>: the lifecycle lock is held and the context is usable.
E launchCommon(Runtime& r, const char* name, const void* typed_args, kcStream_t stream, bool chunked, unsigned workers) {
    if (!name) {
        kcamd::setDetail("kernel name is null");
        return kc::Error::InvalidValue;
    }
    const kcKernelEntry* entry = nullptr;
    {
        std::lock_guard lk(r.kernels_mutex);
        auto it = r.kernels.find(name);
        if (it == r.kernels.end()) {
            kcamd::setDetail("no kernel registered as '%s'", name);
            return kc::Error::KernelNotFound;
        }
        entry = it->second;
    }
    kcStream_st* st = nullptr;
    if (E e = findStream(r, stream, &st); e != ok) return e;
    if (!typed_args) {
        kcamd::setDetail("typed_args is null");
        return kc::Error::InvalidValue;
    }
    if (chunked) {
        if (!entry->chunkable) {
            kcamd::setDetail("kernel '%s' is not registered as chunkable", name);
            return kc::Error::UnsupportedOperation;
        }
        if (workers == 0 || workers > 1024) {
            kcamd::setDetail("workers must be in [1, 1024]");
            return kc::Error::InvalidValue;
        }
    }
    kcLaunchContext ctx{0};
    if (int e = entry->validate(typed_args, &ctx); e != 0) {
        if (!kcamd::hasDetail()) kcamd::setDetail("kernel '%s': argument validation failed", name);
        return err(e);
    }

    std::lock_guard cap(r.capture_mutex);  // serializes launches with capture-state changes
    hipStream_t hs = st->s;
    int side = -1;
    if (st->capturing && st->concurrent) {  // a branch of the open concurrent group
        if (st->side_used >= static_cast<size_t>(kMaxSideStreams)) {
            kcamd::setDetail("more than %d launches in one concurrent group", kMaxSideStreams);
            return kc::Error::UnsupportedOperation;
        }
        side = static_cast<int>(st->side_used++);
        while (st->side.size() <= static_cast<size_t>(side)) {
            hipStream_t s2 = nullptr;
            hipEvent_t e2 = nullptr;
            if (int e = kcamd::fromHip(hipStreamCreateWithFlags(&s2, hipStreamNonBlocking), "hipStreamCreate"))
                return err(e);
            if (int e = kcamd::fromHip(hipEventCreateWithFlags(&e2, hipEventDisableTiming), "hipEventCreate")) {
                (void)hipStreamDestroy(s2);
                return err(e);
            }
            st->side.push_back(s2);
            st->side_done.push_back(e2);
        }
        hs = st->side[side];
        if (int e = kcamd::fromHip(hipStreamWaitEvent(hs, st->fork, 0), "hipStreamWaitEvent")) return err(e);
    }
    (void)hipGetLastError();
    if (int e = entry->launch(typed_args, hs); e != 0) {
        if (!kcamd::hasDetail()) kcamd::setDetail("kernel '%s': launch failed", name);
        return err(e);
    }
    if (int e = kcamd::fromHip(hipGetLastError(), name)) return err(e == KC_ERROR_KERNEL_FAULT ? e : KC_ERROR_LAUNCH_FAILURE);
    if (side >= 0) {
        if (int e = kcamd::fromHip(hipEventRecord(st->side_done[side], hs), "hipEventRecord")) return err(e);
        return ok;
    }
    if (!stream && !st->capturing) return err(kcamd::fromHip(hipStreamSynchronize(hs), name));
    return ok;
}

}  // namespace

// ================================================================ internal helpers

namespace kcamd {

void setDetail(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    try {
        t_detail = buf;
    } catch (...) {
    }
}

bool hasDetail() { return !t_detail.empty(); }

int checkRange(const void* ptr, size_t bytes, const char* what) {
    if (bytes == 0) return 0;
    if (!ptr) {
        setDetail("%s: null device pointer", what);
        return KC_ERROR_INVALID_POINTER;
    }
    Runtime& r = R();
    std::shared_lock lk(r.alloc_mutex);
    const auto key = reinterpret_cast<uintptr_t>(ptr);
    auto it = r.allocs.upper_bound(key);
    if (it == r.allocs.begin()) {
        setDetail("%s: pointer %p is not inside any allocation", what, ptr);
        return KC_ERROR_INVALID_POINTER;
    }
    --it;
    const size_t size = it->second.bytes;
    const uintptr_t off = key - it->first;
    if (off >= size) {
        setDetail("%s: pointer %p is not inside any allocation", what, ptr);
        return KC_ERROR_INVALID_POINTER;
    }
    if (bytes > size - off) {
        setDetail("%s: range [%p, +%zu) exceeds the allocation of %zu bytes at offset %zu", what, ptr, bytes, size,
                  static_cast<size_t>(off));
        return KC_ERROR_INVALID_POINTER;
    }
    return 0;
}

bool dimsAgree(const int* dims, const int* want, int n) {
    if (!dims) return true;
    Runtime& r = R();
    std::shared_lock lk(r.alloc_mutex);
    const auto key = reinterpret_cast<uintptr_t>(dims);
    auto it = r.allocs.upper_bound(key);
    if (it == r.allocs.begin()) return true;
    --it;
    const Allocation& a = it->second;
    const size_t off = key - it->first;
    const size_t bytes = size_t(n) * sizeof(int);
    if (a.shadow.empty() || off + bytes > a.bytes) return true;
    for (size_t i = 0; i < bytes; ++i)
        if (!a.known[off + i]) return true;
    if (std::memcmp(a.shadow.data() + off, want, bytes) != 0) {
        setDetail("dims disagree with the sizes in the arguments");
        return false;
    }
    return true;
}

void* streamScratch(void* stream, size_t bytes) {
    Runtime& r = R();
    const auto s = static_cast<hipStream_t>(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) return nullptr;
    const bool capturing = cs != hipStreamCaptureStatusNone;
    std::lock_guard lk(r.scratch_mutex);
    Runtime::Scratch& sc = r.scratch[s];
    if (sc.p && sc.bytes >= bytes) {
        sc.in_graph |= capturing;
        return sc.p;
    }
    if (capturing) return nullptr;  // no allocation inside a capture
    if (hipStreamSynchronize(s) != hipSuccess) return nullptr;
    const size_t want = std::max(bytes, 2 * sc.bytes);
    if (sc.p) {
        if (sc.in_graph) r.retired_scratch.push_back(sc.p);
        else (void)hipFree(sc.p);
    }
    sc = Runtime::Scratch{};
    if (hipMalloc(&sc.p, want) != hipSuccess) {
        sc = Runtime::Scratch{};
        return nullptr;
    }
    sc.bytes = want;
    return sc.p;
}

int option(const char* name) {
    Runtime& r = R();
    std::lock_guard lk(r.options_mutex);
    auto it = r.options.find(name);
    return it == r.options.end() ? 0 : it->second;
}

unsigned optionsGeneration() { return R().options_gen.load(); }

int fromHip(int hip_status, const char* what) {
    const hipError_t s = static_cast<hipError_t>(hip_status);
    if (s == hipSuccess) return 0;
    if (s == hipErrorNotReady) return KC_ERROR_NOT_READY;
    setDetail("%s: %s", what ? what : "HIP", hipGetErrorString(s));
    if (s == hipErrorOutOfMemory || s == hipErrorMemoryAllocation) return KC_ERROR_OUT_OF_MEMORY;
    if (s == hipErrorInvalidValue) return KC_ERROR_INVALID_VALUE;
    if (s == hipErrorInvalidDevice || s == hipErrorNoDevice) return KC_ERROR_INVALID_DEVICE;
    if (s == hipErrorInvalidResourceHandle || s == hipErrorContextIsDestroyed) return KC_ERROR_INVALID_RESOURCE_HANDLE;
    if (isFault(s)) {
        recordFault(R(), hip_status, what);
        return KC_ERROR_KERNEL_FAULT;
    }
    if (s == hipErrorInvalidDeviceFunction || s == hipErrorNoBinaryForGpu || s == hipErrorInvalidImage)
        return KC_ERROR_INVALID_KERNEL_IMAGE;
    if (s == hipErrorLaunchOutOfResources || s == hipErrorInvalidConfiguration) return KC_ERROR_LAUNCH_FAILURE;
    if (s == hipErrorStreamCaptureUnsupported || s == hipErrorStreamCaptureInvalidated ||
        s == hipErrorStreamCaptureUnjoined || s == hipErrorStreamCaptureImplicit)
        return KC_ERROR_UNSUPPORTED_OPERATION;
    return KC_ERROR_INTERNAL;
}

}  // namespace kcamd

// ================================================================ lifecycle

kcError_t kcInit() noexcept {
    return exclusive("kcInit", [](Runtime& r) {
        if (r.initialized) return ok;
        if (E e = startDevice(r); e != ok) {
            stopDevice(r);
            return e;
        }
        r.initialized = true;
        return ok;
    });
}

kcError_t kcShutdown() noexcept {
    return exclusive("kcShutdown", [](Runtime& r) {
        if (!r.initialized) return ok;
        const size_t leaked = stopDevice(r);
        {
            std::lock_guard lk(r.kernels_mutex);
            r.kernels.clear();
        }
        r.initialized = false;
        if (leaked) kcamd::setDetail("kcShutdown freed %zu allocation(s) still live", leaked);
        return ok;
    });
}

kcError_t kcDeviceReset() noexcept {
    return exclusive("kcDeviceReset", [](Runtime& r) {
        if (E e = stateError(r, Need::Init); e != ok) return e;
        stopDevice(r);
        if (E e = startDevice(r); e != ok) {
            stopDevice(r);
            r.initialized = false;
            return e;
        }
        return ok;
    });
}

// ================================================================ device

kcError_t kcGetDeviceCount(int* count) noexcept {
    return gated<Need::Init>("kcGetDeviceCount", [&](Runtime& r) {
        if (!count) return kc::Error::InvalidValue;
        *count = 1;
        return ok;
    });
}

kcError_t kcGetDeviceProperties(kcDeviceProperties* props, int device) noexcept {
    return gated<Need::Init>("kcGetDeviceProperties", [&](Runtime& r) {
        if (!props) return kc::Error::InvalidValue;
        if (device != 0) {
            kcamd::setDetail("device %d does not exist (only device 0)", device);
            return kc::Error::InvalidDevice;
        }
        hipDeviceProp_t hp{};
        if (int e = kcamd::fromHip(hipGetDeviceProperties(&hp, r.device), "hipGetDeviceProperties")) return err(e);
        kcDeviceProperties p{};
        std::snprintf(p.name, sizeof p.name, "%s (%s)", hp.name[0] ? hp.name : "AMD GPU", hp.gcnArchName);
        p.worker_count = static_cast<unsigned>(hp.multiProcessorCount);
        p.performance_workers = p.worker_count;
        p.total_memory = hp.totalGlobalMem;
        p.is_hardware_gpu = true;
        p.guard_pages = false;
        p.large_pages = false;
        p.kernel_stack_bytes = 0;
        *props = p;
        return ok;
    });
}

kcError_t kcDeviceGetMemoryInfo(size_t* free_bytes, size_t* total_bytes) noexcept {
    return gated<Need::Live>("kcDeviceGetMemoryInfo", [&](Runtime& r) {
        if (!free_bytes || !total_bytes) return kc::Error::InvalidValue;
        size_t f = 0, t = 0;
        if (int e = kcamd::fromHip(hipMemGetInfo(&f, &t), "hipMemGetInfo")) return err(e);
        *free_bytes = f;
        *total_bytes = t;
        return ok;
    });
}

kcError_t kcSetDevice(int device) noexcept {
    return gated<Need::Init>("kcSetDevice", [&](Runtime& r) {
        if (device != 0) {
            kcamd::setDetail("device %d does not exist (only device 0)", device);
            return kc::Error::InvalidDevice;
        }
        return err(kcamd::fromHip(hipSetDevice(r.device), "hipSetDevice"));
    });
}

kcError_t kcGetDevice(int* device) noexcept {
    return gated<Need::Init>("kcGetDevice", [&](Runtime& r) {
        if (!device) return kc::Error::InvalidValue;
        *device = 0;
        return ok;
    });
}

kcError_t kcDeviceSynchronize() noexcept {
    return gated<Need::Init>("kcDeviceSynchronize", [&](Runtime& r) {
        if (E e = rejectDuringCapture(r, "kcDeviceSynchronize"); e != ok) return e;
        if (E e = waitAllIdle(r, "kcDeviceSynchronize"); e != ok) return e;
        return stateError(r, Need::Live);
    });
}

// ================================================================ memory

kcError_t kcMalloc(void** ptr, size_t bytes) noexcept {
    return gated<Need::Live>("kcMalloc", [&](Runtime& r) {
        if (!ptr) {
            kcamd::setDetail("ptr is null");
            return kc::Error::InvalidValue;
        }
        *ptr = nullptr;
        if (bytes == 0) {
            kcamd::setDetail("zero-byte allocations are rejected");
            return kc::Error::InvalidValue;
        }
        void* p = nullptr;
        if (int e = kcamd::fromHip(hipMalloc(&p, bytes), "hipMalloc")) return err(e);
        Allocation a;
        a.bytes = bytes;
        if (bytes <= kShadowMax) {
            a.shadow.assign(bytes, 0);
            a.known.assign(bytes, 0);
        }
        {
            std::unique_lock lk(r.alloc_mutex);
            r.allocs.emplace(reinterpret_cast<uintptr_t>(p), std::move(a));
        }
        *ptr = p;
        return ok;
    });
}

kcError_t kcFree(void* ptr) noexcept {
    return gated<Need::Init>("kcFree", [&](Runtime& r) {
        if (E e = rejectDuringCapture(r, "kcFree"); e != ok) return e;
        if (!ptr) return ok;
        {
            std::shared_lock lk(r.alloc_mutex);
            if (!r.allocs.count(reinterpret_cast<uintptr_t>(ptr))) {
                kcamd::setDetail("pointer %p is not the base of a live allocation", ptr);
                return kc::Error::InvalidPointer;
            }
        }
        (void)waitAllIdle(r, "kcFree");  // a queued kernel may still use this memory
        {
            std::unique_lock lk(r.alloc_mutex);
            r.allocs.erase(reinterpret_cast<uintptr_t>(ptr));
        }
        return err(kcamd::fromHip(hipFree(ptr), "hipFree"));
    });
}

kcError_t kcMemcpy(void* dst, const void* src, size_t bytes, kcCopyKind_t kind) noexcept {
    return gated<Need::Live>("kcMemcpy", [&](Runtime& r) {
        if (E e = rejectDuringCapture(r, "kcMemcpy"); e != ok) return e;
        const int k = static_cast<int>(kind);
        if (k < 0 || k > 3) {
            kcamd::setDetail("invalid CopyKind");
            return kc::Error::InvalidValue;
        }
        if (bytes == 0) return ok;
        if (!dst || !src) {
            kcamd::setDetail("null pointer with non-zero byte count");
            return kc::Error::InvalidValue;
        }
        const bool dev_dst = k == KC_HOST_TO_DEVICE || k == KC_DEVICE_TO_DEVICE;
        const bool dev_src = k == KC_DEVICE_TO_HOST || k == KC_DEVICE_TO_DEVICE;
        if (dev_dst)
            if (int e = kcamd::checkRange(dst, bytes, "dst")) return err(e);
        if (dev_src)
            if (int e = kcamd::checkRange(src, bytes, "src")) return err(e);
        if (E e = waitAllIdle(r, "kcMemcpy"); e != ok) return e;
        if (k == KC_HOST_TO_HOST) {
            std::memmove(dst, src, bytes);
            return ok;
        }
        const hipMemcpyKind hk = k == KC_HOST_TO_DEVICE   ? hipMemcpyHostToDevice
                                 : k == KC_DEVICE_TO_HOST ? hipMemcpyDeviceToHost
                                                          : hipMemcpyDeviceToDevice;
        if (int e = kcamd::fromHip(hipMemcpy(dst, src, bytes, hk), "hipMemcpy")) return err(e);
        if (k == KC_HOST_TO_DEVICE) shadowWrite(r, dst, src, 0, bytes);
        if (k == KC_DEVICE_TO_DEVICE) shadowWrite(r, dst, nullptr, 0, bytes);
        return ok;
    });
}

kcError_t kcMemset(void* dst, int value, size_t bytes) noexcept {
    return gated<Need::Live>("kcMemset", [&](Runtime& r) {
        if (E e = rejectDuringCapture(r, "kcMemset"); e != ok) return e;
        if (bytes == 0) return ok;
        if (int e = kcamd::checkRange(dst, bytes, "dst")) return err(e);
        if (E e = waitAllIdle(r, "kcMemset"); e != ok) return e;
        if (int e = kcamd::fromHip(hipMemset(dst, value, bytes), "hipMemset")) return err(e);
        if (int e = kcamd::fromHip(hipDeviceSynchronize(), "hipMemset")) return err(e);
        shadowWrite(r, dst, reinterpret_cast<const void*>(1), value, bytes);
        return ok;
    });
}

// ================================================================ kernels

kcError_t kcRegisterKernel(const kcKernelEntry* entry) noexcept {
    return gated<Need::Init>("kcRegisterKernel", [&](Runtime& r) {
        if (!entry || !entry->name || !entry->name[0] || !entry->validate || !entry->launch) {
            kcamd::setDetail("entry needs a name, validate and launch");
            return kc::Error::InvalidValue;
        }
        std::lock_guard lk(r.kernels_mutex);
        auto it = r.kernels.find(entry->name);
        if (it != r.kernels.end() && it->second != entry) {
            kcamd::setDetail("a different kernel is already registered as '%s'", entry->name);
            return kc::Error::InvalidValue;
        }
        r.kernels[entry->name] = entry;
        return ok;
    });
}

kcError_t kcLaunchKernel(const char* name, const void* typed_args, kcStream_t stream) noexcept {
    return gated<Need::Live>("kcLaunchKernel", [&](Runtime& r) { return launchCommon(r, name, typed_args, stream, false, 1); });
}

kcError_t kcLaunchKernelChunked(const char* name, const void* typed_args, unsigned workers, int64_t,
                                kcStream_t stream) noexcept {
    return gated<Need::Live>("kcLaunchKernelChunked", [&](Runtime& r) { return launchCommon(r, name, typed_args, stream, true, workers); });
}

kcError_t kcLaunchMatmulNoAlloc(const char* name, const kcMatmulKQ8Args* args, kcStream_t stream) noexcept {
    return gated<Need::Live>("kcLaunchMatmulNoAlloc", [&](Runtime& r) {
        static const struct {
            const char* name;
            bool q6k, per256;
        } names[] = {{"matmul_q4k_q8x4", false, false},  {"matmul_q4k_q8x8", false, false},
                     {"matmul_q6k_q8x4", true, false},   {"matmul_q6k_q8x8", true, false},
                     {"matmul_q4k_q8kx4", false, true},  {"matmul_q4k_q8kx8", false, true},
                     {"matmul_q6k_q8kx4", true, true},   {"matmul_q6k_q8kx8", true, true}};
        int which = -1;
        for (int i = 0; name && i < 8; ++i)
            if (std::strcmp(name, names[i].name) == 0) which = i;
        if (which < 0) {
            kcamd::setDetail("'%s' is not one of the matmul_{q4k,q6k}_q8{,k}x{4,8} names", name ? name : "(null)");
            return kc::Error::InvalidValue;
        }
        if (!args) return kc::Error::InvalidValue;
        const kcKernelEntry* entry = nullptr;
        {
            std::lock_guard lk(r.kernels_mutex);
            auto it = r.kernels.find(name);
            if (it == r.kernels.end()) {
                kcamd::setDetail("no kernel registered as '%s'", name);
                return kc::Error::KernelNotFound;
            }
            entry = it->second;
        }
        kcStream_st* st = nullptr;
        if (E e = findStream(r, stream, &st); e != ok) return e;
        kcLaunchContext ctx{0};
        if (int e = entry->validate(args, &ctx); e != 0) {
            if (!kcamd::hasDetail()) kcamd::setDetail("kernel '%s': argument validation failed", name);
            return err(e);
        }
        std::lock_guard cap(r.capture_mutex);
        if (st->capturing && st->concurrent) {  // a branch would need a side stream created for it
            kcamd::setDetail("kcLaunchMatmulNoAlloc does not run inside a concurrent group");
            return kc::Error::UnsupportedOperation;
        }
        (void)hipGetLastError();
        if (int e = kcamd::launchMatmulKqNoAlloc(names[which].q6k, names[which].per256, *args, st->s); e != 0)
            return err(e);
        if (int e = kcamd::fromHip(hipGetLastError(), name)) return err(e == KC_ERROR_KERNEL_FAULT ? e : KC_ERROR_LAUNCH_FAILURE);
        if (!stream && !st->capturing) return err(kcamd::fromHip(hipStreamSynchronize(st->s), name));
        return ok;
    });
}

kcError_t kcCheckDeviceRange(const kcLaunchContext* ctx, const void* ptr, size_t bytes, const char* what) noexcept {
    return gated<Need::Nothing>("kcCheckDeviceRange", [&](Runtime& r) {
        if (!ctx) return kc::Error::InvalidValue;
        return err(kcamd::checkRange(ptr, bytes, what ? what : "buffer"));
    });
}

// ================================================================ streams and events

kcError_t kcStreamCreate(kcStream_t* stream) noexcept {
    return gated<Need::Live>("kcStreamCreate", [&](Runtime& r) {
        if (!stream) return kc::Error::InvalidValue;
        auto s = std::make_unique<kcStream_st>();
        if (E e = createStream(s.get()); e != ok) return e;
        kcStream_t h = s.get();
        std::lock_guard lk(r.objects_mutex);
        r.streams.emplace(h, std::move(s));
        *stream = h;
        return ok;
    });
}

kcError_t kcStreamDestroy(kcStream_t stream) noexcept {
    return gated<Need::Init>("kcStreamDestroy", [&](Runtime& r) {
        std::unique_ptr<kcStream_st> owned;
        {
            std::lock_guard lk(r.objects_mutex);
            auto it = r.streams.find(stream);
            if (!stream || it == r.streams.end()) {
                kcamd::setDetail("unknown stream handle");
                return kc::Error::InvalidResourceHandle;
            }
            if (it->second->capturing) {
                kcamd::setDetail("the stream is capturing");
                return kc::Error::UnsupportedOperation;
            }
            owned = std::move(it->second);
            r.streams.erase(it);
        }
        destroyStream(owned.get());  // drains first
        return ok;
    });
}

kcError_t kcStreamSynchronize(kcStream_t stream) noexcept {
    return gated<Need::Init>("kcStreamSynchronize", [&](Runtime& r) {
        kcStream_st* s = nullptr;
        if (E e = findStream(r, stream, &s); e != ok) return e;
        if (s->capturing) return rejectDuringCapture(r, "kcStreamSynchronize on a capturing stream");
        if (int e = kcamd::fromHip(hipStreamSynchronize(s->s), "kcStreamSynchronize")) return err(e);
        return stateError(r, Need::Live);
    });
}

kcError_t kcStreamQuery(kcStream_t stream) noexcept {
    return gated<Need::Init>("kcStreamQuery", [&](Runtime& r) {
        kcStream_st* s = nullptr;
        if (E e = findStream(r, stream, &s); e != ok) return e;
        return err(kcamd::fromHip(hipStreamQuery(s->s), "kcStreamQuery"));
    });
}

namespace {
struct HostCall {
    void (*fn)(void*);
    void* user;
};
void hostTrampoline(void* p) {
    std::unique_ptr<HostCall> c(static_cast<HostCall*>(p));
    t_in_host_func = true;
    c->fn(c->user);
    t_in_host_func = false;
}
}  // namespace

kcError_t kcLaunchHostFunc(kcStream_t stream, void (*fn)(void*), void* user) noexcept {
    return gated<Need::Live>("kcLaunchHostFunc", [&](Runtime& r) {
        if (!fn) return kc::Error::InvalidValue;
        kcStream_st* s = nullptr;
        if (E e = findStream(r, stream, &s); e != ok) return e;
        if (s->capturing) return rejectDuringCapture(r, "kcLaunchHostFunc on a capturing stream");
        if (!stream) {  // the default stream is synchronous: drain it, then run on this thread
            if (int e = kcamd::fromHip(hipStreamSynchronize(s->s), "kcLaunchHostFunc")) return err(e);
            t_in_host_func = true;
            fn(user);
            t_in_host_func = false;
            return ok;
        }
        auto* c = new HostCall{fn, user};
        if (int e = kcamd::fromHip(hipLaunchHostFunc(s->s, hostTrampoline, c), "hipLaunchHostFunc")) {
            delete c;
            return err(e);
        }
        return ok;
    });
}

// Called through gated<Need::Live>.
static kcError_t eventCreate(Runtime& r, kcEvent_t* event, bool timed) {
    if (!event) return kc::Error::InvalidValue;
    auto ev = std::make_unique<kcEvent_st>();
    ev->timed = timed;
    if (int e = kcamd::fromHip(hipEventCreateWithFlags(&ev->ev, timed ? hipEventDefault : hipEventDisableTiming),
                               "hipEventCreate"))
        return err(e);
    kcEvent_t h = ev.get();
    std::lock_guard lk(r.objects_mutex);
    r.events.emplace(h, std::move(ev));
    *event = h;
    return ok;
}

kcError_t kcEventCreate(kcEvent_t* event) noexcept {
    return gated<Need::Live>("kcEventCreate", [&](Runtime& r) { return eventCreate(r, event, false); });
}

kcError_t kcEventCreateTimed(kcEvent_t* event) noexcept {
    return gated<Need::Live>("kcEventCreateTimed", [&](Runtime& r) { return eventCreate(r, event, true); });
}

kcError_t kcEventDestroy(kcEvent_t event) noexcept {
    return gated<Need::Init>("kcEventDestroy", [&](Runtime& r) {
        std::unique_ptr<kcEvent_st> owned;
        {
            std::lock_guard lk(r.objects_mutex);
            auto it = r.events.find(event);
            if (!event || it == r.events.end()) {
                kcamd::setDetail("unknown event handle");
                return kc::Error::InvalidResourceHandle;
            }
            owned = std::move(it->second);
            r.events.erase(it);
        }
        (void)hipEventSynchronize(owned->ev);
        return err(kcamd::fromHip(hipEventDestroy(owned->ev), "hipEventDestroy"));
    });
}

kcError_t kcEventRecord(kcEvent_t event, kcStream_t stream) noexcept {
    return gated<Need::Live>("kcEventRecord", [&](Runtime& r) {
        kcEvent_st* ev = nullptr;
        if (E e = findEvent(r, event, &ev); e != ok) return e;
        kcStream_st* s = nullptr;
        if (E e = findStream(r, stream, &s); e != ok) return e;
        if (s->capturing) return rejectDuringCapture(r, "kcEventRecord on a capturing stream");
        return err(kcamd::fromHip(hipEventRecord(ev->ev, s->s), "hipEventRecord"));
    });
}

kcError_t kcEventSynchronize(kcEvent_t event) noexcept {
    return gated<Need::Init>("kcEventSynchronize", [&](Runtime& r) {
        kcEvent_st* ev = nullptr;
        if (E e = findEvent(r, event, &ev); e != ok) return e;
        if (int e = kcamd::fromHip(hipEventSynchronize(ev->ev), "hipEventSynchronize")) return err(e);
        return stateError(r, Need::Live);
    });
}

kcError_t kcEventQuery(kcEvent_t event) noexcept {
    return gated<Need::Init>("kcEventQuery", [&](Runtime& r) {
        kcEvent_st* ev = nullptr;
        if (E e = findEvent(r, event, &ev); e != ok) return e;
        return err(kcamd::fromHip(hipEventQuery(ev->ev), "hipEventQuery"));
    });
}

kcError_t kcEventElapsedTime(float* ms, kcEvent_t start, kcEvent_t end) noexcept {
    return gated<Need::Init>("kcEventElapsedTime", [&](Runtime& r) {
        if (!ms) return kc::Error::InvalidValue;
        kcEvent_st *a = nullptr, *b = nullptr;
        if (E e = findEvent(r, start, &a); e != ok) return e;
        if (E e = findEvent(r, end, &b); e != ok) return e;
        if (!a->timed || !b->timed) {
            kcamd::setDetail("both events must come from kcEventCreateTimed");
            return kc::Error::InvalidValue;
        }
        return err(kcamd::fromHip(hipEventElapsedTime(ms, a->ev, b->ev), "hipEventElapsedTime"));
    });
}

kcError_t kcStreamWaitEvent(kcStream_t stream, kcEvent_t event) noexcept {
    return gated<Need::Live>("kcStreamWaitEvent", [&](Runtime& r) {
        kcEvent_st* ev = nullptr;
        if (E e = findEvent(r, event, &ev); e != ok) return e;
        kcStream_st* s = nullptr;
        if (E e = findStream(r, stream, &s); e != ok) return e;
        if (s->capturing) return rejectDuringCapture(r, "kcStreamWaitEvent on a capturing stream");
        return err(kcamd::fromHip(hipStreamWaitEvent(s->s, ev->ev, 0), "hipStreamWaitEvent"));
    });
}

kcError_t kcStreamGetNative(kcStream_t stream, void** hip_stream) noexcept {
    return gated<Need::Init>("kcStreamGetNative", [&](Runtime& r) {
        if (!hip_stream) return kc::Error::InvalidValue;
        kcStream_st* s = nullptr;
        if (E e = findStream(r, stream, &s); e != ok) return e;
        *hip_stream = s->s;
        return ok;
    });
}

// ================================================================ graphs

kcError_t kcStreamBeginCapture(kcStream_t stream) noexcept {
    return gated<Need::Live>("kcStreamBeginCapture", [&](Runtime& r) {
        kcStream_st* s = nullptr;
        if (E e = findStream(r, stream, &s); e != ok) return e;
        std::lock_guard lk(r.capture_mutex);
        if (s->capturing) {
            kcamd::setDetail("the stream is already capturing");
            return kc::Error::InvalidValue;
        }
        if (int e = kcamd::fromHip(hipStreamBeginCapture(s->s, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture"))
            return err(e);
        s->capturing = true;
        s->concurrent = false;
        r.capture_count.fetch_add(1);
        return ok;
    });
}

kcError_t kcStreamEndCapture(kcStream_t stream, kcGraph_t* graph) noexcept {
    return gated<Need::Init>("kcStreamEndCapture", [&](Runtime& r) {
        if (!graph) return kc::Error::InvalidValue;
        *graph = nullptr;
        kcStream_st* s = nullptr;
        if (E e = findStream(r, stream, &s); e != ok) return e;
        hipGraph_t g = nullptr;
        {
            std::lock_guard lk(r.capture_mutex);
            if (!s->capturing) {
                kcamd::setDetail("the stream is not capturing");
                return kc::Error::InvalidValue;
            }
            if (s->concurrent) {  // close the group so every branch joins the capture
                for (size_t i = 0; i < s->side_used; ++i) (void)hipStreamWaitEvent(s->s, s->side_done[i], 0);
                s->concurrent = false;
                s->side_used = 0;
            }
            const hipError_t st = hipStreamEndCapture(s->s, &g);
            s->capturing = false;
            r.capture_count.fetch_sub(1);
            if (int e = kcamd::fromHip(st, "hipStreamEndCapture")) return err(e);
        }
        auto out = std::make_unique<kcGraph_st>();
        out->graph = g;
        if (int e = kcamd::fromHip(hipGraphInstantiate(&out->exec, g, nullptr, nullptr, 0), "hipGraphInstantiate")) {
            (void)hipGraphDestroy(g);
            return err(e);
        }
        kcGraph_t h = out.get();
        std::lock_guard lk(r.objects_mutex);
        r.graphs.emplace(h, std::move(out));
        *graph = h;
        return ok;
    });
}

kcError_t kcGraphLaunch(kcGraph_t graph, kcStream_t stream) noexcept {
    return gated<Need::Live>("kcGraphLaunch", [&](Runtime& r) {
        hipGraphExec_t exec = nullptr;
        {
            std::lock_guard lk(r.objects_mutex);
            auto it = r.graphs.find(graph);
            if (!graph || it == r.graphs.end()) {
                kcamd::setDetail("unknown graph handle");
                return kc::Error::InvalidResourceHandle;
            }
            exec = it->second->exec;
        }
        kcStream_st* s = nullptr;
        if (E e = findStream(r, stream, &s); e != ok) return e;
        if (s->capturing) {
            kcamd::setDetail("kcGraphLaunch on a capturing stream");
            return kc::Error::UnsupportedOperation;
        }
        if (int e = kcamd::fromHip(hipGraphLaunch(exec, s->s), "hipGraphLaunch")) return err(e);
        if (!stream) return err(kcamd::fromHip(hipStreamSynchronize(s->s), "kcGraphLaunch"));
        return ok;
    });
}

kcError_t kcStreamConcurrentBegin(kcStream_t stream) noexcept {
    return gated<Need::Init>("kcStreamConcurrentBegin", [&](Runtime& r) {
        kcStream_st* s = nullptr;
        if (E e = findStream(r, stream, &s); e != ok) return e;
        std::lock_guard lk(r.capture_mutex);
        if (!s->capturing) {
            kcamd::setDetail("the stream is not capturing");
            return kc::Error::InvalidValue;
        }
        if (s->concurrent) {
            kcamd::setDetail("a concurrent group is already open");
            return kc::Error::InvalidValue;
        }
        if (!s->fork)
            if (int e = kcamd::fromHip(hipEventCreateWithFlags(&s->fork, hipEventDisableTiming), "hipEventCreate"))
                return err(e);
        if (int e = kcamd::fromHip(hipEventRecord(s->fork, s->s), "hipEventRecord")) return err(e);
        s->concurrent = true;
        s->side_used = 0;
        return ok;
    });
}

kcError_t kcStreamConcurrentEnd(kcStream_t stream) noexcept {
    return gated<Need::Init>("kcStreamConcurrentEnd", [&](Runtime& r) {
        kcStream_st* s = nullptr;
        if (E e = findStream(r, stream, &s); e != ok) return e;
        std::lock_guard lk(r.capture_mutex);
        if (!s->concurrent) {
            kcamd::setDetail("no concurrent group is open");
            return kc::Error::InvalidValue;
        }
        for (size_t i = 0; i < s->side_used; ++i)
            if (int e = kcamd::fromHip(hipStreamWaitEvent(s->s, s->side_done[i], 0), "hipStreamWaitEvent"))
                return err(e);
        s->concurrent = false;
        s->side_used = 0;
        return ok;
    });
}

kcError_t kcGraphDestroy(kcGraph_t graph) noexcept {
    return gated<Need::Init>("kcGraphDestroy", [&](Runtime& r) {
        std::unique_ptr<kcGraph_st> owned;
        {
            std::lock_guard lk(r.objects_mutex);
            auto it = r.graphs.find(graph);
            if (!graph || it == r.graphs.end()) {
                kcamd::setDetail("unknown graph handle");
                return kc::Error::InvalidResourceHandle;
            }
            owned = std::move(it->second);
            r.graphs.erase(it);
        }
        // hipGraphExecDestroy waits for pending launches of this graph.
        (void)waitAllIdle(r, "kcGraphDestroy");
        if (owned->exec) (void)hipGraphExecDestroy(owned->exec);
        if (owned->graph) (void)hipGraphDestroy(owned->graph);
        return ok;
    });
}

// ================================================================ code generation path

kcError_t kcSetKernelCodegen(kcCodegen_t codegen) noexcept {
    return gated<Need::Nothing>("kcSetKernelCodegen", [&](Runtime& r) {
        const int c = static_cast<int>(codegen);
        if (c < KC_CODEGEN_AUTO || c > KC_CODEGEN_HIP) {
            kcamd::setDetail("codegen must be Auto, Booth, Native, Simd or Hip");
            return kc::Error::InvalidValue;
        }
        if (c != KC_CODEGEN_AUTO && c != KC_CODEGEN_HIP) {
            kcamd::setDetail("the CPU code paths do not exist on this device: every kernel runs as gfx950 code");
            return kc::Error::UnsupportedOperation;
        }
        r.codegen.store(c);
        return ok;
    });
}

kcError_t kcGetKernelCodegen(kcCodegen_t* codegen) noexcept {
    return gated<Need::Nothing>("kcGetKernelCodegen", [&](Runtime& r) {
        if (!codegen) return kc::Error::InvalidValue;
        *codegen = static_cast<kcCodegen_t>(r.codegen.load());
        return ok;
    });
}

kcError_t kcGetKernelCodegenFor(const char* name, kcCodegen_t* used) noexcept {
    return gated<Need::Init>("kcGetKernelCodegenFor", [&](Runtime& r) {
        if (!name || !used) return kc::Error::InvalidValue;
        std::lock_guard lk(r.kernels_mutex);
        if (!r.kernels.count(name)) {
            kcamd::setDetail("no kernel registered as '%s'", name);
            return kc::Error::KernelNotFound;
        }
        *used = static_cast<kcCodegen_t>(KC_CODEGEN_HIP);
        return ok;
    });
}

const char* kcCodegenName(kcCodegen_t codegen) noexcept {
    switch (static_cast<int>(codegen)) {
        case KC_CODEGEN_AUTO: return "auto";
        case KC_CODEGEN_BOOTH: return "booth";
        case KC_CODEGEN_NATIVE: return "native";
        case KC_CODEGEN_SIMD: return "simd";
        case KC_CODEGEN_HIP: return "hip";
        default: return "unknown";
    }
}

// ================================================================ options and diagnostics

kcError_t kcSetKernelOption(const char* option, int value) noexcept {
    return gated<Need::Nothing>("kcSetKernelOption", [&](Runtime& r) {
        static const char* known[] = {"matvec_waves", "matvec_pipe", "matvec_nt", "matmul_path", "decode_path", "attn_path", "prefill_act", "swiglu_pre",
                                      "qkv_tiles", "matmul_waves", "ggml_extra_fusions", "matvec_af", "matmul_ws",
                                      "matmul_split6", "qk_fuse", "addnorm_lds"};
        if (!option) return kc::Error::InvalidValue;
        bool found = false;
        for (const char* k : known) found |= std::strcmp(k, option) == 0;
        if (!found) {
            kcamd::setDetail("unknown kernel option '%s'", option);
            return kc::Error::InvalidValue;
        }
        if (value < 0) return kc::Error::InvalidValue;
        std::lock_guard lk(r.options_mutex);
        r.options[option] = value;
        r.options_gen.fetch_add(1);
        return ok;
    });
}

kcError_t kcGetKernelOption(const char* option, int* value) noexcept {
    return gated<Need::Nothing>("kcGetKernelOption", [&](Runtime& r) {
        if (!option || !value) return kc::Error::InvalidValue;
        *value = kcamd::option(option);
        return ok;
    });
}

kcError_t kcGetLastFault(kcFaultInfo* info) noexcept {
    return gated<Need::Nothing>("kcGetLastFault", [&](Runtime& r) {
        if (!info) return kc::Error::InvalidValue;
        std::lock_guard lk(r.fault_mutex);
        if (!r.has_fault) {
            kcamd::setDetail("no kernel fault recorded");
            return kc::Error::InvalidValue;
        }
        *info = r.last_fault;
        return ok;
    });
}

const char* kcGetErrorString(kcError_t error) noexcept {
    switch (static_cast<int>(error)) {
        case KC_SUCCESS: return "Success";
        case KC_ERROR_NOT_INITIALIZED: return "NotInitialized";
        case KC_ERROR_INVALID_VALUE: return "InvalidValue";
        case KC_ERROR_INVALID_DEVICE: return "InvalidDevice";
        case KC_ERROR_OUT_OF_MEMORY: return "OutOfMemory";
        case KC_ERROR_INVALID_POINTER: return "InvalidPointer";
        case KC_ERROR_INVALID_RESOURCE_HANDLE: return "InvalidResourceHandle";
        case KC_ERROR_UNSUPPORTED_OPERATION: return "UnsupportedOperation";
        case KC_ERROR_INVALID_KERNEL_IMAGE: return "InvalidKernelImage";
        case KC_ERROR_KERNEL_NOT_FOUND: return "KernelNotFound";
        case KC_ERROR_DYNAMIC_CODE_BLOCKED: return "DynamicCodeBlocked";
        case KC_ERROR_LAUNCH_FAILURE: return "LaunchFailure";
        case KC_ERROR_KERNEL_FAULT: return "KernelFault";
        case KC_ERROR_CONTEXT_POISONED: return "ContextPoisoned";
        case KC_ERROR_NOT_READY: return "NotReady";
        case KC_ERROR_INTERNAL: return "InternalError";
        default: return "UnknownError";
    }
}

const char* kcGetLastErrorDetail() noexcept { return t_detail.c_str(); }
