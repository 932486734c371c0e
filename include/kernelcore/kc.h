/*
 * kc.h -- C ABI of the Kernelcore runtime on MI355X (gfx950, HIP).
 *
 * One header for C and C++. In C++ the error, copy-kind and codegen types are the reference's
 * enum classes (kc::Error, kc::CopyKind, kc::Codegen, all `int`-sized), and trailing arguments
 * carry the reference's defaults, so C++ code written against the reference's
 * include/kernelcore/api.hpp compiles unchanged against <kernelcore/api.hpp> here. In C the same
 * symbols return `int` codes with the same values. Every entry point has C linkage, takes plain
 * pointers and sizes, and never throws.
 *
 * Device memory is HBM on the current GPU (hipMalloc); "kc memory is host memory" no longer
 * holds, so host code must move data with kcMemcpy. Each function names the reference
 * declaration it replaces (include/kernelcore/api.hpp:LINE in arasheedu/Kernelcore).
 */
#ifndef KERNELCORE_KC_H
#define KERNELCORE_KC_H

#include <stddef.h>
#include <stdint.h>
#ifndef __cplusplus
#include <stdbool.h>
#endif

#if defined(__cplusplus)
#define KC_EXTERN_C extern "C"
#define KC_NOEXCEPT noexcept
#define KC_DEF(v) = v
#else
#define KC_EXTERN_C
#define KC_NOEXCEPT
#define KC_DEF(v)
#endif
#define KC_API KC_EXTERN_C __attribute__((visibility("default")))

/* ---- error codes: values of include/kernelcore/error.hpp:8-25 (append only) ---------------- */
#define KC_SUCCESS 0
#define KC_ERROR_NOT_INITIALIZED 1
#define KC_ERROR_INVALID_VALUE 2
#define KC_ERROR_INVALID_DEVICE 3
#define KC_ERROR_OUT_OF_MEMORY 4
#define KC_ERROR_INVALID_POINTER 5
#define KC_ERROR_INVALID_RESOURCE_HANDLE 6
#define KC_ERROR_UNSUPPORTED_OPERATION 7
#define KC_ERROR_INVALID_KERNEL_IMAGE 8
#define KC_ERROR_KERNEL_NOT_FOUND 9
#define KC_ERROR_DYNAMIC_CODE_BLOCKED 10
#define KC_ERROR_LAUNCH_FAILURE 11
#define KC_ERROR_KERNEL_FAULT 12
#define KC_ERROR_CONTEXT_POISONED 13
#define KC_ERROR_NOT_READY 14
#define KC_ERROR_INTERNAL 15

/* copy kinds (include/kernelcore/types.hpp:8) */
#define KC_HOST_TO_DEVICE 0
#define KC_DEVICE_TO_HOST 1
#define KC_DEVICE_TO_DEVICE 2
#define KC_HOST_TO_HOST 3

/* code paths (include/kernelcore/types.hpp:17). The CPU paths (1-3) do not exist on this device;
 * KC_CODEGEN_HIP is appended: every kernel runs as gfx950 code. */
#define KC_CODEGEN_AUTO 0
#define KC_CODEGEN_BOOTH 1
#define KC_CODEGEN_NATIVE 2
#define KC_CODEGEN_SIMD 3
#define KC_CODEGEN_HIP 4

#ifdef __cplusplus
namespace kc {
enum class Error : int {
    Success = 0,
    NotInitialized,
    InvalidValue,
    InvalidDevice,
    OutOfMemory,
    InvalidPointer,
    InvalidResourceHandle,
    UnsupportedOperation,
    InvalidKernelImage,
    KernelNotFound,
    DynamicCodeBlocked,
    LaunchFailure,
    KernelFault,
    ContextPoisoned,
    NotReady,
    InternalError
};
enum class CopyKind : int { HostToDevice = 0, DeviceToHost = 1, DeviceToDevice = 2, HostToHost = 3 };
enum class Codegen : int { Auto = 0, Booth = 1, Native = 2, Simd = 3, Hip = 4 };
}  // namespace kc
typedef kc::Error kcError_t;
typedef kc::CopyKind kcCopyKind_t;
typedef kc::Codegen kcCodegen_t;
#else
typedef int kcError_t;
typedef int kcCopyKind_t;
typedef int kcCodegen_t;
#endif

/* include/kernelcore/types.hpp:19-30. On MI355X: the GPU's name, compute units as workers,
 * HBM bytes as total_memory, is_hardware_gpu = true. */
typedef struct kcDeviceProperties {
    char name[128];
    unsigned worker_count;
    unsigned performance_workers;
    size_t total_memory;
    bool is_hardware_gpu;
    bool guard_pages;
    bool large_pages;
    size_t kernel_stack_bytes;
} kcDeviceProperties;

/* include/kernelcore/error.hpp:28-36. Filled from the HIP error when a kernel faults. */
typedef struct kcFaultInfo {
    uint32_t code;
    uint64_t fault_address;
    uint32_t access_type;
    uint64_t instruction;
    bool in_kernel_image;
    uint64_t code_offset;
    char kernel[64];
} kcFaultInfo;

#ifdef __cplusplus
namespace kc {
typedef ::kcDeviceProperties DeviceProperties;
typedef ::kcFaultInfo FaultInfo;
}  // namespace kc
#endif

typedef struct kcStream_st* kcStream_t; /* NULL = the default stream (synchronous launches) */
typedef struct kcEvent_st* kcEvent_t;
typedef struct kcGraph_st* kcGraph_t;

/* ---- kernel registration ------------------------------------------------------------------------
 * Replaces kc::KernelEntry / LaunchContext (include/kernelcore/kernel_registry.hpp:24-56): the
 * System V register image of the CPU executor becomes a validate step plus a HIP launch.
 *   validate(typed_args, ctx): check every buffer with kcCheckDeviceRange; return a kc error code.
 *   launch(typed_args, hip_stream): enqueue the kernel(s) on the hipStream_t; return a kc code.
 *   chunkable: non-zero if kcLaunchKernelChunked may be used (one grid either way on the GPU). */
typedef struct kcLaunchContext kcLaunchContext;
typedef struct kcKernelEntry {
    const char* name;
    int (*validate)(const void* typed_args, const kcLaunchContext* ctx);
    int (*launch)(const void* typed_args, void* hip_stream);
    int chunkable;
} kcKernelEntry;
#ifdef __cplusplus
namespace kc {
typedef ::kcKernelEntry KernelEntry;
typedef ::kcLaunchContext LaunchContext;
}  // namespace kc
#endif

/* ---- lifecycle (api.hpp:15-17) ---------------------------------------------------------------- */
KC_API kcError_t kcInit(void) KC_NOEXCEPT;
KC_API kcError_t kcShutdown(void) KC_NOEXCEPT;
KC_API kcError_t kcDeviceReset(void) KC_NOEXCEPT;

/* ---- device (api.hpp:20-24). One device: the GPU this process runs on. -------------------------- */
KC_API kcError_t kcGetDeviceCount(int* count) KC_NOEXCEPT;
KC_API kcError_t kcGetDeviceProperties(kcDeviceProperties* props, int device) KC_NOEXCEPT;
KC_API kcError_t kcSetDevice(int device) KC_NOEXCEPT;
KC_API kcError_t kcGetDevice(int* device) KC_NOEXCEPT;
KC_API kcError_t kcDeviceSynchronize(void) KC_NOEXCEPT;

/* ---- memory (api.hpp:27-30) --------------------------------------------------------------------- */
KC_API kcError_t kcMalloc(void** ptr, size_t bytes) KC_NOEXCEPT;
KC_API kcError_t kcFree(void* ptr) KC_NOEXCEPT;
KC_API kcError_t kcMemcpy(void* dst, const void* src, size_t bytes, kcCopyKind_t kind) KC_NOEXCEPT;
KC_API kcError_t kcMemset(void* dst, int value, size_t bytes) KC_NOEXCEPT;

/* ---- kernels (api.hpp:33-39) -------------------------------------------------------------------- */
KC_API kcError_t kcRegisterKernel(const kcKernelEntry* entry) KC_NOEXCEPT;
KC_API kcError_t kcLaunchKernel(const char* name, const void* typed_args, kcStream_t stream KC_DEF(nullptr)) KC_NOEXCEPT;
/* workers / min_chunk are validated as in the reference ([1, 1024]) and otherwise ignored: the
 * launch is one grid over the whole GPU. */
KC_API kcError_t kcLaunchKernelChunked(const char* name, const void* typed_args, unsigned workers,
                                       int64_t min_chunk KC_DEF(4096), kcStream_t stream KC_DEF(nullptr)) KC_NOEXCEPT;
/* Range check for kcKernelEntry::validate (LaunchContext::checkDeviceRange, kernel_registry.hpp:27-31). */
KC_API kcError_t kcCheckDeviceRange(const kcLaunchContext* ctx, const void* ptr, size_t bytes,
                                    const char* what) KC_NOEXCEPT;

/* ---- streams and events (api.hpp:42-53) ----------------------------------------------------------- */
KC_API kcError_t kcStreamCreate(kcStream_t* stream) KC_NOEXCEPT;
KC_API kcError_t kcStreamDestroy(kcStream_t stream) KC_NOEXCEPT;
KC_API kcError_t kcStreamSynchronize(kcStream_t stream) KC_NOEXCEPT;
KC_API kcError_t kcStreamQuery(kcStream_t stream) KC_NOEXCEPT;
KC_API kcError_t kcLaunchHostFunc(kcStream_t stream, void (*fn)(void*), void* user) KC_NOEXCEPT;
KC_API kcError_t kcEventCreate(kcEvent_t* event) KC_NOEXCEPT;
KC_API kcError_t kcEventDestroy(kcEvent_t event) KC_NOEXCEPT;
KC_API kcError_t kcEventRecord(kcEvent_t event, kcStream_t stream KC_DEF(nullptr)) KC_NOEXCEPT;
KC_API kcError_t kcEventSynchronize(kcEvent_t event) KC_NOEXCEPT;
KC_API kcError_t kcEventQuery(kcEvent_t event) KC_NOEXCEPT;
/* Implemented here (hipStreamWaitEvent); the reference returns UnsupportedOperation (api.hpp:53). */
KC_API kcError_t kcStreamWaitEvent(kcStream_t stream, kcEvent_t event) KC_NOEXCEPT;

/* ---- graphs (api.hpp:56-72): capture is hipStreamBeginCapture; a concurrent group forks the
 * captured launches onto side streams and joins them, so they become parallel graph branches. -- */
KC_API kcError_t kcStreamBeginCapture(kcStream_t stream) KC_NOEXCEPT;
KC_API kcError_t kcStreamEndCapture(kcStream_t stream, kcGraph_t* graph) KC_NOEXCEPT;
KC_API kcError_t kcGraphLaunch(kcGraph_t graph, kcStream_t stream KC_DEF(nullptr)) KC_NOEXCEPT;
KC_API kcError_t kcStreamConcurrentBegin(kcStream_t stream KC_DEF(nullptr)) KC_NOEXCEPT;
KC_API kcError_t kcStreamConcurrentEnd(kcStream_t stream KC_DEF(nullptr)) KC_NOEXCEPT;
KC_API kcError_t kcGraphDestroy(kcGraph_t graph) KC_NOEXCEPT;

/* ---- code generation path (api.hpp:75-80) ------------------------------------------------------ */
KC_API kcError_t kcSetKernelCodegen(kcCodegen_t codegen) KC_NOEXCEPT;
KC_API kcError_t kcGetKernelCodegen(kcCodegen_t* codegen) KC_NOEXCEPT;
KC_API kcError_t kcGetKernelCodegenFor(const char* name, kcCodegen_t* used) KC_NOEXCEPT;
KC_API const char* kcCodegenName(kcCodegen_t codegen) KC_NOEXCEPT;

/* ---- diagnostics (api.hpp:83-88) ----------------------------------------------------------------- */
KC_API kcError_t kcGetLastFault(kcFaultInfo* info) KC_NOEXCEPT;
KC_API const char* kcGetErrorString(kcError_t error) KC_NOEXCEPT;
KC_API const char* kcGetLastErrorDetail(void) KC_NOEXCEPT;

/* ---- additions of this device (no reference counterpart) --------------------------------------- */
/* The hipStream_t behind a kc stream (NULL = the default stream), for interop and timing. */
KC_API kcError_t kcStreamGetNative(kcStream_t stream, void** hip_stream) KC_NOEXCEPT;
/* Timed events (the reference's events have no timer): milliseconds between two recorded events. */
KC_API kcError_t kcEventCreateTimed(kcEvent_t* event) KC_NOEXCEPT;
KC_API kcError_t kcEventElapsedTime(float* ms, kcEvent_t start, kcEvent_t end) KC_NOEXCEPT;
/* Launch-shape options of the built-in kernels (name = value), e.g. "matvec_waves" = 1 makes the
 * K-quant matvecs accumulate each row in one lane in the reference's order. 0 restores the
 * default. Unknown names: InvalidValue. */
KC_API kcError_t kcSetKernelOption(const char* option, int value) KC_NOEXCEPT;
KC_API kcError_t kcGetKernelOption(const char* option, int* value) KC_NOEXCEPT;
/* Free and total HBM bytes of the device (hipMemGetInfo): what the ggml backend's get_memory
 * reports (the reference's dev_get_memory returns 0 / 0, ggml-kernelcore.cpp:823-826). */
KC_API kcError_t kcDeviceGetMemoryInfo(size_t* free_bytes, size_t* total_bytes) KC_NOEXCEPT;

#endif /* KERNELCORE_KC_H */
