// internal.hpp -- shared between the runtime (runtime.cpp) and the built-in kernel table
// (llm_kernels.cpp). Not installed; the public surface is include/kernelcore/kc.h.
#pragma once

#include <kernelcore/llm_kernels.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <string>

namespace kcamd {

// Thread-local detail text of the current API call (kcGetLastErrorDetail).
void setDetail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
bool hasDetail();

// Looks up [ptr, ptr + bytes) in the live allocations (reference: AllocationRegistry::checkRange,
// src/allocation_registry.cpp:37-60). bytes == 0 always succeeds.
int checkRange(const void* ptr, size_t bytes, const char* what);

// If the runtime holds a host copy of the `n` ints at `dims` (written with kcMemcpy/kcMemset),
// compares them with `want`: returns false on a mismatch, true when they agree or no copy is held.
bool dimsAgree(const int* dims, const int* want, int n);

// Device scratch for a launch on HIP stream `stream` of at least `bytes`: the runtime's own memory
// (not a kcMalloc allocation), one buffer per stream, reused by every launch on it. Returns nullptr
// when the buffer would have to grow while the stream is capturing (or HIP fails): the caller then
// takes a path without scratch. Freed by kcStreamDestroy, kcShutdown and kcDeviceReset; a buffer
// that a capture may have recorded is kept until kcShutdown / kcDeviceReset.
void* streamScratch(void* stream, size_t bytes);

// Launch options (kcSetKernelOption).
int option(const char* name);
// The current device's compute units (cached per device).
int cuCount();
// Changes with every kcSetKernelOption call: work recorded under other options (a kept graph) is stale.
unsigned optionsGeneration();

// The built-in kernels, registered by kcInit.
const kcKernelEntry* builtinKernels(size_t* count);

// Maps a HIP status to a kc code, recording a fault when the device reports one.
int fromHip(int hip_status, const char* what);

}  // namespace kcamd

struct kcLaunchContext {
    int unused;
};
