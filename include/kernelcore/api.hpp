// api.hpp -- the reference's C++ runtime header (include/kernelcore/api.hpp in
// arasheedu/Kernelcore), on MI355X. Every function keeps its reference signature
// (kc::Error results, default arguments) and has C linkage; kc.h declares the same symbols for C.
#pragma once

#include <kernelcore/kc.h>
#include <kernelcore/llm_kernels.h>
