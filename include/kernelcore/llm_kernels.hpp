// llm_kernels.hpp -- typed kernel arguments in namespace llm (reference llm/llm_kernels.hpp).
#pragma once

#include <kernelcore/api.hpp>
