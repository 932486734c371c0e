// types.hpp -- kc::CopyKind, kc::Codegen, kc::DeviceProperties and the opaque handles
// (reference include/kernelcore/types.hpp:8-39).
#pragma once

#include <kernelcore/kc.h>
