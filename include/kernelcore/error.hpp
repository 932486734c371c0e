// error.hpp -- kc::Error and kc::FaultInfo (reference include/kernelcore/error.hpp:8-36).
#pragma once

#include <kernelcore/kc.h>
