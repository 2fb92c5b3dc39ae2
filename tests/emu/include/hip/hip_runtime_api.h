// The runtime API types of the HIP stand-in (tests/emu/include/hip/hip_runtime.h).
#pragma once
#include "hip_runtime.h"
