// Host-side helpers shared by the extern "C" entry points of libllmy.
//
// Every entry point validates its arguments before it launches anything and
// returns hipErrorInvalidValue on a bad argument (the convention of the
// reference op hooks, llmy_cuda/src/llmy.cpp:216-217,230-233); otherwise it
// returns the launch status (hipGetLastError, which also clears it).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "llmy.h"  // definitions below must match the exported declarations

#define LLMY_REQUIRE(cond)                                              \
  do {                                                                  \
    if (!(cond)) return static_cast<int32_t>(hipErrorInvalidValue);     \
  } while (0)

namespace llmy {

inline bool aligned(const void* p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int32_t launch_status() { return static_cast<int32_t>(hipGetLastError()); }

}  // namespace llmy
