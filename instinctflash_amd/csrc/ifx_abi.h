// Internal glue shared by the .hip translation units: status codes and launch
// checks. The public declarations live in include/ifx_fp8.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ifx_fp8.h"

namespace ifx {

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? IFX_OK : static_cast<int>(e);
}

}  // namespace ifx
