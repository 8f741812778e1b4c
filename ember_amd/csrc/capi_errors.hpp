// The per-thread "last error" of the C ABI, shared by every translation unit
// that implements part of include/ember_hip.h.
#pragma once

#include <hip/hip_runtime.h>

namespace ember::hip {

// Records a printf-style message for ember_hip_last_error(); returns `code`.
int set_error(int code, const char *fmt, ...);

// EMBER_OK for hipSuccess; otherwise records "what: <hip error string>" and
// returns the hipError_t as a positive code.
int hip_status(hipError_t e, const char *what);

}  // namespace ember::hip
