// The per-thread "last error" of the C ABI, shared by every translation unit
// that implements part of include/ember_hip.h.
#pragma once

namespace ember::hip {

// Records a printf-style message for ember_hip_last_error(); returns `code`.
int set_error(int code, const char *fmt, ...);

}  // namespace ember::hip
