// Host-side helpers of the C ABI: per-thread error message, launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>

#include "../../include/vortex_hip.h"

namespace vtx {

// Records a printf-style message as this thread's last error; returns `code`.
int fail(int code, const char* fmt, ...);

// Clears this thread's last error.
void clear_error();

// Checks the launch that was just issued; returns VTX_OK or VTX_E_LAUNCH.
int check_launch(const char* what);

// Compute units of the current device (cached per device).
int device_cu_count();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// log2(d) when d is a power of two, else -1 (the `shift` of vtx::div_c).
inline int log2_exact(int d) { return d > 0 && (d & (d - 1)) == 0 ? __builtin_ctz((unsigned)d) : -1; }

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

}  // namespace vtx
