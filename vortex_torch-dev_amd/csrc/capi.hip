// Error plumbing and device queries shared by all C-ABI entry points.
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "vtx_host.h"

namespace vtx {

namespace {
thread_local std::string g_last_error;
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(VTX_E_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return VTX_OK;
}

int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return -1;
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace vtx

extern "C" const char* vtx_last_error(void) { return vtx::g_last_error.c_str(); }

extern "C" const char* vtx_version(void) { return "vortex-mi355x 0.1.0 (gfx950)"; }

extern "C" int vtx_stream_capture_id(void* stream, unsigned long long* id) {
  vtx::clear_error();
  if (!id) return vtx::fail(VTX_E_INVALID, "vtx_stream_capture_id: id is null");
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long cid = 0;
  hipError_t e = hipStreamGetCaptureInfo((hipStream_t)stream, &status, &cid);
  if (e != hipSuccess)
    return vtx::fail(VTX_E_DEVICE, "vtx_stream_capture_id: %s", hipGetErrorString(e));
  *id = status == hipStreamCaptureStatusActive ? cid + 1 : 0;
  return VTX_OK;
}
