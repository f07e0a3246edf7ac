// Self-check of the device's bf16 rounding: the conversion instruction the
// kernels use (vtx::f32_to_bf16) against the integer round-to-nearest-even
// formulation (vtx::f32_to_bf16_rne_int), over every fp32 bit pattern.
#include "vtx_device.h"
#include "vtx_host.h"

namespace {

__global__ __launch_bounds__(256) void bf16_rounding_check_kernel(unsigned long long* counts) {
  const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t nthreads = (uint64_t)gridDim.x * blockDim.x;
  unsigned long long bad = 0, nan_bad = 0;
  for (uint64_t v = tid; v < (1ull << 32); v += nthreads) {
    const float f = __uint_as_float((uint32_t)v);
    const uint32_t hw = vtx::f32_to_bf16(f);
    const uint32_t ref = vtx::f32_to_bf16_rne_int(f);
    const float r = vtx::bf16r(f);
    if (f != f) {
      nan_bad += (hw != 0x7fc0u) + (r == r);
    } else {
      bad += (hw != ref) + (__float_as_uint(r) != (ref << 16));
    }
  }
  if (bad) atomicAdd(&counts[0], bad);
  if (nan_bad) atomicAdd(&counts[1], nan_bad);
}

}  // namespace

extern "C" int vtx_bf16_rounding_check(unsigned long long* counts, void* stream) {
  vtx::clear_error();
  if (!counts) return vtx::fail(VTX_E_INVALID, "bf16_rounding_check: null counts");
  bf16_rounding_check_kernel<<<4096, 256, 0, vtx::as_stream(stream)>>>(counts);
  return vtx::check_launch("bf16_rounding_check");
}
