// Device-side helpers shared by the gfx950 kernels: bf16 bit conversions,
// order-preserving score keys, wave64 reductions/scans, error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vortex_hip.h"

namespace vtx {

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 bits
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
// Low / high bf16 of a packed 32-bit word, widened to fp32 (exact).
__device__ __forceinline__ float bf16_lo(uint32_t w) {
  return __uint_as_float(w << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t w) {
  return __uint_as_float(w & 0xffff0000u);
}

// fp32 -> bf16 with round-to-nearest-even, by gfx950's conversion
// instruction (v_cvt_pk_bf16_f32).  For every non-NaN input it gives the bits
// of the integer formulation (add 0x7fff plus the lowest kept bit, truncate)
// — vtx_bf16_rounding_check compares the two over all 2^32 inputs.  Every
// NaN becomes the quiet NaN 0x7fc0, as in torch's conversion.
__device__ __forceinline__ uint32_t f32_to_bf16_rne_int(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  if (__builtin_isnan(f)) return 0x7fc0u;
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

// f rounded to the nearest bf16 (ties to even), as an fp32 value; a NaN
// stays a NaN (its payload is not specified).
__device__ __forceinline__ float bf16r(float f) { return (float)(__bf16)f; }

// Maps a bf16 bit pattern to a 16-bit unsigned key whose unsigned order is
// the numeric order of the scores; -0.0 and +0.0 map to the same key.
__device__ __forceinline__ uint32_t score_key(uint32_t bits16) {
  bits16 &= 0xffffu;
  if (bits16 == 0x8000u) bits16 = 0u;
  return (bits16 & 0x8000u) ? (~bits16 & 0xffffu) : (bits16 | 0x8000u);
}

// ------------------------------------------------------------ wave helpers
__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Number of set bits of `mask` in lanes strictly below this lane.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Treat a value as wave-uniform (moves it to a scalar register).
__device__ __forceinline__ int uniform(int v) {
  return __builtin_amdgcn_readfirstlane(v);
}

// v of lane (lane ^ d).  For d = 1, 2, 4, 8, 16 or 32 known at compile time
// (after unrolling) this is VALU only: DPP row operations for d <= 8 (quad
// permutes, the two 4-lane row shifts and a select, an 8-lane row rotate)
// and gfx950's permlane swaps between 16-lane rows and 32-lane halves, about
// a third of the dependent latency of the LDS permute behind __shfl_xor
// (measured: 24 against 71 cycles per shuffle-and-add step); any other d
// falls back to __shfl_xor.  Every lane of the wave must be active.
__device__ __forceinline__ uint32_t xshfl_u32(uint32_t v, int d) {
  if (__builtin_constant_p(d)) {
    const int lane = lane_id();
    switch (d) {
      case 1: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
      case 2: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
      case 4: {
        const int up = __builtin_amdgcn_update_dpp(0, (int)v, 0x104, 0xF, 0xF, false);  // row_shl:4 (lane + 4)
        const int dn = __builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);  // row_shr:4 (lane - 4)
        return (uint32_t)((lane & 4) ? dn : up);
      }
      case 8: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);  // row_ror:8
      case 16: {
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16) ? p[0] : p[1];
      }
      case 32: {
        const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane & 32) ? p[0] : p[1];
      }
      default: break;
    }
  }
  return (uint32_t)__shfl_xor((int)v, d, kWave);
}
__device__ __forceinline__ float xshfl(float v, int d) {
  return __uint_as_float(xshfl_u32(__float_as_uint(v), d));
}
__device__ __forceinline__ uint32_t xshfl(uint32_t v, int d) { return xshfl_u32(v, d); }
__device__ __forceinline__ int xshfl(int v, int d) { return (int)xshfl_u32((uint32_t)v, d); }
__device__ __forceinline__ long long xshfl(long long v, int d) {
  const uint64_t u = (uint64_t)v;
  return (long long)(((uint64_t)xshfl_u32((uint32_t)(u >> 32), d) << 32) | xshfl_u32((uint32_t)u, d));
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += xshfl(v, d);
  return v;
}

// Inclusive prefix sum over the 64 lanes (lane l gets the sum over lanes
// <= l) with DPP: shifts by 1, 2, 4, 8 inside each 16-lane row, then the
// last lane of row 0 / row 2 is added to rows 1 / 3 and the last lane of
// row 1 to rows 2 and 3.  Lanes whose DPP source is outside the row or
// masked off add 0.  No LDS traffic, unlike lane shuffles.
__device__ __forceinline__ uint32_t wave_prefix_sum(uint32_t v) {
  int x = (int)v;
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
  return (uint32_t)x;
}

// C semantics of x / d and of (x % d == 0) for a positive divisor d, given
// shift = log2(d) when d is a power of two (else -1): shifts and masks then
// (the quotient truncated toward zero for negative x, as C truncates), the
// 64-bit division otherwise, which costs a long instruction sequence.
__device__ __forceinline__ long long div_c(long long x, int d, int shift) {
  if (shift >= 0) return x >= 0 ? (x >> shift) : -((-x) >> shift);
  return x / d;
}
__device__ __forceinline__ bool divides(long long x, int d, int shift) {
  if (shift >= 0) return (x & ((1LL << shift) - 1)) == 0;
  return x % d == 0;
}

// Value of v in lane `src` (src wave-uniform), read through a scalar register.
__device__ __forceinline__ uint32_t lane_value(uint32_t v, int src) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, src);
}

// 16-byte vector load/store of raw words.
struct alignas(16) U4 {
  uint32_t x, y, z, w;
};
__device__ __forceinline__ U4 ld16(const void* p) {
  return *reinterpret_cast<const U4*>(p);
}
// Streaming 16-byte load for data read once per launch (centroid rows, K
// tiles): the nontemporal hint keeps it from displacing reusable lines and
// measured 15-25 % faster than a plain load for random 256-byte row gathers.
__device__ __forceinline__ U4 ld16_stream(const void* p) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
  return U4{t.x, t.y, t.z, t.w};
}
__device__ __forceinline__ void st16(void* p, const U4& v) {
  *reinterpret_cast<U4*>(p) = v;
}

// Widens 8 packed bf16 values to fp32.
__device__ __forceinline__ void unpack8(const U4& t, float* f) {
  f[0] = bf16_lo(t.x);
  f[1] = bf16_hi(t.x);
  f[2] = bf16_lo(t.y);
  f[3] = bf16_hi(t.y);
  f[4] = bf16_lo(t.z);
  f[5] = bf16_hi(t.z);
  f[6] = bf16_lo(t.w);
  f[7] = bf16_hi(t.w);
}

// Two bf16 products added to an fp32 sum by gfx950's v_dot2c_f32_bf16:
// c + lo(a) * lo(b) + hi(a) * hi(b), a and b each two packed bf16 values.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// The bf16 bits of two fp32 values that are bf16 values (exact).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}

// This lane's share of a row dot product: VPL vectors of 8 bf16 against the
// fp32 query slice, whose values are bf16 values (the callers' queries are
// bf16 rows or bf16-rounded means), as a chain of four two-product steps
// (dot2_bf16) per vector in column order.  Every scoring kernel uses it, so
// their scores agree bit for bit.
template <int VPL>
__device__ __forceinline__ float dot_row(const U4 (&w)[VPL], const float (&xs)[VPL][8]) {
  float s = 0.f;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    s = dot2_bf16(w[v].x, pack_bf16x2(xs[v][0], xs[v][1]), s);
    s = dot2_bf16(w[v].y, pack_bf16x2(xs[v][2], xs[v][3]), s);
    s = dot2_bf16(w[v].z, pack_bf16x2(xs[v][4], xs[v][5]), s);
    s = dot2_bf16(w[v].w, pack_bf16x2(xs[v][6], xs[v][7]), s);
  }
  return s;
}

// The query slice xs (bf16 values) as the packed bf16 pairs dot_row feeds
// its steps (exact).
template <int VPL>
__device__ __forceinline__ void pack_query(const float (&xs)[VPL][8], U4 (&xq)[VPL]) {
#pragma unroll
  for (int v = 0; v < VPL; ++v)
    xq[v] = U4{pack_bf16x2(xs[v][0], xs[v][1]), pack_bf16x2(xs[v][2], xs[v][3]), pack_bf16x2(xs[v][4], xs[v][5]),
               pack_bf16x2(xs[v][6], xs[v][7])};
}

// dot_row with the query slice as packed bf16 pairs (xq[v] holds the bits
// pack_bf16x2 makes of xs[v]): the same steps, the same bits.
template <int VPL>
__device__ __forceinline__ float dot_row_packed(const U4 (&w)[VPL], const U4 (&xq)[VPL]) {
  float s = 0.f;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    s = dot2_bf16(w[v].x, xq[v].x, s);
    s = dot2_bf16(w[v].y, xq[v].y, s);
    s = dot2_bf16(w[v].z, xq[v].z, s);
    s = dot2_bf16(w[v].w, xq[v].w, s);
  }
  return s;
}

}  // namespace vtx
