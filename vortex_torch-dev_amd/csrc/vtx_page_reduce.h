// Page-finish reduction building blocks shared by the page-reduce kernels
// (page_reduce.hip) and the fused indexer (indexer_fused.hip), which runs a
// layer's decode CMean inside its own launch.  Sharing the code keeps the
// two bit-identical.
#pragma once

#include "vtx_device.h"

namespace vtx {

constexpr int kPageReduceMaxOut = 4;

struct PageReduceArgs {
  const uint16_t* x;
  int64_t x_rows;
  int32_t rows_per_tile;  // R
  int32_t cols;           // C
  void* out[kPageReduceMaxOut];
  int32_t out_dtype[kPageReduceMaxOut];
  int32_t out_type[kPageReduceMaxOut];
  int32_t n_out;
  int64_t out_rows;
  const int64_t* loc;
  int64_t nnz;
  int32_t heads;
  int32_t page;
};

struct Acc {
  float sum, sq, mx, mn;
};

// Statistics a launch needs (bit mask): only these are accumulated and
// folded across lanes.
constexpr int kNeedSum = 1, kNeedMax = 2, kNeedMin = 4, kNeedSq = 8, kNeedAll = 15;

__host__ __device__ constexpr int need_of(int type) {
  return type == VTX_REDUCE_MEAN ? kNeedSum
         : type == VTX_REDUCE_MAX ? kNeedMax
         : type == VTX_REDUCE_MIN ? kNeedMin
                                  : kNeedSq;
}

template <int NEED = kNeedAll>
__device__ __forceinline__ void acc_init(Acc& a) {
  a.sum = 0.f;
  a.sq = 0.f;
  a.mx = -INFINITY;
  a.mn = INFINITY;
}
template <int NEED = kNeedAll>
__device__ __forceinline__ void acc_add(Acc& a, float v) {
  if constexpr ((NEED & kNeedSum) != 0) a.sum += v;
  if constexpr ((NEED & kNeedSq) != 0) a.sq = fmaf(v, v, a.sq);
  if constexpr ((NEED & kNeedMax) != 0) a.mx = fmaxf(a.mx, v);
  if constexpr ((NEED & kNeedMin) != 0) a.mn = fminf(a.mn, v);
}
template <int NEED = kNeedAll>
__device__ __forceinline__ void acc_merge_xor(Acc& a, int d) {
  if constexpr ((NEED & kNeedSum) != 0) a.sum += __shfl_xor(a.sum, d, kWave);
  if constexpr ((NEED & kNeedSq) != 0) a.sq += __shfl_xor(a.sq, d, kWave);
  if constexpr ((NEED & kNeedMax) != 0) a.mx = fmaxf(a.mx, __shfl_xor(a.mx, d, kWave));
  if constexpr ((NEED & kNeedMin) != 0) a.mn = fminf(a.mn, __shfl_xor(a.mn, d, kWave));
}
// Final value of reduction `type` over `count` elements, rounded to bf16 bits.
__device__ __forceinline__ uint32_t acc_value(const Acc& a, int type, int count) {
  float v;
  switch (type) {
    case VTX_REDUCE_MEAN: v = a.sum / (float)count; break;
    case VTX_REDUCE_MAX: v = a.mx; break;
    case VTX_REDUCE_MIN: v = a.mn; break;
    default: v = sqrtf(a.sq); break;
  }
  return f32_to_bf16(v);
}

// Collects the first tile row (page * H) of every page closed by the loc
// entries e0 .. e0 + kColl - 1 (threads below kColl each look at one; every
// thread of the block must call this), in loc order, into first_row; returns
// the page count.  wave_count: LDS scratch of kColl / 64 ints.  Args:
// PageReduceArgs or any struct with the same loc, nnz, page and heads.
template <int kColl, typename Args>
__device__ __forceinline__ int collect_pages(const Args& a, long long e0, long long* first_row, int* wave_count) {
  static_assert(kColl % kWave == 0, "whole waves scan loc");
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const long long e = e0 + threadIdx.x;
  long long pos = 0;
  bool closes = false;
  if ((int)threadIdx.x < kColl && e < a.nnz) {
    pos = a.loc[e];
    closes = (pos + 1) % a.page == 0;
  }
  const uint64_t m = __ballot(closes);
  if (lane == 0 && wave < kColl / kWave) wave_count[wave] = __popcll(m);
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kColl / kWave; ++w) {
    before += (w < wave) ? wave_count[w] : 0;
    total += wave_count[w];
  }
  if (closes) first_row[before + lanes_below(m)] = (pos / a.page) * a.heads;
  __syncthreads();
  return total;
}

// dim-1 statistics of tile `row` ([R, C] bf16, C = 8 * LPR, LPR | 64) for
// the lane's 16-byte column vector cv: lane (grp, cv) accumulates rows grp,
// grp + 64/LPR, ... in order, then the row groups are folded by an xor tree
// (strides LPR .. 32), so every lane of a column ends with the whole tile's
// statistics of its 8 columns.  All 64 lanes of the wave take part.
template <int LPR, int NEED>
__device__ __forceinline__ void tile_stats_vec(const uint16_t* x, long long row, int R, int cols, int grp, int cv,
                                               Acc (&acc)[8]) {
  constexpr int kGroups = kWave / LPR;
  const uint16_t* base = x + row * (long long)R * cols + cv * 8;
#pragma unroll
  for (int e = 0; e < 8; ++e) acc_init<NEED>(acc[e]);
#pragma unroll 4
  for (int r = grp; r < R; r += kGroups) {
    const U4 v = ld16_stream(base + (long long)r * cols);
    acc_add<NEED>(acc[0], bf16_lo(v.x));
    acc_add<NEED>(acc[1], bf16_hi(v.x));
    acc_add<NEED>(acc[2], bf16_lo(v.y));
    acc_add<NEED>(acc[3], bf16_hi(v.y));
    acc_add<NEED>(acc[4], bf16_lo(v.z));
    acc_add<NEED>(acc[5], bf16_hi(v.z));
    acc_add<NEED>(acc[6], bf16_lo(v.w));
    acc_add<NEED>(acc[7], bf16_hi(v.w));
  }
#pragma unroll
  for (int d = LPR; d < kWave; d <<= 1)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc_merge_xor<NEED>(acc[e], d);
}

// Writes every output's value of the lane's 8 columns of tile `row`.
__device__ __forceinline__ void tile_store_vec(const PageReduceArgs& a, long long row, int cv, const Acc (&acc)[8]) {
  const long long elem = row * a.cols + cv * 8;
  const int R = a.rows_per_tile;
#pragma unroll
  for (int o = 0; o < kPageReduceMaxOut; ++o) {
    if (o >= a.n_out) break;
    uint32_t b[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = acc_value(acc[e], a.out_type[o], R);
    if (a.out_dtype[o] == VTX_DTYPE_BF16) {
      st16(reinterpret_cast<uint16_t*>(a.out[o]) + elem,
           U4{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)});
    } else {
      uint32_t* dst = reinterpret_cast<uint32_t*>(a.out[o]) + elem;
      st16(dst, U4{b[0] << 16, b[1] << 16, b[2] << 16, b[3] << 16});
      st16(dst + 4, U4{b[4] << 16, b[5] << 16, b[6] << 16, b[7] << 16});
    }
  }
}

// Whether page-reduce writes tile `row` (the kernels skip rows outside the
// pool or the output).
template <typename Args>
__device__ __forceinline__ bool tile_in_range(const Args& a, long long row) {
  return row >= 0 && row < a.x_rows && row < a.out_rows;
}

}  // namespace vtx
