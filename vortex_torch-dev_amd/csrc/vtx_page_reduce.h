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
  int32_t page_shift;  // log2(page) for a power of two, else -1
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
// acc_add when `in`, else the accumulator unchanged (bit for bit)
template <int NEED = kNeedAll>
__device__ __forceinline__ void acc_add_if(Acc& a, float v, bool in) {
  if constexpr ((NEED & kNeedSum) != 0) a.sum = in ? a.sum + v : a.sum;
  if constexpr ((NEED & kNeedSq) != 0) a.sq = in ? fmaf(v, v, a.sq) : a.sq;
  if constexpr ((NEED & kNeedMax) != 0) a.mx = in ? fmaxf(a.mx, v) : a.mx;
  if constexpr ((NEED & kNeedMin) != 0) a.mn = in ? fminf(a.mn, v) : a.mn;
}
template <int NEED = kNeedAll>
__device__ __forceinline__ void acc_merge_xor(Acc& a, int d) {
  if constexpr ((NEED & kNeedSum) != 0) a.sum += xshfl(a.sum, d);
  if constexpr ((NEED & kNeedSq) != 0) a.sq += xshfl(a.sq, d);
  if constexpr ((NEED & kNeedMax) != 0) a.mx = fmaxf(a.mx, xshfl(a.mx, d));
  if constexpr ((NEED & kNeedMin) != 0) a.mn = fminf(a.mn, xshfl(a.mn, d));
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
// PageReduceArgs or any struct with the same loc, nnz, page, page_shift and
// heads.
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
    closes = divides(pos + 1, a.page, a.page_shift);
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
  if (closes) first_row[before + lanes_below(m)] = div_c(pos, a.page, a.page_shift) * a.heads;
  __syncthreads();
  return total;
}

// dim-1 statistics of tile `row` ([R, C] bf16, C = 8 * LPR, LPR | 64) for
// the lane's 16-byte column vector cv: lane (grp, cv) accumulates rows grp,
// grp + 64/LPR, ... in order, then the row groups are folded by an xor tree
// (strides LPR .. 32), so every lane of a column ends with the whole tile's
// statistics of its 8 columns.  All 64 lanes of the wave take part.
//
// A lane's rows are loaded kBatch at a time, all issued before the first is
// used, so a 16-row tile costs one memory round trip rather than one per row
// (R is a runtime value, and a plain loop over it waits on every load).  Rows
// past R load row R - 1 again and are not accumulated.
template <int LPR, int NEED>
__device__ __forceinline__ void tile_stats_vec(const uint16_t* x, long long row, int R, int cols, int grp, int cv,
                                               Acc (&acc)[8]) {
  constexpr int kGroups = kWave / LPR;
  constexpr int kBatch = 16 / kGroups < 2 ? 2 : (16 / kGroups > 8 ? 8 : 16 / kGroups);  // a 16-row tile per batch
  const uint16_t* base = x + row * (long long)R * cols + cv * 8;
#pragma unroll
  for (int e = 0; e < 8; ++e) acc_init<NEED>(acc[e]);
  for (int r0 = grp; r0 < R; r0 += kBatch * kGroups) {
    U4 v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int r = r0 + u * kGroups;
      v[u] = ld16_stream(base + (long long)(r < R ? r : R - 1) * cols);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      // a select, not a branch: a branch would let the compiler sink each
      // load into it, one round trip per row again
      const bool in = r0 + u * kGroups < R;
      acc_add_if<NEED>(acc[0], bf16_lo(v[u].x), in);
      acc_add_if<NEED>(acc[1], bf16_hi(v[u].x), in);
      acc_add_if<NEED>(acc[2], bf16_lo(v[u].y), in);
      acc_add_if<NEED>(acc[3], bf16_hi(v[u].y), in);
      acc_add_if<NEED>(acc[4], bf16_lo(v[u].z), in);
      acc_add_if<NEED>(acc[5], bf16_hi(v[u].z), in);
      acc_add_if<NEED>(acc[6], bf16_lo(v[u].w), in);
      acc_add_if<NEED>(acc[7], bf16_hi(v[u].w), in);
    }
  }
#pragma unroll
  for (int d = LPR; d < kWave; d <<= 1)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc_merge_xor<NEED>(acc[e], d);
}

// acc = combine(lower, higher): the fold one level of the xor tree in
// tile_stats_vec performs in the lane of the lower row group.
template <int NEED>
__device__ __forceinline__ void acc_fold(const Acc& lower, Acc& higher) {
  if constexpr ((NEED & kNeedSum) != 0) higher.sum = lower.sum + higher.sum;
  if constexpr ((NEED & kNeedSq) != 0) higher.sq = lower.sq + higher.sq;
  if constexpr ((NEED & kNeedMax) != 0) higher.mx = fmaxf(lower.mx, higher.mx);
  if constexpr ((NEED & kNeedMin) != 0) higher.mn = fminf(lower.mn, higher.mn);
}

// Statistics of row groups kG0 .. kG0 + kN - 1 (group g: rows g, g + G,
// g + 2G, ... below R, in order) of the lane's column, folded pairwise in
// the order of tile_stats_vec's xor tree: ((0 + 1) + (2 + 3)) + ...
template <int G, int kG0, int kN, int NEED>
__device__ __forceinline__ void fold_groups(const U4 (&v)[16], int R, Acc (&s)[8]) {
  if constexpr (kN == 1) {
#pragma unroll
    for (int e = 0; e < 8; ++e) acc_init<NEED>(s[e]);
#pragma unroll
    for (int r = kG0; r < 16; r += G) {
      const bool in = r < R;
      acc_add_if<NEED>(s[0], bf16_lo(v[r].x), in);
      acc_add_if<NEED>(s[1], bf16_hi(v[r].x), in);
      acc_add_if<NEED>(s[2], bf16_lo(v[r].y), in);
      acc_add_if<NEED>(s[3], bf16_hi(v[r].y), in);
      acc_add_if<NEED>(s[4], bf16_lo(v[r].z), in);
      acc_add_if<NEED>(s[5], bf16_hi(v[r].z), in);
      acc_add_if<NEED>(s[6], bf16_lo(v[r].w), in);
      acc_add_if<NEED>(s[7], bf16_hi(v[r].w), in);
    }
  } else {
    Acc lower[8];
    fold_groups<G, kG0, kN / 2, NEED>(v, R, lower);
    fold_groups<G, kG0 + kN / 2, kN / 2, NEED>(v, R, s);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc_fold<NEED>(lower[e], s[e]);
  }
}

// Whether tile_stats_lane's registers fit for this width and statistic set
// (16 loaded rows plus one partial per level of the group fold).
template <int LPR, int NEED>
__host__ __device__ constexpr bool lane_tiles_fit() {
  constexpr int G = kWave / LPR;
  constexpr int levels = G == 1 ? 1 : G == 2 ? 2 : G == 4 ? 3 : 4;
  constexpr int stats = ((NEED & 1) != 0) + ((NEED & 2) != 0) + ((NEED & 4) != 0) + ((NEED & 8) != 0);
  return levels * stats <= 8;
}

// tile_stats_vec's result, bit for bit, computed by one lane alone: lane cv
// reads every row (R <= 16) of its 16-byte column vector of tile `row`,
// accumulates the row groups tile_stats_vec spreads over 64 / LPR lanes
// (rows g, g + 64/LPR, ...) one after another and folds them in the xor
// tree's order.  No cross-lane operations, so the 64 / LPR lane groups of a
// wave can each take a different tile, and all 16 rows of a lane are in
// flight at once.  Rows past R load row R - 1 again and are not accumulated.
template <int LPR, int NEED>
__device__ __forceinline__ void tile_stats_lane(const uint16_t* x, long long row, int R, int cols, int cv,
                                                Acc (&acc)[8]) {
  constexpr int G = kWave / LPR;
  const uint16_t* base = x + row * (long long)R * cols + cv * 8;
  U4 v[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) v[r] = ld16_stream(base + (long long)(r < R ? r : R - 1) * cols);
  fold_groups<G, 0, G, NEED>(v, R, acc);
}

// The 8 bf16 values of reduction kType (a compile-time constant, so no
// per-element switch) packed into one 16-byte vector.
template <int kType>
__device__ __forceinline__ U4 pack_type(const Acc (&acc)[8], int count) {
  uint32_t b[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) b[e] = acc_value(acc[e], kType, count);
  return U4{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
}

// Writes every output's value of the lane's 8 columns of tile `row` (one
// branch on the output's type, not one per element).
__device__ __forceinline__ void tile_store_vec(const PageReduceArgs& a, long long row, int cv, const Acc (&acc)[8]) {
  const long long elem = row * a.cols + cv * 8;
  const int R = a.rows_per_tile;
#pragma unroll
  for (int o = 0; o < kPageReduceMaxOut; ++o) {
    if (o >= a.n_out) break;
    U4 p;
    switch (a.out_type[o]) {
      case VTX_REDUCE_MEAN: p = pack_type<VTX_REDUCE_MEAN>(acc, R); break;
      case VTX_REDUCE_MAX: p = pack_type<VTX_REDUCE_MAX>(acc, R); break;
      case VTX_REDUCE_MIN: p = pack_type<VTX_REDUCE_MIN>(acc, R); break;
      default: p = pack_type<VTX_REDUCE_L2NORM>(acc, R); break;
    }
    if (a.out_dtype[o] == VTX_DTYPE_BF16) {
      st16(reinterpret_cast<uint16_t*>(a.out[o]) + elem, p);
    } else {
      uint32_t* dst = reinterpret_cast<uint32_t*>(a.out[o]) + elem;
      st16(dst, U4{p.x << 16, p.x & 0xffff0000u, p.y << 16, p.y & 0xffff0000u});
      st16(dst + 4, U4{p.z << 16, p.z & 0xffff0000u, p.w << 16, p.w & 0xffff0000u});
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
