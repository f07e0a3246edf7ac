// The row-scoring passes shared by the fused indexer kernels and the paged
// GeMM: kG fp32 query rows against up to kPass gathered bf16 rows (or row
// pairs), one wave, every row load issued before any arithmetic.
#pragma once

#include "vtx_device.h"

namespace vtx {

// Positions per wave pass: 64 when a row is one 16-byte vector per lane,
// else 32.
template <int VPL>
constexpr int segment_pass() {
  return VPL == 1 ? 64 : 32;
}

// One wave pass over `cnt` <= kPass consecutive positions; lane l (< cnt)
// holds the l-th position's row id in my_row, naming row my_row of each of
// the kRows pools ys[] ([y_rows, D] bf16).  A row is split over LPR lanes x
// VPL 16-byte vectors (kRowsPerLoad = 64 / LPR rows per wave-wide load,
// kSlots = kPass / kRowsPerLoad rows per lane); every lane issues its row
// loads before any arithmetic (kBatch slots at a time for wide rows), then
// part(rows, g) gives the lane's fp32 partial of query g over its columns,
// and for each query a reduce-scatter over the LPR lanes leaves each finished
// value on one lane: sc[g] (the partials combined by an xor tree with strides
// LPR/2 .. 1), at position *r of the pass; *r = -1 on lanes that own no
// position.  Rows outside the pools give 0.
template <int LPR, int VPL, int kPass, int kG, int kRows, typename Part>
__device__ __forceinline__ void row_pass(const uint16_t* const (&ys)[kRows], long long y_rows, int D, int my_row,
                                         int cnt, int grp, int col, int* r, float (&sc)[kG], Part part) {
  constexpr int kRowsPerLoad = kWave / LPR;
  constexpr int kSlots = kPass / kRowsPerLoad;
  constexpr int kWide = kRows == 1 ? (VPL <= 2 ? kSlots : 2) : (VPL == 1 ? 8 : (VPL == 2 ? 4 : 1));
  constexpr int kBatch = kSlots < kWide ? kSlots : kWide;  // slots loaded together
  static_assert(kSlots >= 1 && kSlots <= LPR && kSlots * kRowsPerLoad == kPass, "pass geometry");
  static_assert(kSlots % kBatch == 0, "batches must tile the slots");
  int first = __builtin_amdgcn_readlane(my_row, 0);  // (lane 0's row: a scalar read, no LDS permute)
  if (first < 0 || first >= y_rows) first = 0;
  float acc[kG][kSlots];
#pragma unroll
  for (int i0 = 0; i0 < kSlots; i0 += kBatch) {
    U4 buf[kBatch][kRows][VPL];
    bool live[kBatch];
#pragma unroll
    for (int ii = 0; ii < kBatch; ++ii) {
      const int row = __shfl(my_row, (i0 + ii) * kRowsPerLoad + grp, kWave);
      live[ii] = row >= 0 && row < y_rows;
      if ((i0 + ii) * kRowsPerLoad < cnt) {  // wave-uniform: slots past the pass are skipped
        const long long off = (long long)(live[ii] ? row : first) * D;
#pragma unroll
        for (int k = 0; k < kRows; ++k)
#pragma unroll
          for (int v = 0; v < VPL; ++v) buf[ii][k][v] = ld16_stream(ys[k] + off + (v * LPR + col) * 8);
      } else {
#pragma unroll
        for (int k = 0; k < kRows; ++k)
#pragma unroll
          for (int v = 0; v < VPL; ++v) buf[ii][k][v] = U4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int ii = 0; ii < kBatch; ++ii)
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        const float s = part(buf[ii], g);
        acc[g][i0 + ii] = live[ii] ? s : 0.f;
      }
  }
  // Reduce-scatter over the slots (lane keeps slot bits of col from the top),
  // then fold the lanes that still share a slot.  The strides run LPR/2 down
  // to 1 in both parts, so each value is the xor-tree sum of its partials.
#pragma unroll
  for (int g = 0; g < kG; ++g) {
#pragma unroll
    for (int half = kSlots / 2, stride = LPR / 2; half >= 1; half >>= 1, stride >>= 1) {
      const bool upper = (col & stride) != 0;
#pragma unroll
      for (int t = 0; t < half; ++t) {
        const float send = upper ? acc[g][t] : acc[g][t + half];
        const float keep = upper ? acc[g][t + half] : acc[g][t];
        acc[g][t] = keep + xshfl(send, stride);
      }
    }
    constexpr int kShare = LPR / kSlots;  // lanes holding the same slot
#pragma unroll
    for (int d = kShare / 2; d >= 1; d >>= 1) acc[g][0] += xshfl(acc[g][0], d);
    sc[g] = acc[g][0];
  }
  constexpr int kShare = LPR / kSlots;
  const int pos = (col / kShare) * kRowsPerLoad + grp;
  *r = ((col % kShare) == 0 && pos < cnt) ? pos : -1;
}

// The two halves of a one-pool, one-query pass whose slots load in one
// batch (row_pass with kRows = kG = 1 and every slot in flight together), so
// that other loads and arithmetic can sit between the loads and their use:
// row_issue issues the pass's row loads into a RowLoads, row_score consumes
// them with row_pass's arithmetic (the same partials, the same
// reduce-scatter), so the scores carry the same bits.
template <int LPR, int VPL, int kPass>
struct RowLoads {
  static constexpr int kSlots = kPass / (kWave / LPR);
  U4 buf[kSlots][VPL];
  bool live[kSlots];
};

template <int LPR, int VPL, int kPass>
__device__ __forceinline__ void row_issue(const uint16_t* y, long long y_rows, int D, int my_row, int grp, int col,
                                          RowLoads<LPR, VPL, kPass>& rl) {
  constexpr int kRowsPerLoad = kWave / LPR;
  constexpr int kSlots = RowLoads<LPR, VPL, kPass>::kSlots;
  static_assert(kSlots >= 1 && kSlots <= LPR && kSlots * kRowsPerLoad == kPass, "pass geometry");
  int first = __builtin_amdgcn_readlane(my_row, 0);
  if (first < 0 || first >= y_rows) first = 0;
  // Every slot is loaded (a slot past the pass reads row `first` again and
  // is not live): no branch, so no value waits for its load here.
#pragma unroll
  for (int ii = 0; ii < kSlots; ++ii) {
    const int row = __shfl(my_row, ii * kRowsPerLoad + grp, kWave);
    rl.live[ii] = row >= 0 && row < y_rows;
    const long long off = (long long)(rl.live[ii] ? row : first) * D;
#pragma unroll
    for (int v = 0; v < VPL; ++v) rl.buf[ii][v] = ld16_stream(y + off + (v * LPR + col) * 8);
  }
}

// (the query slice as packed bf16 pairs, dot_row_packed: the bits of
// dot_row's partials)
template <int LPR, int VPL, int kPass>
__device__ __forceinline__ float row_score(const RowLoads<LPR, VPL, kPass>& rl, const U4 (&xq)[VPL], int cnt, int grp,
                                           int col, int* r) {
  constexpr int kRowsPerLoad = kWave / LPR;
  constexpr int kSlots = RowLoads<LPR, VPL, kPass>::kSlots;
  float acc[kSlots];
#pragma unroll
  for (int ii = 0; ii < kSlots; ++ii) {
    const float s = dot_row_packed<VPL>(rl.buf[ii], xq);
    acc[ii] = rl.live[ii] ? s : 0.f;
  }
#pragma unroll
  for (int half = kSlots / 2, stride = LPR / 2; half >= 1; half >>= 1, stride >>= 1) {
    const bool upper = (col & stride) != 0;
#pragma unroll
    for (int t = 0; t < half; ++t) {
      const float send = upper ? acc[t] : acc[t + half];
      const float keep = upper ? acc[t + half] : acc[t];
      acc[t] = keep + xshfl(send, stride);
    }
  }
  constexpr int kShare = LPR / kSlots;
#pragma unroll
  for (int d = kShare / 2; d >= 1; d >>= 1) acc[0] += xshfl(acc[0], d);
  const int pos = (col / kShare) * kRowsPerLoad + grp;
  *r = ((col % kShare) == 0 && pos < cnt) ? pos : -1;
  return acc[0];
}

// Dot products of kG fp32 query rows with one gathered row per position:
// the lane's partial is the vtx::dot_row chain over its columns.
template <int LPR, int VPL, int kPass, int kG>
__device__ __forceinline__ void score_pass_multi(const uint16_t* y, long long y_rows, int D, int my_row, int cnt,
                                                 const float (&xs)[kG][VPL][8], int grp, int col, int* r,
                                                 float (&sc)[kG]) {
  const uint16_t* const ys[1] = {y};
  row_pass<LPR, VPL, kPass, kG, 1>(ys, y_rows, D, my_row, cnt, grp, col, r, sc,
                                   [&](const U4 (&rows)[1][VPL], int g) { return dot_row<VPL>(rows[0], xs[g]); });
}

// Quest page scores (arXiv:2406.10774) of kG fp32 query rows against each
// position's key envelope (rows of ymax and ymin):
//   sum_d max(bf16(q_d * max_d), bf16(q_d * min_d))
// with the lane's partial summed in column order from 0 — the elementwise
// multiply, maximum and row-sum kernels' arithmetic, in their order.  The
// maximum is taken before the rounding: rounding is monotonic, so
// bf16(max(a, b)) = max(bf16(a), bf16(b)) for all a, b (a NaN product is
// dropped by the maximum either way), with one conversion instead of two.
template <int LPR, int VPL, int kPass, int kG>
__device__ __forceinline__ void quest_pass_multi(const uint16_t* ymax, const uint16_t* ymin, long long y_rows, int D,
                                                 int my_row, int cnt, const float (&xs)[kG][VPL][8], int grp,
                                                 int col, int* r, float (&sc)[kG]) {
  const uint16_t* const ys[2] = {ymax, ymin};
  row_pass<LPR, VPL, kPass, kG, 2>(ys, y_rows, D, my_row, cnt, grp, col, r, sc,
                                   [&](const U4 (&rows)[2][VPL], int g) {
                                     float s = 0.f;
#pragma unroll
                                     for (int v = 0; v < VPL; ++v) {
                                       float mx[8], mn[8];
                                       unpack8(rows[0][v], mx);
                                       unpack8(rows[1][v], mn);
#pragma unroll
                                       for (int e = 0; e < 8; ++e)
                                         s += bf16r(fmaxf(xs[g][v][e] * mx[e], xs[g][v][e] * mn[e]));
                                     }
                                     return s;
                                   });
}

// score_pass with the query slice as packed bf16 pairs (dot_row_packed:
// the same partials, the same bits).
template <int LPR, int VPL, int kPass>
__device__ __forceinline__ float score_pass_packed(const uint16_t* y, long long y_rows, int D, int my_row, int cnt,
                                                   const U4 (&xq)[VPL], int grp, int col, int* r) {
  const uint16_t* const ys[1] = {y};
  float sc[1];
  row_pass<LPR, VPL, kPass, 1, 1>(ys, y_rows, D, my_row, cnt, grp, col, r, sc,
                                  [&](const U4 (&rows)[1][VPL], int) { return dot_row_packed<VPL>(rows[0], xq); });
  return sc[0];
}

// Single-query form: returns the lane's finished score.
template <int LPR, int VPL, int kPass>
__device__ __forceinline__ float score_pass(const uint16_t* y, long long y_rows, int D, int my_row, int cnt,
                                            const float (&xs)[VPL][8], int grp, int col, int* r) {
  float sc[1];
  score_pass_multi<LPR, VPL, kPass, 1>(y, y_rows, D, my_row, cnt,
                                       reinterpret_cast<const float(&)[1][VPL][8]>(xs), grp, col, r, sc);
  return sc[0];
}

}  // namespace vtx
