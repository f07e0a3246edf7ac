// The row-scoring pass shared by the fused indexer and the paged GeMM:
// dot products of kG fp32 query rows with up to kPass gathered bf16 rows,
// one wave, every row load issued before any arithmetic.
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
// holds the l-th position's row id of y ([y_rows, D] bf16) in my_row.  A row
// is split over LPR lanes x VPL 16-byte vectors (kRowsPerLoad = 64 / LPR rows
// per wave-wide load, kSlots = kPass / kRowsPerLoad rows per lane); every lane
// issues its row loads before any arithmetic (kBatch slots at a time for
// wide rows), then for each query g a reduce-scatter over the LPR lanes
// leaves each finished score on one lane: sc[g] (fp32, the vtx::dot_row chain
// of the lane's columns, then an xor tree with strides LPR/2 .. 1), at
// position *r of the pass; *r = -1 on lanes that own no position.  Rows
// outside y score 0.
template <int LPR, int VPL, int kPass, int kG>
__device__ __forceinline__ void score_pass_multi(const uint16_t* y, long long y_rows, int D, int my_row, int cnt,
                                                 const float (&xs)[kG][VPL][8], int grp, int col, int* r,
                                                 float (&sc)[kG]) {
  constexpr int kRowsPerLoad = kWave / LPR;
  constexpr int kSlots = kPass / kRowsPerLoad;
  constexpr int kBatch = VPL <= 2 ? kSlots : (kSlots < 2 ? kSlots : 2);  // slots loaded together
  static_assert(kSlots >= 1 && kSlots <= LPR && kSlots * kRowsPerLoad == kPass, "pass geometry");
  int first = __shfl(my_row, 0, kWave);
  if (first < 0 || first >= y_rows) first = 0;
  float acc[kG][kSlots];
#pragma unroll
  for (int i0 = 0; i0 < kSlots; i0 += kBatch) {
    U4 buf[kBatch][VPL];
    bool live[kBatch];
#pragma unroll
    for (int ii = 0; ii < kBatch; ++ii) {
      const int row = __shfl(my_row, (i0 + ii) * kRowsPerLoad + grp, kWave);
      live[ii] = row >= 0 && row < y_rows;
      if ((i0 + ii) * kRowsPerLoad < cnt) {  // wave-uniform: slots past the pass are skipped
        const uint16_t* yr = y + (long long)(live[ii] ? row : first) * D;
#pragma unroll
        for (int v = 0; v < VPL; ++v) buf[ii][v] = ld16_stream(yr + (v * LPR + col) * 8);
      } else {
#pragma unroll
        for (int v = 0; v < VPL; ++v) buf[ii][v] = U4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int ii = 0; ii < kBatch; ++ii)
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        const float s = dot_row<VPL>(buf[ii], xs[g]);
        acc[g][i0 + ii] = live[ii] ? s : 0.f;
      }
  }
  // Reduce-scatter over the slots (lane keeps slot bits of col from the top),
  // then fold the lanes that still share a slot.  The strides run LPR/2 down
  // to 1 in both parts.
#pragma unroll
  for (int g = 0; g < kG; ++g) {
#pragma unroll
    for (int half = kSlots / 2, stride = LPR / 2; half >= 1; half >>= 1, stride >>= 1) {
      const bool upper = (col & stride) != 0;
#pragma unroll
      for (int t = 0; t < half; ++t) {
        const float send = upper ? acc[g][t] : acc[g][t + half];
        const float keep = upper ? acc[g][t + half] : acc[g][t];
        acc[g][t] = keep + __shfl_xor(send, stride, kWave);
      }
    }
    constexpr int kShare = LPR / kSlots;  // lanes holding the same slot
#pragma unroll
    for (int d = kShare / 2; d >= 1; d >>= 1) acc[g][0] += __shfl_xor(acc[g][0], d, kWave);
    sc[g] = acc[g][0];
  }
  constexpr int kShare = LPR / kSlots;
  const int pos = (col / kShare) * kRowsPerLoad + grp;
  *r = ((col % kShare) == 0 && pos < cnt) ? pos : -1;
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
