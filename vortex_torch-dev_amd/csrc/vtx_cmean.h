// A layer's decode page reduce run inside a fused indexer launch: the mean
// over each closed page's [rows_per_tile, cols] K tile into the centroid pool
// the launch scores (block-sparse and GQA kernels), or its max and min into
// the envelope pools (Quest kernel).
// The tiles are reduced with the page-reduce kernel's own code
// (vtx_page_reduce.h), and a scored page whose centroid the launch rewrites
// is scored against the centroid recomputed from its K tile, so the launch
// writes what a page-reduce launch followed by the indexer would.
#pragma once

#include "vtx_device.h"
#include "vtx_page_reduce.h"

namespace vtx {

constexpr int kCmLoc = 256;  // loc entries a launch with an in-kernel CMean scans

struct CmArgs {
  const uint16_t* x;  // K pool [x_rows, rows_per_tile, cols]
  int64_t x_rows;
  int32_t rows_per_tile, cols;
  uint16_t* out;      // the centroid pool the launch scores (the max envelope for kEnvelope)
  uint16_t* out2;     // the min envelope (kEnvelope)
  int64_t out_rows;
  const int64_t* loc;
  int64_t nnz;
  int32_t heads, page;
  int32_t page_shift;  // log2(page) for a power of two, else -1
};

// What the in-launch page reduce writes: the mean (CMean) or the max and min
// envelopes (CMax + CMin, as one page_reduce_multi pass writes them).
enum CmKind { kCentroid = 0, kEnvelope = 1 };

// The pages the CMean closes, as one wave holds them (no LDS, no barrier):
// lane l keeps, for loc entries j * 64 + l (j < kLocRegs), the first tile
// row (page * H) of the page the entry closes, or -1; mask[j] is the ballot
// of the closing entries, so "the i-th closed page" is the i-th set bit in
// loc order, the order the page-reduce kernel lists them in.
template <int kLocRegs>
struct Closing {
  int base[kLocRegs];
  uint64_t mask[kLocRegs];
  int count;
};

// Issues the loads of loc (first in a kernel, so that waiting for them
// waits for nothing else).
template <int kLocRegs>
__device__ __forceinline__ void closing_load(const int64_t* loc, long long nnz, long long (&pos)[kLocRegs]) {
  const int lane = lane_id();
#pragma unroll
  for (int j = 0; j < kLocRegs; ++j) {
    const long long e = (long long)j * kWave + lane;
    pos[j] = e < nnz ? loc[e] : 0;
  }
}

template <int kLocRegs>
__device__ __forceinline__ void closing_load(const CmArgs& cm, long long (&pos)[kLocRegs]) {
  closing_load(cm.loc, cm.nnz, pos);
}

template <int kLocRegs>
__device__ __forceinline__ Closing<kLocRegs> closing_build(const CmArgs& cm, const long long (&pos)[kLocRegs]) {
  const int lane = lane_id();
  Closing<kLocRegs> c;
  c.count = 0;
#pragma unroll
  for (int j = 0; j < kLocRegs; ++j) {
    const long long e = (long long)j * kWave + lane;
    const bool closes = e < cm.nnz && divides(pos[j] + 1, cm.page, cm.page_shift);  // C semantics, as page-reduce
    c.base[j] = closes ? (int)(div_c(pos[j], cm.page, cm.page_shift) * cm.heads) : -1;
    c.mask[j] = __ballot(closes);
    c.count += __popcll(c.mask[j]);
  }
  return c;
}

// First tile row of the i-th closed page (i < c.count); wave-uniform i.
template <int kLocRegs>
__device__ __forceinline__ int closing_base(const Closing<kLocRegs>& c, int i) {
#pragma unroll
  for (int j = 0; j < kLocRegs; ++j) {
    const int n = __popcll(c.mask[j]);
    if (i < n) {
      uint64_t m = c.mask[j];
      for (int k = 0; k < i; ++k) m &= m - 1;
      return __builtin_amdgcn_readlane(c.base[j], __ffsll((long long)m) - 1);
    }
    i -= n;
  }
  return -1;
}

__device__ __forceinline__ U4 pack_value(const Acc (&acc)[8], int type, int count) {
  uint32_t b[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) b[e] = acc_value(acc[e], type, count);
  return U4{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
}

// Tiles first, first + stride, ... of the closed pages (tile t: head t % H
// of closed page t / H): the mean (kCentroid) or the max and min (kEnvelope)
// over each tile's rows into cm.out (and cm.out2), exactly as
// reduce_rows_vec_kernel computes them (max and min are exact, whatever
// else that kernel accumulates).  Wave-level.
template <int LPR, int kLocRegs, int kKind>
__device__ __forceinline__ void cmean_tiles(const CmArgs& cm, const Closing<kLocRegs>& c, int first, int stride,
                                            int grp, int cv) {
  constexpr int kNeed = kKind == kCentroid ? kNeedSum : (kNeedMax | kNeedMin);
  const int tiles = c.count * cm.heads;
  for (int t = first; t < tiles; t += stride) {
    const long long row = (long long)closing_base(c, t / cm.heads) + (t % cm.heads);
    if (!tile_in_range(cm, row)) continue;
    Acc acc[8];
    tile_stats_vec<LPR, kNeed>(cm.x, row, cm.rows_per_tile, cm.cols, grp, cv, acc);
    if (grp == 0) {
      const long long elem = row * cm.cols + cv * 8;
      if constexpr (kKind == kCentroid) {
        st16(cm.out + elem, pack_value(acc, VTX_REDUCE_MEAN, cm.rows_per_tile));
      } else {
        st16(cm.out + elem, pack_value(acc, VTX_REDUCE_MAX, cm.rows_per_tile));
        st16(cm.out2 + elem, pack_value(acc, VTX_REDUCE_MIN, cm.rows_per_tile));
      }
    }
  }
}

// The centroid of tile row `rid` as the CMean writes it, for the lane's 16-byte
// column vector: all 64 lanes take part (lane = grp * LPR + col) and every
// row group ends with the same vector.  Rows of one vector per lane.
template <int LPR>
__device__ __forceinline__ U4 fresh_centroid(const CmArgs& cm, int rid, int grp, int col) {
  Acc acc[8];
  tile_stats_vec<LPR, kNeedSum>(cm.x, rid, cm.rows_per_tile, cm.cols, grp, col, acc);
  return pack_value(acc, VTX_REDUCE_MEAN, cm.rows_per_tile);
}

// The max and min envelope vectors of tile row `rid`, as CMax and CMin write
// them (same lane layout as fresh_centroid).
template <int LPR>
__device__ __forceinline__ void fresh_envelope(const CmArgs& cm, int rid, int grp, int col, U4& mx, U4& mn) {
  Acc acc[8];
  tile_stats_vec<LPR, kNeedMax | kNeedMin>(cm.x, rid, cm.rows_per_tile, cm.cols, grp, col, acc);
  mx = pack_value(acc, VTX_REDUCE_MAX, cm.rows_per_tile);
  mn = pack_value(acc, VTX_REDUCE_MIN, cm.rows_per_tile);
}

// The score of a query slice (xs: the lane's 8 columns) against a centroid
// vector: the lane's dot_row chain and the xor tree over the LPR lanes — the
// bits the scoring pass gives for that row.  Every lane of the row's lane
// group returns it.
template <int LPR>
__device__ __forceinline__ float score_vec(const U4& cen, const float (&xs)[1][8]) {
  const U4 row[1] = {cen};
  float f = dot_row<1>(row, xs);
#pragma unroll
  for (int d = LPR / 2; d >= 1; d >>= 1) f += xshfl(f, d);
  return f;
}

// Tile `row` reduced with the arithmetic of the page-reduce launch for its
// width (vtx_page_reduce.h): rows split over 64 / (cols / 8) lane groups and
// folded across them (reduce_rows_vec_kernel, cols / 8 = 8, 16, 32, 64),
// else rows summed in order by one lane per 16-byte column vector
// (reduce_colvec_kernel).  kCentroid: the mean row into dst; kEnvelope: the
// max row into dst and the min row into dst2 (global or LDS rows of cols
// bf16).  Wave-level; the tile must be in range.
template <int LPRT, int kKind>
__device__ __forceinline__ void tile_reduce_vec(const CmArgs& cm, long long row, uint16_t* dst, uint16_t* dst2) {
  constexpr int kNeed = kKind == kCentroid ? kNeedSum : (kNeedMax | kNeedMin);
  const int lane = lane_id();
  const int grp = lane / LPRT, cv = lane % LPRT;
  Acc acc[8];
  tile_stats_vec<LPRT, kNeed>(cm.x, row, cm.rows_per_tile, cm.cols, grp, cv, acc);
  if (grp == 0) {
    if constexpr (kKind == kCentroid) {
      st16(dst + cv * 8, pack_value(acc, VTX_REDUCE_MEAN, cm.rows_per_tile));
    } else {
      st16(dst + cv * 8, pack_value(acc, VTX_REDUCE_MAX, cm.rows_per_tile));
      st16(dst2 + cv * 8, pack_value(acc, VTX_REDUCE_MIN, cm.rows_per_tile));
    }
  }
}

// tile_reduce_vec or the column-vector form, chosen by the row width
// (kNV = cols / 8 16-byte vectors, a compile-time constant of the caller).
template <int kNV, int kKind>
__device__ __forceinline__ void tile_reduce_any(const CmArgs& cm, long long row, uint16_t* dst, uint16_t* dst2) {
  if constexpr (kNV == 8 || kNV == 16 || kNV == 32 || kNV == 64) {
    tile_reduce_vec<kNV, kKind>(cm, row, dst, dst2);
  } else {
    constexpr int kNeed = kKind == kCentroid ? kNeedSum : (kNeedMax | kNeedMin);
    constexpr int kRowBatch = 8;
    const int R = cm.rows_per_tile;
    constexpr int C = kNV * 8;
    const uint16_t* tile = cm.x + row * (long long)R * C;
    for (int cv = lane_id(); cv < kNV; cv += kWave) {
      Acc acc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc_init<kNeed>(acc[e]);
      for (int r0 = 0; r0 < R; r0 += kRowBatch) {
        U4 v[kRowBatch];
#pragma unroll
        for (int u = 0; u < kRowBatch; ++u)
          v[u] = r0 + u < R ? ld16_stream(tile + (long long)(r0 + u) * C + cv * 8) : U4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int u = 0; u < kRowBatch; ++u) {
          if (r0 + u < R) {  // uniform (no break: the loads stay in registers)
            float f[8];
            unpack8(v[u], f);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc_add<kNeed>(acc[e], f[e]);
          }
        }
      }
      if constexpr (kKind == kCentroid) {
        st16(dst + cv * 8, pack_value(acc, VTX_REDUCE_MEAN, R));
      } else {
        st16(dst + cv * 8, pack_value(acc, VTX_REDUCE_MAX, R));
        st16(dst2 + cv * 8, pack_value(acc, VTX_REDUCE_MIN, R));
      }
    }
  }
}

// Columns blk * 64 + lane of tile `row` for rows of kNV 16-byte vectors that
// are not a tile_reduce_vec width: each lane sums its column vector's rows in
// order from 0 (reduce_colvec_kernel's arithmetic), its loads issued
// kColRows rows at a time (one memory trip for pages of up to kColRows
// tokens).  Wave-level; the tile must be in range.
constexpr int kColRows = 16;

template <int kNV, int kKind>
__device__ __forceinline__ void tile_reduce_colvec_part(const CmArgs& cm, long long row, int blk, uint16_t* dst,
                                                        uint16_t* dst2) {
  constexpr int kNeed = kKind == kCentroid ? kNeedSum : (kNeedMax | kNeedMin);
  constexpr int C = kNV * 8;
  const int R = cm.rows_per_tile;
  const int cv = blk * kWave + lane_id();
  const bool on = cv < kNV;
  const uint16_t* tile = cm.x + row * (long long)R * C + (on ? cv : 0) * 8;
  Acc acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc_init<kNeed>(acc[e]);
  for (int r0 = 0; r0 < R; r0 += kColRows) {
    U4 v[kColRows];
#pragma unroll
    for (int u = 0; u < kColRows; ++u)
      v[u] = r0 + u < R ? ld16_stream(tile + (long long)(r0 + u) * C) : U4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int u = 0; u < kColRows; ++u) {
      if (r0 + u < R) {  // uniform (no break: the loads stay in registers)
        float f[8];
        unpack8(v[u], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc_add<kNeed>(acc[e], f[e]);
      }
    }
  }
  if (on) {
    if constexpr (kKind == kCentroid) {
      st16(dst + cv * 8, pack_value(acc, VTX_REDUCE_MEAN, R));
    } else {
      st16(dst + cv * 8, pack_value(acc, VTX_REDUCE_MAX, R));
      st16(dst2 + cv * 8, pack_value(acc, VTX_REDUCE_MIN, R));
    }
  }
}

// Tiles of the closed pages reduced as the page-reduce launch for rows of
// kNV 16-byte vectors would, for kernels whose scoring layout is not the tile
// layout; wave-level, work units first, first + stride, ...  A unit is a
// tile for the tile_reduce_vec widths (kNV 8, 16, 32, 64), else a part of 64
// column vectors of a tile (tile_reduce_colvec_part), so that the waves
// share a wide tile and each issues its loads in one trip.
template <int kNV>
__host__ __device__ constexpr int tile_parts() {
  return (kNV == 8 || kNV == 16 || kNV == 32 || kNV == 64) ? 1 : (kNV + kWave - 1) / kWave;
}

template <int kNV, int kLocRegs, int kKind>
__device__ __forceinline__ void cmean_tiles_any(const CmArgs& cm, const Closing<kLocRegs>& c, int first, int stride) {
  constexpr int kParts = tile_parts<kNV>();
  constexpr bool kVecWidth = kNV == 8 || kNV == 16 || kNV == 32 || kNV == 64;
  const int units = c.count * cm.heads * kParts;
  for (int t = first; t < units; t += stride) {
    const int tile = t / kParts;
    const long long row = (long long)closing_base(c, tile / cm.heads) + (tile % cm.heads);
    if (!tile_in_range(cm, row)) continue;
    uint16_t* dst = cm.out + row * cm.cols;
    uint16_t* dst2 = cm.out2 ? cm.out2 + row * cm.cols : nullptr;
    if constexpr (kVecWidth) tile_reduce_vec<kNV, kKind>(cm, row, dst, dst2);
    else tile_reduce_colvec_part<kNV, kKind>(cm, row, t % kParts, dst, dst2);
  }
}

// The centroid of tile row `rid` as the CMean launch writes it, delivered in
// a scoring layout of LPR lanes x VPL 16-byte vectors per row (lane = grp *
// LPR + col holds vectors v * LPR + col).  One vector per lane: the tile
// layout is the scoring layout (fresh_centroid).  Wider rows: reduced into
// the wave's LDS row `scratch` (cols bf16), then read back.  Wave-level.
template <int LPR, int VPL>
__device__ __forceinline__ void fresh_centroid_rows(const CmArgs& cm, int rid, uint16_t* scratch, int grp, int col,
                                                    U4 (&cen)[VPL]) {
  if constexpr (VPL == 1) {
    cen[0] = fresh_centroid<LPR>(cm, rid, grp, col);
  } else {
    tile_reduce_any<LPR * VPL, kCentroid>(cm, rid, scratch, nullptr);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // the row is read by other lanes of the wave
#pragma unroll
    for (int v = 0; v < VPL; ++v) cen[v] = ld16(scratch + (v * LPR + col) * 8);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // read before the scratch row is reused
  }
}

// score_vec for rows of VPL vectors per lane: the lane's dot_row chain over
// its vectors, then the xor tree over the LPR lanes (the scoring pass's bits).
template <int LPR, int VPL>
__device__ __forceinline__ float score_vec_rows(const U4 (&cen)[VPL], const float (&xs)[VPL][8]) {
  float f = dot_row<VPL>(cen, xs);
#pragma unroll
  for (int d = LPR / 2; d >= 1; d >>= 1) f += xshfl(f, d);
  return f;
}

// score_vec_rows with the query slice as packed bf16 pairs (the same bits).
template <int LPR, int VPL>
__device__ __forceinline__ float score_vec_rows_packed(const U4 (&cen)[VPL], const U4 (&xq)[VPL]) {
  float f = dot_row_packed<VPL>(cen, xq);
#pragma unroll
  for (int d = LPR / 2; d >= 1; d >>= 1) f += xshfl(f, d);
  return f;
}

// Whether the lane's pass position (r >= 0, row my_rid) is a tile the
// in-kernel CMean writes: a row in [page * H, page * H + H) of a closed page,
// inside the pool and the centroid pool.
template <int kLocRegs>
__device__ __forceinline__ bool closes_here(const CmArgs& cm, const Closing<kLocRegs>& c, int r, int my_rid) {
  const bool cand = r >= 0 && my_rid >= 0 && my_rid < cm.x_rows && my_rid < cm.out_rows;
  bool fix = false;
#pragma unroll
  for (int j = 0; j < kLocRegs; ++j) {
    uint64_t m = c.mask[j];
    while (m) {  // wave-uniform
      const int l = __ffsll((long long)m) - 1;
      m &= m - 1;
      const int base = __builtin_amdgcn_readlane(c.base[j], l);
      fix |= (unsigned)(my_rid - base) < (unsigned)cm.heads;
    }
  }
  return cand && fix;
}

}  // namespace vtx
