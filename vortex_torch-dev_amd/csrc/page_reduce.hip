// Page-finish reductions (CMean / CMax / CMin / CL2Norm) for gfx950.
//
// Semantics follow the reference reduce_pp_kernel
// (vortex_torch/cache/triton_kernels/reduce_impl.py:7-62): for every loc entry
// whose token closes a page ((loc+1) % page_size == 0) and every kv head h,
// tile row = (loc / page_size) * H + h of x [rows, R, C] is reduced over its
// R axis (dim 1, output [rows, 1, C]) or its C axis (dim 2, output [rows, R, 1]).
//
// Design (pure HBM streaming, 4 KB per tile at R=16, C=128):
//   * each workgroup scans 256 loc entries with coalesced loads and compacts
//     the pages they close into an LDS list, so no wave is spent on the
//     15 of 16 tokens that close nothing (the reference launches one program
//     per (token, head) and returns early from most of them);
//   * each wave then reduces whole (page, head) tiles: for dim 1 a row of C
//     bf16 is split over C/8 lanes with one 16-byte load each; with tiles of
//     up to 16 rows each lane walks every row of its column (64/(C/8) tiles
//     per wave at once, all rows in flight), otherwise the remaining lanes
//     take further rows, every lane accumulates fp32 over its rows and a
//     shuffle tree folds the row groups together (the same bits either way);
//   * widths whose 16-byte column count does not divide 64 (D = 576) give
//     each lane one column vector and load 8 rows of it at a time;
//   * one pass over the tile feeds up to four outputs (the fused entry point),
//     so CMean + CMax read K once.
#include "vtx_device.h"
#include "vtx_host.h"
#include "vtx_page_reduce.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / vtx::kWave;
constexpr int kMaxOut = vtx::kPageReduceMaxOut;
using ReduceArgs = vtx::PageReduceArgs;
using vtx::Acc;
using vtx::acc_add;
using vtx::acc_init;
using vtx::acc_merge_xor;
using vtx::acc_value;
using vtx::kNeedAll;
using vtx::kNeedMax;
using vtx::kNeedMin;
using vtx::kNeedSq;
using vtx::kNeedSum;
using vtx::need_of;

__device__ __forceinline__ void store_one(const ReduceArgs& a, int o, long long elem, uint32_t bits) {
  if (a.out_dtype[o] == VTX_DTYPE_BF16)
    reinterpret_cast<uint16_t*>(a.out[o])[elem] = (uint16_t)bits;
  else
    reinterpret_cast<uint32_t*>(a.out[o])[elem] = bits << 16;
}

// The pages closed by this block's 256 loc entries (the workgroups that share
// a block of entries split its tiles by index, so they all see the same list).
__device__ __forceinline__ int collect_pages(const ReduceArgs& a, long long* first_row, int* wave_count) {
  return vtx::collect_pages<kThreads>(a, (long long)blockIdx.x * kThreads, first_row, wave_count);
}

// dim 1, C = 8 * LPR with LPR | 64.  Bursts of tiles of up to 16 rows (and
// a statistic set whose registers fit): lane = (tile slot, 16-byte column
// vector), a wave takes 64 / LPR tiles at once and each lane reduces all rows
// of its column alone (vtx::tile_stats_lane), so all of a tile's rows are in
// flight together, nothing crosses lanes and every lane writes its own
// outputs.  Otherwise lane = (row group, column vector), one tile per wave,
// folded by an xor tree (vtx::tile_stats_vec).  Both give the same bits.
// NEED: statistics to accumulate (kNeed* mask covering every output's type).
template <int LPR, int NEED>
__global__ __launch_bounds__(kThreads) void reduce_rows_vec_kernel(ReduceArgs a) {
  __shared__ long long first_row[kThreads];
  __shared__ int wave_count[kWavesPerBlock];
  const int pages = collect_pages(a, first_row, wave_count);
  const int lane = vtx::lane_id();
  const int grp = lane / LPR;
  const int cv = lane % LPR;
  const int wave = threadIdx.x / vtx::kWave;
  const int R = a.rows_per_tile;
  const int tiles = pages * a.heads;

  if constexpr (vtx::lane_tiles_fit<LPR, NEED>()) {
    // (a decode-sized loc, whose few tiles are spread over several
    // workgroups, keeps one tile per wave: more waves share the latency)
    if (R <= 16 && gridDim.y == 1) {  // uniform
      constexpr int kSlots = vtx::kWave / LPR;  // tiles per wave at once; lane group grp takes slot grp
      for (int t0 = (blockIdx.y * kWavesPerBlock + wave) * kSlots; t0 < tiles;
           t0 += gridDim.y * kWavesPerBlock * kSlots) {
        const int t = t0 + grp;
        if (t >= tiles) continue;
        const long long row = first_row[t / a.heads] + (t % a.heads);
        if (!vtx::tile_in_range(a, row)) continue;
        Acc acc[8];
        vtx::tile_stats_lane<LPR, NEED>(a.x, row, R, a.cols, cv, acc);
        vtx::tile_store_vec(a, row, cv, acc);
      }
      return;
    }
  }
  for (int t = blockIdx.y * kWavesPerBlock + wave; t < tiles; t += gridDim.y * kWavesPerBlock) {
    const long long row = first_row[t / a.heads] + (t % a.heads);
    if (!vtx::tile_in_range(a, row)) continue;
    Acc acc[8];
    vtx::tile_stats_vec<LPR, NEED>(a.x, row, R, a.cols, grp, cv, acc);
    if (grp == 0) vtx::tile_store_vec(a, row, cv, acc);
  }
}

// dim 1, C = 8 * nv for any nv (e.g. 576 = 8 * 72): lane = one 16-byte
// column vector; a wave covers 64 column vectors of a tile per round and each
// lane loads its vector from 8 rows at a time before accumulating them.
template <int NEED>
__global__ __launch_bounds__(kThreads) void reduce_colvec_kernel(ReduceArgs a) {
  constexpr int kRowBatch = 8;
  __shared__ long long first_row[kThreads];
  __shared__ int wave_count[kWavesPerBlock];
  const int pages = collect_pages(a, first_row, wave_count);
  const int lane = vtx::lane_id();
  const int wave = threadIdx.x / vtx::kWave;
  const int R = a.rows_per_tile;
  const int C = a.cols;
  const int nv = C / 8;
  const int tiles = pages * a.heads;

  for (int t = blockIdx.y * kWavesPerBlock + wave; t < tiles; t += gridDim.y * kWavesPerBlock) {
    const long long row = first_row[t / a.heads] + (t % a.heads);
    if (row < 0 || row >= a.x_rows || row >= a.out_rows) continue;
    const uint16_t* tile = a.x + row * (long long)R * C;
    for (int cv = lane; cv < nv; cv += vtx::kWave) {
      Acc acc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc_init<NEED>(acc[e]);
      for (int r0 = 0; r0 < R; r0 += kRowBatch) {
        vtx::U4 v[kRowBatch];
#pragma unroll
        for (int u = 0; u < kRowBatch; ++u)
          v[u] = r0 + u < R ? vtx::ld16_stream(tile + (long long)(r0 + u) * C + cv * 8) : vtx::U4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int u = 0; u < kRowBatch; ++u) {
          if (r0 + u >= R) break;
          float f[8];
          vtx::unpack8(v[u], f);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc_add<NEED>(acc[e], f[e]);
        }
      }
      const long long elem = row * C + cv * 8;
#pragma unroll
      for (int o = 0; o < kMaxOut; ++o) {
        if (o >= a.n_out) break;
        uint32_t b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) b[e] = acc_value(acc[e], a.out_type[o], R);
        if (a.out_dtype[o] == VTX_DTYPE_BF16) {
          vtx::st16(reinterpret_cast<uint16_t*>(a.out[o]) + elem,
                    vtx::U4{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16),
                            b[6] | (b[7] << 16)});
        } else {
          uint32_t* dst = reinterpret_cast<uint32_t*>(a.out[o]) + elem;
          vtx::st16(dst, vtx::U4{b[0] << 16, b[1] << 16, b[2] << 16, b[3] << 16});
          vtx::st16(dst + 4, vtx::U4{b[4] << 16, b[5] << 16, b[6] << 16, b[7] << 16});
        }
      }
    }
  }
}

// Any shape.  dim 1: lanes stride over columns, each lane walks all R rows.
// dim 2: the wave walks the R rows, lanes stride over columns, a wave
// reduction finishes each row.
__global__ __launch_bounds__(kThreads) void reduce_generic_kernel(ReduceArgs a, int dim) {
  __shared__ long long first_row[kThreads];
  __shared__ int wave_count[kWavesPerBlock];
  const int pages = collect_pages(a, first_row, wave_count);
  const int lane = vtx::lane_id();
  const int wave = threadIdx.x / vtx::kWave;
  const int R = a.rows_per_tile;
  const int C = a.cols;
  const int tiles = pages * a.heads;

  for (int t = blockIdx.y * kWavesPerBlock + wave; t < tiles; t += gridDim.y * kWavesPerBlock) {
    const long long row = first_row[t / a.heads] + (t % a.heads);
    if (row < 0 || row >= a.x_rows || row >= a.out_rows) continue;
    const uint16_t* tile = a.x + row * (long long)R * C;
    if (dim == 1) {
      for (int c = lane; c < C; c += vtx::kWave) {
        Acc acc;
        acc_init(acc);
#pragma unroll 8
        for (int r = 0; r < R; ++r) acc_add(acc, vtx::bf16_to_f32(tile[(long long)r * C + c]));
#pragma unroll
        for (int o = 0; o < kMaxOut; ++o)
          if (o < a.n_out) store_one(a, o, row * C + c, acc_value(acc, a.out_type[o], R));
      }
    } else {
      for (int r = 0; r < R; ++r) {
        Acc acc;
        acc_init(acc);
        for (int c = lane; c < C; c += vtx::kWave)
          acc_add(acc, vtx::bf16_to_f32(tile[(long long)r * C + c]));
#pragma unroll
        for (int d = 1; d < vtx::kWave; d <<= 1) acc_merge_xor(acc, d);
        if (lane == 0) {
#pragma unroll
          for (int o = 0; o < kMaxOut; ++o)
            if (o < a.n_out) store_one(a, o, row * R + r, acc_value(acc, a.out_type[o], C));
        }
      }
    }
  }
}

// Single reductions and CMean + CMax get their own code; other mixes
// accumulate every statistic.
template <int LPR>
void launch_vec(const ReduceArgs& a, int need, dim3 grid, hipStream_t s) {
  switch (need) {
    case kNeedSum: reduce_rows_vec_kernel<LPR, kNeedSum><<<grid, kThreads, 0, s>>>(a); break;
    case kNeedMax: reduce_rows_vec_kernel<LPR, kNeedMax><<<grid, kThreads, 0, s>>>(a); break;
    case kNeedMin: reduce_rows_vec_kernel<LPR, kNeedMin><<<grid, kThreads, 0, s>>>(a); break;
    case kNeedSq: reduce_rows_vec_kernel<LPR, kNeedSq><<<grid, kThreads, 0, s>>>(a); break;
    case kNeedSum | kNeedMax:
      reduce_rows_vec_kernel<LPR, kNeedSum | kNeedMax><<<grid, kThreads, 0, s>>>(a);
      break;
    default: reduce_rows_vec_kernel<LPR, kNeedAll><<<grid, kThreads, 0, s>>>(a); break;
  }
}

int launch_reduce(ReduceArgs& a, int dim, void* stream) {
  if (a.nnz <= 0) return VTX_OK;
  if (a.rows_per_tile < 1 || a.cols < 1)
    return vtx::fail(VTX_E_INVALID, "page_reduce: empty tile (%d x %d)", a.rows_per_tile, a.cols);
  if (a.heads < 1 || a.page < 1)
    return vtx::fail(VTX_E_INVALID, "page_reduce: num_kv_heads and page_size must be >= 1");
  if (dim != 1 && dim != 2) return vtx::fail(VTX_E_INVALID, "page_reduce: dim must be 1 or 2");
  if (a.n_out < 1 || a.n_out > kMaxOut)
    return vtx::fail(VTX_E_INVALID, "page_reduce: 1..%d outputs supported", kMaxOut);
  if (!a.x || !a.loc) return vtx::fail(VTX_E_INVALID, "page_reduce: null pointer");
  bool out_aligned = true;
  for (int o = 0; o < a.n_out; ++o) {
    if (!a.out[o]) return vtx::fail(VTX_E_INVALID, "page_reduce: null output %d", o);
    if (a.out_type[o] < VTX_REDUCE_MEAN || a.out_type[o] > VTX_REDUCE_L2NORM)
      return vtx::fail(VTX_E_INVALID, "page_reduce: unknown reduce type %d", a.out_type[o]);
    if (a.out_dtype[o] != VTX_DTYPE_BF16 && a.out_dtype[o] != VTX_DTYPE_F32)
      return vtx::fail(VTX_E_INVALID, "page_reduce: unknown output dtype %d", a.out_dtype[o]);
    out_aligned = out_aligned && vtx::aligned16(a.out[o]);
  }
  for (int o = a.n_out; o < kMaxOut; ++o) {
    a.out[o] = nullptr;
    a.out_dtype[o] = VTX_DTYPE_BF16;
    a.out_type[o] = VTX_REDUCE_MEAN;
  }
  const long long blocks = (a.nnz + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffffLL) return vtx::fail(VTX_E_INVALID, "page_reduce: loc too long");
  hipStream_t s = vtx::as_stream(stream);
  // Few loc entries (a decode step): the closed pages' tiles of one block of
  // entries are spread over up to 16 workgroups (each rescans the same
  // entries), so the tiles are reduced side by side rather than by 4 waves.
  long long split = (512 + blocks - 1) / blocks;
  if (split > 16) split = 16;
  if (split < 1) split = 1;
  const dim3 grid((unsigned)blocks, (unsigned)split);
  const bool vec = dim == 1 && (a.cols % 8 == 0) && vtx::aligned16(a.x) && out_aligned;
  const int lpr = a.cols / 8;
  int need = 0;
  for (int o = 0; o < a.n_out; ++o) need |= need_of(a.out_type[o]);
  if (vec && lpr == 8) {
    launch_vec<8>(a, need, grid, s);
  } else if (vec && lpr == 16) {
    launch_vec<16>(a, need, grid, s);
  } else if (vec && lpr == 32) {
    launch_vec<32>(a, need, grid, s);
  } else if (vec && lpr == 64) {
    launch_vec<64>(a, need, grid, s);
  } else if (vec) {
    switch (need) {
      case kNeedSum: reduce_colvec_kernel<kNeedSum><<<grid, kThreads, 0, s>>>(a); break;
      case kNeedMax: reduce_colvec_kernel<kNeedMax><<<grid, kThreads, 0, s>>>(a); break;
      case kNeedSum | kNeedMax: reduce_colvec_kernel<kNeedSum | kNeedMax><<<grid, kThreads, 0, s>>>(a); break;
      default: reduce_colvec_kernel<kNeedAll><<<grid, kThreads, 0, s>>>(a); break;
    }
  } else {
    reduce_generic_kernel<<<grid, kThreads, 0, s>>>(a, dim);
  }
  return vtx::check_launch("page_reduce");
}

}  // namespace

extern "C" int vtx_page_reduce(const uint16_t* x, int64_t x_rows, int32_t rows_per_tile,
                               int32_t cols, void* out, int32_t out_dtype, int64_t out_rows,
                               const int64_t* loc, int64_t nnz, int32_t num_kv_heads,
                               int32_t page_size, int32_t dim, int32_t reduce_type, void* stream) {
  vtx::clear_error();
  ReduceArgs a;
  a.x = x;
  a.x_rows = x_rows;
  a.rows_per_tile = rows_per_tile;
  a.cols = cols;
  a.out[0] = out;
  a.out_dtype[0] = out_dtype;
  a.out_type[0] = reduce_type;
  a.n_out = 1;
  a.out_rows = out_rows;
  a.loc = loc;
  a.nnz = nnz;
  a.heads = num_kv_heads;
  a.page = page_size;
  a.page_shift = vtx::log2_exact(page_size);
  return launch_reduce(a, dim, stream);
}

extern "C" int vtx_page_reduce_multi(const uint16_t* x, int64_t x_rows, int32_t rows_per_tile,
                                     int32_t cols, int32_t n_out, void* const* outs,
                                     const int32_t* out_dtypes, const int32_t* reduce_types,
                                     int64_t out_rows, const int64_t* loc, int64_t nnz,
                                     int32_t num_kv_heads, int32_t page_size, int32_t dim,
                                     void* stream) {
  vtx::clear_error();
  if (n_out < 1 || n_out > kMaxOut || !outs || !out_dtypes || !reduce_types)
    return vtx::fail(VTX_E_INVALID, "page_reduce_multi: need 1..%d outputs", kMaxOut);
  ReduceArgs a;
  a.x = x;
  a.x_rows = x_rows;
  a.rows_per_tile = rows_per_tile;
  a.cols = cols;
  for (int o = 0; o < n_out; ++o) {
    a.out[o] = outs[o];
    a.out_dtype[o] = out_dtypes[o];
    a.out_type[o] = reduce_types[o];
  }
  a.n_out = n_out;
  a.out_rows = out_rows;
  a.loc = loc;
  a.nnz = nnz;
  a.heads = num_kv_heads;
  a.page = page_size;
  a.page_shift = vtx::log2_exact(page_size);
  return launch_reduce(a, dim, stream);
}
