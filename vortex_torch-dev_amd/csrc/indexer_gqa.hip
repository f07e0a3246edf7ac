// Fused indexer step of the GQA flow for gfx950: GeMM of the G query heads
// against every middle page's centroid, the segment softmax of each query
// head's scores (optional), the maximum over the query heads and the top-k
// select — one launch, one workgroup per segment (request, kv head).
//
// It produces exactly what the separate kernels produce for a block table
// built by the decode planner, at every middle page p of a segment with more
// than topk of them:
//   score[p, 0, g] = bf16(q[s*G+g] . y[dense[p]])            (GeMM, mm_bpr)
//   score[p, 0, g] = bf16(softmax over the segment's pages)   (Softmax, in place)
//   aggr[p]        = max_g score[p, 0, g]                      (Max, dim 2)
//   sparse[sparse_indptr[s]+bos+i] = the i-th best page by aggr (topK)
// The scores use the shared scoring pass (vtx_score.h) and the softmax the
// shared column statistics (vtx_segment.h), so every bit equals the separate
// kernels' output.  Segments with up to row_cap middle pages keep the raw
// scores, keys and page ids in LDS; longer ones stage them in the output
// buffers.
#include "vtx_cmean.h"
#include "vtx_device.h"
#include "vtx_fused_schedule.h"
#include "vtx_host.h"
#include "vtx_score.h"
#include "vtx_segment.h"
#include "vtx_select.h"

namespace {

struct GqaArgs {
  const uint16_t* q;  // [segments * G, D]
  const uint16_t* y;  // [y_rows, D]
  int64_t y_rows;
  uint16_t* score;    // [score_rows, 1, G]
  int64_t score_rows;
  uint16_t* aggr;     // [aggr_len]
  int64_t aggr_len;
  const int32_t* dindptr;
  const int32_t* sindptr;
  const int32_t* didx;
  int64_t didx_len;
  int32_t* sidx;
  int64_t sidx_len;
  int32_t segments, G, dim, topk, bos, eos, row_cap;
  int32_t softmax;
  float scale;
  const int32_t* sched;  // the planner's workgroup schedule, or null (passed to the kernel up front)
};

// kCmRegs > 0: the launch also runs the layer's decode CMean into y (loc: up
// to 64 * kCmRegs entries, rows of one vector per lane), as the block-sparse
// fused kernel does (vtx_cmean.h); its tiles go to the workgroups that finish
// first, after their own select.
//
// With the planner's workgroup schedule (sched, vtx_fused_schedule.h) the
// workgroups take the segments in its order, every compute unit a short and
// a long one; the bounds it holds are checked against the block tables in
// the round trip of the first row ids, before anything is written, so a
// stale schedule costs time, never a result.  The schedule, loc and their
// sizes lead the argument list, so that the dispatch preloads them into
// SGPRs and the first loads wait for no kernel-argument load.
template <int T, int LPR, int VPL, int kG, int kCmRegs>
__global__ __launch_bounds__(T, (VPL == 1 ? 4 : (VPL <= 4 ? 2 : 1))) void gqa_fused_kernel(
    const int32_t* sched, const int64_t* loc, int32_t segments, int32_t loc_n, GqaArgs a, vtx::CmArgs cma) {
  static_assert(T >= vtx::kScanThreads, "the softmax statistics need kScanThreads threads");
  constexpr int kWaves = T / vtx::kWave;
  constexpr int kRowsPerLoad = vtx::kWave / LPR;
  constexpr int kPass = vtx::segment_pass<VPL>();
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ vtx::SelectShared<T> sh;
  __shared__ vtx::BitonicShared<T> bsh;  // cached segments of up to T pages with k <= 32
  __shared__ float pm[vtx::kScanThreads];
  __shared__ float ps[vtx::kScanThreads];

  constexpr bool cm_on = kCmRegs > 0 && VPL == 1;
  constexpr int kLocRegs = kCmRegs > 0 ? kCmRegs : 1;

  const int tid = threadIdx.x;
  const int lane = vtx::lane_id();
  const int wave = vtx::uniform(tid / vtx::kWave);
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int k = a.topk;
  const int D = a.dim;
  const int G = a.G;

  long long cm_pos[kLocRegs];
  if constexpr (cm_on) vtx::closing_load(loc, loc_n, cm_pos);
  const vtx::SchedPick pick = vtx::sched_pick(sched, segments);
  const int seg = pick.seg;
  long long start, n, obase;
  if (pick.predicted) {
    start = (long long)pick.pe[0] + a.bos;
    n = (long long)pick.pe[1] - a.eos - start;
    obase = (long long)pick.pe[2] + a.bos;
  } else {
    start = (long long)a.dindptr[seg] + a.bos;
    n = (long long)a.dindptr[seg + 1] - a.eos - start;
    obase = (long long)a.sindptr[seg] + a.bos;
  }
  auto is_active = [&]() {
    return k > 0 && n > k && start >= 0 && start + n <= a.score_rows && start + n <= a.aggr_len &&
           start + n <= a.didx_len && obase >= 0 && obase + k <= a.sidx_len;
  };
  bool active = is_active();
  if constexpr (!cm_on) {
    if (!active && !pick.predicted) return;  // uniform: the separate ops write nothing for this segment either
  }
  // the first pass's row ids, then the check of the predicted bounds (one
  // vector load: lane 0 dense begin, lane 1 dense end, lane 2 sparse
  // begin), both in one round trip
  long long share = 0;
  int my_row = -1;
  auto first_pass = [&]() {
    share = (n + kWaves - 1) / kWaves;
    share = (share + kRowsPerLoad - 1) / kRowsPerLoad * kRowsPerLoad;
    if (share > kPass) share = kPass;
    const long long p0 = (long long)wave * share;
    const long long cnt = p0 < n ? min(share, n - p0) : 0;
    my_row = lane < cnt ? a.didx[start + p0 + lane] : -1;
  };
  if (active) first_pass();  // uniform
  if (pick.predicted) {      // uniform
    const int32_t* bp = lane == 1 ? a.dindptr + seg + 1 : lane == 2 ? a.sindptr + seg : a.dindptr + seg;
    const int32_t bv = *bp;
    const int32_t t0 = __builtin_amdgcn_readlane(bv, 0), t1 = __builtin_amdgcn_readlane(bv, 1),
                  t2 = __builtin_amdgcn_readlane(bv, 2);
    if ((t0 != pick.pe[0]) | (t1 != pick.pe[1]) | (t2 != pick.pe[2])) {  // uniform; not for a current schedule
      start = (long long)t0 + a.bos;
      n = (long long)t1 - a.eos - start;
      obase = (long long)t2 + a.bos;
      active = is_active();
      if (active) first_pass();
    }
  }
  if constexpr (!cm_on) {
    if (!active) return;  // uniform
  }
  const bool cached = n <= a.row_cap;
  // the bitonic select (one key per thread, from LDS) when every page fits
  // one thread each and k <= 32: it needs no histogram
  const bool bitonic = cached && n <= T && k <= vtx::kMaxBitonicK;  // uniform
  uint64_t* sel = reinterpret_cast<uint64_t*>(smem);
  int32_t* rows = reinterpret_cast<int32_t*>(smem + (size_t)vtx::sel_slots(k) * sizeof(uint64_t));
  uint16_t* keys = reinterpret_cast<uint16_t*>(rows + a.row_cap);
  uint16_t* raw = keys + a.row_cap;  // [row_cap, G]
  uint16_t* sc_out = a.score + start * G;
  const int32_t* dseg = a.didx + start;
  const uint16_t* qs = a.q + (long long)seg * G * D;
  vtx::Closing<kLocRegs> closing{};
  int n_close = 0;
  if constexpr (cm_on) {
    closing = vtx::closing_build(cma, cm_pos);
    n_close = closing.count;
  }
  // this launch's CMean: wave w of the workgroup of tile rank r reduces tiles
  // w * grid + r, ... once its own segment is done (rank 0: the shortest
  // segment under a schedule)
  auto cm_tiles = [&]() {
    if constexpr (cm_on)
      vtx::cmean_tiles<LPR, kLocRegs, vtx::kCentroid>(cma, closing, wave * (int)gridDim.x + pick.tile_rank,
                                                       kWaves * (int)gridDim.x, grp, col);
  };
  if (!active) {  // uniform (only with the CMean)
    cm_tiles();
    return;
  }
  if (!bitonic) vtx::select_init<T>(sel, k, sh);

  // ---- scores of every middle page for every query head
  for (long long p0 = (long long)wave * share; p0 < n; p0 += (long long)kWaves * share) {
    const int cnt = (int)min(share, n - p0);
    if (p0 != (long long)wave * share) my_row = lane < cnt ? dseg[p0 + lane] : -1;  // later passes
    int r = -1;
    for (int g0 = 0; g0 < G; g0 += kG) {
      float xs[kG][VPL][8];
      // heads past G read head G - 1 and are zeroed by a select (no branch
      // around the load, which would make the wave wait for it there)
#pragma unroll
      for (int gg = 0; gg < kG; ++gg)
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
          const bool in = g0 + gg < G;
          float f[8];
          vtx::unpack8(vtx::ld16(qs + (long long)(in ? g0 + gg : G - 1) * D + (v * LPR + col) * 8), f);
#pragma unroll
          for (int e = 0; e < 8; ++e) xs[gg][v][e] = in ? f[e] : 0.f;
        }
      float sc[kG];
      vtx::score_pass_multi<LPR, VPL, kPass, kG>(a.y, a.y_rows, D, my_row, cnt, xs, grp, col, &r, sc);
      if (r >= 0) {
#pragma unroll
        for (int gg = 0; gg < kG; ++gg) {
          if (g0 + gg >= G) break;
          const uint16_t b = (uint16_t)vtx::f32_to_bf16(sc[gg]);
          if (cached) raw[(p0 + r) * G + g0 + gg] = b;
          else sc_out[(p0 + r) * G + g0 + gg] = b;
        }
      }
    }
    const int my_rid = __shfl(my_row, r < 0 ? 0 : r, vtx::kWave);
    if (cached && r >= 0) rows[p0 + r] = my_rid;
    if constexpr (cm_on) {
      if (n_close > 0) {  // uniform
        // pages whose centroid this launch's CMean rewrites: their raw scores
        // redone against the centroid recomputed from the K tile, one page at
        // a time per wave, stored by the lane that stored the first ones
        uint64_t m = __ballot(vtx::closes_here(cma, closing, r, my_rid));
        while (m) {  // uniform
          const int l = __ffsll((long long)m) - 1;
          m &= m - 1;
          const vtx::U4 cen = vtx::fresh_centroid<LPR>(cma, __builtin_amdgcn_readlane(my_rid, l), grp, col);
          for (int g = 0; g < G; ++g) {
            float xg[1][8];
            vtx::unpack8(vtx::ld16(qs + (long long)g * D + col * 8), xg[0]);
            const float f = vtx::score_vec<LPR>(cen, xg);
            if (lane == l) {
              const uint16_t b = (uint16_t)vtx::f32_to_bf16(f);
              if (cached) raw[(p0 + r) * G + g] = b;
              else sc_out[(p0 + r) * G + g] = b;
            }
          }
        }
      }
    }
  }
  __syncthreads();

  // ---- softmax statistics of each query head over the segment, then the
  // softmax values, their maximum over the query heads and the keys.  The
  // raw scores are read through a pointer of one kind per path (LDS when
  // cached, global otherwise), so the reads are LDS reads, not generic ones.
  auto stats_and_keys = [&](auto raw_at) {
    if (a.softmax) {
      float vals[vtx::kScanRegs];
      bool in_regs;
      vtx::column_scan_stats(raw_at, n, G, a.scale, true, pm, ps, vals, in_regs);
    }
    for (long long i = tid; i < n; i += T) {
      float m = -INFINITY;
      for (int g = 0; g < G; ++g) {
        const float v = raw_at(i, g);
        const uint32_t o = a.softmax ? vtx::f32_to_bf16(vtx::softmax_value(v, a.scale, pm[g], ps[g]))
                                     : vtx::f32_to_bf16(v);
        sc_out[i * G + g] = (uint16_t)o;
        m = fmaxf(m, vtx::bf16_to_f32(o));
      }
      const uint32_t ab = vtx::f32_to_bf16(m);
      a.aggr[start + i] = (uint16_t)ab;
      const uint32_t key = vtx::score_key(ab);
      if (cached) keys[i] = (uint16_t)key;
      if (!bitonic) vtx::select_count<T>(key, sh);
    }
  };
  if (cached) {  // uniform
    stats_and_keys([&](long long i, int g) -> float { return vtx::bf16_to_f32(raw[i * G + g]); });
  } else {
    stats_and_keys([&](long long i, int g) -> float { return vtx::bf16_to_f32(sc_out[i * G + g]); });
  }
  __syncthreads();

  // ---- top-k of the segment: the bitonic select (one key per thread, from
  // LDS) when every page fits one thread each and k <= 32, else the radix
  // select over the counted keys
  if (bitonic) {  // uniform
    const int i = threadIdx.x;
    const uint32_t comp = vtx::bitonic_comp(i < n, i < n ? (uint32_t)keys[i] : 0u, i);
    vtx::select_bitonic<T>(comp, k, bsh, [&](int rk, uint32_t c) { a.sidx[obase + rk] = rows[vtx::bitonic_position(c)]; });
    cm_tiles();
    return;
  }
  if (cached) {
    vtx::select_topk_counted<T>([&](long long i) { return (uint32_t)keys[i]; }, n, k, sel, sh);
  } else {
    const uint16_t* ag = a.aggr + start;
    vtx::select_topk_counted<T>([&](long long i) { return vtx::score_key(ag[i]); }, n, k, sel, sh);
  }
  vtx::select_emit<T>(sel, k, n, [&](int rk, long long pos) { a.sidx[obase + rk] = cached ? rows[pos] : dseg[pos]; });
  cm_tiles();
}

constexpr int kLdsBudget = 52 * 1024;  // dynamic LDS; the select tables and statistics take up to ~8 KB more
constexpr int kMaxTopk = 4096;
constexpr int kMaxGroup = 8;

template <int T, int kG>
int launch_dim(const GqaArgs& a, const vtx::CmArgs* cm, int grid, size_t lds, hipStream_t s) {
  const vtx::CmArgs none{};
  if (cm) {  // the in-kernel CMean: rows of one 16-byte vector per lane
    const bool one = cm->nnz <= vtx::kWave;
    const int32_t nnz = (int32_t)cm->nnz;  // at most vtx::kCmLoc
    switch (a.dim) {
      case 64:
        if (one) gqa_fused_kernel<T, 8, 1, kG, 1>
            <<<grid, T, lds, s>>>(a.sched, cm->loc, a.segments, nnz, a, *cm);
        else gqa_fused_kernel<T, 8, 1, kG, vtx::kCmLoc / vtx::kWave>
            <<<grid, T, lds, s>>>(a.sched, cm->loc, a.segments, nnz, a, *cm);
        break;
      case 128:
        if (one) gqa_fused_kernel<T, 16, 1, kG, 1>
            <<<grid, T, lds, s>>>(a.sched, cm->loc, a.segments, nnz, a, *cm);
        else gqa_fused_kernel<T, 16, 1, kG, vtx::kCmLoc / vtx::kWave>
            <<<grid, T, lds, s>>>(a.sched, cm->loc, a.segments, nnz, a, *cm);
        break;
      default: return vtx::fail(VTX_E_INVALID, "indexer_gqa_fused: in-kernel CMean needs head_dim 64 or 128");
    }
    return vtx::check_launch("indexer_gqa_fused (with CMean)");
  }
  switch (a.dim) {
    case 64:
      gqa_fused_kernel<T, 8, 1, kG, 0><<<grid, T, lds, s>>>(a.sched, nullptr, a.segments, 0, a, none);
      break;
    case 128:
      gqa_fused_kernel<T, 16, 1, kG, 0><<<grid, T, lds, s>>>(a.sched, nullptr, a.segments, 0, a, none);
      break;
    case 256:
      gqa_fused_kernel<T, 16, 2, 1, 0><<<grid, T, lds, s>>>(a.sched, nullptr, a.segments, 0, a, none);
      break;
    // wide rows keep their query slice in registers: fewer threads, no spills
    case 512:
      gqa_fused_kernel<(T > 512 ? 512 : T), 16, 4, 1, 0>
          <<<grid, (T > 512 ? 512 : T), lds, s>>>(a.sched, nullptr, a.segments, 0, a, none);
      break;
    case 576:
      gqa_fused_kernel<256, 8, 9, 1, 0><<<grid, 256, lds, s>>>(a.sched, nullptr, a.segments, 0, a, none);
      break;
    default: return vtx::fail(VTX_E_INVALID, "indexer_gqa_fused: head_dim %d not supported", a.dim);
  }
  return vtx::check_launch("indexer_gqa_fused");
}

template <int T>
int launch_g(const GqaArgs& a, const vtx::CmArgs* cm, int grid, size_t lds, hipStream_t s) {
  return a.G >= 2 ? launch_dim<T, 2>(a, cm, grid, lds, s) : launch_dim<T, 1>(a, cm, grid, lds, s);
}

}  // namespace

extern "C" int vtx_indexer_gqa_fused_supported(int32_t head_dim, int32_t group_size) {
  return (head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512 || head_dim == 576) &&
         group_size >= 1 && group_size <= kMaxGroup;
}

namespace {

// The decode CMean a GQA launch may run first (vtx_indexer_gqa_fused_cmean).
struct CmeanSpec {
  const uint16_t* k;
  int64_t k_rows;
  int32_t page_size, heads;
  const int64_t* loc;
  int64_t nnz;
};

int gqa_impl(const uint16_t* q, int64_t q_rows, int32_t group_size, const uint16_t* y, int64_t y_rows,
             int32_t head_dim, uint16_t* score, int64_t score_rows, uint16_t* aggr, int64_t aggr_len,
             const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr, const int32_t* dense_kv_indices,
             int64_t dense_kv_indices_len, int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
             int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos, int32_t reserved_eos,
             int32_t max_num_pages, int32_t softmax, float scale, const CmeanSpec* cms,
             const int32_t* schedule, int64_t schedule_len, void* stream);

}  // namespace

extern "C" int vtx_indexer_gqa_fused(const uint16_t* q, int64_t q_rows, int32_t group_size, const uint16_t* y,
                                     int64_t y_rows, int32_t head_dim, uint16_t* score, int64_t score_rows,
                                     uint16_t* aggr, int64_t aggr_len, const int32_t* dense_kv_indptr,
                                     const int32_t* sparse_kv_indptr, const int32_t* dense_kv_indices,
                                     int64_t dense_kv_indices_len, int32_t* sparse_kv_indices,
                                     int64_t sparse_kv_indices_len, int32_t eff_batch_size, int32_t topk_val,
                                     int32_t reserved_bos, int32_t reserved_eos, int32_t max_num_pages,
                                     int32_t softmax, float scale, const int32_t* schedule,
                                     int64_t schedule_len, void* stream) {
  vtx::clear_error();
  return gqa_impl(q, q_rows, group_size, y, y_rows, head_dim, score, score_rows, aggr, aggr_len, dense_kv_indptr,
                  sparse_kv_indptr, dense_kv_indices, dense_kv_indices_len, sparse_kv_indices, sparse_kv_indices_len,
                  eff_batch_size, topk_val, reserved_bos, reserved_eos, max_num_pages, softmax, scale, nullptr,
                  schedule, schedule_len, stream);
}

extern "C" int vtx_indexer_gqa_fused_cmean(const uint16_t* q, int64_t q_rows, int32_t group_size, uint16_t* y,
                                           int64_t y_rows, int32_t head_dim, uint16_t* score, int64_t score_rows,
                                           uint16_t* aggr, int64_t aggr_len, const int32_t* dense_kv_indptr,
                                           const int32_t* sparse_kv_indptr, const int32_t* dense_kv_indices,
                                           int64_t dense_kv_indices_len, int32_t* sparse_kv_indices,
                                           int64_t sparse_kv_indices_len, int32_t eff_batch_size, int32_t topk_val,
                                           int32_t reserved_bos, int32_t reserved_eos, int32_t max_num_pages,
                                           int32_t softmax, float scale, const uint16_t* k_cache, int64_t k_rows,
                                           int32_t page_size, int32_t num_kv_heads, const int64_t* loc,
                                           int64_t nnz, const int32_t* schedule, int64_t schedule_len,
                                           void* stream) {
  vtx::clear_error();
  if (!k_cache || (nnz > 0 && !loc))
    return vtx::fail(VTX_E_INVALID, "indexer_gqa_fused_cmean: null K pool or loc");
  if (page_size < 1 || num_kv_heads < 1 || k_rows < 0 || nnz < 0)
    return vtx::fail(VTX_E_INVALID, "indexer_gqa_fused_cmean: bad CMean sizes");
  const CmeanSpec cm{k_cache, k_rows, page_size, num_kv_heads, loc, nnz};
  return gqa_impl(q, q_rows, group_size, y, y_rows, head_dim, score, score_rows, aggr, aggr_len, dense_kv_indptr,
                  sparse_kv_indptr, dense_kv_indices, dense_kv_indices_len, sparse_kv_indices, sparse_kv_indices_len,
                  eff_batch_size, topk_val, reserved_bos, reserved_eos, max_num_pages, softmax, scale, &cm, schedule,
                  schedule_len, stream);
}

namespace {

int gqa_impl(const uint16_t* q, int64_t q_rows, int32_t group_size, const uint16_t* y, int64_t y_rows,
             int32_t head_dim, uint16_t* score, int64_t score_rows, uint16_t* aggr, int64_t aggr_len,
             const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr, const int32_t* dense_kv_indices,
             int64_t dense_kv_indices_len, int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
             int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos, int32_t reserved_eos,
             int32_t max_num_pages, int32_t softmax, float scale, const CmeanSpec* cms,
             const int32_t* schedule, int64_t schedule_len, void* stream) {
  const char* what = "indexer_gqa_fused";
  if (eff_batch_size < 0 || reserved_bos < 0 || reserved_eos < 0)
    return vtx::fail(VTX_E_INVALID, "%s: negative size", what);
  if (!vtx_indexer_gqa_fused_supported(head_dim, group_size))
    return vtx::fail(VTX_E_INVALID, "%s: head_dim %d with group size %d not supported", what, head_dim,
                     group_size);
  if (topk_val > kMaxTopk) return vtx::fail(VTX_E_INVALID, "%s: topk_val %d exceeds %d", what, topk_val, kMaxTopk);
  if (q_rows < (long long)eff_batch_size * group_size)
    return vtx::fail(VTX_E_INVALID, "%s: %lld query rows for %d segments of %d heads", what, (long long)q_rows,
                     eff_batch_size, group_size);
  // The CMean runs inside the launch for rows of one 16-byte vector per lane
  // and decode-sized loc; otherwise as its own launch, first.
  const bool cm_inside = cms && (head_dim == 64 || head_dim == 128) && cms->nnz <= vtx::kCmLoc;
  if (cms && !cm_inside && cms->nnz > 0) {
    const int rc = vtx_page_reduce(cms->k, cms->k_rows, cms->page_size, head_dim, const_cast<uint16_t*>(y),
                                   VTX_DTYPE_BF16, y_rows, cms->loc, cms->nnz, cms->heads, cms->page_size, 1,
                                   VTX_REDUCE_MEAN, stream);
    if (rc != VTX_OK) return rc;
  }
  if (eff_batch_size == 0) return VTX_OK;
  if (!q || !y || !score || !aggr || !dense_kv_indptr || !sparse_kv_indptr || !dense_kv_indices || !sparse_kv_indices)
    return vtx::fail(VTX_E_INVALID, "%s: null pointer", what);
  if (y_rows <= 0) return vtx::fail(VTX_E_INVALID, "%s: empty centroid pool", what);
  if (!vtx::aligned16(q) || !vtx::aligned16(y))
    return vtx::fail(VTX_E_INVALID, "%s: query and centroid rows must be 16-byte aligned", what);
  GqaArgs a;
  a.q = q;
  a.y = y;
  a.y_rows = y_rows;
  a.score = score;
  a.score_rows = score_rows;
  a.aggr = aggr;
  a.aggr_len = aggr_len;
  a.dindptr = dense_kv_indptr;
  a.sindptr = sparse_kv_indptr;
  a.didx = dense_kv_indices;
  a.didx_len = dense_kv_indices_len;
  a.sidx = sparse_kv_indices;
  a.sidx_len = sparse_kv_indices_len;
  a.segments = eff_batch_size;
  a.G = group_size;
  a.dim = head_dim;
  a.topk = topk_val > 0 ? topk_val : 0;
  a.bos = reserved_bos;
  a.eos = reserved_eos;
  a.softmax = softmax != 0;
  a.scale = scale;
  // a schedule too short for this launch is not used (the kernel would also
  // ignore one whose header names another segment count)
  a.sched = schedule && schedule_len >= vtx::sched_len(1, eff_batch_size) ? schedule : nullptr;
  const long long want = max_num_pages > 0 ? max_num_pages : 0;
  const long long per = 4 + 2 + 2LL * group_size;  // page id, key, raw scores
  const long long room = (kLdsBudget - (long long)vtx::sel_slots(a.topk) * 8) / per;
  long long cap = want < room ? want : room;
  cap &= ~7LL;
  if (cap < 0) cap = 0;
  a.row_cap = (int32_t)cap;
  const size_t lds = (size_t)vtx::sel_slots(a.topk) * 8 + (size_t)cap * per;
  hipStream_t s = vtx::as_stream(stream);
  vtx::CmArgs cma{};
  const bool cm_launch = cm_inside && cms->nnz > 0;
  if (cm_launch) {
    cma.x = cms->k;
    cma.x_rows = cms->k_rows;
    cma.rows_per_tile = cms->page_size;
    cma.cols = head_dim;
    cma.out = const_cast<uint16_t*>(y);
    cma.out_rows = y_rows;
    cma.loc = cms->loc;
    cma.nnz = cms->nnz;
    cma.heads = cms->heads;
    cma.page = cms->page_size;
    cma.page_shift = vtx::log2_exact(cms->page_size);
  }
  const vtx::CmArgs* cmp = cm_launch ? &cma : nullptr;
  if (max_num_pages <= 256) return launch_g<256>(a, cmp, eff_batch_size, lds, s);
  if (max_num_pages <= 1024) return launch_g<512>(a, cmp, eff_batch_size, lds, s);
  return launch_g<1024>(a, cmp, eff_batch_size, lds, s);
}

}  // namespace
