// Fused indexer step of one sparse layer for gfx950: query head-group mean,
// GeMV scoring of every middle page, top-k selection — one launch, one
// workgroup per segment (request, kv head).
//
// It produces exactly what the three separate ops produce for a block table
// built by the decode planner:
//   q_mean[s]  = bf16(fp32 sum_g q[s, g, :] * (1/G))        (torch's mean)
//   score[p]   = bf16(fp32 q_mean[s] . y[dense[p]])  for the middle pages
//                p in [indptr[s]+bos, indptr[s+1]-eos) of segments with more
//                than topk of them                           (GeMV / mv_bpr)
//   sparse[sparse_indptr[s]+bos+i] = the i-th best of those pages (topK)
// and writes q_mean and the scores as well, so both stay observable.
//
// Why fused: at decode batch sizes each of the three kernels is dominated by
// its launch and its chain of dependent memory round trips, not by bytes.
// Here the chain is: segment bounds -> one coalesced load of the pass's page
// ids -> centroid rows (the only bulk traffic, 2*D bytes per page) -> LDS
// select -> stores.  The scores never leave the chip for the select and,
// for segments that fit the LDS row cache, neither do the winners' page ids.
//
// The layer's decode CMean (vtx_indexer_fused_cmean): the page-finish mean
// of the pages the step's tokens close runs in the same launch.  Every wave
// reads loc first (at most 256 entries, held in registers: no LDS, no
// barrier) and after its passes reduces its share of the closed tiles with
// the page-reduce kernel's own code (vtx_page_reduce.h); a scored page whose
// centroid this CMean rewrites (a closed page that is a middle page: eos = 0,
// or loc entries of earlier pages) is scored after the loop against the
// centroid recomputed from its K tile, the bits the separate launches give.
//
// Row scoring: a segment's middle pages are split evenly over the waves, at
// most kPass pages per wave pass (64 for rows of one 16-byte vector per lane,
// 32 for wider rows), LPR lanes x VPL 16-byte vectors per row.  The per-lane
// dot product (vtx::dot_row) and the reduce-scatter tree over the LPR lanes
// are the ones gemv.hip uses, so the scores are bit-identical to the GeMV
// kernel's for the same query.
#include <algorithm>

#include "vtx_device.h"
#include "vtx_fused_schedule.h"
#include "vtx_host.h"
#include "vtx_cmean.h"
#include "vtx_page_reduce.h"
#include "vtx_score.h"
#include "vtx_select.h"

namespace {


struct FusedArgs {
  const uint16_t* q;  // [S, G, D] when G > 0
  int32_t G;
  float inv_g;        // torch's mean factor (1 / G, as torch rounds it)
  const uint16_t* x;  // [S, D] when G == 0
  uint16_t* x_out;    // q_mean [S, D], optional
  int64_t q_rows;     // S
  const uint16_t* y;
  int64_t y_rows;
  uint16_t* score;
  int64_t score_len;
  const int32_t* dindptr;
  const int32_t* sindptr;
  const int32_t* didx;
  int64_t didx_len;
  int32_t* sidx;
  int64_t sidx_len;
  int32_t topk, bos, eos;
  int32_t dim;
  int32_t row_cap;   // segments up to this many middle pages are held in LDS
  int32_t segments;  // eff_batch_size; the grid covers all q_rows
  const int32_t* sched;  // the planner's workgroup schedule (vtx_fused_schedule.h), or null
  // split layout: per segment, kStageLists lists of kStageListLen staged
  // (composite << 32 | row id) winners, one per chunk workgroup, or null (no
  // staging)
  uint64_t* stage;
};

// The staging zone of the split layout's pre-selection: kStageLists lists
// of kStageListLen entries for each of up to kStageMaxSegments segments, at
// the end of the caller's workspace (kStageZoneInts int32, two of them
// slack for the 8-byte alignment).  Its place depends only on the
// workspace's length, so no call's counters (at the workspace's start, at
// most length - kStageZoneInts of them) ever overlap lists an earlier call
// staged, whatever the segment counts of the two calls.
constexpr int kStageLists = 16;        // staged lists per segment: chunk workgroups that pre-select
constexpr int kStageListLen = 64;      // entries per list (k <= 64)
constexpr int kStageMaxSegments = 512;  // segments of a call that stages (the split layout's range)
constexpr long long kStageZoneInts = (long long)kStageMaxSegments * kStageLists * kStageListLen * 2 + 2;

constexpr int kMaxQueryDim = 576;  // the widest supported head_dim

// The bf16 mean of the G query rows at qb ([G, D]) for every column, in
// torch.mean(dim=1)'s order (its reduction over a strided dimension keeps
// four fp32 accumulators, row g going to accumulator g % 4 in increasing g,
// each starting from 0, combined as ((a0 + a1) + a2) + a3, then times the
// factor inv_g), into qm (LDS row of D bf16) and, when `store`, into x_out
// row `row`.  Two threads share 16-byte column vector c < D / 8: thread c
// keeps accumulators 0 and 1, thread D / 8 + c accumulators 2 and 3 and
// hands them over through `part` (LDS, D / 8 rows of 16 floats); each loads its 8
// rows of a round of 16 before adding any, so up to 16 rows take one memory
// round trip.  Every thread of the workgroup calls it (it holds a barrier);
// qm is complete after the caller's next barrier.
constexpr int kMeanRowsIn = 8;  // rows per thread loaded before any is added
constexpr int kMeanPartStride = 17;  // floats per column in `part`: 16, padded off the LDS banks' period

__device__ __forceinline__ void query_mean_lds(const FusedArgs& a, const uint16_t* qb, int row, bool store,
                                               uint16_t* qm, float (*part)[kMeanPartStride]) {
  const int D = a.dim;
  const int nv = D / 8;
  for (int base = 0; base < 2 * nv; base += blockDim.x) {  // the same trip count in every thread
    const int t = base + (int)threadIdx.x;
    const bool on = t < 2 * nv;
    const int h = t < nv ? 0 : 1;  // accumulators 2h, 2h + 1
    const int c = on ? t - h * nv : 0;
    float acc[2][8];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
    if (on) {
      for (int g0 = 0; g0 < a.G; g0 += 2 * kMeanRowsIn) {
        // row g0 + 4 (j / 2) + 2h + j % 2 goes to accumulator j % 2; rows
        // past G re-read row G - 1 and are not added (a select, not a
        // branch, which would let the compiler wait for each row alone)
        vtx::U4 r[kMeanRowsIn];
#pragma unroll
        for (int j = 0; j < kMeanRowsIn; ++j) {
          const int g = g0 + 4 * (j / 2) + 2 * h + j % 2;
          r[j] = vtx::ld16(qb + (long long)(g < a.G ? g : a.G - 1) * D + c * 8);
        }
#pragma unroll
        for (int j = 0; j < kMeanRowsIn; ++j) {
          const bool in = g0 + 4 * (j / 2) + 2 * h + j % 2 < a.G;
          float f[8];
          vtx::unpack8(r[j], f);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[j % 2][e] = in ? acc[j % 2][e] + f[e] : acc[j % 2][e];
        }
      }
      if (h == 1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          part[c][e] = acc[0][e];
          part[c][8 + e] = acc[1][e];
        }
      }
    }
    __syncthreads();
    if (on && h == 0) {
      uint32_t b[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        b[e] = vtx::f32_to_bf16((((acc[0][e] + acc[1][e]) + part[c][e]) + part[c][8 + e]) * a.inv_g);
      const vtx::U4 m{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
      vtx::st16(qm + c * 8, m);
      if (store && a.x_out) vtx::st16(a.x_out + (long long)row * D + c * 8, m);
    }
    if (base + (int)blockDim.x < 2 * nv) __syncthreads();  // `part` is read before the next round writes it
  }
}

// query_mean_lds in two halves, for a mean of one round (G <= 2 *
// kMeanRowsIn rows, 2 * D / 8 threads at most the workgroup's): issue loads
// the thread's rows, finish adds them and completes the mean with
// query_mean_lds's arithmetic in its order (the same bits), so that the
// caller can issue other loads in between, which then share the round trip.
struct MeanLoads {
  vtx::U4 r[kMeanRowsIn];
};

__device__ __forceinline__ bool query_mean_one_round(const FusedArgs& a) {
  return a.G <= 2 * kMeanRowsIn && 2 * (a.dim / 8) <= (int)blockDim.x;
}

// Every thread issues its loads (threads past 2 * D / 8 read column 0 again
// and do not use it): no branch, so the count of loads in flight is the same
// on every path and a later wait for these rows waits for nothing issued
// after them.
__device__ __forceinline__ void query_mean_issue(const FusedArgs& a, const uint16_t* qb, MeanLoads& ml) {
  const int D = a.dim;
  const int nv = D / 8;
  const int t = (int)threadIdx.x;
  const bool on = t < 2 * nv;
  const int h = on && t >= nv ? 1 : 0;
  const int c = on ? t - h * nv : 0;
#pragma unroll
  for (int j = 0; j < kMeanRowsIn; ++j) {
    const int g = 4 * (j / 2) + 2 * h + j % 2;
    ml.r[j] = vtx::ld16(qb + (long long)(g < a.G ? g : a.G - 1) * D + c * 8);
  }
}

__device__ __forceinline__ void query_mean_finish(const FusedArgs& a, const MeanLoads& ml, int row, bool store,
                                                  uint16_t* qm, float (*part)[kMeanPartStride]) {
  const int D = a.dim;
  const int nv = D / 8;
  const int t = (int)threadIdx.x;
  const bool on = t < 2 * nv;
  const int h = on && t >= nv ? 1 : 0;
  const int c = on ? t - h * nv : 0;
  // (added in every thread, so that no use of the loads sits in a branch the
  // compiler could move them into)
  float acc[2][8];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
#pragma unroll
  for (int j = 0; j < kMeanRowsIn; ++j) {
    const bool in = 4 * (j / 2) + 2 * h + j % 2 < a.G;
    float f[8];
    vtx::unpack8(ml.r[j], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j % 2][e] = in ? acc[j % 2][e] + f[e] : acc[j % 2][e];
  }
  if (on && h == 1) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      part[c][e] = acc[0][e];
      part[c][8 + e] = acc[1][e];
    }
  }
  __syncthreads();
  if (on && h == 0) {
    uint32_t b[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      b[e] = vtx::f32_to_bf16((((acc[0][e] + acc[1][e]) + part[c][e]) + part[c][8 + e]) * a.inv_g);
    const vtx::U4 m{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
    vtx::st16(qm + c * 8, m);
    if (store && a.x_out) vtx::st16(a.x_out + (long long)row * D + c * 8, m);
  }
}

// Query row of segment `seg` for this lane's columns: the bf16-rounded
// fp32 mean of its G rows (torch's mean), or the row itself when G == 0.
// Lanes with `store` set (one lane group per row) also write the mean to x_out.
// The rows come from qv when q_in_regs (G <= kQRegs; G == 0: the row in
// qv[0]), else from qb; kRegsOnly: callers that only get here with them in
// qv (the scoring loop), so no address into q stays live across it.
template <int LPR, int VPL, int kQRegs, bool kRegsOnly = false>
__device__ __forceinline__ void query_row(const FusedArgs& a, const vtx::U4 (&qv)[kQRegs][VPL],
                                          bool q_in_regs, const uint16_t* qb, int seg, bool store,
                                          int col, float (&xs)[VPL][8]) {
  if constexpr (kRegsOnly) q_in_regs = true;
  const int D = a.dim;
  if (a.G > 0) {
#pragma unroll
    for (int v = 0; v < VPL; ++v)
#pragma unroll
      for (int e = 0; e < 8; ++e) xs[v][e] = 0.f;
    for (int g = 0; g < a.G; ++g) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        vtx::U4 t;
        if (q_in_regs) {
          t = qv[0][v];
#pragma unroll
          for (int gg = 1; gg < kQRegs; ++gg)
            if (gg == g) t = qv[gg][v];
        } else {
          t = vtx::ld16(qb + (long long)g * D + (v * LPR + col) * 8);
        }
        xs[v][0] += vtx::bf16_lo(t.x);
        xs[v][1] += vtx::bf16_hi(t.x);
        xs[v][2] += vtx::bf16_lo(t.y);
        xs[v][3] += vtx::bf16_hi(t.y);
        xs[v][4] += vtx::bf16_lo(t.z);
        xs[v][5] += vtx::bf16_hi(t.z);
        xs[v][6] += vtx::bf16_lo(t.w);
        xs[v][7] += vtx::bf16_hi(t.w);
      }
    }
    uint32_t mb[VPL][8];
#pragma unroll
    for (int v = 0; v < VPL; ++v)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        mb[v][e] = vtx::f32_to_bf16(xs[v][e] * a.inv_g);
        xs[v][e] = vtx::bf16_to_f32(mb[v][e]);
      }
    if (store && a.x_out) {
      uint16_t* xo = a.x_out + (long long)seg * D;
#pragma unroll
      for (int v = 0; v < VPL; ++v)
        vtx::st16(xo + (v * LPR + col) * 8,
                  vtx::U4{mb[v][0] | (mb[v][1] << 16), mb[v][2] | (mb[v][3] << 16),
                          mb[v][4] | (mb[v][5] << 16), mb[v][6] | (mb[v][7] << 16)});
    }
  } else {
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const vtx::U4 t = q_in_regs ? qv[0][v] : vtx::ld16(qb + (v * LPR + col) * 8);
      xs[v][0] = vtx::bf16_lo(t.x);
      xs[v][1] = vtx::bf16_hi(t.x);
      xs[v][2] = vtx::bf16_lo(t.y);
      xs[v][3] = vtx::bf16_hi(t.y);
      xs[v][4] = vtx::bf16_lo(t.z);
      xs[v][5] = vtx::bf16_hi(t.z);
      xs[v][6] = vtx::bf16_lo(t.w);
      xs[v][7] = vtx::bf16_hi(t.w);
    }
  }
}

// One workgroup per segment.  When every wave scores at most one pass (the
// segment has at most waves * kPass middle pages: all of C2), each score
// stays in the register of the lane that produced it and the selection runs
// on those registers (vtx::select_regs); longer segments keep their keys in
// LDS (or re-read their stored scores) and use vtx::select_topk_counted.
//
// The operands of the first loads (the schedule, loc and their sizes) come
// again as leading scalar arguments, ahead of the argument structs: the
// build preloads leading scalar kernel arguments into SGPRs
// (-amdgpu-kernarg-preload-count), so these loads issue with the wave's
// first instructions rather than after a kernel-argument round trip.
template <int T, int LPR, int VPL, int kCmRegs>
__global__ __launch_bounds__(T, (VPL == 1 ? 4 : 2)) void indexer_fused_kernel(const int32_t* sched,
                                                                               const int64_t* loc,
                                                                               int32_t segments, int32_t loc_n,
                                                                               FusedArgs a, vtx::CmArgs cma) {
  constexpr int kWaves = T / vtx::kWave;
  constexpr int kRowsPerLoad = vtx::kWave / LPR;
  constexpr int kPass = vtx::segment_pass<VPL>();
  constexpr int kQRegs = VPL <= 2 ? 2 : 1;  // query rows prefetched
  // one pass per wave, one position per lane: the register selection
  constexpr bool kRegSelect = VPL == 1 && (LPR == 8 || LPR == 16) && kPass / kRowsPerLoad == LPR;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ vtx::SelectShared<T> sh;
  __shared__ vtx::BitonicShared<T> bsh;  // kRegSelect with k <= 32: the bitonic select
  __shared__ __align__(16) uint16_t qm_row[VPL * LPR * 8];  // query mean, G > kQRegs
  __shared__ float qm_part[VPL * LPR][kMeanPartStride];      // its second half's accumulators

  const int tid = threadIdx.x;
  const int lane = vtx::lane_id();
  const int wave = vtx::uniform(tid / vtx::kWave);
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int k = a.topk;
  const int D = a.dim;
  const bool store_mean = wave == 0 && grp == 0;
  // kCmRegs > 0: this launch runs the layer's CMean over up to 64 * kCmRegs loc entries
  constexpr bool cm_on = kCmRegs > 0 && VPL == 1;
  constexpr int kLocRegs = kCmRegs > 0 ? kCmRegs : 1;

  // ---- 0. with the in-kernel CMean, loc (issued first, so that waiting for
  // it waits for nothing else)
  long long cm_pos[kLocRegs];
  if constexpr (cm_on) vtx::closing_load(loc, loc_n, cm_pos);

  // ---- 1. this workgroup's segment and its bounds: from the planner's
  // schedule when its header names this launch (the bounds it holds are a
  // prediction, checked against the block tables below), else segment
  // blockIdx.x and the block tables
  const vtx::SchedPick pick = vtx::sched_pick(sched, segments);
  const int seg = pick.seg;
  const bool predicted = pick.predicted;
  const int tile_rank = pick.tile_rank;  // this workgroup's share of the CMean tiles
  const int32_t* pe = pick.pe;           // predicted dense begin, dense end, sparse begin
  const bool is_seg = seg < segments;
  long long start = 0, n = 0, obase = 0;
  if (predicted) {
    start = (long long)pe[0] + a.bos;
    n = (long long)pe[1] - a.eos - start;
    obase = (long long)pe[2] + a.bos;
  } else if (is_seg) {
    start = (long long)a.dindptr[seg] + a.bos;
    n = (long long)a.dindptr[seg + 1] - a.eos - start;
    obase = (long long)a.sindptr[seg] + a.bos;
  }

  // ---- 2. query rows (issued early: only needed once centroid rows arrive;
  // G == 0: the averaged row itself, in qv[0])
  vtx::U4 qv[kQRegs][VPL];
  const bool q_in_regs = a.G <= kQRegs;
  const int q_rows_in = a.G > 0 ? a.G : 1;
  const uint16_t* qb = a.G > 0 ? a.q + (long long)seg * a.G * D : a.x + (long long)seg * D;
  if (q_in_regs) {
    // rows past G load row G - 1 again (query_row reads only the first G):
    // no branch around a load, so nothing waits for them here
#pragma unroll
    for (int g = 0; g < kQRegs; ++g)
#pragma unroll
      for (int v = 0; v < VPL; ++v)
        qv[g][v] = vtx::ld16(qb + (long long)(g < q_rows_in ? g : q_rows_in - 1) * D + (v * LPR + col) * 8);
  }

  vtx::Closing<kLocRegs> closing{};
  int n_close = 0;
  auto is_active = [&]() {
    return is_seg && k > 0 && n > k && start >= 0 && start + n <= a.score_len && start + n <= a.didx_len &&
           obase >= 0 && obase + k <= a.sidx_len;
  };
  bool active = is_active();
  uint64_t* sel = reinterpret_cast<uint64_t*>(smem);
  int32_t* rows = reinterpret_cast<int32_t*>(smem + (size_t)vtx::sel_slots(k) * sizeof(uint64_t));
  uint16_t* keys = reinterpret_cast<uint16_t*>(rows + a.row_cap);
  int32_t* sel_pay = reinterpret_cast<int32_t*>(keys + a.row_cap);  // select_regs' payloads

  float xs[VPL][8];
  // The pages are split evenly over the waves (one pass each up to
  // kWaves * kPass pages, so no wave waits on a second round trip while
  // others idle); row ids come straight from global memory.
  long long share = 0, p0 = 0;
  int my_row = -1;  // row ids of the first pass, requested before the CMean tiles
  auto first_pass = [&]() {
    share = (n + kWaves - 1) / kWaves;
    share = (share + kRowsPerLoad - 1) / kRowsPerLoad * kRowsPerLoad;
    if (share > kPass) share = kPass;
    p0 = (long long)wave * share;
    my_row = -1;
    if (p0 < n) {
      const int cnt = (int)min(share, n - p0);
      my_row = lane < cnt ? a.didx[start + p0 + lane] : -1;
    }
  };
  // The row ids, then the segment's bounds from the block tables (the check
  // of the prediction: one vector load, lane 0 dense begin, lane 1 dense
  // end, lane 2 sparse begin) are requested before the barrier, and nothing
  // waits for them before it: both come back in one round trip, and the
  // barrier does not hold a wave whose loads are back for the others'.
  if (active) first_pass();  // uniform
  const int32_t* bp = lane == 1 ? a.dindptr + seg + 1 : lane == 2 ? a.sindptr + seg : a.dindptr + seg;
  const int32_t bv = predicted ? *bp : 0;
  // The radix selects count into the LDS histogram, which is cleared first
  // (one barrier); the bitonic select of one-pass segments counts nothing,
  // so there the waves go on to their rows without waiting for each other.
  auto needs_hist = [&]() {
    return !(kRegSelect && n <= (long long)kWaves * kPass && k <= vtx::kMaxBitonicK && n <= a.row_cap);
  };
  bool hist = active && needs_hist();  // uniform
  if (hist) {
    vtx::select_init<T>(sel, k, sh);
    __syncthreads();  // histogram cleared before any wave counts into it
  }
  int32_t tb[3] = {pe[0], pe[1], pe[2]};
  if (predicted) {  // uniform
    tb[0] = __builtin_amdgcn_readlane(bv, 0);
    tb[1] = __builtin_amdgcn_readlane(bv, 1);
    tb[2] = __builtin_amdgcn_readlane(bv, 2);
  }
  // The pages this launch's CMean closes (its tiles are reduced at the end
  // of the workgroup, see cm_tiles)
  if constexpr (cm_on) {
    closing = vtx::closing_build(cma, cm_pos);
    n_close = closing.count;
  }
  // This launch's CMean: wave w of the workgroup of tile rank r reduces tiles
  // w * grid + r, + waves * grid, ... (one tile per wave 0 for up to `grid`
  // tiles), after its own segment is done; under a schedule rank 0 is the
  // workgroup with the shortest segment, so the tiles go to the workgroups
  // that finish first, while the long segments still stream.  A page whose
  // centroid it rewrites is scored against the centroid recomputed from its
  // K tile, so the order against other workgroups' reads does not matter.
  auto cm_tiles = [&]() {
    if constexpr (cm_on)
      vtx::cmean_tiles<LPR, kLocRegs, vtx::kCentroid>(cma, closing, wave * (int)gridDim.x + tile_rank,
                                                       kWaves * (int)gridDim.x, grp, col);
  };
  // (bitwise, not short-circuit: a load behind || would wait for the others)
  if (predicted & ((tb[0] != pe[0]) | (tb[1] != pe[1]) | (tb[2] != pe[2]))) {  // uniform; not for a current schedule
    start = (long long)tb[0] + a.bos;
    n = (long long)tb[1] - a.eos - start;
    obase = (long long)tb[2] + a.bos;
    active = is_active();
    if (active) {
      if (!hist && needs_hist()) {
        vtx::select_init<T>(sel, k, sh);
        __syncthreads();
        hist = true;
      }
      first_pass();
    }
  }
  if (!active) {
    if (a.x_out) {
      if (q_in_regs) query_row<LPR, VPL, kQRegs>(a, qv, q_in_regs, qb, seg, store_mean, col, xs);
      else query_mean_lds(a, qb, seg, true, qm_row, qm_part);
    }
    cm_tiles();
    return;
  }
  const bool cached = n <= a.row_cap;
  const int32_t* dseg = a.didx + start;

  bool have_mean = false;
  if (!q_in_regs) {  // (more than kQRegs rows to average: formed in LDS, before the loop)
    query_mean_lds(a, qb, seg, true, qm_row, qm_part);
    __syncthreads();
#pragma unroll
    for (int v = 0; v < VPL; ++v) vtx::unpack8(vtx::ld16(qm_row + (v * LPR + col) * 8), xs[v]);
    have_mean = true;
  }

  if constexpr (kRegSelect) {
    if (n <= (long long)kWaves * kPass) {  // uniform: at most one pass per wave
      // k <= 32 with the row ids in LDS: the bitonic select; else the radix
      // select on registers (select_regs)
      const bool bitonic = k <= vtx::kMaxBitonicK && n <= a.row_cap;  // uniform
      bool have = false, deferred = false;
      uint32_t key = 0;
      int rid = -1, r = -1;
      if (p0 < n) {  // uniform
        const int cnt = (int)min(share, n - p0);
        if (!have_mean) {
          query_row<LPR, VPL, kQRegs, true>(a, qv, q_in_regs, qb, seg, store_mean, col, xs);
          have_mean = true;
        }
        const float sc = vtx::score_pass<LPR, VPL, kPass>(a.y, a.y_rows, a.dim, my_row, cnt, xs, grp, col, &r);
        rid = __shfl(my_row, r < 0 ? 0 : r, vtx::kWave);  // row id of this lane's page
        if (r >= 0) {
          if (cm_on && n_close > 0 && vtx::closes_here(cma, closing, r, rid)) {
            deferred = true;  // this launch's CMean rewrites the page's centroid
          } else {
            const uint32_t sb = vtx::f32_to_bf16(sc);
            key = vtx::score_key(sb);
            a.score[start + p0 + r] = (uint16_t)sb;
            if (!bitonic) vtx::select_count<T>(key, sh);
            have = true;
          }
        }
      }
      if constexpr (cm_on) {  // this wave's pages with a rewritten centroid, one at a time
        uint64_t m = __ballot(deferred);
        while (m) {  // uniform
          const int l = __ffsll((long long)m) - 1;
          m &= m - 1;
          const int fr = __builtin_amdgcn_readlane(rid, l);
          const float f = vtx::score_vec<LPR>(vtx::fresh_centroid<LPR>(cma, fr, grp, col), xs);
          if (lane == l) {
            const uint32_t sb = vtx::f32_to_bf16(f);
            key = vtx::score_key(sb);
            a.score[start + p0 + r] = (uint16_t)sb;
            if (!bitonic) vtx::select_count<T>(key, sh);
            have = true;
          }
        }
      }
      if (bitonic) {
        if (have) rows[p0 + r] = rid;  // payload by position (visible after the select's first barrier)
        vtx::select_bitonic<T>(vtx::bitonic_comp(have, key, (int)(p0 + r)), k, bsh, [&](int rank, uint32_t c) {
          a.sidx[obase + rank] = rows[vtx::bitonic_position(c)];
        });
      } else {
        __syncthreads();  // every key counted
        vtx::select_regs<T, LPR>(have, key, p0 + r, rid, k, sel, sel_pay, sh,
                                 [&](int rank, int payload) { a.sidx[obase + rank] = payload; });
      }
      cm_tiles();
      return;
    }
  }

  // ---- 4. scores of longer segments: several passes per wave; keys and row
  // ids cached in LDS (or the stored scores re-read).  The query mean is
  // formed first, so the raw query rows are dead inside the loop.
  if (!have_mean) {
    query_row<LPR, VPL, kQRegs, true>(a, qv, q_in_regs, qb, seg, store_mean, col, xs);
    have_mean = true;
  }
  for (bool first = true; p0 < n; p0 += (long long)kWaves * share, first = false) {
    const int cnt = (int)min(share, n - p0);
    // one coalesced load of the pass's row ids (lane l holds position l)
    if (!first) my_row = lane < cnt ? dseg[p0 + lane] : -1;
    int r;
    float sc = vtx::score_pass<LPR, VPL, kPass>(a.y, a.y_rows, a.dim, my_row, cnt, xs, grp, col, &r);
    const int my_rid = __shfl(my_row, r < 0 ? 0 : r, vtx::kWave);  // row id of this lane's page
    if constexpr (cm_on) {
      if (n_close > 0) {  // uniform
        // pages whose centroid this launch's CMean rewrites: scored against
        // the centroid recomputed from the K tile, one at a time per wave
        uint64_t m = __ballot(vtx::closes_here(cma, closing, r, my_rid));
        while (m) {  // uniform
          const int l = __ffsll((long long)m) - 1;
          m &= m - 1;
          const int fr = __builtin_amdgcn_readlane(my_rid, l);
          const float f = vtx::score_vec<LPR>(vtx::fresh_centroid<LPR>(cma, fr, grp, col), xs);
          if (lane == l) sc = f;
        }
      }
    }
    if (r >= 0) {
      const uint32_t sb = vtx::f32_to_bf16(sc);
      const uint32_t key = vtx::score_key(sb);
      a.score[start + p0 + r] = (uint16_t)sb;
      if (cached) {
        keys[p0 + r] = (uint16_t)key;
        rows[p0 + r] = my_rid;
      }
      vtx::select_count<T>(key, sh);
    }
  }
  __syncthreads();

  // ---- 5. top-k of the segment
  if (cached) {
    vtx::select_topk_counted<T>([&](long long i) { return (uint32_t)keys[i]; }, n, k, sel, sh);
  } else {
    const uint16_t* sc = a.score + start;  // this workgroup's own stores
    vtx::select_topk_counted<T>([&](long long i) { return vtx::score_key(sc[i]); }, n, k, sel, sh);
  }
  vtx::select_emit<T>(sel, k, n, [&](int r, long long pos) { a.sidx[obase + r] = cached ? rows[pos] : dseg[pos]; });
  cm_tiles();
}

// Stores / loads performed at device scope (every XCD sees them once the
// store has completed; no copy in a non-coherent cache is used).
template <typename V>
__device__ __forceinline__ void store_coherent(V* p, V v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename V>
__device__ __forceinline__ V load_coherent(const V* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A device-scope fetch-add of 1 by one lane, its result waited for only
// where it is used: the address is passed through a VGPR, so the compiler's
// atomic optimizer (which combines the active lanes' adds into one and
// waits for its result right away to hand each lane its share) leaves it
// alone and the round trip overlaps the work that follows.
__device__ __forceinline__ int fetch_add_one_deferred(int32_t* p) {
  asm volatile("" : "+v"(p));
  // (a global-memory pointer again: a flat atomic would also hold up the
  // next wait for LDS)
  auto* g = (__attribute__((address_space(1))) int32_t*)p;
  return __hip_atomic_fetch_add(g, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Histogram copies of the split layout's selection (vtx::SelectShared).
constexpr int kSplitHistCopies = 8;

// Tries of the selecting workgroup's wait for a staged entry (each a
// device-scope load and a short sleep, about a microsecond): the entries it
// waits for are stored by workgroups that counted in before it and store
// them right after their select, so the bound is only a guard; an entry it
// gives up on counts as no item, and its rank's output is -1.
constexpr int kStageSpins = 1 << 16;

// The split layout's final select over the staged lists at `lists` (list j
// at j * kStageListLen: the best cnt_j = min(k, pages of chunk j) of chunk
// j, descending, composites in the high half, row ids in the low half; a
// staged entry is never 0): the k best of the workers lists, emit(rank,
// composite) for rank 0 .. k-1 (from wave 0, composite 0 for a rank without
// an item); each row id goes to rid_lds at its composite's segment position.
// List `own` (this workgroup's) was not stored and is read from own_lds; the
// other lists may still be on their way (every list place is 0 until its
// workgroup stores it): an entry that is still 0 is loaded again.  Every
// entry read from the zone is cleared after it is read, so the zone is all
// zero again when the launch ends.
// Lane l of wave w holds the elements g = (w * 64 + l) * kR + u, element g
// being place g % lk of list g / lk (lk = k rounded up to a power of two, so
// the lists are sorted runs of lk elements), every other list reversed when
// a wave holds several, so that the bitonic sort starts at runs of 2 * lk.
// Every thread of the workgroup calls it (it holds barriers).
template <int T, int kR, typename Emit>
__device__ __forceinline__ void merge_staged(uint64_t* lists, int workers, int own, const uint64_t* own_lds, int k,
                                             int lk, long long n, int chunk, int32_t* rid_lds,
                                             vtx::BitonicRunShared<T>& bs, vtx::BitonicShared<T>& bs32, Emit emit) {
  const int lane = vtx::lane_id();
  const int wave = vtx::uniform(threadIdx.x / vtx::kWave);
  const bool alternate = vtx::kWave * kR >= 2 * lk;
  uint64_t e[kR];
  int at[kR];    // list * kStageListLen + place of an entry to read from the zone, else -1
  int kept[kR];  // place in own_lds of this workgroup's entry, else -1
#pragma unroll
  for (int u = 0; u < kR; ++u) {  // every load issued before any is used (list 0, place 0 always exists)
    const int g = (wave * vtx::kWave + lane) * kR + u;
    const int list = g / lk, p = g % lk;
    const int place = (alternate && (list & 1)) ? lk - 1 - p : p;
    const bool ok = list < workers && place < k && place < n - (long long)list * chunk;
    const bool mine = list == own;
    at[u] = ok && !mine ? list * kStageListLen + place : -1;
    kept[u] = ok && mine ? place : -1;
    e[u] = load_coherent(lists + (at[u] >= 0 ? at[u] : 0));
  }
  // then the own list's entries, and the wait for entries not yet stored
  // (the LDS reads come after every load has been issued, so that a read the
  // compiler puts in a branch does not hold up the loads after it)
#pragma unroll
  for (int u = 0; u < kR; ++u) {
    if (kept[u] >= 0) e[u] = own_lds[kept[u]];
    else if (at[u] < 0) e[u] = 0;
    else
      for (int t = 0; e[u] == 0 && t < kStageSpins; ++t) {
        __builtin_amdgcn_s_sleep(2);
        e[u] = load_coherent(lists + at[u]);
      }
  }
  uint32_t comp[kR];
#pragma unroll
  for (int u = 0; u < kR; ++u) {
    comp[u] = (uint32_t)(e[u] >> 32);
    if (comp[u]) rid_lds[vtx::bitonic_position(comp[u])] = (int32_t)(uint32_t)e[u];
  }
  // cleared after the row ids' LDS writes, which would otherwise wait for
  // these stores
#pragma unroll
  for (int u = 0; u < kR; ++u)
    if (at[u] >= 0) store_coherent(lists + at[u], (uint64_t)0);
  const int run = alternate ? lk : vtx::kWave * kR;
  if constexpr (kR == 1) {  // (lists of 32 where k <= 32: one register per lane in the merges)
    if (k <= vtx::kMaxBitonicK) {
      vtx::select_bitonic<T>(comp[0], k, bs32, emit, run);
      return;
    }
  }
  vtx::select_bitonic_run<T, kR>(comp, k, bs, emit, run);
}

// Split segments: a segment's middle pages are dealt, kChunk = kWaves * kPass
// at a time, to `cps` workgroups (chunk c takes chunks c, c + cps, ...).  Each
// workgroup scores its pages and stores the scores; the one that counts in
// last (per-segment arrival counter in `counters`) selects the top-k, from
// the stored scores or, for a staged segment, from the chunks' pre-selected
// lists.  No workgroup waits for one that has not counted in: an unstaged
// segment's workgroups wait for nobody, and a staged segment's selecting
// workgroup waits only for lists of workgroups that counted in before it
// (running, and waiting for nobody), so every workgroup runs to completion.
// The last one resets the counter to zero for the next launch.
//
// Work ids are laid out XCD by XCD (workgroup b runs on XCD b % 8), so the
// chunks of one segment usually share an L2 and the selecting workgroup reads
// the other chunks' scores from it.
//
// The query mean of more than kQRegs rows is formed once per workgroup in
// LDS (query_mean_lds).  With kCmRegs > 0 the layer's decode CMean runs in
// the launch: tile t of the closed pages is reduced by wave t % waves of
// work id t / waves once that workgroup's scores are counted in, with the
// page-reduce launch's arithmetic for the row width, and a scored page whose
// centroid the launch rewrites is scored against the centroid recomputed
// from its K tile (reduced into the wave's LDS row, read back in the scoring
// layout).
//
// As in indexer_fused_kernel, the operands of the first loads (the block
// tables' bounds, loc and the sizes the work id needs, gridDim.x / 8
// included: the grid size is itself a kernel argument) lead the argument
// list, so that they are preloaded into SGPRs.  Rows of one vector per lane
// ask for four waves per SIMD (at most 128 VGPRs), so that 16 waves of
// split workgroups fit a CU, as the host's chunk sizing assumes.
template <int T, int LPR, int VPL, int kPass, int kCmRegs>
__global__ __launch_bounds__(T, (VPL == 1 ? 4 : 1)) void indexer_split_kernel(const int32_t* dindptr,
                                                                              const int32_t* sindptr,
                                                          const int64_t* loc, int32_t segments, int32_t loc_n,
                                                          int32_t cps, int32_t per_xcd, FusedArgs a,
                                                          int32_t* counters, vtx::CmArgs cma) {
  constexpr int kWaves = T / vtx::kWave;
  constexpr int kRowsPerLoad = vtx::kWave / LPR;
  constexpr int kChunk = kWaves * kPass;
  constexpr int kQRegs = VPL <= 2 ? 2 : 1;
  constexpr int kTailR = 8;  // scores per thread the selecting workgroup holds in registers
  constexpr bool cm_on = kCmRegs > 0;
  constexpr int kLocRegs = kCmRegs > 0 ? kCmRegs : 1;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ vtx::SelectShared<T, kSplitHistCopies> sh;
  __shared__ vtx::BitonicRunShared<T> bsr;  // the selecting workgroup's bitonic select
  __shared__ int s_last;
  __shared__ vtx::BitonicShared<T> bs32;                 // staged selects of k <= 32 (lists of 32)
  __shared__ uint64_t own_list[kStageListLen];             // staged: the selecting workgroup's own list
  __shared__ __align__(16) uint16_t qm_row[kMaxQueryDim];                      // query mean, G > kQRegs
  __shared__ float qm_part[VPL * LPR][kMeanPartStride];                        // its second half's accumulators
  __shared__ __align__(16) uint16_t fresh_row[cm_on && VPL > 1 ? kWaves * kMaxQueryDim : 8];  // per wave, CMean

  const int tid = threadIdx.x;
  const int lane = vtx::lane_id();
  const int wave = vtx::uniform(tid / vtx::kWave);
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int k = a.topk;
  const int D = a.dim;

  long long cm_pos[kLocRegs];
  if constexpr (cm_on) vtx::closing_load(loc, loc_n, cm_pos);
  // per_xcd = the work ids per XCD (8 * per_xcd workgroups take work ids;
  // the host rounds them to a multiple of 8), passed so that the work id
  // waits for no kernel-argument load
  const long long w = (long long)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  const long long chunk_items = (long long)segments * cps;
  const long long slots = 8LL * per_xcd;
  vtx::Closing<kLocRegs> closing{};
  int n_close = 0;
  // the closed pages of loc (waits for the loc loads: called once the
  // work id's other first loads are issued)
  auto build_closing = [&]() {
    if constexpr (cm_on) {
      closing = vtx::closing_build(cma, cm_pos);
      n_close = closing.count;
    }
  };
  // The CMean's work units (tiles, or parts of wide tiles).  For wide rows
  // (D >= 512) the host appends workgroups of their own past the work ids:
  // they reduce every unit as the launch starts, unit r * waves + wave, +
  // tile workgroups * waves, ..., so no unit waits behind a segment's select
  // or delays one (handed to the work ids after their count-in, a unit landed
  // on a selecting workgroup in some launches and delayed its end by 1-2 us
  // at C5).  Narrower rows (and a grid without them) share the units out
  // over the work ids after their count-in: unit w * waves + wave, + grid *
  // waves, ...
  constexpr bool kTileGroups = cm_on && VPL > 2;
  auto cm_tiles = [&]() {
    if constexpr (cm_on) {
      const bool shared = !kTileGroups || (long long)gridDim.x == slots;
      if (shared && w * kWaves < (long long)n_close * cma.heads * vtx::tile_parts<LPR * VPL>())  // uniform
        vtx::cmean_tiles_any<LPR * VPL, kLocRegs, vtx::kCentroid>(cma, closing, (int)(w * kWaves) + wave,
                                                       (int)gridDim.x * kWaves);
    }
  };
  if constexpr (kTileGroups) {
    if ((long long)blockIdx.x >= slots) {  // uniform: a CMean tile workgroup
      build_closing();
      vtx::cmean_tiles_any<LPR * VPL, kLocRegs, vtx::kCentroid>(
          cma, closing, (int)(blockIdx.x - slots) * kWaves + wave, (int)(gridDim.x - slots) * kWaves);
      return;
    }
  }
  vtx::U4 xq[VPL];  // the query mean as packed bf16 pairs (what the dot steps take)
  vtx::U4 qv[kQRegs][VPL];
  if (w >= chunk_items) {  // query rows past the segments: only their mean
    build_closing();
    const long long row = segments + (w - chunk_items);
    if (a.x_out && a.G > 0 && row < a.q_rows) {
      if (a.G <= kQRegs) {
        float xs[VPL][8];
        query_row<LPR, VPL, kQRegs>(a, qv, false, a.q + row * a.G * D, (int)row, wave == 0 && grp == 0, col, xs);
      } else
        query_mean_lds(a, a.q + row * a.G * D, (int)row, true, qm_row, qm_part);
    }
    cm_tiles();
    return;
  }
  const int seg = (int)(w / cps);
  const int c = (int)(w % cps);
  const bool store_mean = c == 0 && wave == 0 && grp == 0;

  // the segment's bounds in one vector load (lane 0: dense begin, lane 1:
  // dense end, lane 2: sparse begin; one round trip, where three scalar-path
  // loads would each wait for the one before)
  const int32_t* bp = lane == 1 ? dindptr + seg + 1 : lane == 2 ? sindptr + seg : dindptr + seg;
  const int32_t bv = *bp;
  const bool q_in_regs = a.G > 0 && a.G <= kQRegs;
  const uint16_t* qb = a.G > 0 ? a.q + (long long)seg * a.G * D : a.x + (long long)seg * D;
  if (q_in_regs) {  // rows past G load row G - 1 again (query_row reads only the first G)
#pragma unroll
    for (int g = 0; g < kQRegs; ++g)
#pragma unroll
      for (int v = 0; v < VPL; ++v)
        qv[g][v] = vtx::ld16(qb + (long long)(g < a.G ? g : a.G - 1) * D + (v * LPR + col) * 8);
  }
  build_closing();

  const long long start = (long long)__builtin_amdgcn_readlane(bv, 0) + a.bos;
  const long long n = (long long)__builtin_amdgcn_readlane(bv, 1) - a.eos - start;
  const long long obase = (long long)__builtin_amdgcn_readlane(bv, 2) + a.bos;
  bool active = k > 0 && n > k;
  if (active && (start < 0 || start + n > a.score_len || start + n > a.didx_len || obase < 0 ||
                 obase + k > a.sidx_len))
    active = false;
  const long long nchunks = active ? (n + kChunk - 1) / kChunk : 0;
  const int workers = (int)min(nchunks, (long long)cps);  // workgroups that take part
  const bool mean_in_lds = a.G > kQRegs;
  if (c >= workers) {  // nothing to score (or an inactive segment): only the mean
    if (c == 0 && a.x_out) {
      if (mean_in_lds) {
        query_mean_lds(a, qb, seg, true, qm_row, qm_part);
      } else {
        float xs[VPL][8];
        query_row<LPR, VPL, kQRegs>(a, qv, q_in_regs, qb, seg, store_mean, col, xs);
      }
    }
    cm_tiles();
    return;
  }
  uint64_t* sel = reinterpret_cast<uint64_t*>(smem);
  int32_t* sel_pay = reinterpret_cast<int32_t*>(smem + (size_t)vtx::sel_slots(k) * sizeof(uint64_t));
  uint16_t* keys = reinterpret_cast<uint16_t*>(sel_pay + k);
  constexpr int kRunR = 4;  // scores per thread of the tail's bitonic select
  const bool tail_bitonic = k <= vtx::kMaxBitonicRunK && n <= a.row_cap && n <= (long long)T * kRunR;
  const int32_t* dseg = a.didx + start;
  // this wave's positions of chunk ch: [p0, p0 + cnt), none when cnt <= 0
  auto wave_share = [&](long long ch, long long& p0, int& cnt) {
    const long long c0 = ch * kChunk;
    const long long cn = min((long long)kChunk, n - c0);
    long long share = (cn + kWaves - 1) / kWaves;
    share = (share + kRowsPerLoad - 1) / kRowsPerLoad * kRowsPerLoad;
    p0 = c0 + (long long)wave * share;
    cnt = p0 < c0 + cn ? (int)min(share, c0 + cn - p0) : 0;
  };
  // ---- scores of this workgroup's chunks
  // Staged pre-selection: when every workgroup of the segment scores one
  // chunk, k <= 64 and the segment has at most kStageLists chunks, each
  // workgroup selects its chunk's best k itself (its row ids by chunk
  // position in LDS) and stages them as one sorted list, so that the
  // selecting workgroup only merges the lists.  The composites carry the
  // segment position, unique per page, so the merged best k are exactly the
  // segment's best k.  The selecting workgroup then reads only the lists:
  // the scores are stored with ordinary stores (visible when the launch
  // ends), only the lists are written through for the hand-off.
  const bool hier = a.stage != nullptr && seg < kStageMaxSegments && k <= vtx::kMaxBitonicRunK &&
                    nchunks <= cps && workers <= kStageLists && n <= a.row_cap && n <= 0xffff;  // uniform
  // the histograms of the final selection (the radix selects) are cleared
  // now, off its path (the barriers of the arrival order this before the
  // counting); the staged merge and the tail's bitonic select use none
  if (!tail_bitonic && !hier) vtx::select_init<T>(sel, k, sh);
  int32_t* rid_lds = reinterpret_cast<int32_t*>(keys + a.row_cap);  // row ids by position (row_cap entries)
  uint32_t hcomp = 0;  // hier: this lane's composite and its row id
  int hrid = 0;
  // a scored pass at positions p0 + ...: this lane's score sc, at position r
  auto pass_done = [&](long long p0, int my_row, int r, float sc) {
    if constexpr (cm_on) {
      if (n_close > 0) {  // uniform
        // pages whose centroid this launch's CMean rewrites: scored against
        // the centroid recomputed from the K tile, one at a time per wave
        const int my_rid = __shfl(my_row, r < 0 ? 0 : r, vtx::kWave);
        uint64_t m = __ballot(vtx::closes_here(cma, closing, r, my_rid));
        while (m) {  // uniform
          const int l = __ffsll((long long)m) - 1;
          m &= m - 1;
          vtx::U4 cen[VPL];
          vtx::fresh_centroid_rows<LPR, VPL>(cma, __builtin_amdgcn_readlane(my_rid, l),
                                             fresh_row + wave * kMaxQueryDim, grp, col, cen);
          const float f = vtx::score_vec_rows_packed<LPR, VPL>(cen, xq);
          if (lane == l) sc = f;
        }
      }
    }
    const uint16_t sb = (uint16_t)vtx::f32_to_bf16(sc);
    if (r >= 0) {
      if (hier) a.score[start + p0 + r] = sb;  // read by no other workgroup of the launch
      else store_coherent(a.score + start + p0 + r, sb);
    }
    if (hier) {  // uniform
      hrid = __shfl(my_row, r < 0 ? 0 : r, vtx::kWave);
      hcomp = vtx::bitonic_comp(r >= 0, vtx::score_key(sb), (int)(p0 + r));
    }
  };
  // chunks ch0, ch0 + cps, ... with the query mean in xq (have_mean), or
  // formed from qv / qb at the first pass
  auto score_chunks = [&](long long ch0, bool have_mean) {
    for (long long ch = ch0; ch < nchunks; ch += cps) {
      long long p0;
      int cnt;
      wave_share(ch, p0, cnt);
      if (cnt <= 0) continue;  // wave-uniform
      const int my_row = lane < cnt ? dseg[p0 + lane] : -1;
      if (!have_mean) {
        float xs[VPL][8];
        query_row<LPR, VPL, kQRegs>(a, qv, q_in_regs, qb, seg, store_mean, col, xs);
        vtx::pack_query<VPL>(xs, xq);
        have_mean = true;
      }
      int r;
      const float sc = vtx::score_pass_packed<LPR, VPL, kPass>(a.y, a.y_rows, a.dim, my_row, cnt, xq, grp, col, &r);
      pass_done(p0, my_row, r, sc);
    }
  };
  // the mean formed in LDS, read as packed pairs
  auto load_xq = [&]() {
#pragma unroll
    for (int v = 0; v < VPL; ++v) xq[v] = vtx::ld16(qm_row + (v * LPR + col) * 8);
  };
  auto score_all = [&]() {
    if (mean_in_lds) {  // workgroup-uniform
      query_mean_lds(a, qb, seg, c == 0, qm_row, qm_part);
      __syncthreads();
      load_xq();
    }
    score_chunks(c, mean_in_lds);
  };
  // Wide rows and a mean of one round: the query rows and the first chunk's
  // row ids are requested together, the first chunk's rows right after the
  // row ids, and the mean is formed while the rows are in flight (the query
  // loads, issued first, are back before the row loads).  The raw query rows
  // are not held in registers on this path.
  if constexpr (VPL > 2) {
    if (mean_in_lds && query_mean_one_round(a)) {  // uniform
      MeanLoads ml;
      query_mean_issue(a, qb, ml);
      __builtin_amdgcn_sched_barrier(0);  // the query loads stay ahead of the row loads
      long long p0;
      int cnt;
      wave_share(c, p0, cnt);
      // (loaded unconditionally, as the query rows: a wave without pages in
      // the chunk reads position 0's row id and pool row 0 and uses neither)
      const int rid = dseg[lane < cnt ? p0 + lane : 0];
      const int my_row = lane < cnt ? rid : -1;
      vtx::RowLoads<LPR, VPL, kPass> rl;
      vtx::row_issue<LPR, VPL, kPass>(a.y, a.y_rows, a.dim, my_row, grp, col, rl);
      query_mean_finish(a, ml, seg, c == 0, qm_row, qm_part);
      __syncthreads();
      load_xq();
      if (cnt > 0) {  // uniform
        int r;
        const float sc = vtx::row_score<LPR, VPL, kPass>(rl, xq, cnt, grp, col, &r);
        pass_done(p0, my_row, r, sc);
      }
      score_chunks(c + cps, true);
    } else {
      score_all();
    }
  } else {
    score_all();
  }
  // (wave 0 of chunk 0 always has pages, so the mean has been stored)
  // Staged segments: this chunk's best k, handed over as list c of the
  // segment.  The selecting workgroup reads the lists by content: a staged
  // entry is never 0, the zone is all zero between launches (the selecting
  // workgroup clears every entry it reads), and an entry that is still 0 is
  // loaded again, so no store has to have completed when a workgroup counts
  // in.  The count-in goes out before the chunk's select, its round trip
  // hidden by the select; the last one to count in keeps its own list in
  // LDS only and merges.  It only waits for entries of workgroups that
  // counted in before it, each of which stores its list right after its
  // select and waits for nobody: every wait ends.
  if (hier) {  // uniform (c < workers)
    const long long c0 = (long long)c * kChunk;
    if (hcomp) rid_lds[vtx::bitonic_position(hcomp) - c0] = hrid;
    uint64_t* lists = a.stage + (long long)seg * kStageLists * kStageListLen;
    uint64_t* list = lists + (long long)c * kStageListLen;
    int old = 0;
    if (tid == 0) old = fetch_add_one_deferred(&counters[seg]);
    auto hand = [&](int rank, uint32_t cmp) {  // (wave 0; cmp 0: a rank past the chunk's pages)
      const uint64_t e = cmp ? ((uint64_t)cmp << 32) | (uint32_t)rid_lds[vtx::bitonic_position(cmp) - c0] : 0;
      if (__builtin_amdgcn_readlane(old, 0) == workers - 1) own_list[rank] = e;
      else if (cmp) store_coherent(list + rank, e);
    };
    if (k <= vtx::kMaxBitonicK) {
      vtx::select_bitonic<T>(hcomp, k, bs32, hand);  // (lists of 32)
    } else {
      uint32_t cv[1] = {hcomp};
      vtx::select_bitonic_run<T, 1>(cv, k, bsr, hand);
    }
    if (tid == 0) {
      const int last = old == workers - 1;
      if (last) __hip_atomic_store(&counters[seg], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    if (s_last) {
      // entries: workers lists of lk = k rounded up to a power of two
      // places, kR per thread
      const int lk = k <= 1 ? 1 : 1 << (32 - __builtin_clz((unsigned)(k - 1)));
      const int total = workers * lk;
      auto merge = [&](auto kr_tag) {
        constexpr int kR = decltype(kr_tag)::value;
        merge_staged<T, kR>(lists, workers, c, own_list, k, lk, n, kChunk, rid_lds, bsr, bs32,
                            [&](int rank, uint32_t cv) {
                              // (a rank without an item only after a wait given up on)
                              a.sidx[obase + rank] = cv ? rid_lds[vtx::bitonic_position(cv)] : -1;
                            });
      };
      if (total <= T) {
        merge(std::integral_constant<int, 1>{});
      } else if constexpr (T >= 512) {  // (total <= kStageLists * kStageListLen = 2 * 512)
        merge(std::integral_constant<int, 2>{});
      } else {
        if (total <= 2 * T) merge(std::integral_constant<int, 2>{});
        else merge(std::integral_constant<int, 4>{});
      }
    }
    cm_tiles();
    return;
  }

  // ---- arrival (unstaged segments): the last of the `workers` workgroups
  // selects.  This is a release/acquire handoff written out for its one kind
  // of payload: the scores are device-scope atomic stores (written through
  // to the point of coherence, never held dirty in an XCD's L2), and a
  // release then only needs each wave to wait until its own stores have
  // completed (s_waitcnt 0), which happens before the barrier after which
  // one thread counts the workgroup in with a device-scope atomic.  The last
  // workgroup reads them with device-scope atomic loads issued after that
  // count.  The compiler fences keep the compiler from moving memory
  // operations across either side.  (A device-scope release fence or release
  // RMW would also write back the XCD's whole L2 in every workgroup:
  // measured 2.8 to 5.5 times the launch time at C3 and C5.)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (tid == 0) {
    const int old = __hip_atomic_fetch_add(&counters[seg], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = old == workers - 1;
    if (last) __hip_atomic_store(&counters[seg], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) {
    cm_tiles();
    return;
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);

  // ---- top-k of the segment, from the stored scores (device-coherent loads)
  const uint16_t* scs = a.score + start;
  if (tail_bitonic) {  // uniform
    // thread t holds positions u * T + t (each load coalesced across the
    // workgroup; the sort takes its items in any order, each composite
    // carries its position), past n: position n - 1 again, not an item; the
    // row ids go to LDS by position for the emit
    uint16_t v[kRunR];
    int rid[kRunR];
#pragma unroll
    for (int u = 0; u < kRunR; ++u) {
      const long long i = (long long)u * T + tid;
      const long long ic = i < n ? i : n - 1;
      v[u] = load_coherent(scs + ic);
      rid[u] = dseg[ic];
    }
    uint32_t comp[kRunR];
#pragma unroll
    for (int u = 0; u < kRunR; ++u) {
      const long long i = (long long)u * T + tid;
      comp[u] = vtx::bitonic_comp(i < n, vtx::score_key(v[u]), (int)i);
      rid_lds[i < n ? i : n - 1] = rid[u];
    }
    vtx::select_bitonic_run<T, kRunR>(comp, k, bsr, [&](int rank, uint32_t c) {
      a.sidx[obase + rank] = rid_lds[vtx::bitonic_position(c)];
    });
    cm_tiles();
    return;
  }
  if (n <= (long long)T * kTailR) {  // uniform: every score and row id in registers
    // thread t holds positions t * kTailR + u: a thread's items are
    // consecutive, so one prefix over the lanes ranks the ties
    bool have[kTailR];
    uint16_t v[kTailR];
    int rid[kTailR];
#pragma unroll
    for (int u = 0; u < kTailR; ++u) {
      const long long i = (long long)tid * kTailR + u;
      have[u] = i < n;
      v[u] = have[u] ? load_coherent(scs + i) : (uint16_t)0;
      rid[u] = have[u] ? dseg[i] : -1;
    }
    uint32_t key[kTailR];
#pragma unroll
    for (int u = 0; u < kTailR; ++u) {
      key[u] = vtx::score_key(v[u]);
      if (have[u]) vtx::select_count<T>(key[u], sh);
    }
    __syncthreads();
    vtx::select_regs_run<T, kTailR>(have, key, rid, k, sel, sel_pay, sh,
                                    [&](int rank, int payload) { a.sidx[obase + rank] = payload; });
    cm_tiles();
    return;
  }
  const bool cached = n <= a.row_cap;
  __syncthreads();
  // kU loads per thread in flight before any is used
  constexpr int kU = 8;
  for (long long base = 0; base < n; base += (long long)T * kU) {
    uint16_t v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const long long i = base + (long long)u * T + tid;
      v[u] = load_coherent(scs + (i < n ? i : n - 1));  // past n: position n - 1, not used
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const long long i = base + (long long)u * T + tid;
      const uint32_t key = vtx::score_key(v[u]);
      if (cached) keys[i < n ? i : n - 1] = (uint16_t)key;  // past n: position n - 1's own key again
      if (i < n) vtx::select_count<T>(key, sh);
    }
  }
  __syncthreads();
  if (cached) {
    vtx::select_topk_counted<T>([&](long long i) { return (uint32_t)keys[i]; }, n, k, sel, sh);
  } else {
    vtx::select_topk_counted<T>([&](long long i) { return vtx::score_key(load_coherent(scs + i)); }, n, k,
                                sel, sh);
  }
  vtx::select_emit<T>(sel, k, n, [&](int r, long long pos) { a.sidx[obase + r] = dseg[pos]; });
  cm_tiles();
}

constexpr int kLdsBudget = 56 * 1024;  // dynamic LDS; the select tables take up to ~6 KB more
constexpr int kMaxTopk = 4096;

template <int T>
int launch_dim(const FusedArgs& a, const vtx::CmArgs* cm, int blocks, size_t lds, hipStream_t s) {
  const vtx::CmArgs none{};
  if (cm) {  // the in-kernel CMean: rows of one 16-byte vector per lane
    const bool one = cm->nnz <= vtx::kWave;  // loc in one register per lane
    const int32_t nnz = (int32_t)cm->nnz;   // at most vtx::kCmLoc
    switch (a.dim) {
      case 64:
        if (one) indexer_fused_kernel<T, 8, 1, 1>
            <<<blocks, T, lds, s>>>(a.sched, cm->loc, a.segments, nnz, a, *cm);
        else indexer_fused_kernel<T, 8, 1, vtx::kCmLoc / vtx::kWave>
            <<<blocks, T, lds, s>>>(a.sched, cm->loc, a.segments, nnz, a, *cm);
        break;
      case 128:
        if (one) indexer_fused_kernel<T, 16, 1, 1>
            <<<blocks, T, lds, s>>>(a.sched, cm->loc, a.segments, nnz, a, *cm);
        else indexer_fused_kernel<T, 16, 1, vtx::kCmLoc / vtx::kWave>
            <<<blocks, T, lds, s>>>(a.sched, cm->loc, a.segments, nnz, a, *cm);
        break;
      default: return vtx::fail(VTX_E_INVALID, "indexer_fused: in-kernel CMean needs head_dim 64 or 128");
    }
    return vtx::check_launch("indexer_fused (with CMean)");
  }
  switch (a.dim) {
    case 64:
      indexer_fused_kernel<T, 8, 1, 0><<<blocks, T, lds, s>>>(a.sched, nullptr, a.segments, 0, a, none);
      break;
    case 128:
      indexer_fused_kernel<T, 16, 1, 0><<<blocks, T, lds, s>>>(a.sched, nullptr, a.segments, 0, a, none);
      break;
    case 256:
      indexer_fused_kernel<T, 16, 2, 0><<<blocks, T, lds, s>>>(a.sched, nullptr, a.segments, 0, a, none);
      break;
    case 512:
      if constexpr (T <= 512)
        indexer_fused_kernel<T, 16, 4, 0><<<blocks, T, lds, s>>>(a.sched, nullptr, a.segments, 0, a, none);
      break;
    case 576:
      if constexpr (T <= 512)
        indexer_fused_kernel<T, 8, 9, 0><<<blocks, T, lds, s>>>(a.sched, nullptr, a.segments, 0, a, none);
      break;
    default: return vtx::fail(VTX_E_INVALID, "indexer_fused: head_dim %d not supported", a.dim);
  }
  return vtx::check_launch("indexer_fused");
}

// Threads per split workgroup and pages per wave pass, for small chunks and
// large ones (twice the pages per workgroup), by head dim:
//   D = 64, 128, 256: 512 threads x 32 / 32 / 16 pages, large twice the pass
//            (rows of up to two vectors per lane; unstaged, 512 threads let
//            the selecting workgroup hold at most four of a 2046-page
//            segment's scores per thread: C3 17.2 us against 20.9 with 256);
//   D = 128 with the staged pre-selection (`quad`): small chunks of the same
//            256 pages as 256 threads x 64 (four waves, one score per lane:
//            the chunk's select merges four full lists in two rounds instead
//            of eight half-full ones in three; C3 15.2 -> 14.7 us per launch);
//   D >= 512: 256 threads x 16 pages, large 32 (two workgroups per CU fit
//            their registers; 512 threads measured 0.5 us slower at C5).
int split_threads(int dim, bool large, bool quad) { return dim <= 256 && !(quad && !large) ? 512 : 256; }
int split_pass(int dim, bool large, bool quad) {
  if (quad && !large) return 64;
  return (dim <= 128 ? 32 : 16) * (large ? 2 : 1);
}
int split_chunk(int dim, bool large, bool quad) {
  return (split_threads(dim, large, quad) / 64) * split_pass(dim, large, quad);
}

// blocks: the grid, xcd: work ids per XCD (8 * xcd workgroups take work
// ids, the rest are CMean tile workgroups)
template <int P, int kCm>
int launch_split_cm(const FusedArgs& a, int32_t* counters, int cps, int blocks, int32_t xcd, size_t lds,
                    hipStream_t s, const vtx::CmArgs& cm, bool quad) {
  const int32_t nnz = (int32_t)cm.nnz;  // at most vtx::kCmLoc with the CMean, else 0
  switch (a.dim) {
    case 64:
      indexer_split_kernel<512, 8, 1, 2 * P, kCm>
          <<<blocks, 512, lds, s>>>(a.dindptr, a.sindptr, cm.loc, a.segments, nnz, cps, xcd, a, counters, cm);
      break;
    case 128:  // (P = 16: small chunks, 32: large; quad: split_threads, split_pass)
      if (P == 16 && quad)
        indexer_split_kernel<256, 16, 1, 64, kCm>
            <<<blocks, 256, lds, s>>>(a.dindptr, a.sindptr, cm.loc, a.segments, nnz, cps, xcd, a, counters, cm);
      else
        indexer_split_kernel<512, 16, 1, 2 * P, kCm>
            <<<blocks, 512, lds, s>>>(a.dindptr, a.sindptr, cm.loc, a.segments, nnz, cps, xcd, a, counters, cm);
      break;
    case 256:
      indexer_split_kernel<512, 16, 2, P, kCm>
          <<<blocks, 512, lds, s>>>(a.dindptr, a.sindptr, cm.loc, a.segments, nnz, cps, xcd, a, counters, cm);
      break;
    case 512:
      indexer_split_kernel<256, 16, 4, P, kCm>
          <<<blocks, 256, lds, s>>>(a.dindptr, a.sindptr, cm.loc, a.segments, nnz, cps, xcd, a, counters, cm);
      break;
    case 576:
      indexer_split_kernel<256, 8, 9, P, kCm>
          <<<blocks, 256, lds, s>>>(a.dindptr, a.sindptr, cm.loc, a.segments, nnz, cps, xcd, a, counters, cm);
      break;
    default: return vtx::fail(VTX_E_INVALID, "indexer_fused: head_dim %d not supported", a.dim);
  }
  return vtx::check_launch(kCm ? "indexer_fused (split, with CMean)" : "indexer_fused (split)");
}

template <int P>
int launch_split_pass(const FusedArgs& a, int32_t* counters, int cps, int blocks, int32_t xcd, size_t lds,
                      hipStream_t s, const vtx::CmArgs* cm, bool quad) {
  if (cm) return launch_split_cm<P, vtx::kCmLoc / vtx::kWave>(a, counters, cps, blocks, xcd, lds, s, *cm, quad);
  return launch_split_cm<P, 0>(a, counters, cps, blocks, xcd, lds, s, vtx::CmArgs{}, quad);
}

int launch_split(const FusedArgs& a, int32_t* counters, int cps, bool large, bool quad, int blocks, int32_t xcd,
                 size_t lds, hipStream_t s, const vtx::CmArgs* cm) {
  return large ? launch_split_pass<32>(a, counters, cps, blocks, xcd, lds, s, cm, quad)
               : launch_split_pass<16>(a, counters, cps, blocks, xcd, lds, s, cm, quad);
}

// Work units of the in-launch CMean per closed (page, head) tile: parts of
// 64 column vectors for row widths other than 8, 16, 32 or 64 vectors
// (vtx::tile_parts for the kernel's width).
int cmean_tile_parts(int head_dim) {
  const int nv = head_dim / 8;
  return (nv == 8 || nv == 16 || nv == 32 || nv == 64) ? 1 : (nv + vtx::kWave - 1) / vtx::kWave;
}
constexpr long long kMaxTileWorkgroups = 64;  // CMean tile workgroups a split launch appends at most

}  // namespace

extern "C" int vtx_indexer_fused_supported(int32_t head_dim) {
  return head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512 || head_dim == 576;
}

extern "C" int64_t vtx_indexer_fused_workspace_len(int32_t segments) {
  return segments < 0 ? -1 : (int64_t)segments + kStageZoneInts;
}

namespace {

// The decode CMean a fused launch may run first (vtx_indexer_fused_cmean).
struct CmeanSpec {
  const uint16_t* k;
  int64_t k_rows;
  int32_t page_size, heads;
  const int64_t* loc;
  int64_t nnz;
};

int fused_impl(const uint16_t* q, int64_t q_rows, int32_t group_size, const uint16_t* x, uint16_t* x_out,
               const uint16_t* y, int64_t y_rows, uint16_t* score, int64_t score_len,
               const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr, const int32_t* dense_kv_indices,
               int64_t dense_kv_indices_len, int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
               int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos, int32_t reserved_eos,
               int32_t max_num_pages, int32_t head_dim, int32_t* seg_counters, int64_t seg_counters_len,
               int32_t mode, const CmeanSpec* cms, const int32_t* schedule, int64_t schedule_len, void* stream);

}  // namespace

extern "C" int vtx_indexer_fused(const uint16_t* q, int64_t q_rows, int32_t group_size,
                                 const uint16_t* x, uint16_t* x_out, const uint16_t* y,
                                 int64_t y_rows, uint16_t* score, int64_t score_len,
                                 const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr,
                                 const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                                 int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                                 int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos,
                                 int32_t reserved_eos, int32_t max_num_pages, int32_t head_dim,
                                 int32_t* seg_counters, int64_t seg_counters_len, int32_t mode,
                                 const int32_t* schedule, int64_t schedule_len, void* stream) {
  vtx::clear_error();
  return fused_impl(q, q_rows, group_size, x, x_out, y, y_rows, score, score_len, dense_kv_indptr,
                    sparse_kv_indptr, dense_kv_indices, dense_kv_indices_len, sparse_kv_indices,
                    sparse_kv_indices_len, eff_batch_size, topk_val, reserved_bos, reserved_eos, max_num_pages,
                    head_dim, seg_counters, seg_counters_len, mode, nullptr, schedule, schedule_len, stream);
}

extern "C" int vtx_indexer_fused_cmean(const uint16_t* q, int64_t q_rows, int32_t group_size,
                                       const uint16_t* x, uint16_t* x_out, uint16_t* y, int64_t y_rows,
                                       uint16_t* score, int64_t score_len, const int32_t* dense_kv_indptr,
                                       const int32_t* sparse_kv_indptr, const int32_t* dense_kv_indices,
                                       int64_t dense_kv_indices_len, int32_t* sparse_kv_indices,
                                       int64_t sparse_kv_indices_len, int32_t eff_batch_size, int32_t topk_val,
                                       int32_t reserved_bos, int32_t reserved_eos, int32_t max_num_pages,
                                       int32_t head_dim, int32_t* seg_counters, int64_t seg_counters_len,
                                       int32_t mode, const uint16_t* k_cache, int64_t k_rows,
                                       int32_t page_size, int32_t num_kv_heads, const int64_t* loc, int64_t nnz,
                                       const int32_t* schedule, int64_t schedule_len, void* stream) {
  vtx::clear_error();
  if (!k_cache || (nnz > 0 && !loc)) return vtx::fail(VTX_E_INVALID, "indexer_fused_cmean: null K pool or loc");
  if (page_size < 1 || num_kv_heads < 1 || k_rows < 0 || nnz < 0)
    return vtx::fail(VTX_E_INVALID, "indexer_fused_cmean: bad CMean sizes");
  CmeanSpec cm{k_cache, k_rows, page_size, num_kv_heads, loc, nnz};
  return fused_impl(q, q_rows, group_size, x, x_out, y, y_rows, score, score_len, dense_kv_indptr,
                    sparse_kv_indptr, dense_kv_indices, dense_kv_indices_len, sparse_kv_indices,
                    sparse_kv_indices_len, eff_batch_size, topk_val, reserved_bos, reserved_eos, max_num_pages,
                    head_dim, seg_counters, seg_counters_len, mode, &cm, schedule, schedule_len, stream);
}

namespace {

int fused_impl(const uint16_t* q, int64_t q_rows, int32_t group_size, const uint16_t* x, uint16_t* x_out,
               const uint16_t* y, int64_t y_rows, uint16_t* score, int64_t score_len,
               const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr, const int32_t* dense_kv_indices,
               int64_t dense_kv_indices_len, int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
               int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos, int32_t reserved_eos,
               int32_t max_num_pages, int32_t head_dim, int32_t* seg_counters, int64_t seg_counters_len,
               int32_t mode, const CmeanSpec* cms, const int32_t* schedule, int64_t schedule_len, void* stream) {
  if (eff_batch_size < 0 || group_size < 0 || reserved_bos < 0 || reserved_eos < 0)
    return vtx::fail(VTX_E_INVALID, "indexer_fused: negative size");
  if (!vtx_indexer_fused_supported(head_dim))
    return vtx::fail(VTX_E_INVALID, "indexer_fused: head_dim %d not supported", head_dim);
  if (topk_val > kMaxTopk)
    return vtx::fail(VTX_E_INVALID, "indexer_fused: topk_val %d exceeds %d", topk_val, kMaxTopk);
  if (q_rows < eff_batch_size)
    return vtx::fail(VTX_E_INVALID, "indexer_fused: %lld query rows for %d segments",
                     (long long)q_rows, eff_batch_size);
  if (group_size > 0 ? !q : !x) return vtx::fail(VTX_E_INVALID, "indexer_fused: null query");
  if (!y || !score || !dense_kv_indptr || !sparse_kv_indptr || !dense_kv_indices || !sparse_kv_indices)
    return vtx::fail(VTX_E_INVALID, "indexer_fused: null pointer");
  if (y_rows <= 0) return vtx::fail(VTX_E_INVALID, "indexer_fused: empty centroid pool");
  const void* qp = group_size > 0 ? (const void*)q : (const void*)x;
  if (!vtx::aligned16(qp) || !vtx::aligned16(y) || (x_out && !vtx::aligned16(x_out)))
    return vtx::fail(VTX_E_INVALID, "indexer_fused: query, centroid and q_mean rows must be 16-byte aligned");

  FusedArgs a;
  a.q = q;
  a.G = group_size;
  // torch's mean factor: (float)(outputs) / (inputs, converted to float)
  a.inv_g = group_size > 0 && q_rows > 0
                ? (float)(q_rows * (long long)head_dim) / (float)(q_rows * (long long)group_size * head_dim)
                : 1.0f;
  a.x = x;
  a.x_out = group_size > 0 ? x_out : nullptr;
  a.q_rows = q_rows;
  a.y = y;
  a.y_rows = y_rows;
  a.score = score;
  a.score_len = score_len;
  a.dindptr = dense_kv_indptr;
  a.sindptr = sparse_kv_indptr;
  a.didx = dense_kv_indices;
  a.didx_len = dense_kv_indices_len;
  a.sidx = sparse_kv_indices;
  a.sidx_len = sparse_kv_indices_len;
  a.topk = topk_val > 0 ? topk_val : 0;
  a.bos = reserved_bos;
  a.eos = reserved_eos;
  a.dim = head_dim;
  a.row_cap = 0;
  a.sched = nullptr;
  a.stage = nullptr;

  if (mode < VTX_FUSED_AUTO || mode > VTX_FUSED_SPLIT)
    return vtx::fail(VTX_E_INVALID, "indexer_fused: unknown mode %d", mode);
  // The workspace: the arrival counters at its start; when it is at least
  // kStageZoneInts long, the staging zone at its end, and the counters are
  // the int32s before the zone (so none of them ever holds a staged list)
  long long counter_cap = seg_counters ? seg_counters_len : 0;
  uint64_t* zone = nullptr;
  if (seg_counters && seg_counters_len >= kStageZoneInts) {
    counter_cap = seg_counters_len - kStageZoneInts;
    long long off = counter_cap;
    if (reinterpret_cast<uintptr_t>(seg_counters + off) % 8) ++off;
    zone = reinterpret_cast<uint64_t*>(seg_counters + off);
  }
  const bool have_counters = seg_counters && counter_cap >= eff_batch_size;
  if (mode == VTX_FUSED_SPLIT && !have_counters)
    return vtx::fail(VTX_E_INVALID, "indexer_fused: split mode needs %d segment counters, got %lld",
                     eff_batch_size, counter_cap);
  a.segments = eff_batch_size;
  const long long want = max_num_pages > 0 ? max_num_pages : 0;
  hipStream_t s = vtx::as_stream(stream);
  const int cus = vtx::device_cu_count();
  if (cus <= 0) return vtx::fail(VTX_E_DEVICE, "indexer_fused: cannot query the compute unit count");

  // One workgroup per segment fills the chip when there are at least two
  // segments per CU; fewer (long contexts, MLA's single latent head) leave
  // CUs idle, so their pages are split over several workgroups.
  const bool split = mode == VTX_FUSED_SPLIT ||
                     (mode == VTX_FUSED_AUTO && have_counters && (long long)eff_batch_size < 2LL * cus);
  // The CMean runs inside the launch for decode-sized loc and a 16-byte
  // aligned K pool: in the segment layout for rows of one 16-byte vector per
  // lane (its tile layout is then the scoring layout), in the split layout
  // for every supported width; otherwise as its own launch, first.
  const bool cm_inside = cms && cms->nnz <= vtx::kCmLoc && vtx::aligned16(cms->k) &&
                         (split || head_dim == 64 || head_dim == 128);
  vtx::CmArgs cma{};
  const bool cm_launch = cm_inside && cms->nnz > 0;
  if (cm_launch) {  // the tiles are spread over the launch's own waves
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
  if (cms && !cm_inside && cms->nnz > 0) {
    const int rc = vtx_page_reduce(cms->k, cms->k_rows, cms->page_size, head_dim, const_cast<uint16_t*>(y),
                                   VTX_DTYPE_BF16, y_rows, cms->loc, cms->nnz, cms->heads, cms->page_size, 1,
                                   VTX_REDUCE_MEAN, stream);
    if (rc != VTX_OK) return rc;
  }
  if (split) {
    // Small chunks when every segment's chunks fit on the chip at once
    // (16 waves of split workgroups per CU), else twice as large; past that,
    // workgroups loop over several chunks.  Rows of four or more vectors per
    // lane (D >= 512) always take the large chunks: a workgroup's fixed work
    // (its query mean of up to 16 heads, its staged list, its count-in) then
    // serves twice the pages, and a segment hands over half as many lists
    // (C5: 13.7 -> 12.8 us per launch; at C3 the large chunks are slower).
    const long long mid = want - reserved_bos - reserved_eos > 1 ? want - reserved_bos - reserved_eos : 1;
    // (split workgroups resident at once: 16 waves per CU)
    const long long small = split_chunk(head_dim, false, false);
    const long long small_chunks = (mid + small - 1) / small;
    // four-wave workgroups at D = 128 when every chunk of every segment is
    // one workgroup's and the chunks stage their lists
    const bool quad = head_dim == 128 && zone != nullptr && a.topk <= vtx::kMaxBitonicRunK &&
                      eff_batch_size <= kStageMaxSegments && small_chunks <= kStageLists &&
                      (long long)eff_batch_size * small_chunks <= (1024LL / 256) * cus;
    const bool large = head_dim >= 512 ||
                       (long long)eff_batch_size * small_chunks > (1024LL / split_threads(head_dim, false, quad)) * cus;
    const long long resident = (1024LL / split_threads(head_dim, large, quad)) * cus;
    const int chunk = split_chunk(head_dim, large, quad);
    long long cps = (mid + chunk - 1) / chunk;
    const long long fill = eff_batch_size > 0 ? resident / eff_batch_size : 1;
    if (cps > fill) cps = fill;
    if (cps < 1) cps = 1;
    const long long room = (kLdsBudget - (long long)vtx::sel_slots(a.topk) * 8 - (long long)a.topk * 4) / 6;
    long long cap = want < room ? want : room;
    cap &= ~7LL;
    if (cap < 0) cap = 0;
    a.row_cap = (int32_t)cap;
    // sel, payloads, keys, and the bitonic select's row ids by position
    const size_t lds = (size_t)vtx::sel_slots(a.topk) * 8 + (size_t)a.topk * 4 + (size_t)cap * 6;
    long long items = (long long)eff_batch_size * cps + (a.x_out ? q_rows - eff_batch_size : 0);
    items = (items + 7) / 8 * 8;  // work ids are laid out per XCD
    if (items == 0) return VTX_OK;
    // the in-launch CMean's own workgroups, for wide rows: enough for one
    // unit per wave if every loc entry closed a page (a loc entry closes at
    // most one).  Narrower rows share the units out over the work ids after
    // their count-in (measured: C5 12.73 -> 12.59 us per launch with tile
    // workgroups; C3 14.44 -> 14.53, so not there)
    long long tile_wgs = 0;
    if (cmp && head_dim >= 512) {
      const long long waves = split_threads(head_dim, large, quad) / vtx::kWave;
      const long long units = cma.nnz * cma.heads * cmean_tile_parts(head_dim);
      tile_wgs = std::min((units + waves - 1) / waves, kMaxTileWorkgroups);
    }
    if (items + tile_wgs > 0x7fffffffLL) return vtx::fail(VTX_E_INVALID, "indexer_fused: too many workgroups");
    a.stage = zone;  // the staged pre-selection's lists (segments past kStageMaxSegments do not stage)
    return launch_split(a, seg_counters, (int)cps, large, quad, (int)(items + tile_wgs), (int32_t)(items / 8), lds,
                        s, cmp);
  }

  // the planner's schedule, when it covers this launch's segments
  if (schedule && schedule_len >= vtx::sched_len(1, eff_batch_size)) a.sched = schedule;
  const long long room = (kLdsBudget - (long long)vtx::sel_slots(a.topk) * 8 - (long long)a.topk * 4) / 6;
  long long cap = want < room ? want : room;
  cap &= ~7LL;
  if (cap < 0) cap = 0;
  a.row_cap = (int32_t)cap;
  const size_t lds = (size_t)vtx::sel_slots(a.topk) * 8 + (size_t)a.topk * 4 + (size_t)cap * 6;  // + select_regs' payloads
  // With a q_mean output every query row gets a workgroup (rows past the
  // segments only write their mean).
  const long long grid = a.x_out ? q_rows : eff_batch_size;
  if (grid > 0x7fffffffLL) return vtx::fail(VTX_E_INVALID, "indexer_fused: too many query rows");
  const long long blocks = grid;
  if (blocks == 0) return VTX_OK;
  if (max_num_pages <= 256) return launch_dim<256>(a, cmp, (int)blocks, lds, s);
  // (rows of four or more vectors per lane need more than the 128 registers
  // a lane of a 1024-thread workgroup can have)
  if (max_num_pages <= 1024 || head_dim >= 512) return launch_dim<512>(a, cmp, (int)blocks, lds, s);
  return launch_dim<1024>(a, cmp, (int)blocks, lds, s);
}

}  // namespace

// ---------------------------------------------------------------------------
// vtx_indexer_fused_noalloc: vtx_indexer_fused with its workspace (the split
// layout's per-segment arrival counters and the staging zone of its
// pre-selection) in a file-scope device array instead of a caller buffer,
// for callers that cannot allocate.  Every device keeps its own copy of the
// array until the process ends; the kernels take its device address
// (queried once per device with that device current), never the host-side
// name.  Each launch that completes leaves every counter it used, and every
// staged list place, at zero, so the array is cleared (by a fill kernel) on
// the first call on a device, by vtx_indexer_fused_noalloc_reset, and again
// before the next call after a launch this entry point could not issue.
// Calls that overlap on one device share the array and race.
#include <mutex>

namespace {

constexpr int64_t kStaticCounters = 65536;  // segments a no-allocation call may have
constexpr int64_t kStaticInts = kStaticCounters + kStageZoneInts;  // 4.25 MiB
static __device__ __align__(256) int32_t scratch[kStaticInts];

__global__ void clear_counters_kernel(int32_t* c, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    c[i] = 0;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int32_t* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch`, per device
bool g_scratch_dirty[kMaxDevices] = {};    // array to clear before the next call

// Clears the counters and the staging zone on stream s; outside a graph
// capture it also waits for the fill, so that a first call on another stream
// cannot run before it.
int clear_counters(int32_t* p, hipStream_t s) {
  clear_counters_kernel<<<256, 256, 0, s>>>(p, kStaticInts);
  int rc = vtx::check_launch("indexer_fused_noalloc (clearing the counters)");
  if (rc != VTX_OK) return rc;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess)
    return vtx::fail(VTX_E_DEVICE, "indexer_fused_noalloc: cannot query the stream's capture state");
  if (st == hipStreamCaptureStatusNone && hipStreamSynchronize(s) != hipSuccess)
    return vtx::fail(VTX_E_DEVICE, "indexer_fused_noalloc: clearing the counters failed");
  return VTX_OK;
}

// This device's workspace, set up (address looked up, counters cleared) on
// the first call on the device and cleared again when marked dirty.
int static_counters(hipStream_t s, bool force_clear, int32_t** out, int* dev_out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return vtx::fail(VTX_E_DEVICE, "indexer_fused_noalloc: no usable current device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return vtx::fail(VTX_E_DEVICE, "indexer_fused_noalloc: cannot get the counters' address: %s",
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<int32_t*>(p);
    g_scratch_dirty[dev] = true;
  }
  if (g_scratch_dirty[dev] || force_clear) {
    const int rc = clear_counters(g_scratch_ptr[dev], s);
    if (rc != VTX_OK) return rc;
    g_scratch_dirty[dev] = false;
  }
  *out = g_scratch_ptr[dev];
  *dev_out = dev;
  return VTX_OK;
}

}  // namespace

extern "C" int vtx_indexer_fused_noalloc(const uint16_t* q, int64_t q_rows, int32_t group_size,
                                         const uint16_t* x, uint16_t* x_out, const uint16_t* y,
                                         int64_t y_rows, uint16_t* score, int64_t score_len,
                                         const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr,
                                         const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                                         int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                                         int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos,
                                         int32_t reserved_eos, int32_t max_num_pages, int32_t head_dim,
                                         int32_t mode, const int32_t* schedule, int64_t schedule_len,
                                         void* stream) {
  vtx::clear_error();
  if (eff_batch_size > kStaticCounters)
    return vtx::fail(VTX_E_INVALID, "indexer_fused_noalloc: %d segments exceed the %lld it serves",
                     eff_batch_size, (long long)kStaticCounters);
  int32_t* counters = nullptr;
  int dev = -1;
  int rc = static_counters(vtx::as_stream(stream), false, &counters, &dev);
  if (rc != VTX_OK) return rc;
  rc = fused_impl(q, q_rows, group_size, x, x_out, y, y_rows, score, score_len, dense_kv_indptr, sparse_kv_indptr,
                  dense_kv_indices, dense_kv_indices_len, sparse_kv_indices, sparse_kv_indices_len, eff_batch_size,
                  topk_val, reserved_bos, reserved_eos, max_num_pages, head_dim, counters, kStaticInts, mode, nullptr,
                  schedule, schedule_len, stream);
  if (rc == VTX_E_LAUNCH) {  // a launch that did not run may leave counters behind: clear before the next call
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    g_scratch_dirty[dev] = true;
  }
  return rc;
}

extern "C" int vtx_indexer_fused_noalloc_reset(void* stream) {
  vtx::clear_error();
  int32_t* counters = nullptr;
  int dev = -1;
  return static_counters(vtx::as_stream(stream), true, &counters, &dev);
}
