// Workgroup-wide top-k selection over 16-bit order keys (see score_key).
//
// select_topk() finds the k best of n items — largest key first, ties to the
// lower position — and stores their composites (key << 32 | ~position) in
// `sel[0..k)`, unordered.  rank_of() then gives a winner's output rank.
//
//   1. two 8-bit radix-histogram passes in LDS find the key `thr` of the k-th
//      best item, the number of items above it and how many of the items
//      equal to it are needed (`take`);
//   2. items above `thr` win; items equal to `thr` win in position order
//      until `take` are in: per-(tile, wave) tie counts are written once,
//      after one barrier every wave knows how many ties precede each of its
//      items.
//
// The passes give each thread kSelU items per round with their key reads
// issued together, and winners are appended with one LDS atomic per wave
// and round (ballot + prefix), so the cost is a few LDS round trips per
// pass rather than one per item.
//
// Every thread of the workgroup must call it (it contains barriers).
#pragma once

#include "vtx_device.h"

namespace vtx {

constexpr int kSelU = 4;          // items per thread per round
constexpr int kSelTieTiles = 64;  // tiles (of T items) with precomputed tie counts

// The two 256-bin histograms are kept in NC copies (lane l counts into copy
// l % NC): the keys of one segment share few high bytes, so with one copy
// most lanes of a wave add to the same LDS word and the atomics serialize.
// Copies sit kStride words apart (16 bytes of padding shift each copy by four
// banks).  Readers sum the copies.
template <int T, int NC = 1>
struct SelectShared {
  static constexpr int kCopies = NC;
  static constexpr int kStride = NC > 1 ? 260 : 256;
  alignas(16) uint32_t hist[2][NC * kStride];  // read 16 bytes per lane in sel_find_bin_wave
  uint32_t wave_ties[T / kWave];
  uint32_t wave_gt[T / kWave];        // select_regs: items above the threshold, per wave
  uint32_t tie_counts[kSelTieTiles * (T / kWave)];  // [tile][wave]
  int count;
};

// Adds one item to bin `bin` of histogram h (the lane's copy).
template <int T, int NC>
__device__ __forceinline__ void sel_hist_add(SelectShared<T, NC>& sh, int h, uint32_t bin) {
  const int cp = NC > 1 ? (lane_id() % NC) : 0;
  atomicAdd(&sh.hist[h][cp * SelectShared<T, NC>::kStride + bin], 1u);
}

// Items in bin `bin` of histogram h (all copies).
template <int T, int NC>
__device__ __forceinline__ uint32_t sel_hist_count(const SelectShared<T, NC>& sh, int h, uint32_t bin) {
  uint32_t c = 0;
#pragma unroll
  for (int cp = 0; cp < NC; ++cp) c += sh.hist[h][cp * SelectShared<T, NC>::kStride + bin];
  return c;
}

// Appends this wave's winners (win set) to sel with one LDS atomic for the
// wave; `comp` is the lane's composite.  Wave-uniform control flow.
__device__ __forceinline__ void sel_append(bool win, uint64_t comp, uint64_t* sel, int k, int* count) {
  const uint64_t m = __ballot(win);
  if (m) {
    int base = 0;
    if (lane_id() == 0) base = atomicAdd(count, (int)__popcll(m));
    base = __builtin_amdgcn_readfirstlane(base);  // lane 0 is active here
    const int slot = base + lanes_below(m);
    if (win && slot < k) sel[slot] = comp;
  }
}

// Winner slots allocated for a top-k of k: k rounded up to 16, the slots past
// k held at zero, so a rank is counted over whole 16-slot blocks (a zero
// slot never beats a winner: a composite is at least 1).
__host__ __device__ constexpr int sel_slots(int k) { return (k + 15) & ~15; }

__device__ __forceinline__ uint64_t sel_composite(uint32_t key, long long pos) {
  return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)pos);
}
__device__ __forceinline__ long long sel_position(uint64_t c) {
  return (long long)(0xffffffffu - (uint32_t)c);
}

// Run by one full wave (every lane gets the answer): the bin b of `hist`
// (256 bins, higher = better) holding the kt-th best item, i.e.
// above(b) < kt <= above(b) + hist[b], and above(b) (and hist[b] when
// `count` is given).
template <int NC = 1, int kStride = 256>
__device__ __forceinline__ void sel_find_bin_wave(const uint32_t* hist, uint32_t kt, int* bin, int* above,
                                                  int* count = nullptr) {
  const int l = lane_id();
  U4 c = ld16(hist + 4 * l);
#pragma unroll
  for (int cp = 1; cp < NC; ++cp) {
    const U4 d = ld16(hist + cp * kStride + 4 * l);
    c.x += d.x;
    c.y += d.y;
    c.z += d.z;
    c.w += d.w;
  }
  const uint32_t tot = c.x + c.y + c.z + c.w;
  const uint32_t incl = wave_prefix_sum(tot);
  const uint32_t a3 = lane_value(incl, kWave - 1) - incl;  // items in the bins of higher lanes
  const uint32_t a2 = a3 + c.w;
  const uint32_t a1 = a2 + c.z;
  const uint32_t a0 = a1 + c.y;
  int b = -1;
  uint32_t ab = 0, cb = 0;
  if (a3 < kt && kt <= a2) {
    b = 4 * l + 3;
    ab = a3;
    cb = c.w;
  } else if (a2 < kt && kt <= a1) {
    b = 4 * l + 2;
    ab = a2;
    cb = c.z;
  } else if (a1 < kt && kt <= a0) {
    b = 4 * l + 1;
    ab = a1;
    cb = c.y;
  } else if (a0 < kt && kt <= a0 + c.x) {
    b = 4 * l;
    ab = a0;
    cb = c.x;
  }
  const uint64_t m = __ballot(b >= 0);
  const int src = m ? (int)__builtin_ctzll(m) : 0;
  *bin = m ? (int)lane_value((uint32_t)b, src) : 0;
  *above = m ? (int)lane_value(ab, src) : 0;
  if (count) *count = m ? (int)lane_value(cb, src) : 0;
}

// The bin of histogram h holding the kt-th best item (see sel_find_bin_wave).
template <int T, int NC>
__device__ __forceinline__ void sel_find_bin(const SelectShared<T, NC>& sh, int h, uint32_t kt, int* bin,
                                             int* above) {
  sel_find_bin_wave<NC, SelectShared<T, NC>::kStride>(sh.hist[h], kt, bin, above);
}

// Clears the histograms, the winner count and the winner slots (no barrier).
template <int T, int NC>
__device__ __forceinline__ void select_init(uint64_t* sel, int k, SelectShared<T, NC>& sh) {
  const int tid = threadIdx.x;
  for (int i = tid; i < NC * SelectShared<T, NC>::kStride; i += T) {
    sh.hist[0][i] = 0u;
    sh.hist[1][i] = 0u;
  }
  if (tid == 0) sh.count = 0;
  for (int j = tid; j < sel_slots(k); j += T) sel[j] = 0;  // decodes to a position >= n
}

// Adds one item to the high-byte histogram (callers that produce the keys
// themselves build it on the fly and then call select_topk_counted).
template <int T, int NC>
__device__ __forceinline__ void select_count(uint32_t key, SelectShared<T, NC>& sh) {
  sel_hist_add(sh, 0, key >> 8);
}

// The selection once hist[0] holds every item (and a barrier made it visible).
template <int T, int NC, typename KeyAt>
__device__ __forceinline__ void select_topk_counted(KeyAt key_at, long long n, int k, uint64_t* sel,
                                                    SelectShared<T, NC>& sh) {
  constexpr int kWaves = T / kWave;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;

  // Every wave reads the threshold bins off the LDS histograms itself, so
  // no barrier is needed to broadcast them.
  int hi_bin = 0, above_hi = 0;
  sel_find_bin(sh, 0, (uint32_t)k, &hi_bin, &above_hi);
  const uint32_t hi = (uint32_t)hi_bin;

  // kSelU keys per thread per round, their reads issued together (positions
  // past n read position n - 1, ignored by every use: no branch around a
  // read, which would let the compiler wait for each on its own); the keys
  // of the first round stay in registers for the second pass.
  auto load = [&](long long i0, uint32_t (&key)[kSelU]) {
#pragma unroll
    for (int u = 0; u < kSelU; ++u) {
      const long long i = i0 + (long long)u * T + tid;
      key[u] = key_at(i < n ? i : n - 1);
    }
  };
  auto count_lo = [&](long long i0, const uint32_t (&key)[kSelU]) {
#pragma unroll
    for (int u = 0; u < kSelU; ++u) {
      const long long i = i0 + (long long)u * T + tid;
      if (i < n && (key[u] >> 8) == hi) sel_hist_add(sh, 1, key[u] & 255u);
    }
  };
  uint32_t key0[kSelU];
  load(0, key0);
  count_lo(0, key0);
  for (long long i0 = (long long)T * kSelU; i0 < n; i0 += (long long)T * kSelU) {
    uint32_t key[kSelU];
    load(i0, key);
    count_lo(i0, key);
  }
  __syncthreads();
  int lo_bin = 0, above_lo = 0;
  sel_find_bin(sh, 1, (uint32_t)(k - above_hi), &lo_bin, &above_lo);
  const uint32_t thr = (hi << 8) | (uint32_t)lo_bin;
  const int take = k - (above_hi + above_lo);  // >= 1 items equal to thr win
  const bool all_ties = (take == (int)sel_hist_count(sh, 1, thr & 255u));
  const long long tiles = (n + T - 1) / T;
  const bool tie_table = !all_ties && tiles <= kSelTieTiles;

  // Items above the threshold (and, when every tie wins, the ties); the
  // per-(tile, wave) tie counts are recorded on the way.
  auto collect = [&](long long i0, const uint32_t (&key)[kSelU]) {
#pragma unroll
    for (int u = 0; u < kSelU; ++u) {
      if (i0 + (long long)u * T >= n) break;  // uniform: the rest of the round is past the end
      const long long i = i0 + (long long)u * T + tid;
      const bool in = i < n;
      const bool win = in && (key[u] > thr || (all_ties && key[u] == thr));
      sel_append(win, sel_composite(key[u], i), sel, k, &sh.count);
      if (tie_table) {
        const uint64_t m = __ballot(in && key[u] == thr);
        const long long tile = i0 / T + u;
        if (lane == 0 && tile < tiles) sh.tie_counts[tile * kWaves + wave] = (uint32_t)__popcll(m);
      }
    }
  };
  collect(0, key0);
  for (long long i0 = (long long)T * kSelU; i0 < n; i0 += (long long)T * kSelU) {
    uint32_t key[kSelU];
    load(i0, key);
    collect(i0, key);
  }
  if (tie_table) {
    __syncthreads();
    // Ties before tile j: sum of earlier tiles' counts; within tile j, the
    // counts of lower waves, then lower lanes.
    int before = 0;
    for (long long j = 0; j < tiles && before < take; ++j) {
      int tile_total = 0, lower = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const int c = (int)sh.tie_counts[j * kWaves + w];
        tile_total += c;
        lower += (w < wave) ? c : 0;
      }
      if (tile_total != 0) {
        const long long i = j * T + tid;
        const bool eq = i < n && key_at(i) == thr;
        const uint64_t m = __ballot(eq);
        const bool tw = eq && before + lower + lanes_below(m) < take;
        sel_append(tw, sel_composite(thr, i), sel, k, &sh.count);
      }
      before += tile_total;
    }
  } else if (!all_ties) {
    // Long segments: tile by tile, with the counts of each tile exchanged
    // through LDS.
    int seen = 0;  // tied items in earlier tiles
    for (long long t0 = 0; t0 < n; t0 += T) {
      const long long i = t0 + tid;
      const bool eq = (i < n) && key_at(i) == thr;
      const uint64_t m = __ballot(eq);
      if (lane == 0) sh.wave_ties[wave] = (uint32_t)__popcll(m);
      __syncthreads();
      int before = seen, tile = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const int c = (int)sh.wave_ties[w];
        before += (w < wave) ? c : 0;
        tile += c;
      }
      const bool tw = eq && before + lanes_below(m) < take;
      sel_append(tw, sel_composite(thr, i), sel, k, &sh.count);
      seen += tile;
      __syncthreads();
      if (seen >= take) break;
    }
  }
  __syncthreads();
}

// key_at(i) returns the order key of item i < n.  Requires 0 < k < n.
template <int T, int NC, typename KeyAt>
__device__ __forceinline__ void select_topk(KeyAt key_at, long long n, int k, uint64_t* sel,
                                            SelectShared<T, NC>& sh) {
  select_init<T>(sel, k, sh);
  __syncthreads();
  for (long long i = threadIdx.x; i < n; i += T) select_count<T>(key_at(i), sh);
  __syncthreads();
  select_topk_counted<T>(key_at, n, k, sel, sh);
}

// Output rank of winner `c` among the k winners in sel (best = 0): the
// sel_slots(k) slots read two composites per 16-byte broadcast read, eight
// reads in flight (sel 16-byte aligned, slots past k zero).
__device__ __forceinline__ int rank_of_pairs(uint64_t c, const uint64_t* sel, int k) {
  int r = 0;
  const int slots = sel_slots(k);
  for (int m = 0; m < slots; m += 16) {
    U4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = ld16(sel + m + 2 * u);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      r += (((uint64_t)v[u].y << 32 | v[u].x) > c) ? 1 : 0;
      r += (((uint64_t)v[u].w << 32 | v[u].z) > c) ? 1 : 0;
    }
  }
  return r;
}

__device__ __forceinline__ int rank_of(uint64_t c, const uint64_t* sel, int k) { return rank_of_pairs(c, sel, k); }

// Position rank inside a wave of the scoring layout in which lane
// l = grp * LPR + col holds pass position col * (64 / LPR) + grp: the number
// of lanes in `m` whose position is below this lane's.
template <int LPR>
__device__ __forceinline__ int pass_rank_below(uint64_t m) {
  constexpr int kGroups = kWave / LPR;
  constexpr uint64_t kRep = LPR == 16 ? 0x0001000100010001ull : (LPR == 8 ? 0x0101010101010101ull : 0ull);
  static_assert(kRep != 0, "pass_rank_below: LPR 8 or 16");
  static_assert(kGroups * LPR == kWave, "lane layout");
  const int l = lane_id();
  const int grp = l / LPR, col = l % LPR;
  const uint64_t lower_col = ((1ull << col) - 1ull) * kRep;                       // col' < col
  const uint64_t same_col = ((1ull << col) * kRep) & ((1ull << (grp * LPR)) - 1ull);  // col' == col, grp' < grp
  return __popcll(m & lower_col) + __popcll(m & same_col);
}

// Selection of the k best items (largest key first, ties to the lower
// position) when every item is held in registers by one thread: `have`,
// its 16-bit order key, its position and a payload.  The items of wave w
// have lower positions than those of wave w + 1, and inside a wave they
// follow the scoring layout of pass_rank_below<LPR>.  hist[0] must hold the
// high-byte counts of every item and hist[1] zeros, visible after a barrier.
//
//   1. the threshold key thr from the two 8-bit histogram passes (the same
//      passes as select_topk_counted);
//   2. per-wave counts of the items above thr and equal to thr (one LDS
//      exchange) give each item above thr a winner slot and each tie its
//      rank in position order; the first `take` ties win;
//   3. each winner's output rank is the number of winners with a larger
//      composite (key << 32 | ~position).
// emit(rank, payload) is called once per winner.  sel holds k composites,
// sel_pay k payloads (LDS, 16-byte aligned).  Requires 0 < k < n; every
// thread of the workgroup calls it (it contains barriers).
template <int T, int LPR, int NC, typename Emit>
__device__ __forceinline__ void select_regs(bool have, uint32_t key, long long pos, int payload, int k,
                                            uint64_t* sel, int32_t* sel_pay, SelectShared<T, NC>& sh, Emit emit) {
  constexpr int kWaves = T / kWave;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = uniform(tid / kWave);
  int hi = 0, above_hi = 0;
  sel_find_bin(sh, 0, (uint32_t)k, &hi, &above_hi);
  if (have && (key >> 8) == (uint32_t)hi) sel_hist_add(sh, 1, key & 255u);
  __syncthreads();
  int lo = 0, above_lo = 0;
  sel_find_bin(sh, 1, (uint32_t)(k - above_hi), &lo, &above_lo);
  const uint32_t thr = ((uint32_t)hi << 8) | (uint32_t)lo;
  const int above = above_hi + above_lo;  // items with a key above thr
  const int take = k - above;             // >= 1 of the items equal to thr win
  const bool gt = have && key > thr;
  const bool tie = have && key == thr;
  const uint64_t mg = __ballot(gt);
  const uint64_t mt = __ballot(tie);
  if (lane == 0) {
    sh.wave_gt[wave] = (uint32_t)__popcll(mg);
    sh.wave_ties[wave] = (uint32_t)__popcll(mt);
  }
  __syncthreads();
  int gt_before = 0, tie_before = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (w < wave) {
      gt_before += (int)sh.wave_gt[w];
      tie_before += (int)sh.wave_ties[w];
    }
  }
  const int tie_rank = tie_before + pass_rank_below<LPR>(mt);
  const bool win = gt || (tie && tie_rank < take);
  const int slot = gt ? gt_before + lanes_below(mg) : above + tie_rank;
  if (win) {
    sel[slot] = sel_composite(key, pos);
    sel_pay[slot] = payload;
  }
  __syncthreads();
  for (int j = tid; j < k; j += T) {
    const uint64_t c = sel[j];
    emit(rank_of_pairs(c, sel, k), sel_pay[j]);
  }
}

// select_regs for kR items per thread at consecutive positions: item u of
// thread tid is at position tid * kR + u (have[u], key[u], payload[u]).
// hist[0] must hold the high-byte counts of every item and hist[1] zeros,
// visible after a barrier.  A thread's count of items above and equal to the
// threshold, an inclusive scan over the wave's lanes and one LDS exchange of
// the wave totals give every item its winner slot.  emit(rank, payload) is
// called once per winner.  Requires 0 < k < n; every thread of the
// workgroup calls it.
template <int T, int kR, int NC, typename Emit>
__device__ __forceinline__ void select_regs_run(const bool (&have)[kR], const uint32_t (&key)[kR],
                                                const int (&payload)[kR], int k, uint64_t* sel, int32_t* sel_pay,
                                                SelectShared<T, NC>& sh, Emit emit) {
  constexpr int kWaves = T / kWave;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = uniform(tid / kWave);
  int hi = 0, above_hi = 0;
  sel_find_bin(sh, 0, (uint32_t)k, &hi, &above_hi);
#pragma unroll
  for (int u = 0; u < kR; ++u)
    if (have[u] && (key[u] >> 8) == (uint32_t)hi) sel_hist_add(sh, 1, key[u] & 255u);
  __syncthreads();
  int lo = 0, above_lo = 0;
  sel_find_bin(sh, 1, (uint32_t)(k - above_hi), &lo, &above_lo);
  const uint32_t thr = ((uint32_t)hi << 8) | (uint32_t)lo;
  const int above = above_hi + above_lo;  // items with a key above thr
  const int take = k - above;             // >= 1 of the items equal to thr win
  uint32_t n_gt = 0, n_tie = 0;
#pragma unroll
  for (int u = 0; u < kR; ++u) {
    n_gt += (have[u] && key[u] > thr) ? 1u : 0u;
    n_tie += (have[u] && key[u] == thr) ? 1u : 0u;
  }
  const uint32_t gt_incl = wave_prefix_sum(n_gt);
  const uint32_t tie_incl = wave_prefix_sum(n_tie);
  if (lane == kWave - 1) {
    sh.wave_gt[wave] = gt_incl;
    sh.wave_ties[wave] = tie_incl;
  }
  __syncthreads();
  int gt_slot = (int)(gt_incl - n_gt), tie_rank = (int)(tie_incl - n_tie);
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (w < wave) {
      gt_slot += (int)sh.wave_gt[w];
      tie_rank += (int)sh.wave_ties[w];
    }
  }
#pragma unroll
  for (int u = 0; u < kR; ++u) {
    const bool gt = have[u] && key[u] > thr;
    const bool tie = have[u] && key[u] == thr;
    if (gt || (tie && tie_rank < take)) {
      const int slot = gt ? gt_slot : above + tie_rank;
      sel[slot] = sel_composite(key[u], (long long)tid * kR + u);
      sel_pay[slot] = payload[u];
    }
    gt_slot += gt ? 1 : 0;
    tie_rank += tie ? 1 : 0;
  }
  __syncthreads();
  for (int j = tid; j < k; j += T) {
    const uint64_t c = sel[j];
    emit(rank_of_pairs(c, sel, k), sel_pay[j]);
  }
}

// Calls emit(rank, position) for every winner (rank 0 = best).
template <int T, typename Emit>
__device__ __forceinline__ void select_emit(const uint64_t* sel, int k, long long n, Emit emit) {
  for (int j = threadIdx.x; j < k; j += T) {
    const uint64_t c = sel[j];
    const long long pos = sel_position(c);
    if (pos < n) emit(rank_of(c, sel, k), pos);
  }
}

// ---------------------------------------------------------------------------
// Bitonic top-k for k <= 32 with at most one item per lane (the fused
// indexer's one-pass segments).  An item is the 32-bit composite
// (key << 16) | (0xffff - position) (positions below 65536; 0 = no item): a
// larger composite is a larger key, then a lower position — the order of a
// stable descending sort, and unique per item.  Each wave sorts its 64
// composites with a bitonic network (21 compare-exchange steps on VALU
// shuffles, no barrier, overlapping the other waves' loads), keeps its best
// 32 in LDS, and the lists are merged pairwise (a 32-descending list against
// a reversed one is bitonic: 6 steps) until wave 0 holds the best 32 in
// order; with eight (four) waves the first round merges four lists per
// wave, so that two barrier rounds remain instead of three (one instead of
// two).  kMaxBitonicK is the largest k it serves.
constexpr int kMaxBitonicK = 32;

__device__ __forceinline__ uint32_t bitonic_comp(bool have, uint32_t key, int pos) {
  return have ? ((key << 16) | (0xffffu - (uint32_t)pos)) : 0u;
}
__device__ __forceinline__ int bitonic_position(uint32_t comp) { return (int)(0xffffu - (comp & 0xffffu)); }

// The wave's 64 values sorted descending (lane 0 the largest).  Every lane
// of the wave must be active.
__device__ __forceinline__ uint32_t wave_sort_desc(uint32_t v) {
  const int i = lane_id();
#pragma unroll
  for (int k2 = 2; k2 <= kWave; k2 <<= 1)
#pragma unroll
    for (int j = k2 >> 1; j > 0; j >>= 1) {
      const uint32_t o = xshfl_u32(v, j);
      const bool keep_max = ((i & j) == 0) == ((i & k2) == 0);
      v = keep_max ? (v > o ? v : o) : (v < o ? v : o);
    }
  return v;
}

// A bitonic sequence over the wave's 64 lanes sorted descending.
__device__ __forceinline__ uint32_t wave_merge_desc(uint32_t v) {
  const int i = lane_id();
#pragma unroll
  for (int j = kWave / 2; j > 0; j >>= 1) {
    const uint32_t o = xshfl_u32(v, j);
    v = (i & j) == 0 ? (v > o ? v : o) : (v < o ? v : o);
  }
  return v;
}

// A bitonic sequence over the wave's 64 lanes sorted ascending.
__device__ __forceinline__ uint32_t wave_merge_asc(uint32_t v) {
  const int i = lane_id();
#pragma unroll
  for (int j = kWave / 2; j > 0; j >>= 1) {
    const uint32_t o = xshfl_u32(v, j);
    v = (i & j) == 0 ? (v < o ? v : o) : (v > o ? v : o);
  }
  return v;
}

// The wave's 64 * kR values sorted descending (defined below).
template <int kR>
__device__ __forceinline__ void wave_sort_desc_run(uint32_t (&v)[kR], int sorted_run = 1);

// LDS of select_bitonic: two buffers of 32 composites per wave.
template <int T>
struct BitonicShared {
  uint32_t cand[2][(T / kWave) * 32];
};

// The k (<= 32) best composites of the workgroup, emit(rank, comp) for rank
// 0 .. k-1 (called by lanes 0 .. k-1 of wave 0).  Every thread of the
// workgroup calls it with its item (0: none); it contains barriers.
// sorted_run: as for wave_sort_desc_run (the items already form sorted runs
// of that length, alternately descending and ascending).
template <int T, typename Emit>
__device__ __forceinline__ void select_bitonic(uint32_t comp, int k, BitonicShared<T>& bs, Emit emit,
                                               int sorted_run = 1) {
  constexpr int kWaves = T / kWave;
  const int lane = lane_id();
  const int wave = uniform(threadIdx.x / kWave);
  uint32_t v = comp;
  if (sorted_run > 1) {  // uniform
    uint32_t r[1] = {comp};
    wave_sort_desc_run<1>(r, sorted_run);
    v = r[0];
  } else {
    v = wave_sort_desc(comp);
  }
  if (lane < 32) bs.cand[0][wave * 32 + lane] = v;
  int buf = 0;
  int w0 = kWaves;
  if constexpr (kWaves == 8 || kWaves == 4) {
    // eight (four) lists of 32 become two (one): wave w < kWaves / 4 takes
    // lists 4w .. 4w + 3, each half-wave the best 32 of a pair (a list
    // against the other reversed: a bitonic 32), the halves sorted in
    // opposite directions (together bitonic), then merged
    __syncthreads();
    if (wave < kWaves / 4) {  // uniform
      const int h = lane >> 5, i = lane & 31;
      const int base = (4 * wave + 2 * h) * 32;
      const uint32_t x = bs.cand[0][base + i], y = bs.cand[0][base + 32 + 31 - i];
      v = x > y ? x : y;
#pragma unroll
      for (int j = 16; j > 0; j >>= 1) {
        const uint32_t o = xshfl_u32(v, j);
        v = (((lane & j) == 0) == (h == 0)) ? (v > o ? v : o) : (v < o ? v : o);
      }
      v = wave_merge_desc(v);
      if (kWaves > 4 && lane < 32) bs.cand[1][wave * 32 + lane] = v;
    }
    buf = 1;
    w0 = kWaves / 4;
  }
#pragma unroll
  for (int w = w0; w > 1; w >>= 1) {  // w lists of 32 become w / 2
    __syncthreads();
    if (wave < w / 2) {  // uniform
      const int src = lane < 32 ? (2 * wave) * 32 + lane : (2 * wave + 1) * 32 + (kWave - 1 - lane);
      v = wave_merge_desc(bs.cand[buf][src]);
      if (w > 2 && lane < 32) bs.cand[buf ^ 1][wave * 32 + lane] = v;
    }
    buf ^= 1;
  }
  if (wave == 0 && lane < k) emit(lane, v);
}

// ---------------------------------------------------------------------------
// The bitonic select for kR items per lane and k <= 64 (the split layout's
// selecting workgroup): lane l of a wave holds elements l * kR + u.  Each
// wave sorts its 64 * kR composites descending (strides below kR inside a
// lane, the others across lanes) and keeps its best 64; pairs of 64-lists are
// merged, one element per lane, keeping the best 64 of each pair, until wave
// 0 holds the best 64 in order.
constexpr int kMaxBitonicRunK = 64;

template <int T>
struct BitonicRunShared {
  uint32_t cand[2][(T / kWave) * 64];
};

// Compare-exchange of the element pair (lo, hi = lo ^ j, lo with bit j
// clear): the lower element keeps the maximum when keep_max.
__device__ __forceinline__ void bitonic_cx(uint32_t& lo, uint32_t& hi, bool keep_max) {
  const uint32_t a = lo > hi ? lo : hi, b = lo > hi ? hi : lo;
  lo = keep_max ? a : b;
  hi = keep_max ? b : a;
}

// The wave's 64 * kR values sorted descending (element lane * kR + u).
// sorted_run (a power of two): the elements already form sorted runs of
// that length, run r descending for even r and ascending for odd r (what
// the network's earlier stages leave), so those stages are skipped.
template <int kR>
__device__ __forceinline__ void wave_sort_desc_run(uint32_t (&v)[kR], int sorted_run) {
  constexpr int N = kWave * kR;
  const int lane = lane_id();
#pragma unroll
  for (int k2 = 2; k2 <= N; k2 <<= 1) {
    if (k2 <= sorted_run) continue;  // uniform
#pragma unroll
    for (int j = k2 >> 1; j > 0; j >>= 1) {
      if (j < kR) {
#pragma unroll
        for (int u = 0; u < kR; ++u)
          if ((u & j) == 0) bitonic_cx(v[u], v[u | j], ((lane * kR + u) & k2) == 0);
      } else {
#pragma unroll
        for (int u = 0; u < kR; ++u) {
          const uint32_t o = xshfl_u32(v[u], j / kR);
          const int e = lane * kR + u;
          const bool keep_max = ((e & j) == 0) == ((e & k2) == 0);
          v[u] = keep_max ? (v[u] > o ? v[u] : o) : (v[u] < o ? v[u] : o);
        }
      }
    }
  }
}

// The k (<= 64) best of the T / 64 lists of 64 composites in bs.cand[0]
// (list w at w * 64, each sorted descending, 0 for no item), merged pairwise
// until wave 0 holds the best 64 in order: emit(rank, comp) for rank
// 0 .. k-1, from lanes 0 .. k-1 of wave 0.  A pair's best 64 are, lane by
// lane, the larger of list a's place l and list b's place 63 - l (the first
// compare-exchange of the bitonic merge of a and reversed b; the smaller
// halves are dropped), a bitonic sequence that 6 steps sort (one register
// per lane).  Every thread of the workgroup calls it; it starts with a
// barrier (after which bs.cand[0] and whatever else the caller wrote to LDS
// are visible) and holds one per merge round.
template <int T, typename Emit>
__device__ __forceinline__ void merge_lists_bitonic_run(int k, BitonicRunShared<T>& bs, Emit emit) {
  constexpr int kWaves = T / kWave;
  static_assert(kWaves >= 2, "two or more lists");
  const int lane = lane_id();
  const int wave = uniform(threadIdx.x / kWave);
  uint32_t v = 0u;
  int buf = 0;
  int w0 = kWaves;
  if constexpr (kWaves == 4 || kWaves == 8) {
    // first round, four lists per wave (wave w < kWaves / 4 takes lists
    // 4w .. 4w + 3): each pair to its best 64, one sorted descending and
    // the other ascending (together bitonic), then the best 64 of both
    __syncthreads();
    if (wave < kWaves / 4) {  // uniform
      const int b0 = 4 * wave * 64;
      const uint32_t a = bs.cand[0][b0 + lane], b = bs.cand[0][b0 + 64 + 63 - lane];
      const uint32_t c = bs.cand[0][b0 + 128 + lane], d = bs.cand[0][b0 + 192 + 63 - lane];
      const uint32_t x = wave_merge_desc(a > b ? a : b);
      const uint32_t y = wave_merge_asc(c > d ? c : d);
      v = wave_merge_desc(x > y ? x : y);
      if (kWaves > 4) bs.cand[1][wave * 64 + lane] = v;
    }
    buf = 1;
    w0 = kWaves / 4;
  }
#pragma unroll
  for (int w = w0; w > 1; w >>= 1) {  // w lists of 64 become w / 2
    __syncthreads();
    if (wave < w / 2) {  // uniform
      const uint32_t a = bs.cand[buf][(2 * wave) * 64 + lane];
      const uint32_t b = bs.cand[buf][(2 * wave + 1) * 64 + 63 - lane];
      v = wave_merge_desc(a > b ? a : b);
      if (w > 2) bs.cand[buf ^ 1][wave * 64 + lane] = v;
    }
    buf ^= 1;
  }
  if (wave == 0 && lane < k) emit(lane, v);
}

// The k (<= 64) best of the workgroup's composites, kR per thread (0: none):
// each wave sorts its 64 * kR composites descending (strides below kR inside
// a lane, the others across lanes) and keeps its best 64, then the lists are
// merged (merge_lists_bitonic_run).  emit(rank, comp) for rank 0 .. k-1,
// from wave 0.  sorted_run: as for wave_sort_desc_run.  Every thread of the
// workgroup calls it; it contains barriers.
template <int T, int kR, typename Emit>
__device__ __forceinline__ void select_bitonic_run(uint32_t (&comp)[kR], int k, BitonicRunShared<T>& bs, Emit emit,
                                                   int sorted_run = 1) {
  static_assert(kR >= 1 && (kR & (kR - 1)) == 0 && 64 % kR == 0, "kR: a power of two dividing 64");
  constexpr int kWaves = T / kWave;
  const int lane = lane_id();
  const int wave = uniform(threadIdx.x / kWave);
  if constexpr (kR == 2 && kWaves > 1) {
    if (sorted_run >= 64) {  // uniform: two sorted runs of 64, the second ascending
      // the wave's best 64: element e of the first run against element
      // e + 64 (lane + 32, same register), then lane i takes the i-th and
      // the bitonic sequence is sorted in 6 steps
      uint32_t top[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t o = xshfl_u32(comp[u], 32);
        top[u] = comp[u] > o ? comp[u] : o;
      }
      const uint32_t t0 = (uint32_t)__shfl((int)top[0], lane >> 1, kWave);
      const uint32_t t1 = (uint32_t)__shfl((int)top[1], lane >> 1, kWave);
      bs.cand[0][wave * 64 + lane] = wave_merge_desc((lane & 1) ? t1 : t0);
      merge_lists_bitonic_run<T>(k, bs, emit);
      return;
    }
  }
  wave_sort_desc_run<kR>(comp, sorted_run);
  if constexpr (kWaves == 1) {
#pragma unroll
    for (int u = 0; u < kR; ++u)
      if (lane * kR + u < k) emit(lane * kR + u, comp[u]);
    return;
  } else {
    if (lane * kR < 64) {
#pragma unroll
      for (int u = 0; u < kR; ++u) bs.cand[0][wave * 64 + lane * kR + u] = comp[u];
    }
    merge_lists_bitonic_run<T>(k, bs, emit);
  }
}

}  // namespace vtx
