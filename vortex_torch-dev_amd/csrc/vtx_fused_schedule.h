// The fused indexer's workgroup schedule: which segment each workgroup of a
// segment-layout launch takes, written by the decode planner.
//
// One workgroup per segment fills the chip in rounds of one workgroup per
// compute unit, and the hardware places workgroup b and b + CUs on the same
// compute unit.  With the segments in their natural order a unit can hold two
// long segments while another holds two short ones, and the launch ends when
// the busiest unit does.  The planner sorts the segments by page count (fewer
// pages first, ties by segment index) and deals them to workgroups in snake
// order over rounds of `round` workgroups: round 0, dispatched first, takes
// the shortest segments in order, round 1 the next ones in reverse order (the
// longest, for S = 2 * round), and so on, so that every unit gets a short and
// a long segment.  (Measured at C2: the long segments dispatched second end
// sooner than the other way round, and the short ones, done first, carry the
// in-launch CMean's tiles.)
//
// Layout (int32): a header {kSchedMagic, S, round, 0}, then for workgroup w
// {segment, dense_kv_indptr[segment], dense_kv_indptr[segment + 1],
//  sparse_kv_indptr[segment]}.
//
// The schedule only steers speed: the fused kernel uses it when the header
// names the launch's segment count, takes the bounds it holds as a
// prediction, and checks them against the block tables in the same memory
// round trip (a mismatch costs one more trip, never a wrong result).  Every
// schedule the planner writes is a permutation of the S segments.
#pragma once

#include <stdint.h>

namespace vtx {

constexpr int32_t kSchedMagic = 0x56545853;  // "VTXS"

__host__ __device__ inline long long sched_len(long long batch, long long heads) {
  return 4 + 4 * batch * heads;
}

// Workgroup of the i-th shortest of S segments (snake order over rounds of
// `round` workgroups); an involution of [0, S).
__host__ __device__ inline long long sched_slot(long long i, long long S, long long round) {
  const long long r = i / round;
  if ((r & 1) == 0) return i;
  const long long end = (r + 1) * round < S ? (r + 1) * round : S;
  return end - 1 - (i - r * round);
}

__device__ __forceinline__ void sched_write_header(int32_t* s, int32_t segments, int32_t round) {
  s[0] = kSchedMagic;
  s[1] = segments;
  s[2] = round;
  s[3] = 0;
}

// Rank of workgroup b's segment counted from the shortest (0 = shortest)
// under a schedule of S segments and rounds of `round`; workgroups past the
// segments keep their index.  A permutation of the launch's workgroups, which
// puts side work (the in-launch CMean's tiles) on the workgroups that finish
// first.  32-bit arithmetic (one unsigned division), for the kernel's head.
__device__ __forceinline__ int sched_short_rank32(uint32_t b, uint32_t S, uint32_t round) {
  if (b >= S) return (int)b;
  const uint32_t r = b / round;
  if ((r & 1u) == 0) return (int)b;
  const uint32_t end = (r + 1u) * round < S ? (r + 1u) * round : S;
  return (int)(end - 1u - (b - r * round));
}

// What workgroup blockIdx.x of a one-workgroup-per-segment launch takes:
// its segment, whether the schedule names this launch (then pe holds the
// predicted dense begin, dense end and sparse begin, to be checked against
// the indptrs before anything is written), and its rank for side work
// (sched_short_rank32).  Without a schedule (sched null): segment blockIdx.x.
// The header and the entry are loaded together, and everything after them
// is branch-free: a load whose value is used only inside a branch is moved
// into it, and the entry would then wait for the header.
struct SchedPick {
  int seg;
  bool predicted;
  int32_t pe[3];
  int tile_rank;
};

__device__ __forceinline__ SchedPick sched_pick(const int32_t* sched, int32_t segments) {
  SchedPick p{(int)blockIdx.x, false, {0, 0, 0}, (int)blockIdx.x};
  if (sched) {  // uniform
    // workgroups past the segments read the last entry and ignore it
    const bool mine = (int)blockIdx.x < segments;
    const int32_t* e = sched + 4 + 4 * (long long)(mine ? blockIdx.x : segments - 1);
    const int32_t h0 = sched[0], h1 = sched[1], h2 = sched[2];
    const int32_t e0 = e[0], e1 = e[1], e2 = e[2], e3 = e[3];
    const bool ok = (h0 == kSchedMagic) & (h1 == segments) & (h2 >= 1);
    p.predicted = mine & ok & (e0 >= 0) & (e0 < segments);
    p.seg = p.predicted ? e0 : p.seg;
    p.pe[0] = e1;  // read only when predicted
    p.pe[1] = e2;
    p.pe[2] = e3;
    const int32_t rounds = h2 >= 1 ? h2 : 1;
    const int rank = sched_short_rank32(blockIdx.x, (uint32_t)segments, (uint32_t)rounds);
    p.tile_rank = ok ? rank : p.tile_rank;
  }
  return p;
}

__device__ __forceinline__ void sched_write_entry(int32_t* s, long long wg, int32_t seg, int32_t dense_begin,
                                                  int32_t dense_end, int32_t sparse_begin) {
  int32_t* e = s + 4 + 4 * wg;
  e[0] = seg;
  e[1] = dense_begin;
  e[2] = dense_end;
  e[3] = sparse_begin;
}

}  // namespace vtx
