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
// Row scoring: a segment's middle pages are split evenly over the waves, at
// most kPass pages per wave pass (64 for rows of one 16-byte vector per lane,
// 32 for wider rows), LPR lanes x VPL 16-byte vectors per row.  The per-lane
// dot product (vtx::dot_row) and the reduce-scatter tree over the LPR lanes
// are the ones gemv.hip uses, so the scores are bit-identical to the GeMV
// kernel's for the same query.
#include "vtx_device.h"
#include "vtx_host.h"
#include "vtx_select.h"

namespace {

struct FusedArgs {
  const uint16_t* q;  // [S, G, D] when G > 0
  int32_t G;
  float inv_g;        // 1.0f / G
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
};

// Query row of segment `seg` for this lane's columns: the bf16-rounded
// fp32 mean of its G rows (torch's mean), or the row itself when G == 0.
// Lane group 0 of wave 0 also stores the mean to x_out.
template <int LPR, int VPL, int kQRegs>
__device__ __forceinline__ void query_row(const FusedArgs& a, const vtx::U4 (&qv)[kQRegs][VPL],
                                          bool q_in_regs, const uint16_t* qb, int seg, int wave,
                                          int grp, int col, float (&xs)[VPL][8]) {
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
    if (a.x_out && wave == 0 && grp == 0) {
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
      const vtx::U4 t = vtx::ld16(qb + (v * LPR + col) * 8);
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

template <int T, int LPR, int VPL>
__global__ __launch_bounds__(T, (VPL == 1 ? 4 : 2)) void indexer_fused_kernel(FusedArgs a) {
  constexpr int kWaves = T / vtx::kWave;
  constexpr int kRowsPerLoad = vtx::kWave / LPR;
  constexpr int kPass = VPL == 1 ? 64 : 32;        // at most this many pages per wave pass
  constexpr int kSlots = kPass / kRowsPerLoad;     // pages per lane per pass
  constexpr int kBatch = VPL <= 2 ? kSlots : 2;    // slots loaded together
  constexpr int kQRegs = VPL <= 2 ? 2 : 1;         // query rows prefetched
  static_assert(kSlots >= 1 && kSlots <= LPR, "pass geometry");
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ vtx::SelectShared<T> sh;

  const int seg = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = vtx::lane_id();
  const int wave = tid / vtx::kWave;
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int k = a.topk;
  const int D = a.dim;

  // ---- 1. query rows (issued first: only needed once centroid rows arrive)
  vtx::U4 qv[kQRegs][VPL];
  const bool q_in_regs = a.G > 0 && a.G <= kQRegs;
  const uint16_t* qb = a.G > 0 ? a.q + (long long)seg * a.G * D : a.x + (long long)seg * D;
  if (q_in_regs) {
#pragma unroll
    for (int g = 0; g < kQRegs; ++g)
#pragma unroll
      for (int v = 0; v < VPL; ++v)
        qv[g][v] = g < a.G ? vtx::ld16(qb + (long long)g * D + (v * LPR + col) * 8) : vtx::U4{0u, 0u, 0u, 0u};
  }

  // ---- 2. segment bounds
  const bool is_seg = seg < a.segments;
  long long start = 0, n = 0, obase = 0;
  if (is_seg) {
    start = (long long)a.dindptr[seg] + a.bos;
    n = (long long)a.dindptr[seg + 1] - a.eos - start;
    obase = (long long)a.sindptr[seg] + a.bos;
  }
  bool active = is_seg && k > 0 && n > k;
  if (active && (start < 0 || start + n > a.score_len || start + n > a.didx_len || obase < 0 ||
                 obase + k > a.sidx_len))
    active = false;
  const bool cached = active && n <= a.row_cap;
  uint64_t* sel = reinterpret_cast<uint64_t*>(smem);
  int32_t* rows = reinterpret_cast<int32_t*>(smem + (size_t)k * sizeof(uint64_t));
  uint16_t* keys = reinterpret_cast<uint16_t*>(rows + a.row_cap);

  // ---- 3. query mean (bf16 of the fp32 mean, as torch's mean rounds it);
  // evaluated after the first row ids are requested so the waits overlap
  float xs[VPL][8];
  if (!active) {  // uniform over the workgroup
    if (a.x_out) query_row<LPR, VPL, kQRegs>(a, qv, q_in_regs, qb, seg, wave, grp, col, xs);
    return;
  }
  vtx::select_init<T>(sel, k, sh);
  __syncthreads();  // histogram cleared before any wave counts into it
  bool have_mean = false;

  // ---- 4. scores: the pages are split evenly over the waves (one pass
  // each up to kWaves * kPass pages, so no wave waits on a second round
  // trip while others idle); row ids come straight from global memory
  const int32_t* dseg = a.didx + start;
  long long share = (n + kWaves - 1) / kWaves;
  share = (share + kRowsPerLoad - 1) / kRowsPerLoad * kRowsPerLoad;
  if (share > kPass) share = kPass;
  for (long long p0 = (long long)wave * share; p0 < n; p0 += (long long)kWaves * share) {
    const int cnt = (int)min(share, n - p0);
    // one coalesced load of the pass's row ids (lane l holds position l),
    // handed to the lanes that need them with shuffles
    const int my_row = lane < cnt ? dseg[p0 + lane] : -1;
    if (!have_mean) {
      query_row<LPR, VPL, kQRegs>(a, qv, q_in_regs, qb, seg, wave, grp, col, xs);
      have_mean = true;
    }
    int first = __shfl(my_row, 0, vtx::kWave);
    if (first < 0 || first >= a.y_rows) first = 0;
    float acc[kSlots];
#pragma unroll
    for (int i0 = 0; i0 < kSlots; i0 += kBatch) {
      vtx::U4 buf[kBatch][VPL];
      bool live[kBatch];
#pragma unroll
      for (int ii = 0; ii < kBatch; ++ii) {
        const int row = __shfl(my_row, (i0 + ii) * kRowsPerLoad + grp, vtx::kWave);
        live[ii] = row >= 0 && row < a.y_rows;
        if ((i0 + ii) * kRowsPerLoad < cnt) {  // wave-uniform: slots past the share are skipped
          const uint16_t* yr = a.y + (long long)(live[ii] ? row : first) * D;
#pragma unroll
          for (int v = 0; v < VPL; ++v) buf[ii][v] = vtx::ld16(yr + (v * LPR + col) * 8);
        } else {
#pragma unroll
          for (int v = 0; v < VPL; ++v) buf[ii][v] = vtx::U4{0u, 0u, 0u, 0u};
        }
      }
#pragma unroll
      for (int ii = 0; ii < kBatch; ++ii) {
        const float s = vtx::dot_row<VPL>(buf[ii], xs);
        acc[i0 + ii] = live[ii] ? s : 0.f;
      }
    }
    // Reduce-scatter over the slots (lane keeps slot bits of col from the
    // top), then fold the lanes that still share a slot.
#pragma unroll
    for (int half = kSlots / 2, stride = LPR / 2; half >= 1; half >>= 1, stride >>= 1) {
      const bool upper = (col & stride) != 0;
#pragma unroll
      for (int t = 0; t < half; ++t) {
        const float send = upper ? acc[t] : acc[t + half];
        const float keep = upper ? acc[t + half] : acc[t];
        acc[t] = keep + __shfl_xor(send, stride, vtx::kWave);
      }
    }
    constexpr int kShare = LPR / kSlots;  // lanes holding the same slot
#pragma unroll
    for (int d = 1; d < kShare; d <<= 1) acc[0] += __shfl_xor(acc[0], d, vtx::kWave);
    const int slot = col / kShare;
    const int r = slot * kRowsPerLoad + grp;
    const int my_rid = __shfl(my_row, r, vtx::kWave);  // row id of this lane's page
    if ((col % kShare) == 0 && r < cnt) {
      const uint32_t sb = vtx::f32_to_bf16(acc[0]);
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
  for (int j = tid; j < k; j += T) {
    const uint64_t c = sel[j];
    const long long pos = vtx::sel_position(c);
    if (pos < n) a.sidx[obase + vtx::rank_of(c, sel, k)] = cached ? rows[pos] : dseg[pos];
  }
}

constexpr int kLdsBudget = 60 * 1024;
constexpr int kMaxTopk = 4096;

template <int T>
int launch_dim(const FusedArgs& a, int blocks, size_t lds, hipStream_t s) {
  switch (a.dim) {
    case 64: indexer_fused_kernel<T, 8, 1><<<blocks, T, lds, s>>>(a); break;
    case 128: indexer_fused_kernel<T, 16, 1><<<blocks, T, lds, s>>>(a); break;
    case 256: indexer_fused_kernel<T, 16, 2><<<blocks, T, lds, s>>>(a); break;
    case 512: indexer_fused_kernel<T, 16, 4><<<blocks, T, lds, s>>>(a); break;
    case 576: indexer_fused_kernel<T, 8, 9><<<blocks, T, lds, s>>>(a); break;
    default: return vtx::fail(VTX_E_INVALID, "indexer_fused: head_dim %d not supported", a.dim);
  }
  return vtx::check_launch("indexer_fused");
}

}  // namespace

extern "C" int vtx_indexer_fused_supported(int32_t head_dim) {
  return head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512 || head_dim == 576;
}

extern "C" int vtx_indexer_fused(const uint16_t* q, int64_t q_rows, int32_t group_size,
                                 const uint16_t* x, uint16_t* x_out, const uint16_t* y,
                                 int64_t y_rows, uint16_t* score, int64_t score_len,
                                 const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr,
                                 const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                                 int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                                 int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos,
                                 int32_t reserved_eos, int32_t max_num_pages, int32_t head_dim,
                                 void* stream) {
  vtx::clear_error();
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
  a.inv_g = group_size > 0 ? 1.0f / (float)group_size : 1.0f;
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

  long long want = max_num_pages > 0 ? max_num_pages : 0;
  const long long room = (kLdsBudget - (long long)a.topk * 8) / 6;
  long long cap = want < room ? want : room;
  cap &= ~7LL;
  if (cap < 0) cap = 0;
  a.row_cap = (int32_t)cap;
  const size_t lds = (size_t)a.topk * 8 + (size_t)cap * 6;

  a.segments = eff_batch_size;
  // With a q_mean output every query row gets a workgroup (rows past the
  // segments only write their mean).
  const long long grid = a.x_out ? q_rows : eff_batch_size;
  if (grid > 0x7fffffffLL) return vtx::fail(VTX_E_INVALID, "indexer_fused: too many query rows");
  if (grid == 0) return VTX_OK;

  hipStream_t s = vtx::as_stream(stream);
  if (max_num_pages <= 256) return launch_dim<256>(a, (int)grid, lds, s);
  if (max_num_pages <= 1024) return launch_dim<512>(a, (int)grid, lds, s);
  return launch_dim<1024>(a, (int)grid, lds, s);
}
