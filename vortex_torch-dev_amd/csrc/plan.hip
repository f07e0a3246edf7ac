// Decode planner for gfx950: dense/sparse block tables, last-page lengths and
// the GeMV workload list, in one launch.
//
// Semantics follow the reference planner (csrc/utils_sglang.cu:123-309,
// host 313-460).  Design: grid (request b, page slab y).  Every workgroup
// derives its request's offsets from a block-wide sum over the earlier
// requests' lengths, so no cross-workgroup scan (and no second launch) is
// needed; slab 0 of each request also writes the request's indptr entries,
// last-page lengths and workload entries.  One thread per page reads the
// page's first token slot from req_to_token once and writes that page's
// entry for all H kv heads (consecutive threads -> consecutive addresses).
#include "vtx_device.h"
#include "vtx_fused_schedule.h"
#include "vtx_host.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPagesPerSlab = kThreads;

struct PlanArgs {
  const int32_t* seq_lens;
  int32_t batch;
  int32_t* dense_indptr;
  int32_t* dense_idx;
  int64_t dense_cap;
  int32_t* sparse_indptr;
  int32_t* sparse_idx;
  int64_t sparse_cap;
  int32_t* last_len;
  const int32_t* r2t;
  int64_t r2t_rows;
  int64_t r2t_stride;
  const int64_t* req_idx;
  int32_t* wq;
  int32_t* woff;
  int32_t* wlen;
  int64_t wcap;
  int32_t* wnum;
  int32_t* wchunk;
  // FA3 variant outputs (all optional): per-segment page tables
  // [pt_rows, pt_stride] and per-segment cache sequence lengths
  int32_t* dpt;
  int32_t* spt;
  int64_t pt_rows;
  int64_t pt_stride;
  int32_t* dcs;
  int32_t* scs;
  int64_t cs_len;
  // optional: the fused indexer's workgroup schedule (vtx_fused_schedule.h)
  int32_t* sched;
  int64_t sched_len;
  int32_t sched_round;
  int32_t page, heads, topk, bos, eos, chunk;
};

__device__ __forceinline__ int pages_of(int32_t len, int32_t page) {
  return (len + page - 1) / page;
}

// Middle pages the GeMV scores for one segment of n pages: the reference
// stores n - bos - eos in an int16 and keeps it only when it exceeds topk
// (csrc/utils_sglang.cu:221-225).
__device__ __forceinline__ int middle_pages(int n, const PlanArgs& a) {
  const int16_t w = (int16_t)(n - a.bos - a.eos);
  return ((int)w > a.topk) ? (int)(uint16_t)w : 0;
}

__device__ __forceinline__ int chunks_of(int n, const PlanArgs& a) {
  return (middle_pages(n, a) + a.chunk - 1) / a.chunk;
}

__global__ __launch_bounds__(kThreads) void plan_decode_kernel(PlanArgs a) {
  __shared__ long long part[4][kThreads / vtx::kWave];
  const int b = blockIdx.x;
  const int slab = blockIdx.y;
  const int tid = threadIdx.x;

  const bool want_sched = a.sched && a.sched_len >= vtx::sched_len(a.batch, a.heads);
  if (a.batch == 0) {
    if (b == 0 && slab == 0 && tid == 0) {
      a.dense_indptr[0] = 0;
      a.sparse_indptr[0] = 0;
      *a.wnum = 0;
      *a.wchunk = a.chunk;
      if (want_sched) vtx::sched_write_header(a.sched, 0, a.sched_round);
    }
    return;
  }

  const int budget = a.topk + a.bos + a.eos;
  const bool head_slab = (slab == 0);

  // Offsets of request b: sums over requests b' < b; with a schedule, also
  // the request's rank by page count (fewer pages first, ties by index).
  const int L = a.seq_lens[b];
  const int n = pages_of(L, a.page);
  const bool rank_it = head_slab && want_sched;
  long long sd = 0, ss = 0, sc = 0, rk = 0;
  const int scan_to = rank_it ? a.batch : b;
  for (int r = tid; r < scan_to; r += kThreads) {
    const int nr = pages_of(a.seq_lens[r], a.page);
    if (r < b) {
      sd += nr;
      ss += min(budget, nr);
      if (head_slab) sc += chunks_of(nr, a);
    }
    if (rank_it) rk += (nr < n || (nr == n && r < b)) ? 1 : 0;
  }
  sd = vtx::wave_sum(sd);
  ss = vtx::wave_sum(ss);
  sc = vtx::wave_sum(sc);
  rk = vtx::wave_sum(rk);
  const int wave = tid / vtx::kWave;
  if (vtx::lane_id() == 0) {
    part[0][wave] = sd;
    part[1][wave] = ss;
    part[2][wave] = sc;
    part[3][wave] = rk;
  }
  __syncthreads();
  sd = ss = sc = rk = 0;
#pragma unroll
  for (int w = 0; w < kThreads / vtx::kWave; ++w) {
    sd += part[0][w];
    ss += part[1][w];
    sc += part[2][w];
    rk += part[3][w];
  }

  const int H = a.heads;
  const int sn = min(budget, n);
  const long long dbase = (long long)H * sd;
  const long long sbase = (long long)H * ss;

  if (head_slab) {
    const int rem = L % a.page;
    const int last_page = (rem == 0) ? a.page : rem;
    for (int h = tid; h < H; h += kThreads) {
      const long long s = (long long)b * H + h;
      a.dense_indptr[s] = (int32_t)(dbase + (long long)h * n);
      a.sparse_indptr[s] = (int32_t)(sbase + (long long)h * sn);
      if (a.last_len) a.last_len[s] = last_page;
      if (s < a.cs_len) {
        // FA3: the KV length each segment's attention reads (all of it, or
        // the budget's pages with the last one partial)
        if (a.dcs) a.dcs[s] = L;
        if (a.scs) a.scs[s] = (int32_t)min((long long)(budget - 1) * a.page + last_page, (long long)L);
      }
    }
    const int mid = middle_pages(n, a);
    const int ck = (mid + a.chunk - 1) / a.chunk;
    int last = mid % a.chunk;
    if (last == 0) last = a.chunk;
    const long long wbase = (long long)H * sc;
    const int total = H * ck;
    for (int t = tid; t < total; t += kThreads) {
      const int h = t / ck;
      const int k = t - h * ck;
      const long long wi = wbase + t;
      if (wi < a.wcap) {
        a.wq[wi] = b * H + h;
        a.wlen[wi] = (k != ck - 1) ? a.chunk : last;
        a.woff[wi] = (int32_t)(dbase + (long long)h * n + (long long)k * a.chunk + a.bos);
      }
    }
    if (rank_it) {  // this request's segments in the fused indexer's workgroup order
      const long long S = (long long)a.batch * H;
      for (int h = tid; h < H; h += kThreads) {
        const long long s = (long long)b * H + h;
        const long long wg = vtx::sched_slot(rk * H + h, S, a.sched_round);
        vtx::sched_write_entry(a.sched, wg, (int32_t)s, (int32_t)(dbase + (long long)h * n),
                               (int32_t)(dbase + (long long)(h + 1) * n), (int32_t)(sbase + (long long)h * sn));
      }
      if (b == 0 && tid == 0) vtx::sched_write_header(a.sched, (int32_t)S, a.sched_round);
    }
    if (b == a.batch - 1 && tid == 0) {
      const long long s = (long long)a.batch * H;
      a.dense_indptr[s] = (int32_t)(dbase + (long long)H * n);
      a.sparse_indptr[s] = (int32_t)(sbase + (long long)H * sn);
      const long long nw = wbase + total;
      *a.wnum = (int32_t)(nw < a.wcap ? nw : a.wcap);
      *a.wchunk = a.chunk;
    }
  }

  // Block-table entries of the pages in this slab.
  const long long j = (long long)slab * kPagesPerSlab + tid;
  if (j >= n) return;
  const long long ri = a.req_idx[b];
  const long long col = j * a.page;
  if (ri < 0 || ri >= a.r2t_rows || col >= a.r2t_stride) return;
  const int32_t tok = a.r2t[ri * a.r2t_stride + col];
  const int32_t phys = tok / a.page;
  const bool copy_all = (n <= budget);
  const bool is_bos = j < a.bos;
  const bool is_eos = j >= (long long)n - a.eos;
  // position of this page in the segment's sparse list (-1: left for top-k)
  const long long lp = (copy_all || is_bos) ? j : (is_eos ? budget - n + j : -1);
  for (int h = 0; h < H; ++h) {
    const int32_t v = phys * H + h;
    const long long s = (long long)b * H + h;
    const long long di = dbase + (long long)h * n + j;
    if (di < a.dense_cap) a.dense_idx[di] = v;
    const long long si = lp >= 0 ? sbase + (long long)h * sn + lp : -1;
    if (si >= 0 && si < a.sparse_cap) a.sparse_idx[si] = v;
    if (s < a.pt_rows) {
      if (a.dpt && j < a.pt_stride) a.dpt[s * a.pt_stride + j] = v;
      if (a.spt && lp >= 0 && lp < a.pt_stride) a.spt[s * a.pt_stride + lp] = v;
    }
  }
}

// Validates the arguments shared by both planners, fills `a` and launches.
// With kv_last_page_len NULL (the FA3 variant) that output is not written.
int plan_launch(PlanArgs& a, const char* what, const int32_t* cached_seq_lens, int32_t batch_size,
                int32_t* dense_kv_indptr, int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                int32_t* sparse_kv_indptr, int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                int32_t* kv_last_page_len, bool need_last_len, const int32_t* req_to_token,
                int64_t req_to_token_rows, int64_t req_to_token_stride, const int64_t* req_indices,
                int32_t* winfo_q_indices, int32_t* winfo_kv_offsets, int32_t* winfo_kv_lens, int64_t winfo_capacity,
                int32_t* winfo_num_workloads, int32_t* winfo_chunk_size, int32_t page_size, int32_t num_kv_heads,
                int32_t topk_val, int32_t page_reserved_bos, int32_t page_reserved_eos, int32_t max_chunk_size,
                void* stream) {
  if (batch_size < 0) return vtx::fail(VTX_E_INVALID, "%s: batch_size < 0", what);
  if (a.sched && a.sched_round < 1) return vtx::fail(VTX_E_INVALID, "%s: schedule round must be >= 1", what);
  if (page_size < 1 || num_kv_heads < 1 || max_chunk_size < 1)
    return vtx::fail(VTX_E_INVALID,
                     "%s: page_size (%d), num_kv_heads (%d) and max_chunk_size (%d) must be >= 1", what,
                     page_size, num_kv_heads, max_chunk_size);
  if (topk_val < 0 || page_reserved_bos < 0 || page_reserved_eos < 0)
    return vtx::fail(VTX_E_INVALID, "%s: topk/bos/eos must be >= 0", what);
  if (!cached_seq_lens && batch_size > 0) return vtx::fail(VTX_E_INVALID, "%s: null cached_seq_lens", what);
  if (!dense_kv_indptr || !sparse_kv_indptr || !winfo_num_workloads || !winfo_chunk_size)
    return vtx::fail(VTX_E_INVALID, "%s: null output pointer", what);
  if (batch_size > 0 && (!dense_kv_indices || !sparse_kv_indices || (need_last_len && !kv_last_page_len) ||
                         !req_to_token || !req_indices || req_to_token_stride < 1))
    return vtx::fail(VTX_E_INVALID, "%s: null input/output pointer or empty req_to_token", what);
  if (batch_size > 0 && (winfo_capacity > 0) && (!winfo_q_indices || !winfo_kv_offsets || !winfo_kv_lens))
    return vtx::fail(VTX_E_INVALID, "%s: null winfo pointer", what);

  a.seq_lens = cached_seq_lens;
  a.batch = batch_size;
  a.dense_indptr = dense_kv_indptr;
  a.dense_idx = dense_kv_indices;
  a.dense_cap = dense_kv_indices_len;
  a.sparse_indptr = sparse_kv_indptr;
  a.sparse_idx = sparse_kv_indices;
  a.sparse_cap = sparse_kv_indices_len;
  a.last_len = kv_last_page_len;
  a.r2t = req_to_token;
  a.r2t_rows = req_to_token_rows;
  a.r2t_stride = req_to_token_stride;
  a.req_idx = req_indices;
  a.wq = winfo_q_indices;
  a.woff = winfo_kv_offsets;
  a.wlen = winfo_kv_lens;
  a.wcap = winfo_capacity;
  a.wnum = winfo_num_workloads;
  a.wchunk = winfo_chunk_size;
  a.page = page_size;
  a.heads = num_kv_heads;
  a.topk = topk_val;
  a.bos = page_reserved_bos;
  a.eos = page_reserved_eos;
  a.chunk = max_chunk_size;

  const long long max_pages = batch_size > 0 ? (req_to_token_stride + page_size - 1) / page_size : 1;
  long long slabs = (max_pages + kPagesPerSlab - 1) / kPagesPerSlab;
  if (slabs < 1) slabs = 1;
  if (slabs > 65535) return vtx::fail(VTX_E_INVALID, "plan_decode: req_to_token row too long");
  dim3 grid(batch_size > 0 ? batch_size : 1, (unsigned)slabs);
  plan_decode_kernel<<<grid, kThreads, 0, vtx::as_stream(stream)>>>(a);
  return vtx::check_launch(what);
}

}  // namespace

extern "C" int vtx_plan_decode(
    const int32_t* cached_seq_lens, int32_t batch_size, int32_t* dense_kv_indptr,
    int32_t* dense_kv_indices, int64_t dense_kv_indices_len, int32_t* sparse_kv_indptr,
    int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len, int32_t* kv_last_page_len,
    const int32_t* req_to_token, int64_t req_to_token_rows, int64_t req_to_token_stride,
    const int64_t* req_indices, int32_t* winfo_q_indices, int32_t* winfo_kv_offsets,
    int32_t* winfo_kv_lens, int64_t winfo_capacity, int32_t* winfo_num_workloads,
    int32_t* winfo_chunk_size, int32_t page_size, int32_t num_kv_heads, int32_t topk_val,
    int32_t page_reserved_bos, int32_t page_reserved_eos, int32_t max_chunk_size,
    int32_t min_chunk_size, int32_t* fused_schedule, int64_t fused_schedule_len, int32_t schedule_round,
    void* stream) {
  vtx::clear_error();
  (void)min_chunk_size;  // sizes the caller's winfo capacity only
  PlanArgs a{};
  a.sched = fused_schedule;
  a.sched_len = fused_schedule ? fused_schedule_len : 0;
  a.sched_round = schedule_round;
  return plan_launch(a, "plan_decode", cached_seq_lens, batch_size, dense_kv_indptr, dense_kv_indices,
                     dense_kv_indices_len, sparse_kv_indptr, sparse_kv_indices, sparse_kv_indices_len,
                     kv_last_page_len, true, req_to_token, req_to_token_rows, req_to_token_stride, req_indices,
                     winfo_q_indices, winfo_kv_offsets, winfo_kv_lens, winfo_capacity, winfo_num_workloads,
                     winfo_chunk_size, page_size, num_kv_heads, topk_val, page_reserved_bos, page_reserved_eos,
                     max_chunk_size, stream);
}

extern "C" int vtx_plan_decode_fa3(
    const int32_t* cached_seq_lens, int32_t batch_size, int32_t* dense_kv_indptr,
    int32_t* dense_kv_indices, int64_t dense_kv_indices_len, int32_t* sparse_kv_indptr,
    int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len, int32_t* dense_page_table,
    int32_t* dense_cache_seqlens, int32_t* sparse_page_table, int32_t* sparse_cache_seqlens,
    int64_t page_table_rows, int64_t page_table_stride, int64_t cache_seqlens_len,
    const int32_t* req_to_token, int64_t req_to_token_rows, int64_t req_to_token_stride,
    const int64_t* req_indices, int32_t* winfo_q_indices, int32_t* winfo_kv_offsets,
    int32_t* winfo_kv_lens, int64_t winfo_capacity, int32_t* winfo_num_workloads,
    int32_t* winfo_chunk_size, int32_t page_size, int32_t num_kv_heads, int32_t topk_val,
    int32_t page_reserved_bos, int32_t page_reserved_eos, int32_t max_chunk_size,
    int32_t min_chunk_size, void* stream) {
  vtx::clear_error();
  (void)min_chunk_size;
  if (batch_size > 0 && (!dense_page_table || !sparse_page_table || !dense_cache_seqlens || !sparse_cache_seqlens))
    return vtx::fail(VTX_E_INVALID, "plan_decode_fa3: null page table or cache_seqlens");
  if (page_table_rows < 0 || page_table_stride < 0 || cache_seqlens_len < 0)
    return vtx::fail(VTX_E_INVALID, "plan_decode_fa3: negative page table or cache_seqlens size");
  PlanArgs a{};
  a.dpt = dense_page_table;
  a.spt = sparse_page_table;
  a.pt_rows = page_table_rows;
  a.pt_stride = page_table_stride;
  a.dcs = dense_cache_seqlens;
  a.scs = sparse_cache_seqlens;
  a.cs_len = cache_seqlens_len;
  return plan_launch(a, "plan_decode_fa3", cached_seq_lens, batch_size, dense_kv_indptr, dense_kv_indices,
                     dense_kv_indices_len, sparse_kv_indptr, sparse_kv_indices, sparse_kv_indices_len, nullptr,
                     false, req_to_token, req_to_token_rows, req_to_token_stride, req_indices, winfo_q_indices,
                     winfo_kv_offsets, winfo_kv_lens, winfo_capacity, winfo_num_workloads, winfo_chunk_size,
                     page_size, num_kv_heads, topk_val, page_reserved_bos, page_reserved_eos, max_chunk_size, stream);
}
