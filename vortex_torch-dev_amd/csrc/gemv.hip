// Paged GeMV scorer for gfx950: scores = q_mean . centroid[dense_idx[p]].
//
// Semantics follow the reference's mv_bpr
// (vortex_torch/indexer/triton_kernels/mv_impl.py:6-81): for every workload
// (segment q, offset, length) of the planner's list, o[p] = dot(x[q], y[dense[p]])
// for the covered positions only, bf16 inputs, fp32 accumulation, bf16 output.
//
// The work is HBM-bound (one centroid row, 2*D bytes, per score), so it runs
// on the VALU, not MFMA.  Design:
//   * one wave processes 64 consecutive positions of a workload per pass;
//   * a row of D bf16 is split over LPR lanes holding VPL 16-byte vectors each,
//     so one wave-wide load instruction covers 64/LPR whole rows, and every
//     lane issues all of its row loads for the pass before doing arithmetic;
//   * the 64 row indices are loaded with one coalesced load and broadcast
//     with lane shuffles;
//   * partial dot products are combined with a recursive-halving
//     reduce-scatter inside each LPR-lane group, so that afterwards every lane
//     owns exactly one finished score and the wave writes 64 scores at once;
//   * workloads are dealt to waves round-robin over a fixed grid (the
//     workload count lives on the device, so the launch is capture-safe).
#include "vtx_device.h"
#include "vtx_host.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / vtx::kWave;
constexpr int kPass = 64;  // positions per wave pass

struct GemvArgs {
  const uint16_t* x;
  int64_t x_rows;
  const uint16_t* y;
  int64_t y_rows;
  uint16_t* o;
  int64_t o_len;
  const int32_t* dense;
  int64_t dense_len;
  const int32_t* wq;
  const int32_t* woff;
  const int32_t* wlen;
  int64_t wcap;
  const int32_t* wnum;
  int32_t dim;
  int32_t passes_per_workload;
};

__device__ __forceinline__ long long workload_count(const GemvArgs& a) {
  long long nw = *a.wnum;
  if (nw > a.wcap) nw = a.wcap;
  if (nw < 0) nw = 0;
  return nw;
}

// LPR lanes per row, VPL 16-byte vectors per lane: dim == LPR * VPL * 8.
template <int LPR, int VPL>
__global__ __launch_bounds__(kThreads, (VPL == 1 ? 4 : 2)) void gemv_paged_kernel(GemvArgs a) {
  constexpr int kRowsPerLoad = vtx::kWave / LPR;
  constexpr int kSlots = LPR;  // rows per lane per pass = kPass / kRowsPerLoad
  constexpr int kBatch = VPL <= 2 ? kSlots : (VPL <= 4 ? 4 : 2);
  static_assert(kSlots * kRowsPerLoad == kPass, "pass geometry");

  const int lane = vtx::lane_id();
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int wave = vtx::uniform(threadIdx.x / vtx::kWave);
  const long long stride = (long long)gridDim.x * kWavesPerBlock;
  const long long unit_cap = a.wcap * a.passes_per_workload;
  long long u = (long long)blockIdx.x * kWavesPerBlock + wave;

  // The first unit's descriptor is fetched together with the workload count
  // (it only needs to be in bounds, not valid), which takes one dependent
  // memory round trip off the start of every wave.
  int nq = 0, noff = 0, nlen = 0;
  if (u < unit_cap) {
    const long long w = u / a.passes_per_workload;
    nq = a.wq[w];
    noff = a.woff[w];
    nlen = a.wlen[w];
  }
  const long long units = workload_count(a) * a.passes_per_workload;

  int cur_q = -1;
  float xs[VPL][8];
#pragma unroll
  for (int v = 0; v < VPL; ++v)
#pragma unroll
    for (int e = 0; e < 8; ++e) xs[v][e] = 0.f;

  for (; u < units; u += stride) {
    const long long w = u / a.passes_per_workload;
    const int first_pass = (int)(u - w * a.passes_per_workload);
    const int q = nq;
    const int off = noff;
    const int len = nlen;
    if (u + stride < units) {
      const long long wn = (u + stride) / a.passes_per_workload;
      nq = a.wq[wn];
      noff = a.woff[wn];
      nlen = a.wlen[wn];
    }

    if (q != cur_q) {
      const bool ok = (q >= 0) && (q < a.x_rows);
      const uint16_t* xr = a.x + (long long)(ok ? q : 0) * a.dim;
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        vtx::U4 t = ok ? vtx::ld16(xr + (v * LPR + col) * 8) : vtx::U4{0u, 0u, 0u, 0u};
        xs[v][0] = vtx::bf16_lo(t.x);
        xs[v][1] = vtx::bf16_hi(t.x);
        xs[v][2] = vtx::bf16_lo(t.y);
        xs[v][3] = vtx::bf16_hi(t.y);
        xs[v][4] = vtx::bf16_lo(t.z);
        xs[v][5] = vtx::bf16_hi(t.z);
        xs[v][6] = vtx::bf16_lo(t.w);
        xs[v][7] = vtx::bf16_hi(t.w);
      }
      cur_q = q;
    }

    for (int pass = first_pass; (long long)pass * kPass < len; pass += a.passes_per_workload) {
      const long long p0 = (long long)off + (long long)pass * kPass;
      const int cnt = min(kPass, len - pass * kPass);

      int my_row = -1;
      if (lane < cnt) {
        const long long p = p0 + lane;
        if (p >= 0 && p < a.dense_len) {
          const int r = a.dense[p];
          if (r >= 0 && r < a.y_rows) my_row = r;
        }
      }
      // Lanes whose slot is empty or invalid re-read the first valid row of
      // the pass (same cache lines, no extra HBM traffic) and drop the result.
      int fallback = __builtin_amdgcn_readlane(my_row, 0);
      if (fallback < 0) fallback = 0;

      // Rows are loaded in batches of kBatch slots (all of them when a row is
      // one or two vectors per lane) so wide heads do not run out of registers.
      float acc[kSlots];
#pragma unroll
      for (int i0 = 0; i0 < kSlots; i0 += kBatch) {
        vtx::U4 buf[kBatch][VPL];
        bool live[kBatch];
#pragma unroll
        for (int ii = 0; ii < kBatch; ++ii) {
          const int r = __shfl(my_row, (i0 + ii) * kRowsPerLoad + grp, vtx::kWave);
          live[ii] = r >= 0;
          const uint16_t* yr = a.y + (long long)(live[ii] ? r : fallback) * a.dim;
#pragma unroll
          for (int v = 0; v < VPL; ++v) buf[ii][v] = vtx::ld16_stream(yr + (v * LPR + col) * 8);
        }
#pragma unroll
        for (int ii = 0; ii < kBatch; ++ii) {
          const float s = vtx::dot_row<VPL>(buf[ii], xs);
          acc[i0 + ii] = live[ii] ? s : 0.f;
        }
      }

      // Reduce-scatter over the LPR lanes of the group: after step `half`
      // each lane keeps the half of its slots selected by bit `half` of col.
#pragma unroll
      for (int half = kSlots / 2; half >= 1; half >>= 1) {
        const bool upper = (col & half) != 0;
#pragma unroll
        for (int t = 0; t < half; ++t) {
          const float send = upper ? acc[t] : acc[t + half];
          const float keep = upper ? acc[t + half] : acc[t];
          acc[t] = keep + vtx::xshfl(send, half);
        }
      }
      // This lane now owns slot `col`, i.e. row col * kRowsPerLoad + grp.
      const int r = col * kRowsPerLoad + grp;
      if (r < cnt) {
        const long long p = p0 + r;
        if (p >= 0 && p < a.o_len) a.o[p] = (uint16_t)vtx::f32_to_bf16(acc[0]);
      }
    }
  }
}

// Any head_dim (or unaligned rows): one wave per position, lanes stride over D.
__global__ __launch_bounds__(kThreads) void gemv_paged_generic_kernel(GemvArgs a) {
  const int lane = vtx::lane_id();
  const int wave = vtx::uniform(threadIdx.x / vtx::kWave);
  const long long units = workload_count(a) * a.passes_per_workload;
  const long long stride = (long long)gridDim.x * kWavesPerBlock;
  for (long long u = (long long)blockIdx.x * kWavesPerBlock + wave; u < units; u += stride) {
    const long long w = u / a.passes_per_workload;
    const int first_pass = (int)(u - w * a.passes_per_workload);
    const int q = a.wq[w];
    const int off = a.woff[w];
    const int len = a.wlen[w];
    if (q < 0 || q >= a.x_rows) continue;
    const uint16_t* xr = a.x + (long long)q * a.dim;
    for (int pass = first_pass; (long long)pass * kPass < len; pass += a.passes_per_workload) {
      const int cnt = min(kPass, len - pass * kPass);
      for (int t = 0; t < cnt; ++t) {
        const long long p = (long long)off + (long long)pass * kPass + t;
        if (p < 0 || p >= a.dense_len || p >= a.o_len) continue;
        const int r = a.dense[p];
        if (r < 0 || r >= a.y_rows) continue;
        const uint16_t* yr = a.y + (long long)r * a.dim;
        float s = 0.f;
        for (int d = lane; d < a.dim; d += vtx::kWave)
          s = fmaf(vtx::bf16_to_f32(xr[d]), vtx::bf16_to_f32(yr[d]), s);
        s = vtx::wave_sum(s);
        if (lane == 0) a.o[p] = (uint16_t)vtx::f32_to_bf16(s);
      }
    }
  }
}

template <int LPR, int VPL>
void launch(const GemvArgs& a, int blocks, hipStream_t s) {
  gemv_paged_kernel<LPR, VPL><<<blocks, kThreads, 0, s>>>(a);
}

}  // namespace

extern "C" int vtx_gemv_paged(const uint16_t* x, int64_t x_rows, const uint16_t* y,
                              int64_t y_rows, uint16_t* o, int64_t o_len,
                              const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                              const int32_t* winfo_q_indices, const int32_t* winfo_kv_offsets,
                              const int32_t* winfo_kv_lens, int64_t winfo_capacity,
                              const int32_t* winfo_num_workloads, int32_t head_dim,
                              int32_t max_chunk_size, void* stream) {
  vtx::clear_error();
  if (head_dim < 1) return vtx::fail(VTX_E_INVALID, "gemv_paged: head_dim must be >= 1");
  if (max_chunk_size < 1) return vtx::fail(VTX_E_INVALID, "gemv_paged: max_chunk_size must be >= 1");
  if (!winfo_num_workloads) return vtx::fail(VTX_E_INVALID, "gemv_paged: null winfo_num_workloads");
  if (winfo_capacity <= 0 || o_len <= 0 || y_rows <= 0 || x_rows <= 0) return VTX_OK;  // nothing to do
  if (!x || !y || !o || !dense_kv_indices || !winfo_q_indices || !winfo_kv_offsets || !winfo_kv_lens)
    return vtx::fail(VTX_E_INVALID, "gemv_paged: null pointer");

  GemvArgs a;
  a.x = x;
  a.x_rows = x_rows;
  a.y = y;
  a.y_rows = y_rows;
  a.o = o;
  a.o_len = o_len;
  a.dense = dense_kv_indices;
  a.dense_len = dense_kv_indices_len;
  a.wq = winfo_q_indices;
  a.woff = winfo_kv_offsets;
  a.wlen = winfo_kv_lens;
  a.wcap = winfo_capacity;
  a.wnum = winfo_num_workloads;
  a.dim = head_dim;
  a.passes_per_workload = (max_chunk_size + kPass - 1) / kPass;

  const int cus = vtx::device_cu_count();
  if (cus <= 0) return vtx::fail(VTX_E_DEVICE, "gemv_paged: cannot query compute units");
  const long long max_units = winfo_capacity * (long long)a.passes_per_workload;
  long long blocks = (max_units + kWavesPerBlock - 1) / kWavesPerBlock;
  const long long cap = (long long)cus * 8;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;

  hipStream_t s = vtx::as_stream(stream);
  const bool vec_ok = (head_dim % 8 == 0) && vtx::aligned16(x) && vtx::aligned16(y);
  if (vec_ok && head_dim == 64) {
    launch<8, 1>(a, (int)blocks, s);
  } else if (vec_ok && head_dim == 128) {
    launch<16, 1>(a, (int)blocks, s);
  } else if (vec_ok && head_dim == 256) {
    launch<16, 2>(a, (int)blocks, s);
  } else if (vec_ok && head_dim == 512) {
    launch<16, 4>(a, (int)blocks, s);
  } else if (vec_ok && head_dim == 576) {
    launch<8, 9>(a, (int)blocks, s);
  } else {
    gemv_paged_generic_kernel<<<(int)blocks, kThreads, 0, s>>>(a);
  }
  return vtx::check_launch("gemv_paged");
}
