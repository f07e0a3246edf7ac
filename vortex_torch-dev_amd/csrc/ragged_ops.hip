// The indexer's workload-walking ops for gfx950: GeMM, elementwise binary
// and unary ops, reductions over one tile axis, and the in-place segment
// softmax / normalize that the GQA and Quest flows are built from.
//
// Every op except the segment ops visits exactly the packed positions of the
// decode planner's workload list: workload w covers winfo_kv_lens[w]
// positions from winfo_kv_offsets[w], all of segment winfo_q_indices[w].  An
// operand's row at position p of workload w is
//   VTX_ROWS_BATCHED: winfo_q_indices[w]   (the segment's query rows)
//   VTX_ROWS_PAGED:   dense_kv_indices[p]  (a page of a cache pool)
//   VTX_ROWS_RAGGED:  p                    (a per-position buffer)
// and the output row is p.  Positions outside the workloads are not written;
// a row outside its operand is skipped (its output is not written).
//
// Work distribution: one wave per workload, dealt round robin over a grid of
// at most 8 workgroups per CU; the workload count is read on the device, so
// every launch can be recorded into a graph.  None of these ops is
// GEMM-shaped at decode sizes (a [G, K] x [K] product per page), so they run
// on the VALU and are bound by HBM and latency.
#include "vtx_device.h"
#include "vtx_host.h"
#include "vtx_score.h"
#include "vtx_segment.h"

#include <cstring>

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / vtx::kWave;

struct Walk {
  const int32_t* wq;
  const int32_t* woff;
  const int32_t* wlen;
  int64_t wcap;
  const int32_t* wnum;
  const int32_t* dense;
  int64_t dense_len;
  int64_t out_rows;
};

struct Opnd {
  const uint16_t* p;
  int64_t rows;
  int32_t d0, d1, mode;
};

__device__ __forceinline__ int workload_count(const Walk& w) {
  const int n = *w.wnum;
  if (n < 0) return 0;
  return (long long)n > w.wcap ? (int)w.wcap : n;
}

// Positions of workload i clipped to the output rows; false when empty.
__device__ __forceinline__ bool workload(const Walk& w, int i, int* q, long long* off, int* len) {
  const long long o = w.woff[i];
  long long l = w.wlen[i];
  if (o < 0 || l <= 0 || o >= w.out_rows) return false;
  if (o + l > w.out_rows) l = w.out_rows - o;
  *q = w.wq ? w.wq[i] : 0;  // only BATCHED operands read it; they require the list
  *off = o;
  *len = (int)l;
  return true;
}

// Row of operand x at position p (of a workload of segment q), or -1.
__device__ __forceinline__ long long opnd_row(const Opnd& x, const Walk& w, int q, long long p) {
  long long r;
  if (x.mode == VTX_ROWS_BATCHED) {
    r = q;
  } else if (x.mode == VTX_ROWS_PAGED) {
    r = (p >= 0 && p < w.dense_len) ? (long long)w.dense[p] : -1;
  } else {
    r = p;
  }
  return (r >= 0 && r < x.rows) ? r : -1;
}

using vtx::bf16r;

// ------------------------------------------------------------------ GeMM
// o[p, c, g] = bf16(fp32 sum_k x[rx, g, k] * y[ry, c, k]); o is
// [out_rows, C = y.d0, G = x.d0], K = x.d1 = y.d1 (a multiple of 8).
// LPR lanes share a position (each one K/8/LPR 16-byte vectors: one chain
// of two-product steps, vtx::dot2_bf16, in increasing k), the LPR partial
// sums are combined by an xor tree; kG query rows are scored per pass over
// y's row.
struct GemmArgs {
  Walk w;
  Opnd x, y;
  uint16_t* o;
};

template <int LPR, int kG>
__global__ __launch_bounds__(kThreads) void gemm_ragged_kernel(GemmArgs a) {
  constexpr int kPos = vtx::kWave / LPR;
  const int lane = vtx::lane_id();
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int wid = blockIdx.x * kWavesPerBlock + threadIdx.x / vtx::kWave;
  const int waves = gridDim.x * kWavesPerBlock;
  const int C = a.y.d0, G = a.x.d0, K = a.x.d1;
  const int units = K / 8;
  const int nw = workload_count(a.w);
  for (int i = wid; i < nw; i += waves) {
    int q, len;
    long long off;
    if (!workload(a.w, i, &q, &off, &len)) continue;
    for (int t0 = 0; t0 < len; t0 += kPos) {
      const int t = t0 + grp;
      const long long p = off + t;
      const long long ry = t < len ? opnd_row(a.y, a.w, q, p) : -1;
      const long long rx = t < len ? opnd_row(a.x, a.w, q, p) : -1;
      const bool ok = ry >= 0 && rx >= 0;
      for (int c = 0; c < C; ++c) {
        const uint16_t* yr = a.y.p + ((ok ? ry : 0) * C + c) * (long long)K;
        for (int g0 = 0; g0 < G; g0 += kG) {
          float acc[kG];
#pragma unroll
          for (int gg = 0; gg < kG; ++gg) acc[gg] = 0.f;
          for (int v = col; v < units; v += LPR) {
            const vtx::U4 yv = vtx::ld16(yr + v * 8);
#pragma unroll
            for (int gg = 0; gg < kG; ++gg) {
              if (g0 + gg < G) {
                const vtx::U4 xv = vtx::ld16(a.x.p + ((ok ? rx : 0) * G + g0 + gg) * (long long)K + v * 8);
                // the four two-product steps of vtx::dot_row, in its order
                acc[gg] = vtx::dot2_bf16(yv.x, xv.x, acc[gg]);
                acc[gg] = vtx::dot2_bf16(yv.y, xv.y, acc[gg]);
                acc[gg] = vtx::dot2_bf16(yv.z, xv.z, acc[gg]);
                acc[gg] = vtx::dot2_bf16(yv.w, xv.w, acc[gg]);
              }
            }
          }
#pragma unroll
          for (int gg = 0; gg < kG; ++gg)
#pragma unroll
            for (int d = LPR / 2; d >= 1; d >>= 1) acc[gg] += __shfl_xor(acc[gg], d, vtx::kWave);
          if (col == 0 && ok) {
#pragma unroll
            for (int gg = 0; gg < kG; ++gg)
              if (g0 + gg < G) a.o[(p * C + c) * G + g0 + gg] = (uint16_t)vtx::f32_to_bf16(acc[gg]);
          }
        }
      }
    }
  }
}

// Fast path for one y row per position (C == 1) and BATCHED x, the GeMM of
// the GQA flow: a wave takes up to kPass positions of a workload at once,
// issues every y row load before any arithmetic and scores kG query rows of
// the segment per load (vtx::score_pass_multi); K = LPR * VPL * 8.
template <int LPR, int VPL, int kG>
__global__ __launch_bounds__(kThreads) void gemm_rows_kernel(GemmArgs a) {
  constexpr int kPass = vtx::segment_pass<VPL>();
  const int lane = vtx::lane_id();
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int wid = blockIdx.x * kWavesPerBlock + threadIdx.x / vtx::kWave;
  const int waves = gridDim.x * kWavesPerBlock;
  const int G = a.x.d0, K = a.x.d1;
  const int nw = workload_count(a.w);
  for (int i = wid; i < nw; i += waves) {
    int q, len;
    long long off;
    if (!workload(a.w, i, &q, &off, &len)) continue;
    const long long rx = opnd_row(a.x, a.w, q, off);
    if (rx < 0) continue;
    for (int p0 = 0; p0 < len; p0 += kPass) {
      const int cnt = min(kPass, len - p0);
      int my_row = -1;
      if (lane < cnt) {
        const long long r = opnd_row(a.y, a.w, q, off + p0 + lane);
        my_row = r >= 0 ? (int)r : -1;
      }
      for (int g0 = 0; g0 < G; g0 += kG) {
        float xs[kG][VPL][8];
#pragma unroll
        for (int gg = 0; gg < kG; ++gg)
#pragma unroll
          for (int v = 0; v < VPL; ++v) {
            if (g0 + gg < G) {
              vtx::unpack8(vtx::ld16(a.x.p + (rx * G + g0 + gg) * (long long)K + (v * LPR + col) * 8), xs[gg][v]);
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e) xs[gg][v][e] = 0.f;
            }
          }
        int r;
        float sc[kG];
        vtx::score_pass_multi<LPR, VPL, kPass, kG>(a.y.p, a.y.rows, K, my_row, cnt, xs, grp, col, &r, sc);
        const int rrow = __shfl(my_row, r < 0 ? 0 : r, vtx::kWave);  // row of the lane's position
        if (r >= 0 && rrow >= 0) {
          const long long p = off + p0 + r;
#pragma unroll
          for (int gg = 0; gg < kG; ++gg)
            if (g0 + gg < G) a.o[p * G + g0 + gg] = (uint16_t)vtx::f32_to_bf16(sc[gg]);
        }
      }
    }
  }
}

// ------------------------------------------------- elementwise binary / unary
// Binary: o[p, i, j] = op(x[rx, i', j'], y[ry, i'', j'']) where an operand
// axis of size 1 broadcasts.  bf16 in and out; max / min compare the values,
// mul rounds the exact product, add rounds alpha*x and beta*y (alpha, beta
// first rounded to bf16) and then their sum, as bf16 arithmetic does.
// Unary (x RAGGED, o same tile shape), with a = bf16(alpha), b = bf16(beta)
// and z = bf16(bf16(b*x) + a):
//   RELU     x >= a ? x : b        SIGMOID  1 / (1 + exp(z))
//   SILU     x / (1 + exp(z))      ABS      |z|
//   ADD_MUL  z
// (the sigmoid and SiLU forms, including the sign, are the reference's).
struct EwArgs {
  Walk w;
  Opnd x, y;  // y unused by unary ops
  uint16_t* o;
  int32_t o_d0, o_d1;
  int32_t op;
  float alpha, beta;  // already bf16-rounded
};

__device__ __forceinline__ float binary_op(int op, float xv, float yv, float alpha, float beta) {
  switch (op) {
    case VTX_BINARY_MAXIMUM: return fmaxf(xv, yv);
    case VTX_BINARY_MINIMUM: return fminf(xv, yv);
    case VTX_BINARY_ADD: return bf16r(alpha * xv) + bf16r(beta * yv);
    default: return xv * yv;
  }
}

__device__ __forceinline__ float unary_op(int op, float xv, float alpha, float beta) {
  if (op == VTX_UNARY_RELU) return xv >= alpha ? xv : beta;
  const float z = bf16r(bf16r(beta * xv) + alpha);
  switch (op) {
    case VTX_UNARY_SIGMOID: return 1.0f / (1.0f + expf(z));
    case VTX_UNARY_SILU: return xv / (1.0f + expf(z));
    case VTX_UNARY_ABS: return fabsf(z);
    default: return z;  // VTX_UNARY_ADD_MUL
  }
}

// One workgroup per workload; kVec: 8 consecutive j per lane (o_d1 % 8 == 0
// and no operand broadcasts along j), otherwise one element per lane.  Each
// thread takes kU items per round and issues all their loads before any
// arithmetic.
template <bool kBinary, bool kVec>
__global__ __launch_bounds__(kThreads) void elementwise_ragged_kernel(EwArgs a) {
  constexpr int kW = kVec ? 8 : 1;
  constexpr int kU = 4;
  const int tid = threadIdx.x;
  const int nj = a.o_d1 / kW;
  const int per_pos = a.o_d0 * nj;
  const int nw = workload_count(a.w);
  for (int i = blockIdx.x; i < nw; i += gridDim.x) {
    int q, len;
    long long off;
    if (!workload(a.w, i, &q, &off, &len)) continue;
    const long long items = (long long)len * per_pos;
    for (long long base = 0; base < items; base += (long long)kThreads * kU) {
      vtx::U4 xv[kU], yv[kU];
      long long oi[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const long long it = base + (long long)u * kThreads + tid;
        oi[u] = -1;
        if (it >= items) continue;
        const int t = (int)(it / per_pos);
        const int e = (int)(it - (long long)t * per_pos);
        const int i0 = e / nj;
        const int j0 = (e - i0 * nj) * kW;
        const long long p = off + t;
        const long long rx = opnd_row(a.x, a.w, q, p);
        const long long ry = kBinary ? opnd_row(a.y, a.w, q, p) : 0;
        if (rx < 0 || ry < 0) continue;
        const long long xo = (rx * a.x.d0 + (a.x.d0 == 1 ? 0 : i0)) * a.x.d1;
        const long long yo = kBinary ? (ry * a.y.d0 + (a.y.d0 == 1 ? 0 : i0)) * a.y.d1 : 0;
        oi[u] = (p * a.o_d0 + i0) * a.o_d1 + j0;
        if (kVec) {
          xv[u] = vtx::ld16(a.x.p + xo + j0);
          if (kBinary) yv[u] = vtx::ld16(a.y.p + yo + j0);
        } else {
          xv[u].x = a.x.p[xo + (a.x.d1 == 1 ? 0 : j0)];
          if (kBinary) yv[u].x = a.y.p[yo + (a.y.d1 == 1 ? 0 : j0)];
        }
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        if (oi[u] < 0) continue;
        if (kVec) {
          float xf[8], yf[8];
          vtx::unpack8(xv[u], xf);
          if (kBinary) vtx::unpack8(yv[u], yf);
          uint32_t r[8];
#pragma unroll
          for (int k = 0; k < 8; ++k)
            r[k] = vtx::f32_to_bf16(kBinary ? binary_op(a.op, xf[k], yf[k], a.alpha, a.beta)
                                            : unary_op(a.op, xf[k], a.alpha, a.beta));
          vtx::st16(a.o + oi[u],
                    vtx::U4{r[0] | (r[1] << 16), r[2] | (r[3] << 16), r[4] | (r[5] << 16), r[6] | (r[7] << 16)});
        } else {
          const float xf = vtx::bf16_to_f32(xv[u].x);
          const float res = kBinary ? binary_op(a.op, xf, vtx::bf16_to_f32(yv[u].x), a.alpha, a.beta)
                                    : unary_op(a.op, xf, a.alpha, a.beta);
          a.o[oi[u]] = (uint16_t)vtx::f32_to_bf16(res);
        }
      }
    }
  }
}

// -------------------------------------------------------------- reductions
// o[p] = reduce of the tile x[p] ([D0, D1]) over axis `dim` (1: D0 -> o is
// [*, 1, D1]; 2: D1 -> o is [*, D0, 1]), in fp32, rounded to bf16:
// mean = sum / count, max, min, L2 = sqrt(sum of squares), sum.  One lane
// per output element; along a contiguous axis that is a multiple of 8 the
// lane reads 16-byte vectors.
struct ReduceArgs {
  Walk w;
  Opnd x;
  uint16_t* o;
  int32_t dim, type;
};

struct RAcc {
  float s, m, n;
};
__device__ __forceinline__ void racc_add(RAcc& r, float v, int type) {
  if (type == VTX_REDUCE_MAX) r.m = fmaxf(r.m, v);
  else if (type == VTX_REDUCE_MIN) r.m = fminf(r.m, v);
  else if (type == VTX_REDUCE_L2NORM) r.s = fmaf(v, v, r.s);
  else r.s += v;
}
__device__ __forceinline__ float racc_out(const RAcc& r, int type, int count) {
  switch (type) {
    case VTX_REDUCE_MEAN: return r.s / (float)count;
    case VTX_REDUCE_MAX:
    case VTX_REDUCE_MIN: return r.m;
    case VTX_REDUCE_L2NORM: return sqrtf(r.s);
    default: return r.s;
  }
}

__device__ __forceinline__ float racc_merge(float a, float b, int type) {
  if (type == VTX_REDUCE_MAX) return fmaxf(a, b);
  if (type == VTX_REDUCE_MIN) return fminf(a, b);
  return a + b;
}

// One workgroup per workload.  Along a contiguous axis that is a multiple of
// 8 wide, L lanes (a power of two <= 16 dividing the axis' 16-byte vectors)
// share an output: each reads every L-th vector, kU loads issued together,
// and the L partials are merged by an xor tree.  Otherwise a lane computes
// one output, reading kU elements per round.
__global__ __launch_bounds__(kThreads) void reduce_ragged_kernel(ReduceArgs a) {
  constexpr int kU = 4;
  const int tid = threadIdx.x;
  const int D0 = a.x.d0, D1 = a.x.d1;
  const int per_pos = a.dim == 1 ? D1 : D0;
  const int count = a.dim == 1 ? D0 : D1;
  const bool vec = a.dim == 2 && (D1 % 8) == 0;
  const int nvec = D1 / 8;
  int L = 1;
  if (vec)
    while (L < 16 && nvec % (2 * L) == 0) L *= 2;
  const float init = a.type == VTX_REDUCE_MAX ? -INFINITY : (a.type == VTX_REDUCE_MIN ? INFINITY : 0.f);
  const int nw = workload_count(a.w);
  for (int i = blockIdx.x; i < nw; i += gridDim.x) {
    int q, len;
    long long off;
    if (!workload(a.w, i, &q, &off, &len)) continue;
    const long long outputs = (long long)len * per_pos;
    const long long tasks = outputs * L;  // L lanes per output (aligned groups within a wave)
    for (long long base = 0; base < tasks; base += kThreads) {
      const long long it = base + tid;
      const long long oidx = it / L;
      const int sub = (int)(it - oidx * L);
      const bool in = it < tasks;
      long long t = in ? oidx / per_pos : 0;
      const int e = in ? (int)(oidx - t * per_pos) : 0;
      const long long p = off + t;
      const long long rx = in ? opnd_row(a.x, a.w, q, p) : -1;
      RAcc r{0.f, init, 0.f};
      if (rx >= 0) {
        const uint16_t* tile = a.x.p + rx * (long long)D0 * D1;
        if (vec) {
          const uint16_t* row = tile + (long long)e * D1;
          for (int v0 = sub; v0 < nvec; v0 += L * kU) {
            vtx::U4 buf[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) {
              const int v = v0 + u * L;
              buf[u] = v < nvec ? vtx::ld16(row + v * 8) : vtx::U4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < kU; ++u) {
              if (v0 + u * L >= nvec) break;
              float f[8];
              vtx::unpack8(buf[u], f);
#pragma unroll
              for (int k = 0; k < 8; ++k) racc_add(r, f[k], a.type);
            }
          }
        } else {
          const long long stride = a.dim == 1 ? D1 : 1;
          const uint16_t* base_p = a.dim == 1 ? tile + e : tile + (long long)e * D1;
          for (int d0 = 0; d0 < count; d0 += kU) {
            float v[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) v[u] = d0 + u < count ? vtx::bf16_to_f32(base_p[(d0 + u) * stride]) : 0.f;
#pragma unroll
            for (int u = 0; u < kU; ++u)
              if (d0 + u < count) racc_add(r, v[u], a.type);
          }
        }
      }
      float val = (a.type == VTX_REDUCE_MAX || a.type == VTX_REDUCE_MIN) ? r.m : r.s;
      for (int d = L / 2; d >= 1; d >>= 1) val = racc_merge(val, __shfl_xor(val, d, vtx::kWave), a.type);
      if (rx >= 0 && sub == 0) {
        RAcc fin{val, val, 0.f};
        a.o[p * per_pos + e] = (uint16_t)vtx::f32_to_bf16(racc_out(fin, a.type, count));
      }
    }
  }
}

// ------------------------------------------------------ segment softmax / L2
// In place over the middle pages of each segment s < segments with more
// than topk of them (n = indptr[s+1] - indptr[s] > bos + eos + topk), for
// every column c of the [cols] tile of each page:
//   SOFTMAX:    x = bf16(exp(v - M) / S), v = fp32(x) * scale, M = max v,
//               S = sum exp(v - M)
//   NORMALIZE:  x = bf16(fp32(x) / max(sqrt(sum fp32(x)^2), 1e-12))
// One workgroup per segment.  With cols <= kThreads each thread keeps a
// running (max, sum) of one column over every (kThreads / cols)-th page,
// the partials are merged in LDS, then the pages are rewritten; wider tiles
// give each thread whole columns.
struct SegArgs {
  uint16_t* x;
  int64_t rows;
  int32_t cols;
  const int32_t* indptr;
  int32_t segments;
  float scale;
  int32_t bos, eos, topk;
  int32_t op;
};

static_assert(kThreads == vtx::kScanThreads, "the segment scan runs the shared column statistics");
__global__ __launch_bounds__(kThreads) void segment_scan_kernel(SegArgs a) {
  __shared__ float pm[kThreads];
  __shared__ float ps[kThreads];
  const int seg = blockIdx.x;
  const int tid = threadIdx.x;
  const long long start = a.indptr[seg];
  const long long n = (long long)a.indptr[seg + 1] - start;
  if (n <= (long long)a.bos + a.eos + a.topk) return;
  const long long cnt = n - a.bos - a.eos;
  const long long base = start + a.bos;
  if (cnt <= 0 || base < 0 || base + cnt > a.rows) return;
  const int cols = a.cols;
  uint16_t* x = a.x + base * cols;
  const bool softmax = a.op == VTX_SEGMENT_SOFTMAX;
  const float kLow = -1e30f;  // start of the running maximum

  if (cols <= kThreads) {
    const int per_col = kThreads / cols;  // threads per column
    const int c = tid % cols;
    const int r0 = tid / cols;
    const bool active = r0 < per_col;
    float vals[vtx::kScanRegs];
    bool in_regs;
    vtx::column_scan_stats([&](long long r, int col) { return vtx::bf16_to_f32(x[r * cols + col]); }, cnt, cols,
                           a.scale, softmax, pm, ps, vals, in_regs);
    if (!active) return;
    const float M = pm[c], S = ps[c];
    const float norm = fmaxf(sqrtf(S), 1e-12f);
    if (in_regs) {
#pragma unroll
      for (int k = 0; k < vtx::kScanRegs; ++k) {
        const long long r = r0 + (long long)k * per_col;
        if (r < cnt) {
          const float o = softmax ? vtx::softmax_value(vals[k], a.scale, M, S) : vals[k] / norm;
          x[r * cols + c] = (uint16_t)vtx::f32_to_bf16(o);
        }
      }
    } else {
      for (long long r = r0; r < cnt; r += per_col) {
        const float v = vtx::bf16_to_f32(x[r * cols + c]);
        const float o = softmax ? vtx::softmax_value(v, a.scale, M, S) : v / norm;
        x[r * cols + c] = (uint16_t)vtx::f32_to_bf16(o);
      }
    }
  } else {
    for (int c = tid; c < cols; c += kThreads) {
      float M = kLow, S = 0.f;
      for (long long r = 0; r < cnt; ++r) {
        const float v = vtx::bf16_to_f32(x[r * cols + c]);
        if (softmax) {
          const float u = v * a.scale;
          if (u > M) {
            S = S * __expf(M - u) + 1.f;
            M = u;
          } else {
            S += __expf(u - M);
          }
        } else {
          S = fmaf(v, v, S);
        }
      }
      const float norm = fmaxf(sqrtf(S), 1e-12f);
      for (long long r = 0; r < cnt; ++r) {
        const float v = vtx::bf16_to_f32(x[r * cols + c]);
        const float o = softmax ? __expf(v * a.scale - M) / S : v / norm;
        x[r * cols + c] = (uint16_t)vtx::f32_to_bf16(o);
      }
    }
  }
}

// ------------------------------------------------------------------- host
int check_walk(const char* what, const int32_t* woff, const int32_t* wlen, int64_t wcap, const int32_t* wnum,
               const int32_t* wq, bool need_q) {
  if (!wnum) return vtx::fail(VTX_E_INVALID, "%s: null winfo_num_workloads", what);
  if (wcap < 0) return vtx::fail(VTX_E_INVALID, "%s: negative workload capacity", what);
  if (wcap > 0 && (!woff || !wlen || (need_q && !wq)))
    return vtx::fail(VTX_E_INVALID, "%s: null workload list", what);
  return VTX_OK;
}

int check_opnd(const char* what, const char* name, const Opnd& x, bool paged_ok, bool batched_ok) {
  if (!x.p) return vtx::fail(VTX_E_INVALID, "%s: null %s", what, name);
  if (x.rows < 1 || x.d0 < 1 || x.d1 < 1) return vtx::fail(VTX_E_INVALID, "%s: empty %s", what, name);
  if (x.mode < VTX_ROWS_BATCHED || x.mode > VTX_ROWS_RAGGED ||
      (x.mode == VTX_ROWS_PAGED && !paged_ok) || (x.mode == VTX_ROWS_BATCHED && !batched_ok))
    return vtx::fail(VTX_E_INVALID, "%s: row mode %d not supported for %s", what, x.mode, name);
  return VTX_OK;
}

int grid_for(int64_t wcap) {
  const int cus = vtx::device_cu_count();
  long long g = (wcap + kWavesPerBlock - 1) / kWavesPerBlock;
  const long long cap = 8LL * (cus > 0 ? cus : 256);
  if (g > cap) g = cap;
  return (int)(g < 1 ? 1 : g);
}

// One workgroup per workload, at most 16 per CU (the rest loop).
int grid_blocks(int64_t wcap) {
  const int cus = vtx::device_cu_count();
  long long g = wcap;
  const long long cap = 16LL * (cus > 0 ? cus : 256);
  if (g > cap) g = cap;
  return (int)(g < 1 ? 1 : g);
}

Walk make_walk(const int32_t* dense, int64_t dense_len, const int32_t* wq, const int32_t* woff,
               const int32_t* wlen, int64_t wcap, const int32_t* wnum, int64_t out_rows) {
  Walk w;
  w.wq = wq;
  w.woff = woff;
  w.wlen = wlen;
  w.wcap = wcap;
  w.wnum = wnum;
  w.dense = dense;
  w.dense_len = dense ? dense_len : 0;
  w.out_rows = out_rows;
  return w;
}

float to_bf16_value(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return f;
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

template <int LPR>
int launch_gemm(const GemmArgs& a, int grid, hipStream_t s) {
  if (a.x.d0 >= 8) {
    gemm_ragged_kernel<LPR, 8><<<grid, kThreads, 0, s>>>(a);
  } else if (a.x.d0 >= 4) {
    gemm_ragged_kernel<LPR, 4><<<grid, kThreads, 0, s>>>(a);
  } else if (a.x.d0 >= 2) {
    gemm_ragged_kernel<LPR, 2><<<grid, kThreads, 0, s>>>(a);
  } else {
    gemm_ragged_kernel<LPR, 1><<<grid, kThreads, 0, s>>>(a);
  }
  return vtx::check_launch("ragged_gemm");
}

}  // namespace

extern "C" int vtx_ragged_gemm(const uint16_t* x, int64_t x_rows, int32_t x_mode, int32_t x_d0,
                               const uint16_t* y, int64_t y_rows, int32_t y_mode, int32_t y_d0, int32_t k,
                               uint16_t* o, int64_t o_rows, const int32_t* dense_kv_indices,
                               int64_t dense_kv_indices_len, const int32_t* winfo_q_indices,
                               const int32_t* winfo_kv_offsets, const int32_t* winfo_kv_lens,
                               int64_t winfo_capacity, const int32_t* winfo_num_workloads, void* stream) {
  vtx::clear_error();
  const char* what = "ragged_gemm";
  const Opnd xo{x, x_rows, x_d0, k, x_mode};
  const Opnd yo{y, y_rows, y_d0, k, y_mode};
  int rc;
  if ((rc = check_walk(what, winfo_kv_offsets, winfo_kv_lens, winfo_capacity, winfo_num_workloads,
                       winfo_q_indices, x_mode == VTX_ROWS_BATCHED)))
    return rc;
  if ((rc = check_opnd(what, "x", xo, false, true)) || (rc = check_opnd(what, "y", yo, true, false))) return rc;
  if (k % 8 != 0) return vtx::fail(VTX_E_INVALID, "%s: K = %d must be a multiple of 8", what, k);
  if (!o || o_rows < 0) return vtx::fail(VTX_E_INVALID, "%s: null output", what);
  if (y_mode == VTX_ROWS_PAGED && !dense_kv_indices)
    return vtx::fail(VTX_E_INVALID, "%s: paged y needs dense_kv_indices", what);
  if (!vtx::aligned16(x) || !vtx::aligned16(y))
    return vtx::fail(VTX_E_INVALID, "%s: x and y must be 16-byte aligned", what);
  if (winfo_capacity == 0 || o_rows == 0) return VTX_OK;
  GemmArgs a;
  a.w = make_walk(dense_kv_indices, dense_kv_indices_len, winfo_q_indices, winfo_kv_offsets, winfo_kv_lens,
                  winfo_capacity, winfo_num_workloads, o_rows);
  a.x = xo;
  a.y = yo;
  a.o = o;
  const int units = k / 8;
  const int grid = grid_for(winfo_capacity);
  hipStream_t s = vtx::as_stream(stream);
  if (y_d0 == 1 && x_mode == VTX_ROWS_BATCHED) {
    const bool two = x_d0 >= 2;
    switch (k) {
      case 64:
        if (two) gemm_rows_kernel<8, 1, 2><<<grid, kThreads, 0, s>>>(a);
        else gemm_rows_kernel<8, 1, 1><<<grid, kThreads, 0, s>>>(a);
        return vtx::check_launch("ragged_gemm");
      case 128:
        if (two) gemm_rows_kernel<16, 1, 2><<<grid, kThreads, 0, s>>>(a);
        else gemm_rows_kernel<16, 1, 1><<<grid, kThreads, 0, s>>>(a);
        return vtx::check_launch("ragged_gemm");
      case 256: gemm_rows_kernel<16, 2, 1><<<grid, kThreads, 0, s>>>(a); return vtx::check_launch("ragged_gemm");
      case 512: gemm_rows_kernel<16, 4, 1><<<grid, kThreads, 0, s>>>(a); return vtx::check_launch("ragged_gemm");
      case 576: gemm_rows_kernel<8, 9, 1><<<grid, kThreads, 0, s>>>(a); return vtx::check_launch("ragged_gemm");
      default: break;
    }
  }
  if (units % 16 == 0) return launch_gemm<16>(a, grid, s);
  if (units % 8 == 0) return launch_gemm<8>(a, grid, s);
  if (units % 4 == 0) return launch_gemm<4>(a, grid, s);
  if (units % 2 == 0) return launch_gemm<2>(a, grid, s);
  return launch_gemm<1>(a, grid, s);
}

namespace {

int elementwise(bool binary, int32_t op, float alpha, float beta, const Opnd& xo, const Opnd& yo, uint16_t* o,
                int64_t o_rows, int32_t o_d0, int32_t o_d1, const int32_t* dense, int64_t dense_len,
                const int32_t* wq, const int32_t* woff, const int32_t* wlen, int64_t wcap, const int32_t* wnum,
                void* stream) {
  const char* what = binary ? "ragged_binary" : "ragged_unary";
  int rc;
  const bool need_q = xo.mode == VTX_ROWS_BATCHED || (binary && yo.mode == VTX_ROWS_BATCHED);
  if ((rc = check_walk(what, woff, wlen, wcap, wnum, wq, need_q))) return rc;
  if ((rc = check_opnd(what, "x", xo, false, binary))) return rc;
  if (binary && (rc = check_opnd(what, "y", yo, true, false))) return rc;
  if (!o || o_rows < 0 || o_d0 < 1 || o_d1 < 1) return vtx::fail(VTX_E_INVALID, "%s: bad output", what);
  if (binary ? (op < VTX_BINARY_MAXIMUM || op > VTX_BINARY_MUL) : (op < VTX_UNARY_RELU || op > VTX_UNARY_ADD_MUL))
    return vtx::fail(VTX_E_INVALID, "%s: unknown op %d", what, op);
  const Opnd* ops[2] = {&xo, &yo};
  for (int i = 0; i < (binary ? 2 : 1); ++i) {
    const Opnd& t = *ops[i];
    if ((t.d0 != o_d0 && t.d0 != 1) || (t.d1 != o_d1 && t.d1 != 1))
      return vtx::fail(VTX_E_INVALID, "%s: operand tile [%d, %d] does not broadcast to [%d, %d]", what, t.d0,
                       t.d1, o_d0, o_d1);
  }
  if (!binary && (xo.d0 != o_d0 || xo.d1 != o_d1))
    return vtx::fail(VTX_E_INVALID, "%s: output tile must equal the input tile", what);
  if (binary && yo.mode == VTX_ROWS_PAGED && !dense)
    return vtx::fail(VTX_E_INVALID, "%s: paged y needs dense_kv_indices", what);
  if (wcap == 0 || o_rows == 0) return VTX_OK;
  EwArgs a;
  a.w = make_walk(dense, dense_len, wq, woff, wlen, wcap, wnum, o_rows);
  a.x = xo;
  a.y = binary ? yo : xo;
  a.o = o;
  a.o_d0 = o_d0;
  a.o_d1 = o_d1;
  a.op = op;
  a.alpha = to_bf16_value(alpha);
  a.beta = to_bf16_value(beta);
  const bool vec = (o_d1 % 8) == 0 && xo.d1 == o_d1 && (!binary || yo.d1 == o_d1) && vtx::aligned16(xo.p) &&
                   (!binary || vtx::aligned16(yo.p)) && vtx::aligned16(o);
  const int grid = grid_blocks(wcap);
  hipStream_t s = vtx::as_stream(stream);
  if (binary) {
    if (vec) elementwise_ragged_kernel<true, true><<<grid, kThreads, 0, s>>>(a);
    else elementwise_ragged_kernel<true, false><<<grid, kThreads, 0, s>>>(a);
  } else {
    if (vec) elementwise_ragged_kernel<false, true><<<grid, kThreads, 0, s>>>(a);
    else elementwise_ragged_kernel<false, false><<<grid, kThreads, 0, s>>>(a);
  }
  return vtx::check_launch(what);
}

}  // namespace

extern "C" int vtx_ragged_binary(int32_t op, float alpha, float beta, const uint16_t* x, int64_t x_rows,
                                 int32_t x_mode, int32_t x_d0, int32_t x_d1, const uint16_t* y, int64_t y_rows,
                                 int32_t y_mode, int32_t y_d0, int32_t y_d1, uint16_t* o, int64_t o_rows,
                                 int32_t o_d0, int32_t o_d1, const int32_t* dense_kv_indices,
                                 int64_t dense_kv_indices_len, const int32_t* winfo_q_indices,
                                 const int32_t* winfo_kv_offsets, const int32_t* winfo_kv_lens,
                                 int64_t winfo_capacity, const int32_t* winfo_num_workloads, void* stream) {
  vtx::clear_error();
  return elementwise(true, op, alpha, beta, Opnd{x, x_rows, x_d0, x_d1, x_mode}, Opnd{y, y_rows, y_d0, y_d1, y_mode},
                     o, o_rows, o_d0, o_d1, dense_kv_indices, dense_kv_indices_len, winfo_q_indices,
                     winfo_kv_offsets, winfo_kv_lens, winfo_capacity, winfo_num_workloads, stream);
}

extern "C" int vtx_ragged_unary(int32_t op, float alpha, float beta, const uint16_t* x, int64_t x_rows,
                                int32_t d0, int32_t d1, uint16_t* o, int64_t o_rows,
                                const int32_t* winfo_kv_offsets, const int32_t* winfo_kv_lens,
                                int64_t winfo_capacity, const int32_t* winfo_num_workloads, void* stream) {
  vtx::clear_error();
  const Opnd xo{x, x_rows, d0, d1, VTX_ROWS_RAGGED};
  return elementwise(false, op, alpha, beta, xo, xo, o, o_rows, d0, d1, nullptr, 0, nullptr, winfo_kv_offsets,
                     winfo_kv_lens, winfo_capacity, winfo_num_workloads, stream);
}

extern "C" int vtx_ragged_reduce(const uint16_t* x, int64_t x_rows, int32_t d0, int32_t d1, uint16_t* o,
                                 int64_t o_rows, int32_t dim, int32_t reduce_type,
                                 const int32_t* winfo_kv_offsets, const int32_t* winfo_kv_lens,
                                 int64_t winfo_capacity, const int32_t* winfo_num_workloads, void* stream) {
  vtx::clear_error();
  const char* what = "ragged_reduce";
  int rc;
  if ((rc = check_walk(what, winfo_kv_offsets, winfo_kv_lens, winfo_capacity, winfo_num_workloads, nullptr,
                       false)))
    return rc;
  const Opnd xo{x, x_rows, d0, d1, VTX_ROWS_RAGGED};
  if ((rc = check_opnd(what, "x", xo, false, false))) return rc;
  if (dim != 1 && dim != 2) return vtx::fail(VTX_E_INVALID, "%s: dim must be 1 or 2, got %d", what, dim);
  if (reduce_type < VTX_REDUCE_MEAN || reduce_type > VTX_REDUCE_SUM)
    return vtx::fail(VTX_E_INVALID, "%s: unknown reduce type %d", what, reduce_type);
  if (!o || o_rows < 0) return vtx::fail(VTX_E_INVALID, "%s: null output", what);
  if (dim == 2 && d1 % 8 == 0 && !vtx::aligned16(x))
    return vtx::fail(VTX_E_INVALID, "%s: x must be 16-byte aligned", what);
  if (winfo_capacity == 0 || o_rows == 0) return VTX_OK;
  ReduceArgs a;
  a.w = make_walk(nullptr, 0, nullptr, winfo_kv_offsets, winfo_kv_lens, winfo_capacity, winfo_num_workloads,
                  o_rows < x_rows ? o_rows : x_rows);
  // the RAGGED rows of x and o are the same positions: clip to both
  a.x = xo;
  a.o = o;
  a.dim = dim;
  a.type = reduce_type;
  reduce_ragged_kernel<<<grid_blocks(winfo_capacity), kThreads, 0, vtx::as_stream(stream)>>>(a);
  return vtx::check_launch(what);
}

extern "C" int vtx_segment_scan(int32_t op, float scale, uint16_t* x, int64_t x_rows, int32_t cols,
                                const int32_t* dense_kv_indptr, int32_t eff_batch_size, int32_t topk_val,
                                int32_t reserved_bos, int32_t reserved_eos, void* stream) {
  vtx::clear_error();
  const char* what = "segment_scan";
  if (op != VTX_SEGMENT_SOFTMAX && op != VTX_SEGMENT_NORMALIZE)
    return vtx::fail(VTX_E_INVALID, "%s: unknown op %d", what, op);
  if (eff_batch_size < 0 || reserved_bos < 0 || reserved_eos < 0 || cols < 1 || x_rows < 0)
    return vtx::fail(VTX_E_INVALID, "%s: negative size", what);
  if (eff_batch_size == 0) return VTX_OK;
  if (!x || !dense_kv_indptr) return vtx::fail(VTX_E_INVALID, "%s: null pointer", what);
  SegArgs a;
  a.x = x;
  a.rows = x_rows;
  a.cols = cols;
  a.indptr = dense_kv_indptr;
  a.segments = eff_batch_size;
  a.scale = scale;
  a.bos = reserved_bos;
  a.eos = reserved_eos;
  a.topk = topk_val;
  a.op = op;
  segment_scan_kernel<<<eff_batch_size, kThreads, 0, vtx::as_stream(stream)>>>(a);
  return vtx::check_launch(what);
}
