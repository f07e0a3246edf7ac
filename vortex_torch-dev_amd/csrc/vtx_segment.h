// Per-column statistics of a segment's middle positions, shared by the
// in-place segment softmax / normalize and the fused GQA indexer so that
// both produce the same bits.
#pragma once

#include "vtx_device.h"

namespace vtx {

constexpr int kScanThreads = 256;  // threads that take part in column_scan_stats
constexpr int kScanRegs = 8;       // rows a thread keeps in registers

// For each of cols <= kScanThreads columns of cnt rows (val_at(r, c) -> fp32):
//   softmax: pm[c] = M = max_r v * scale, ps[c] = S = sum_r exp(v * scale - M)
//   else:    ps[c] = sum_r v^2
// Thread t < kScanThreads takes column t % cols and rows t / cols + k * per_col
// (per_col = kScanThreads / cols), in increasing r: a running maximum
// (from -1e30) with rescaled sum, or a sum of squares.  The partials are then
// merged in a fixed order — for power-of-two cols <= 64 a butterfly within
// each wave and the waves in order, else an LDS tree (step h: thread row r0
// absorbs r0 + h) — so the result depends only on (cnt, cols) and the values.  Threads at or past
// kScanThreads only take part in the barriers: every thread of the block
// must call it.  pm / ps: LDS arrays of kScanThreads floats.  When in_regs
// comes back true, vals[k] holds the thread's row r0 + k * per_col.
template <typename ValAt>
__device__ __forceinline__ void column_scan_stats(ValAt val_at, long long cnt, int cols, float scale, bool softmax,
                                                  float* pm, float* ps, float (&vals)[kScanRegs], bool& in_regs) {
  const int tid = threadIdx.x;
  const int per_col = kScanThreads / cols;
  const int c = tid % cols;
  const int r0 = tid / cols;
  const bool active = tid < kScanThreads && r0 < per_col;
  in_regs = cnt <= (long long)per_col * kScanRegs;  // uniform
  if (in_regs && cnt > 0) {
    // every read issued before any is used: rows past cnt (and threads past
    // the scan) read row 0 and drop it through a select, with no branch
    // around a read for the compiler to sink it into
#pragma unroll
    for (int k = 0; k < kScanRegs; ++k) {
      const long long r = r0 + (long long)k * per_col;
      const bool in = active && r < cnt;
      const float v = val_at(in ? r : 0, c);
      vals[k] = in ? v : 0.f;
    }
  } else if (in_regs) {
#pragma unroll
    for (int k = 0; k < kScanRegs; ++k) vals[k] = 0.f;
  }
  float m = -1e30f, s = 0.f;
  auto add = [&](float v) {
    if (softmax) {
      const float u = v * scale;
      if (u > m) {
        s = s * __expf(m - u) + 1.f;
        m = u;
      } else {
        s += __expf(u - m);
      }
    } else {
      s = fmaf(v, v, s);
    }
  };
  if (active) {
    if (in_regs) {
#pragma unroll
      for (int k = 0; k < kScanRegs; ++k)
        if (r0 + (long long)k * per_col < cnt) add(vals[k]);
    } else {
      for (long long r = r0; r < cnt; r += per_col) add(val_at(r, c));
    }
  }
  auto merge = [&](float& m1, float& s1, float m2, float s2) {
    if (softmax) {
      const float M = fmaxf(m1, m2);
      s1 = s1 * __expf(m1 - M) + s2 * __expf(m2 - M);
      m1 = M;
    } else {
      s1 += s2;
    }
  };
  if ((cols & (cols - 1)) == 0 && cols <= kWave) {
    // Power-of-two columns: the lanes of a wave that share a column merge by
    // an xor butterfly (strides cols .. 32), then thread c < cols merges the
    // waves' partials in wave order — two barriers instead of a tree.
    // (strides cols .. 32 as compile-time constants, so that the shuffles are
    // VALU ones: d >= cols is uniform)
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1)
      if (d >= cols) merge(m, s, xshfl(m, d), xshfl(s, d));
    const int wave = tid / kWave;
    if (tid < kScanThreads && (tid % kWave) < cols) {
      pm[wave * cols + c] = m;
      ps[wave * cols + c] = s;
    }
    __syncthreads();
    if (tid < cols) {
      float M = pm[c], S = ps[c];
      for (int w = 1; w < kScanThreads / kWave; ++w) merge(M, S, pm[w * cols + c], ps[w * cols + c]);
      pm[c] = M;
      ps[c] = S;
    }
    __syncthreads();
    return;
  }
  if (tid < kScanThreads) {
    pm[tid] = m;
    ps[tid] = s;
  }
  __syncthreads();
  for (int h = 1; h < per_col; h <<= 1) {
    if (active && (r0 % (2 * h)) == 0 && r0 + h < per_col) {
      const int o = (r0 + h) * cols + c;
      if (softmax) {
        const float m1 = pm[tid], m2 = pm[o];
        const float M = fmaxf(m1, m2);
        ps[tid] = ps[tid] * __expf(m1 - M) + ps[o] * __expf(m2 - M);
        pm[tid] = M;
      } else {
        ps[tid] += ps[o];
      }
    }
    __syncthreads();
  }
}

// The softmax of one value given its column's statistics (M, S).
__device__ __forceinline__ float softmax_value(float v, float scale, float M, float S) {
  return __expf(v * scale - M) / S;
}

}  // namespace vtx
