// Paged decode attention over a block table for gfx950: the consumer of the
// indexer's sparse block table (or of the dense one, for full attention).
//
// Segment s = b * H + h (request b, kv head h) attends to the tokens of the
// pages kv_indices[kv_indptr[s] .. kv_indptr[s+1]) — each entry a row of the
// K / V pools [rows, P, D] (page * H + h) — all P tokens of every page but
// the last, of which kv_last_page_len[s]; its G query heads (rows s*G + g of
// q [B*H*G, D]) each get
//   o[s*G + g] = sum_t softmax_t(sm_scale * q . K[t]) V[t]      (bf16 out)
// with fp32 scores, an fp32 online softmax and fp32 accumulation.  A segment
// with no tokens writes zeros.
//
// One workgroup (4 waves) per segment.  A wave takes every fourth group of
// kRowsPerLoad consecutive tokens (LPR lanes per token, 16-byte vectors of
// K and V), kB groups per batch with all their K and V loads issued before
// any arithmetic, and keeps a running max and per-lane partial sums; the
// waves' (max, sum, accumulator) are merged in LDS.  At decode batch sizes
// the q . K products are G rows against a few hundred tokens: HBM-bound, so
// the kernel runs on the VALU.
#include "vtx_device.h"
#include "vtx_host.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / vtx::kWave;

struct AttnArgs {
  const uint16_t* q;
  uint16_t* o;
  const uint16_t* k;
  const uint16_t* v;
  int64_t rows;  // pool rows (page * H + h)
  const int32_t* indptr;
  const int32_t* indices;
  int64_t indices_len;
  const int32_t* last_len;
  int32_t segments, G, D, P;
  float scale;
};

template <int LPR, int VPL, int kG>
__global__ __launch_bounds__(kThreads) void paged_decode_attention_kernel(AttnArgs a) {
  constexpr int kRowsPerLoad = vtx::kWave / LPR;  // tokens per wave-wide load
  constexpr int kB = VPL == 1 ? 8 : 4;             // token groups per batch
  __shared__ float s_m[kWaves][kG];
  __shared__ float s_l[kWaves][kG];
  __shared__ float s_acc[kWaves][kG][LPR * VPL * 8];

  const int seg = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = tid / vtx::kWave;
  const int lane = vtx::lane_id();
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int G = a.G, D = a.D, P = a.P;

  const long long start = a.indptr[seg];
  const long long m = (long long)a.indptr[seg + 1] - start;
  long long T = 0;  // tokens of the segment
  if (m > 0 && start >= 0 && start + m <= a.indices_len) {
    int last = a.last_len[seg];
    last = last < 0 ? 0 : (last > P ? P : last);
    T = (m - 1) * P + last;
  }

  // query slice of this lane (columns (v * LPR + col) * 8 .. + 8)
  float qs[kG][VPL][8];
#pragma unroll
  for (int g = 0; g < kG; ++g)
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      if (g < G) {
        vtx::unpack8(vtx::ld16(a.q + ((long long)seg * G + g) * D + (v * LPR + col) * 8), qs[g][v]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qs[g][v][e] = 0.f;
      }
    }

  float mx[kG], l[kG], acc[kG][VPL][8];
#pragma unroll
  for (int g = 0; g < kG; ++g) {
    mx[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int v = 0; v < VPL; ++v)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][v][e] = 0.f;
  }

  const long long groups = (T + kRowsPerLoad - 1) / kRowsPerLoad;
  for (long long g0 = wave; g0 < groups; g0 += (long long)kWaves * kB) {
    vtx::U4 kv[kB][VPL], vv[kB][VPL];
    bool ok[kB];
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const long long t = (g0 + (long long)i * kWaves) * kRowsPerLoad + grp;
      ok[i] = t < T;
      long long row = 0;
      int slot = 0;
      if (ok[i]) {
        row = a.indices[start + t / P];
        slot = (int)(t % P);
        if (row < 0 || row >= a.rows) {
          ok[i] = false;
          row = 0;
        }
      }
      const long long base = (row * P + slot) * (long long)D;
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        if (ok[i]) {
          kv[i][v] = vtx::ld16_stream(a.k + base + (v * LPR + col) * 8);
          vv[i][v] = vtx::ld16_stream(a.v + base + (v * LPR + col) * 8);
        } else {
          kv[i][v] = vtx::U4{0u, 0u, 0u, 0u};
          vv[i][v] = vtx::U4{0u, 0u, 0u, 0u};
        }
      }
    }
    // scores: every lane of a token's LPR group ends with the full dot
    float sc[kB][kG];
#pragma unroll
    for (int i = 0; i < kB; ++i)
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        float s = vtx::dot_row<VPL>(kv[i], qs[g]);
#pragma unroll
        for (int d = LPR / 2; d >= 1; d >>= 1) s += __shfl_xor(s, d, vtx::kWave);
        sc[i][g] = ok[i] ? s * a.scale : -INFINITY;
      }
    // online softmax: the wave's running max covers every token it has seen
#pragma unroll
    for (int g = 0; g < kG; ++g) {
      float bm = sc[0][g];
#pragma unroll
      for (int i = 1; i < kB; ++i) bm = fmaxf(bm, sc[i][g]);
      for (int d = LPR; d < vtx::kWave; d <<= 1) bm = fmaxf(bm, __shfl_xor(bm, d, vtx::kWave));
      const float nm = fmaxf(mx[g], bm);
      if (nm == -INFINITY) continue;  // nothing seen yet (wave-uniform)
      const float r = __expf(mx[g] - nm);
      l[g] *= r;
#pragma unroll
      for (int v = 0; v < VPL; ++v)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][v][e] *= r;
#pragma unroll
      for (int i = 0; i < kB; ++i) {
        const float p = __expf(sc[i][g] - nm);  // 0 for masked tokens
        l[g] += p;
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
          float vf[8];
          vtx::unpack8(vv[i][v], vf);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[g][v][e] = fmaf(p, vf[e], acc[g][v][e]);
        }
      }
      mx[g] = nm;
    }
  }
  // fold the token groups of the wave (lanes that share col), then the waves
#pragma unroll
  for (int g = 0; g < kG; ++g) {
    for (int d = LPR; d < vtx::kWave; d <<= 1) {
      l[g] += __shfl_xor(l[g], d, vtx::kWave);
#pragma unroll
      for (int v = 0; v < VPL; ++v)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][v][e] += __shfl_xor(acc[g][v][e], d, vtx::kWave);
    }
    if (lane == 0) {
      s_m[wave][g] = mx[g];
      s_l[wave][g] = l[g];
    }
    if (grp == 0) {
#pragma unroll
      for (int v = 0; v < VPL; ++v)
#pragma unroll
        for (int e = 0; e < 8; ++e) s_acc[wave][g][(v * LPR + col) * 8 + e] = acc[g][v][e];
    }
  }
  __syncthreads();
  // one thread per (g, column) writes the merged output
  for (int idx = tid; idx < G * D; idx += kThreads) {
    const int g = idx / D;
    const int d = idx - g * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][g]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float f = __expf(s_m[w][g] - M);
        L = fmaf(s_l[w][g], f, L);
        O = fmaf(s_acc[w][g][d], f, O);
      }
    }
    a.o[((long long)seg * G + g) * D + d] = (uint16_t)vtx::f32_to_bf16(L > 0.f ? O / L : 0.f);
  }
}

template <int LPR, int VPL>
int launch_g(const AttnArgs& a, hipStream_t s) {
  if (a.G <= 1) paged_decode_attention_kernel<LPR, VPL, 1><<<a.segments, kThreads, 0, s>>>(a);
  else if (a.G <= 2) paged_decode_attention_kernel<LPR, VPL, 2><<<a.segments, kThreads, 0, s>>>(a);
  else if (a.G <= 4) paged_decode_attention_kernel<LPR, VPL, 4><<<a.segments, kThreads, 0, s>>>(a);
  else paged_decode_attention_kernel<LPR, VPL, 8><<<a.segments, kThreads, 0, s>>>(a);
  return vtx::check_launch("paged_decode_attention");
}

}  // namespace

extern "C" int vtx_paged_decode_attention_supported(int32_t head_dim, int32_t group_size) {
  return (head_dim == 64 || head_dim == 128 || head_dim == 256) && group_size >= 1 && group_size <= 8;
}

extern "C" int vtx_paged_decode_attention(const uint16_t* q, uint16_t* o, const uint16_t* k_cache,
                                          const uint16_t* v_cache, int64_t cache_rows, const int32_t* kv_indptr,
                                          const int32_t* kv_indices, int64_t kv_indices_len,
                                          const int32_t* kv_last_page_len, int32_t batch_size,
                                          int32_t num_kv_heads, int32_t group_size, int32_t head_dim,
                                          int32_t page_size, float sm_scale, void* stream) {
  vtx::clear_error();
  const char* what = "paged_decode_attention";
  if (batch_size < 0 || num_kv_heads < 1 || page_size < 1 || cache_rows < 0 || kv_indices_len < 0)
    return vtx::fail(VTX_E_INVALID, "%s: bad sizes", what);
  if (!vtx_paged_decode_attention_supported(head_dim, group_size))
    return vtx::fail(VTX_E_INVALID, "%s: head_dim %d with %d query heads per kv head not supported", what,
                     head_dim, group_size);
  const long long segments = (long long)batch_size * num_kv_heads;
  if (segments == 0) return VTX_OK;
  if (segments > 0x7fffffffLL) return vtx::fail(VTX_E_INVALID, "%s: too many segments", what);
  if (!q || !o || !k_cache || !v_cache || !kv_indptr || !kv_last_page_len || (kv_indices_len > 0 && !kv_indices))
    return vtx::fail(VTX_E_INVALID, "%s: null pointer", what);
  if (!vtx::aligned16(q) || !vtx::aligned16(k_cache) || !vtx::aligned16(v_cache))
    return vtx::fail(VTX_E_INVALID, "%s: q, k_cache and v_cache must be 16-byte aligned", what);
  AttnArgs a;
  a.q = q;
  a.o = o;
  a.k = k_cache;
  a.v = v_cache;
  a.rows = cache_rows;
  a.indptr = kv_indptr;
  a.indices = kv_indices;
  a.indices_len = kv_indices_len;
  a.last_len = kv_last_page_len;
  a.segments = (int32_t)segments;
  a.G = group_size;
  a.D = head_dim;
  a.P = page_size;
  a.scale = sm_scale;
  hipStream_t s = vtx::as_stream(stream);
  switch (head_dim) {
    case 64: return launch_g<8, 1>(a, s);
    case 128: return launch_g<16, 1>(a, s);
    default: return launch_g<16, 2>(a, s);
  }
}
