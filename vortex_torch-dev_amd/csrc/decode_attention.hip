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
// One workgroup per segment (8 waves, or 4 for wide G x D).  The segment's
// page rows are staged in LDS first (one load per page, up to kPageCap
// pages; longer segments read them from the table), so each batch of a
// wave costs one memory round trip: a wave takes every kWaves-th batch of
// kB groups of kRowsPerLoad consecutive tokens (LPR lanes per token, 16-byte
// vectors of K and V; a batch is one contiguous run of rows), and issues the
// next batch's K and V loads
// before it computes on the current one (two register buffers).  It keeps a
// running max and per-lane partial sums (online softmax); the waves'
// (max, sum, accumulator) are merged in LDS.  At decode batch sizes the
// q . K products are G rows against a few hundred tokens: HBM-bound, so the
// kernel runs on the VALU.
#include "vtx_device.h"
#include "vtx_host.h"

namespace {

constexpr int kPageCap = 2048;  // page rows staged in LDS

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

// Threads per workgroup: 8 waves where a wave's registers fit 128 (rows of
// one 16-byte vector per lane, at most two query heads), else 4.
template <int LPR, int VPL, int kG>
constexpr int attn_threads() {
  return VPL == 1 && kG <= 2 ? 512 : 256;
}
// Token groups per batch (two batches in registers at a time).
template <int VPL, int kG>
constexpr int attn_batch() {
  return VPL == 1 ? (kG == 1 ? 4 : (kG == 2 ? 3 : 2)) : (kG == 1 ? 2 : 1);
}

// With 8 waves, at most 128 registers (four waves per SIMD: two workgroups per CU).
template <int LPR, int VPL, int kG>
__global__ __launch_bounds__((attn_threads<LPR, VPL, kG>()),
                             (attn_threads<LPR, VPL, kG>() == 512 ? 4 : 1)) void paged_decode_attention_kernel(AttnArgs a) {
  constexpr int T = attn_threads<LPR, VPL, kG>();
  constexpr int kWaves = T / vtx::kWave;
  constexpr int kRowsPerLoad = vtx::kWave / LPR;  // tokens per wave-wide load
  constexpr int kB = attn_batch<VPL, kG>();        // token groups per batch
  __shared__ int32_t s_rows[kPageCap];
  __shared__ float s_m[kWaves][kG];
  __shared__ float s_l[kWaves][kG];
  __shared__ float s_acc[kWaves][kG][LPR * VPL * 8];

  const int seg = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = vtx::uniform(tid / vtx::kWave);
  const int lane = vtx::lane_id();
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int G = a.G, D = a.D, P = a.P;

  const long long start = a.indptr[seg];
  const long long m = (long long)a.indptr[seg + 1] - start;
  int T_tok = 0;  // tokens of the segment
  if (m > 0 && start >= 0 && start + m <= a.indices_len && a.rows > 0) {
    int last = a.last_len[seg];
    last = last < 0 ? 0 : (last > P ? P : last);
    const long long t = (m - 1) * P + last;
    T_tok = t < (1LL << 30) ? (int)t : 0;  // (token indices, with the prefetch past the end, fit an int)
  }
  // query slice of this lane (columns (v * LPR + col) * 8 .. + 8), requested
  // first so that it arrives with the page rows; heads past G read head
  // G - 1 and are zeroed by a select (no branch around the load, which would
  // make the wave wait for it there)
  vtx::U4 qraw[kG][VPL];
#pragma unroll
  for (int g = 0; g < kG; ++g)
#pragma unroll
    for (int v = 0; v < VPL; ++v)
      qraw[g][v] = vtx::ld16(a.q + ((long long)seg * G + (g < G ? g : G - 1)) * D + (v * LPR + col) * 8);

  // the segment's page rows (-1: outside the pool)
  const bool staged = m <= kPageCap;
  if (staged && T_tok > 0) {
    for (int i = tid; i < (int)m; i += T) {
      const int r = a.indices[start + i];
      s_rows[i] = (r >= 0 && r < a.rows) ? r : -1;
    }
  }

  float qs[kG][VPL][8];
#pragma unroll
  for (int g = 0; g < kG; ++g)
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      float f[8];
      vtx::unpack8(qraw[g][v], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) qs[g][v][e] = g < G ? f[e] : 0.f;
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
  __syncthreads();  // page rows staged

  const int groups = (T_tok + kRowsPerLoad - 1) / kRowsPerLoad;
  // batches of this wave: groups (wave + kWaves * j) * kB + i, i < kB (a
  // batch is kB consecutive groups: one contiguous run of a page's rows)
  const int batches = (groups + kB - 1) / kB;
  const int nb = batches > wave ? (batches - wave + kWaves - 1) / kWaves : 0;

  // K and V of batch j; tokens past the segment or on rows outside the pool
  // load the pool's first row (a valid address) and are masked off
  auto load = [&](int j, vtx::U4 (&kv)[kB][VPL], vtx::U4 (&vv)[kB][VPL], bool (&ok)[kB]) {
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const int t = ((wave + kWaves * j) * kB + i) * kRowsPerLoad + grp;
      int row = -1, slot = 0;
      if (t < T_tok) {
        const int pg = t / P;
        slot = t - pg * P;
        if (staged) {
          row = s_rows[pg];
        } else {
          const int r = a.indices[start + pg];
          row = (r >= 0 && r < a.rows) ? r : -1;
        }
      }
      ok[i] = row >= 0;
      const long long base = ok[i] ? ((long long)row * P + slot) * (long long)D : 0;
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        kv[i][v] = vtx::ld16_stream(a.k + base + (v * LPR + col) * 8);
        vv[i][v] = vtx::ld16_stream(a.v + base + (v * LPR + col) * 8);
      }
    }
  };
  auto compute = [&](const vtx::U4 (&kv)[kB][VPL], const vtx::U4 (&vv)[kB][VPL], const bool (&ok)[kB]) {
    // scores: every lane of a token's LPR group ends with the full dot
    float sc[kB][kG];
#pragma unroll
    for (int i = 0; i < kB; ++i)
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        float s = vtx::dot_row<VPL>(kv[i], qs[g]);
#pragma unroll
        for (int d = LPR / 2; d >= 1; d >>= 1) s += vtx::xshfl(s, d);
        sc[i][g] = ok[i] ? s * a.scale : -INFINITY;
      }
    // online softmax: the wave's running max covers every token it has seen
#pragma unroll
    for (int g = 0; g < kG; ++g) {
      float bm = sc[0][g];
#pragma unroll
      for (int i = 1; i < kB; ++i) bm = fmaxf(bm, sc[i][g]);
#pragma unroll
      for (int d = LPR; d < vtx::kWave; d <<= 1) bm = fmaxf(bm, vtx::xshfl(bm, d));
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
  };

  // two register buffers: batch j + 1's loads are in flight while batch j
  // is computed (the loads are unconditional, so the wait for a buffer is
  // for its own loads only)
  if (nb > 0) {  // uniform over the wave
    vtx::U4 ka[kB][VPL], va[kB][VPL], kb[kB][VPL], vb[kB][VPL];
    bool oka[kB], okb[kB];
    load(0, ka, va, oka);
    for (int j = 0; j < nb; j += 2) {
      load(j + 1, kb, vb, okb);
      compute(ka, va, oka);
      load(j + 2, ka, va, oka);
      if (j + 1 < nb) compute(kb, vb, okb);
    }
  }

  // fold the token groups of the wave (lanes that share col), then the waves
#pragma unroll
  for (int g = 0; g < kG; ++g) {
#pragma unroll
    for (int d = LPR; d < vtx::kWave; d <<= 1) {
      l[g] += vtx::xshfl(l[g], d);
#pragma unroll
      for (int v = 0; v < VPL; ++v)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][v][e] += vtx::xshfl(acc[g][v][e], d);
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
  for (int idx = tid; idx < G * D; idx += T) {
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

template <int LPR, int VPL, int kG>
void launch_one(const AttnArgs& a, hipStream_t s) {
  paged_decode_attention_kernel<LPR, VPL, kG><<<a.segments, attn_threads<LPR, VPL, kG>(), 0, s>>>(a);
}

template <int LPR, int VPL>
int launch_g(const AttnArgs& a, hipStream_t s) {
  if (a.G <= 1) launch_one<LPR, VPL, 1>(a, s);
  else if (a.G <= 2) launch_one<LPR, VPL, 2>(a, s);
  else if (a.G <= 4) launch_one<LPR, VPL, 4>(a, s);
  else launch_one<LPR, VPL, 8>(a, s);
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
