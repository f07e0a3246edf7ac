// Segmented top-k page select for gfx950 with reserved BOS/EOS pages.
//
// Semantics follow the reference topk_output / TopKOutput_BF16_Kernel
// (csrc/topk.cu:56-203), which stably sorts each segment's middle scores in
// descending order and keeps the first topk_val: the output is the topk_val
// best pages, best first, ties resolved toward the lower position.
//
// Instead of sorting the whole segment this kernel selects and then orders
// only the k winners.  One workgroup per segment.  A segment of at most one
// page per thread with k <= 32 takes the bitonic select (vtx_select.h).
// Otherwise every score becomes a
// 16-bit order key (bf16 bits with the sign folded, -0.0 == +0.0), cached in
// LDS; a two-pass radix select (vtx_select.h) collects the k winners; each
// winner's output rank is the number of winners with a larger composite
// (key << 32 | ~position), i.e. score descending, position ascending — the
// order a stable descending sort produces.
#include "vtx_device.h"
#include "vtx_host.h"
#include "vtx_select.h"

namespace {

struct TopkArgs {
  const uint16_t* score;
  int64_t score_len;
  const int32_t* dindptr;
  const int32_t* sindptr;
  const int32_t* didx;
  int64_t didx_len;
  int32_t* sidx;
  int64_t sidx_len;
  int32_t topk, bos, eos;
  int32_t key_cap;  // segments up to this many pages keep their keys in LDS
};

template <int T>
__global__ __launch_bounds__(T) void topk_select_kernel(TopkArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ vtx::SelectShared<T> sh;
  __shared__ vtx::BitonicShared<T> bsh;

  const int seg = blockIdx.x;
  const int tid = threadIdx.x;
  const int k = a.topk;

  const long long start = (long long)a.dindptr[seg] + a.bos;
  const long long end = (long long)a.dindptr[seg + 1] - a.eos;
  const long long n = end - start;
  if (k <= 0 || n <= k) return;  // the planner already placed every page
  if (start < 0 || end > a.score_len || end > a.didx_len) return;
  const long long obase = (long long)a.sindptr[seg] + a.bos;
  if (obase < 0 || obase + k > a.sidx_len) return;

  uint64_t* sel = reinterpret_cast<uint64_t*>(smem);
  uint16_t* keys = reinterpret_cast<uint16_t*>(smem + (size_t)vtx::sel_slots(k) * sizeof(uint64_t));
  const uint16_t* sc = a.score + start;

  if (n <= T && k <= vtx::kMaxBitonicK) {  // uniform: one score per thread, the bitonic select
    const int i = tid;
    const uint16_t v = sc[i < n ? i : n - 1];  // (past n: position n - 1, not used)
    const uint32_t comp = vtx::bitonic_comp(i < n, vtx::score_key(v), i);
    vtx::select_bitonic<T>(comp, k, bsh, [&](int r, uint32_t c) {
      a.sidx[obase + r] = a.didx[start + vtx::bitonic_position(c)];
    });
    return;
  }

  if (n <= a.key_cap) {
    constexpr int kU = 4;  // score loads in flight per thread
    for (long long i0 = 0; i0 < n; i0 += (long long)T * kU) {
      // positions past n read (and rewrite) position n - 1: no branch around
      // a load, which would let the compiler wait for each load on its own
      uint16_t v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const long long i = i0 + (long long)u * T + tid;
        v[u] = sc[i < n ? i : n - 1];
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const long long i = i0 + (long long)u * T + tid;
        keys[i < n ? i : n - 1] = (uint16_t)vtx::score_key(v[u]);
      }
    }
    __syncthreads();
    vtx::select_topk<T>([&](long long i) { return (uint32_t)keys[i]; }, n, k, sel, sh);
  } else {
    vtx::select_topk<T>([&](long long i) { return vtx::score_key(sc[i]); }, n, k, sel, sh);
  }

  vtx::select_emit<T>(sel, k, n, [&](int r, long long pos) { a.sidx[obase + r] = a.didx[start + pos]; });
}

constexpr int kMaxTopk = 4096;
constexpr int kLdsBudget = 56 * 1024;  // dynamic LDS per workgroup (the select tables take ~6 KB more)

}  // namespace

extern "C" int vtx_topk_select(const uint16_t* score, int64_t score_len,
                               const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr,
                               const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                               int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                               int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos,
                               int32_t reserved_eos, int32_t max_num_pages, void* stream) {
  vtx::clear_error();
  if (eff_batch_size < 0) return vtx::fail(VTX_E_INVALID, "topk_select: eff_batch_size < 0");
  if (reserved_bos < 0 || reserved_eos < 0)
    return vtx::fail(VTX_E_INVALID, "topk_select: reserved_bos/eos must be >= 0");
  if (topk_val > kMaxTopk)
    return vtx::fail(VTX_E_INVALID, "topk_select: topk_val %d exceeds %d", topk_val, kMaxTopk);
  if (eff_batch_size == 0 || topk_val <= 0) return VTX_OK;
  if (!score || !dense_kv_indptr || !sparse_kv_indptr || !dense_kv_indices || !sparse_kv_indices)
    return vtx::fail(VTX_E_INVALID, "topk_select: null pointer");

  TopkArgs a;
  a.score = score;
  a.score_len = score_len;
  a.dindptr = dense_kv_indptr;
  a.sindptr = sparse_kv_indptr;
  a.didx = dense_kv_indices;
  a.didx_len = dense_kv_indices_len;
  a.sidx = sparse_kv_indices;
  a.sidx_len = sparse_kv_indices_len;
  a.topk = topk_val;
  a.bos = reserved_bos;
  a.eos = reserved_eos;

  long long want = max_num_pages > 0 ? max_num_pages : 0;
  const long long room = (kLdsBudget - (long long)vtx::sel_slots(topk_val) * 8) / 2;
  long long cap = want < room ? want : room;
  cap &= ~7LL;
  if (cap < 0) cap = 0;
  a.key_cap = (int32_t)cap;
  const size_t lds = (size_t)vtx::sel_slots(topk_val) * 8 + (size_t)cap * 2;

  hipStream_t s = vtx::as_stream(stream);
  // (up to 512 pages and k <= 32: 512 threads, one page each, for the
  // bitonic select)
  if (max_num_pages <= 256 || (max_num_pages <= 512 && topk_val > vtx::kMaxBitonicK)) {
    topk_select_kernel<256><<<eff_batch_size, 256, lds, s>>>(a);
  } else if (max_num_pages <= 2048) {
    topk_select_kernel<512><<<eff_batch_size, 512, lds, s>>>(a);
  } else {
    topk_select_kernel<1024><<<eff_batch_size, 1024, lds, s>>>(a);
  }
  return vtx::check_launch("topk_select");
}
