// Writes the new tokens' keys and values into the paged K / V pools for
// gfx950 (the step before forward_cache in a decode or prefill).
//
// For token i < nnz and kv head h < H, with pos = loc[i]:
//   row = (pos / P) * (P * H) + h * P + pos % P
//   k_cache[row, :] = new_k[i, h, :],  v_cache[row, :] = new_v[i, h, :]
// i.e. pool row (page * H + h) of [pool * H, P, D], token slot pos % P —
// the layout CMean and the indexer read.  Rows are copied as raw elements
// (the pools hold the new tokens' dtype).  A token whose row falls outside
// the pool (negative or too large loc) is skipped.
//
// One wave copies 64 / LPR (token, head) rows at a time, LPR lanes per row,
// 16-byte vectors; rows of other widths take 4-byte or element-wide copies.
#include "vtx_device.h"
#include "vtx_host.h"

namespace {

constexpr int kThreads = 256;

struct SetKvArgs {
  unsigned char* k;
  unsigned char* v;
  int64_t cache_rows;
  const unsigned char* nk;
  const unsigned char* nv;
  const int64_t* loc;
  int64_t nnz;
  int32_t heads, page;
  int64_t row_bytes;
};

// kW bytes per copy unit (16, 4 or the element size handled as 2 / 1).
template <int kW>
__global__ __launch_bounds__(kThreads) void set_kv_kernel(SetKvArgs a) {
  const int64_t units = a.row_bytes / kW;
  const long long rows = a.nnz * a.heads;
  const long long total = rows * units;
  for (long long it = (long long)blockIdx.x * kThreads + threadIdx.x; it < total;
       it += (long long)gridDim.x * kThreads) {
    const long long r = it / units;
    const long long u = it - r * units;
    const long long i = r / a.heads;
    const int h = (int)(r - i * a.heads);
    const long long pos = a.loc[i];
    if (pos < 0) continue;
    const long long dst = (pos / a.page) * ((long long)a.page * a.heads) + (long long)h * a.page + pos % a.page;
    if (dst >= a.cache_rows) continue;
    const long long so = r * a.row_bytes + u * kW;
    const long long d_o = dst * a.row_bytes + u * kW;
    if (kW == 16) {
      vtx::st16(a.k + d_o, vtx::ld16(a.nk + so));
      vtx::st16(a.v + d_o, vtx::ld16(a.nv + so));
    } else if (kW == 4) {
      *reinterpret_cast<uint32_t*>(a.k + d_o) = *reinterpret_cast<const uint32_t*>(a.nk + so);
      *reinterpret_cast<uint32_t*>(a.v + d_o) = *reinterpret_cast<const uint32_t*>(a.nv + so);
    } else {
      a.k[d_o] = a.nk[so];
      a.v[d_o] = a.nv[so];
    }
  }
}

}  // namespace

extern "C" int vtx_set_kv_buffer(void* k_cache, void* v_cache, int64_t cache_rows, const void* new_k,
                                 const void* new_v, const int64_t* loc, int64_t nnz, int32_t num_kv_heads,
                                 int32_t head_dim, int32_t elem_bytes, int32_t page_size, void* stream) {
  vtx::clear_error();
  if (nnz < 0 || num_kv_heads < 1 || head_dim < 1 || page_size < 1 || cache_rows < 0)
    return vtx::fail(VTX_E_INVALID, "set_kv_buffer: nnz, heads, head_dim and page_size must be positive");
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8)
    return vtx::fail(VTX_E_INVALID, "set_kv_buffer: element size %d not supported", elem_bytes);
  if (nnz == 0) return VTX_OK;
  if (!k_cache || !v_cache || !new_k || !new_v || !loc) return vtx::fail(VTX_E_INVALID, "set_kv_buffer: null pointer");
  SetKvArgs a;
  a.k = static_cast<unsigned char*>(k_cache);
  a.v = static_cast<unsigned char*>(v_cache);
  a.cache_rows = cache_rows;
  a.nk = static_cast<const unsigned char*>(new_k);
  a.nv = static_cast<const unsigned char*>(new_v);
  a.loc = loc;
  a.nnz = nnz;
  a.heads = num_kv_heads;
  a.page = page_size;
  a.row_bytes = (int64_t)head_dim * elem_bytes;
  const bool all16 = a.row_bytes % 16 == 0 && vtx::aligned16(k_cache) && vtx::aligned16(v_cache) &&
                     vtx::aligned16(new_k) && vtx::aligned16(new_v);
  const bool all4 = a.row_bytes % 4 == 0 && ((uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)new_k |
                                             (uintptr_t)new_v) % 4 == 0;
  const int w = all16 ? 16 : (all4 ? 4 : 1);
  const long long total = nnz * num_kv_heads * (a.row_bytes / w);
  const int cus = vtx::device_cu_count();
  long long grid = (total + kThreads - 1) / kThreads;
  const long long cap = 8LL * (cus > 0 ? cus : 256);
  if (grid > cap) grid = cap;
  hipStream_t s = vtx::as_stream(stream);
  if (w == 16) set_kv_kernel<16><<<(int)grid, kThreads, 0, s>>>(a);
  else if (w == 4) set_kv_kernel<4><<<(int)grid, kThreads, 0, s>>>(a);
  else set_kv_kernel<1><<<(int)grid, kThreads, 0, s>>>(a);
  return vtx::check_launch("set_kv_buffer");
}
