// Bandwidth probes of the box, for the measurement: what the HBM delivers to
// a kernel that does nothing but read, in the two access patterns of this
// path.  They have no counterpart in the reference; bench.py reports their
// rates beside the indexer's as the achievable ceiling.
//
//   vtx_probe_read   a sequential read of `bytes` (16-byte nontemporal
//                    loads, 8 in flight per lane, grid-stride);
//   vtx_probe_gather the indexer's bulk without its arithmetic: each wave
//                    takes a pass of consecutive entries of a row-id list
//                    (64 for 256-byte rows, 16 for 1152-byte rows: the
//                    scoring passes of the indexer; one coalesced load) and
//                    reads those rows of a pool (16-byte nontemporal loads,
//                    all of the pass in flight before any is used).  With an
//                    indptr array, each workgroup first loads an entry of it
//                    and only then its row ids — the fused kernel's chain of
//                    dependent trips (bounds, row ids, rows).
//
// The loaded words are folded into one value per lane, stored only when it
// equals a value the caller passes and the data never produce (so the loads
// cannot be dropped and the stores do not add traffic).
#include "vtx_device.h"
#include "vtx_host.h"

namespace {

constexpr int kProbeThreads = 512;
constexpr int kReadBatch = 8;  // 16-byte loads per lane in flight

__global__ __launch_bounds__(kProbeThreads) void probe_read_kernel(const vtx::U4* src, long long n16, uint32_t* sink,
                                                                   uint32_t magic) {
  uint32_t acc = 0;
  const long long stride = (long long)gridDim.x * kProbeThreads;
  long long i = (long long)blockIdx.x * kProbeThreads + threadIdx.x;
  for (; i + (kReadBatch - 1) * stride < n16; i += kReadBatch * stride) {
    vtx::U4 v[kReadBatch];
#pragma unroll
    for (int u = 0; u < kReadBatch; ++u) v[u] = vtx::ld16_stream(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < kReadBatch; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const vtx::U4 v = vtx::ld16_stream(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == magic) sink[blockIdx.x * kProbeThreads + threadIdx.x] = acc;
}

// kVec 16-byte vectors per row; kLanes lanes per row (a wave-wide load
// covers 64 / kLanes rows); kPassRows rows per wave, every load of them in
// flight before any is used — the indexer's scoring pass.
template <int kVec, int kLanes, int kPassRows>
__global__ __launch_bounds__(kProbeThreads) void probe_gather_kernel(const uint16_t* pool, long long pool_rows,
                                                                     const int32_t* rows, long long n_rows,
                                                                     const int32_t* indptr, int32_t segs,
                                                                     uint32_t* sink, uint32_t magic) {
  constexpr int kRowsPerLoad = vtx::kWave / kLanes;
  constexpr int kVpl = kVec / kLanes;  // vectors per lane per row
  constexpr int kSlots = kPassRows / kRowsPerLoad;
  static_assert(kSlots * kRowsPerLoad == kPassRows && kVpl * kLanes == kVec, "geometry");
  const int lane = vtx::lane_id();
  const int wave = threadIdx.x / vtx::kWave;
  const int grp = lane / kLanes, col = lane % kLanes;
  long long base = ((long long)blockIdx.x * (kProbeThreads / vtx::kWave) + wave) * kPassRows;
  if (indptr)  // the fused kernel's head: the row ids wait for a load of the segment's bounds
    base += indptr[blockIdx.x % (unsigned)segs] == INT32_MIN ? 1 : 0;
  if (base >= n_rows) return;
  const int my_row = lane < kPassRows && base + lane < n_rows ? rows[base + lane] : -1;
  uint32_t acc = 0;
  vtx::U4 v[kSlots][kVpl];
#pragma unroll
  for (int ii = 0; ii < kSlots; ++ii) {
    long long r = __shfl(my_row, ii * kRowsPerLoad + grp, vtx::kWave);
    if (r < 0 || r >= pool_rows) r = 0;
#pragma unroll
    for (int u = 0; u < kVpl; ++u) v[ii][u] = vtx::ld16_stream(pool + r * kVec * 8 + (u * kLanes + col) * 8);
  }
#pragma unroll
  for (int ii = 0; ii < kSlots; ++ii)
#pragma unroll
    for (int u = 0; u < kVpl; ++u) acc ^= v[ii][u].x ^ v[ii][u].y ^ v[ii][u].z ^ v[ii][u].w;
  if (acc == magic) sink[(long long)blockIdx.x * kProbeThreads + threadIdx.x] = acc;
}

}  // namespace

extern "C" int vtx_probe_read(const void* src, int64_t bytes, uint32_t* sink, int64_t sink_len, uint32_t magic,
                              void* stream) {
  vtx::clear_error();
  if (!src || !sink || bytes < 0 || !vtx::aligned16(src))
    return vtx::fail(VTX_E_INVALID, "probe_read: bad arguments");
  const int cus = vtx::device_cu_count();
  if (cus <= 0) return vtx::fail(VTX_E_DEVICE, "probe_read: cannot query the compute unit count");
  const long long blocks = 4LL * cus;  // two 512-thread workgroups per CU, twice over
  if (sink_len < blocks * kProbeThreads)
    return vtx::fail(VTX_E_INVALID, "probe_read: sink needs %lld entries", blocks * kProbeThreads);
  if (bytes < 16) return VTX_OK;
  probe_read_kernel<<<(int)blocks, kProbeThreads, 0, vtx::as_stream(stream)>>>(
      static_cast<const vtx::U4*>(src), bytes / 16, sink, magic);
  return vtx::check_launch("probe_read");
}

extern "C" int vtx_probe_gather(const uint16_t* pool, int64_t pool_rows, int32_t row_bytes, const int32_t* rows,
                                int64_t n_rows, const int32_t* indptr, int32_t segments, uint32_t* sink,
                                int64_t sink_len, uint32_t magic, void* stream) {
  vtx::clear_error();
  if (!pool || !rows || !sink || pool_rows <= 0 || n_rows < 0 || !vtx::aligned16(pool) ||
      (indptr && segments <= 0))
    return vtx::fail(VTX_E_INVALID, "probe_gather: bad arguments");
  if (row_bytes != 256 && row_bytes != 1152)
    return vtx::fail(VTX_E_INVALID, "probe_gather: row_bytes %d not supported (256, 1152)", row_bytes);
  const int pass = row_bytes == 256 ? 64 : 16;  // rows per wave, as the indexer's scoring passes
  const long long waves = (n_rows + pass - 1) / pass;
  const long long blocks = (waves + kProbeThreads / vtx::kWave - 1) / (kProbeThreads / vtx::kWave);
  if (sink_len < blocks * kProbeThreads)
    return vtx::fail(VTX_E_INVALID, "probe_gather: sink needs %lld entries", blocks * kProbeThreads);
  if (blocks == 0) return VTX_OK;
  hipStream_t s = vtx::as_stream(stream);
  if (row_bytes == 256)
    probe_gather_kernel<16, 16, 64><<<(int)blocks, kProbeThreads, 0, s>>>(pool, pool_rows, rows, n_rows, indptr,
                                                                           segments, sink, magic);
  else
    probe_gather_kernel<72, 8, 16><<<(int)blocks, kProbeThreads, 0, s>>>(pool, pool_rows, rows, n_rows, indptr,
                                                                          segments, sink, magic);
  return vtx::check_launch("probe_gather");
}
