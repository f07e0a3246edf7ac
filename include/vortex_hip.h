/*
 * vortex_hip.h — C ABI of the MI355X (gfx950) sparse-attention indexer + cache
 * hot path.
 *
 * Every entry point takes plain device pointers, element counts and a
 * hipStream_t (passed as void*), launches asynchronously on that stream, never
 * synchronises, never reads device memory from the host and never allocates.
 * All of them are therefore safe to record into a HIP graph.
 *
 * Return value: 0 on success, a negative VTX_E_* code otherwise; the message
 * of the last failure on the calling thread is available from
 * vtx_last_error().
 *
 * Element types: "bf16" buffers hold raw bfloat16 bit patterns (uint16_t);
 * index / indptr / workload buffers are int32; loc and req_indices are int64.
 * All buffers are caller-owned and dense (row-major, no strides).
 *
 * Length arguments ("*_len", "*_rows", "*_capacity") are the number of
 * elements (rows) the caller allocated.  Kernels never touch memory beyond
 * them: an index that would leave a buffer is skipped instead of followed.
 */
#ifndef VORTEX_HIP_H
#define VORTEX_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VTX_OK 0
#define VTX_E_INVALID (-1)   /* bad argument (shape, size, alignment, enum) */
#define VTX_E_LAUNCH (-2)    /* the HIP runtime refused the launch */
#define VTX_E_DEVICE (-3)    /* device query failed */

/* Message describing the last failure on this thread ("" if none). */
const char* vtx_last_error(void);

/* Library version string. */
const char* vtx_version(void);

/*
 * *id = 0 if `stream` is not being captured into a graph, otherwise a value
 * that identifies the capture in progress (the same for every stream taking
 * part in it, different for every capture).  Host-side query, no launch.
 * No counterpart in the reference: the Python layer uses it to keep work it
 * records for a later launch (the page-finish mean a flow's forward_cache
 * leaves for the next forward_indexer) inside the capture it was recorded in.
 */
int vtx_stream_capture_id(void* stream, unsigned long long* id);

/*
 * Decode planner: builds the per-step dense/sparse block tables and the GeMV
 * workload list for all sparse layers.
 *
 * Replaces sglang_plan_decode (reference csrc/utils_sglang.cu:313-460, kernels
 * :123-309), bound in Python at vortex_torch/indexer/utils_sglang.py:15-44.
 *
 * Segment s = b*num_kv_heads + h.  n_b = ceil(cached_seq_lens[b]/page_size),
 * budget = topk_val + page_reserved_bos + page_reserved_eos.
 *   dense_kv_indptr[s]   = H*sum_{b'<b} n_b' + h*n_b      (B*H+1 entries)
 *   sparse_kv_indptr[s]  = same with min(budget, n_b)
 *   dense_kv_indices[dense_kv_indptr[s]+j] =
 *        (req_to_token[req_indices[b]*req_to_token_stride + j*P] / P)*H + h
 *   sparse_kv_indices: all pages if n_b <= budget, else the BOS pages at the
 *        front and the EOS pages at the back of the segment (middle left for
 *        top-k).
 *   kv_last_page_len[s]  = L_b % P, or P when that is 0.
 *   winfo_*: chunks of max_chunk_size pages over the middle pages of every
 *        segment whose int16(n_b - bos - eos) exceeds topk_val.
 *
 * req_to_token_stride is the row length of req_to_token (elements); it also
 * bounds the pages one request can have (ceil(stride / page_size)).
 * Unlike the reference there is no limit on batch_size (reference: 1024 for
 * the indptr scan, 8192 segments for the workload list).
 *
 * fused_schedule (optional, NULL for none; no counterpart in the reference):
 * int32 [fused_schedule_len >= 4 + 4 * batch_size * num_kv_heads], the
 * workgroup order of vtx_indexer_fused's one-workgroup-per-segment layout:
 * segments sorted by page count and dealt in snake order over rounds of
 * schedule_round workgroups (the device's compute-unit count), so that each
 * compute unit gets a long and a short segment.  Pass it to the indexer
 * launches of the same step; it changes their speed, never their results.
 */
int vtx_plan_decode(const int32_t* cached_seq_lens, int32_t batch_size,
                    int32_t* dense_kv_indptr, int32_t* dense_kv_indices,
                    int64_t dense_kv_indices_len, int32_t* sparse_kv_indptr,
                    int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                    int32_t* kv_last_page_len, const int32_t* req_to_token,
                    int64_t req_to_token_rows, int64_t req_to_token_stride,
                    const int64_t* req_indices, int32_t* winfo_q_indices,
                    int32_t* winfo_kv_offsets, int32_t* winfo_kv_lens,
                    int64_t winfo_capacity, int32_t* winfo_num_workloads,
                    int32_t* winfo_chunk_size, int32_t page_size,
                    int32_t num_kv_heads, int32_t topk_val,
                    int32_t page_reserved_bos, int32_t page_reserved_eos,
                    int32_t max_chunk_size, int32_t min_chunk_size,
                    int32_t* fused_schedule, int64_t fused_schedule_len,
                    int32_t schedule_round, void* stream);

/*
 * FA3 variant of the decode planner: the block tables, indptrs and workload
 * list of vtx_plan_decode (kv_last_page_len is not an output), plus, for
 * every segment s = b*H + h < page_table_rows:
 *   dense_page_table[s * page_table_stride + j]  = dense index of page j
 *   sparse_page_table[s * page_table_stride + i] = sparse_kv_indices entry i
 *        for the entries the planner writes (all pages when n_b <= budget,
 *        else the BOS and EOS slots; the top-k slots are left untouched)
 * (entries past page_table_stride are not written), and for s < cache_seqlens_len:
 *   dense_cache_seqlens[s]  = cached_seq_lens[b]
 *   sparse_cache_seqlens[s] = min((budget - 1) * page_size + last_page_len,
 *                                 cached_seq_lens[b])
 * Replaces sglang_plan_decode_fa3 (reference csrc/utils_sglang.cu:1085-1239,
 * kernels 950-1082), bound at vortex_torch/indexer/utils_sglang.py:135-168.
 * One launch; no limit on batch_size (reference: 1024 requests, 8192 segments).
 */
int vtx_plan_decode_fa3(const int32_t* cached_seq_lens, int32_t batch_size,
                        int32_t* dense_kv_indptr, int32_t* dense_kv_indices,
                        int64_t dense_kv_indices_len, int32_t* sparse_kv_indptr,
                        int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                        int32_t* dense_page_table, int32_t* dense_cache_seqlens,
                        int32_t* sparse_page_table, int32_t* sparse_cache_seqlens,
                        int64_t page_table_rows, int64_t page_table_stride,
                        int64_t cache_seqlens_len, const int32_t* req_to_token,
                        int64_t req_to_token_rows, int64_t req_to_token_stride,
                        const int64_t* req_indices, int32_t* winfo_q_indices,
                        int32_t* winfo_kv_offsets, int32_t* winfo_kv_lens,
                        int64_t winfo_capacity, int32_t* winfo_num_workloads,
                        int32_t* winfo_chunk_size, int32_t page_size, int32_t num_kv_heads,
                        int32_t topk_val, int32_t page_reserved_bos,
                        int32_t page_reserved_eos, int32_t max_chunk_size,
                        int32_t min_chunk_size, void* stream);

/*
 * Paged GeMV scorer: for every workload w < *winfo_num_workloads and every
 * t < winfo_kv_lens[w], with p = winfo_kv_offsets[w] + t:
 *     o[p] = bf16( sum_d float(x[winfo_q_indices[w], d]) *
 *                        float(y[dense_kv_indices[p], d]) )
 * accumulated in fp32, rounded to nearest-even.  Positions not covered by a
 * workload are not written.
 *
 * Replaces the Triton mv_bpr kernel (reference
 * vortex_torch/indexer/triton_kernels/mv_impl.py:6-81) behind
 * GeMV.execute (vortex_torch/indexer/matmul.py:153-189).
 *
 * x: bf16 [x_rows, head_dim]; y: bf16 [y_rows, head_dim]; o: bf16 [o_len].
 * max_chunk_size is the planner's chunk length (sizes the work split).
 */
int vtx_gemv_paged(const uint16_t* x, int64_t x_rows, const uint16_t* y,
                   int64_t y_rows, uint16_t* o, int64_t o_len,
                   const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                   const int32_t* winfo_q_indices,
                   const int32_t* winfo_kv_offsets,
                   const int32_t* winfo_kv_lens, int64_t winfo_capacity,
                   const int32_t* winfo_num_workloads, int32_t head_dim,
                   int32_t max_chunk_size, void* stream);

/*
 * Segmented top-k page select with reserved BOS/EOS pages.
 * For each segment s < eff_batch_size:
 *   start = dense_kv_indptr[s] + bos, end = dense_kv_indptr[s+1] - eos,
 *   n = end - start; nothing is written when n <= topk_val.
 *   Otherwise the topk_val positions with the largest bf16 score (ties: the
 *   lower position first; -0.0 == +0.0) are written, best first, as
 *   sparse_kv_indices[sparse_kv_indptr[s] + bos + i] = dense_kv_indices[start + pos_i].
 *
 * Replaces topk_output / TopKOutput_BF16_Kernel (reference csrc/topk.cu:56-203),
 * bound at vortex_torch/indexer/output_func.py:223-234 (argument order of
 * csrc/topk.cu:117-128).  max_num_pages (pages per request) only sizes the
 * launch; the reference's 4096-page cap is lifted.  topk_val <= 4096.
 */
int vtx_topk_select(const uint16_t* score, int64_t score_len,
                    const int32_t* dense_kv_indptr,
                    const int32_t* sparse_kv_indptr,
                    const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                    int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                    int32_t eff_batch_size, int32_t topk_val,
                    int32_t reserved_bos, int32_t reserved_eos,
                    int32_t max_num_pages, void* stream);

/* Work layouts of vtx_indexer_fused. */
#define VTX_FUSED_AUTO 0     /* the library chooses */
#define VTX_FUSED_SEGMENT 1  /* one workgroup per segment */
#define VTX_FUSED_SPLIT 2    /* a segment's pages over several workgroups */

/*
 * Fused indexer step of one sparse layer: query head-group mean, GeMV over
 * every segment's middle pages, top-k select — one launch.  No single
 * counterpart in the reference: it is the composition of
 * `q.mean(dim=1, keepdim=True)` (vortex_torch/flow/algorithms.py:168), GeMV
 * (mv_bpr, indexer/triton_kernels/mv_impl.py:6-81) over the planner's
 * workload list and topK (csrc/topk.cu:56-203), for a block table built by
 * the decode planner.  Writes x_out[s] = bf16(fp32 sum_g q[s, g, :] * (1/G))
 * for every s < q_rows when x_out is not NULL, and per segment
 * s < eff_batch_size (q_rows >= eff_batch_size):
 *   score[p]   = bf16(fp32 q_mean[s] . y[dense_kv_indices[p]]) for p in
 *                [indptr[s]+bos, indptr[s+1]-eos) when that range holds more
 *                than topk_val pages
 *   sparse_kv_indices[sparse_kv_indptr[s] + bos + i] = i-th best of them.
 * With group_size == 0 the query rows are taken from x [S, D] instead.
 * q: bf16 [q_rows, group_size, head_dim]; y: bf16 [y_rows, head_dim].
 *
 * seg_counters (optional, int32, seg_counters_len entries) is the split
 * layout's workspace: it lets the library split long segments over several
 * workgroups.  Its first entries are per-segment arrival counters, all zero
 * before the first call: the last workgroup of a segment to finish selects
 * its top-k and sets the segment's counter back to zero.  A workspace of
 * vtx_indexer_fused_workspace_len(S) entries serves every call with up to
 * S segments: it also holds, at its end, the staging zone in which each
 * workgroup of a segment split over at most 16 of them pre-selects its
 * chunk's best k (k <= 64), so that the last one only merges the lists; the
 * zone, like the counters (the entries before it), is all zero before the
 * first call, and every call that completes leaves it all zero.
 * A shorter buffer (at least eff_batch_size entries) holds counters only.
 * Calls that share one workspace must be ordered on one stream.  mode: VTX_FUSED_AUTO
 * (split when there are fewer than two segments per compute unit and the
 * counters are given), VTX_FUSED_SEGMENT or VTX_FUSED_SPLIT.  Outputs are
 * identical in every mode.
 *
 * schedule (optional, NULL for none): the fused_schedule vtx_plan_decode
 * wrote for this block table.  The segment layout then takes its segments
 * in that order; each workgroup checks the bounds the schedule holds against
 * the indptrs, so a schedule from an earlier plan only costs time.
 */
int vtx_indexer_fused(const uint16_t* q, int64_t q_rows, int32_t group_size,
                      const uint16_t* x, uint16_t* x_out, const uint16_t* y,
                      int64_t y_rows, uint16_t* score, int64_t score_len,
                      const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr,
                      const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                      int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                      int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos,
                      int32_t reserved_eos, int32_t max_num_pages, int32_t head_dim,
                      int32_t* seg_counters, int64_t seg_counters_len, int32_t mode,
                      const int32_t* schedule, int64_t schedule_len, void* stream);

/*
 * Entries (int32) of a vtx_indexer_fused workspace that serves calls with up
 * to `segments` segments, staged pre-selection included; -1 for a negative
 * count.  Allocate it zeroed once and pass it to every call.
 */
int64_t vtx_indexer_fused_workspace_len(int32_t segments);

/*
 * vtx_indexer_fused without the seg_counters workspace: the split layout's
 * workspace (65,536 arrival counters and the staging zone, 4.25 MiB per
 * device, held until the process ends) is a device array of the library, so
 * the call allocates nothing and takes no workspace.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under graph
 * capture, tight serving loops, harnesses that forbid allocation).  The
 * first call on a device looks the array up and clears it (a fill kernel on
 * `stream`, waited for unless the stream is being captured).  At
 * most 65,536 segments (eff_batch_size), else VTX_E_INVALID.  Every call on
 * a device shares the array: calls that overlap on one device (other
 * streams, other threads) race and must be serialized by the caller.  A
 * launch that fails (VTX_E_LAUNCH) has the array cleared again before the
 * next call; after a launch that was issued but did not complete (an aborted
 * stream), call vtx_indexer_fused_noalloc_reset.
 */
int vtx_indexer_fused_noalloc(const uint16_t* q, int64_t q_rows, int32_t group_size,
                              const uint16_t* x, uint16_t* x_out, const uint16_t* y,
                              int64_t y_rows, uint16_t* score, int64_t score_len,
                              const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr,
                              const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                              int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                              int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos,
                              int32_t reserved_eos, int32_t max_num_pages, int32_t head_dim,
                              int32_t mode, const int32_t* schedule, int64_t schedule_len, void* stream);

/*
 * Clears the workspace of vtx_indexer_fused_noalloc (arrival counters and
 * staging zone) on the current device (a fill kernel on `stream`, waited for
 * unless the stream is being captured).  Allocates nothing.  No counterpart in the reference.
 */
int vtx_indexer_fused_noalloc_reset(void* stream);

/* 1 if vtx_indexer_fused handles this head_dim (64, 128, 256, 512, 576). */
int vtx_indexer_fused_supported(int32_t head_dim);

/*
 * vtx_indexer_fused preceded by the layer's page-finish mean into y: the
 * results of vtx_page_reduce(k_cache, k_rows, page_size, head_dim, y, BF16,
 * y_rows, loc, nnz, num_kv_heads, page_size, 1, VTX_REDUCE_MEAN) followed by
 * vtx_indexer_fused with the same arguments, bit for bit (y is written).  No
 * single counterpart in the reference: it is CMean
 * (cache/triton_kernels/reduce_impl.py:7-89, the cache step of
 * block_sparse_attention, vortex_torch/flow/algorithms.py:20-235) and the
 * layer's indexer step in one launch.  For head_dim 64 / 128, nnz <= 256 and
 * the one-workgroup-per-segment layout the mean's tiles are spread over the
 * launch's own waves, and a scored page whose centroid it rewrites is scored
 * against the fresh centroid; otherwise it is its own launch, first.
 * k_cache: bf16 [k_rows, page_size, head_dim] with row = page * H + h.
 */
int vtx_indexer_fused_cmean(const uint16_t* q, int64_t q_rows, int32_t group_size,
                            const uint16_t* x, uint16_t* x_out, uint16_t* y, int64_t y_rows,
                            uint16_t* score, int64_t score_len,
                            const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr,
                            const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                            int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                            int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos,
                            int32_t reserved_eos, int32_t max_num_pages, int32_t head_dim,
                            int32_t* seg_counters, int64_t seg_counters_len, int32_t mode,
                            const uint16_t* k_cache, int64_t k_rows, int32_t page_size,
                            int32_t num_kv_heads, const int64_t* loc, int64_t nnz,
                            const int32_t* schedule, int64_t schedule_len, void* stream);

/*
 * Fused indexer step of the GQA flow: GeMM of the group_size query heads
 * with every middle page's centroid, optional segment softmax per query
 * head, maximum over the query heads, top-k select — one launch, one
 * workgroup per segment.  No single counterpart in the reference: it is the
 * composition of GeMM (mm_bpr, indexer/triton_kernels/matmul_impl.py:6-113),
 * Softmax (softmax_inplace_r, indexer/triton_kernels/softmax_impl.py:6-112),
 * Max(dim=2) (reduce_rr, indexer/triton_kernels/reduce_impl.py:8-146) and
 * topK (csrc/topk.cu:56-203) as gqa_block_sparse_attention chains them
 * (vortex_torch/flow/algorithms.py:238-352), for a block table built by the
 * decode planner.  For each segment s < eff_batch_size whose middle range
 * [indptr[s]+bos, indptr[s+1]-eos) holds more than topk_val pages, at each
 * of its pages p:
 *   score[p*G + g] = bf16(q[s*G + g] . y[dense_kv_indices[p]])     (GeMM)
 *   score[p*G + g] = bf16(softmax_p(score * scale)) if softmax != 0
 *   aggr[p]        = max_g score[p*G + g]
 *   sparse_kv_indices[sparse_kv_indptr[s] + bos + i] = i-th best page by aggr
 * bit for bit what vtx_ragged_gemm, vtx_segment_scan, vtx_ragged_reduce and
 * vtx_topk_select write for the same inputs.  q: bf16 [q_rows, head_dim]
 * (q_rows >= eff_batch_size * group_size); y: bf16 [y_rows, head_dim];
 * score_rows = pages of score ([score_rows, 1, group_size]); aggr_len =
 * pages of aggr.  group_size 1..8; topk_val <= 4096.
 *
 * schedule (optional, NULL for none): the fused_schedule vtx_plan_decode
 * wrote for this block table, as for vtx_indexer_fused: the workgroups take
 * the segments in its order and check the bounds it holds against the
 * indptrs, so a schedule from an earlier plan only costs time.
 */
int vtx_indexer_gqa_fused(const uint16_t* q, int64_t q_rows, int32_t group_size,
                          const uint16_t* y, int64_t y_rows, int32_t head_dim,
                          uint16_t* score, int64_t score_rows, uint16_t* aggr, int64_t aggr_len,
                          const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr,
                          const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                          int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                          int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos,
                          int32_t reserved_eos, int32_t max_num_pages, int32_t softmax,
                          float scale, const int32_t* schedule, int64_t schedule_len,
                          void* stream);

/*
 * vtx_indexer_gqa_fused preceded by the layer's page-finish mean into y: the
 * results of vtx_page_reduce(k_cache, k_rows, page_size, head_dim, y, BF16,
 * y_rows, loc, nnz, num_kv_heads, page_size, 1, VTX_REDUCE_MEAN) followed by
 * vtx_indexer_gqa_fused with the same arguments, bit for bit (y is written).
 * No single counterpart in the reference: CMean (the cache step of
 * gqa_block_sparse_attention, vortex_torch/flow/algorithms.py:238-352) and
 * the layer's GQA indexer step in one launch, for head_dim 64 / 128 and
 * nnz <= 256 (otherwise the mean is its own launch, first).
 */
int vtx_indexer_gqa_fused_cmean(const uint16_t* q, int64_t q_rows, int32_t group_size,
                                uint16_t* y, int64_t y_rows, int32_t head_dim,
                                uint16_t* score, int64_t score_rows, uint16_t* aggr, int64_t aggr_len,
                                const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr,
                                const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                                int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                                int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos,
                                int32_t reserved_eos, int32_t max_num_pages, int32_t softmax,
                                float scale, const uint16_t* k_cache, int64_t k_rows,
                                int32_t page_size, int32_t num_kv_heads, const int64_t* loc,
                                int64_t nnz, const int32_t* schedule, int64_t schedule_len,
                                void* stream);

/* 1 if vtx_indexer_gqa_fused handles this head_dim and group size. */
int vtx_indexer_gqa_fused_supported(int32_t head_dim, int32_t group_size);

/*
 * Fused indexer step of the Quest flow: envelope scores of every middle page
 * for the group_size query heads, maximum over the query heads, top-k select
 * — one launch, one workgroup per segment.  No single counterpart in the
 * reference: it is the composition of Multiply twice and Maximum
 * (elementwise_binary_bpr / _rrr, indexer/triton_kernels/elementwise_binary_impl.py),
 * Sum(dim=2) and Max(dim=1) (reduce_rr, indexer/triton_kernels/reduce_impl.py:8-146)
 * and topK (csrc/topk.cu:56-203) as gqa_quest_sparse_attention chains them
 * (vortex_torch/flow/algorithms.py:356-496), for a block table built by the
 * decode planner.  For each segment s < eff_batch_size whose middle range
 * holds more than topk_val pages, at each of its pages p (e = dense[p]):
 *   sum[p*G + g] = bf16(sum_d max(bf16(q[s*G+g, d] * ymax[e, d]),
 *                                 bf16(q[s*G+g, d] * ymin[e, d])))
 *   aggr[p]      = max_g sum[p*G + g]
 *   sparse_kv_indices[sparse_kv_indptr[s] + bos + i] = i-th best page by aggr
 * bit for bit what vtx_ragged_binary, vtx_ragged_reduce and vtx_topk_select
 * write for the same inputs; the [pages, G, D] products are not written.
 * q: bf16 [q_rows, head_dim] (q_rows >= eff_batch_size * group_size);
 * ymax, ymin: bf16 [y_rows, head_dim]; sum_rows = pages of sum
 * ([sum_rows, group_size, 1]); group_size 1..8; topk_val <= 4096.
 * schedule (optional, NULL for none): the planner's fused_schedule, as for
 * vtx_indexer_gqa_fused.
 */
int vtx_indexer_quest_fused(const uint16_t* q, int64_t q_rows, int32_t group_size,
                            const uint16_t* ymax, const uint16_t* ymin, int64_t y_rows,
                            int32_t head_dim, uint16_t* sum, int64_t sum_rows,
                            uint16_t* aggr, int64_t aggr_len,
                            const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr,
                            const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                            int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                            int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos,
                            int32_t reserved_eos, int32_t max_num_pages,
                            const int32_t* schedule, int64_t schedule_len, void* stream);

/*
 * vtx_indexer_quest_fused preceded by the layer's CMax + CMin into ymax and
 * ymin: the results of vtx_page_reduce_multi(k_cache, k_rows, page_size,
 * head_dim, 2, {ymax, ymin}, {BF16, BF16}, {VTX_REDUCE_MAX, VTX_REDUCE_MIN},
 * y_rows, loc, nnz, num_kv_heads, page_size, 1) followed by
 * vtx_indexer_quest_fused with the same arguments, bit for bit (ymax and
 * ymin are written).  No single counterpart in the reference: the cache
 * step of gqa_quest_sparse_attention (vortex_torch/flow/algorithms.py:356-496)
 * and its indexer step in one launch, for head_dim 64 / 128 and nnz <= 256
 * (otherwise the page reduce is its own launch, first).
 */
int vtx_indexer_quest_fused_cmean(const uint16_t* q, int64_t q_rows, int32_t group_size,
                                  uint16_t* ymax, uint16_t* ymin, int64_t y_rows, int32_t head_dim,
                                  uint16_t* sum, int64_t sum_rows, uint16_t* aggr, int64_t aggr_len,
                                  const int32_t* dense_kv_indptr, const int32_t* sparse_kv_indptr,
                                  const int32_t* dense_kv_indices, int64_t dense_kv_indices_len,
                                  int32_t* sparse_kv_indices, int64_t sparse_kv_indices_len,
                                  int32_t eff_batch_size, int32_t topk_val, int32_t reserved_bos,
                                  int32_t reserved_eos, int32_t max_num_pages, const uint16_t* k_cache,
                                  int64_t k_rows, int32_t page_size, int32_t num_kv_heads,
                                  const int64_t* loc, int64_t nnz, const int32_t* schedule,
                                  int64_t schedule_len, void* stream);

/* 1 if vtx_indexer_quest_fused handles this head_dim and group size. */
int vtx_indexer_quest_fused_supported(int32_t head_dim, int32_t group_size);

/* Reduction kinds (values of the reference's ReduceType, vortex_torch/utils.py:11-16). */
#define VTX_REDUCE_MEAN 0
#define VTX_REDUCE_MAX 1
#define VTX_REDUCE_MIN 2
#define VTX_REDUCE_L2NORM 3
#define VTX_REDUCE_SUM 4

/* Output element types. */
#define VTX_DTYPE_BF16 0
#define VTX_DTYPE_F32 1

/*
 * Page-finish reduction (CMean / CMax / CMin / CL2Norm).
 * x: bf16 pool [x_rows, rows_per_tile, cols]; row = (loc/page_size)*H + h.
 * For every i < nnz with (loc[i]+1) % page_size == 0 and every h < H:
 *   dim == 1: out[row, 0, :] = reduce over the rows_per_tile axis
 *   dim == 2: out[row, :, 0] = reduce over the cols axis
 * Mean = fp32 sum / count, L2Norm = sqrt(fp32 sum of squares); the result
 * is rounded to bf16 (also when out is fp32, as the reference stores a bf16
 * value into the output).  Rows not triggered are untouched.
 *
 * Replaces reduce_pp / reduce_pp_kernel (reference
 * vortex_torch/cache/triton_kernels/reduce_impl.py:7-89) behind
 * Reduce.execute (vortex_torch/cache/reduce.py:299-350).
 */
int vtx_page_reduce(const uint16_t* x, int64_t x_rows, int32_t rows_per_tile,
                    int32_t cols, void* out, int32_t out_dtype, int64_t out_rows,
                    const int64_t* loc, int64_t nnz, int32_t num_kv_heads,
                    int32_t page_size, int32_t dim, int32_t reduce_type,
                    void* stream);

/*
 * Fused page-finish reduction: one pass over each finished K tile producing
 * up to four reductions at once (e.g. CMean and CMax), each into its own
 * output.  Same semantics per output as vtx_page_reduce.  No counterpart in
 * the reference, which runs one kernel (one full read of K) per reduction.
 */
int vtx_page_reduce_multi(const uint16_t* x, int64_t x_rows,
                          int32_t rows_per_tile, int32_t cols, int32_t n_out,
                          void* const* outs, const int32_t* out_dtypes,
                          const int32_t* reduce_types, int64_t out_rows,
                          const int64_t* loc, int64_t nnz, int32_t num_kv_heads,
                          int32_t page_size, int32_t dim, void* stream);

/* ------------------------------------------------------------------------
 * Workload-walking indexer ops (GeMM, elementwise, reductions, segment
 * softmax / normalize): the ops of the GQA and Quest flows.
 *
 * Each visits exactly the packed positions of the planner's workload list:
 * workload w < min(*winfo_num_workloads, winfo_capacity) covers
 * winfo_kv_lens[w] positions from winfo_kv_offsets[w], of segment
 * winfo_q_indices[w].  An operand's row at position p is, by row mode,
 *   VTX_ROWS_BATCHED: winfo_q_indices[w]   (query rows [S, d0, d1])
 *   VTX_ROWS_PAGED:   dense_kv_indices[p]  (a cache pool [rows, d0, d1])
 *   VTX_ROWS_RAGGED:  p                    (a per-position buffer)
 * and the output row is p.  Operands and outputs are bf16 tiles [d0, d1]
 * per row; positions outside the workloads are not written; a row outside
 * its operand's `rows` is skipped.  Compute is fp32, results rounded to bf16.
 * ---------------------------------------------------------------------- */
#define VTX_ROWS_BATCHED 0
#define VTX_ROWS_PAGED 1
#define VTX_ROWS_RAGGED 2

/* Values of the reference's ElementwiseBinaryOpType (vortex_torch/utils.py:19-23). */
#define VTX_BINARY_MAXIMUM 0
#define VTX_BINARY_MINIMUM 1
#define VTX_BINARY_ADD 2
#define VTX_BINARY_MUL 3

/* Values of the reference's ElementwiseOpType (vortex_torch/utils.py:26-31). */
#define VTX_UNARY_RELU 0
#define VTX_UNARY_SIGMOID 1
#define VTX_UNARY_SILU 2
#define VTX_UNARY_ABS 3
#define VTX_UNARY_ADD_MUL 4

/*
 * o[p, c, g] = bf16(fp32 sum_k x[rx, g, k] * y[ry, c, k]); o is
 * [o_rows, y_d0, x_d0], K = k (a multiple of 8).  x: BATCHED or RAGGED;
 * y: PAGED or RAGGED.
 * Replaces mm_bpr / mm_rrr / mm_rpr (reference
 * vortex_torch/indexer/triton_kernels/matmul_impl.py:6-113, 127-391) behind
 * GeMM (vortex_torch/indexer/matmul.py:193-398).
 */
int vtx_ragged_gemm(const uint16_t* x, int64_t x_rows, int32_t x_mode, int32_t x_d0,
                    const uint16_t* y, int64_t y_rows, int32_t y_mode, int32_t y_d0, int32_t k,
                    uint16_t* o, int64_t o_rows, const int32_t* dense_kv_indices,
                    int64_t dense_kv_indices_len, const int32_t* winfo_q_indices,
                    const int32_t* winfo_kv_offsets, const int32_t* winfo_kv_lens,
                    int64_t winfo_capacity, const int32_t* winfo_num_workloads, void* stream);

/*
 * o[p, i, j] = op(x[rx, i, j], y[ry, i, j]) with size-1 operand axes
 * broadcast to the output tile [o_d0, o_d1].  MAXIMUM / MINIMUM compare the
 * values, MUL rounds the product, ADD rounds bf16(alpha)*x and bf16(beta)*y
 * to bf16 and then their sum.  x: BATCHED or RAGGED; y: PAGED or RAGGED.
 * Replaces elementwise_binary_{bpr,rrr,rpr} (reference
 * vortex_torch/indexer/triton_kernels/elementwise_binary_impl.py:7-510)
 * behind Maximum / Minimum / Add / Multiply
 * (vortex_torch/indexer/elementwise_binary.py:8-326).
 */
int vtx_ragged_binary(int32_t op, float alpha, float beta, const uint16_t* x, int64_t x_rows,
                      int32_t x_mode, int32_t x_d0, int32_t x_d1, const uint16_t* y, int64_t y_rows,
                      int32_t y_mode, int32_t y_d0, int32_t y_d1, uint16_t* o, int64_t o_rows,
                      int32_t o_d0, int32_t o_d1, const int32_t* dense_kv_indices,
                      int64_t dense_kv_indices_len, const int32_t* winfo_q_indices,
                      const int32_t* winfo_kv_offsets, const int32_t* winfo_kv_lens,
                      int64_t winfo_capacity, const int32_t* winfo_num_workloads, void* stream);

/*
 * o[p] = op(x[p]) elementwise on RAGGED rows, tile [d0, d1], with
 * a = bf16(alpha), b = bf16(beta), z = bf16(bf16(b*x) + a):
 * RELU x >= a ? x : b; SIGMOID 1/(1+exp(z)); SILU x/(1+exp(z)); ABS |z|;
 * ADD_MUL z.
 * Replaces elementwise_rr (reference
 * vortex_torch/indexer/triton_kernels/elementwise_impl.py:7-171) behind
 * Relu / Sigmoid / Silu / Abs / Add_Mul (vortex_torch/indexer/elementwise.py).
 */
int vtx_ragged_unary(int32_t op, float alpha, float beta, const uint16_t* x, int64_t x_rows,
                     int32_t d0, int32_t d1, uint16_t* o, int64_t o_rows,
                     const int32_t* winfo_kv_offsets, const int32_t* winfo_kv_lens,
                     int64_t winfo_capacity, const int32_t* winfo_num_workloads, void* stream);

/*
 * o[p] = reduction of the RAGGED tile x[p] ([d0, d1]) over axis dim (1: d0,
 * o is [o_rows, 1, d1]; 2: d1, o is [o_rows, d0, 1]): MEAN (sum / count),
 * MAX, MIN, L2NORM (sqrt of the sum of squares) or SUM, in fp32.
 * Replaces reduce_rr (reference
 * vortex_torch/indexer/triton_kernels/reduce_impl.py:8-146) behind
 * Max / Mean / Min / L2Norm / Sum (vortex_torch/indexer/reduce.py:8-438).
 */
int vtx_ragged_reduce(const uint16_t* x, int64_t x_rows, int32_t d0, int32_t d1, uint16_t* o,
                      int64_t o_rows, int32_t dim, int32_t reduce_type,
                      const int32_t* winfo_kv_offsets, const int32_t* winfo_kv_lens,
                      int64_t winfo_capacity, const int32_t* winfo_num_workloads, void* stream);

#define VTX_SEGMENT_SOFTMAX 0
#define VTX_SEGMENT_NORMALIZE 1

/*
 * In place, for every segment s < eff_batch_size whose page count
 * n = dense_kv_indptr[s+1] - dense_kv_indptr[s] exceeds
 * reserved_bos + reserved_eos + topk_val, over its middle positions
 * [indptr[s] + bos, indptr[s+1] - eos) and each of the `cols` values of a
 * position's tile, independently per column:
 *   SOFTMAX:   x = bf16(exp(v - max v) / sum exp(v - max v)), v = x * scale
 *   NORMALIZE: x = bf16(x / max(sqrt(sum x^2), 1e-12))
 * Replaces softmax_inplace_r / normalize_inplace_r (reference
 * vortex_torch/indexer/triton_kernels/softmax_impl.py:6-130,
 * normalize_impl.py:6-118) behind Softmax / Normalize
 * (vortex_torch/indexer/scan.py:8-388).
 */
int vtx_segment_scan(int32_t op, float scale, uint16_t* x, int64_t x_rows, int32_t cols,
                     const int32_t* dense_kv_indptr, int32_t eff_batch_size, int32_t topk_val,
                     int32_t reserved_bos, int32_t reserved_eos, void* stream);

/*
 * Self-check of the device's bf16 rounding; no counterpart in the reference.
 * Every kernel rounds fp32 to bf16 with gfx950's conversion instruction; this
 * compares it, over all 2^32 fp32 bit patterns, with the integer
 * round-to-nearest-even formulation the oracle uses, and adds to the device
 * counters counts[0] the non-NaN inputs (conversion to bits, and rounding
 * back to fp32, checked separately) whose result differs, and to counts[1]
 * the NaN inputs whose bits are not 0x7fc0 or whose fp32 rounding is not a
 * NaN.  Both stay 0 on a conforming device.  Takes a few milliseconds.
 */
int vtx_bf16_rounding_check(unsigned long long* counts, void* stream);

/*
 * Writes new keys and values into the paged pools: for token i < nnz and
 * kv head h, with pos = loc[i], pool row
 *   (pos / page_size) * (page_size * H) + h * page_size + pos % page_size
 * of k_cache / v_cache ([cache_rows, head_dim] elements of elem_bytes each,
 * i.e. [pages * H, page_size, head_dim]) receives new_k[i, h, :] /
 * new_v[i, h, :] ([nnz, H, head_dim]).  Raw element copy; tokens whose row
 * is outside the pool are skipped.
 * Replaces set_kv_buffer_launcher / set_kv_buffer_kernel (reference
 * vortex_torch/cache/triton_kernels/set_kv.py:5-63).
 */
int vtx_set_kv_buffer(void* k_cache, void* v_cache, int64_t cache_rows, const void* new_k,
                      const void* new_v, const int64_t* loc, int64_t nnz, int32_t num_kv_heads,
                      int32_t head_dim, int32_t elem_bytes, int32_t page_size, void* stream);

/*
 * Paged decode attention over a block table (the consumer of the sparse
 * table the indexer builds; given the dense table it is full attention).
 * Segment s = b * num_kv_heads + h attends to the pages
 * kv_indices[kv_indptr[s] .. kv_indptr[s+1]) of the K / V pools
 * ([cache_rows, page_size, head_dim] bf16; entry = page * H + h), every page
 * full but the last, which holds kv_last_page_len[s] tokens.  Its query heads
 * q[s * group_size + g, :] ([B * H * G, head_dim] bf16) each get
 *   o[s * group_size + g, :] = softmax_t(sm_scale * q . K[t]) @ V
 * in fp32, rounded to bf16; a segment without tokens gets zeros.
 * No counterpart in the reference, which hands this table to FlashInfer's
 * paged decode inside its (un-vendored) SGLang fork; the table format is
 * the one csrc/utils_sglang.cu:123-184 and csrc/topk.cu:56-113 write.
 * head_dim 64, 128 or 256; group_size 1..8.
 */
int vtx_paged_decode_attention(const uint16_t* q, uint16_t* o, const uint16_t* k_cache,
                               const uint16_t* v_cache, int64_t cache_rows, const int32_t* kv_indptr,
                               const int32_t* kv_indices, int64_t kv_indices_len,
                               const int32_t* kv_last_page_len, int32_t batch_size,
                               int32_t num_kv_heads, int32_t group_size, int32_t head_dim,
                               int32_t page_size, float sm_scale, void* stream);

/* 1 if vtx_paged_decode_attention handles this head_dim and group size. */
int vtx_paged_decode_attention_supported(int32_t head_dim, int32_t group_size);

/*
 * Bandwidth probes (measurement only; no counterpart in the reference).
 * vtx_probe_read reads `bytes` of src sequentially (16-byte nontemporal
 * loads, grid-stride over four 512-thread workgroups per compute unit).
 * vtx_probe_gather reads rows rows[0 .. n_rows) of pool ([pool_rows,
 * row_bytes] bytes, row_bytes 256 or 1152) in the indexer's scoring passes
 * (per wave one coalesced load of 64 or 16 row ids, then every row load of
 * the pass in flight); with indptr (segments entries) each workgroup first
 * loads one indptr entry and only then its row ids, the fused kernel's chain
 * of dependent trips.  Neither writes anything unless a lane's fold of the
 * loaded words equals `magic` (sink: one uint32 per thread, at least 2048 per
 * compute unit for the read and one per row id rounded up to 512 for the
 * gather).
 */
int vtx_probe_read(const void* src, int64_t bytes, uint32_t* sink, int64_t sink_len, uint32_t magic,
                   void* stream);
int vtx_probe_gather(const uint16_t* pool, int64_t pool_rows, int32_t row_bytes, const int32_t* rows,
                     int64_t n_rows, const int32_t* indptr, int32_t segments, uint32_t* sink,
                     int64_t sink_len, uint32_t magic, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VORTEX_HIP_H */
