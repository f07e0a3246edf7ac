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
                    void* stream);

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
 * seg_counters (optional, int32, at least eff_batch_size entries, all zero
 * before the first call) lets the library split long segments over several
 * workgroups: the last workgroup of a segment to finish selects its top-k
 * and sets the segment's counter back to zero.  Calls that share one
 * counter buffer must be ordered on one stream.  mode: VTX_FUSED_AUTO
 * (split when there are fewer than two segments per compute unit and the
 * counters are given), VTX_FUSED_SEGMENT or VTX_FUSED_SPLIT.  Outputs are
 * identical in every mode.
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
                      void* stream);

/* 1 if vtx_indexer_fused handles this head_dim (64, 128, 256, 512, 576). */
int vtx_indexer_fused_supported(int32_t head_dim);

/* Reduction kinds (values of the reference's ReduceType, vortex_torch/utils.py:11-16). */
#define VTX_REDUCE_MEAN 0
#define VTX_REDUCE_MAX 1
#define VTX_REDUCE_MIN 2
#define VTX_REDUCE_L2NORM 3

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

#ifdef __cplusplus
}
#endif

#endif /* VORTEX_HIP_H */
