"""CPU oracle of the Vortex sparse-attention indexer + cache path.

TEST INFRASTRUCTURE ONLY.  This module is the checker for the gfx950 kernels:
only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it.  The product path (vortex_torch) never calls it and has no CPU
fallback.

Each function restates one reference function in numpy, following the cited
reference file:line.  Conventions:

* bf16 data is carried as its raw bit pattern (``np.uint16``);
* integer division and remainder follow C (truncation toward zero), as the
  reference's CUDA and Triton code do;
* floating-point reductions accumulate in float64 and round once to fp32 and
  then to bf16 (round-to-nearest-even) — the reference GPU code accumulates
  in bf16 (CMean) or rounds every product to bf16 (GeMV); the north-star
  contract compares against fp32 accumulation within rtol 1e-2 / atol 1e-3.

How each function is pinned (tests/test_oracle.py): the planner and top-k by
independent pure-Python restatements on small inputs plus closed-form
invariants; bf16 rounding against torch's own conversion; the reductions and
GeMV against torch.amax/amin/mean/matmul in float64 and closed forms.
"""
from __future__ import annotations

import numpy as np

# --------------------------------------------------------------------------
# bf16 bit helpers
# --------------------------------------------------------------------------


def bf16_to_f32(bits) -> np.ndarray:
    """bf16 bit patterns -> float32 (exact)."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return b.view(np.float32)


def f32_to_bf16(x) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even; every NaN becomes
    the quiet NaN 0x7FC0 (as torch's conversion does)."""
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, 0x7FC0, r)
    return r.astype(np.uint16)


def c_div(a, b):
    """C integer division (truncates toward zero)."""
    a = np.asarray(a, dtype=np.int64)
    q = np.abs(a) // abs(int(b))
    return np.where((a < 0) != (int(b) < 0), -q, q)


def c_mod(a, b):
    """C remainder (sign of the dividend)."""
    a = np.asarray(a, dtype=np.int64)
    return a - c_div(a, b) * int(b)


def _int16(v: int) -> int:
    return ((int(v) + 32768) % 65536) - 32768


# --------------------------------------------------------------------------
# A.1 decode planner — csrc/utils_sglang.cu:123-309 (host 313-460)
# --------------------------------------------------------------------------


def plan_decode(seq_lens, req_to_token, req_indices, page_size: int, num_kv_heads: int,
                topk_val: int, bos: int, eos: int, max_chunk_size: int) -> dict:
    """Returns the block tables and workload list the reference planner writes.

    Keys: dense_indptr, dense_indices, sparse_indptr, sparse_indices,
    sparse_written (bool mask: the planner leaves the top-k slots of long
    segments untouched), kv_last_page_len, winfo_q, winfo_off, winfo_len,
    num_workloads, chunk_size.
    """
    L = np.asarray(seq_lens, dtype=np.int64)
    r2t = np.asarray(req_to_token, dtype=np.int64)
    ridx = np.asarray(req_indices, dtype=np.int64)
    P, H = int(page_size), int(num_kv_heads)
    B = L.shape[0]
    budget = topk_val + bos + eos
    n = c_div(L + P - 1, P)                       # utils_sglang.cu:267
    sn = np.minimum(budget, n)                    # utils_sglang.cu:282

    # indptr: inclusive pair scan, H entries per request (utils_sglang.cu:257-309)
    dense_len = np.repeat(n, H)
    sparse_len = np.repeat(sn, H)
    dense_indptr = np.zeros(B * H + 1, dtype=np.int64)
    sparse_indptr = np.zeros(B * H + 1, dtype=np.int64)
    dense_indptr[1:] = np.cumsum(dense_len)
    sparse_indptr[1:] = np.cumsum(sparse_len)

    total_dense = int(dense_indptr[-1])
    total_sparse = int(sparse_indptr[-1])
    dense = np.zeros(total_dense, dtype=np.int64)
    sparse = np.zeros(total_sparse, dtype=np.int64)
    written = np.zeros(total_sparse, dtype=bool)
    last = np.zeros(B * H, dtype=np.int64)

    # indices (utils_sglang.cu:123-184)
    for b in range(B):
        nb = int(n[b])
        rem = int(c_mod(L[b], P))
        cols = np.arange(nb, dtype=np.int64) * P
        phys = c_div(r2t[ridx[b], cols], P) if nb > 0 else np.zeros(0, dtype=np.int64)
        for h in range(H):
            s = b * H + h
            last[s] = P if rem == 0 else rem
            enc = phys * H + h
            d0 = int(dense_indptr[s])
            dense[d0:d0 + nb] = enc
            s0 = int(sparse_indptr[s])
            if nb <= budget:
                sparse[s0:s0 + nb] = enc
                written[s0:s0 + nb] = True
            else:
                sparse[s0:s0 + bos] = enc[:bos]
                written[s0:s0 + bos] = True
                for e in range(eos):                   # utils_sglang.cu:174-181
                    sparse[s0 + budget - 1 - e] = enc[nb - 1 - e]
                    written[s0 + budget - 1 - e] = True

    # workload list (utils_sglang.cu:188-254): segments in order, chunks of C
    C = int(max_chunk_size)
    wq, wo, wl = [], [], []
    for s in range(B * H):
        w = _int16(int(dense_indptr[s + 1] - dense_indptr[s]) - bos - eos)
        pc = (w & 0xFFFF) if w > topk_val else 0
        nchunks = (pc + C - 1) // C
        tail = pc % C or C
        for k in range(nchunks):
            wq.append(s)
            wl.append(C if k != nchunks - 1 else tail)
            wo.append(int(dense_indptr[s]) + k * C + bos)

    return {
        "dense_indptr": dense_indptr.astype(np.int32),
        "dense_indices": dense.astype(np.int32),
        "sparse_indptr": sparse_indptr.astype(np.int32),
        "sparse_indices": sparse.astype(np.int32),
        "sparse_written": written,
        "kv_last_page_len": last.astype(np.int32),
        "winfo_q": np.asarray(wq, dtype=np.int32),
        "winfo_off": np.asarray(wo, dtype=np.int32),
        "winfo_len": np.asarray(wl, dtype=np.int32),
        "num_workloads": len(wq),
        "chunk_size": C,
    }


# --------------------------------------------------------------------------
# A.2 page-finish reduction — cache/triton_kernels/reduce_impl.py:7-62
# --------------------------------------------------------------------------

MEAN, MAX, MIN, L2NORM = 0, 1, 2, 3


def page_reduce(x_bits, out, loc, num_kv_heads: int, page_size: int, dim: int, reduce_type: int):
    """Returns (new_out, written_rows).

    x_bits: uint16 [rows, R, C] (bf16 bits).  out: uint16 bf16 bits or float32
    array [rows, 1, C] (dim 1) / [rows, R, 1] (dim 2).  The value stored is the
    bf16-rounded reduction (widened for a float32 out), as the reference
    stores its bf16 result into the output.
    """
    x = bf16_to_f32(x_bits).astype(np.float64)
    loc = np.asarray(loc, dtype=np.int64)
    P, H = int(page_size), int(num_kv_heads)
    out = np.array(out, copy=True)
    rows_out = out.shape[0]
    trig = c_mod(loc + 1, P) == 0                     # reduce_impl.py:24
    pages = c_div(loc[trig], P)                        # reduce_impl.py:26
    rows = (pages[:, None] * H + np.arange(H)[None, :]).reshape(-1)
    rows = rows[(rows >= 0) & (rows < x.shape[0]) & (rows < rows_out)]
    rows = np.unique(rows)
    axis = 1 if dim == 1 else 2
    if rows.size:
        t = x[rows]
        if reduce_type == MEAN:
            v = t.sum(axis=axis) / t.shape[axis]
        elif reduce_type == MAX:
            v = t.max(axis=axis)
        elif reduce_type == MIN:
            v = t.min(axis=axis)
        elif reduce_type == L2NORM:
            v = np.sqrt((t * t).sum(axis=axis))
        else:
            raise ValueError(f"unknown reduce type {reduce_type}")
        bits = f32_to_bf16(v.astype(np.float32))
        if dim == 1:
            bits = bits[:, None, :]
        else:
            bits = bits[:, :, None]
        if out.dtype == np.uint16:
            out[rows] = bits
        else:
            out[rows] = bf16_to_f32(bits)
    return out, rows


# --------------------------------------------------------------------------
# A.3 GeMV — indexer/triton_kernels/mv_impl.py:6-81
# --------------------------------------------------------------------------


def gemv(x_bits, y_bits, dense_indices, winfo_q, winfo_off, winfo_len, num_workloads: int,
         out_len: int):
    """Returns (scores as bf16 bits [out_len], covered mask [out_len])."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    y = bf16_to_f32(y_bits).astype(np.float64)
    D = x.shape[-1]
    x = x.reshape(-1, D)
    y = y.reshape(-1, D)
    dense = np.asarray(dense_indices, dtype=np.int64)
    scores = np.zeros(out_len, dtype=np.uint16)
    covered = np.zeros(out_len, dtype=bool)
    nw = int(num_workloads)
    if nw == 0:
        return scores, covered
    lens = np.asarray(winfo_len[:nw], dtype=np.int64)
    offs = np.asarray(winfo_off[:nw], dtype=np.int64)
    qs = np.asarray(winfo_q[:nw], dtype=np.int64)
    # every covered position p with the query row of its workload
    first = np.repeat(np.cumsum(lens) - lens, lens)
    p = np.repeat(offs, lens) + (np.arange(int(lens.sum())) - first)
    q = np.repeat(qs, lens)
    v = np.einsum("ij,ij->i", y[dense[p]], x[q])
    scores[p] = f32_to_bf16(v.astype(np.float32))
    covered[p] = True
    return scores, covered


# --------------------------------------------------------------------------
# A.4 topK — csrc/topk.cu:56-113 (host 117-203)
# --------------------------------------------------------------------------


def topk(score_bits, dense_indptr, sparse_indptr, dense_indices, sparse_indices,
         eff_batch_size: int, topk_val: int, bos: int, eos: int):
    """Returns (new_sparse_indices, written mask).

    Per segment: stable descending sort of the middle scores (ties keep the
    lower position first; -0.0 == +0.0), first topk_val dense indices written
    after the BOS slots.  Segments with n <= topk_val are untouched.
    """
    sc = bf16_to_f32(score_bits).astype(np.float64)
    dip = np.asarray(dense_indptr, dtype=np.int64)
    sip = np.asarray(sparse_indptr, dtype=np.int64)
    didx = np.asarray(dense_indices)
    out = np.array(sparse_indices, copy=True)
    written = np.zeros(out.shape[0], dtype=bool)
    for s in range(int(eff_batch_size)):
        start = dip[s] + bos
        end = dip[s + 1] - eos
        n = end - start
        if n <= topk_val or topk_val <= 0:
            continue
        keys = sc[start:end] + 0.0            # folds -0.0 into +0.0
        order = np.argsort(-keys, kind="stable")[:topk_val]
        o0 = sip[s] + bos
        out[o0:o0 + topk_val] = didx[start + order]
        written[o0:o0 + topk_val] = True
    return out, written


# --------------------------------------------------------------------------
# helper: the indexer pipeline of block_sparse_attention
# (flow/algorithms.py:114-170)
# --------------------------------------------------------------------------


def q_group_mean(q_bits) -> np.ndarray:
    """[S, G, D] bf16 bits -> [S, 1, D] bf16 bits (fp32-accurate mean)."""
    q = bf16_to_f32(q_bits).astype(np.float64)
    return f32_to_bf16(q.mean(axis=1, keepdims=True).astype(np.float32))


# --------------------------------------------------------------------------
# A.5 workload-walking indexer ops of the GQA and Quest flows
#     GeMM       indexer/triton_kernels/matmul_impl.py:6-113 (bpr), 127-391 (rrr, rpr)
#     binary     indexer/triton_kernels/elementwise_binary_impl.py:7-510
#     unary      indexer/triton_kernels/elementwise_impl.py:7-171
#     reduce     indexer/triton_kernels/reduce_impl.py:8-146
#     softmax    indexer/triton_kernels/softmax_impl.py:6-130
#     normalize  indexer/triton_kernels/normalize_impl.py:6-118
# Row modes (the reference's FORMAT pairs): 0 BATCHED -> the workload's
# segment, 1 PAGED -> dense_indices[p], 2 RAGGED -> p.
# --------------------------------------------------------------------------

ROWS_BATCHED, ROWS_PAGED, ROWS_RAGGED = 0, 1, 2


def workload_positions(winfo_q, winfo_off, winfo_len, num_workloads: int):
    """(p, q) of every position the workload list covers, in workload order."""
    nw = int(num_workloads)
    lens = np.asarray(winfo_len[:nw], dtype=np.int64)
    offs = np.asarray(winfo_off[:nw], dtype=np.int64)
    qs = np.asarray(winfo_q[:nw], dtype=np.int64) if winfo_q is not None else np.zeros(nw, np.int64)
    first = np.repeat(np.cumsum(lens) - lens, lens)
    p = np.repeat(offs, lens) + (np.arange(int(lens.sum())) - first)
    return p, np.repeat(qs, lens)


def _rows_of(mode: int, p, q, dense_indices):
    if mode == ROWS_BATCHED:
        return q
    if mode == ROWS_PAGED:
        return np.asarray(dense_indices, dtype=np.int64)[p]
    return p


def _tile3(bits):
    a = np.asarray(bits)
    return a if a.ndim == 3 else a.reshape(a.shape[0], 1, -1)


def ragged_gemm(x_bits, x_mode: int, y_bits, y_mode: int, out_bits, dense_indices, winfo_q, winfo_off,
                winfo_len, num_workloads: int):
    """o[p, c, g] = sum_k x[rx, g, k] * y[ry, c, k] (float64, rounded once to
    fp32 then bf16) at every covered position; returns (out bits, covered)."""
    x = bf16_to_f32(_tile3(x_bits)).astype(np.float64)
    y = bf16_to_f32(_tile3(y_bits)).astype(np.float64)
    out = np.array(_tile3(out_bits), copy=True)
    covered = np.zeros(out.shape[0], dtype=bool)
    p, q = workload_positions(winfo_q, winfo_off, winfo_len, num_workloads)
    if p.size == 0:
        return out, covered
    v = np.einsum("pgk,pck->pcg", x[_rows_of(x_mode, p, q, dense_indices)], y[_rows_of(y_mode, p, q, dense_indices)])
    out[p] = f32_to_bf16(v.astype(np.float32)).reshape(out[p].shape)
    covered[p] = True
    return out, covered


def _bf16_round(v):
    return bf16_to_f32(f32_to_bf16(np.asarray(v, dtype=np.float32))).astype(np.float64)


BINARY_MAXIMUM, BINARY_MINIMUM, BINARY_ADD, BINARY_MUL = 0, 1, 2, 3


def ragged_binary(op: int, alpha: float, beta: float, x_bits, x_mode: int, y_bits, y_mode: int, out_bits,
                  dense_indices, winfo_q, winfo_off, winfo_len, num_workloads: int):
    """o[p] = op(x[rx], y[ry]) with size-1 tile axes broadcast; bf16
    arithmetic: max/min of the values, mul = bf16(x*y), add = bf16(bf16(a*x)
    + bf16(b*y)) with a, b = bf16(alpha), bf16(beta).  Returns (out, covered)."""
    x = bf16_to_f32(_tile3(x_bits)).astype(np.float64)
    y = bf16_to_f32(_tile3(y_bits)).astype(np.float64)
    out = np.array(_tile3(out_bits), copy=True)
    covered = np.zeros(out.shape[0], dtype=bool)
    p, q = workload_positions(winfo_q, winfo_off, winfo_len, num_workloads)
    if p.size == 0:
        return out, covered
    xs = x[_rows_of(x_mode, p, q, dense_indices)]
    ys = y[_rows_of(y_mode, p, q, dense_indices)]
    if op == BINARY_MAXIMUM:
        v = np.maximum(xs, ys)
    elif op == BINARY_MINIMUM:
        v = np.minimum(xs, ys)
    elif op == BINARY_ADD:
        a, b = _bf16_round(alpha), _bf16_round(beta)
        v = _bf16_round(a * xs) + _bf16_round(b * ys)
    else:
        v = xs * ys
    out[p] = f32_to_bf16(np.broadcast_to(v, (p.size,) + out.shape[1:]).astype(np.float32))
    covered[p] = True
    return out, covered


UNARY_RELU, UNARY_SIGMOID, UNARY_SILU, UNARY_ABS, UNARY_ADD_MUL = 0, 1, 2, 3, 4


def ragged_unary(op: int, alpha: float, beta: float, x_bits, out_bits, winfo_off, winfo_len, num_workloads: int):
    """Elementwise op on RAGGED rows with a = bf16(alpha), b = bf16(beta),
    z = bf16(bf16(b*x) + a): relu x >= a ? x : b; sigmoid 1/(1+exp(z)); silu
    x/(1+exp(z)); abs |z|; add_mul z.  Returns (out, covered)."""
    x = bf16_to_f32(_tile3(x_bits)).astype(np.float64)
    out = np.array(_tile3(out_bits), copy=True)
    covered = np.zeros(out.shape[0], dtype=bool)
    p, _ = workload_positions(None, winfo_off, winfo_len, num_workloads)
    if p.size == 0:
        return out, covered
    xs = x[p]
    a, b = _bf16_round(alpha), _bf16_round(beta)
    z = _bf16_round(_bf16_round(b * xs) + a)
    with np.errstate(over="ignore"):
        if op == UNARY_RELU:
            v = np.where(xs >= a, xs, b)
        elif op == UNARY_SIGMOID:
            v = 1.0 / (1.0 + np.exp(z))
        elif op == UNARY_SILU:
            v = xs / (1.0 + np.exp(z))
        elif op == UNARY_ABS:
            v = np.abs(z)
        else:
            v = z
    out[p] = f32_to_bf16(v.astype(np.float32))
    covered[p] = True
    return out, covered


REDUCE_SUM = 4


def ragged_reduce(x_bits, out_bits, dim: int, reduce_type: int, winfo_off, winfo_len, num_workloads: int):
    """o[p] = reduction of the tile x[p] over axis dim (1 -> [1, D1], 2 ->
    [D0, 1]): mean, max, min, L2 = sqrt(sum x^2), sum (float64, rounded once).
    Returns (out, covered)."""
    x = bf16_to_f32(_tile3(x_bits)).astype(np.float64)
    out = np.array(out_bits, copy=True)
    covered = np.zeros(out.shape[0], dtype=bool)
    p, _ = workload_positions(None, winfo_off, winfo_len, num_workloads)
    if p.size == 0:
        return out, covered
    t = x[p]
    ax = 1 if dim == 1 else 2
    if reduce_type == MEAN:
        v = t.mean(axis=ax, keepdims=True)
    elif reduce_type == MAX:
        v = t.max(axis=ax, keepdims=True)
    elif reduce_type == MIN:
        v = t.min(axis=ax, keepdims=True)
    elif reduce_type == L2NORM:
        v = np.sqrt((t * t).sum(axis=ax, keepdims=True))
    else:
        v = t.sum(axis=ax, keepdims=True)
    out[p] = f32_to_bf16(v.astype(np.float32)).reshape(out[p].shape)
    covered[p] = True
    return out, covered


SEGMENT_SOFTMAX, SEGMENT_NORMALIZE = 0, 1


def segment_scan(op: int, scale: float, x_bits, dense_indptr, eff_batch_size: int, topk_val: int, bos: int,
                 eos: int):
    """In place (on a copy) per segment with n > bos + eos + topk_val pages,
    over the middle positions and per tile column: softmax of
    fp32(x) * fp32(scale), or x / max(||x||_2, 1e-12).  Returns (out, touched)."""
    out = np.array(x_bits, copy=True)
    flat = out.reshape(out.shape[0], -1)
    touched = np.zeros(out.shape[0], dtype=bool)
    dip = np.asarray(dense_indptr, dtype=np.int64)
    for s in range(int(eff_batch_size)):
        n = dip[s + 1] - dip[s]
        if n <= bos + eos + topk_val:
            continue
        a, b = dip[s] + bos, dip[s + 1] - eos
        v = bf16_to_f32(flat[a:b]).astype(np.float64)
        if op == SEGMENT_SOFTMAX:
            u = (bf16_to_f32(flat[a:b]) * np.float32(scale)).astype(np.float64)
            e = np.exp(u - u.max(axis=0, keepdims=True))
            r = e / e.sum(axis=0, keepdims=True)
        else:
            r = v / np.maximum(np.sqrt((v * v).sum(axis=0, keepdims=True)), 1e-12)
        flat[a:b] = f32_to_bf16(r.astype(np.float32))
        touched[a:b] = True
    return out, touched


# --------------------------------------------------------------------------
# A.6 set_kv_buffer — cache/triton_kernels/set_kv.py:5-63
# --------------------------------------------------------------------------


def set_kv_buffer(k_cache, v_cache, new_k, new_v, loc, page_size: int):
    """Returns copies of the pools with token i / head h written at pool row
    (loc // P) * (P * H) + h * P + loc % P (C division), rows outside the
    pool skipped.  Pools [rows, P, D] are viewed as [rows * P, D]."""
    k = np.array(k_cache, copy=True)
    v = np.array(v_cache, copy=True)
    kf = k.reshape(-1, k.shape[-1])
    vf = v.reshape(-1, v.shape[-1])
    nk = np.asarray(new_k)
    nv = np.asarray(new_v)
    nnz, H = nk.shape[0], nk.shape[1]
    pos = np.asarray(loc, dtype=np.int64)[:nnz]
    for h in range(H):
        dst = c_div(pos, page_size) * (page_size * H) + h * page_size + c_mod(pos, page_size)
        ok = (pos >= 0) & (dst < kf.shape[0])
        kf[dst[ok]] = nk[ok, h]
        vf[dst[ok]] = nv[ok, h]
    return k, v


# --------------------------------------------------------------------------
# A.7 FA3 decode planner — csrc/utils_sglang.cu:950-1082 (host 1085-1239)
# --------------------------------------------------------------------------


def plan_decode_fa3(seq_lens, req_to_token, req_indices, page_size: int, num_kv_heads: int, topk_val: int,
                    bos: int, eos: int, max_chunk_size: int, page_table_stride: int) -> dict:
    """plan_decode's block tables and workload list (the FA3 planner writes no
    kv_last_page_len) plus, per segment s = b*H + h:
      dense_page_table[s, j]  = dense index of page j (j < stride)
      sparse_page_table[s, i] = sparse entry i where the planner writes it
                                (masks *_pt_written say which entries)
      dense_cache_seqlens[s]  = L_b
      sparse_cache_seqlens[s] = min((budget - 1) * P + last_page_len, L_b)
    (utils_sglang.cu:966-977 for the lengths, 1041-1078 for the tables)."""
    r = plan_decode(seq_lens, req_to_token, req_indices, page_size, num_kv_heads, topk_val, bos, eos,
                    max_chunk_size)
    L = np.asarray(seq_lens, dtype=np.int64)
    H, P, W = int(num_kv_heads), int(page_size), int(page_table_stride)
    S = L.shape[0] * H
    budget = topk_val + bos + eos
    dip, sip = r["dense_indptr"].astype(np.int64), r["sparse_indptr"].astype(np.int64)
    dpt = np.zeros((S, W), np.int32)
    spt = np.zeros((S, W), np.int32)
    dpt_w = np.zeros((S, W), bool)
    spt_w = np.zeros((S, W), bool)
    for s in range(S):
        k = min(int(dip[s + 1] - dip[s]), W)
        dpt[s, :k] = r["dense_indices"][dip[s]:dip[s] + k]
        dpt_w[s, :k] = True
        m = min(int(sip[s + 1] - sip[s]), W)
        w = r["sparse_written"][sip[s]:sip[s] + m]
        spt[s, :m][w] = r["sparse_indices"][sip[s]:sip[s] + m][w]
        spt_w[s, :m] = w
    last = r["kv_last_page_len"].astype(np.int64)
    dcs = np.repeat(L, H)
    scs = np.minimum((budget - 1) * P + last, dcs)
    r.update({"dense_page_table": dpt, "sparse_page_table": spt, "dense_pt_written": dpt_w,
              "sparse_pt_written": spt_w, "dense_cache_seqlens": dcs.astype(np.int32),
              "sparse_cache_seqlens": scs.astype(np.int32)})
    return r


# --------------------------------------------------------------------------
# A.8 paged decode attention over a block table (the consumer of the sparse
#     table: FlashInfer's paged decode in the reference's SGLang fork; table
#     format csrc/utils_sglang.cu:123-184, csrc/topk.cu:56-113)
# --------------------------------------------------------------------------


def paged_decode_attention(q_bits, k_bits, v_bits, kv_indptr, kv_indices, kv_last_page_len, batch_size: int,
                           num_kv_heads: int, sm_scale: float):
    """q [B*H*G, D], pools [rows, P, D] (bf16 bits) -> o bits [B*H*G, D]:
    softmax(sm_scale * q K^T) V in float64 over each segment's tokens (every
    page full but the last, which holds kv_last_page_len[s] tokens)."""
    k = bf16_to_f32(k_bits).astype(np.float64)
    v = bf16_to_f32(v_bits).astype(np.float64)
    P, D = k.shape[1], k.shape[2]
    S = int(batch_size) * int(num_kv_heads)
    q = bf16_to_f32(np.asarray(q_bits).reshape(-1, D)).astype(np.float64)
    G = q.shape[0] // max(S, 1)
    out = np.zeros((q.shape[0], D), dtype=np.float64)
    ip = np.asarray(kv_indptr, dtype=np.int64)
    idx = np.asarray(kv_indices, dtype=np.int64)
    last = np.asarray(kv_last_page_len, dtype=np.int64)
    for s in range(S):
        pages = idx[ip[s]:ip[s + 1]]
        if pages.size == 0:
            continue
        kk = k[pages].reshape(-1, D)[:(pages.size - 1) * P + int(last[s])]
        vv = v[pages].reshape(-1, D)[:(pages.size - 1) * P + int(last[s])]
        if kk.shape[0] == 0:
            continue
        sc = q[s * G:(s + 1) * G] @ kk.T * float(np.float32(sm_scale))
        w = np.exp(sc - sc.max(axis=1, keepdims=True))
        out[s * G:(s + 1) * G] = (w / w.sum(axis=1, keepdims=True)) @ vv
    return f32_to_bf16(out.astype(np.float32))
