"""Writes tests/golden/c1_golden.npz: config-1 inputs and the oracle's outputs.

The reference publishes no test vectors and its kernels need CUDA, so these
fixtures come from the CPU oracle (itself pinned in tests/test_oracle.py).
They freeze the C1 inputs and expected outputs so that the GPU kernels and
any later change of the oracle are compared against the same bits:

* planner outputs for C1 (1 request x 4096 tokens, 512-page pool, H_kv 8);
* a seeded bf16 score vector and the top-30 (+1 BOS +1 EOS) selection;
* CMean / CMax of 3 closed pages (all 8 heads) of a seeded K tile set;
* GeMV scores of a seeded head-group-mean query against seeded centroids
  (segments 0 and 1; the other centroid rows are zero).

Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "tests"), os.path.join(ROOT, "vortex_torch-dev_amd"), ROOT]

import workloads as W  # noqa: E402
from oracle import vortex_oracle as O  # noqa: E402


def build():
    b = W.c1()
    H, G, D, P = b.num_kv_heads, b.group_size, b.head_dim, b.page_size
    plan = O.plan_decode(b.seq_lens.numpy(), b.req_to_token.numpy(), b.req_indices.numpy(), P, H, b.topk, b.bos,
                         b.eos, b.max_chunk)
    rng = np.random.default_rng(2024)
    n = int(plan["dense_indptr"][-1])
    scores = O.f32_to_bf16((rng.standard_normal(n) * 2).astype(np.float32))
    sel, _ = O.topk(scores, plan["dense_indptr"], plan["sparse_indptr"], plan["dense_indices"],
                    plan["sparse_indices"], b.batch * H, b.topk, b.bos, b.eos)
    # page-finish reduction on a compact pool of 4 pages (3 of them closed)
    k_tiles = O.f32_to_bf16(rng.standard_normal((4 * H, P, D)).astype(np.float32))
    loc = np.array([0 * P + 15, 2 * P + 15, 3 * P + 7, 1 * P + 15], dtype=np.int64)
    cmean, _ = O.page_reduce(k_tiles, np.zeros((4 * H, 1, D), np.uint16), loc, H, P, 1, O.MEAN)
    cmax, _ = O.page_reduce(k_tiles, np.zeros((4 * H, 1, D), np.uint16), loc, H, P, 1, O.MAX)
    # GeMV through the C1 block table; only the centroid rows of segments 0
    # and 1 are stored (the rest of the pool is zero)
    q = O.f32_to_bf16(rng.standard_normal((b.batch * H, G, D)).astype(np.float32))
    qm = O.q_group_mean(q)
    cen = np.zeros((b.pool_pages * H, 1, D), np.uint16)
    kept = np.unique(plan["dense_indices"][:plan["dense_indptr"][2]])
    cen[kept] = O.f32_to_bf16((rng.standard_normal((kept.size, 1, D)) * 0.25).astype(np.float32))
    gemv, cov = O.gemv(qm, cen, plan["dense_indices"], plan["winfo_q"], plan["winfo_off"], plan["winfo_len"],
                       plan["num_workloads"], n)
    cov[plan["dense_indptr"][2]:] = False
    return dict(
        seq_lens=b.seq_lens.numpy(), req_to_token=b.req_to_token.numpy(), req_indices=b.req_indices.numpy(),
        dense_indptr=plan["dense_indptr"], dense_indices=plan["dense_indices"],
        sparse_indptr=plan["sparse_indptr"], sparse_indices_plan=plan["sparse_indices"],
        sparse_written=plan["sparse_written"], kv_last_page_len=plan["kv_last_page_len"],
        winfo_q=plan["winfo_q"], winfo_off=plan["winfo_off"], winfo_len=plan["winfo_len"],
        scores=scores, sparse_indices_topk=sel,
        k_tiles=k_tiles, loc=loc, cmean=cmean, cmax=cmax,
        q=q, q_mean=qm, centroid_rows=kept, centroids=cen[kept], gemv=gemv, gemv_covered=cov,
    )


if __name__ == "__main__":
    out = os.path.join(HERE, "c1_golden.npz")
    np.savez_compressed(out, **build())
    print(out, os.path.getsize(out), "bytes")
