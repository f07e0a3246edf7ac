"""Config-1 golden vectors (tests/golden/c1_golden.npz, written by
tests/golden/make_golden.py): the oracle must keep reproducing them (CPU),
and the gfx950 kernels must reproduce them through the C ABI (GPU; bit-exact
for the block tables, the selection and CMax, rtol 1e-2 / atol 1e-3 for
CMean and GeMV)."""
import os

import numpy as np
import pytest
import torch

import workloads as W
from oracle import vortex_oracle as O

G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "c1_golden.npz"))
H, P, D, TOPK, BOS, EOS, CHUNK = 8, 16, 128, 30, 1, 1, 64


def test_fixture_inputs_match_generator():
    b = W.c1()
    np.testing.assert_array_equal(b.seq_lens.numpy(), G["seq_lens"])
    np.testing.assert_array_equal(b.req_to_token.numpy(), G["req_to_token"])
    np.testing.assert_array_equal(b.req_indices.numpy(), G["req_indices"])


def test_oracle_reproduces_fixture():
    plan = O.plan_decode(G["seq_lens"], G["req_to_token"], G["req_indices"], P, H, TOPK, BOS, EOS, CHUNK)
    for k in ("dense_indptr", "dense_indices", "sparse_indptr", "kv_last_page_len"):
        np.testing.assert_array_equal(plan[k], G[k])
    np.testing.assert_array_equal(plan["sparse_written"], G["sparse_written"])
    np.testing.assert_array_equal(plan["winfo_q"], G["winfo_q"])
    np.testing.assert_array_equal(plan["winfo_off"], G["winfo_off"])
    np.testing.assert_array_equal(plan["winfo_len"], G["winfo_len"])
    sel, _ = O.topk(G["scores"], plan["dense_indptr"], plan["sparse_indptr"], plan["dense_indices"],
                    G["sparse_indices_plan"], 8, TOPK, BOS, EOS)
    np.testing.assert_array_equal(sel, G["sparse_indices_topk"])
    n_rows = G["k_tiles"].shape[0]
    cm, _ = O.page_reduce(G["k_tiles"], np.zeros((n_rows, 1, D), np.uint16), G["loc"], H, P, 1, O.MEAN)
    np.testing.assert_array_equal(cm, G["cmean"])
    np.testing.assert_array_equal(O.q_group_mean(G["q"]), G["q_mean"])


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if a.dtype == np.uint16:
        t = t.view(torch.int16).view(torch.bfloat16)
    return t.to(dev) if dtype is None else t.to(dev, dtype)


@pytest.mark.gpu
def test_kernels_reproduce_fixture(gpu):
    from vortex_torch import _hip

    dev = gpu
    i32 = dict(dtype=torch.int32, device=dev)
    nd, ns = G["dense_indices"].size, G["sparse_written"].size
    dptr, sptr = torch.zeros(9, **i32), torch.zeros(9, **i32)
    dense, sparse = torch.zeros(nd, **i32), torch.full((ns,), -1, **i32)
    last = torch.zeros(8, **i32)
    wq, wo, wl = (torch.full((200,), -1, **i32) for _ in range(3))
    nw, cs = torch.zeros(1, **i32), torch.zeros(1, **i32)
    _hip.plan_decode(_t(G["seq_lens"], dev), dptr, dense, sptr, sparse, last, _t(G["req_to_token"], dev),
                     _t(G["req_indices"], dev), wq, wo, wl, nw, cs, P, H, TOPK, BOS, EOS, CHUNK, 16)
    np.testing.assert_array_equal(dptr.cpu().numpy(), G["dense_indptr"])
    np.testing.assert_array_equal(dense.cpu().numpy(), G["dense_indices"])
    np.testing.assert_array_equal(last.cpu().numpy(), G["kv_last_page_len"])
    w = G["sparse_written"]
    np.testing.assert_array_equal(sparse.cpu().numpy()[w], G["sparse_indices_plan"][w])
    k = int(nw.item())
    assert k == G["winfo_q"].size
    np.testing.assert_array_equal(wo.cpu().numpy()[:k], G["winfo_off"])
    # top-k on the fixture's scores
    _hip.topk_select(_t(G["scores"], dev), dptr, sptr, dense, sparse, 8, TOPK, BOS, EOS, 256)
    np.testing.assert_array_equal(sparse.cpu().numpy(), G["sparse_indices_topk"])
    # CMean / CMax
    kt = _t(G["k_tiles"], dev)
    rows = kt.shape[0]
    cm = torch.zeros((rows, 1, D), dtype=torch.bfloat16, device=dev)
    cx = torch.zeros_like(cm)
    loc = _t(G["loc"], dev)
    _hip.page_reduce(kt, cm, loc, H, P, 1, _hip.REDUCE_MEAN)
    _hip.page_reduce(kt, cx, loc, H, P, 1, _hip.REDUCE_MAX)
    np.testing.assert_array_equal(cx.view(torch.int16).cpu().numpy().view(np.uint16), G["cmax"])
    np.testing.assert_allclose(O.bf16_to_f32(cm.view(torch.int16).cpu().numpy().view(np.uint16)),
                               O.bf16_to_f32(G["cmean"]), rtol=1e-2, atol=1e-3)
    # q-mean + GeMV (fused kernel and separate kernels)
    cen = torch.zeros((512 * H, 1, D), dtype=torch.bfloat16, device=dev)
    cen[torch.from_numpy(G["centroid_rows"]).to(dev)] = _t(G["centroids"], dev)
    q = _t(G["q"], dev)
    qm = q.mean(dim=1, keepdim=True)
    np.testing.assert_array_equal(qm.view(torch.int16).cpu().numpy().view(np.uint16), G["q_mean"])
    sc = torch.zeros((nd, 1, 1), dtype=torch.bfloat16, device=dev)
    _hip.gemv_paged(qm, cen, sc, dense, wq, wo, wl, nw, CHUNK)
    cov = G["gemv_covered"]
    got = O.bf16_to_f32(sc.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1))
    np.testing.assert_allclose(got[cov], O.bf16_to_f32(G["gemv"])[cov], rtol=1e-2, atol=1e-3)
    for mode in (_hip.FUSED_SEGMENT, _hip.FUSED_SPLIT):
        sc2 = torch.zeros_like(sc)
        qm2 = torch.empty_like(qm)
        sp2 = torch.full_like(sparse, -1)
        counters = torch.zeros(8, dtype=torch.int32, device=dev)
        _hip.indexer_fused(q, qm2, cen, sc2, dptr, sptr, dense, sp2, 8, TOPK, BOS, EOS, 256,
                           seg_counters=counters, mode=mode)
        assert torch.equal(qm2, qm)
        got2 = O.bf16_to_f32(sc2.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1))
        np.testing.assert_allclose(got2[cov], O.bf16_to_f32(G["gemv"])[cov], rtol=1e-2, atol=1e-3)
        # its selection is the top-k kernel's selection on its own scores
        sp3 = torch.full_like(sparse, -1)
        _hip.topk_select(sc2, dptr, sptr, dense, sp3, 8, TOPK, BOS, EOS, 256)
        assert torch.equal(sp2, sp3)
        assert int(counters.abs().sum()) == 0
