"""Pins the oracle's workload-walking indexer ops (GeMM, elementwise binary
and unary, tile reductions, segment softmax / normalize) before they check
the GPU kernels.

The layouts come from the oracle planner (itself pinned in test_oracle.py).
Every function is checked against a computation written differently:
per-position Python loops for the row addressing, and torch for the
arithmetic (float64 einsum / softmax / normalize / reductions, torch's own
bf16 arithmetic for the elementwise ops, whose products and sums torch
rounds to bf16 one operation at a time).  One test plants a transposed
output in a copy of the GeMM and shows the pin catches it.
"""
import numpy as np
import pytest
import torch

from oracle import vortex_oracle as O


def _layout(seed, B=5, H=2, P=4, topk=3, bos=1, eos=1, chunk=4):
    rng = np.random.default_rng(seed)
    L = rng.integers(1, 80, size=B)
    n = (L + P - 1) // P
    pool = int(n.sum()) + 7
    perm = rng.permutation(pool)
    T = int(n.max()) * P
    r2t = np.zeros((B, T), np.int32)
    off = 0
    for b in range(B):
        for j in range(int(n[b])):
            r2t[b, j * P:(j + 1) * P] = perm[off + j] * P + np.arange(P)
        off += int(n[b])
    plan = O.plan_decode(L.astype(np.int32), r2t, np.arange(B, dtype=np.int64), P, H, topk, bos, eos, chunk)
    plan["pool"] = pool
    plan["H"], plan["B"], plan["topk"], plan["bos"], plan["eos"] = H, B, topk, bos, eos
    return plan


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def _bits(t):
    return t.view(torch.int16).numpy().view(np.uint16)


def _walk(plan):
    """[(p, q)] of every covered position, by explicit loops over workloads."""
    out = []
    for w in range(int(plan["num_workloads"])):
        for t in range(int(plan["winfo_len"][w])):
            out.append((int(plan["winfo_off"][w]) + t, int(plan["winfo_q"][w])))
    return out


def _row(mode, p, q, plan):
    return q if mode == O.ROWS_BATCHED else (int(plan["dense_indices"][p]) if mode == O.ROWS_PAGED else p)


def _w(plan):
    return plan["winfo_q"], plan["winfo_off"], plan["winfo_len"], int(plan["num_workloads"])


def test_workload_positions_match_loops():
    plan = _layout(0)
    p, q = O.workload_positions(*_w(plan))
    assert list(zip(p.tolist(), q.tolist())) == _walk(plan)
    assert len(set(p.tolist())) == p.size  # no position twice


@pytest.mark.parametrize("modes", [(O.ROWS_BATCHED, O.ROWS_PAGED), (O.ROWS_RAGGED, O.ROWS_RAGGED),
                                   (O.ROWS_RAGGED, O.ROWS_PAGED)])
@pytest.mark.parametrize("seed", range(3))
def test_ragged_gemm_against_einsum(modes, seed):
    plan = _layout(seed)
    S, G, C, K = int(plan["dense_indptr"][-1]), 3, 2, 16
    xm, ym = modes
    x = _bf16((plan["B"] * plan["H"] if xm == O.ROWS_BATCHED else S, G, K), seed + 10)
    y = _bf16((plan["pool"] * plan["H"] if ym == O.ROWS_PAGED else S, C, K), seed + 20)
    out0 = np.full((S, C, G), 0x1234, np.uint16)
    got, cov = O.ragged_gemm(_bits(x), xm, _bits(y), ym, out0, plan["dense_indices"], *_w(plan))
    exp = out0.copy()
    for p, q in _walk(plan):
        v = torch.einsum("gk,ck->cg", x[_row(xm, p, q, plan)].double(), y[_row(ym, p, q, plan)].double())
        exp[p] = _bits(v.float().to(torch.bfloat16))
    np.testing.assert_array_equal(got, exp)
    assert cov.sum() == len(_walk(plan))


def test_ragged_gemm_one_hot_rows():
    plan = _layout(4)
    S, K = int(plan["dense_indptr"][-1]), 16
    x = _bf16((plan["B"] * plan["H"], 2, K), 1)
    y = torch.zeros((plan["pool"] * plan["H"], 1, K), dtype=torch.bfloat16)
    y[:, 0, 5] = 1.0  # every page row selects k = 5
    got, cov = O.ragged_gemm(_bits(x), O.ROWS_BATCHED, _bits(y), O.ROWS_PAGED, np.zeros((S, 1, 2), np.uint16),
                             plan["dense_indices"], *_w(plan))
    for p, q in _walk(plan):
        np.testing.assert_array_equal(got[p, 0], _bits(x[q, :, 5].contiguous()))


def test_planted_gemm_transpose_is_caught(monkeypatch):
    plan = _layout(1)
    S = int(plan["dense_indptr"][-1])
    x = _bf16((plan["B"] * plan["H"], 3, 16), 2)
    y = _bf16((plan["pool"] * plan["H"], 2, 16), 3)
    real = np.einsum
    monkeypatch.setattr(O.np, "einsum", lambda spec, *a: real(spec.replace("->pcg", "->pgc"), *a).reshape(
        a[0].shape[0], 2, 3) if "->pcg" in spec else real(spec, *a))
    got, _ = O.ragged_gemm(_bits(x), O.ROWS_BATCHED, _bits(y), O.ROWS_PAGED, np.zeros((S, 2, 3), np.uint16),
                           plan["dense_indices"], *_w(plan))
    p, q = _walk(plan)[0]
    exp = _bits(torch.einsum("gk,ck->cg", x[q].double(), y[int(plan["dense_indices"][p])].double())
                .float().to(torch.bfloat16))
    assert not np.array_equal(got[p], exp), "a transposed GeMM output went unnoticed"


@pytest.mark.parametrize("op", [O.BINARY_MAXIMUM, O.BINARY_MINIMUM, O.BINARY_ADD, O.BINARY_MUL])
@pytest.mark.parametrize("case", ["bpr", "rrr", "rpr_bcast"])
def test_ragged_binary_against_torch_bf16(op, case):
    plan = _layout(2)
    S, H = int(plan["dense_indptr"][-1]), plan["H"]
    if case == "bpr":  # Quest: q [S_q, G, D] times an envelope [pool, 1, D]
        xm, ym, xs, ys = O.ROWS_BATCHED, O.ROWS_PAGED, (plan["B"] * H, 3, 8), (plan["pool"] * H, 1, 8)
    elif case == "rrr":
        xm, ym, xs, ys = O.ROWS_RAGGED, O.ROWS_RAGGED, (S, 3, 8), (S, 3, 8)
    else:
        xm, ym, xs, ys = O.ROWS_RAGGED, O.ROWS_PAGED, (S, 3, 1), (plan["pool"] * H, 1, 8)
    x, y = _bf16(xs, 5), _bf16(ys, 6)
    alpha, beta = 0.7, -1.3
    out0 = np.zeros((S, 3, 8), np.uint16)
    got, _ = O.ragged_binary(op, alpha, beta, _bits(x), xm, _bits(y), ym, out0, plan["dense_indices"], *_w(plan))
    a = torch.tensor(alpha, dtype=torch.bfloat16)
    b = torch.tensor(beta, dtype=torch.bfloat16)
    exp = out0.copy()
    for p, q in _walk(plan):
        xv, yv = x[_row(xm, p, q, plan)], y[_row(ym, p, q, plan)]
        if op == O.BINARY_MAXIMUM:
            v = torch.maximum(xv, yv)
        elif op == O.BINARY_MINIMUM:
            v = torch.minimum(xv, yv)
        elif op == O.BINARY_ADD:
            v = a * xv + b * yv
        else:
            v = xv * yv
        exp[p] = _bits(v.expand(3, 8).contiguous())
    np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("op", [O.UNARY_RELU, O.UNARY_SIGMOID, O.UNARY_SILU, O.UNARY_ABS, O.UNARY_ADD_MUL])
def test_ragged_unary_against_torch(op):
    plan = _layout(3)
    S = int(plan["dense_indptr"][-1])
    x = _bf16((S, 2, 8), 7, scale=3.0)
    alpha, beta = 0.3, -0.8
    got, _ = O.ragged_unary(op, alpha, beta, _bits(x), np.zeros((S, 2, 8), np.uint16), plan["winfo_off"],
                            plan["winfo_len"], int(plan["num_workloads"]))
    a = torch.tensor(alpha, dtype=torch.bfloat16)
    b = torch.tensor(beta, dtype=torch.bfloat16)
    for p, _ in _walk(plan):
        xv = x[p]
        z = b * xv + a  # torch rounds each bf16 operation
        if op == O.UNARY_RELU:
            v = torch.where(xv >= a, xv, b)
        elif op == O.UNARY_SIGMOID:
            v = (1.0 / (1.0 + torch.exp(z.double()))).float().to(torch.bfloat16)
        elif op == O.UNARY_SILU:
            v = (xv.double() / (1.0 + torch.exp(z.double()))).float().to(torch.bfloat16)
        elif op == O.UNARY_ABS:
            v = torch.abs(z)
        else:
            v = z
        np.testing.assert_array_equal(got[p], _bits(v.contiguous()))


@pytest.mark.parametrize("rtype", [O.MEAN, O.MAX, O.MIN, O.L2NORM, O.REDUCE_SUM])
@pytest.mark.parametrize("dim", [1, 2])
def test_ragged_reduce_against_torch(rtype, dim):
    plan = _layout(5)
    S = int(plan["dense_indptr"][-1])
    x = _bf16((S, 3, 16), 8)
    shape = (S, 1, 16) if dim == 1 else (S, 3, 1)
    got, cov = O.ragged_reduce(_bits(x), np.zeros(shape, np.uint16), dim, rtype, plan["winfo_off"],
                               plan["winfo_len"], int(plan["num_workloads"]))
    t = x.double()
    f = {O.MEAN: lambda v: v.mean(dim=dim, keepdim=True), O.MAX: lambda v: v.amax(dim=dim, keepdim=True),
         O.MIN: lambda v: v.amin(dim=dim, keepdim=True), O.L2NORM: lambda v: v.norm(dim=dim, keepdim=True),
         O.REDUCE_SUM: lambda v: v.sum(dim=dim, keepdim=True)}[rtype]
    ref = _bits(f(t).float().to(torch.bfloat16).contiguous())
    covered = [p for p, _ in _walk(plan)]
    np.testing.assert_array_equal(got[covered], ref[covered])
    assert not got[~cov].any()


@pytest.mark.parametrize("op", [O.SEGMENT_SOFTMAX, O.SEGMENT_NORMALIZE])
def test_segment_scan_against_torch(op):
    plan = _layout(6, B=6, topk=4)
    S, E = int(plan["dense_indptr"][-1]), plan["B"] * plan["H"]
    x = _bf16((S, 1, 3), 9, scale=4.0)
    scale = 0.09
    got, touched = O.segment_scan(op, scale, _bits(x), plan["dense_indptr"], E, plan["topk"], plan["bos"],
                                  plan["eos"])
    exp = _bits(x.clone()).copy()
    dip = plan["dense_indptr"]
    n_touched = 0
    for s in range(E):
        n = int(dip[s + 1] - dip[s])
        if n <= plan["bos"] + plan["eos"] + plan["topk"]:
            continue
        a, b = int(dip[s]) + plan["bos"], int(dip[s + 1]) - plan["eos"]
        v = x[a:b].float()
        if op == O.SEGMENT_SOFTMAX:
            r = torch.softmax((v * scale).double(), dim=0)
        else:
            r = torch.nn.functional.normalize(v.double(), dim=0, eps=1e-12)
        exp[a:b] = _bits(r.float().to(torch.bfloat16).contiguous())
        n_touched += b - a
    np.testing.assert_array_equal(got, exp)
    assert touched.sum() == n_touched > 0


def test_segment_softmax_closed_form():
    # a constant column over cnt middle pages: every entry is 1/cnt
    plan = _layout(7, B=3, topk=2)
    S, E = int(plan["dense_indptr"][-1]), plan["B"] * plan["H"]
    x = torch.full((S, 1, 1), 2.5, dtype=torch.bfloat16)
    got, touched = O.segment_scan(O.SEGMENT_SOFTMAX, 1.0, _bits(x), plan["dense_indptr"], E, 2, 1, 1)
    dip = plan["dense_indptr"]
    for s in range(E):
        n = int(dip[s + 1] - dip[s])
        if n > 4:
            a, b = int(dip[s]) + 1, int(dip[s + 1]) - 1
            assert (got[a:b].reshape(-1) == O.f32_to_bf16(np.float32(1.0 / (b - a))).reshape(-1)[0]).all()


def test_set_kv_buffer_against_loops():
    rng = np.random.default_rng(3)
    P, H, D, pages = 4, 3, 5, 6
    k = rng.integers(0, 1000, size=(pages * H, P, D)).astype(np.uint16)
    v = rng.integers(0, 1000, size=(pages * H, P, D)).astype(np.uint16)
    nnz = 9
    nk = rng.integers(0, 1000, size=(nnz, H, D)).astype(np.uint16)
    nv = rng.integers(0, 1000, size=(nnz, H, D)).astype(np.uint16)
    loc = rng.permutation(pages * P)[:nnz].astype(np.int64)
    loc[2] = -5              # skipped
    loc[5] = pages * P + 3   # past the pool: skipped
    gk, gv = O.set_kv_buffer(k, v, nk, nv, loc, P)
    ek, ev = k.copy(), v.copy()
    for i in range(nnz):
        pos = int(loc[i])
        if pos < 0 or pos >= pages * P:
            continue
        for h in range(H):
            ek[(pos // P) * H + h, pos % P] = nk[i, h]   # pool row page*H + h, slot pos % P
            ev[(pos // P) * H + h, pos % P] = nv[i, h]
    np.testing.assert_array_equal(gk, ek)
    np.testing.assert_array_equal(gv, ev)


def _attn_case(seed, P=4, H=2, G=3, D=8, pages=20, B=3):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((pages * H, P, D), generator=g).to(torch.bfloat16)
    v = torch.randn((pages * H, P, D), generator=g).to(torch.bfloat16)
    q = torch.randn((B * H * G, D), generator=g).to(torch.bfloat16)
    rng = np.random.default_rng(seed)
    lens, idx = [], []
    for s in range(B * H):
        m = int(rng.integers(0, 6))
        pg = rng.permutation(pages)[:m]
        idx.extend((pg * H + s % H).tolist())
        lens.append(m)
    ip = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    last = rng.integers(1, P + 1, size=B * H).astype(np.int32)
    return q, k, v, ip, np.asarray(idx, np.int32), last, B, H, G


def test_paged_decode_attention_against_sdpa():
    q, k, v, ip, idx, last, B, H, G = _attn_case(0)
    P, D = k.shape[1], k.shape[2]
    scale = 0.37
    got = O.paged_decode_attention(_bits(q), _bits(k), _bits(v), ip, idx, last, B, H, scale)
    for s in range(B * H):
        pages = idx[ip[s]:ip[s + 1]]
        rows = q[s * G:(s + 1) * G]
        if pages.size == 0:
            assert not got[s * G:(s + 1) * G].any()
            continue
        n = (pages.size - 1) * P + int(last[s])
        kk = k[torch.as_tensor(pages, dtype=torch.long)].reshape(-1, D)[:n].double()
        vv = v[torch.as_tensor(pages, dtype=torch.long)].reshape(-1, D)[:n].double()
        ref = torch.nn.functional.scaled_dot_product_attention(
            rows.double()[None], kk[None], vv[None], scale=float(np.float32(scale)))[0]
        np.testing.assert_array_equal(got[s * G:(s + 1) * G], _bits(ref.float().to(torch.bfloat16)))


def test_paged_decode_attention_closed_forms():
    # one token: the output is its value row; equal keys: the mean of the values
    q, k, v, ip, idx, last, B, H, G = _attn_case(1, P=4)
    P = k.shape[1]
    one_ip = np.arange(B * H + 1, dtype=np.int32)
    one_idx = np.asarray([s % H for s in range(B * H)], np.int32)  # page 0 of each head
    ones = np.ones(B * H, np.int32)
    got = O.paged_decode_attention(_bits(q), _bits(k), _bits(v), one_ip, one_idx, ones, B, H, 1.0)
    for s in range(B * H):
        for gq in range(G):
            np.testing.assert_array_equal(got[s * G + gq], _bits(v[one_idx[s], 0].contiguous()))
    kc = k.clone()
    kc[:] = k[0, 0]
    full = np.full(B * H, P, np.int32)
    got = O.paged_decode_attention(_bits(q), _bits(kc), _bits(v), ip, idx, full, B, H, 1.0)
    for s in range(B * H):
        pages = idx[ip[s]:ip[s + 1]]
        if pages.size:
            mean = v[torch.as_tensor(pages, dtype=torch.long)].reshape(-1, k.shape[2]).double().mean(0)
            np.testing.assert_array_equal(got[s * G], _bits(mean.float().to(torch.bfloat16)))
