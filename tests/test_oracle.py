"""Pins the CPU oracle (oracle/vortex_oracle.py) before it is trusted as the
GPU kernels' checker.

Each function is checked against something other than a retyping of its own
formula: an independent pure-Python restatement on small inputs (planner,
top-k), a library routine (torch's bf16 conversion, amax/amin/mean/norm,
matmul), closed forms and invariants.  Two tests plant a mistake in a copy of
the oracle and show the corresponding check catches it.
"""
import math

import numpy as np
import pytest
import torch

import workloads as W
from oracle import vortex_oracle as O


# ----------------------------------------------------------------- helpers
def _py_trunc_div(a, b):
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b > 0) else -q


def brute_plan(seq_lens, r2t, ridx, P, H, topk, bos, eos, C):
    """Straight-line restatement of the reference planner
    (csrc/utils_sglang.cu:123-309), one request / head / page at a time."""
    budget = topk + bos + eos
    B = len(seq_lens)
    n = [_py_trunc_div(int(L) + P - 1, P) for L in seq_lens]
    dptr, sptr = [0], [0]
    for b in range(B):
        for h in range(H):
            dptr.append(dptr[-1] + n[b])
            sptr.append(sptr[-1] + min(budget, n[b]))
    dense = [None] * dptr[-1]
    sparse = [None] * sptr[-1]
    last = []
    for b in range(B):
        for h in range(H):
            s = b * H + h
            rem = int(seq_lens[b]) - _py_trunc_div(int(seq_lens[b]), P) * P
            last.append(P if rem == 0 else rem)
            for j in range(n[b]):
                tok = int(r2t[int(ridx[b])][j * P])
                dense[dptr[s] + j] = _py_trunc_div(tok, P) * H + h
            if n[b] <= budget:
                for j in range(n[b]):
                    sparse[sptr[s] + j] = dense[dptr[s] + j]
            else:
                for j in range(bos):
                    sparse[sptr[s] + j] = dense[dptr[s] + j]
                for e in range(eos):
                    sparse[sptr[s] + budget - 1 - e] = dense[dptr[s] + n[b] - 1 - e]
    wq, wo, wl = [], [], []
    for s in range(B * H):
        m = dptr[s + 1] - dptr[s] - bos - eos
        w16 = m & 0xFFFF
        if w16 >= 0x8000:
            w16 -= 0x10000
        pc = w16 if w16 > topk else 0
        chunks = (pc + C - 1) // C
        for k in range(chunks):
            wq.append(s)
            wo.append(dptr[s] + k * C + bos)
            wl.append(C if k < chunks - 1 else (pc % C or C))
    return dptr, dense, sptr, sparse, last, wq, wo, wl


def brute_topk_segment(vals, k):
    """Indices of the k best values, best first, ties to the lower index."""
    return sorted(range(len(vals)), key=lambda i: (-vals[i], i))[:k]


# ----------------------------------------------------------------- bf16
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 3,
        (rng.standard_normal(5000) * 1e-38).astype(np.float32),  # subnormals
        np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 3.0e38, -3.0e38, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8],
                 dtype=np.float32),
    ])
    # values exactly halfway between two bf16 numbers (ties to even); finite
    # only: NaN is outside the contract (and torch's own CPU paths disagree on it)
    base = rng.integers(0, 0x7F7F, 4000).astype(np.uint32) << np.uint32(16)
    half = (base | np.uint32(0x8000)).view(np.float32)
    x = np.concatenate([x, half])
    ours = O.f32_to_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, ref)
    np.testing.assert_array_equal(O.bf16_to_f32(ref), torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_c_division_semantics():
    for a in range(-40, 41):
        for b in (1, 3, 16):
            assert int(O.c_div(a, b)) == int(math.trunc(a / b))
            assert int(O.c_mod(a, b)) == a - int(math.trunc(a / b)) * b


# ----------------------------------------------------------------- planner
def _check_plan_against_brute(batch):
    r2t = batch.req_to_token.numpy()
    got = O.plan_decode(batch.seq_lens.numpy(), r2t, batch.req_indices.numpy(), batch.page_size,
                        batch.num_kv_heads, batch.topk, batch.bos, batch.eos, batch.max_chunk)
    dptr, dense, sptr, sparse, last, wq, wo, wl = brute_plan(
        batch.seq_lens.tolist(), r2t.tolist(), batch.req_indices.tolist(), batch.page_size,
        batch.num_kv_heads, batch.topk, batch.bos, batch.eos, batch.max_chunk)
    assert got["dense_indptr"].tolist() == dptr
    assert got["sparse_indptr"].tolist() == sptr
    assert got["dense_indices"].tolist() == dense
    assert got["kv_last_page_len"].tolist() == last
    w = got["sparse_written"]
    assert [None if not w[i] else int(v) for i, v in enumerate(got["sparse_indices"])] == sparse
    assert got["winfo_q"].tolist() == wq
    assert got["winfo_off"].tolist() == wo
    assert got["winfo_len"].tolist() == wl
    assert got["num_workloads"] == len(wq)


@pytest.mark.parametrize("seed", range(30))
def test_plan_matches_bruteforce_small(seed):
    _check_plan_against_brute(W.random_small(seed))


def test_plan_matches_bruteforce_c1():
    _check_plan_against_brute(W.c1())


def test_plan_int16_wraparound():
    # a request with n - bos - eos = 32770 middle pages: the planner's int16
    # makes it negative, so no workload is emitted for it (reference quirk)
    P = 1
    L = 32770 + 2
    batch = W.make_batch([L, 500], pool_pages=L + 600, seed=5, page_size=P, num_kv_heads=1, topk=30,
                         bos=1, eos=1, max_chunk=4096, min_chunk=1024)
    got = O.plan_decode(batch.seq_lens.numpy(), batch.req_to_token.numpy(), batch.req_indices.numpy(), P, 1,
                        30, 1, 1, 4096)
    assert set(got["winfo_q"].tolist()) == {1}
    _check_plan_against_brute(batch)


def test_plan_invariants_c2():
    batch = W.c2()
    H, P = batch.num_kv_heads, batch.page_size
    budget = batch.topk + batch.bos + batch.eos
    g = O.plan_decode(batch.seq_lens.numpy(), batch.req_to_token.numpy(), batch.req_indices.numpy(), P, H,
                      batch.topk, batch.bos, batch.eos, batch.max_chunk)
    n = (batch.seq_lens.numpy().astype(np.int64) + P - 1) // P
    assert g["dense_indptr"][-1] == H * n.sum()
    assert g["sparse_indptr"][-1] == H * np.minimum(n, budget).sum()
    assert (np.diff(g["dense_indptr"]) >= 0).all()
    # every dense entry names a page of its own request, in token order
    for b in range(batch.batch):
        for h in (0, H - 1):
            s = b * H + h
            seg = g["dense_indices"][g["dense_indptr"][s]:g["dense_indptr"][s + 1]]
            assert ((seg - h) % H == 0).all()
            np.testing.assert_array_equal((seg - h) // H, batch.pages[b].numpy())
    # the workloads tile exactly the middle pages of segments with more than topk of them
    cov = np.zeros(g["dense_indptr"][-1], dtype=np.int64)
    for off, ln in zip(g["winfo_off"], g["winfo_len"]):
        assert 1 <= ln <= batch.max_chunk
        cov[off:off + ln] += 1
    expect = np.zeros_like(cov)
    for s in range(batch.batch * H):
        a, e = g["dense_indptr"][s] + batch.bos, g["dense_indptr"][s + 1] - batch.eos
        if e - a > batch.topk:
            expect[a:e] = 1
    np.testing.assert_array_equal(cov, expect)
    assert (g["kv_last_page_len"] == np.repeat(np.where(batch.seq_lens.numpy() % P == 0, P,
                                                        batch.seq_lens.numpy() % P), H)).all()


# ----------------------------------------------------------------- top-k
def _topk_case(n_list, topk, bos, eos, values, H=1):
    batch = W.make_batch([n * 1 for n in n_list], pool_pages=sum(n_list) + 3, seed=7, page_size=1,
                         num_kv_heads=H, topk=topk, bos=bos, eos=eos)
    plan = O.plan_decode(batch.seq_lens.numpy(), batch.req_to_token.numpy(), batch.req_indices.numpy(), 1, H,
                         topk, bos, eos, 64)
    bits = O.f32_to_bf16(values[:plan["dense_indptr"][-1]])
    out, written = O.topk(bits, plan["dense_indptr"], plan["sparse_indptr"], plan["dense_indices"],
                          plan["sparse_indices"], batch.batch * H, topk, bos, eos)
    return plan, bits, out, written


@pytest.mark.parametrize("seed", range(20))
def test_topk_matches_bruteforce(seed):
    rng = np.random.default_rng(seed)
    n_list = rng.integers(1, 90, rng.integers(1, 6)).tolist()
    topk = int(rng.integers(1, 12))
    bos, eos = int(rng.integers(0, 3)), int(rng.integers(0, 3))
    kind = seed % 3
    total = sum(n_list) * 2
    if kind == 0:
        vals = rng.standard_normal(total).astype(np.float32)
    elif kind == 1:
        vals = rng.integers(-2, 3, total).astype(np.float32)  # heavy ties
    else:
        vals = np.where(rng.random(total) < 0.5, -0.0, 0.0).astype(np.float32)  # signed zeros
    plan, bits, out, written = _topk_case(n_list, topk, bos, eos, vals, H=2)
    f = O.bf16_to_f32(bits)
    expect_written = np.zeros_like(written)
    for s in range(len(n_list) * 2):
        a, e = plan["dense_indptr"][s] + bos, plan["dense_indptr"][s + 1] - eos
        o0 = plan["sparse_indptr"][s] + bos
        if e - a > topk:
            expect_written[o0:o0 + topk] = True
    np.testing.assert_array_equal(written, expect_written)  # short segments untouched
    for s in range(len(n_list) * 2):
        a, e = plan["dense_indptr"][s] + bos, plan["dense_indptr"][s + 1] - eos
        o0 = plan["sparse_indptr"][s] + bos
        if e - a <= topk:
            continue
        seg = [float(v) for v in f[a:e]]
        idx = brute_topk_segment(seg, topk)
        assert out[o0:o0 + topk].tolist() == [int(plan["dense_indices"][a + i]) for i in idx]


def test_topk_special_cases():
    # all equal: the first k positions, in order
    plan, bits, out, _ = _topk_case([40], 5, 1, 1, np.full(40, 0.5, np.float32))
    assert out[1:6].tolist() == plan["dense_indices"][1:6].tolist()
    # n == topk: untouched (the planner already placed every page)
    plan, bits, out, written = _topk_case([7], 5, 1, 1, np.arange(7, dtype=np.float32))
    assert not written.any()
    # n == topk + 1: the worst middle page is dropped
    vals = np.array([9, 1, 5, 0.25, 7, 3, 9], np.float32)
    plan, bits, out, _ = _topk_case([7], 4, 1, 1, vals)
    mid = plan["dense_indices"][1:6]
    assert out[1:5].tolist() == [mid[3], mid[1], mid[4], mid[0]]


# ----------------------------------------------------------------- reductions
@pytest.mark.parametrize("rtype", [O.MEAN, O.MAX, O.MIN, O.L2NORM])
@pytest.mark.parametrize("dim", [1, 2])
def test_page_reduce_against_torch(rtype, dim):
    rng = np.random.default_rng(3)
    H, P, C, pages = 3, 16, 24, 10
    x = O.f32_to_bf16(rng.standard_normal((pages * H, P, C)).astype(np.float32))
    loc = np.array([2 * P + 15, 5 * P + 3, 7 * P + 15, 9 * P + 15], dtype=np.int64)
    oshape = (pages * H, 1, C) if dim == 1 else (pages * H, P, 1)
    out0 = np.full(oshape, 0x3F80, np.uint16)  # 1.0
    got, rows = O.page_reduce(x, out0, loc, H, P, dim, rtype)
    expect_rows = sorted(p * H + h for p in (2, 7, 9) for h in range(H))
    assert rows.tolist() == expect_rows
    t = torch.from_numpy(O.bf16_to_f32(x)).double()
    axis = 1 if dim == 1 else 2
    ref = {O.MEAN: t.mean(axis, keepdim=True), O.MAX: t.amax(axis, keepdim=True),
           O.MIN: t.amin(axis, keepdim=True), O.L2NORM: torch.linalg.vector_norm(t, dim=axis, keepdim=True)}[rtype]
    ref_bits = ref.float().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got[expect_rows], ref_bits[expect_rows])
    untouched = np.setdiff1d(np.arange(pages * H), expect_rows)
    assert (got[untouched] == 0x3F80).all()


def test_page_reduce_closed_forms_and_f32_output():
    H, P, C = 2, 16, 8
    x = np.zeros((4 * H, P, C), np.uint16)
    x[2] = O.f32_to_bf16(np.full((P, C), -1.5, np.float32))
    out, _ = O.page_reduce(x, np.zeros((4 * H, 1, C), np.float32), np.array([P + 15]), H, P, 1, O.MEAN)
    assert (out[2] == -1.5).all() and (out[3] == 0).all()
    out, _ = O.page_reduce(x, np.zeros((4 * H, 1, C), np.float32), np.array([P + 15]), H, P, 1, O.L2NORM)
    np.testing.assert_allclose(out[2], 1.5 * 4.0)  # sqrt(16 * 1.5^2)
    # an fp32 output holds the bf16-rounded value
    rng = np.random.default_rng(1)
    x = O.f32_to_bf16(rng.standard_normal((H, P, C)).astype(np.float32))
    o32, _ = O.page_reduce(x, np.zeros((H, 1, C), np.float32), np.array([15]), H, P, 1, O.MEAN)
    o16, _ = O.page_reduce(x, np.zeros((H, 1, C), np.uint16), np.array([15]), H, P, 1, O.MEAN)
    np.testing.assert_array_equal(o32, O.bf16_to_f32(o16))
    # C semantics of loc: -1 closes "page 0"; -2 closes nothing
    o, rows = O.page_reduce(x, np.zeros((H, 1, C), np.uint16), np.array([-1]), H, P, 1, O.MAX)
    assert rows.tolist() == [0, 1]
    o, rows = O.page_reduce(x, np.zeros((H, 1, C), np.uint16), np.array([-2]), H, P, 1, O.MAX)
    assert rows.tolist() == []


# ----------------------------------------------------------------- GeMV
def test_gemv_against_matmul_and_one_hot():
    batch = W.random_small(4)
    plan = O.plan_decode(batch.seq_lens.numpy(), batch.req_to_token.numpy(), batch.req_indices.numpy(),
                         batch.page_size, batch.num_kv_heads, batch.topk, batch.bos, batch.eos, batch.max_chunk)
    rng = np.random.default_rng(2)
    H, D = batch.num_kv_heads, 32
    S = batch.batch * H
    x = O.f32_to_bf16(rng.standard_normal((S, D)).astype(np.float32))
    y = O.f32_to_bf16(rng.standard_normal((batch.pool_pages * H, D)).astype(np.float32))
    n = int(plan["dense_indptr"][-1])
    sc, cov = O.gemv(x, y, plan["dense_indices"], plan["winfo_q"], plan["winfo_off"], plan["winfo_len"],
                     plan["num_workloads"], n)
    X = torch.from_numpy(O.bf16_to_f32(x)).double()
    Y = torch.from_numpy(O.bf16_to_f32(y)).double()
    for w in range(plan["num_workloads"]):
        q, off, ln = plan["winfo_q"][w], plan["winfo_off"][w], plan["winfo_len"][w]
        rows = torch.from_numpy(plan["dense_indices"][off:off + ln].astype(np.int64))
        ref = (Y[rows] @ X[q]).float().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        np.testing.assert_array_equal(sc[off:off + ln], ref)
    assert cov.sum() == plan["winfo_len"].sum()
    # one-hot query picks a column of the centroid rows exactly
    xo = np.zeros_like(x)
    xo[:, 5] = O.f32_to_bf16(np.float32(1.0))
    sc1, _ = O.gemv(xo, y, plan["dense_indices"], plan["winfo_q"], plan["winfo_off"], plan["winfo_len"],
                    plan["num_workloads"], n)
    np.testing.assert_array_equal(sc1[cov], y[plan["dense_indices"][cov], 5])


def test_q_group_mean_matches_torch():
    rng = np.random.default_rng(9)
    q = O.f32_to_bf16(rng.standard_normal((64, 2, 128)).astype(np.float32))
    ours = O.q_group_mean(q)
    ref = torch.from_numpy(q.view(np.int16)).view(torch.bfloat16).mean(dim=1, keepdim=True)
    np.testing.assert_array_equal(ours, ref.view(torch.int16).numpy().view(np.uint16))


# ----------------------------------------------------------------- planted mistakes
def test_planted_tie_order_mistake_is_caught(monkeypatch):
    """A top-k that breaks ties toward the higher position must fail the
    brute-force comparison used above."""
    real = O.topk

    def wrong(score_bits, dip, sip, didx, sidx, eff, topk, bos, eos):
        sc = O.bf16_to_f32(score_bits).astype(np.float64)
        out = np.array(sidx, copy=True)
        written = np.zeros(out.shape[0], dtype=bool)
        for s in range(eff):
            a, e = dip[s] + bos, dip[s + 1] - eos
            if e - a <= topk:
                continue
            keys = sc[a:e] + 0.0
            order = np.lexsort((-np.arange(e - a), -keys))[:topk]  # ties: higher position first
            out[sip[s] + bos:sip[s] + bos + topk] = didx[a + order]
            written[sip[s] + bos:sip[s] + bos + topk] = True
        return out, written

    monkeypatch.setattr(O, "topk", wrong)
    with pytest.raises(AssertionError):
        test_topk_matches_bruteforce(1)  # the heavy-ties case
    monkeypatch.setattr(O, "topk", real)
    test_topk_matches_bruteforce(1)


def test_planted_planner_mistake_is_caught(monkeypatch):
    """Dropping the int16 truncation of the middle-page count must fail."""
    real = O._int16
    monkeypatch.setattr(O, "_int16", lambda v: int(v))
    with pytest.raises(AssertionError):
        test_plan_int16_wraparound()
    monkeypatch.setattr(O, "_int16", real)


@pytest.mark.parametrize("seed", range(12))
def test_plan_fa3_matches_bruteforce(seed):
    """FA3 planner extras, restated per segment from the brute-force planner:
    padded dense / sparse page tables (the FA3 indices kernel's writes,
    utils_sglang.cu:1041-1078) and cache lengths (utils_sglang.cu:966-977)."""
    batch = W.random_small(seed)
    P, H = batch.page_size, batch.num_kv_heads
    L = batch.seq_lens.numpy()
    args = (L, batch.req_to_token.numpy(), batch.req_indices.numpy(), P, H, batch.topk, batch.bos, batch.eos,
            batch.max_chunk)
    stride = max(1, batch.max_pages_per_request - 3)  # also exercises rows longer than the table
    got = O.plan_decode_fa3(*args, stride)
    dptr, dense, sptr, sparse, last, wq, wo, wl = brute_plan(*args)
    budget = batch.topk + batch.bos + batch.eos
    for b in range(len(L)):
        nb = _py_trunc_div(int(L[b]) + P - 1, P)
        for h in range(H):
            s = b * H + h
            assert got["dense_cache_seqlens"][s] == L[b]
            assert got["sparse_cache_seqlens"][s] == min((budget - 1) * P + last[s], int(L[b]))
            for j in range(stride):
                if j < nb:
                    assert got["dense_pt_written"][s, j] and got["dense_page_table"][s, j] == dense[dptr[s] + j]
                else:
                    assert not got["dense_pt_written"][s, j]
            if nb <= budget:
                slots = list(range(nb))
            else:
                slots = list(range(batch.bos)) + [budget - 1 - e for e in range(batch.eos)]
            for i in range(stride):
                if i in slots:
                    assert got["sparse_pt_written"][s, i] and got["sparse_page_table"][s, i] == sparse[sptr[s] + i]
                else:
                    assert not got["sparse_pt_written"][s, i]
    np.testing.assert_array_equal(got["dense_indices"], np.asarray(dense, dtype=np.int32))
