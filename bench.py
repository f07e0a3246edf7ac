"""Benchmark of the Vortex indexer + cache hot path on one MI355X.

Headline (BASELINE.json metric, configs[1] = C2): one decode step of
block_sparse_attention at Qwen3-1.7B shape — plan_decode once, then for each
of the 27 sparse layers forward_cache (CMean of the pages the new tokens
close) and forward_indexer (q head-group mean, GeMV, topK) — for batch 64,
L ~ U[1024, 8192], page 16, top-30 + 1 BOS + 1 EOS.  Every layer has its own
centroid pool and K pool (together far larger than the 256 MB Infinity
Cache, so replays do not hit in it).  The step is captured once as a HIP
graph and replayed; `value` is µs per step (HIP events on the replay stream).

Extra fields: achieved_GBps (algorithmic bytes of the step / time); roofline
(the fused indexer kernel — the dominant one — timed alone from a graph of
its 27 per-layer launches); unfused_us_per_step (the same step with every op
launched separately, VORTEX_FUSE=0); cpu_baseline (the CPU oracle on a
bounded sample of the same step).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "vortex_torch-dev_amd"), os.path.join(ROOT, "tests"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402
import torch  # noqa: E402

import workloads as W  # noqa: E402

METRIC = json.load(open(os.path.join(ROOT, "BASELINE.json")))["metric"]
HBM_PEAK_GBPS = 8000.0


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=27)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-unfused", action="store_true", help="skip the unfused comparison")
    ap.add_argument("--kernel-reps", type=int, default=20)
    return ap.parse_args()


class DecodeStep:
    """All device state of one C2 decode step, built through the public API."""

    def __init__(self, batch: W.DecodeBatch, layers: int, dev: torch.device, seed: int = 7):
        from vortex_torch import flow as vflow
        from vortex_torch.abs import FORMAT, as_vtensor

        self.batch, self.layers, self.dev = batch, layers, dev
        H, G, D, P, B = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size, batch.batch
        self.ictx, self.cctx = W.make_contexts(batch, dev)
        db = batch.to(dev)
        self.seq_lens, self.req_to_token, self.req_indices = db.seq_lens, db.req_to_token, db.req_indices
        self.loc_host = W.decode_loc(batch).numpy()
        self.loc = torch.from_numpy(self.loc_host).to(dev)

        self.flows, self.caches, self.qs = [], [], []
        self.plain = []  # (k, centroids, q) without the layout tag
        rows = batch.pool_pages * H
        for layer in range(layers):
            f = vflow.build_vflow("block_sparse_attention")
            k = W.randn_bf16((rows, P, D), seed + 3 * layer, dev)
            cen = W.randn_bf16((rows, 1, D), seed + 3 * layer + 1, dev, std=0.25)
            qp = W.randn_bf16((B * H, G, D), seed + 3 * layer + 2, dev)
            self.plain.append((k, cen, qp))
            self.flows.append(f)
            self.caches.append({"k": as_vtensor(k, FORMAT.PAGED), "centroids": as_vtensor(cen, FORMAT.PAGED)})
            self.qs.append(as_vtensor(qp, FORMAT.BATCHED))
        self.o = as_vtensor(self.ictx.sparse_kv_indices.view(-1, 1, 1), FORMAT.RAGGED)

        self.ictx.profile()
        self.cctx.profile()
        for f, cache, q in zip(self.flows, self.caches, self.qs):
            f.forward_cache(cache, self.loc, self.cctx)
            f.forward_indexer(q, self.o, cache, self.ictx)
        self.ictx.execute()
        self.cctx.execute()
        self.qmean = torch.empty((B * H, 1, D), device=dev, dtype=torch.bfloat16)

    def run(self):
        from vortex_torch.indexer.utils_sglang import plan_decode

        plan_decode(self.seq_lens, self.req_to_token, self.req_indices, self.ictx)
        for f, cache, q in zip(self.flows, self.caches, self.qs):
            f.forward_cache(cache, self.loc, self.cctx)
            f.forward_indexer(q, self.o, cache, self.ictx)

    def indexer_kernels_only(self):
        """The fused indexer kernel of every layer, launched directly."""
        from vortex_torch import _hip

        ic, b = self.ictx, self.batch
        for f, (_, cen, qp) in zip(self.flows, self.plain):
            with torch._C.DisableTorchFunctionSubclass():
                _hip.indexer_fused(qp, self.qmean, cen, f.gemv.output_buffer, ic.dense_kv_indptr,
                                   ic.sparse_kv_indptr, ic.dense_kv_indices, ic.sparse_kv_indices,
                                   b.batch * b.num_kv_heads, b.topk, b.bos, b.eos,
                                   b.max_pages_per_request)


def algorithmic_bytes(batch: W.DecodeBatch, plan: dict, layers: int, loc_host: np.ndarray) -> dict:
    """Bytes each part of the step must move at least once (each counted once)."""
    H, G, D, P, B = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size, batch.batch
    covered = int(plan["winfo_len"].sum())
    dip = plan["dense_indptr"]
    seg_n = np.diff(dip.astype(np.int64)) - batch.bos - batch.eos
    sel_segs = int((seg_n > batch.topk).sum())
    q_in = B * H * G * 2 * D
    q_out = B * H * 2 * D
    # GeMV: centroid row + row id + score per scored page, plus the query rows
    gemv = covered * (2 * D + 4 + 2) + q_out
    # topK: score + row id per candidate page, top-k ids written
    topk = covered * (2 + 4) + sel_segs * batch.topk * 4
    qmean = q_in + q_out
    # fused kernel: query in, mean out, row ids + centroid rows in, scores out, ids out
    fused = q_in + q_out + covered * (4 + 2 * D + 2) + sel_segs * batch.topk * 4 + (B * H + 1) * 8
    ndense = int(dip[-1])
    plan_b = ndense * 4 + (ndense // H) * 4 + 2 * (B * H + 1) * 4 + int(plan["sparse_indptr"][-1]) * 4 + B * 16
    finishing = int(((loc_host + 1) % P == 0).sum()) * H
    cmean = finishing * (P * 2 * D + 2 * D) + B * 8
    per_layer = gemv + topk + qmean + cmean
    return {"gemv": gemv, "topk": topk, "qmean": qmean, "cmean": cmean, "plan": plan_b, "fused": fused,
            "step": plan_b + layers * per_layer, "covered_pages": covered}


def time_graph(graph: torch.cuda.CUDAGraph, reps: int, warmup: int) -> float:
    """Mean milliseconds per replay; replays and events on the current stream."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(reps):
        graph.replay()
    t1.record(stream)
    t1.synchronize()
    return t0.elapsed_time(t1) / reps


def capture(fn) -> torch.cuda.CUDAGraph:
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up outside the graph (allocations, lazy init)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        fn()
    torch.cuda.synchronize()
    return g


def cpu_baseline(batch: W.DecodeBatch, step: DecodeStep, sample_layers: int = 8) -> dict:
    """The CPU oracle (numpy, one thread) on the same data: plan + `sample_layers`
    layers of (CMean of closed pages, q-mean, GeMV, topK), scaled to the step."""
    from threadpoolctl import threadpool_limits

    from oracle import vortex_oracle as O

    def bits(t):
        return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    H, D, P = batch.num_kv_heads, batch.head_dim, batch.page_size
    sl, r2t, ri = batch.seq_lens.numpy(), batch.req_to_token.numpy(), batch.req_indices.numpy()
    n_layers = min(sample_layers, step.layers)
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        plan = O.plan_decode(sl, r2t, ri, P, H, batch.topk, batch.bos, batch.eos, batch.max_chunk)
        t_plan = time.perf_counter() - t0
        t_layers = 0.0
        for layer in range(n_layers):
            k_pool, cen_pool, q_plain = step.plain[layer]
            trig = step.loc_host[(step.loc_host + 1) % P == 0]
            rows = np.unique((trig[:, None] // P * H + np.arange(H)[None, :]).reshape(-1))
            k_rows = bits(k_pool[torch.as_tensor(rows, device=step.dev)]) if rows.size else np.zeros((0, P, D), np.uint16)
            cen, q = bits(cen_pool), bits(q_plain)
            t0 = time.perf_counter()
            # CMean of the closed pages; the compact copy holds page i at rows i*H..i*H+H-1
            O.page_reduce(k_rows, np.zeros((rows.size, 1, D), np.uint16),
                          np.arange(0, rows.size // H) * P + (P - 1), H, P, 1, O.MEAN)
            qm = O.q_group_mean(q)
            sc, _ = O.gemv(qm, cen, plan["dense_indices"], plan["winfo_q"], plan["winfo_off"],
                           plan["winfo_len"], plan["num_workloads"], int(plan["dense_indptr"][-1]))
            O.topk(sc, plan["dense_indptr"], plan["sparse_indptr"], plan["dense_indices"],
                   plan["sparse_indices"], batch.batch * H, batch.topk, batch.bos, batch.eos)
            t_layers += time.perf_counter() - t0
    per_step = t_plan + t_layers * step.layers / n_layers
    return {"value": round(per_step * 1e6, 1), "unit": "us/step", "cores": 1, "kind": "port",
            "sample": f"plan + {n_layers} of {step.layers} layers of the same C2 step (oracle, numpy, "
                      f"1 thread), layer time scaled to {step.layers} layers; measured "
                      f"{t_plan + t_layers:.2f} s"}


def main():
    args = _parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus above 1 is not supported "
                                   "(the indexer shards by request / kv head with no exchange)"}))
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(2)
    from vortex_torch import _hip

    _hip.load_library()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    batch = W.c2()
    print(f"[bench] building C2 step: {batch.batch} requests, {args.layers} layers", file=sys.stderr, flush=True)
    step = DecodeStep(batch, args.layers, dev)

    from oracle import vortex_oracle as O  # sizes the algorithmic byte count only

    plan = O.plan_decode(batch.seq_lens.numpy(), batch.req_to_token.numpy(), batch.req_indices.numpy(),
                         batch.page_size, batch.num_kv_heads, batch.topk, batch.bos, batch.eos, batch.max_chunk)
    nbytes = algorithmic_bytes(batch, plan, args.layers, step.loc_host)

    os.environ["VORTEX_FUSE"] = "1"
    g = capture(step.run)
    us_step = time_graph(g, args.steps, args.warmup) * 1000.0
    print(f"[bench] step {us_step:.1f} us", file=sys.stderr, flush=True)

    gk = capture(step.indexer_kernels_only)
    us_fused = time_graph(gk, args.kernel_reps, 3) * 1000.0 / args.layers
    fused_gbps = nbytes["fused"] / (us_fused * 1e-6) / 1e9
    print(f"[bench] fused indexer {us_fused:.2f} us/launch, {fused_gbps:.0f} GB/s", file=sys.stderr, flush=True)

    unfused = None
    if not args.no_unfused:
        os.environ["VORTEX_FUSE"] = "0"
        gu = capture(step.run)
        unfused = round(time_graph(gu, max(5, args.steps // 5), 3) * 1000.0, 2)
        os.environ["VORTEX_FUSE"] = "1"
        del gu
        print(f"[bench] unfused step {unfused:.1f} us", file=sys.stderr, flush=True)

    gbps = nbytes["step"] / (us_step * 1e-6) / 1e9
    out = {
        "metric": METRIC,
        "value": round(us_step, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_step / 1000.0, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded; random-init K, centroid and query tensors of the C2 shapes)",
        "config": {
            "workload": "C2: decode step, batch 64, L~U[1024,8192], 27 sparse layers, Qwen3-1.7B "
                        "head shape (H_q 16, H_kv 8, D 128), page 16, top-30 + 1 BOS + 1 EOS, "
                        "40k-page shared pool, per-layer pools; one HIP graph per step",
            "batch": batch.batch,
            "layers": args.layers,
            "dense_pages": int(plan["dense_indptr"][-1]),
            "scored_pages_per_layer": nbytes["covered_pages"],
            "max_chunk_size": batch.max_chunk,
        },
        "achieved_GBps": round(gbps, 1),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "algorithmic_bytes_per_step": nbytes["step"],
        "unfused_us_per_step": unfused,
        "roofline": {
            "kernel": "indexer_fused_kernel<512,16,1> (q-mean + GeMV + top-k, one layer)",
            "bound": "hbm",
            "achieved": round(fused_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(fused_gbps / HBM_PEAK_GBPS, 4),
            "traffic": None,
            "us_per_launch": round(us_fused, 3),
            "bytes_per_launch": nbytes["fused"],
        },
    }
    if not args.no_cpu:
        print("[bench] cpu baseline (oracle)", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(batch, step)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
