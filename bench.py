"""Benchmark of the Vortex indexer + cache hot path on one MI355X.

Headline (BASELINE.json metric, configs[1] = C2): one decode step of
block_sparse_attention at Qwen3-1.7B shape — plan_decode once, then for each
of the 27 sparse layers forward_cache (CMean of the pages the new tokens
close) and forward_indexer (q head-group mean, GeMV, topK) — for batch 64,
L ~ U[1024, 8192], page 16, top-30 + 1 BOS + 1 EOS.  Every layer has its own
centroid pool and K pool (together far larger than the 256 MB Infinity
Cache, so replays do not hit in it).  The step is captured once as a HIP
graph; `--steps` replays are timed one by one with HIP events on the replay
stream and `value` is their median in µs (min, max and mean in replay_us).

Extra fields: achieved_GBps (algorithmic bytes of the step / time); roofline
(the fused indexer kernel — the dominant one — timed alone from a graph of
its 27 per-layer launches, at least 50 replays, median per launch; with the
box's ceiling beside it: a bare gather of the same rows, the same gather
behind one dependent load of the segment bounds, and a sequential read of
1 GiB, as achievable_GBps, frac_of_achievable, ceiling and seq_read);
unfused_us_per_step (the same step with every op launched separately,
VORTEX_FUSE=0); cpu_baseline (the CPU oracle on the same step, one thread
per host core, median of 3 runs); configs (C3, C4 and C5 measured the same
way: their step, or C4's burst, and their dominant kernel's roofline).

Other invocations:
  --config c3 / c5   a line for the C3 (8 x 32k tokens, top-64) or C5 (MLA
                     latent cache, D 576, G 16, top-32) decode step;
  --config c4        page-finish burst: CMean + CMax of 65,536 pages (1M loc
                     entries) into a 70k-page pool, fused (one pass over K)
                     and as two separate ops.
  --traffic-probe    launches the fused indexer kernel of every layer eagerly
                     (with --probe-unfused also the step with every op on its
                     own; at C4 the burst), then a bf16 negation of a 512 MiB
                     buffer (a copy kernel of known size), and exits: the
                     program the counter passes (rocprofv3 --pmc) profile;
  --traffic-from DIR turns those passes into profiles/traffic.json, which the
                     roofline's `traffic` reads (only while the kernel, its
                     algorithmic bytes and the kernel sources still match).
  --attention        paged decode attention over the sparse table the indexer
                     selects and over the dense table (all pages), per layer;
  --flow gqa / quest the same decode step with gqa_block_sparse_attention or
                     gqa_quest_sparse_attention.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]
                       [--config c2|c3|c4|c5] [--flow block_sparse|gqa|quest] [--attention]
                       [--layers N] [--traffic-probe [--probe-unfused]] [--traffic-from DIR]
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

# HBM bytes per launch of each configuration's dominant kernel come from the
# FETCH_SIZE and WRITE_SIZE counter passes over --traffic-probe, each scaled
# by what the counter reads for the probe's copy kernel of known size;
# `--traffic-from DIR` turns those passes into profiles/traffic.json, keyed by
# configuration, with the kernel's name, its algorithmic bytes and a hash of
# the kernel sources.  A run uses a figure only when all three match its own
# (kernel_sources_hash below); otherwise `traffic` is null and
# `traffic_note` says why, so a kernel change cannot leave a stale figure.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def kernel_sources_hash() -> str:
    """sha256 (first 16 hex digits) of every kernel source and header."""
    import hashlib

    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "vortex_torch-dev_amd", "csrc")
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".hip", ".h")):
            h.update(name.encode())
            with open(os.path.join(csrc, name), "rb") as fh:
                h.update(fh.read())
    return h.hexdigest()[:16]


def traffic_for(cfg: str, kernel: str, bytes_per_launch: int):
    """(HBM bytes per launch, None) from profiles/traffic.json when it was
    measured for this kernel, these algorithmic bytes and these sources;
    else (None, the reason)."""
    try:
        with open(TRAFFIC_FILE) as fh:
            rec = json.load(fh).get(cfg)
    except (OSError, ValueError):
        return None, "no profiles/traffic.json"
    if rec is None:
        return None, f"no counter passes recorded for {cfg}"
    if rec.get("kernel") != kernel:
        return None, f"counter passes were of {rec.get('kernel')}, this run launches {kernel}"
    if rec.get("bytes_per_launch") != bytes_per_launch:
        return None, f"algorithmic bytes differ from the counter passes' ({rec.get('bytes_per_launch')})"
    if rec.get("sources") != kernel_sources_hash():
        return None, "kernel sources changed since the counter passes"
    return int(rec["traffic"]), None


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=27)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-unfused", action="store_true", help="skip the unfused comparison")
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--config", default="c2", choices=["c2", "c3", "c4", "c5"])
    ap.add_argument("--flow", default="block_sparse", choices=sorted(FLOWS),
                    help="registered flow of the decode step (side measurement unless block_sparse)")
    ap.add_argument("--attention", action="store_true",
                    help="side measurement: paged decode attention over the sparse and the dense table")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run the kernels a counter pass profiles, print their sizes, exit")
    ap.add_argument("--probe-unfused", action="store_true",
                    help="with --traffic-probe: also run the step with every op launched on its own")
    ap.add_argument("--no-extra", action="store_true", help="skip the C3 / C4 / C5 keys of the C2 line")
    ap.add_argument("--traffic-from", metavar="DIR",
                    help="write profiles/traffic.json from the counter passes under DIR (no GPU needed), exit")
    return ap.parse_args()


FLOWS = {"block_sparse": "block_sparse_attention", "gqa": "gqa_block_sparse_attention",
         "quest": "gqa_quest_sparse_attention"}

DECODE_CONFIGS = {
    "c2": ("C2: decode step, batch 64, L~U[1024,8192], 27 sparse layers, Qwen3-1.7B head shape "
           "(H_q 16, H_kv 8, D 128), page 16, top-30 + 1 BOS + 1 EOS, 40k-page shared pool, "
           "per-layer pools; one HIP graph per step"),
    "c3": ("C3: decode step, batch 8 x 32768 tokens (2048 pages per request), 27 sparse layers, "
           "H_q 16, H_kv 8, D 128, page 16, top-64 + 1 BOS + 1 EOS; K = N(0,1) noise + per-(page, head) "
           "offsets ~ N(0, 0.5), centroids = its CMean; one HIP graph per step"),
    "c5": ("C5: MLA latent-cache decode step, batch 32, L~U[4096,16384], 27 sparse layers, "
           "1 latent head, G 16, D 576, page 16, top-32 + 1 BOS + 1 EOS; one HIP graph per step"),
}


def fused_kernel_name(batch: W.DecodeBatch) -> str:
    """Kernel instance the fused launch selects (VTX_FUSED_AUTO: split layout
    when there are fewer than two segments per compute unit)."""
    from vortex_torch._deferred import fused_layout

    lpr, vpl = {64: (8, 1), 128: (16, 1), 256: (16, 2), 512: (16, 4), 576: (8, 9)}[batch.head_dim]
    segments = batch.batch * batch.num_kv_heads
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    layout = fused_layout()
    if layout == 2 or (layout == 0 and segments < 2 * cus):
        # the library's split_threads / split_pass / chunk choice, with the
        # topK op's workspace (staging zone present)
        D = batch.head_dim
        small_pass = 32 if D <= 128 else 16
        waves_small = 8 if D <= 256 else 4
        mid = max(1, batch.max_pages_per_request - batch.bos - batch.eos)
        small_chunks = -(-mid // (waves_small * small_pass))
        quad = (D == 128 and batch.topk <= 64 and segments <= 512 and small_chunks <= 16
                and segments * small_chunks <= 4 * cus)
        threads_small = 256 if quad else 64 * waves_small
        large = D >= 512 or segments * small_chunks > (1024 // threads_small) * cus
        cm = 4 if batch.batch <= 256 else 0  # the decode CMean in the launch (loc in four registers per lane)
        if quad and not large:
            T, kpass = 256, 64
        else:
            T, kpass = (512 if D <= 256 else 256), small_pass * (2 if large else 1)
        return f"indexer_split_kernel<{T}, {lpr}, {vpl}, {kpass}, {cm}>"
    mp = batch.max_pages_per_request
    T = 256 if mp <= 256 else (512 if mp <= 1024 else 1024)
    # the decode CMean (loc: one token per request) runs in the same launch
    # for rows of one vector per lane, with loc in one register per lane up
    # to 64 tokens, four up to 256
    cm = (1 if batch.batch <= 64 else 4) if vpl == 1 and batch.batch <= 256 else 0
    return f"indexer_fused_kernel<{T}, {lpr}, {vpl}, {cm}>"


class DecodeStep:
    """All device state of one C2 decode step, built through the public API."""

    def __init__(self, batch: W.DecodeBatch, layers: int, dev: torch.device, seed: int = 7,
                 flow_name: str = "block_sparse_attention"):
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
        # C3: K with per-(page, head) offsets and the centroids its CMean writes;
        # otherwise K ~ N(0, 1) and centroid rows ~ N(0, 0.25^2), the spread of a
        # mean of 16 such rows
        offsets = bool(batch.extra.get("k_page_offsets"))
        for layer in range(layers):
            f = vflow.build_vflow(flow_name)
            if offsets:
                k = W.k_pool(batch, seed + 3 * layer, dev, page_offsets=True)
            else:
                k = W.randn_bf16((rows, P, D), seed + 3 * layer, dev)
            qp = W.randn_bf16((B * H, G, D), seed + 3 * layer + 2, dev)
            cache = {"k": as_vtensor(k, FORMAT.PAGED)}
            for j, (name, (r, c)) in enumerate(f.create_cache(P, D).items()):
                if offsets and name == "centroids":
                    pool = W.centroids_from_k(k, batch)
                else:
                    pool = W.randn_bf16((rows, r, c), seed + 3 * layer + 1 + 101 * j, dev, std=0.25)
                cache[name] = as_vtensor(pool, FORMAT.PAGED)
            cen = cache.get("centroids")
            self.plain.append((k, cen, qp))
            self.flows.append(f)
            self.caches.append(cache)
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
        self.premeaned = None
        from vortex_torch.indexer.matmul import MEAN_IN_KERNEL_MAX_G
        if G > MEAN_IN_KERNEL_MAX_G:
            with torch._C.DisableTorchFunctionSubclass():
                self.premeaned = [qp.mean(dim=1, keepdim=True) for (_, _, qp) in self.plain]

    def run(self):
        from vortex_torch.indexer.utils_sglang import plan_decode

        plan_decode(self.seq_lens, self.req_to_token, self.req_indices, self.ictx)
        for f, cache, q in zip(self.flows, self.caches, self.qs):
            f.forward_cache(cache, self.loc, self.cctx)
            f.forward_indexer(q, self.o, cache, self.ictx)

    def indexer_kernels_only(self):
        """The fused indexer kernel of every layer, launched directly as the
        step launches it: with the layer's decode CMean (the mean that
        forward_cache leaves for forward_indexer) in the same launch."""
        from vortex_torch import _hip
        from vortex_torch._deferred import fused_layout

        ic, b = self.ictx, self.batch
        for i, (f, (k, cen, qp)) in enumerate(zip(self.flows, self.plain)):
            with torch._C.DisableTorchFunctionSubclass():
                if self.premeaned is not None:  # the step hands the kernel torch's mean
                    q, x_out = self.premeaned[i], None
                else:
                    q, x_out = qp, self.qmean
                _hip.indexer_fused(q, x_out, cen, f.gemv.output_buffer, ic.dense_kv_indptr,
                                   ic.sparse_kv_indptr, ic.dense_kv_indices, ic.sparse_kv_indices,
                                   b.batch * b.num_kv_heads, b.topk, b.bos, b.eos,
                                   b.max_pages_per_request, seg_counters=f.output_func.seg_counters,
                                   mode=fused_layout(), cmean=(k, self.loc, b.num_kv_heads),
                                   schedule=ic._fused_schedule)


def gather_ceiling(step: DecodeStep, plan: dict, args) -> dict:
    """The bare gather of the rows the fused kernel scores, from the same 27
    per-layer centroid pools (vtx_probe_gather: one coalesced load of a
    pass's row ids, then the rows, nothing computed), and the same gather
    with one dependent load of the segment bounds first (the fused kernel's
    chain of trips); each as a graph of the layers' launches, median per
    launch of max(50, --kernel-reps) replays."""
    from vortex_torch import _hip

    b = step.batch
    dip = plan["dense_indptr"].astype(np.int64)
    pos = [np.arange(dip[s] + b.bos, dip[s + 1] - b.eos) for s in range(len(dip) - 1)
           if dip[s + 1] - b.eos - (dip[s] + b.bos) > b.topk]
    with torch._C.DisableTorchFunctionSubclass():
        rows = step.ictx.dense_kv_indices[torch.from_numpy(np.concatenate(pos)).to(step.dev)].contiguous()
        pools = [cen.view(cen.shape[0], -1) for (_, cen, _) in step.plain]
        indptr = step.ictx.dense_kv_indptr
    sink = torch.zeros(4 * rows.numel() + 4096, dtype=torch.int32, device=step.dev)  # one entry per thread
    row_bytes = pools[0].shape[1] * 2
    nbytes = rows.numel() * (row_bytes + 4)
    out = {"rows": int(rows.numel()), "row_bytes": int(row_bytes), "bytes_per_launch": int(nbytes)}
    for key, ip in (("gather", None), ("gather_head", indptr)):
        g = capture(lambda: [_hip.probe_gather(p, rows, sink, indptr=ip) for p in pools])
        us = replay_stats(time_replays(g, max(50, args.kernel_reps), 3), per=len(pools))["median"]
        del g
        out[f"{key}_us"] = us
        out[f"{key}_GBps"] = round(nbytes / (us * 1e-6) / 1e9, 1)
    return out


def seq_read_ceiling(dev, args) -> dict:
    """A sequential read of 1 GiB (vtx_probe_read), median of max(20,
    --kernel-reps) launches: the box's streaming-read rate."""
    from vortex_torch import _hip

    n = 1 << 30
    src = torch.empty(n // 2, dtype=torch.int16, device=dev).fill_(1)
    sink = torch.zeros(4096 * 512, dtype=torch.int32, device=dev)
    g = capture(lambda: _hip.probe_read(src, sink))
    us = replay_stats(time_replays(g, max(20, args.kernel_reps), 3))["median"]
    del g, src
    return {"bytes": n, "us": us, "GBps": round(n / (us * 1e-6) / 1e9, 1)}


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
    # fused kernel: query in (the G heads, or torch's mean past 16 heads), mean
    # out, row ids + centroid rows in, scores out, ids out
    from vortex_torch.indexer.matmul import MEAN_IN_KERNEL_MAX_G
    fused_q = q_in + q_out if G <= MEAN_IN_KERNEL_MAX_G else q_out
    ndense = int(dip[-1])
    plan_b = ndense * 4 + (ndense // H) * 4 + 2 * (B * H + 1) * 4 + int(plan["sparse_indptr"][-1]) * 4 + B * 16
    finishing = int(((loc_host + 1) % P == 0).sum()) * H
    # CMean: the K tiles of the pages the step's tokens close, their centroids
    # out, and loc
    cmean = finishing * (P * 2 * D + 2 * D) + loc_host.size * 8
    # the fused launch also runs the layer's CMean
    fused = fused_q + covered * (4 + 2 * D + 2) + sel_segs * batch.topk * 4 + (B * H + 1) * 8 + cmean
    per_layer = gemv + topk + qmean + cmean
    return {"gemv": gemv, "topk": topk, "qmean": qmean, "cmean": cmean, "plan": plan_b, "fused": fused,
            "step": plan_b + layers * per_layer, "covered_pages": covered}


def time_replays(graph: torch.cuda.CUDAGraph, reps: int, warmup: int) -> np.ndarray:
    """Milliseconds of each of `reps` back-to-back replays: a HIP event is
    recorded on the replay stream before the first replay and after every
    replay, so replay i is the interval between events i and i + 1."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    ev[0].record(stream)
    for i in range(reps):
        graph.replay()
        ev[i + 1].record(stream)
    ev[-1].synchronize()
    return np.array([ev[i].elapsed_time(ev[i + 1]) for i in range(reps)])


def time_graph(graph: torch.cuda.CUDAGraph, reps: int, warmup: int) -> float:
    """Median milliseconds per replay (see time_replays)."""
    return float(np.median(time_replays(graph, reps, warmup)))


def replay_stats(ms: np.ndarray, per: float = 1.0) -> dict:
    """Median, min, max and mean in µs of per-replay times, divided by `per`."""
    us = ms * 1000.0 / per
    return {"median": round(float(np.median(us)), 3), "min": round(float(us.min()), 3),
            "max": round(float(us.max()), 3), "mean": round(float(us.mean()), 3), "n": int(us.size)}


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


def cpu_baseline(batch: W.DecodeBatch, step: DecodeStep, reps: int = 3) -> dict:
    """The CPU oracle (numpy) on the same data: the whole step — plan, then
    for every layer the CMean of the closed pages, q-mean, GeMV and topK —
    with the layers spread over one thread per host core the process may
    use (numpy's own thread pools held to one thread each), `reps` times;
    the median wall time is reported."""
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits

    from oracle import vortex_oracle as O

    def bits(t):
        return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    H, D, P = batch.num_kv_heads, batch.head_dim, batch.page_size
    sl, r2t, ri = batch.seq_lens.numpy(), batch.req_to_token.numpy(), batch.req_indices.numpy()
    cores = len(os.sched_getaffinity(0))
    trig = step.loc_host[(step.loc_host + 1) % P == 0]
    rows = np.unique((trig[:, None] // P * H + np.arange(H)[None, :]).reshape(-1))
    host = []  # each layer's inputs on the host (copied before the timed region)
    for k_pool, cen_pool, q_plain in step.plain:
        k_rows = bits(k_pool[torch.as_tensor(rows, device=step.dev)]) if rows.size else np.zeros((0, P, D), np.uint16)
        host.append((k_rows, bits(cen_pool), bits(q_plain)))

    def layer(plan, i):
        k_rows, cen, q = host[i]
        # CMean of the closed pages; the compact copy holds page i at rows i*H..i*H+H-1
        O.page_reduce(k_rows, np.zeros((rows.size, 1, D), np.uint16),
                      np.arange(0, rows.size // H) * P + (P - 1), H, P, 1, O.MEAN)
        qm = O.q_group_mean(q)
        sc, _ = O.gemv(qm, cen, plan["dense_indices"], plan["winfo_q"], plan["winfo_off"], plan["winfo_len"],
                       plan["num_workloads"], int(plan["dense_indptr"][-1]))
        O.topk(sc, plan["dense_indptr"], plan["sparse_indptr"], plan["dense_indices"], plan["sparse_indices"],
               batch.batch * H, batch.topk, batch.bos, batch.eos)

    times = []
    with threadpool_limits(limits=1), ThreadPoolExecutor(max_workers=cores) as pool:
        for _ in range(reps):
            t0 = time.perf_counter()
            plan = O.plan_decode(sl, r2t, ri, P, H, batch.topk, batch.bos, batch.eos, batch.max_chunk)
            list(pool.map(lambda i: layer(plan, i), range(len(host))))
            times.append(time.perf_counter() - t0)
    return {"value": round(float(np.median(times)) * 1e6, 1), "unit": "us/step", "cores": cores, "kind": "port",
            "sample": f"the whole step (plan + {len(host)} layers) of the same data, layers spread over "
                      f"{cores} threads (one per host core of the process), median of {reps} runs: "
                      + ", ".join(f"{t:.2f} s" for t in times)}


def plan_summary(step: DecodeStep) -> dict:
    """The planner's outputs the byte count needs, read back from the device
    after the timed region (segment bounds and the workload list)."""
    ic, b = step.ictx, step.batch
    S = b.batch * b.num_kv_heads
    with torch._C.DisableTorchFunctionSubclass():
        nw = int(ic.winfo_num_workloads[0].item())
        return {
            "dense_indptr": ic.dense_kv_indptr[:S + 1].cpu().numpy(),
            "sparse_indptr": ic.sparse_kv_indptr[:S + 1].cpu().numpy(),
            "winfo_len": ic.winfo_kv_lens[:nw].cpu().numpy(),
        }


def measure_decode(cfg: str, args, dev, unfused: bool = False, cpu: bool = False) -> dict:
    """One decode configuration: the step graph (args.steps replays, each
    timed), the fused indexer kernel of every layer from a graph of its
    launches (at least 50 replays, each timed), their algorithmic bytes, and
    optionally the unfused step and the CPU baseline."""
    import gc

    batch = getattr(W, cfg)()
    print(f"[bench] building {cfg.upper()} step: {batch.batch} requests, {args.layers} layers",
          file=sys.stderr, flush=True)
    step = DecodeStep(batch, args.layers, dev)
    os.environ["VORTEX_FUSE"] = "1"
    g = capture(step.run)
    step_ms = time_replays(g, args.steps, args.warmup)
    del g
    st = replay_stats(step_ms)
    print(f"[bench] {cfg} step {st['median']:.1f} us (min {st['min']:.1f}, max {st['max']:.1f})",
          file=sys.stderr, flush=True)
    plan = plan_summary(step)
    nbytes = algorithmic_bytes(batch, plan, args.layers, step.loc_host)

    gk = capture(step.indexer_kernels_only)
    kern = replay_stats(time_replays(gk, max(50, args.kernel_reps), 3), per=args.layers)
    del gk
    us_fused = kern["median"]
    fused_gbps = nbytes["fused"] / (us_fused * 1e-6) / 1e9
    print(f"[bench] {cfg} fused indexer {us_fused:.2f} us/launch, {fused_gbps:.0f} GB/s", file=sys.stderr, flush=True)
    ceil = gather_ceiling(step, plan, args)
    print(f"[bench] {cfg} bare gather of the same rows {ceil['gather_us']:.2f} us/launch "
          f"({ceil['gather_GBps']:.0f} GB/s), with the bounds trip first {ceil['gather_head_us']:.2f} us",
          file=sys.stderr, flush=True)
    kname = fused_kernel_name(batch)
    traffic, note = traffic_for(cfg, kname, nbytes["fused"])
    res = {
        "workload": DECODE_CONFIGS[cfg],
        "us_per_step": st,
        "batch": batch.batch,
        "layers": args.layers,
        "dense_pages": int(plan["dense_indptr"][-1]),
        "scored_pages_per_layer": nbytes["covered_pages"],
        "max_chunk_size": batch.max_chunk,
        "algorithmic_bytes_per_step": nbytes["step"],
        "achieved_GBps": round(nbytes["step"] / (st["median"] * 1e-6) / 1e9, 1),
        "roofline": {
            "kernel": f"{kname} (CMean of the closed pages + q-mean + GeMV + top-k, one layer)",
            "bound": "hbm",
            "achieved": round(fused_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(fused_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "us_per_launch": us_fused,
            "us_per_launch_stats": kern,
            "bytes_per_launch": nbytes["fused"],
            # the box's ceiling for this access pattern: a kernel that only
            # gathers the same rows (vtx_probe_gather), and the fused kernel's
            # rate as a fraction of it (frac stays against the 8 TB/s peak)
            "achievable_GBps": round(ceil["gather_GBps"], 1),
            "frac_of_achievable": round(fused_gbps / ceil["gather_GBps"], 4),
            "ceiling": ceil,
        },
    }
    if note:
        res["roofline"]["traffic_note"] = note
    if unfused:
        os.environ["VORTEX_FUSE"] = "0"
        gu = capture(step.run)
        res["unfused_us_per_step"] = replay_stats(time_replays(gu, max(10, args.steps // 5), 3))["median"]
        os.environ["VORTEX_FUSE"] = "1"
        del gu
        print(f"[bench] {cfg} unfused step {res['unfused_us_per_step']:.1f} us", file=sys.stderr, flush=True)
    if cpu:
        print("[bench] cpu baseline (oracle)", file=sys.stderr, flush=True)
        res["cpu_baseline"] = cpu_baseline(batch, step)
    del step
    gc.collect()
    torch.cuda.empty_cache()
    return res


def bench_decode(args, dev) -> dict:
    if args.traffic_probe:
        batch = getattr(W, args.config)()
        return traffic_probe(DecodeStep(batch, args.layers, dev), dev, unfused=args.probe_unfused, cfg=args.config)
    m = measure_decode(args.config, args, dev, unfused=not args.no_unfused, cpu=not args.no_cpu)
    st = m["us_per_step"]
    out = {
        "metric": METRIC,
        "value": st["median"],
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(st["median"] / 1000.0, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic (seeded; random-init K, centroid and query tensors of the "
                f"{args.config.upper()} shapes)",
        "config": {k: m[k] for k in ("workload", "batch", "layers", "dense_pages", "scored_pages_per_layer",
                                     "max_chunk_size")},
        "replay_us": st,
        "achieved_GBps": m["achieved_GBps"],
        "hbm_frac": round(m["achieved_GBps"] / HBM_PEAK_GBPS, 4),
        "algorithmic_bytes_per_step": m["algorithmic_bytes_per_step"],
        "unfused_us_per_step": m.get("unfused_us_per_step"),
        "roofline": m["roofline"],
    }
    out["roofline"]["seq_read"] = seq_read_ceiling(dev, args)
    print(f"[bench] sequential read of 1 GiB: {out['roofline']['seq_read']['GBps']:.0f} GB/s", file=sys.stderr,
          flush=True)
    if "cpu_baseline" in m:
        out["cpu_baseline"] = m["cpu_baseline"]
    if args.config == "c2" and not args.no_extra:
        # the other configurations of the scope table, measured the same way
        extra = {}
        for cfg in ("c3", "c5"):
            m = measure_decode(cfg, args, dev)
            extra[cfg] = {k: m[k] for k in ("workload", "us_per_step", "achieved_GBps", "roofline")}
        b = bench_burst(args, dev)
        extra["c4"] = {"workload": b["config"]["workload"], "us_per_burst": b["replay_us"],
                       "achieved_GBps": b["achieved_GBps"], "separate_ops_us": b["separate_ops_us"],
                       "roofline": b["roofline"]}
        out["configs"] = extra
    return out


def bench_flow(args, dev) -> dict:
    """Side measurement: the decode step of another registered flow, its ops
    run as the package runs them (GQA: the fused GeMM + softmax + max + top-k
    kernel; Quest: one launch per op), one HIP graph per step."""
    batch = getattr(W, args.config)()
    name = FLOWS[args.flow]
    print(f"[bench] building {args.config.upper()} step of {name}: {batch.batch} requests, {args.layers} layers",
          file=sys.stderr, flush=True)
    step = DecodeStep(batch, args.layers, dev, flow_name=name)
    g = capture(step.run)
    us_step = time_graph(g, args.steps, args.warmup) * 1000.0
    plan = plan_summary(step)
    H, G, D, B = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.batch
    covered = int(plan["winfo_len"].sum())
    seg_n = np.diff(plan["dense_indptr"].astype(np.int64)) - batch.bos - batch.eos
    sel = int((seg_n > batch.topk).sum()) * batch.topk * 4
    # per covered page: its row(s) (envelopes max + min, or one centroid), its
    # page id, and the fused kernel's outputs (per-head scores + page score)
    rows_per_page = 2 if args.flow == "quest" else 1
    outs = 2 * G + 2
    per_layer = B * H * G * D * 2 + covered * (rows_per_page * 2 * D + 4 + outs) + sel
    gbps = per_layer * args.layers / (us_step * 1e-6) / 1e9
    print(f"[bench] {name} step {us_step:.1f} us", file=sys.stderr, flush=True)
    return {
        "metric": f"us per decode step of {name} (indexer + cache), side measurement",
        "value": round(us_step, 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(us_step / 1000.0, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded)",
        "config": {"workload": f"{DECODE_CONFIGS[args.config]}; flow {name}", "layers": args.layers},
        "min_bytes_per_layer": per_layer,
        "achieved_GBps_of_min_bytes": round(gbps, 1),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
    }


def bench_attention(args, dev) -> dict:
    """Side measurement: paged decode attention at C2 shapes over the sparse
    table (the indexer's selection) and over the dense table (every page)."""
    from vortex_torch import _hip
    from vortex_torch.decode_attention import dense_decode_attention, sparse_decode_attention
    from vortex_torch.indexer.utils_sglang import plan_decode

    batch = getattr(W, args.config)()
    H, G, D, P, B = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size, batch.batch
    ic, _ = W.make_contexts(batch, dev)
    db = batch.to(dev)
    plan_decode(db.seq_lens, db.req_to_token, db.req_indices, ic)
    sc = W.randn_bf16((ic.dense_kv_indices.numel(), 1, 1), 5, dev)
    _hip.topk_select(sc, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, ic.sparse_kv_indices,
                     B * H, batch.topk, batch.bos, batch.eos, batch.max_pages_per_request)
    layers = max(1, min(args.layers, 8))  # per-layer pools, far beyond the Infinity Cache
    pools = [(W.randn_bf16((batch.pool_pages * H, P, D), 11 + 2 * i, dev),
              W.randn_bf16((batch.pool_pages * H, P, D), 12 + 2 * i, dev)) for i in range(layers)]
    q = W.randn_bf16((B * H * G, D), 13, dev)
    o = torch.empty_like(q)
    out = {}
    with torch._C.DisableTorchFunctionSubclass():
        for name, fn, ip in (("sparse", sparse_decode_attention, ic.sparse_kv_indptr),
                             ("dense", dense_decode_attention, ic.dense_kv_indptr)):
            g = capture(lambda: [fn(q, k, v, ic, out=o) for k, v in pools])
            us = time_graph(g, args.steps, args.warmup) * 1000.0 / layers
            S = B * H
            pages = int(ip[S].item())
            last = ic.kv_last_page_len[:S].to(torch.int64)
            n_seg = torch.diff(ip[:S + 1].to(torch.int64))
            tokens = int(((n_seg - 1).clamp(min=0) * P + torch.where(n_seg > 0, last, torch.zeros_like(last))).sum())
            nbytes = tokens * D * 2 * 2 + pages * 4 + 2 * q.numel() * 2
            out[name] = {"us_per_layer": round(us, 2), "pages": pages, "tokens": tokens, "bytes": nbytes,
                         "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
            print(f"[bench] {name} decode attention {us:.2f} us/layer, {out[name]['GBps']} GB/s",
                  file=sys.stderr, flush=True)
    frac = out["sparse"]["GBps"] / HBM_PEAK_GBPS
    return {
        "metric": "us per layer of paged decode attention over the block table, side measurement",
        "value": out["sparse"]["us_per_layer"], "unit": "us/layer", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "higher_is_better": False, "dtype": "bf16", "data": "synthetic (seeded)",
        "config": {"workload": f"{DECODE_CONFIGS[args.config]}; decode attention, sm_scale 1/sqrt(D)"},
        "sparse": out["sparse"], "dense": out["dense"], "hbm_frac": round(frac, 4),
        "speedup_sparse_over_dense": round(out["dense"]["us_per_layer"] / out["sparse"]["us_per_layer"], 2),
    }


def traffic_probe(step: DecodeStep, dev, unfused: bool = False, cfg: str = "c2") -> dict:
    """Kernels for a counter pass: every layer's fused indexer launch (twice:
    the second pass is the one to read, the first warms the code object and
    the TLB like the timed replays), optionally the step with every op
    launched on its own (GeMV, topK, CMean), then a copy kernel of known size.
    Returns what --traffic-from needs besides the counters: the kernel's name,
    its algorithmic bytes per launch and the kernel sources' hash."""
    os.environ["VORTEX_FUSE"] = "1"
    step.run()  # the planner fills the block tables the kernels read
    nbytes = algorithmic_bytes(step.batch, plan_summary(step), step.layers, step.loc_host)
    with torch._C.DisableTorchFunctionSubclass():
        for _ in range(2):
            step.indexer_kernels_only()
    if unfused:
        os.environ["VORTEX_FUSE"] = "0"
        step.run()
        os.environ["VORTEX_FUSE"] = "1"
    with torch._C.DisableTorchFunctionSubclass():
        n = 256 << 20  # bf16 elements: 512 MiB read + 512 MiB written
        src = torch.ones(n, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    return {"probe": "traffic", "config": cfg, "kernel": fused_kernel_name(step.batch),
            "bytes_per_launch": nbytes["fused"], "sources": kernel_sources_hash(), "launches": 2 * step.layers,
            "copy_kernel": "neg (bf16)", "copy_read_bytes": 2 * n, "copy_write_bytes": 2 * n}


def traffic_from(pmc_dir: str) -> dict:
    """profiles/traffic.json from the counter passes under pmc_dir: for each
    configuration, <cfg>_fetch/ and <cfg>_write/ (rocprofv3 --pmc FETCH_SIZE,
    then WRITE_SIZE, --output-format csv, over --traffic-probe) and
    probe_<cfg>.json (that program's output line).  HBM bytes per launch =
    the median over the kernel's dispatches of FETCH_SIZE / f + WRITE_SIZE / w
    (KiB), with f and w what the counters read for the probe's copy kernel
    per byte it reads and writes."""
    import csv
    import glob
    import statistics

    def per_dispatch(path, counter):
        sums = {}
        for fn in glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(fn)):
                if r["Counter_Name"] != counter:
                    continue
                key = (r["Kernel_Name"], r["Dispatch_Id"])
                sums[key] = sums.get(key, 0.0) + float(r["Counter_Value"])
        return sums

    def short(name):
        name = name.replace("void ", "").replace("(anonymous namespace)::", "")
        return name[:name.index(">") + 1] if "<" in name else name.split("(")[0]

    out = {}
    for cfg in ("c2", "c3", "c5", "c4"):
        probe_file = os.path.join(pmc_dir, f"probe_{cfg}.json")
        if not os.path.exists(probe_file):
            continue
        probe = json.loads(open(probe_file).read().strip().splitlines()[-1])
        fetch = per_dispatch(os.path.join(pmc_dir, f"{cfg}_fetch"), "FETCH_SIZE")
        write = per_dispatch(os.path.join(pmc_dir, f"{cfg}_write"), "WRITE_SIZE")
        copy_f = [v for (k, _), v in fetch.items() if "neg" in k]
        copy_w = [v for (k, _), v in write.items() if "neg" in k]
        f = copy_f[-1] * 1024.0 / probe["copy_read_bytes"]
        w = copy_w[-1] * 1024.0 / probe["copy_write_bytes"]
        fk = [v for (k, _), v in fetch.items() if short(k) == probe["kernel"]]
        wk = [v for (k, _), v in write.items() if short(k) == probe["kernel"]]
        if not fk or not wk:
            raise SystemExit(f"{cfg}: no dispatches of {probe['kernel']} in the counter passes")
        traffic = statistics.median(fk) * 1024.0 / f + statistics.median(wk) * 1024.0 / w
        out[cfg] = {"kernel": probe["kernel"], "bytes_per_launch": probe["bytes_per_launch"],
                    "sources": probe["sources"], "traffic": int(round(traffic)),
                    "traffic_over_algorithmic": round(traffic / probe["bytes_per_launch"], 4),
                    "fetch_KiB_per_dispatch": round(statistics.median(fk), 1),
                    "write_KiB_per_dispatch": round(statistics.median(wk), 1),
                    "fetch_factor": round(f, 4), "write_factor": round(w, 4), "dispatches": len(fk)}
    with open(TRAFFIC_FILE, "w") as fh:
        json.dump(out, fh, indent=1)
        fh.write("\n")
    return out


def bench_burst(args, dev) -> dict:
    """C4: CMean + CMax of every page a chunked prefill finished."""
    from vortex_torch import cache
    from vortex_torch.abs import FORMAT, as_vtensor
    from vortex_torch.utils import ReduceType

    case = W.c4()
    H, P, D = case.num_kv_heads, case.page_size, case.head_dim
    rows = case.pool_pages * H
    print(f"[bench] building C4 burst: {case.pages.numel()} pages, {case.loc.numel()} loc entries",
          file=sys.stderr, flush=True)
    k = as_vtensor(W.randn_bf16((rows, P, D), 3, dev), FORMAT.PAGED)
    cmean = as_vtensor(torch.zeros((rows, 1, D), device=dev, dtype=torch.bfloat16), FORMAT.PAGED)
    cmax = as_vtensor(torch.zeros((rows, 1, D), device=dev, dtype=torch.bfloat16), FORMAT.PAGED)
    loc = case.loc.to(dev)
    ctx = cache.Context()
    ctx.page_size, ctx.total_num_pages, ctx.head_num, ctx.head_dim = P, case.pool_pages, H, D
    ctx.max_new_tokens_per_batch = int(loc.numel())
    ctx._created = True
    mean_op, max_op = cache.Mean(dim=1), cache.Max(dim=1)
    multi = cache.MultiReduce([ReduceType.Mean, ReduceType.Max], dim=1)
    ctx.profile()
    mean_op(k, cmean, loc=loc, ctx=ctx)
    max_op(k, cmax, loc=loc, ctx=ctx)
    multi(k, [cmean, cmax], loc=loc, ctx=ctx)
    ctx.execute()

    def fused():
        multi(k, [cmean, cmax], loc=loc, ctx=ctx)

    def separate():
        mean_op(k, cmean, loc=loc, ctx=ctx)
        max_op(k, cmax, loc=loc, ctx=ctx)

    n_tiles = case.pages.numel() * H
    k_bytes = n_tiles * P * D * 2
    fused_bytes = k_bytes + 2 * n_tiles * D * 2 + loc.numel() * 8
    separate_bytes = 2 * (k_bytes + n_tiles * D * 2 + loc.numel() * 8)
    if args.traffic_probe:
        for _ in range(2):
            fused()
        separate()
        n = 256 << 20  # bf16 elements: 512 MiB read + 512 MiB written
        src = torch.ones(n, dtype=torch.bfloat16, device=dev)
        torch.neg(src, out=torch.empty_like(src))
        torch.cuda.synchronize()
        return {"probe": "traffic", "config": "c4", "kernel": "reduce_rows_vec_kernel<16, 3>",
                "bytes_per_launch": fused_bytes, "sources": kernel_sources_hash(), "copy_kernel": "neg (bf16)",
                "copy_read_bytes": 2 * n, "copy_write_bytes": 2 * n}
    st = replay_stats(time_replays(capture(fused), args.steps, args.warmup))
    us_fused = st["median"]
    us_sep = replay_stats(time_replays(capture(separate), max(10, args.steps // 2), 3))["median"]
    gbps = fused_bytes / (us_fused * 1e-6) / 1e9
    print(f"[bench] C4 fused {us_fused:.1f} us ({gbps:.0f} GB/s), separate {us_sep:.1f} us",
          file=sys.stderr, flush=True)
    need = 1 | 2  # Sum | Max statistics
    c4_traffic, c4_note = traffic_for("c4", f"reduce_rows_vec_kernel<16, {need}>", fused_bytes)
    out = {
        "metric": "us per page-finish burst (CMean + CMax) and achieved HBM GB/s",
        "value": round(us_fused, 2),
        "unit": "us/burst",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_fused / 1000.0, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded; K ~ N(0,1) bf16, pages and loc order seeded permutations)",
        "config": {"workload": "C4: page-finish burst, 65,536 pages x 8 heads (1,048,576 loc entries) "
                               "of a 70k-page pool, D 128, page 16, CMean + CMax bf16 outputs",
                   "pages": int(case.pages.numel()), "loc_entries": int(loc.numel())},
        "replay_us": st,
        "achieved_GBps": round(gbps, 1),
        "separate_ops_us": round(us_sep, 2),
        "separate_ops_GBps": round(separate_bytes / (us_sep * 1e-6) / 1e9, 1),
        "roofline": {
            "kernel": f"reduce_rows_vec_kernel<16, {need}> (CMean + CMax, one pass over K)",
            "bound": "hbm",
            "achieved": round(gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": c4_traffic,
            "us_per_launch": us_fused,
            "bytes_per_launch": fused_bytes,
        },
    }
    if c4_note:
        out["roofline"]["traffic_note"] = c4_note
    return out


def main():
    args = _parse()
    if args.traffic_from:
        print(json.dumps(traffic_from(args.traffic_from)))
        return
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
    if args.config == "c4":
        out = bench_burst(args, dev)
    elif args.attention:
        out = bench_attention(args, dev)
    elif args.flow != "block_sparse":
        out = bench_flow(args, dev)
    else:
        out = bench_decode(args, dev)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
