"""Seeded synthetic workloads of the configurations in BASELINE.json.

Used by the parity tests and by bench.py.  Small integer data (lengths, block
tables) is drawn on the CPU from a seeded ``torch.Generator`` so that every
device sees the same tables; large float pools are drawn on the target
device from a device generator with the same seed.

C1  1 request x 4096 tokens, GQA 16/8, D 128, topk 30 (+1 BOS +1 EOS), 512-page pool
C2  64 requests, L ~ U[1024, 8192], 27 sparse layers, shared shuffled 40k-page pool
C3  8 requests x 32768 tokens, topk 64, per-page offsets N(0, 0.5) + N(0, 1) noise
C4  page-finish burst: 65,536 pages scattered over a 70k-page pool, CMean + CMax
C5  MLA latent cache: 1 head, G 16, D 576, 32 requests L ~ U[4096, 16384], topk 32
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch


@dataclass
class DecodeBatch:
    """One decode step's request layout and indexer configuration."""

    seq_lens: torch.Tensor      # int32 [B]
    req_to_token: torch.Tensor  # int32 [R, T]: token -> pool slot
    req_indices: torch.Tensor   # int64 [B]: row of req_to_token per request
    pages: list                 # per request: int64 tensor of physical page ids
    pool_pages: int
    page_size: int = 16
    num_kv_heads: int = 8
    group_size: int = 2
    head_dim: int = 128
    topk: int = 30
    bos: int = 1
    eos: int = 1
    max_chunk: int = 64
    min_chunk: int = 16
    extra: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return int(self.seq_lens.shape[0])

    @property
    def n_pages(self) -> torch.Tensor:
        return (self.seq_lens.to(torch.int64) + self.page_size - 1) // self.page_size

    @property
    def max_pages_per_request(self) -> int:
        return (int(self.req_to_token.shape[1]) + self.page_size - 1) // self.page_size

    def to(self, device) -> "DecodeBatch":
        out = DecodeBatch(**{k: getattr(self, k) for k in self.__dataclass_fields__})
        out.seq_lens = self.seq_lens.to(device)
        out.req_to_token = self.req_to_token.to(device)
        out.req_indices = self.req_indices.to(device)
        return out

    # buffer sizes a serving runtime would allocate for this batch
    def dense_capacity(self) -> int:
        return int(self.n_pages.sum()) * self.num_kv_heads

    def sparse_capacity(self) -> int:
        budget = self.topk + self.bos + self.eos
        return int(torch.clamp(self.n_pages, max=budget).sum()) * self.num_kv_heads

    def workload_capacity(self) -> int:
        return self.dense_capacity() // max(1, self.min_chunk) + self.batch * self.num_kv_heads


def make_batch(seq_lens, pool_pages: int, seed: int, page_size: int = 16, spare_rows: int = 2,
               row_tokens: Optional[int] = None, **cfg) -> DecodeBatch:
    """Requests take consecutive slices of one shuffled pool of pages; the
    req_to_token rows are placed in a shuffled order (req_indices)."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.as_tensor(seq_lens, dtype=torch.int64)
    B = int(lens.shape[0])
    P = page_size
    n = (lens + P - 1) // P
    total = int(n.sum())
    if total > pool_pages:
        raise ValueError(f"pool of {pool_pages} pages cannot hold {total} pages")
    perm = torch.randperm(pool_pages, generator=g)
    T = row_tokens if row_tokens is not None else max(P, int(((int(lens.max()) if B else 0) + P - 1) // P * P))
    R = B + spare_rows
    rows = torch.randperm(R, generator=g)[:B]
    r2t = torch.zeros((R, T), dtype=torch.int32)
    pages = []
    off = 0
    tok = torch.arange(T, dtype=torch.int64)
    for b in range(B):
        pg = perm[off:off + int(n[b])]
        off += int(n[b])
        pages.append(pg)
        L = int(lens[b])
        if L:
            r2t[rows[b], :L] = (pg[tok[:L] // P] * P + tok[:L] % P).to(torch.int32)
    return DecodeBatch(seq_lens=lens.to(torch.int32), req_to_token=r2t, req_indices=rows.to(torch.int64),
                       pages=pages, pool_pages=pool_pages, page_size=P, **cfg)


def c1() -> DecodeBatch:
    return make_batch([4096], pool_pages=512, seed=0, num_kv_heads=8, group_size=2, head_dim=128,
                      topk=30, bos=1, eos=1)


def c2(seed: int = 1) -> DecodeBatch:
    g = torch.Generator().manual_seed(seed + 1000)
    lens = torch.randint(1024, 8193, (64,), generator=g)
    return make_batch(lens, pool_pages=40000, seed=seed, num_kv_heads=8, group_size=2, head_dim=128,
                      topk=30, bos=1, eos=1, row_tokens=8192, extra={"layers": 27})


def c3(seed: int = 2) -> DecodeBatch:
    """C3: 8 x 32k tokens, top-64.  extra["k_page_offsets"]: its K pool carries
    a per-(page, head) offset ~ N(0, 0.5) over N(0, 1) noise (k_pool) and its
    centroids are that pool's CMean (centroids_from_k), as configured."""
    return make_batch([32768] * 8, pool_pages=20000, seed=seed, num_kv_heads=8, group_size=2,
                      head_dim=128, topk=64, bos=1, eos=1, row_tokens=32768, extra={"k_page_offsets": True})


def c5(seed: int = 4) -> DecodeBatch:
    g = torch.Generator().manual_seed(seed + 1000)
    lens = torch.randint(4096, 16385, (32,), generator=g)
    return make_batch(lens, pool_pages=32 * 1024 + 1024, seed=seed, num_kv_heads=1, group_size=16,
                      head_dim=576, topk=32, bos=1, eos=1, row_tokens=16384)


@dataclass
class BurstCase:
    """A page-finish burst: every slot of `pages` appears in loc (shuffled)."""

    loc: torch.Tensor    # int64 [pages * page_size]
    pages: torch.Tensor  # int64 [n] physical pages that close
    pool_pages: int
    page_size: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128


def c4(seed: int = 3, pool_pages: int = 70000, n_pages: int = 65536) -> BurstCase:
    """C4: 65,536 pages of a 70k-page pool finish at once (after a chunked
    prefill); loc lists all 16 slots of each, in shuffled order."""
    g = torch.Generator().manual_seed(seed)
    pages = torch.randperm(pool_pages, generator=g)[:n_pages]
    P = 16
    slots = (pages[:, None] * P + torch.arange(P)[None, :]).reshape(-1)
    loc = slots[torch.randperm(slots.numel(), generator=g)]
    return BurstCase(loc=loc.to(torch.int64), pages=pages.to(torch.int64), pool_pages=pool_pages, page_size=P)


def random_small(seed: int) -> DecodeBatch:
    """Small random layout with edge cases (empty requests, exact page
    multiples, segments shorter than the budget, bos/eos 0)."""
    g = torch.Generator().manual_seed(seed)
    B = int(torch.randint(1, 7, (1,), generator=g))
    P = [1, 4, 16][int(torch.randint(0, 3, (1,), generator=g))]
    H = [1, 2, 3, 8][int(torch.randint(0, 4, (1,), generator=g))]
    topk = [1, 3, 8, 30][int(torch.randint(0, 4, (1,), generator=g))]
    bos = int(torch.randint(0, 3, (1,), generator=g))
    eos = int(torch.randint(0, 3, (1,), generator=g))
    lens = []
    for _ in range(B):
        kind = int(torch.randint(0, 5, (1,), generator=g))
        if kind == 0:
            lens.append(0)
        elif kind == 1:
            lens.append(P * int(torch.randint(1, 40, (1,), generator=g)))
        elif kind == 2:
            lens.append(int(torch.randint(1, (topk + bos + eos + 1) * P + 1, (1,), generator=g)))
        else:
            lens.append(int(torch.randint(1, 1200, (1,), generator=g)))
    n_total = sum((L + P - 1) // P for L in lens)
    chunk = [4, 16, 64, 100][int(torch.randint(0, 4, (1,), generator=g))]
    return make_batch(lens, pool_pages=n_total + 7, seed=seed, page_size=P, num_kv_heads=H,
                      group_size=2, head_dim=128, topk=topk, bos=bos, eos=eos, max_chunk=chunk,
                      min_chunk=max(1, chunk // 4))


def make_contexts(batch: DecodeBatch, device):
    """Indexer and cache contexts sized for `batch`, as a serving runtime
    would populate them (buffers on `device`, execute mode not yet set)."""
    from vortex_torch.cache import Context as CContext
    from vortex_torch.indexer import Context as IContext

    H, G, D, P, B = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size, batch.batch
    i32 = dict(dtype=torch.int32, device=device)
    ic = IContext()
    ic.dense_kv_indptr = torch.zeros(B * H + 1, **i32)
    ic.sparse_kv_indptr = torch.zeros(B * H + 1, **i32)
    ic.dense_kv_indices = torch.zeros(max(1, batch.dense_capacity()), **i32)
    ic.sparse_kv_indices = torch.full((max(1, batch.sparse_capacity()),), -1, **i32)
    ic.kv_last_page_len = torch.zeros(max(1, B * H), **i32)
    nw = batch.workload_capacity()
    ic.winfo_q_indices = torch.zeros(nw, **i32)
    ic.winfo_kv_offsets = torch.zeros(nw, **i32)
    ic.winfo_kv_lens = torch.zeros(nw, **i32)
    ic.winfo_num_workloads = torch.zeros(1, **i32)
    ic.winfo_chunk_size = torch.zeros(1, **i32)
    ic.max_num_workloads = nw
    ic.max_chunk_size, ic.min_chunk_size = batch.max_chunk, batch.min_chunk
    ic.group_size, ic.num_kv_heads, ic.num_qo_heads, ic.head_dim = G, H, G * H, D
    dev = torch.device(device)
    ic.num_sms = torch.cuda.get_device_properties(dev).multi_processor_count if dev.type == "cuda" else 1
    ic.page_size = P
    ic.max_num_pages = max(1, batch.dense_capacity())
    ic.max_num_pages_per_request = batch.max_pages_per_request
    ic.topk_val, ic.page_reserved_bos, ic.page_reserved_eos = batch.topk, batch.bos, batch.eos
    ic._fused_schedule = torch.zeros(4 + 4 * B * H, **i32)
    ic._created = True
    cc = CContext()
    cc.page_size, cc.total_num_pages, cc.head_num, cc.head_dim = P, batch.pool_pages, H, D
    cc.max_new_tokens_per_batch = max(B, 1)
    cc._created = True
    return ic, cc


def decode_loc(batch: DecodeBatch):
    """Pool slot of every request's newest token (position L-1)."""
    P = batch.page_size
    out = []
    for b in range(batch.batch):
        j = int(batch.seq_lens[b]) - 1
        out.append(int(batch.pages[b][j // P]) * P + j % P if j >= 0 else 0)
    return torch.as_tensor(out, dtype=torch.int64)


# ---------------------------------------------------------------- float data
def randn_bf16(shape, seed: int, device, std: float = 1.0) -> torch.Tensor:
    g = torch.Generator(device=device).manual_seed(seed)
    t = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if std != 1.0:
        t.mul_(std)
    return t.to(torch.bfloat16)


def k_pool(batch: DecodeBatch, seed: int, device, page_offsets: bool = False) -> torch.Tensor:
    """bf16 K pool [pool_pages * H, P, D] ~ N(0,1); with page_offsets a
    per-(page, head) vector ~ N(0, 0.5) is added to all tokens of the page."""
    H, P, D = batch.num_kv_heads, batch.page_size, batch.head_dim
    k = torch.randn((batch.pool_pages * H, P, D), generator=torch.Generator(device=device).manual_seed(seed),
                    device=device, dtype=torch.float32)
    if page_offsets:
        off = torch.randn((batch.pool_pages * H, 1, D), generator=torch.Generator(device=device).manual_seed(seed + 1),
                          device=device, dtype=torch.float32) * (0.5 ** 0.5)
        k.add_(off)
    return k.to(torch.bfloat16)


def centroids_from_k(k: torch.Tensor, batch: DecodeBatch) -> torch.Tensor:
    """The centroid pool [pool_pages * H, 1, D] bf16 of a K pool: the package's
    CMean (the page-reduce kernel) over every page of the pool, one loc entry
    per page (its last slot), as the cache side writes them page by page."""
    from vortex_torch import _hip

    H, P, D = batch.num_kv_heads, batch.page_size, batch.head_dim
    cen = torch.zeros((batch.pool_pages * H, 1, D), device=k.device, dtype=torch.bfloat16)
    loc = torch.arange(batch.pool_pages, device=k.device, dtype=torch.int64) * P + (P - 1)
    _hip.page_reduce(k, cen, loc, H, P, 1, _hip.REDUCE_MEAN)
    return cen


def cmean_case(name: str):
    """(batch, loc) for a fused launch that runs the layer's CMean: decode
    configurations and layouts where the closed pages are scored (eos 0, or
    loc slots closing middle pages), plus the cases that fall back to a
    page-reduce launch of their own (more loc entries than one launch scans,
    head_dim 256)."""
    if name == "eos0":  # every request's last page closes and is a middle page (eos 0)
        b = make_batch([1024, 2048, 640, 4096, 512], pool_pages=900, seed=21, eos=0, topk=12)
        return b, decode_loc(b)
    if name == "mid":  # closing slots of middle pages, several per request
        b = make_batch([3000, 5000, 1800], pool_pages=700, seed=22, topk=20)
        g = torch.Generator().manual_seed(5)
        slots = []
        for pages in b.pages:
            pick = torch.randperm(len(pages) - 2, generator=g)[:9] + 1
            slots += [int(pages[i]) * b.page_size + b.page_size - 1 for i in pick]
        slots += [7, 16 * 3 + 2]  # tokens that close nothing
        return b, torch.as_tensor(slots, dtype=torch.int64)
    if name == "d64":
        b = make_batch([3000, 1500, 700], pool_pages=400, seed=23, head_dim=64, group_size=1, eos=0)
        return b, decode_loc(b)
    if name == "big_loc":  # more loc entries than one launch scans: CMean launched first
        b = make_batch([4096, 4096], pool_pages=600, seed=24)
        return b, torch.arange(300, dtype=torch.int64) * 3
    if name == "d576":  # MLA rows (one latent head of 576), eos 0: closed pages are scored
        b = make_batch([4096, 5000, 2048, 3072], pool_pages=1200, seed=26, num_kv_heads=1, group_size=16,
                       head_dim=576, topk=32, bos=1, eos=0)
        return b, decode_loc(b)
    if name == "d576many":  # MLA rows, 256 loc entries each closing a different page (scored ones
        # among them): more CMean work units than the split launch's tile workgroups have waves
        b = make_batch([4096, 5000, 2048, 3072], pool_pages=1200, seed=27, num_kv_heads=1, group_size=16,
                       head_dim=576, topk=32, bos=1, eos=0)
        g = torch.Generator().manual_seed(9)
        pages = torch.cat([torch.as_tensor(p, dtype=torch.int64) for p in b.pages])
        pick = pages[torch.randperm(pages.numel(), generator=g)[:256]]
        return b, pick * b.page_size + b.page_size - 1
    if name == "d256":  # wider rows
        b = make_batch([2000, 3000], pool_pages=400, seed=25, head_dim=256, eos=0)
        return b, decode_loc(b)
    if name.startswith("r"):
        b = random_small(int(name[1:]))
        return b, decode_loc(b)
    b = globals()[name]()
    return b, decode_loc(b)
