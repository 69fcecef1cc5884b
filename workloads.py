"""Seeded inputs and work accounting for the five BASELINE.json configs.

Shared by bench.py, tests/ and __graft_entry__.  Inputs are generated on the
CPU with ``torch.Generator().manual_seed(seed)`` (values ``randn`` in fp32,
then cast), so the same bits reach every device.  Packing helpers build the
three layouts of ``flash_attention_v2`` from per-sequence ``[L,H,D]``
tensors the way the reference test suite does (tests/test_attention.py:
159-243), plus the shuffled-pool / ``-1``-padded paged cache of the
reference benchmark (benchmarks/attention.py:351-431) with independent K and
V page permutations.

c1  dense causal MHA      1x8x512x64 fp16
c2  dense causal GQA      B2 Hq32 Hkv8 L2048 D128 (fp16, bf16)
c3  ragged causal self    16 seqs, L ~ U[128,4096], Hq32 Hkv8 D128 bf16
c4  paged chunked prefill 32 seqs, ctx ~ U[512,8192], page 16, shuffled pool
                          of ceil(sum/16)+256 pages, q = last 128 tokens
                          (bottom-right causal), Hq32 Hkv8 D128 bf16
c5  non-causal MQA cross  B4 Hq32 Hkv1 q1024 kv16384 D128 bf16 (+fp32 run)

Decode-side workloads (not BASELINE configs; HBM-bound, reported in GB/s):
d1  paged decode_attention at the reference decode benchmark's largest
    point (benchmarks/decode.py:30-44, 170-230): B16, QH8/KVH8, N 8192, D64,
    page 16, bf16
d2  paged decode_attention, serving shape: 64 seqs, ctx ~ U[512,8192],
    shuffled pool of ceil(sum/16)+256 pages, Hq32 Hkv8 D128 bf16
s1  paged speculative_decode_attention, causal, M 8 drafts, at the
    reference benchmark's shape (benchmarks/speculative_decode.py:29-50):
    B16, QH8/KVH8, N 8192 + 8 drafts, D64, page 16, bf16
s2  paged speculative_decode_attention, causal, M 8, serving shape of d2
    (context + 8 drafts per sequence), Hq32 Hkv8 D128 bf16
a1  paged_kv_append: write c4's whole context (32 seqs, ctx ~ U[512,8192],
    Hkv8 D128 bf16) into its shuffled K and V page pools (a prefill's cache
    fill); HBM-bound copy, reported in GB/s of bytes read + written
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

CONFIGS = ("c1", "c2", "c3", "c4", "c5", "d1", "d2", "s1", "s2", "a1")
PAGE = 16


@dataclass
class Workload:
    name: str
    layout: str                 # dense | ragged | paged
    dtype: torch.dtype
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    is_causal: bool
    causal_alignment: str = "top_left"
    q_indptr: torch.Tensor | None = None
    kv_indptr: torch.Tensor | None = None
    k_block_table: torch.Tensor | None = None
    v_block_table: torch.Tensor | None = None
    kv_page_size: int | None = None
    q_lens: list = field(default_factory=list)
    kv_lens: list = field(default_factory=list)
    q_heads: int = 0
    kv_heads: int = 0
    head_dim: int = 0
    kind: str = "prefill"       # prefill (flash_attention_v2) | decode | speculative | append
    k_new: torch.Tensor | None = None     # append: rows to write [T, Hkv, D]
    v_new: torch.Tensor | None = None
    new_indptr: torch.Tensor | None = None

    def kwargs(self) -> dict:
        if self.kind == "decode":
            kw = {}
        elif self.kind == "speculative":
            kw = dict(causal=self.is_causal)
        else:
            kw = dict(is_causal=self.is_causal)
            if self.causal_alignment != "top_left":
                kw["causal_alignment"] = self.causal_alignment
        for n in ("q_indptr", "kv_indptr", "k_block_table", "v_block_table", "kv_page_size"):
            val = getattr(self, n)
            if val is not None:
                kw[n] = val
        return kw

    def to(self, device) -> "Workload":
        out = Workload(**{f: getattr(self, f) for f in self.__dataclass_fields__})
        for n in ("q", "k", "v", "q_indptr", "kv_indptr", "k_block_table", "v_block_table",
                  "k_new", "v_new", "new_indptr"):
            t = getattr(out, n)
            if t is not None:
                setattr(out, n, t.to(device))
        return out


# ---------------------------------------------------------------------------
# algorithmic work
# ---------------------------------------------------------------------------

def visible_pairs(Lq: int, Lk: int, is_causal: bool, alignment: str = "top_left") -> int:
    """Number of (query, key) pairs the mask admits."""
    if not is_causal:
        return Lq * Lk
    off = (Lk - Lq) if alignment == "bottom_right" else 0
    total = 0
    # rows i with i + off + 1 keys, clipped to [0, Lk]
    for i in range(Lq):
        total += min(max(i + off + 1, 0), Lk)
    return total


def flops(w: Workload) -> float:
    """4 * D * Hq * sum of visible pairs (QK^T and PV, 2 FLOP per MAC)."""
    if w.kind == "append":
        return 0.0
    pairs = sum(visible_pairs(lq, lk, w.is_causal, w.causal_alignment)
                for lq, lk in zip(w.q_lens, w.kv_lens))
    return 4.0 * w.head_dim * w.q_heads * pairs


def hbm_bytes(w: Workload) -> float:
    """Q and O once at Hq, K and V once at Hkv (tokens actually attended);
    append: the new K and V rows read once and written once."""
    es = torch.tensor([], dtype=w.dtype).element_size()
    if w.kind == "append":
        return 2.0 * 2 * es * w.k_new.numel()
    if w.kind != "prefill":
        sq = sum(w.q_lens)
    else:
        sq = sum(w.q_lens) if w.layout == "ragged" else w.q.shape[0] * w.q.shape[2]
    sk = sum(w.kv_lens)
    return es * w.head_dim * (2 * sq * w.q_heads + 2 * sk * w.kv_heads)


# ---------------------------------------------------------------------------
# packing (per-sequence [L,H,D] -> layouts)
# ---------------------------------------------------------------------------

def pack_dense(seqs, L: int) -> torch.Tensor:
    """[L_b,H,D] list -> zero-padded [B,H,L,D] (tests/test_attention.py:159-170)."""
    B, H, D = len(seqs), seqs[0].shape[1], seqs[0].shape[2]
    out = torch.zeros((B, H, L, D), dtype=seqs[0].dtype, device=seqs[0].device)
    for b, s in enumerate(seqs):
        out[b, :, : s.shape[0]] = s.transpose(0, 1)
    return out


def indptr(lens, device="cpu") -> torch.Tensor:
    return torch.tensor([0] + list(lens), dtype=torch.int32, device=device).cumsum(0).to(torch.int32)


def paged_cache_contiguous(seqs, page: int):
    """Reference test construction (tests/test_attention.py:101-134): pages in
    sequence order, tail slots zero, unused table entries 0."""
    lens = [s.shape[0] for s in seqs]
    H, D = seqs[0].shape[1], seqs[0].shape[2]
    nb = [(n + page - 1) // page for n in lens]
    cache = torch.zeros((sum(nb) * page, H, D), dtype=seqs[0].dtype)
    table = torch.zeros((len(seqs), max(nb) if nb else 0), dtype=torch.int32)
    cur = 0
    for b, s in enumerate(seqs):
        for j in range(nb[b]):
            table[b, j] = cur
            chunk = s[j * page: min((j + 1) * page, lens[b])]
            cache[cur * page: cur * page + chunk.shape[0]] = chunk
            cur += 1
    return cache, table


def paged_cache_shuffled(seqs, page: int, extra_pages: int, gen: torch.Generator,
                         fill: float | None = None):
    """Pool of ceil(sum/page)+extra pages in a random order, table padded with
    -1 (benchmarks/attention.py:415-420).  Unused pool slots hold ``fill``
    (NaN by default, so a read outside the table shows up in the output)."""
    lens = [s.shape[0] for s in seqs]
    H, D = seqs[0].shape[1], seqs[0].shape[2]
    nb = [(n + page - 1) // page for n in lens]
    pool = sum(nb) + extra_pages
    perm = torch.randperm(pool, generator=gen)
    cache = torch.full((pool * page, H, D), float("nan") if fill is None else fill,
                       dtype=seqs[0].dtype)
    table = torch.full((len(seqs), max(nb) if nb else 0), -1, dtype=torch.int32)
    cur = 0
    for b, s in enumerate(seqs):
        for j in range(nb[b]):
            pg = int(perm[cur])
            cur += 1
            table[b, j] = pg
            chunk = s[j * page: min((j + 1) * page, lens[b])]
            cache[pg * page: pg * page + chunk.shape[0]] = chunk
            if chunk.shape[0] < page:
                cache[pg * page + chunk.shape[0]: (pg + 1) * page] = 0
    return cache, table


def gather_paged(cache, table, lens, page):
    """Inverse of the paged construction: list of [L_b,H,D] sequences."""
    out = []
    for b, n in enumerate(lens):
        rows = [int(table[b, j // page]) * page + j % page for j in range(n)]
        out.append(cache[rows])
    return out


# ---------------------------------------------------------------------------
# BASELINE configs
# ---------------------------------------------------------------------------

def _randn(gen, shape, dtype):
    return torch.randn(shape, generator=gen, dtype=torch.float32).to(dtype)


def make(name: str, dtype: torch.dtype | None = None, seed: int = 0,
         causal_alignment: str | None = None) -> Workload:
    """Build config ``name`` on the CPU.  ``dtype`` overrides the default."""
    gen = torch.Generator().manual_seed(seed)
    if name == "c1":
        dt = dtype or torch.float16
        B, H, L, D = 1, 8, 512, 64
        q, k, v = (_randn(gen, (B, H, L, D), dt) for _ in range(3))
        return Workload("c1", "dense", dt, q, k, v, True, q_lens=[L] * B, kv_lens=[L] * B,
                        q_heads=H, kv_heads=H, head_dim=D)
    if name == "c2":
        dt = dtype or torch.bfloat16
        B, Hq, Hkv, L, D = 2, 32, 8, 2048, 128
        q = _randn(gen, (B, Hq, L, D), dt)
        k = _randn(gen, (B, Hkv, L, D), dt)
        v = _randn(gen, (B, Hkv, L, D), dt)
        return Workload("c2", "dense", dt, q, k, v, True, q_lens=[L] * B, kv_lens=[L] * B,
                        q_heads=Hq, kv_heads=Hkv, head_dim=D)
    if name == "c3":
        dt = dtype or torch.bfloat16
        Hq, Hkv, D = 32, 8, 128
        lens = torch.randint(128, 4097, (16,), generator=gen).tolist()
        T = sum(lens)
        q = _randn(gen, (T, Hq, D), dt)
        k = _randn(gen, (T, Hkv, D), dt)
        v = _randn(gen, (T, Hkv, D), dt)
        ip = indptr(lens)
        return Workload("c3", "ragged", dt, q, k, v, True, q_indptr=ip, kv_indptr=ip.clone(),
                        q_lens=lens, kv_lens=lens, q_heads=Hq, kv_heads=Hkv, head_dim=D)
    if name == "c4":
        dt = dtype or torch.bfloat16
        B, Hq, Hkv, D, QL = 32, 32, 8, 128, 128
        ctx = torch.randint(512, 8193, (B,), generator=gen).tolist()
        nb = [(c + PAGE - 1) // PAGE for c in ctx]
        pool = sum(nb) + 256
        width = max(nb)
        # physical caches filled directly (every pool slot random), then two
        # independent page permutations give the K and V tables
        kc = _randn(gen, (pool * PAGE, Hkv, D), dt)
        vc = _randn(gen, (pool * PAGE, Hkv, D), dt)
        kperm = torch.randperm(pool, generator=gen)
        vperm = torch.randperm(pool, generator=gen)
        kt = torch.full((B, width), -1, dtype=torch.int32)
        vt = torch.full((B, width), -1, dtype=torch.int32)
        cur = 0
        for b in range(B):
            kt[b, : nb[b]] = kperm[cur: cur + nb[b]].to(torch.int32)
            vt[b, : nb[b]] = vperm[cur: cur + nb[b]].to(torch.int32)
            cur += nb[b]
        q = _randn(gen, (B, Hq, QL, D), dt)
        lens_t = torch.tensor(ctx, dtype=torch.int32)
        return Workload("c4", "paged", dt, q, kc, vc, True,
                        causal_alignment=causal_alignment or "bottom_right",
                        kv_indptr=lens_t, k_block_table=kt, v_block_table=vt, kv_page_size=PAGE,
                        q_lens=[QL] * B, kv_lens=ctx, q_heads=Hq, kv_heads=Hkv, head_dim=D)
    if name == "c5":
        dt = dtype or torch.bfloat16
        B, Hq, Hkv, M, N, D = 4, 32, 1, 1024, 16384, 128
        q = _randn(gen, (B, Hq, M, D), dt)
        k = _randn(gen, (B, Hkv, N, D), dt)
        v = _randn(gen, (B, Hkv, N, D), dt)
        return Workload("c5", "dense", dt, q, k, v, False, q_lens=[M] * B, kv_lens=[N] * B,
                        q_heads=Hq, kv_heads=Hkv, head_dim=D)
    if name in ("d1", "d2", "s1", "s2"):
        return _make_decode(name, dtype or torch.bfloat16, gen)
    if name == "a1":
        c4 = make("c4", dtype=dtype, seed=seed)
        T = sum(c4.kv_lens)
        g2 = torch.Generator().manual_seed(seed + 1)
        kn = _randn(g2, (T, c4.kv_heads, c4.head_dim), c4.dtype)
        vn = _randn(g2, (T, c4.kv_heads, c4.head_dim), c4.dtype)
        return Workload("a1", "paged", c4.dtype, c4.q, torch.zeros_like(c4.k),
                        torch.zeros_like(c4.v), False, kv_indptr=c4.kv_indptr,
                        k_block_table=c4.k_block_table, v_block_table=c4.v_block_table,
                        kv_page_size=PAGE, q_lens=[0] * len(c4.kv_lens), kv_lens=c4.kv_lens,
                        q_heads=c4.q_heads, kv_heads=c4.kv_heads, head_dim=c4.head_dim,
                        kind="append", k_new=kn, v_new=vn, new_indptr=indptr(c4.kv_lens))
    raise KeyError(name)


def spread_pool(w: Workload, gib: float, seed: int = 1) -> Workload:
    """The same paged workload with its pages moved into pools of at least
    `gib` GiB each: every used page goes to a random slot among the pool's
    last 4x-its-page-count slots (all past the 2 GiB mark once `gib` exceeds 2
    plus that span), the tables are remapped, the other slots hold zeros.  Every sequence sees the same K/V rows in the same
    order, so the output must equal the compact pool's bit for bit."""
    assert w.layout == "paged"
    row_bytes = w.k[0].numel() * w.k.element_size()
    page_bytes = w.kv_page_size * row_bytes
    old_pages = w.k.shape[0] // w.kv_page_size
    pages = max(old_pages, -(-int(gib * (1 << 30)) // page_bytes))
    gen = torch.Generator().manual_seed(seed)

    def move(cache, table):
        span = min(pages, 4 * old_pages)
        dst = pages - span + torch.randperm(span, generator=gen)[:old_pages]
        big = torch.zeros((pages * w.kv_page_size,) + tuple(cache.shape[1:]), dtype=cache.dtype)
        big.view(pages, w.kv_page_size, -1)[dst] = cache.view(old_pages, w.kv_page_size, -1)
        t = table.clone().long()
        used = t >= 0
        t[used] = dst[t[used]]
        return big, t.to(torch.int32)

    kc, kt = move(w.k, w.k_block_table)
    vc, vt = move(w.v, w.v_block_table)
    out = Workload(**{f: getattr(w, f) for f in w.__dataclass_fields__})
    out.k, out.v, out.k_block_table, out.v_block_table = kc, vc, kt, vt
    return out


# The reference benchmark's sweep (benchmarks/attention.py:11-55, 487-589):
# B 16, D 128, page 16; layouts x self/cross x MHA 8/8, GQA 8/2, MQA 8/1 x
# fp16/bf16 x causal; q_len in {128, 512}; kv_len = q_len (self) or in
# {128, 512, 2048} (cross); causal points with q_len > kv_len skipped (:505-506).
SWEEP_BATCH, SWEEP_D = 16, 128
SWEEP_TOPOLOGIES = {"mha": (8, 8), "gqa": (8, 2), "mqa": (8, 1)}


def sweep_points():
    """(layout, attn_type, topology, dtype, causal, q_len, kv_len) in the
    reference benchmark's loop order."""
    pts = []
    for layout in ("dense", "ragged", "paged"):
        for attn in ("self", "cross"):
            for topo in SWEEP_TOPOLOGIES:
                for dt in (torch.float16, torch.bfloat16):
                    for causal in (False, True):
                        for ql in (128, 512):
                            for kl in ((128, 512, 2048) if attn == "cross" else (ql,)):
                                if causal and ql > kl:
                                    continue
                                pts.append((layout, attn, topo, dt, causal, ql, kl))
    return pts


def make_sweep(layout, attn_type, topology, dtype, causal, q_len, kv_len, seed=0) -> Workload:
    """One point of the reference benchmark's sweep with seeded inputs.  Every
    sequence has q_len queries and kv_len keys (benchmarks/attention.py:244-270);
    paged caches are built like its build_paged_cache (pages in order, -1
    padding, :351-431), with q laid out [B, Hq, q_len, D] as the entry point
    reads it (the benchmark passes it transposed, :449).  kv_len is a
    multiple of the page size at every point."""
    gen = torch.Generator().manual_seed(seed)
    Hq, Hkv = SWEEP_TOPOLOGIES[topology]
    B, D = SWEEP_BATCH, SWEEP_D
    if attn_type == "self":
        kv_len = q_len
    name = f"sweep {layout} {attn_type} {topology} {'causal' if causal else 'full'} q{q_len} kv{kv_len}"
    qs = [_randn(gen, (q_len, Hq, D), dtype) for _ in range(B)]
    ks = [_randn(gen, (kv_len, Hkv, D), dtype) for _ in range(B)]
    vs = [_randn(gen, (kv_len, Hkv, D), dtype) for _ in range(B)]
    common = dict(q_lens=[q_len] * B, kv_lens=[kv_len] * B, q_heads=Hq, kv_heads=Hkv,
                  head_dim=D)
    if layout == "dense":
        return Workload(name, "dense", dtype, pack_dense(qs, q_len), pack_dense(ks, kv_len),
                        pack_dense(vs, kv_len), causal, **common)
    if layout == "ragged":
        return Workload(name, "ragged", dtype, torch.cat(qs), torch.cat(ks), torch.cat(vs),
                        causal, q_indptr=indptr([q_len] * B), kv_indptr=indptr([kv_len] * B),
                        **common)
    # equal lengths: every table row is full, as build_paged_cache's would be
    kc, kt = paged_cache_contiguous(ks, PAGE)
    vc, vt = paged_cache_contiguous(vs, PAGE)
    return Workload(name, "paged", dtype, pack_dense(qs, q_len), kc, vc, causal,
                    kv_indptr=torch.tensor([kv_len] * B, dtype=torch.int32), k_block_table=kt,
                    v_block_table=vt, kv_page_size=PAGE, **common)


def _make_decode(name, dt, gen) -> Workload:
    """Paged decode / speculative-decode workloads (see the module docstring)."""
    spec = name.startswith("s")
    M = 8 if spec else 1
    if name in ("d1", "s1"):
        B, Hq, Hkv, D = 16, 8, 8, 64
        ctx = [8192] * B
    else:
        B, Hq, Hkv, D = 64, 32, 8, 128
        ctx = torch.randint(512, 8193, (B,), generator=gen).tolist()
    lens = [c + (M if spec else 0) for c in ctx]  # drafts are the last M keys
    nb = [(n + PAGE - 1) // PAGE for n in lens]
    pool = sum(nb) + (256 if name in ("d2", "s2") else 0)
    kc = _randn(gen, (pool * PAGE, Hkv, D), dt)
    vc = _randn(gen, (pool * PAGE, Hkv, D), dt)
    if name in ("d2", "s2"):
        kperm = torch.randperm(pool, generator=gen)
        vperm = torch.randperm(pool, generator=gen)
        pad = -1
    else:  # the reference benchmark's allocate_paged_cache: pages in order, padding 0
        kperm = vperm = torch.arange(pool)
        pad = 0
    kt = torch.full((B, max(nb)), pad, dtype=torch.int32)
    vt = torch.full((B, max(nb)), pad, dtype=torch.int32)
    cur = 0
    for b in range(B):
        kt[b, : nb[b]] = kperm[cur: cur + nb[b]].to(torch.int32)
        vt[b, : nb[b]] = vperm[cur: cur + nb[b]].to(torch.int32)
        cur += nb[b]
    q = _randn(gen, (B, Hq, M, D) if spec else (B, Hq, D), dt)
    return Workload(name, "paged", dt, q, kc, vc, spec,
                    causal_alignment="bottom_right" if spec else "top_left",
                    kv_indptr=torch.tensor(lens, dtype=torch.int32), k_block_table=kt,
                    v_block_table=vt, kv_page_size=PAGE, q_lens=[M] * B, kv_lens=lens,
                    q_heads=Hq, kv_heads=Hkv, head_dim=D,
                    kind="speculative" if spec else "decode")


def sequences(w: Workload):
    """Per-sequence [L,H,D] views (q, k, v lists) of a workload, for the SDPA oracle."""
    qs, ks, vs = [], [], []
    B = len(w.q_lens)
    for b in range(B):
        if w.layout == "dense":
            qs.append(w.q[b].transpose(0, 1))
            ks.append(w.k[b].transpose(0, 1))
            vs.append(w.v[b].transpose(0, 1))
        elif w.layout == "ragged":
            qa, qb = int(w.q_indptr[b]), int(w.q_indptr[b + 1])
            ka, kb = int(w.kv_indptr[b]), int(w.kv_indptr[b + 1])
            qs.append(w.q[qa:qb])
            ks.append(w.k[ka:kb])
            vs.append(w.v[ka:kb])
        else:
            qb = w.q[b].unsqueeze(1) if w.kind == "decode" else w.q[b]
            qs.append(qb.transpose(0, 1))
            ks.append(_gather_one(w.k, w.k_block_table[b], w.kv_lens[b], w.kv_page_size))
            vs.append(_gather_one(w.v, w.v_block_table[b], w.kv_lens[b], w.kv_page_size))
    return qs, ks, vs


def _gather_one(cache, table_row, n, page):
    idx = torch.arange(n, device=cache.device)
    rows = table_row.to(cache.device).long()[idx // page] * page + idx % page
    return cache[rows]


def split_output(w: Workload, out: torch.Tensor):
    """Per-sequence [L,H,D] views of a layout-shaped output."""
    res = []
    for b in range(len(w.q_lens)):
        if w.layout == "ragged":
            a, e = int(w.q_indptr[b]), int(w.q_indptr[b + 1])
            res.append(out[a:e])
        else:
            res.append(out[b, :, : w.q_lens[b]].transpose(0, 1))
    return res
