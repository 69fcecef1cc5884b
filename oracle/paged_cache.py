"""CPU restatement of the reference's paged-cache construction, and of
appending rows to such a cache.

TEST INFRASTRUCTURE ONLY (imported by tests/ as the checker of
``kernels.paged_cache``; never by the product path).

* :func:`allocate_paged_cache` follows tests/test_attention.py:101-134 line
  by line in meaning: pages in sequence order, table padding 0, a zeroed
  cache of ``sum(ceil(L_b / P))`` pages, rows copied page by page.
* :func:`build_paged_cache` follows benchmarks/attention.py:351-431: one
  zeroed ``[P, KVH, D]`` buffer per page, concatenated, table padding -1,
  lengths returned as int32.
* :func:`append` writes new rows at logical positions ``start[b] + j``
  through the tables, one row at a time, skipping rows whose logical page is
  past the table width or whose entry is outside the cache - the contract of
  ``fa2_kv_append`` (include/fa2.h).
* :func:`gather` reads sequence b's first ``n`` rows back through the table
  (the paged attention kernels' addressing, attention.py:575-594).
"""

from __future__ import annotations

import torch


def allocate_paged_cache(tensors, lens, heads, dim, page_size):
    B = len(lens)
    max_blocks = max((n + page_size - 1) // page_size for n in lens)
    total_blocks = sum((n + page_size - 1) // page_size for n in lens)
    cache = torch.zeros((total_blocks * page_size, heads, dim), dtype=tensors[0].dtype)
    table = torch.zeros((B, max_blocks), dtype=torch.int32)
    cur = 0
    for b in range(B):
        for logical in range((lens[b] + page_size - 1) // page_size):
            table[b, logical] = cur
            s, e = logical * page_size, min((logical + 1) * page_size, lens[b])
            cache[cur * page_size: cur * page_size + (e - s)] = tensors[b][s:e].cpu()
            cur += 1
    return cache, table


def build_paged_cache(seqs, page_size):
    kvh, d = seqs[0].shape[1], seqs[0].shape[2]
    lengths = torch.tensor([x.shape[0] for x in seqs], dtype=torch.int32)
    pages, tables, nxt = [], [], 0
    for seq in seqs:
        n = seq.shape[0]
        t = []
        for pg in range((n + page_size - 1) // page_size):
            s, e = pg * page_size, min(pg * page_size + page_size, n)
            buf = torch.zeros((page_size, kvh, d), dtype=seq.dtype)
            buf[: e - s] = seq[s:e].cpu()
            pages.append(buf)
            t.append(nxt)
            nxt += 1
        tables.append(t)
    table = torch.full((len(seqs), max(len(t) for t in tables)), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        table[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
    return torch.cat(pages, 0), lengths, table


def append(cache, table, new, indptr, page_size, start=None):
    """Returns a copy of ``cache`` with ``new``'s rows written (see module doc)."""
    out = cache.clone()
    pages = cache.shape[0] // page_size
    for b in range(indptr.numel() - 1):
        s0 = int(start[b]) if start is not None else 0
        for j in range(int(indptr[b]), int(indptr[b + 1])):
            n = s0 + j - int(indptr[b])
            lp = n // page_size
            if n < 0 or lp >= table.shape[1]:
                continue
            pg = int(table[b, lp])
            if 0 <= pg < pages:
                out[pg * page_size + n % page_size] = new[j].cpu()
    return out


def gather(cache, table, b, n, page_size):
    rows = [int(table[b, j // page_size]) * page_size + j % page_size for j in range(n)]
    return cache[rows]
