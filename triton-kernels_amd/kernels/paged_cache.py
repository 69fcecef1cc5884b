"""Paged KV-cache writer on MI355X: the producer side of the paged layout
that ``flash_attention_v2``, ``decode_attention`` and
``speculative_decode_attention`` read.

The reference has no kernel for this step.  Its paged caches are built on
the host, page by page, by the test helper ``allocate_paged_cache``
(tests/test_attention.py:101-134, repeated in tests/test_decode.py:93 and
tests/test_speculative_decode.py:129: pages in sequence order, table padding
0) and the benchmark helper ``build_paged_cache`` (benchmarks/attention.py:
351-431: table padding -1, also returns the lengths).  The format is theirs:
a cache is ``[num_pages * page_size, kv_heads, head_dim]`` and logical row n
of sequence b lives at row ``table[b, n // page_size] * page_size +
n % page_size``.

* :func:`paged_kv_append` - the device step a serving loop needs: write the
  new K/V rows of every sequence (ragged ``[T, KVH, D]`` with prefix sums
  ``new_indptr``) at logical positions ``start_pos[b] + j`` through the block
  tables, in place, one kernel launch (``fa2_kv_append``, include/fa2.h).
* :func:`allocate_paged_cache` / :func:`build_paged_cache` - the reference
  helpers' signatures and results, with the page scatter done by the same
  kernel instead of per-page host copies.
"""

from __future__ import annotations

import torch

from . import _fa2
from ._launch import DTYPES, index_tensor, table


def paged_kv_append(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor | None,
    k_block_table: torch.Tensor,
    v_block_table: torch.Tensor | None,
    k_new: torch.Tensor,
    v_new: torch.Tensor | None,
    new_indptr: torch.Tensor,
    kv_page_size: int,
    start_pos: torch.Tensor | None = None,
) -> None:
    """Write ``k_new`` / ``v_new`` rows into the caches, in place.

    ``k_cache``/``v_cache``: ``[pages * kv_page_size, KVH, D]`` (or
    ``[pages, kv_page_size, KVH, D]``); ``k_new``/``v_new``: ``[T, KVH, D]``;
    ``new_indptr``: ``[B + 1]`` prefix sums over the new rows;
    ``start_pos``: ``[B]`` logical position of each sequence's first new row
    (``None``: 0); tables ``[B, width]``.  The V arguments may all be
    ``None`` (K only).  Rows whose logical page is past the table width, or
    whose table entry is outside the cache, are not written.
    """
    has_v = v_cache is not None
    assert k_cache.dtype == k_new.dtype and (not has_v or v_cache.dtype == v_new.dtype)
    assert k_cache.device == k_new.device == k_block_table.device == new_indptr.device
    assert k_cache.is_cuda
    if (v_new is None) != (not has_v) or (v_block_table is None) != (not has_v):
        raise ValueError("paged_kv_append: pass v_cache, v_block_table and v_new together")
    if k_cache.dtype not in DTYPES:
        raise TypeError(f"paged_kv_append: unsupported dtype {k_cache.dtype}")
    kc = k_cache.view(-1, k_cache.shape[-2], k_cache.shape[-1]) if k_cache.dim() == 4 else k_cache
    vc = None
    if has_v:
        vc = (v_cache.view(-1, v_cache.shape[-2], v_cache.shape[-1]) if v_cache.dim() == 4
              else v_cache)
        if vc.shape != kc.shape or vc.stride() != kc.stride():
            raise ValueError("paged_kv_append: k_cache and v_cache must have equal layouts")
    H, D = kc.shape[1], kc.shape[2]
    if k_new.dim() != 3 or k_new.shape[1:] != (H, D):
        raise ValueError(f"paged_kv_append: new rows must be [T, {H}, {D}]")
    if has_v and (v_new.shape != k_new.shape):
        raise ValueError("paged_kv_append: k_new and v_new must have equal shapes")
    if kc.stride(-1) != 1:
        raise ValueError("paged_kv_append: the caches' head_dim must be contiguous")
    if kv_page_size <= 0 or kc.shape[0] % kv_page_size:
        raise ValueError("paged_kv_append: cache rows must be a whole number of pages")
    B = new_indptr.numel() - 1
    if B < 0 or k_block_table.shape[0] < B or (has_v and v_block_table.shape[0] < B):
        raise ValueError("paged_kv_append: the block tables need one row per sequence")
    if start_pos is not None and start_pos.numel() < B:
        raise ValueError("paged_kv_append: start_pos needs one entry per sequence")
    dev = kc.device
    kn, vn = k_new, v_new
    if kn.stride(-1) != 1 or (has_v and vn.stride() != kn.stride()):
        kn = kn.contiguous()
        vn = vn.contiguous() if has_v else None
    ip = index_tensor(new_indptr, dev)
    sp = index_tensor(start_pos, dev) if start_pos is not None else None
    kt = table(k_block_table, dev)
    vt = table(v_block_table, dev) if has_v else None

    p = _fa2.KvAppendParams()
    p.dtype = DTYPES[kc.dtype]
    p.batch = B
    p.kv_heads, p.head_dim = H, D
    p.num_rows = kn.shape[0]
    p.page_size = int(kv_page_size)
    p.num_pages = kc.shape[0] // int(kv_page_size)
    p.table_width = kt.shape[1]
    p.k_table_stride = kt.stride(0)
    p.v_table_stride = vt.stride(0) if has_v else 0
    p.new_ts, p.new_hs = kn.stride(0), kn.stride(1)
    p.cache_ts, p.cache_hs = kc.stride(0), kc.stride(1)
    p.k_new, p.k_cache = kn.data_ptr(), kc.data_ptr()
    p.new_indptr, p.k_block_table = ip.data_ptr(), kt.data_ptr()
    if sp is not None:
        p.start_pos = sp.data_ptr()
    if has_v:
        p.v_new, p.v_cache, p.v_block_table = vn.data_ptr(), vc.data_ptr(), vt.data_ptr()
    with torch.cuda.device(dev):
        _fa2.kv_append(p, torch.cuda.current_stream(dev).cuda_stream)


def _contiguous_table(lens, page_size, pad, device):
    """Pages in sequence order (the reference helpers' assignment)."""
    nb = [(n + page_size - 1) // page_size for n in lens]
    width = max(nb) if nb else 0
    tbl = torch.full((len(lens), width), pad, dtype=torch.int32)
    cur = 0
    for b, n in enumerate(nb):
        tbl[b, :n] = torch.arange(cur, cur + n, dtype=torch.int32)
        cur += n
    return tbl.to(device), cur


def allocate_paged_cache(tensors, lens, heads, dim, page_size):
    """tests/test_attention.py:101-134 on the device: scatter the sequences
    ``tensors`` (``[L_b, heads, dim]`` each) into a zeroed cache of
    ``sum(ceil(L_b / page_size))`` pages, pages in sequence order; returns
    ``(cache, block_table)`` (int32, padding 0)."""
    dev = tensors[0].device
    tbl, pages = _contiguous_table(lens, page_size, 0, dev)
    cache = torch.zeros((pages * page_size, heads, dim), dtype=tensors[0].dtype, device=dev)
    src = torch.cat([t[:n] for t, n in zip(tensors, lens)], 0).contiguous()
    ip = torch.tensor([0] + list(lens), dtype=torch.int64).cumsum(0).to(torch.int32).to(dev)
    paged_kv_append(cache, None, tbl, None, src, None, ip, page_size)
    return cache, tbl


def build_paged_cache(seqs, page_size):
    """benchmarks/attention.py:351-431 on the device: ``seqs`` is a list of
    ``[N_b, KVH, D]``; returns ``(cache, lengths, block_table)`` with the
    table padded with -1 and every page's tail zeroed."""
    dev = seqs[0].device
    lens = [s.shape[0] for s in seqs]
    tbl, pages = _contiguous_table(lens, page_size, -1, dev)
    cache = torch.zeros((pages * page_size, seqs[0].shape[1], seqs[0].shape[2]),
                        dtype=seqs[0].dtype, device=dev)
    src = torch.cat(seqs, 0).contiguous()
    ip = torch.tensor([0] + lens, dtype=torch.int64).cumsum(0).to(torch.int32).to(dev)
    paged_kv_append(cache, None, tbl, None, src, None, ip, page_size)
    return cache, torch.tensor(lens, dtype=torch.int32, device=dev), tbl
