"""Seeded restatement of the reference test matrix (tests/test_attention.py).

``make_case`` draws lengths and data like ``generate_sequences``
(tests/test_attention.py:52-77) but from explicit seeds, and ``pack`` lays
them out like the test body (:159-243): dense zero-padded, ragged
concatenated with int32 prefix sums, paged through
``allocate_paged_cache`` (pages in order, table padding 0) or, as an
extension, through a shuffled pool with ``-1`` padding and independent K/V
tables.
"""

from __future__ import annotations

import random
from dataclasses import dataclass

import torch

import workloads as W

LAYOUTS = ["dense", "paged", "ragged"]
ATTN_TYPES = ["self", "cross"]
TOPOLOGIES = ["mha", "gqa", "mqa"]
CAUSAL_FLAGS = [False, True]
DTYPES = [torch.float16, torch.bfloat16, torch.float32]
PAGE_SIZE = 16


def topology_heads(topology):
    return {"mha": (8, 8), "gqa": (8, 2), "mqa": (8, 1)}[topology]


@dataclass
class Case:
    qs: list
    ks: list
    vs: list
    q_lens: list
    kv_lens: list
    QH: int
    KVH: int
    D: int
    dtype: torch.dtype


def make_case(B, QH, KVH, D, attn_type, dtype, layout, seed, q_range=(1, 128),
              kv_range=(1, 256), dense_q_range=(16, 128), dense_kv_range=(16, 256),
              q_lens=None, kv_lens=None) -> Case:
    rng = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    fixed_q = rng.randint(*dense_q_range)
    fixed_kv = fixed_q if attn_type == "self" else rng.randint(*dense_kv_range)
    ql, kl = [], []
    for b in range(B):
        lq = fixed_q if layout == "dense" else rng.randint(*q_range)
        if attn_type == "self":
            lk = lq
        else:
            lk = fixed_kv if layout == "dense" else rng.randint(*kv_range)
        ql.append(lq)
        kl.append(lk)
    if q_lens is not None:
        ql = list(q_lens)
    if kv_lens is not None:
        kl = list(kv_lens)
    qs, ks, vs = [], [], []
    for lq, lk in zip(ql, kl):
        qs.append(torch.randn((lq, QH, D), generator=gen).to(dtype))
        ks.append(torch.randn((lk, KVH, D), generator=gen).to(dtype))
        vs.append(torch.randn((lk, KVH, D), generator=gen).to(dtype))
    return Case(qs, ks, vs, ql, kl, QH, KVH, D, dtype)


def pack(case: Case, layout: str, device="cpu", shuffled_pages=False, seed=0, page=PAGE_SIZE):
    """Return (q, k, v, kwargs) for ``flash_attention_v2`` in ``layout``."""
    B = len(case.qs)
    if layout == "dense":
        q = W.pack_dense(case.qs, max(case.q_lens))
        k = W.pack_dense(case.ks, max(case.kv_lens))
        v = W.pack_dense(case.vs, max(case.kv_lens))
        kw = {}
    elif layout == "ragged":
        q = torch.cat(case.qs, 0)
        k = torch.cat(case.ks, 0)
        v = torch.cat(case.vs, 0)
        kw = dict(q_indptr=W.indptr(case.q_lens), kv_indptr=W.indptr(case.kv_lens))
    else:
        q = W.pack_dense(case.qs, max(case.q_lens))
        if shuffled_pages:
            g = torch.Generator().manual_seed(seed + 7)
            # same pool size (the wrapper asserts equal cache lengths,
            # attention.py:820), independent page orders
            k, kt = W.paged_cache_shuffled(case.ks, page, 5, g)
            v, vt = W.paged_cache_shuffled(case.vs, page, 5, g)
        else:
            k, kt = W.paged_cache_contiguous(case.ks, page)
            v, vt = W.paged_cache_contiguous(case.vs, page)
        kw = dict(kv_indptr=torch.tensor(case.kv_lens, dtype=torch.int32), k_block_table=kt,
                  v_block_table=vt, kv_page_size=page)
    moved = {n: (t.to(device) if isinstance(t, torch.Tensor) else t) for n, t in kw.items()}
    return q.to(device), k.to(device), v.to(device), moved


def unpack(case: Case, layout: str, out: torch.Tensor, kw: dict):
    """Per-sequence [L,H,D] outputs (tests/test_attention.py:172-175, 189-194, 243)."""
    res = []
    if layout == "ragged":
        ip = kw["q_indptr"].cpu()
        for b in range(len(case.qs)):
            res.append(out[int(ip[b]): int(ip[b + 1])])
    else:
        for b in range(len(case.qs)):
            res.append(out[b, :, : case.q_lens[b], :].transpose(0, 1))
    return res
