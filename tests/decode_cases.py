"""Seeded restatement of the reference decode / speculative-decode test
matrices (tests/test_decode.py, tests/test_speculative_decode.py).

``make_decode_case`` draws lengths and data like ``generate_sequences``
(test_decode.py:47-63, test_speculative_decode.py:55-76) from explicit
seeds: q ``[QH, M, D]`` per sequence, a context of ``l_kv`` keys and, for a
causal speculative case, M draft keys appended to it (the kernel sees
``l_kv + M`` keys).  ``pack_decode`` lays the batch out like the test bodies
(test_decode.py:152-238, test_speculative_decode.py:169-320): dense
zero-padded, ragged concatenated with int32 prefix sums, paged through
``allocate_paged_cache`` (pages in order, table padding 0) or, as an
extension, a shuffled NaN-poisoned pool with ``-1`` padding and distinct K/V
tables, optionally as a 4-D ``[pages, page, KVH, D]`` cache.
"""

from __future__ import annotations

import random
from dataclasses import dataclass

import torch

import oracle
import workloads as W

LAYOUTS = ["dense", "ragged", "paged"]
TOPOLOGIES = ["mha", "gqa", "mqa"]
DTYPES = [torch.float16, torch.bfloat16, torch.float32]
M_VALUES = [2, 3, 4, 6, 8, 10, 12, 16]
PAGE_SIZE = 16


@dataclass
class DecodeCase:
    qs: list        # [QH, M, D] per sequence
    ctx_k: list     # [l_kv, KVH, D] context keys per sequence
    ctx_v: list
    draft_k: list   # [M, KVH, D] draft keys (appended when causal)
    draft_v: list
    ctx_lens: list
    M: int
    causal: bool
    QH: int
    KVH: int
    D: int
    dtype: torch.dtype

    @property
    def ks(self):
        """Keys the kernel attends to per sequence ([L, KVH, D])."""
        if self.causal:
            return [torch.cat([k, d], 0) for k, d in zip(self.ctx_k, self.draft_k)]
        return self.ctx_k

    @property
    def vs(self):
        if self.causal:
            return [torch.cat([v, d], 0) for v, d in zip(self.ctx_v, self.draft_v)]
        return self.ctx_v

    @property
    def kv_lens(self):
        return [n + (self.M if self.causal else 0) for n in self.ctx_lens]


def make_decode_case(B, QH, KVH, D, M, dtype, layout, seed, causal=False, kv_range=(1, 256),
                     dense_kv_range=(16, 256), ctx_lens=None) -> DecodeCase:
    rng = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    fixed = rng.randint(*dense_kv_range)
    lens = [fixed if layout == "dense" else rng.randint(*kv_range) for _ in range(B)]
    if ctx_lens is not None:
        lens = list(ctx_lens)
    qs, ck, cv, dk, dv = [], [], [], [], []
    for n in lens:
        qs.append(torch.randn((QH, M, D), generator=gen).to(dtype))
        ck.append(torch.randn((n, KVH, D), generator=gen).to(dtype))
        cv.append(torch.randn((n, KVH, D), generator=gen).to(dtype))
        dk.append(torch.randn((M, KVH, D), generator=gen).to(dtype))
        dv.append(torch.randn((M, KVH, D), generator=gen).to(dtype))
    return DecodeCase(qs, ck, cv, dk, dv, lens, M, causal, QH, KVH, D, dtype)


def pack_decode(case: DecodeCase, layout: str, device="cpu", shuffled=False, seed=0,
                page=PAGE_SIZE, cache4d=False, squeeze_m=False):
    """(q, k, v, kwargs) for ``speculative_decode_attention`` (q ``[B,QH,M,D]``)
    or, with ``squeeze_m`` and M = 1, ``decode_attention`` (q ``[B,QH,D]``)."""
    q = torch.stack(case.qs)
    if squeeze_m:
        q = q.squeeze(2)
    ks, vs, lens = case.ks, case.vs, case.kv_lens
    if layout == "dense":
        k = W.pack_dense(ks, max(lens))
        v = W.pack_dense(vs, max(lens))
        kw = {}
    elif layout == "ragged":
        k = torch.cat(ks, 0)
        v = torch.cat(vs, 0)
        kw = dict(kv_indptr=W.indptr(lens))
    else:
        if shuffled:
            g = torch.Generator().manual_seed(seed + 7)
            k, kt = W.paged_cache_shuffled(ks, page, 5, g)
            v, vt = W.paged_cache_shuffled(vs, page, 5, g)
        else:
            k, kt = W.paged_cache_contiguous(ks, page)
            v, vt = W.paged_cache_contiguous(vs, page)
        if cache4d:
            k = k.reshape(-1, page, k.shape[1], k.shape[2])
            v = v.reshape(-1, page, v.shape[1], v.shape[2])
        kw = dict(kv_indptr=torch.tensor(lens, dtype=torch.int32), k_block_table=kt,
                  v_block_table=vt, kv_page_size=page)
    moved = {n: (t.to(device) if isinstance(t, torch.Tensor) else t) for n, t in kw.items()}
    return q.to(device), k.to(device), v.to(device), moved


def truth(case: DecodeCase, dtype=torch.float64):
    """The reference suites' SDPA oracle at ``dtype``: per sequence ``[QH,M,D]``.

    A sequence without keys is NaN, the reference kernels' 0/0
    (decode.py:192-197); torch's SDPA returns zeros there."""
    if case.M == 1 and not case.causal:
        refs = oracle.sdpa_decode_reference([q[:, 0] for q in case.qs], case.ctx_k, case.ctx_v,
                                            case.QH, case.KVH, dtype=dtype)
        refs = [r.unsqueeze(1) for r in refs]
    else:
        refs = oracle.sdpa_speculative_reference(case.qs, case.ctx_k, case.ctx_v, case.draft_k,
                                                 case.draft_v, case.QH, case.KVH, case.causal,
                                                 dtype=dtype)
    return [torch.full_like(r, float("nan")) if n == 0 else r
            for r, n in zip(refs, case.kv_lens)]
