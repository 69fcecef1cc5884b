"""``speculative_decode_attention`` on MI355X: drop-in for
harsh-vsingh/triton-kernels ``kernels/speculative_decode.py:228-365``.

M <= 16 query (draft) tokens per sequence against a dense, ragged or paged
KV cache whose last M keys are the drafts:

* dense  - q ``[B,QH,M,D]``, k/v ``[B,KVH,N,D]``;
* ragged - q ``[B,QH,M,D]``, k/v ``[total_kv,KVH,D]``, ``kv_indptr`` prefix
  sums ``[B+1]``;
* paged  - q ``[B,QH,M,D]``, k/v caches, ``kv_indptr`` = context LENGTHS
  ``[B]``, ``k/v_block_table`` ``[B, max_blocks]``.

``causal=True`` hides from draft m the drafts after it: key n of a sequence
of N keys is visible to draft m iff ``n < N - M`` or ``n - (N - M) <= m``
(speculative_decode.py:89, 155-160), i.e. bottom-right causal alignment.

Same signature, assertion sequence and mode selection as the reference.
The computation runs in ``libfa2.so`` (``fa2_decode_fwd``, include/fa2.h):
the QH/KVH query heads and the M drafts of a kv-head group are the rows of
one work unit, so each K/V row is streamed from HBM once per kv head; the
KV sweep is split with a log-sum-exp combine (speculative_decode.py:22-225).
No CPU or PyTorch fallback.  Numerics as for ``decode_attention``.
"""

from __future__ import annotations

import torch

from . import _fa2
from .decode import _run_decode


def speculative_decode_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    causal: bool = False,
    kv_indptr: torch.Tensor | None = None,
    k_block_table: torch.Tensor | None = None,
    v_block_table: torch.Tensor | None = None,
    kv_page_size: int | None = None,
    num_splits: int = 0,
) -> torch.Tensor:
    """See the module docstring.  ``num_splits`` (keyword-only, not in the
    reference) forces the split-KV factor; 0 = automatic."""
    # --- assertion sequence of speculative_decode.py:262-297, in order -----
    assert q.dtype == k.dtype == v.dtype, "Tensors must have the same dtype"
    assert q.device == k.device == v.device, "Tensors must be on the same device"
    assert q.is_cuda, "Tensors must be on a CUDA device"

    paged = k_block_table is not None
    ragged = (kv_indptr is not None) and not paged

    if paged:
        assert k_block_table is not None and v_block_table is not None
        assert kv_page_size is not None
        assert kv_indptr is not None, (
            "kv_indptr (sequence context lengths) must be provided for paged mode."
        )
        B, Q_HEADS, M, HEAD_DIM = q.shape
        KV_HEADS = k.shape[2] if k.ndim == 4 else k.shape[1]
        layout = _fa2.LAYOUT_PAGED
    elif ragged:
        if kv_indptr is None:
            raise ValueError("kv_indptr must be provided for ragged mode.")
        B, Q_HEADS, M, HEAD_DIM = q.shape
        total_kv, KV_HEADS, _ = k.shape
        layout = _fa2.LAYOUT_RAGGED
    else:
        B, Q_HEADS, M, HEAD_DIM = q.shape
        _, KV_HEADS, N, _ = k.shape
        layout = _fa2.LAYOUT_DENSE

    assert M <= 16, ("Speculative decode is intended for small draft lengths (M <= 16).")

    out = torch.empty_like(q)
    _run_decode("speculative_decode_attention", q, k, v, out, layout=layout, causal=causal,
                batch=B, q_heads=Q_HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM,
                kv_indptr=kv_indptr, k_block_table=k_block_table, v_block_table=v_block_table,
                kv_page_size=kv_page_size, num_splits=num_splits)
    return out
