"""``decode_attention`` on MI355X: drop-in for harsh-vsingh/triton-kernels
``kernels/decode.py:203-331``.

One query token per sequence, against a dense, ragged or paged KV cache:

* dense  - q ``[B,QH,D]``, k/v ``[B,KVH,N,D]`` (every sequence has N keys);
* ragged - q ``[B,QH,D]``, k/v ``[total_kv,KVH,D]``, ``kv_indptr`` exclusive
  prefix sums ``[B+1]``;
* paged  - q ``[B,QH,D]``, k/v caches ``[pages*page,KVH,D]`` (or
  ``[pages,page,KVH,D]``), ``kv_indptr`` = per-sequence context LENGTHS
  ``[B]``, ``k/v_block_table`` ``[B, max_blocks]``.

Same signature, assertion sequence and mode selection as the reference.
The computation runs in ``libfa2.so`` (``fa2_decode_fwd``, include/fa2.h):
the QH/KVH query heads that share a kv head are the rows of one work unit,
so each K/V row is streamed from HBM once per kv head, and the KV sweep is
split across workgroups with a log-sum-exp combine (the reference's split +
merge, decode.py:22-200).  No CPU or PyTorch fallback.

Numerics: the reference loads every dtype into fp32 and computes in fp32
(decode.py:84, 92-160).  fp32 tensors do the same here, on the fp32 MFMA
(``v_mfma_f32_32x32x2_f32``: fp32 operands and softmax weights), so values
past fp16's range stay finite.  fp16/bf16 tensors are exact in fp32 and run on
the 16-bit MFMA with fp32 accumulation and fp32 softmax statistics; only P is
rounded to the tensor type for the P.V product.  Both are within the
reference test's tolerances (tests/test_decode.py:20-30) and the GPU tests'
strict bar against the reference's fp32 arithmetic.
"""

from __future__ import annotations

import torch

from . import _fa2
from ._launch import check_dtype_and_dim, enqueue, index_tensor, prep, rows_ok, table


def decode_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    kv_indptr: torch.Tensor | None = None,
    k_block_table: torch.Tensor | None = None,
    v_block_table: torch.Tensor | None = None,
    kv_page_size: int | None = None,
    num_splits: int = 0,
) -> torch.Tensor:
    """See the module docstring.  ``num_splits`` (keyword-only, not in the
    reference) forces the split-KV factor; 0 = automatic."""
    # --- assertion sequence of decode.py:236-274, in order -----------------
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
        B, Q_HEADS, HEAD_DIM = q.shape
        KV_HEADS = k.shape[2] if k.ndim == 4 else k.shape[1]
        layout = _fa2.LAYOUT_PAGED
    elif ragged:
        if kv_indptr is None:
            raise ValueError("kv_indptr must be provided for ragged mode.")
        B, Q_HEADS, HEAD_DIM = q.shape
        total_kv, KV_HEADS, _ = k.shape
        layout = _fa2.LAYOUT_RAGGED
    else:
        B, Q_HEADS, HEAD_DIM = q.shape
        _, KV_HEADS, N, _ = k.shape
        layout = _fa2.LAYOUT_DENSE

    out = torch.empty_like(q)
    _run_decode("decode_attention", q.unsqueeze(2), k, v, out.unsqueeze(2), layout=layout,
                causal=False, batch=B, q_heads=Q_HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM,
                kv_indptr=kv_indptr, k_block_table=k_block_table, v_block_table=v_block_table,
                kv_page_size=kv_page_size, num_splits=num_splits)
    return out


def _run_decode(name, q4, k, v, out4, *, layout, causal, batch, q_heads, kv_heads, head_dim,
                kv_indptr, k_block_table, v_block_table, kv_page_size, num_splits=0,
                decode_spin_cap=0, workspace=None):
    """Shared by decode_attention and speculative_decode_attention.

    ``q4`` / ``out4`` are ``[B, QH, M, D]`` views; ``out4`` must be a view
    of the caller's output so the kernels write it in place.
    ``decode_spin_cap`` (tests only, fa2_params.decode_spin_cap) bounds the
    decode kernel's ring waits; 0 = the library's bound.  ``workspace``
    (tests only) is a uint8 device buffer used instead of an allocation."""
    check_dtype_and_dim(name, q4.dtype, head_dim)
    if q_heads % kv_heads != 0:
        raise ValueError(f"{name}: q_heads ({q_heads}) must be a multiple of kv_heads "
                         f"({kv_heads})")
    if k.shape[-1] != head_dim or v.shape[-1] != head_dim or k.shape != v.shape:
        raise ValueError(f"{name}: k and v must have equal shapes with head_dim {head_dim}")
    M = q4.shape[2]
    dev = q4.device
    # shapes the device grid relies on (the reference does not check them)
    if layout == _fa2.LAYOUT_DENSE and k.shape[0] != batch:
        raise ValueError(f"{name}: k/v batch {k.shape[0]} != q batch {batch}")
    if layout == _fa2.LAYOUT_RAGGED and kv_indptr.numel() < batch + 1:
        raise ValueError(f"{name}: kv_indptr needs {batch + 1} prefix sums")
    if layout == _fa2.LAYOUT_PAGED and (kv_indptr.numel() < batch or
                                        k_block_table.shape[0] < batch or
                                        v_block_table.shape[0] < batch):
        raise ValueError(f"{name}: kv_indptr and the block tables need {batch} rows")

    if layout == _fa2.LAYOUT_PAGED and k.ndim == 4:
        # [pages, page, KVH, D] -> [pages * page, KVH, D] (decode.py:136-149
        # addresses (page * page_size + offset) * KVH * D + head * D)
        k = k.reshape(-1, k.shape[2], k.shape[3])
        v = v.reshape(-1, v.shape[2], v.shape[3])
    k = prep(k)
    v = prep(v)
    # one strided run of rows per kv-head group: row r = head * M + m
    # (M = 1: the rows of a group are its heads, the row stride is the head stride)
    def run_ok(t):
        return rows_ok(t) and (M == 1 or t.stride(1) == M * t.stride(2))

    def abi_strides(t):
        return (t.stride(0), t.stride(1), t.stride(2) if M > 1 else t.stride(1))

    if not run_ok(q4):
        q4 = q4.contiguous()
    dst = out4 if run_ok(out4) else torch.empty(out4.shape, dtype=out4.dtype, device=dev)

    kvi = kt = vt = None
    if layout == _fa2.LAYOUT_RAGGED:
        kvi = index_tensor(kv_indptr, dev)
        kv_len = k.shape[0]
    elif layout == _fa2.LAYOUT_PAGED:
        kvi = index_tensor(kv_indptr, dev)
        kt = table(k_block_table, dev)
        vt = table(v_block_table, dev)
        kv_len = k.shape[0]
    else:
        kv_len = k.shape[2]

    mask = _fa2.MASK_BOTTOM_RIGHT if causal else _fa2.MASK_NONE
    enqueue(decode=True, layout=layout, mask=mask, num_splits=num_splits, batch=batch,
            q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, q_len=M, kv_len=kv_len,
            q=q4, k=k, v=v, out=dst, q_strides=abi_strides(q4), o_strides=abi_strides(dst),
            kvi=kvi, kt=kt, vt=vt, page_size=kv_page_size,
            kv_len_max=kt.shape[1] * kv_page_size if kt is not None else 0,
            decode_spin_cap=decode_spin_cap, workspace=workspace)
    if dst is not out4:
        out4.copy_(dst)
