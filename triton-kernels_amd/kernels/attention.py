"""``flash_attention_v2`` on MI355X: drop-in for harsh-vsingh/triton-kernels
``kernels/attention.py:749-927``.

Same signature, same assertion sequence, same mode selection and the same
meaning of every argument as the reference:

* dense  - q ``[B,Hq,M,D]``, k/v ``[B,Hkv,N,D]``;
* ragged - q ``[Tq,Hq,D]``, k/v ``[Tkv,Hkv,D]``, ``q_indptr``/``kv_indptr``
  exclusive prefix sums ``[B+1]`` (attention.py:787-810);
* paged  - q ``[B,Hq,M,D]``, k/v caches ``[pages*page,Hkv,D]``, ``kv_indptr``
  = per-sequence KV LENGTHS ``[B]``, ``k/v_block_table`` ``[B, >= pages]``
  (attention.py:812-834).

The work is done by hand-written gfx950 HIP kernels reached through the C
ABI of ``include/fa2.h`` (``libfa2.so``); this module only validates, lays
out the parameter block, allocates the output and the workspace from torch's
caching allocator, and enqueues on torch's current stream.  There is no CPU
or PyTorch fallback.

Beyond the reference (all keyword-only with defaults, so every reference
call is unchanged):

* ``causal_alignment="bottom_right"`` - query i sees key j iff
  ``j <= i + Lk - Lq`` (chunked prefill); default ``"top_left"`` is the
  reference's mask (attention.py:566-569);
* ``num_splits`` - force the split-KV factor (0 = automatic);
* ``max_workgroups`` - cap the persistent kernel's grid (0 = one workgroup
  per compute unit), e.g. to leave compute units to concurrent work;
* ``kernel`` - ``"auto"`` (default), ``"regular"`` or ``"short"``: whether
  a small call (fp16/bf16, head_dim 64/128) may run the short-problem kernel
  that splits each 32-row query block's KV range over the waves of one
  workgroup (``fa2_params.kernel``); results agree within rounding;
* tensors whose last dimension is not contiguous or whose rows are not
  16-byte aligned are copied to a contiguous layout first (the reference
  silently assumes contiguity, attention.py:465-514).
"""

from __future__ import annotations

import torch

from . import _fa2
from ._launch import (check_dtype_and_dim, enqueue, ext, index_tensor, prep, rows_ok, strides,
                      table)

# The launch goes through the C++ extension (one call: sizes, alignment,
# output, workspace, fa2_fwd) when it is built, else through ctypes; both
# enqueue the same libfa2.so entry point with the same parameter block.
USE_EXT = True


def flash_attention_v2(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    is_causal: bool = False,
    q_indptr: torch.Tensor | None = None,
    kv_indptr: torch.Tensor | None = None,
    k_block_table: torch.Tensor | None = None,
    v_block_table: torch.Tensor | None = None,
    kv_page_size: int | None = None,
    causal_alignment: str = "top_left",
    num_splits: int = 0,
    max_workgroups: int = 0,
    kernel: str = "auto",
) -> torch.Tensor:
    return _attention(q, k, v, is_causal=is_causal, q_indptr=q_indptr, kv_indptr=kv_indptr,
                      k_block_table=k_block_table, v_block_table=v_block_table,
                      kv_page_size=kv_page_size, causal_alignment=causal_alignment,
                      num_splits=num_splits, max_workgroups=max_workgroups,
                      arith=_fa2.ARITH_REFERENCE, kernel=kernel)


_KERNELS = {"auto": _fa2.KERNEL_AUTO, "regular": _fa2.KERNEL_REGULAR, "short": _fa2.KERNEL_SHORT}


def _attention(q, k, v, *, is_causal, q_indptr, kv_indptr, k_block_table, v_block_table,
               kv_page_size, causal_alignment, num_splits, max_workgroups, arith,
               kernel="auto"):
    """The shared body of both entry points; ``arith`` is the fa2_arith of
    fp32 tensors (v2: the reference's fp16 rounding; v1: fp32)."""
    # --- assertion sequence of attention.py:762-834, in order -------------
    assert q.dtype == k.dtype == v.dtype
    assert q.device == k.device == v.device
    assert q.is_cuda

    paged = k_block_table is not None
    ragged = (q_indptr is not None) and not paged

    if not ragged and not paged:
        assert q.ndim == 4
        assert k.ndim == 4
        assert v.ndim == 4

        batch, q_heads, M, head_dim = q.shape
        batch_k, kv_heads, N, head_dim_k = k.shape
        batch_v, kv_heads_v, N_v, head_dim_v = v.shape

        assert batch == batch_k == batch_v
        assert kv_heads == kv_heads_v
        assert N == N_v
        assert head_dim == head_dim_k == head_dim_v
        assert q_heads % kv_heads == 0
        layout = _fa2.LAYOUT_DENSE

    elif ragged:
        assert q.ndim == 3
        assert k.ndim == 3
        assert v.ndim == 3

        total_q, q_heads, head_dim = q.shape
        total_kv, kv_heads, head_dim_k = k.shape
        total_v, kv_heads_v, head_dim_v = v.shape

        assert total_kv == total_v
        assert kv_heads == kv_heads_v
        assert head_dim == head_dim_k == head_dim_v
        assert q_heads % kv_heads == 0

        assert q_indptr is not None
        assert kv_indptr is not None

        batch = q_indptr.numel() - 1
        M = total_q
        N = total_kv
        layout = _fa2.LAYOUT_RAGGED

    else:
        assert q.ndim == 4
        assert k.ndim == 3
        assert v.ndim == 3

        batch, q_heads, M, head_dim = q.shape
        total_cache, kv_heads, head_dim_k = k.shape
        total_cache_v, kv_heads_v, head_dim_v = v.shape

        assert total_cache == total_cache_v
        assert kv_heads == kv_heads_v
        assert head_dim == head_dim_k == head_dim_v
        assert q_heads % kv_heads == 0

        assert kv_page_size is not None
        assert kv_indptr is not None
        assert k_block_table is not None
        assert v_block_table is not None

        N = k_block_table.shape[1] * kv_page_size
        layout = _fa2.LAYOUT_PAGED

    # --- checks of this build (the reference would fail inside Triton) ----
    check_dtype_and_dim("flash_attention_v2", q.dtype, head_dim)
    if causal_alignment not in ("top_left", "bottom_right"):
        raise ValueError("causal_alignment must be 'top_left' or 'bottom_right'")
    if kernel not in _KERNELS:
        raise ValueError("kernel must be 'auto', 'regular' or 'short'")

    mask = (_fa2.MASK_NONE if not is_causal else
            (_fa2.MASK_TOP_LEFT if causal_alignment == "top_left" else _fa2.MASK_BOTTOM_RIGHT))
    x = ext() if USE_EXT else None
    if x is not None:
        return x.fwd(q, k, v, layout, mask, q_indptr if layout == _fa2.LAYOUT_RAGGED else None,
                      kv_indptr if layout != _fa2.LAYOUT_DENSE else None,
                      k_block_table if layout == _fa2.LAYOUT_PAGED else None,
                      v_block_table if layout == _fa2.LAYOUT_PAGED else None,
                      kv_page_size if layout == _fa2.LAYOUT_PAGED else 0, int(num_splits),
                      int(max_workgroups), int(arith), _KERNELS[kernel])

    q = prep(q)
    k = prep(k)
    v = prep(v)
    out = torch.empty_like(q)  # contiguous and aligned when q is (the common case)
    if not q.is_contiguous() and not rows_ok(out):
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)

    dev = q.device
    qi = kvi = kt = vt = None
    if layout == _fa2.LAYOUT_RAGGED:
        qi = index_tensor(q_indptr, dev)
        kvi = index_tensor(kv_indptr, dev)
    elif layout == _fa2.LAYOUT_PAGED:
        kvi = index_tensor(kv_indptr, dev)
        kt = table(k_block_table, dev)
        vt = table(v_block_table, dev)

    enqueue(decode=False, layout=layout, mask=mask, num_splits=num_splits, batch=batch,
            q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, q_len=M,
            kv_len=N if layout != _fa2.LAYOUT_PAGED else total_cache,
            q=q, k=k, v=v, out=out, q_strides=strides(q), o_strides=strides(out),
            qi=qi, kvi=kvi, kt=kt, vt=vt, page_size=kv_page_size,
            max_workgroups=max_workgroups,
            kv_len_max=N if layout == _fa2.LAYOUT_PAGED else 0, arith=arith,
            kernel=_KERNELS[kernel])
    return out


def flash_attention_v1(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    is_causal: bool = False,
    q_indptr: torch.Tensor | None = None,
    kv_indptr: torch.Tensor | None = None,
    k_block_table: torch.Tensor | None = None,
    v_block_table: torch.Tensor | None = None,
    kv_page_size: int | None = None,
) -> torch.Tensor:
    """Drop-in for the reference's ``flash_attention_v1``
    (kernels/attention.py:249-364).

    The reference's v1 has the same signature, the same assertion sequence
    (:261-330, identical to v2's :762-834), the same layouts, head map,
    top-left causal mask and softmax scale as v2.  Its arithmetic differs:
    q, k and v are cast to fp32 and the softmax weights stay fp32 (:177,
    196-197, 225-240), where v2 computes in fp16 (:547-633).  fp32 tensors
    therefore run the fp32-MFMA kernel here (fa2_arith FP32); fp16/bf16
    tensors are exact in either and run v2's kernels, whose softmax weights
    are rounded to the tensor type for the P.V product.
    """
    return _attention(q, k, v, is_causal=is_causal, q_indptr=q_indptr, kv_indptr=kv_indptr,
                      k_block_table=k_block_table, v_block_table=v_block_table,
                      kv_page_size=kv_page_size, causal_alignment="top_left", num_splits=0,
                      max_workgroups=0, arith=_fa2.ARITH_FP32)
