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
* tensors whose last dimension is not contiguous or whose rows are not
  16-byte aligned are copied to a contiguous layout first (the reference
  silently assumes contiguity, attention.py:465-514).
"""

from __future__ import annotations

import torch

from . import _fa2

_DTYPES = {
    torch.float16: _fa2.DTYPE_F16,
    torch.bfloat16: _fa2.DTYPE_BF16,
    torch.float32: _fa2.DTYPE_F32,
}
SUPPORTED_HEAD_DIMS = (64, 128)


def _rows_ok(t: torch.Tensor) -> bool:
    """Last dim contiguous and every row start 16-byte aligned."""
    if t.numel() == 0:
        return True
    if t.stride(-1) != 1:
        return False
    es = t.element_size()
    if t.data_ptr() % 16:
        return False
    return all((s * es) % 16 == 0 for s in t.stride()[:-1])


def _prep(t: torch.Tensor) -> torch.Tensor:
    return t if _rows_ok(t) else t.contiguous()


def _strides(t: torch.Tensor):
    """(batch, head, row) element strides; token-major tensors use (0, head, token)."""
    if t.dim() == 4:
        return t.stride(0), t.stride(1), t.stride(2)
    return 0, t.stride(1), t.stride(0)


def _index_tensor(t: torch.Tensor, device) -> torch.Tensor:
    if t.dtype != torch.int32 or not t.is_contiguous() or t.device != device:
        t = t.to(device=device, dtype=torch.int32).contiguous()
    return t


def _table(t: torch.Tensor, device) -> torch.Tensor:
    if t.dtype != torch.int32 or t.stride(-1) != 1 or t.device != device:
        t = t.to(device=device, dtype=torch.int32).contiguous()
    return t


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
) -> torch.Tensor:
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
    if q.dtype not in _DTYPES:
        raise TypeError(f"flash_attention_v2: unsupported dtype {q.dtype} "
                        "(float16, bfloat16, float32)")
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"flash_attention_v2: head_dim {head_dim} not supported "
                         f"(supported: {SUPPORTED_HEAD_DIMS})")
    if causal_alignment not in ("top_left", "bottom_right"):
        raise ValueError("causal_alignment must be 'top_left' or 'bottom_right'")

    q = _prep(q)
    k = _prep(k)
    v = _prep(v)
    out = torch.empty_like(q)
    if not _rows_ok(out):
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)

    dev = q.device
    mask = (_fa2.MASK_NONE if not is_causal else
            (_fa2.MASK_TOP_LEFT if causal_alignment == "top_left" else _fa2.MASK_BOTTOM_RIGHT))
    qi = kvi = kt = vt = None
    if layout == _fa2.LAYOUT_RAGGED:
        qi = _index_tensor(q_indptr, dev)
        kvi = _index_tensor(kv_indptr, dev)
    elif layout == _fa2.LAYOUT_PAGED:
        kvi = _index_tensor(kv_indptr, dev)
        kt = _table(k_block_table, dev)
        vt = _table(v_block_table, dev)

    # Everything but the pointers depends only on the call signature: build
    # that part of the parameter block (and its workspace size) once.
    key = (layout, q.dtype, mask, int(num_splits), dev.index, q.shape, q.stride(), k.shape,
           k.stride(), v.stride(), out.stride(), batch,
           None if kt is None else (kt.stride(0), vt.stride(0), int(kv_page_size)))
    cached = _PLAN_CACHE.get(key)
    if cached is None:
        p = _fa2.Fa2Params()
        p.layout = layout
        p.dtype = _DTYPES[q.dtype]
        p.mask = mask
        p.num_splits = int(num_splits)
        p.batch = batch
        p.q_heads = q_heads
        p.kv_heads = kv_heads
        p.head_dim = head_dim
        p.q_len = M
        p.kv_len = N if layout != _fa2.LAYOUT_PAGED else total_cache
        p.q_sb, p.q_sh, p.q_ss = _strides(q)
        p.k_sb, p.k_sh, p.k_ss = _strides(k)
        p.v_sb, p.v_sh, p.v_ss = _strides(v)
        p.o_sb, p.o_sh, p.o_ss = _strides(out)
        if kt is not None:
            p.k_table_stride, p.v_table_stride = kt.stride(0), vt.stride(0)
            p.page_size = int(kv_page_size)
        p.softmax_scale = head_dim ** -0.5
        # validation needs the layout's pointers; they are overwritten per call
        p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
        if qi is not None:
            p.q_indptr = qi.data_ptr()
        if kvi is not None:
            p.kv_indptr = kvi.data_ptr()
        if kt is not None:
            p.k_block_table, p.v_block_table = kt.data_ptr(), vt.data_ptr()
        with torch.cuda.device(dev):
            ws_bytes = _fa2.workspace_size(p)
        cached = (bytes(p), ws_bytes)
        if len(_PLAN_CACHE) >= _PLAN_CACHE_MAX:
            _PLAN_CACHE.clear()
        _PLAN_CACHE[key] = cached

    p = _fa2.Fa2Params.from_buffer_copy(cached[0])
    ws_bytes = cached[1]
    p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    if qi is not None:
        p.q_indptr = qi.data_ptr()
    if kvi is not None:
        p.kv_indptr = kvi.data_ptr()
    if kt is not None:
        p.k_block_table, p.v_block_table = kt.data_ptr(), vt.data_ptr()

    switch = dev.index != torch.cuda.current_device()
    if switch:
        prev = torch.cuda.current_device()
        torch.cuda.set_device(dev)
    try:
        stream = torch.cuda.current_stream(dev)
        ws = None
        if ws_bytes:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
            p.workspace, p.workspace_bytes = ws.data_ptr(), ws_bytes
        _fa2.forward(p, stream.cuda_stream)
        if ws is not None:
            ws.record_stream(stream)
    finally:
        if switch:
            torch.cuda.set_device(prev)
    return out


# call signature -> (static bytes of the parameter block, workspace bytes)
_PLAN_CACHE: dict = {}
_PLAN_CACHE_MAX = 4096
