"""Host-side plumbing shared by the attention entry points: tensor checks,
the ``fa2_params`` block, a cache of its call-invariant part, the workspace
(from torch's caching allocator) and the enqueue on torch's current stream.

Everything device-side happens in ``libfa2.so`` through ``_fa2``; this module
never computes attention itself.
"""

from __future__ import annotations

import torch

from . import _fa2

DTYPES = {
    torch.float16: _fa2.DTYPE_F16,
    torch.bfloat16: _fa2.DTYPE_BF16,
    torch.float32: _fa2.DTYPE_F32,
}
SUPPORTED_HEAD_DIMS = (16, 32, 64, 128, 256)


def rows_ok(t: torch.Tensor) -> bool:
    """Last dim contiguous and every row start 16-byte aligned."""
    if t.numel() == 0:
        return True
    if t.is_contiguous():  # every stride is a multiple of the row length
        return t.data_ptr() % 16 == 0 and (t.shape[-1] * t.element_size()) % 16 == 0
    if t.stride(-1) != 1:
        return False
    es = t.element_size()
    if t.data_ptr() % 16:
        return False
    return all((s * es) % 16 == 0 for s in t.stride()[:-1])


def prep(t: torch.Tensor) -> torch.Tensor:
    return t if rows_ok(t) else t.contiguous()


def strides(t: torch.Tensor):
    """(batch, head, row) element strides; token-major tensors use (0, head, token)."""
    if t.dim() == 4:
        return t.stride(0), t.stride(1), t.stride(2)
    return 0, t.stride(1), t.stride(0)


def index_tensor(t: torch.Tensor, device) -> torch.Tensor:
    if t.dtype != torch.int32 or not t.is_contiguous() or t.device != device:
        t = t.to(device=device, dtype=torch.int32).contiguous()
    return t


def table(t: torch.Tensor, device) -> torch.Tensor:
    if t.dtype != torch.int32 or t.stride(-1) != 1 or t.device != device:
        t = t.to(device=device, dtype=torch.int32).contiguous()
    return t


_EXT = None
_EXT_ERROR = None


def ext():
    """The PyTorch-ROCm launch extension (csrc/fa2_torch.cpp, built in-tree by
    build.py next to libfa2.so), or None when it is not built; its launch
    calls the same libfa2.so entry point as the ctypes path below."""
    global _EXT, _EXT_ERROR
    if _EXT is None and _EXT_ERROR is None:
        try:
            from . import fa2_torch
            _EXT = fa2_torch
        except ImportError as e:  # not built: the ctypes path launches
            _EXT_ERROR = e
    return _EXT


def check_dtype_and_dim(name: str, dtype, head_dim: int) -> None:
    """Checks of this build (the reference would fail inside Triton)."""
    if dtype not in DTYPES:
        raise TypeError(f"{name}: unsupported dtype {dtype} (float16, bfloat16, float32)")
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"{name}: head_dim {head_dim} not supported "
                         f"(supported: {SUPPORTED_HEAD_DIMS})")


# torch's current HIP stream of a device as a raw handle (the Stream object
# is only built when a workspace has to be recorded on it)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(dev) -> int:
    if _raw_stream is not None:
        return _raw_stream(dev.index)
    return torch.cuda.current_stream(dev).cuda_stream


# call signature -> (static bytes of the parameter block, workspace bytes)
_PLAN_CACHE: dict = {}
_PLAN_CACHE_MAX = 4096


def enqueue(*, decode: bool, layout: int, mask: int, num_splits: int, batch: int,
            q_heads: int, kv_heads: int, head_dim: int, q_len: int, kv_len: int,
            q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
            q_strides, o_strides, qi=None, kvi=None, kt=None, vt=None,
            page_size=None, max_workgroups: int = 0, kv_len_max: int = 0,
            noalloc: bool = False, arith: int = 0, decode_spin_cap: int = 0,
            kernel: int = 0, workspace: torch.Tensor | None = None) -> None:
    """Fill ``fa2_params`` and enqueue ``fa2_fwd`` (``decode=False``) or
    ``fa2_decode_fwd`` on torch's current stream of ``q``'s device.

    ``q_strides`` / ``o_strides`` are the (batch, head, row) element strides
    the ABI expects; k/v strides are taken from the tensors.  ``kv_len`` is
    the ABI's field (paged: the caches' rows, 0 = unknown), ``kv_len_max`` an
    upper bound of every sequence's KV length (0 = unknown) and
    ``max_workgroups`` the cap on the persistent grid (0 = none), ``arith`` the
    fa2_arith of fp32 tensors (``_fa2.ARITH_FP32``: fp32 throughout),
    ``decode_spin_cap`` the decode kernel's wait bound (tests only), ``kernel``
    the fa2_kernel choice of the forward kernel (``_fa2.KERNEL_AUTO``...), ``workspace``
    a caller's uint8 device buffer of at least the workspace size to use instead of
    an allocation (tests).  ``noalloc``
    enqueues ``fa2_fwd_noalloc`` instead (no workspace; prefill only).  Everything but
    the pointers depends only on the call signature, so that part of the
    parameter block (and its workspace size) is built once per signature.
    """
    dev = q.device
    key = (decode, layout, q.dtype, mask, int(num_splits), dev.index, batch, q_heads, kv_heads,
           head_dim, q_len, kv_len, tuple(q_strides), tuple(o_strides), k.stride(), v.stride(),
           None if kt is None else (kt.stride(0), vt.stride(0), int(page_size)),
           int(max_workgroups), int(kv_len_max), int(arith), int(decode_spin_cap), int(kernel))
    cached = _PLAN_CACHE.get(key)
    if cached is None:
        p = _fa2.Fa2Params()
        p.layout = layout
        p.dtype = DTYPES[q.dtype]
        p.mask = mask
        p.num_splits = int(num_splits)
        p.batch = batch
        p.q_heads = q_heads
        p.kv_heads = kv_heads
        p.head_dim = head_dim
        p.q_len = q_len
        p.kv_len = kv_len
        p.q_sb, p.q_sh, p.q_ss = q_strides
        p.k_sb, p.k_sh, p.k_ss = strides(k)
        p.v_sb, p.v_sh, p.v_ss = strides(v)
        p.o_sb, p.o_sh, p.o_ss = o_strides
        if kt is not None:
            p.k_table_stride, p.v_table_stride = kt.stride(0), vt.stride(0)
            p.page_size = int(page_size)
        p.softmax_scale = head_dim ** -0.5
        p.max_workgroups = int(max_workgroups)
        p.kv_len_max = int(kv_len_max)
        p.arith = int(arith)
        p.decode_spin_cap = int(decode_spin_cap)
        p.kernel = int(kernel)
        # validation needs the layout's pointers; they are overwritten per call
        _set_pointers(p, q, k, v, out, qi, kvi, kt, vt)
        with torch.cuda.device(dev):
            ws_bytes = _fa2.workspace_size(p, decode)
        cached = (bytes(p), ws_bytes)
        if len(_PLAN_CACHE) >= _PLAN_CACHE_MAX:
            _PLAN_CACHE.clear()
        _PLAN_CACHE[key] = cached

    p = _fa2.Fa2Params.from_buffer_copy(cached[0])
    ws_bytes = cached[1]
    _set_pointers(p, q, k, v, out, qi, kvi, kt, vt)

    switch = dev.index != torch.cuda.current_device()
    if switch:
        prev = torch.cuda.current_device()
        torch.cuda.set_device(dev)
    try:
        handle = _stream_handle(dev)
        if noalloc:
            assert not decode, "fa2_fwd_noalloc serves the prefill entry point"
            _fa2.forward_noalloc(p, handle)
            return
        ws = None
        if ws_bytes:
            if workspace is not None:
                if workspace.numel() < ws_bytes or workspace.device != dev:
                    raise ValueError(f"workspace needs {ws_bytes} bytes on {dev}")
                ws = workspace
            else:
                ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
            p.workspace, p.workspace_bytes = ws.data_ptr(), ws_bytes
        _fa2.forward(p, handle, decode)
        if ws is not None:
            ws.record_stream(torch.cuda.current_stream(dev))
    finally:
        if switch:
            torch.cuda.set_device(prev)


def _set_pointers(p, q, k, v, out, qi, kvi, kt, vt) -> None:
    p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    if qi is not None:
        p.q_indptr = qi.data_ptr()
    if kvi is not None:
        p.kv_indptr = kvi.data_ptr()
    if kt is not None:
        p.k_block_table, p.v_block_table = kt.data_ptr(), vt.data_ptr()
