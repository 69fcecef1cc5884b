"""ctypes binding of ``libfa2.so`` (the C ABI declared in include/fa2.h).

The library is built in-tree by ``triton-kernels_amd/build.py`` (hipcc,
``--offload-arch=gfx950``).  There is no fallback: if the library is missing
or does not load, every call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
# FA2_LIBRARY selects another build of the same library, such as the
# host-sanitized one that build.py writes to triton-kernels_amd/_san/.
LIB_PATH = os.environ.get("FA2_LIBRARY") or os.path.join(_HERE, "libfa2.so")

LAYOUT_DENSE, LAYOUT_RAGGED, LAYOUT_PAGED = 0, 1, 2
DTYPE_F16, DTYPE_BF16, DTYPE_F32 = 0, 1, 2
MASK_NONE, MASK_TOP_LEFT, MASK_BOTTOM_RIGHT = 0, 1, 2
ARITH_REFERENCE, ARITH_FP32 = 0, 1
KERNEL_AUTO, KERNEL_REGULAR, KERNEL_SHORT = 0, 1, 2
MAX_SPLITS = 64

ABI_VERSION = 7

# Every symbol include/fa2.h declares.
EXPORTS = ("fa2_fwd_workspace_size", "fa2_fwd", "fa2_fwd_noalloc", "fa2_strerror",
           "fa2_decode_workspace_size", "fa2_decode_fwd", "fa2_decode_wait_giveups",
           "fa2_kv_append",
           "fa2_kv_append_params_size", "fa2_abi_version", "fa2_params_size")
NOALLOC_SCRATCH_BYTES = 32 << 20


class Fa2Params(ctypes.Structure):
    """Mirror of ``struct fa2_params`` (include/fa2.h)."""

    _fields_ = [
        ("layout", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("mask", ctypes.c_int32),
        ("num_splits", ctypes.c_int32),
        ("batch", ctypes.c_int64),
        ("q_heads", ctypes.c_int64),
        ("kv_heads", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("q_len", ctypes.c_int64),
        ("kv_len", ctypes.c_int64),
        ("q_sb", ctypes.c_int64), ("q_sh", ctypes.c_int64), ("q_ss", ctypes.c_int64),
        ("k_sb", ctypes.c_int64), ("k_sh", ctypes.c_int64), ("k_ss", ctypes.c_int64),
        ("v_sb", ctypes.c_int64), ("v_sh", ctypes.c_int64), ("v_ss", ctypes.c_int64),
        ("o_sb", ctypes.c_int64), ("o_sh", ctypes.c_int64), ("o_ss", ctypes.c_int64),
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("q_indptr", ctypes.c_void_p),
        ("kv_indptr", ctypes.c_void_p),
        ("k_block_table", ctypes.c_void_p),
        ("v_block_table", ctypes.c_void_p),
        ("k_table_stride", ctypes.c_int64),
        ("v_table_stride", ctypes.c_int64),
        ("page_size", ctypes.c_int64),
        ("softmax_scale", ctypes.c_float),
        ("max_workgroups", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("kv_len_max", ctypes.c_int64),
        ("arith", ctypes.c_int32),
        ("decode_spin_cap", ctypes.c_int32),
        ("kernel", ctypes.c_int32),
    ]


class KvAppendParams(ctypes.Structure):
    """Mirror of ``struct fa2_kv_append_params`` (include/fa2.h)."""

    _fields_ = [("dtype", ctypes.c_int32), ("reserved0", ctypes.c_int32)] + [
        (n, ctypes.c_int64) for n in (
            "batch", "kv_heads", "head_dim", "num_rows", "page_size", "num_pages",
            "table_width", "k_table_stride", "v_table_stride", "new_ts", "new_hs",
            "cache_ts", "cache_hs")] + [
        (n, ctypes.c_void_p) for n in (
            "k_new", "v_new", "k_cache", "v_cache", "new_indptr", "start_pos",
            "k_block_table", "v_block_table")]


_lib = None
_lock = threading.Lock()


def lib():
    """Load libfa2.so once; raise a clear error when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"flash_attention_v2: HIP library not built ({LIB_PATH} missing); "
                    "run `python triton-kernels_amd/build.py` (hipcc, gfx950)")
            L = ctypes.CDLL(LIB_PATH)
            L.fa2_fwd_workspace_size.argtypes = [ctypes.POINTER(Fa2Params),
                                                 ctypes.POINTER(ctypes.c_size_t)]
            L.fa2_fwd_workspace_size.restype = ctypes.c_int
            L.fa2_fwd.argtypes = [ctypes.POINTER(Fa2Params), ctypes.c_void_p]
            L.fa2_fwd.restype = ctypes.c_int
            L.fa2_fwd_noalloc.argtypes = [ctypes.POINTER(Fa2Params), ctypes.c_void_p]
            L.fa2_fwd_noalloc.restype = ctypes.c_int
            L.fa2_decode_workspace_size.argtypes = [ctypes.POINTER(Fa2Params),
                                                    ctypes.POINTER(ctypes.c_size_t)]
            L.fa2_decode_workspace_size.restype = ctypes.c_int
            L.fa2_decode_fwd.argtypes = [ctypes.POINTER(Fa2Params), ctypes.c_void_p]
            L.fa2_decode_fwd.restype = ctypes.c_int
            L.fa2_decode_wait_giveups.argtypes = [ctypes.POINTER(ctypes.c_uint32), ctypes.c_int]
            L.fa2_decode_wait_giveups.restype = ctypes.c_int
            L.fa2_kv_append.argtypes = [ctypes.POINTER(KvAppendParams), ctypes.c_void_p]
            L.fa2_kv_append.restype = ctypes.c_int
            L.fa2_kv_append_params_size.argtypes = []
            L.fa2_kv_append_params_size.restype = ctypes.c_size_t
            L.fa2_strerror.argtypes = [ctypes.c_int]
            L.fa2_strerror.restype = ctypes.c_char_p
            L.fa2_abi_version.argtypes = []
            L.fa2_abi_version.restype = ctypes.c_int
            L.fa2_params_size.argtypes = []
            L.fa2_params_size.restype = ctypes.c_size_t
            if (L.fa2_params_size() != ctypes.sizeof(Fa2Params) or
                    L.fa2_kv_append_params_size() != ctypes.sizeof(KvAppendParams)):
                raise RuntimeError("libfa2.so: parameter struct layout mismatch with the binding")
            if L.fa2_abi_version() != ABI_VERSION:
                raise RuntimeError(f"libfa2.so: ABI version {L.fa2_abi_version()}, binding "
                                   f"expects {ABI_VERSION}; rebuild the library")
            _lib = L
    return _lib


class Fa2Error(RuntimeError):
    def __init__(self, code: int):
        msg = lib().fa2_strerror(code).decode()
        super().__init__(f"flash_attention_v2: {msg} (fa2 status {code})")
        self.code = code


def workspace_size(p: Fa2Params, decode: bool = False) -> int:
    """Device workspace bytes of ``fa2_fwd`` (or ``fa2_decode_fwd``) for ``p``."""
    n = ctypes.c_size_t(0)
    fn = lib().fa2_decode_workspace_size if decode else lib().fa2_fwd_workspace_size
    rc = fn(ctypes.byref(p), ctypes.byref(n))
    if rc != 0:
        raise Fa2Error(rc)
    return n.value


def forward(p: Fa2Params, stream: int, decode: bool = False) -> None:
    """Enqueue ``fa2_fwd`` (or ``fa2_decode_fwd``) on the HIP stream ``stream``."""
    fn = lib().fa2_decode_fwd if decode else lib().fa2_fwd
    rc = fn(ctypes.byref(p), ctypes.c_void_p(stream))
    if rc != 0:
        raise Fa2Error(rc)


def decode_wait_giveups(reset: bool = False) -> int:
    """Workgroups of the fp16/bf16 decode kernel on the current device whose
    bounded ring waits gave up (their rows are NaN); ``reset`` zeroes the
    count.  Synchronous."""
    n = ctypes.c_uint32(0)
    rc = lib().fa2_decode_wait_giveups(ctypes.byref(n), 1 if reset else 0)
    if rc != 0:
        raise Fa2Error(rc)
    return n.value


def forward_noalloc(p: Fa2Params, stream: int) -> None:
    """Enqueue ``fa2_fwd_noalloc`` (no workspace: the library's static scratch)."""
    rc = lib().fa2_fwd_noalloc(ctypes.byref(p), ctypes.c_void_p(stream))
    if rc != 0:
        raise Fa2Error(rc)


def kv_append(p: KvAppendParams, stream: int) -> None:
    """Enqueue ``fa2_kv_append`` on the HIP stream ``stream``."""
    rc = lib().fa2_kv_append(ctypes.byref(p), ctypes.c_void_p(stream))
    if rc != 0:
        raise Fa2Error(rc)
