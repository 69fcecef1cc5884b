"""CPU oracle for ``flash_attention_v2``, ``decode_attention`` and
``speculative_decode_attention`` (harsh-vsingh/triton-kernels).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` import this package, and only as the
checker.  The product path (``triton-kernels_amd/kernels``) never imports it.

Two restatements live here:

* :func:`oracle_attention` - ctypes front end of ``fa2_oracle.c``, a C
  restatement of the reference algorithm itself: the split-K partial kernel
  and the log-sum-exp merge of ``kernels/attention.py:430-746`` with the host
  logic of ``:749-927`` (layouts, ``kv_indptr`` meaning, block-table
  indexing, top-left causal mask).  It can round operands and P the way the
  reference does (fp16) or the way the bf16 MFMA kernel does, which gives
  the error floor the strict parity check compares against.
* :func:`sdpa_reference` / :func:`sdpa_reference_bottom_right` - the
  reference test suite's own oracle, per-sequence fp32
  ``F.scaled_dot_product_attention`` with ``repeat_interleave``d KV heads
  (``tests/test_attention.py:80-98``), and the explicit bottom-right mask
  construction of ``tests/test_speculative_decode.py:101-114``.
* :func:`attn_tolerances` - the tolerance formula of
  ``tests/test_attention.py:20-30`` (identical in ``tests/test_decode.py:20-30``
  and ``tests/test_speculative_decode.py:20-30``).
* :func:`oracle_decode` - the C restatement of ``decode_attention`` and
  ``speculative_decode_attention`` (``kernels/decode.py``,
  ``kernels/speculative_decode.py``: split kernel with strided key blocks,
  guarded max of the speculative kernel, log-sum-exp merge), and
  :func:`sdpa_decode_reference` / :func:`sdpa_speculative_reference`, those
  suites' own SDPA oracles.

How the C restatement is pinned (tests/test_oracle.py): against fp64 SDPA
(a library routine) on every layout/mask/topology, against committed golden
fixtures written by torch SDPA (tests/golden/), against closed forms
(constant V, one key, equal keys -> prefix means, a dominant logit) and
invariances (layout equivalence, split-K invariance, key permutation, GQA as
repeated heads), and against planted mistakes that each check must catch.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
import threading

import torch
import torch.nn.functional as F

_HERE = os.path.dirname(os.path.abspath(__file__))
# FA2_ORACLE_LIBRARY selects a prebuilt oracle library (the sanitizer build,
# oracle/_san/liboracle.so); build() then leaves it as it is.
_LIB_PATH = os.environ.get("FA2_ORACLE_LIBRARY") or os.path.join(_HERE, "liboracle.so")
_OVERRIDDEN = bool(os.environ.get("FA2_ORACLE_LIBRARY"))
_lib = None
_lock = threading.Lock()

LAYOUT = {"dense": 0, "ragged": 1, "paged": 2}
MASK = {"none": 0, "top_left": 1, "bottom_right": 2}
ROUND = {None: 0, "none": 0, "f16": 1, "bf16": 2}


class _Args(ctypes.Structure):
    _fields_ = [
        ("layout", ctypes.c_int32),
        ("mask", ctypes.c_int32),
        ("operand_round", ctypes.c_int32),
        ("p_round", ctypes.c_int32),
        ("block_m", ctypes.c_int32),
        ("block_n", ctypes.c_int32),
        ("split_k", ctypes.c_int32),
        ("mutation", ctypes.c_int32),
    ] + [(n, ctypes.c_int64) for n in (
        "batch", "q_heads", "kv_heads", "head_dim", "q_len", "kv_len",
        "q_sb", "q_sh", "q_ss", "k_sb", "k_sh", "k_ss",
        "v_sb", "v_sh", "v_ss", "o_sb", "o_sh", "o_ss")] + [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("q_indptr", ctypes.c_void_p),
        ("kv_indptr", ctypes.c_void_p),
        ("k_table", ctypes.c_void_p),
        ("v_table", ctypes.c_void_p),
        ("k_table_stride", ctypes.c_int64),
        ("v_table_stride", ctypes.c_int64),
        ("page_size", ctypes.c_int64),
        ("scale", ctypes.c_float),
        ("reserved2", ctypes.c_int32),
    ]


def build(force: bool = False) -> str:
    """Compile ``liboracle.so`` with gcc (oracle/Makefile)."""
    if _OVERRIDDEN:
        return _LIB_PATH
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def _load():
    global _lib
    with _lock:
        if _lib is None:
            build()
            lib = ctypes.CDLL(_LIB_PATH)
            lib.fa2o_fwd.argtypes = [ctypes.POINTER(_Args)]
            lib.fa2o_fwd.restype = ctypes.c_int
            lib.fa2o_decode.argtypes = [ctypes.POINTER(_Args), ctypes.c_int]
            lib.fa2o_decode.restype = ctypes.c_int
            lib.fa2o_round_f16.argtypes = [ctypes.c_float]
            lib.fa2o_round_f16.restype = ctypes.c_float
            lib.fa2o_round_bf16.argtypes = [ctypes.c_float]
            lib.fa2o_round_bf16.restype = ctypes.c_float
            _lib = lib
    return _lib


def round_scalar(x: float, mode: str) -> float:
    lib = _load()
    return lib.fa2o_round_f16(x) if mode == "f16" else lib.fa2o_round_bf16(x)


def _strides3(t: torch.Tensor):
    """(batch, head, row) element strides; token-major tensors: (0, head, token)."""
    if t.dim() == 4:
        return t.stride(0), t.stride(1), t.stride(2)
    return 0, t.stride(1), t.stride(0)


def oracle_attention(q, k, v, *, is_causal=False, q_indptr=None, kv_indptr=None,
                     k_block_table=None, v_block_table=None, kv_page_size=None,
                     causal_alignment="top_left", operand_round="f16", p_round="f16",
                     block_m=64, block_n=64, split_k=1, scale=None, mutation=0):
    """C restatement of ``flash_attention_v2`` on CPU; returns fp32 output.

    Same arguments and layout rules as the reference entry point
    (kernels/attention.py:749-760).  ``operand_round`` / ``p_round`` select
    the rounding of q,k,v and of P ("f16" is the reference's; "bf16";
    "none" = exact fp32 arithmetic).  ``block_n`` / ``split_k`` are the
    reference's autotuned tile and split factor (:367-429, :836-841).
    """
    paged = k_block_table is not None
    ragged = (q_indptr is not None) and not paged
    qf = q.detach().to("cpu", torch.float32).contiguous()
    kf = k.detach().to("cpu", torch.float32).contiguous()
    vf = v.detach().to("cpu", torch.float32).contiguous()
    out = torch.zeros_like(qf)
    a = _Args()
    a.layout = LAYOUT["paged" if paged else ("ragged" if ragged else "dense")]
    a.mask = MASK[causal_alignment] if is_causal else 0
    a.operand_round = ROUND[operand_round]
    a.p_round = ROUND[p_round]
    a.block_m, a.block_n, a.split_k = block_m, block_n, split_k
    a.mutation = int(mutation)
    keep = []
    if paged:
        a.batch, a.q_heads, a.q_len, a.head_dim = qf.shape
        a.kv_heads = kf.shape[1]
        a.kv_len = 0
        kvi = kv_indptr.detach().to("cpu", torch.int32).contiguous()
        kt = k_block_table.detach().to("cpu", torch.int32).contiguous()
        vt = v_block_table.detach().to("cpu", torch.int32).contiguous()
        keep += [kvi, kt, vt]
        a.kv_indptr, a.k_table, a.v_table = kvi.data_ptr(), kt.data_ptr(), vt.data_ptr()
        a.k_table_stride, a.v_table_stride = kt.stride(0), vt.stride(0)
        a.page_size = int(kv_page_size)
    elif ragged:
        a.q_len, a.q_heads, a.head_dim = qf.shape
        a.kv_len, a.kv_heads = kf.shape[0], kf.shape[1]
        a.batch = q_indptr.numel() - 1
        qi = q_indptr.detach().to("cpu", torch.int32).contiguous()
        kvi = kv_indptr.detach().to("cpu", torch.int32).contiguous()
        keep += [qi, kvi]
        a.q_indptr, a.kv_indptr = qi.data_ptr(), kvi.data_ptr()
    else:
        a.batch, a.q_heads, a.q_len, a.head_dim = qf.shape
        a.kv_heads, a.kv_len = kf.shape[1], kf.shape[2]
    a.q_sb, a.q_sh, a.q_ss = _strides3(qf)
    a.k_sb, a.k_sh, a.k_ss = _strides3(kf)
    a.v_sb, a.v_sh, a.v_ss = _strides3(vf)
    a.o_sb, a.o_sh, a.o_ss = _strides3(out)
    a.q, a.k, a.v, a.o = qf.data_ptr(), kf.data_ptr(), vf.data_ptr(), out.data_ptr()
    a.scale = float(a.head_dim ** -0.5 if scale is None else scale)
    rc = _load().fa2o_fwd(ctypes.byref(a))
    if rc != 0:
        raise RuntimeError(f"fa2o_fwd failed with code {rc}")
    return out


def oracle_v1(q, k, v, *, is_causal=False, q_indptr=None, kv_indptr=None, k_block_table=None,
              v_block_table=None, kv_page_size=None, block_n=64, scale=None):
    """``flash_attention_v1``'s arithmetic (kernels/attention.py:164-244): the
    same layouts, top-left mask and online softmax as v2, without split-K, with
    q, k, v cast to fp32 (:177, :196-197, :228) and the weights P kept in fp32
    for P.V (:225-240) - i.e. the C restatement with no rounding of operands
    or P and one split.  (Triton's default fp32 ``tl.dot`` on NVIDIA rounds
    its inputs to TF32; this restates the fp32 arithmetic the source asks for.)"""
    return oracle_attention(q, k, v, is_causal=is_causal, q_indptr=q_indptr, kv_indptr=kv_indptr,
                            k_block_table=k_block_table, v_block_table=v_block_table,
                            kv_page_size=kv_page_size, operand_round="none", p_round="none",
                            block_n=block_n, split_k=1, scale=scale)


def oracle_decode(q, k, v, *, causal=False, kv_indptr=None, k_block_table=None,
                  v_block_table=None, kv_page_size=None, spec=None, operand_round="none",
                  p_round="none", block_n=64, split_k=1, scale=None, mutation=0):
    """C restatement of ``decode_attention`` (q ``[B,QH,D]``) or
    ``speculative_decode_attention`` (q ``[B,QH,M,D]``) on CPU; fp32 output
    of q's shape.

    Same arguments and layout rules as the reference entry points
    (kernels/decode.py:203-331, kernels/speculative_decode.py:228-365).
    ``spec`` selects the speculative kernel's guarded max (default: True for
    4-D q).  Default rounding "none" is the reference's fp32 arithmetic;
    ``block_n`` / ``split_k`` are its autotuned block and split factor.
    """
    if spec is None:
        spec = q.dim() == 4
    q4 = q if q.dim() == 4 else q.unsqueeze(2)
    paged = k_block_table is not None
    ragged = (kv_indptr is not None) and not paged
    qf = q4.detach().to("cpu", torch.float32).contiguous()
    kf = k.detach().to("cpu", torch.float32)
    vf = v.detach().to("cpu", torch.float32)
    if paged and kf.dim() == 4:  # [pages, page, KVH, D]
        kf = kf.reshape(-1, kf.shape[2], kf.shape[3])
        vf = vf.reshape(-1, vf.shape[2], vf.shape[3])
    kf = kf.contiguous()
    vf = vf.contiguous()
    out = torch.zeros_like(qf)
    a = _Args()
    a.layout = LAYOUT["paged" if paged else ("ragged" if ragged else "dense")]
    a.mask = MASK["bottom_right"] if causal else 0
    a.operand_round = ROUND[operand_round]
    a.p_round = ROUND[p_round]
    a.block_m, a.block_n, a.split_k = 1, block_n, split_k
    a.mutation = int(mutation)
    a.batch, a.q_heads, a.q_len, a.head_dim = qf.shape
    keep = []
    if paged:
        a.kv_heads, a.kv_len = kf.shape[1], 0
        kvi = kv_indptr.detach().to("cpu", torch.int32).contiguous()
        kt = k_block_table.detach().to("cpu", torch.int32).contiguous()
        vt = v_block_table.detach().to("cpu", torch.int32).contiguous()
        keep += [kvi, kt, vt]
        a.kv_indptr, a.k_table, a.v_table = kvi.data_ptr(), kt.data_ptr(), vt.data_ptr()
        a.k_table_stride, a.v_table_stride = kt.stride(0), vt.stride(0)
        a.page_size = int(kv_page_size)
    elif ragged:
        a.kv_heads, a.kv_len = kf.shape[1], kf.shape[0]
        kvi = kv_indptr.detach().to("cpu", torch.int32).contiguous()
        keep.append(kvi)
        a.kv_indptr = kvi.data_ptr()
    else:
        a.kv_heads, a.kv_len = kf.shape[1], kf.shape[2]
    a.q_sb, a.q_sh, a.q_ss = _strides3(qf)
    a.k_sb, a.k_sh, a.k_ss = _strides3(kf)
    a.v_sb, a.v_sh, a.v_ss = _strides3(vf)
    a.o_sb, a.o_sh, a.o_ss = _strides3(out)
    a.q, a.k, a.v, a.o = qf.data_ptr(), kf.data_ptr(), vf.data_ptr(), out.data_ptr()
    a.scale = float(a.head_dim ** -0.5 if scale is None else scale)
    rc = _load().fa2o_decode(ctypes.byref(a), int(bool(spec)))
    if rc != 0:
        raise RuntimeError(f"fa2o_decode failed with code {rc}")
    return out if q.dim() == 4 else out.squeeze(2)


# ---------------------------------------------------------------------------
# The reference test suites' oracles (tests/test_attention.py:80-98,
# tests/test_decode.py:75-99, tests/test_speculative_decode.py:69-126).
# ---------------------------------------------------------------------------

def sdpa_reference(qs, ks, vs, QH, KVH, is_causal, dtype=torch.float32):
    """Per-sequence SDPA on [L,H,D] tensors; returns [L,H,D] in ``dtype``.

    Mirrors tests/test_attention.py:80-98: upcast, repeat_interleave the KV
    heads for GQA/MQA, ``is_causal`` (top-left).  ``dtype=torch.float64``
    gives the exact reference used to measure error floors.
    """
    refs = []
    for q, k, v in zip(qs, ks, vs):
        q_ref = q.transpose(0, 1).unsqueeze(0).to(dtype)
        k_ref = k.transpose(0, 1).unsqueeze(0).to(dtype)
        v_ref = v.transpose(0, 1).unsqueeze(0).to(dtype)
        if QH != KVH:
            g = QH // KVH
            k_ref = k_ref.repeat_interleave(g, dim=1)
            v_ref = v_ref.repeat_interleave(g, dim=1)
        out = F.scaled_dot_product_attention(q_ref, k_ref, v_ref, is_causal=is_causal)
        refs.append(out.squeeze(0).transpose(0, 1))
    return refs


def sdpa_reference_bottom_right(qs, ks, vs, QH, KVH, dtype=torch.float32):
    """Bottom-right causal SDPA (query i sees key j iff j <= i + Lk - Lq).

    Explicit boolean mask built like tests/test_speculative_decode.py:101-114.
    Rows with no visible key are returned as NaN (the reference's 0/0).
    """
    refs = []
    for q, k, v in zip(qs, ks, vs):
        Lq, Lk = q.shape[0], k.shape[0]
        q_ref = q.transpose(0, 1).unsqueeze(0).to(dtype)
        k_ref = k.transpose(0, 1).unsqueeze(0).to(dtype)
        v_ref = v.transpose(0, 1).unsqueeze(0).to(dtype)
        if QH != KVH:
            g = QH // KVH
            k_ref = k_ref.repeat_interleave(g, dim=1)
            v_ref = v_ref.repeat_interleave(g, dim=1)
        mask = torch.ones((Lq, Lk), dtype=torch.bool)
        for i in range(Lq):
            mask[i, max(Lk - Lq + i + 1, 0):] = False
        out = F.scaled_dot_product_attention(q_ref, k_ref, v_ref, attn_mask=mask)
        out = out.squeeze(0).transpose(0, 1).clone()
        empty = ~mask.any(dim=1)
        out[empty] = float("nan")
        refs.append(out)
    return refs


def sdpa_decode_reference(qs, ks, vs, QH, KVH, dtype=torch.float32):
    """tests/test_decode.py:75-99: per sequence, q ``[QH,D]`` against k/v
    ``[L,KVH,D]``, upcast, KV heads repeat_interleaved; returns ``[QH,D]``."""
    refs = []
    for q, k, v in zip(qs, ks, vs):
        q_ref = q.unsqueeze(0).unsqueeze(2).to(dtype)
        k_ref = k.transpose(0, 1).unsqueeze(0).to(dtype)
        v_ref = v.transpose(0, 1).unsqueeze(0).to(dtype)
        if QH != KVH:
            g = QH // KVH
            k_ref = k_ref.repeat_interleave(g, dim=1)
            v_ref = v_ref.repeat_interleave(g, dim=1)
        refs.append(F.scaled_dot_product_attention(q_ref, k_ref, v_ref).squeeze(0).squeeze(1))
    return refs


def sdpa_speculative_reference(qs, ks, vs, dks, dvs, QH, KVH, causal, dtype=torch.float32):
    """tests/test_speculative_decode.py:69-126: per sequence, q ``[QH,M,D]``
    against the context k/v ``[L,KVH,D]`` plus, when causal, the M draft
    rows ``dks``/``dvs`` ``[M,KVH,D]`` appended and hidden from earlier drafts
    (mask row i: keys ``> L + i`` off); returns ``[QH,M,D]``."""
    refs = []
    for q, k, v, dk, dv in zip(qs, ks, vs, dks, dvs):
        q_ref = q.unsqueeze(0).to(dtype)
        k_ref = k.transpose(0, 1).unsqueeze(0).to(dtype)
        v_ref = v.transpose(0, 1).unsqueeze(0).to(dtype)
        if causal:
            k_ref = torch.cat([k_ref, dk.transpose(0, 1).unsqueeze(0).to(dtype)], dim=2)
            v_ref = torch.cat([v_ref, dv.transpose(0, 1).unsqueeze(0).to(dtype)], dim=2)
        if QH != KVH:
            g = QH // KVH
            k_ref = k_ref.repeat_interleave(g, dim=1)
            v_ref = v_ref.repeat_interleave(g, dim=1)
        mask = None
        if causal:
            M = q_ref.shape[2]
            N = k_ref.shape[2] - M
            mask = torch.ones((M, N + M), dtype=torch.bool)
            for i in range(M):
                mask[i, N + i + 1:] = False
        refs.append(F.scaled_dot_product_attention(q_ref, k_ref, v_ref, attn_mask=mask,
                                                   is_causal=False).squeeze(0))
    return refs


BASE_TOL = {
    torch.float16: dict(base_atol=1e-2, rtol=1e-2, eps=2e-3),
    torch.bfloat16: dict(base_atol=2e-2, rtol=2e-2, eps=4e-3),
    torch.float32: dict(base_atol=1e-3, rtol=1e-2, eps=2e-3),
}


def attn_tolerances(dtype, N):
    """tests/test_attention.py:20-30: atol = base_atol*sqrt(max(N,1)) + eps."""
    cfg = BASE_TOL[dtype]
    atol = cfg["base_atol"] * math.sqrt(max(N, 1)) + cfg["eps"]
    return dict(atol=atol, rtol=cfg["rtol"])


def mma_round_for(dtype) -> str:
    """Rounding of the MFMA operands/P in the HIP kernels for a tensor dtype."""
    return "bf16" if dtype == torch.bfloat16 else "f16"
