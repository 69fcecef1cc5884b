"""Parity helpers shared by the GPU tests, smoke() and bench.py checks.

Two bars, both against the same seeded inputs:

1. the reference test suite's bar (tests/test_attention.py:246-251):
   ``torch.testing.assert_close(out.float(), fp32 SDPA, atol=base*sqrt(N)+eps,
   rtol)`` per sequence;
2. a strict bar, because (1) is nearly vacuous at long KV: the kernel's error
   against fp64 SDPA must stay within 4x (max) and 2x (RMS) of the error of
   the CPU oracle run with the kernel's own operand/P rounding and rounded to
   the output dtype, plus a floor of one output ulp.
"""

from __future__ import annotations

import math

import torch

import oracle

ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7, torch.float32: 2.0 ** -20}


def reference_check(outs, refs32, dtype, N):
    tol = oracle.attn_tolerances(dtype, N)
    for o, r in zip(outs, refs32):
        torch.testing.assert_close(o.float().cpu(), r.float().cpu(), **tol)


def _stats(outs, refs):
    """Max and RMS of |o - r| over the elements where r is not NaN (on r's device)."""
    mx, ss, n = 0.0, 0.0, 0
    for o, r in zip(outs, refs):
        r = r.double()
        d = o.to(r.device).double() - r
        fin = ~torch.isnan(r)
        d = d[fin]
        if d.numel() == 0:
            continue
        mx = max(mx, d.abs().max().item())
        ss += (d * d).sum().item()
        n += d.numel()
    return mx, math.sqrt(ss / max(n, 1))


def strict_check(outs, emul, truth64, dtype, scale_max=4.0, scale_rms=2.0):
    """outs: kernel outputs; emul: oracle outputs with the kernel's rounding (fp32);
    truth64: fp64 SDPA.  Also requires NaN exactly where the truth has NaN."""
    for o, t in zip(outs, truth64):
        assert torch.equal(torch.isnan(o.to(t.device).float()), torch.isnan(t)), \
            "NaN pattern differs"
    emul_r = [e.to(dtype).float() for e in emul]  # (tensors may live on any one device)
    k_max, k_rms = _stats(outs, truth64)
    e_max, e_rms = _stats(emul_r, truth64)
    floor = ULP[dtype]
    assert k_max <= scale_max * e_max + floor, (k_max, e_max)
    assert k_rms <= scale_rms * e_rms + floor / 4, (k_rms, e_rms)
    return dict(kernel_max=k_max, kernel_rms=k_rms, emul_max=e_max, emul_rms=e_rms)


def gpu_attention(q, k, v, is_causal, alignment="top_left", scale=None, row_chunk=512,
                  dtype=torch.float32, operand_round=None, p_round=None):
    """Attention of one sequence on the GPU, q [Hq,Lq,D], k/v [Hkv,Lk,D].

    ``dtype`` float32 with no rounding is the reference suite's oracle (fp32
    SDPA math, tests/test_attention.py:80-98, written out as matmuls with
    TF32 off so it never depends on a fused kernel); float64 is the truth
    the strict bar measures errors against.  ``operand_round`` ("f16") and
    ``p_round`` ("f16"/"bf16") emulate a kernel's rounding: operands rounded
    before the products and the softmax weights exp(s - rowmax) rounded
    before the P.V product and the row sum (computed in ``dtype``).  Rows
    with no visible key come out NaN like the reference's 0/0.  Grouped heads
    are computed per kv head (no repeated K/V)."""
    Hq, Lq, D = q.shape
    Hkv, Lk, _ = k.shape
    g = Hq // Hkv
    sc = D ** -0.5 if scale is None else scale
    rdt = {None: None, "none": None, "f16": torch.float16, "bf16": torch.bfloat16}

    def prep(t):
        r = rdt[operand_round]
        t = t.to(r) if r is not None else t
        return t.to(dtype)

    out = torch.empty((Hq, Lq, D), dtype=dtype, device=q.device)
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        off = (Lk - Lq) if alignment == "bottom_right" else 0
        for h in range(Hkv):
            kt = prep(k[h]).transpose(0, 1).contiguous()  # [D, Lk]
            vh = prep(v[h]).contiguous()                   # [Lk, D]
            qh = prep(q[h * g:(h + 1) * g])                # [g, Lq, D]
            for r0 in range(0, Lq, row_chunk):
                r1 = min(Lq, r0 + row_chunk)
                s = torch.matmul(qh[:, r0:r1].contiguous(), kt) * sc
                if is_causal:
                    i = torch.arange(r0, r1, device=q.device)[:, None]
                    j = torch.arange(Lk, device=q.device)[None, :]
                    s = s.masked_fill(j > i + off, float("-inf"))
                m = s.amax(dim=-1, keepdim=True)
                p = torch.exp(s - m)
                if rdt[p_round] is not None:
                    p = p.to(rdt[p_round]).to(dtype)
                out[h * g:(h + 1) * g, r0:r1] = torch.matmul(p, vh) / p.sum(-1, keepdim=True)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    return out
