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
    mx, ss, n = 0.0, 0.0, 0
    for o, r in zip(outs, refs):
        d = o.double().cpu() - r.double().cpu()
        fin = ~torch.isnan(r.double().cpu())
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
        assert torch.equal(torch.isnan(o.float().cpu()), torch.isnan(t.cpu())), "NaN pattern differs"
    emul_r = [e.to(dtype).float() for e in emul]
    k_max, k_rms = _stats(outs, truth64)
    e_max, e_rms = _stats(emul_r, truth64)
    floor = ULP[dtype]
    assert k_max <= scale_max * e_max + floor, (k_max, e_max)
    assert k_rms <= scale_rms * e_rms + floor / 4, (k_rms, e_rms)
    return dict(kernel_max=k_max, kernel_rms=k_rms, emul_max=e_max, emul_rms=e_rms)


def gpu_reference(q, k, v, is_causal, alignment="top_left", scale=None, row_chunk=2048):
    """fp32 attention on the GPU for one sequence, q [Hq,Lq,D], k/v [Hkv,Lk,D].

    Explicit fp32 matmuls with TF32 off (the SDPA math path, written out so
    the reference never depends on a fused kernel); rows with no visible key
    come out NaN like the reference's 0/0."""
    Hq, Lq, D = q.shape
    Hkv, Lk, _ = k.shape
    g = Hq // Hkv
    sc = D ** -0.5 if scale is None else scale
    kf = k.float().repeat_interleave(g, 0)
    vf = v.float().repeat_interleave(g, 0).contiguous()
    kt = kf.transpose(1, 2).contiguous()
    out = torch.empty((Hq, Lq, D), dtype=torch.float32, device=q.device)
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        off = (Lk - Lq) if alignment == "bottom_right" else 0
        for r0 in range(0, Lq, row_chunk):
            r1 = min(Lq, r0 + row_chunk)
            s = torch.matmul(q[:, r0:r1].float().contiguous(), kt) * sc
            if is_causal:
                i = torch.arange(r0, r1, device=q.device)[:, None]
                j = torch.arange(Lk, device=q.device)[None, :]
                s = s.masked_fill(j > i + off, float("-inf"))
            p = torch.softmax(s, dim=-1)
            out[:, r0:r1] = torch.matmul(p, vf)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    return out
