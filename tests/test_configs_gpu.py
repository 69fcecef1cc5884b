"""Parity of flash_attention_v2 on the BASELINE.json workloads at full size.

Each workload is built by ``workloads.make`` (the seeded inputs bench.py
times) and run once through the C ABI; the whole output is then checked on
the GPU, sequence by sequence:

1. the reference suite's bar (tests/test_attention.py:80-98, 246-251):
   ``assert_close`` against fp32 attention with ``atol = base*sqrt(N) + eps``;
2. a strict bar over every element: the error against fp64 attention must
   stay within 4x (max) and 2x (RMS) of the error of an fp64 emulation of
   the kernel's rounding (operands and softmax weights rounded as the kernel
   rounds them, output rounded to the dtype) - the reference tolerance alone
   is nearly vacuous at these lengths; for bf16 the same bar also against an
   emulation of the reference's arithmetic, which rounds bf16 operands and
   the softmax weights to fp16;
3. the strict bar against the C oracle (the restatement of the reference
   algorithm, oracle/fa2_oracle.c) on sampled windows - a range of query rows
   of a few query heads of one (sequence, kv head) - with their fp64 truth on
   the CPU.

These runs take the launch paths of the benchmark itself: the persistent
two-head kernel walks several units per workgroup (c2: 512 units on one
workgroup per CU), the plan kernel orders ragged (c3) and paged (c4) work,
and c5 fp32 runs the register-staged kernel.
"""

from __future__ import annotations

import concurrent.futures as cf

import pytest
import torch

import oracle
import workloads as W
from parity import gpu_attention, strict_check

pytestmark = pytest.mark.gpu

DEV = "cuda"

CONFIGS = [
    ("c1", torch.float16, None),
    ("c2", torch.float16, None),
    ("c2", torch.bfloat16, None),
    ("c3", torch.bfloat16, None),
    ("c4", torch.bfloat16, "bottom_right"),
    ("c4", torch.bfloat16, "top_left"),
    ("c5", torch.bfloat16, None),
    ("c5", torch.float32, None),
]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X")
    from kernels import _fa2
    _fa2.lib()
    yield


def kernel_rounding(dtype):
    """(operand_round, p_round) of the kernels for flash_attention_v2: fp32
    operands are rounded to fp16 as the reference does; P to the MFMA type."""
    if dtype == torch.float32:
        return "f16", "f16"
    return None, oracle.mma_round_for(dtype)


def windows(w, n=3):
    """Sampled (sequence, kv head, first q head, heads, row0, row1) windows
    of about 0.5 GFLOP each: the first, a middle and the last rows of
    different sequences and kv heads."""
    g = w.q_heads // w.kv_heads
    nh = min(g, 4)
    B = len(w.q_lens)
    res = []
    for i in range(n):
        b = (i * 7) % B
        kvh = (i * 3) % w.kv_heads
        h0 = kvh * g + (i % (g // nh)) * nh
        Lq, Lk = w.q_lens[b], w.kv_lens[b]
        rows = max(8, min(64, int(0.5e9 / (4 * w.head_dim * nh * max(Lk, 1)))))
        rows = min(rows, Lq)
        r0 = [0, max(0, (Lq - rows) // 2), Lq - rows][i % 3]
        res.append((b, kvh, h0, nh, r0, r0 + rows))
    return res


def window_inputs(w, qs, ks, vs, win):
    """q [1,nh,rows,D], k/v [1,1,Lk',D] and the mask of a window, equivalent
    to rows r0..r1 of the full problem (a causal window keeps the keys up to
    its last row's diagonal and aligns bottom-right, so row i still sees
    keys j <= i + off)."""
    b, kvh, h0, nh, r0, r1 = win
    Lq, Lk = w.q_lens[b], w.kv_lens[b]
    q = qs[b][r0:r1, h0:h0 + nh].transpose(0, 1).unsqueeze(0)
    if w.is_causal:
        off = (Lk - Lq) if w.causal_alignment == "bottom_right" else 0
        kend = r1 + off
        assert 0 < kend <= Lk
    else:
        kend = Lk
    k = ks[b][:kend, kvh:kvh + 1].transpose(0, 1).unsqueeze(0)
    v = vs[b][:kend, kvh:kvh + 1].transpose(0, 1).unsqueeze(0)
    return q, k, v, ("bottom_right" if w.is_causal else "top_left")


@pytest.mark.parametrize("name,dtype,alignment", CONFIGS,
                         ids=[f"{n}-{str(d)[6:]}-{a or 'default'}" for n, d, a in CONFIGS])
def test_config_full_size(name, dtype, alignment):
    print(f"config {name} {dtype} alignment={alignment}", flush=True)
    from kernels.attention import flash_attention_v2

    w_cpu = W.make(name, dtype=dtype, causal_alignment=alignment)
    w = w_cpu.to(DEV)
    out = flash_attention_v2(w.q, w.k, w.v, **w.kwargs())
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == w.q.shape

    outs = W.split_output(w, out)
    qs, ks, vs = W.sequences(w)
    align = w.causal_alignment if w.is_causal else "top_left"
    o_round, p_round = kernel_rounding(dtype)
    tol = oracle.attn_tolerances(dtype, max(w.kv_lens))
    # bf16: also the reference's own arithmetic (operands and P rounded to
    # fp16, attention.py:547, 572, 607, 614, 633)
    ref_arith = dtype == torch.bfloat16
    kern, emul, truth, emul_ref = [], [], [], []
    for b in range(len(outs)):
        qb, kb, vb = (t.transpose(0, 1) for t in (qs[b], ks[b], vs[b]))  # [H, L, D]
        ob = outs[b].transpose(0, 1).float()
        ref32 = gpu_attention(qb, kb, vb, w.is_causal, align)
        torch.testing.assert_close(ob, ref32, **tol)  # the reference suite's bar
        del ref32
        t64 = gpu_attention(qb, kb, vb, w.is_causal, align, dtype=torch.float64)
        e64 = gpu_attention(qb, kb, vb, w.is_causal, align, dtype=torch.float64,
                            operand_round=o_round, p_round=p_round)
        kern.append(ob)
        emul.append(e64.float())
        truth.append(t64)
        del t64, e64
        if ref_arith:
            emul_ref.append(gpu_attention(qb, kb, vb, w.is_causal, align, dtype=torch.float64,
                                          operand_round="f16", p_round="f16").float())
    stats = strict_check(kern, emul, truth, dtype)  # on the GPU
    print(f"  whole output: {stats}", flush=True)
    if ref_arith:
        st = strict_check(kern, emul_ref, truth, dtype)
        print(f"  whole output vs the reference's fp16 arithmetic: {st}", flush=True)
        del emul_ref
    kern = [t.cpu() for t in kern]
    del emul, truth

    # the C oracle (the reference algorithm) on sampled windows, in parallel
    qc, kc, vc = W.sequences(w_cpu)

    def one(win):
        q, k, v, al = window_inputs(w_cpu, qc, kc, vc, win)
        emu = oracle.oracle_attention(q, k, v, is_causal=w.is_causal, causal_alignment=al,
                                      operand_round=o_round or "none", p_round=p_round)
        tr = oracle.sdpa_reference([q[0].transpose(0, 1)], [k[0].transpose(0, 1)],
                                   [v[0].transpose(0, 1)], q.shape[1], 1, False,
                                   dtype=torch.float64) if not w.is_causal else \
            oracle.sdpa_reference_bottom_right([q[0].transpose(0, 1)], [k[0].transpose(0, 1)],
                                               [v[0].transpose(0, 1)], q.shape[1], 1,
                                               dtype=torch.float64)
        return emu[0].transpose(0, 1), tr[0]

    wins = windows(w_cpu)
    with cf.ThreadPoolExecutor(len(wins)) as ex:
        res = list(ex.map(one, wins))
    for win, (emu, tr) in zip(wins, res):
        b, kvh, h0, nh, r0, r1 = win
        kw = kern[b][h0:h0 + nh, r0:r1].transpose(0, 1)
        st = strict_check([kw], [emu], [tr], dtype)
        print(f"  window {win}: {st}", flush=True)
