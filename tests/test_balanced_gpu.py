"""GPU checks of the two-head kernel's balanced walk (paged K/V, one q-block
per sequence, more two-head units than CUs: csrc/fa2_kernel_pp.h,
pp_bal_locate).

The units of each XCD form one stream per head pair, cut into segments of
equal KV-tile counts, one per workgroup; a unit that a segment boundary cuts
runs as pieces whose partials the last piece to finish merges.  The cut
points follow from the sequence lengths alone, so:

* the output passes the oracle bars (as every path does);
* two calls give the same bits;
* a unit that no boundary cuts gives the same bits as the rounds of whole
  units that max_workgroups > 0 keeps (each unit's arithmetic does not
  depend on where it runs); a cut unit stays within the merge's rounding;
* the merge words need no clearing: whatever the workspace held, the bits
  are those of a fresh workspace.

`split_units` restates the cut points in Python, from the kernel's rule.
"""

import dataclasses
import random

import pytest
import torch

from attn_cases import make_case, pack, unpack
from test_attention_gpu import check_all

pytestmark = pytest.mark.gpu

DEV = "cuda"
XCDS = 8
BN, BM = 64, 128


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X")
    from kernels import _fa2
    _fa2.lib()
    yield


def cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def tiles(Lq, Lk, causal, alignment):
    """KV tiles of a sequence's only q-block (kv_end_for_block)."""
    if not causal:
        end = Lk
    else:
        off = Lk - Lq if alignment == "bottom_right" else 0
        end = max(0, min(Lk, min(BM, Lq) + off))
    return (end + BN - 1) // BN


def split_units(batch, QH, KVH, Lq, kv_lens, causal, alignment, P):
    """(sequence, kv head, head pair) of every unit the balanced walk cuts."""
    group = QH // KVH
    upp = (group + 1) // 2
    npairs = batch * KVH
    cut = set()
    for x in range(XCDS):
        nx = (P - x + XCDS - 1) // XCDS
        ns = nx // upp
        pairs = list(range(x, npairs, XCDS))
        w = [max(tiles(Lq, kv_lens[p // KVH], causal, alignment), 1) for p in pairs]
        total = sum(w)
        C = -(-total // ns) if total > ns else 1
        us = 0
        for p, wt in zip(pairs, w):
            if (us + wt - 1) // C != us // C:
                for g in range(upp):
                    cut.add((p // KVH, p % KVH, g))
            us += wt
    return cut


def run(q, k, v, kw, causal, alignment, max_workgroups=0, workspace=None):
    """One forward call through the C ABI (workspace from torch, or the
    caller's)."""
    from kernels import _fa2
    from kernels._launch import enqueue, index_tensor, strides, table
    out = torch.empty_like(q)
    mask = (_fa2.MASK_NONE if not causal else
            _fa2.MASK_TOP_LEFT if alignment == "top_left" else _fa2.MASK_BOTTOM_RIGHT)
    B, Hq, M, D = q.shape
    N, Hkv = k.shape[0], k.shape[1]
    enqueue(decode=False, layout=_fa2.LAYOUT_PAGED, mask=mask, num_splits=0, batch=B,
            q_heads=Hq, kv_heads=Hkv, head_dim=D, q_len=M, kv_len=N, q=q, k=k, v=v, out=out,
            q_strides=strides(q), o_strides=strides(out),
            kvi=index_tensor(kw["kv_indptr"], q.device), kt=table(kw["k_block_table"], q.device),
            vt=table(kw["v_block_table"], q.device), page_size=kw["kv_page_size"],
            kv_len_max=kw["k_block_table"].shape[1] * kw["kv_page_size"],
            max_workgroups=max_workgroups, workspace=workspace)
    torch.cuda.synchronize()
    return out


def workspace_bytes(q, k, kw, causal, alignment):
    from kernels import _fa2
    from kernels._launch import strides
    p = _fa2.Fa2Params()
    p.layout, p.num_splits = _fa2.LAYOUT_PAGED, 0
    p.dtype = {torch.bfloat16: _fa2.DTYPE_BF16, torch.float16: _fa2.DTYPE_F16}[q.dtype]
    p.mask = (_fa2.MASK_NONE if not causal else
              _fa2.MASK_TOP_LEFT if alignment == "top_left" else _fa2.MASK_BOTTOM_RIGHT)
    p.batch, p.q_heads, p.q_len, p.head_dim = q.shape
    p.kv_heads, p.kv_len = k.shape[1], k.shape[0]
    p.page_size = kw["kv_page_size"]
    p.kv_len_max = kw["k_block_table"].shape[1] * kw["kv_page_size"]
    p.k_table_stride = p.v_table_stride = kw["k_block_table"].shape[1]
    p.q_sb, p.q_sh, p.q_ss = strides(q)
    p.o_sb, p.o_sh, p.o_ss = strides(q)
    p.k_sb, p.k_sh, p.k_ss = 0, k.stride(1), k.stride(0)
    p.v_sb, p.v_sh, p.v_ss = 0, k.stride(1), k.stride(0)
    p.softmax_scale = 1.0
    p.q = p.k = p.v = p.o = 16
    p.kv_indptr = p.k_block_table = p.v_block_table = 16
    with torch.cuda.device(q.device):
        return _fa2.workspace_size(p)


def balanced_case(B, QH, KVH, D, dtype, Lq, kv_lens, seed, causal, alignment):
    case = make_case(B, QH, KVH, D, "cross", dtype, "paged", seed, q_lens=[Lq] * B,
                     kv_lens=kv_lens)
    q, k, v, kw = pack(case, "paged", device=DEV, shuffled_pages=True, seed=seed)
    # the balanced walk's part slots (4 per workgroup) are what make its
    # workspace this large: the plan took it
    assert workspace_bytes(q, k, kw, causal, alignment) >= 4 * cus() * BM * (2 + D) * 4
    return case, q, k, v, kw


# (name, q heads, kv heads, D, dtype, Lq, causal, alignment, batch, kv length range)
CASES = [
    ("c4-like", 16, 4, 128, torch.bfloat16, 128, True, "bottom_right", 40, (128, 2600)),
    ("fp16-d64", 32, 8, 64, torch.float16, 128, False, "top_left", 20, (1, 2200)),
    ("group8", 32, 4, 128, torch.bfloat16, 77, False, "top_left", 40, (1, 1800)),
    ("top-left", 16, 4, 128, torch.float16, 100, True, "top_left", 40, (100, 1500)),
]


@pytest.mark.parametrize("cid", range(len(CASES)), ids=[c[0] for c in CASES])
def test_balanced_walk(cid):
    name, QH, KVH, D, dt, Lq, causal, align, B, (lo, hi) = CASES[cid]
    rng = random.Random(900 + cid)
    kv = [rng.randint(lo, hi) for _ in range(B)]
    if not causal:
        kv[:3] = [lo, 17, 64]
    print(f"balanced walk {name}: {QH}/{KVH} D{D} {dt} Lq{Lq} causal={causal} {align}",
          flush=True)
    case, q, k, v, kw = balanced_case(B, QH, KVH, D, dt, Lq, kv, 7000 + cid, causal, align)
    print("  balanced call", flush=True)
    bal = run(q, k, v, kw, causal, align)
    assert torch.equal(run(q, k, v, kw, causal, align).view(torch.int16), bal.view(torch.int16))
    print("  rounds call", flush=True)
    rounds = run(q, k, v, kw, causal, align, max_workgroups=cus())
    cut = split_units(B, QH, KVH, Lq, kv, causal, align, cus())
    assert 0 < len(cut) < B * KVH * ((QH // KVH + 1) // 2)
    group = QH // KVH
    n_eq = n_cut = 0
    for b in range(B):
        for h in range(QH):
            kvh, g = h // group, (h % group) // 2
            a, r = bal[b, h].float(), rounds[b, h].float()
            if (b, kvh, g) in cut:
                n_cut += 1
                assert torch.allclose(a, r, atol=2e-2, rtol=2e-2), (b, h)
            else:
                n_eq += 1
                assert torch.equal(bal[b, h].view(torch.int16), rounds[b, h].view(torch.int16)), (b, h)
    assert n_eq > 0 and n_cut > 0
    print("  gpu calls done; oracle on 4 sequences", flush=True)
    # the oracle on 2 sequences with cut units and 2 without (the emulated
    # oracle over all 40 takes minutes)
    cut_seqs = sorted({b for b, _, _ in cut})
    whole = [b for b in range(B) if b not in cut_seqs]
    sel = cut_seqs[:2] + whole[:2]
    outs = unpack(case, "paged", bal.cpu(), kw)
    sub = dataclasses.replace(case, qs=[case.qs[b] for b in sel], ks=[case.ks[b] for b in sel],
                              vs=[case.vs[b] for b in sel], q_lens=[case.q_lens[b] for b in sel],
                              kv_lens=[case.kv_lens[b] for b in sel])
    check_all(sub, "paged", causal, [outs[b] for b in sel], alignment=align)
    print("  oracle done", flush=True)


@pytest.mark.parametrize("fill", ["zeros", "ones", "random", "reused"])
def test_balanced_merge_words_need_no_clearing(fill):
    B, QH, KVH, D = 40, 16, 4, 128
    rng = random.Random(77)
    kv = [rng.randint(128, 2000) for _ in range(B)]
    print(f"balanced walk merge words, workspace {fill}", flush=True)
    case, q, k, v, kw = balanced_case(B, QH, KVH, D, torch.bfloat16, 128, kv, 7100, True,
                                      "bottom_right")
    n = workspace_bytes(q, k, kw, True, "bottom_right")
    ref = run(q, k, v, kw, True, "bottom_right",
              workspace=torch.zeros(n, dtype=torch.uint8, device=DEV))
    g = torch.Generator(device=DEV).manual_seed(5)
    ws = torch.zeros(n, dtype=torch.uint8, device=DEV)
    if fill == "ones":
        ws.fill_(255)
    elif fill == "random":
        ws.copy_(torch.randint(0, 256, (n,), generator=g, device=DEV, dtype=torch.uint8))
    elif fill == "reused":
        run(q, k, v, kw, True, "bottom_right", workspace=ws)
    for _ in range(2):
        out = run(q, k, v, kw, True, "bottom_right", workspace=ws)
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
