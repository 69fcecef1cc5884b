"""Seeded random configurations of flash_attention_v2 on the GPU.

The matrix tests vary one dimension at a time around fixed head counts; this
sweep draws every dimension at once from a seed (layout, dtype, head dim,
Hq/Hkv including odd group sizes, self/cross lengths, causal alignment, page
size with a shuffled pool, forced split count), so that combinations no
matrix row names (ragged cross attention with Lq > Lk under bottom-right
causal at head dim 256 and 3 splits, say) are checked against the same two
bars: the reference suite's tolerance (tests/test_attention.py:246-251) for
the reference's own semantics and the strict bar of tests/parity.py.

Sizes are bounded so the fp64 CPU truth of each case stays around a second.
"""

import random

import pytest
import torch

from attn_cases import make_case
from test_attention_gpu import DEV, _gpu, check_all, run_case  # noqa: F401  (fixture)

pytestmark = pytest.mark.gpu

HEADS = [(1, 1), (2, 1), (4, 4), (6, 2), (6, 3), (8, 2), (9, 3), (12, 4), (16, 1), (10, 5)]


def draw(seed):
    rng = random.Random(1000 + seed)
    layout = rng.choice(["dense", "ragged", "paged"])
    dtype = rng.choice([torch.float16, torch.bfloat16, torch.bfloat16, torch.float32])
    D = rng.choice([16, 32, 64, 64, 128, 128, 256])
    QH, KVH = rng.choice(HEADS)
    attn = rng.choice(["self", "cross"])
    causal = rng.random() < 0.6
    alignment = rng.choice(["top_left", "bottom_right"]) if causal else "top_left"
    B = rng.randint(1, 5)
    # keep B * QH * Lq * Lk * D (the fp64 truth's work) near 1e9 at most
    lmax = 700 if D <= 64 else (450 if D == 128 else 260)
    lmax = max(32, int(lmax * min(1.0, (8 / (B * QH)) ** 0.5)))
    q_hi = rng.randint(1, lmax)
    kv_hi = rng.randint(1, lmax)
    page = rng.choice([5, 8, 16, 16, 32])
    shuffled = layout == "paged" and rng.random() < 0.7
    splits = rng.choice([0, 0, 0, 2, 3, 5])
    # paged Q is one dense [B, Hq, M, D] block: under bottom-right causal every
    # sequence's diagonal sits at Lk_b - M, so all sequences get M query rows
    q_lens = None
    if layout == "paged" and alignment == "bottom_right":
        q_lens = [rng.randint(1, q_hi)] * B
    return dict(q_lens=q_lens, layout=layout, dtype=dtype, D=D, QH=QH, KVH=KVH, attn=attn, causal=causal,
                alignment=alignment, B=B, q_range=(1, q_hi), kv_range=(1, kv_hi),
                dense=(max(1, q_hi // 2), q_hi), dense_kv=(max(1, kv_hi // 2), kv_hi),
                page=page, shuffled=shuffled, splits=splits)


@pytest.mark.parametrize("seed", range(48))
def test_random_config(seed):
    c = draw(seed)
    print(f"seed {seed}: {c}", flush=True)
    case = make_case(c["B"], c["QH"], c["KVH"], c["D"], c["attn"], c["dtype"], c["layout"],
                     seed, q_range=c["q_range"], kv_range=c["kv_range"],
                     dense_q_range=c["dense"], dense_kv_range=c["dense_kv"], q_lens=c["q_lens"])
    outs, _ = run_case(case, c["layout"], c["causal"], alignment=c["alignment"],
                       shuffled=c["shuffled"], num_splits=c["splits"], seed=seed, page=c["page"])
    check_all(case, c["layout"], c["causal"], outs, alignment=c["alignment"])


# ---- decode_attention / speculative_decode_attention ------------------------

DEC_HEADS = [(8, 8), (8, 2), (8, 1), (32, 8), (32, 1), (12, 4), (6, 3), (16, 2), (4, 4)]


def draw_decode(seed):
    rng = random.Random(5000 + seed)
    layout = rng.choice(["dense", "ragged", "paged"])
    dtype = rng.choice([torch.float16, torch.bfloat16, torch.bfloat16, torch.float32])
    D = rng.choice([16, 32, 64, 64, 128, 128, 256])
    QH, KVH = rng.choice(DEC_HEADS)
    decode = rng.random() < 0.4
    M = 1 if decode else rng.randint(1, 16)
    causal = (not decode) and rng.random() < 0.6
    B = rng.randint(1, 9)
    hi = rng.choice([64, 300, 1200, 2500])
    lo = 0 if (layout != "dense" and not causal and rng.random() < 0.3) else 1
    page = rng.choice([5, 8, 16, 16, 32])
    shuffled = layout == "paged" and rng.random() < 0.7
    cache4d = layout == "paged" and rng.random() < 0.3
    splits = rng.choice([0, 0, 0, 2, 3, 9])
    return dict(layout=layout, dtype=dtype, D=D, QH=QH, KVH=KVH, decode=decode, M=M,
                causal=causal, B=B, kv_range=(lo, hi), dense_kv=(max(1, hi // 2), hi),
                page=page, shuffled=shuffled, cache4d=cache4d, splits=splits)


@pytest.mark.parametrize("seed", range(40))
def test_random_decode_config(seed):
    from decode_cases import make_decode_case
    from test_decode_gpu import check as check_decode
    from test_decode_gpu import run as run_decode
    c = draw_decode(seed)
    print(f"seed {seed}: {c}", flush=True)
    case = make_decode_case(c["B"], c["QH"], c["KVH"], c["D"], c["M"], c["dtype"], c["layout"],
                            seed=6000 + seed, causal=c["causal"], kv_range=c["kv_range"],
                            dense_kv_range=c["dense_kv"])
    pk = {}
    if c["layout"] == "paged":
        pk = dict(shuffled=c["shuffled"], seed=seed, page=c["page"], cache4d=c["cache4d"])
    outs = run_decode(case, c["layout"], decode=c["decode"], num_splits=c["splits"], **pk)
    check_decode(case, c["layout"], outs)
