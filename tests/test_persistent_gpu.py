"""GPU parity of the persistent two-head kernel when each workgroup walks
many units.

With one workgroup per CU, a problem of more units than CUs runs rounds:
a workgroup takes unit ``r * P + pos`` in round r (odd rounds reversed in
blocks of 8, for the heaviest-first pairing), prefetches the next unit's Q
and first K/V tiles during the current unit's last phases, and rotates its
three LDS slots across units.  ``max_workgroups`` caps the grid, so small
problems exercise all of that: 1 workgroup walks every unit, 3 and 5 give
grids that are not a multiple of the 8 XCDs (plain reversal), 8 and 16 the
blocked reversal (dense) or unit claims (ragged and paged).  The capped output must equal the uncapped output bit for
bit (every unit computes the same arithmetic wherever it runs) and pass the
reference tolerance and the strict bar against the C oracle.
"""

import pytest
import torch

from attn_cases import LAYOUTS, make_case, pack, unpack
from test_attention_gpu import check_all

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X")
    from kernels import _fa2
    _fa2.lib()
    yield


def run(case, layout, causal, max_workgroups=0, num_splits=0, alignment="top_left",
        shuffled=False):
    from kernels.attention import flash_attention_v2
    q, k, v, kw = pack(case, layout, device=DEV, shuffled_pages=shuffled, seed=3)
    extra = {}
    if alignment != "top_left":
        extra["causal_alignment"] = alignment
    # the uncapped baseline pins the persistent kernel too (a small call
    # would otherwise take the short-problem kernel)
    out = flash_attention_v2(q, k, v, is_causal=causal, max_workgroups=max_workgroups,
                             num_splits=num_splits, kernel="regular", **kw, **extra)
    torch.cuda.synchronize()
    return out.cpu(), kw


# (q heads, kv heads): grouped heads (two heads of a kv group per unit) and
# MHA (two q-blocks of one head per unit)
TOPOS = {"gqa": (4, 2), "mha": (4, 4)}


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("topology", list(TOPOS))
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_capped_grid_walks_many_units(layout, topology, causal, dtype):
    QH, KVH = TOPOS[topology]
    D = 128 if dtype == torch.bfloat16 else 64
    seed = 4000 + 13 * LAYOUTS.index(layout) + 7 * int(causal) + (topology == "mha")
    # ragged/paged MHA pairs q-blocks only when sequences average >= 4 blocks
    lens = (520, 700) if topology == "mha" else (100, 500)
    case = make_case(4, QH, KVH, D, "self", dtype, layout, seed, q_range=lens,
                     kv_range=lens, dense_q_range=lens)
    print(f"case {layout} {topology} causal={causal} {dtype} seed={seed}", flush=True)
    base, kw = run(case, layout, causal, shuffled=layout == "paged")
    for wgs in (1, 3, 5, 8, 16):
        out, _ = run(case, layout, causal, max_workgroups=wgs, shuffled=layout == "paged")
        assert torch.equal(out.view(torch.int16), base.view(torch.int16)), wgs
    outs = unpack(case, layout, out, kw)
    check_all(case, layout, causal, outs)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_capped_grid_with_splits(layout):
    """Split KV ranges on a capped grid: units of all splits walk in rounds
    (no prefetch across units then) and the combine merges the partials."""
    case = make_case(3, 8, 2, 128, "cross", torch.bfloat16, layout, 4100 + LAYOUTS.index(layout),
                     q_range=(60, 300), kv_range=(1500, 3000), dense_q_range=(60, 300),
                     dense_kv_range=(1500, 3000))
    base, kw = run(case, layout, False, num_splits=3)
    for wgs in (1, 5):
        out, _ = run(case, layout, False, max_workgroups=wgs, num_splits=3)
        assert torch.equal(out.view(torch.int16), base.view(torch.int16)), wgs
    check_all(case, layout, False, unpack(case, layout, out, kw))


def test_capped_grid_bottom_right_paged():
    """Chunked prefill (bottom-right causal) over a shuffled pool, 2 workgroups."""
    case = make_case(6, 8, 2, 128, "cross", torch.bfloat16, "paged", 4200, q_range=(128, 128),
                     kv_range=(200, 1500))
    base, kw = run(case, "paged", True, alignment="bottom_right", shuffled=True)
    out, _ = run(case, "paged", True, max_workgroups=2, alignment="bottom_right", shuffled=True)
    assert torch.equal(out.view(torch.int16), base.view(torch.int16))
    check_all(case, "paged", True, unpack(case, "paged", out, kw), alignment="bottom_right")


# Ragged and paged launches of >= 8 workgroups (one split) claim their
# units: workgroup g takes unit g, then the next indices of counter g mod 8
# (zeroed by the plan kernel), over a list that keeps each sequence's
# q-blocks together.  Grids of 1, 3 and 5 workgroups walk the static rounds,
# so these caps also compare the two walks bit for bit.
CLAIM_CAPS = (1, 3, 8, 9, 13, 16, 40)
MIXED_Q = [1, 40, 64, 65, 130, 300, 520, 700, 33, 257, 900, 128]
MIXED_KV = [20, 64, 65, 1, 700, 300, 129, 64, 1000, 5, 256, 90]


@pytest.mark.parametrize("layout", ["ragged", "paged"])
@pytest.mark.parametrize("mask", ["none", "top_left", "bottom_right"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_claimed_units_mixed_lengths(layout, mask, dtype):
    """One-tile units (claimed before the first barrier), units of two and
    more tiles (claimed inside the tile loop), sequences shorter than a
    q-block, and many claims per workgroup on the small caps."""
    D = 128 if dtype == torch.bfloat16 else 64
    seed = 4400 + 3 * ["none", "top_left", "bottom_right"].index(mask) + (layout == "paged")
    causal = mask != "none"
    kv = MIXED_Q if mask == "top_left" else MIXED_KV
    # paged q is one padded length, which places the bottom-right diagonal
    ql = [130] * len(MIXED_Q) if (layout, mask) == ("paged", "bottom_right") else MIXED_Q
    case = make_case(len(MIXED_Q), 8, 2, D, "self" if mask == "top_left" else "cross", dtype,
                     layout, seed, q_lens=ql, kv_lens=kv)
    align = "bottom_right" if mask == "bottom_right" else "top_left"
    print(f"claims {layout} {mask} {dtype} seed={seed}", flush=True)
    base, kw = run(case, layout, causal, alignment=align, shuffled=layout == "paged")
    for wgs in CLAIM_CAPS:
        out, _ = run(case, layout, causal, max_workgroups=wgs, alignment=align,
                     shuffled=layout == "paged")
        assert torch.equal(out.view(torch.int16), base.view(torch.int16)), wgs
    check_all(case, layout, causal, unpack(case, layout, base, kw), alignment=align)


@pytest.mark.parametrize("layout", ["ragged", "paged"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_claimed_units_empty_kv(layout, dtype):
    """Sequences with no keys give units of no tiles, which claim through a
    barrier of their own: their rows are NaN (0/0, as the reference), and
    every other sequence's rows equal, bit for bit, a call without them.
    fp32 ragged runs the 16-bit kernels on fp16 copies with fp32 partials and
    combine; fp32 paged the register-staged kernel."""
    from kernels.attention import flash_attention_v2
    ql = [200, 64, 300, 129, 90, 260, 40, 500]
    kl = [300, 1, 700, 65, 1, 128, 64, 900]
    empty = [1, 4]
    case = make_case(len(ql), 8, 2, 128, "cross", dtype, layout, 4500, q_lens=ql,
                     kv_lens=kl)
    keep = [b for b in range(len(ql)) if b not in empty]
    sub = make_case(len(keep), 8, 2, 128, "cross", dtype, layout, 4500,
                    q_lens=[ql[b] for b in keep], kv_lens=[kl[b] for b in keep])
    sub.qs[:] = [case.qs[b] for b in keep]
    sub.ks[:] = [case.ks[b] for b in keep]
    sub.vs[:] = [case.vs[b] for b in keep]
    print(f"claims empty kv {layout} {dtype}", flush=True)
    ref, rkw = run(sub, layout, False, num_splits=1)
    ref = unpack(sub, layout, ref, rkw)
    view = torch.int32 if dtype == torch.float32 else torch.int16
    for wgs in (0, 8, 11):
        q, k, v, kw = pack(case, layout, device=DEV)
        if layout == "ragged":
            ip = [0]
            for b in range(len(kl)):
                ip.append(ip[-1] + (0 if b in empty else kl[b]))
            k = torch.cat([case.ks[b] for b in range(len(kl)) if b not in empty]).to(DEV)
            v = torch.cat([case.vs[b] for b in range(len(kl)) if b not in empty]).to(DEV)
            kw["kv_indptr"] = torch.tensor(ip, dtype=torch.int32, device=DEV)
        else:
            lens = torch.tensor(kl, dtype=torch.int32)
            lens[empty] = 0
            kw["kv_indptr"] = lens.to(DEV)
        out = flash_attention_v2(q, k, v, is_causal=False, max_workgroups=wgs, num_splits=1,
                                 kernel="regular", **kw).cpu()
        outs = unpack(case, layout, out, kw)
        for b in empty:
            assert torch.isnan(outs[b].float()).all(), (wgs, b)
        for i, b in enumerate(keep):
            assert torch.equal(outs[b].view(view), ref[i].view(view)), (wgs, b)


def test_max_workgroups_only_caps():
    """A cap above the CU count, or on a kernel that is not persistent (fp32,
    odd head groups), changes nothing."""
    for QH, KVH, dt in ((8, 2, torch.bfloat16), (6, 2, torch.bfloat16), (8, 2, torch.float32)):
        case = make_case(2, QH, KVH, 64, "self", dt, "dense", 4300 + QH)
        base, _ = run(case, "dense", True)
        for wgs in (1, 100000):
            out, _ = run(case, "dense", True, max_workgroups=wgs)
            assert torch.equal(out.view(torch.int16), base.view(torch.int16))
