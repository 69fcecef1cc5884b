"""GPU parity of the HIP flash_attention_v2 (called through the C ABI).

Mirrors the reference acceptance matrix (tests/test_attention.py:137-251:
layout x self/cross x MHA/GQA/MQA x causal x fp16/bf16/fp32) with seeds,
and adds what it leaves open: head_dim 128, tile-boundary and length-1
sequences, shuffled and -1-padded page pools with distinct K/V tables,
forced split-KV, bottom-right causal, golden fixtures, determinism and
non-contiguous inputs.  Every case is checked against the reference's own
tolerance and the strict bar of tests/parity.py.
"""

import os

import numpy as np
import pytest
import torch

import oracle
from attn_cases import (ATTN_TYPES, CAUSAL_FLAGS, DTYPES, LAYOUTS, TOPOLOGIES, make_case, pack,
                        topology_heads, unpack)
from parity import reference_check, strict_check

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X")
    from kernels import _fa2
    _fa2.lib()  # fail loudly if the HIP library is missing
    yield


def fa2():
    from kernels.attention import flash_attention_v2
    return flash_attention_v2


def run_case(case, layout, causal, alignment="top_left", shuffled=False, num_splits=0,
             seed=0, page=16, kernel="regular"):
    """One flash_attention_v2 call of `case`.  The tests of this module target
    the regular kernels (two-head, one-head LDS, register-staged), so their
    small shapes pin kernel="regular"; test_short_gpu.py runs the same cases
    through the short-problem kernel."""
    q, k, v, kw = pack(case, layout, device=DEV, shuffled_pages=shuffled, seed=seed, page=page)
    extra = {"kernel": kernel}
    if alignment != "top_left":
        extra["causal_alignment"] = alignment
    if num_splits:
        extra["num_splits"] = num_splits
    out = fa2()(q, k, v, is_causal=causal, **kw, **extra)
    torch.cuda.synchronize()
    return unpack(case, layout, out.cpu(), {n: t for n, t in kw.items()}), (q, k, v, kw)


def check_all(case, layout, causal, outs, alignment="top_left", packed=None):
    dt = case.dtype
    if causal and alignment == "bottom_right":
        truth = oracle.sdpa_reference_bottom_right(case.qs, case.ks, case.vs, case.QH, case.KVH,
                                                   dtype=torch.float64)
    else:
        truth = oracle.sdpa_reference(case.qs, case.ks, case.vs, case.QH, case.KVH, causal,
                                      dtype=torch.float64)
        ref32 = oracle.sdpa_reference(case.qs, case.ks, case.vs, case.QH, case.KVH, causal)
        reference_check(outs, ref32, dt, max(case.kv_lens))
    q, k, v, kw = pack(case, layout)
    r = oracle.mma_round_for(dt)
    emul = oracle.oracle_attention(q, k, v, is_causal=causal, causal_alignment=alignment,
                                   operand_round=r, p_round=r, **kw)
    emul = unpack(case, layout, emul, kw)
    stats = strict_check(outs, emul, truth, dt)
    if dt == torch.bfloat16:
        # the same bar against the reference's own arithmetic for bf16 tensors:
        # operands and P rounded to fp16 (attention.py:547, 572, 607, 614, 633),
        # where the kernel keeps bf16 operands and rounds P to bf16
        ref = oracle.oracle_attention(q, k, v, is_causal=causal, causal_alignment=alignment,
                                      operand_round="f16", p_round="f16", **kw)
        strict_check(outs, unpack(case, layout, ref, kw), truth, dt)
    return stats


# ---------------------------------------------------------------------------
# the reference matrix (81 executed cases x 2 seeds)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("seed", [0, 1])
@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("attn_type", ATTN_TYPES)
@pytest.mark.parametrize("topology", TOPOLOGIES)
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
@pytest.mark.parametrize("dtype", DTYPES)
def test_reference_matrix(layout, attn_type, topology, causal, dtype, seed):
    if causal and attn_type == "cross":
        pytest.skip("reference skips causal cross-attention (tests/test_attention.py:145-146)")
    QH, KVH = topology_heads(topology)
    s = 1000 * seed + 17 * LAYOUTS.index(layout) + 5 * TOPOLOGIES.index(topology) + \
        3 * ATTN_TYPES.index(attn_type) + int(causal) + 7 * DTYPES.index(dtype)
    case = make_case(4, QH, KVH, 64, attn_type, dtype, layout, s)
    print(f"case layout={layout} {attn_type} {topology} causal={causal} {dtype} seed={s}",
          flush=True)
    outs, _ = run_case(case, layout, causal)
    check_all(case, layout, causal, outs)


# ---------------------------------------------------------------------------
# beyond the reference matrix
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
def test_head_dim_128(layout, dtype, causal):
    case = make_case(3, 8, 2, 128, "self", dtype, layout, 300 + int(causal))
    outs, _ = run_case(case, layout, causal)
    check_all(case, layout, causal, outs)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("D", [16, 32, 256])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
def test_other_head_dims(layout, D, dtype, causal):
    """Head dims 16 and 32 (the register-staged kernel on 64-dim tiles, the
    padding dims read as zeros and never stored) and 256 (its own
    instantiation): the reference takes any power of two its tl.dot accepts."""
    s = 1300 + D + int(causal) + 7 * DTYPES.index(dtype) + 17 * LAYOUTS.index(layout)
    case = make_case(3, 8, 2, D, "self", dtype, layout, s)
    outs, _ = run_case(case, layout, causal)
    check_all(case, layout, causal, outs)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("D", [16, 32, 256])
@pytest.mark.parametrize("splits", [1, 3])
def test_other_head_dims_mqa_cross(layout, D, splits):
    case = make_case(3, 8, 1, D, "cross", torch.bfloat16, layout, 1400 + D + splits,
                     kv_range=(100, 600), dense_kv_range=(300, 600))
    outs, _ = run_case(case, layout, False, num_splits=splits)
    check_all(case, layout, False, outs)


@pytest.mark.parametrize("D", [16, 32])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_small_head_dim_never_reads_past_its_row(D, dtype):
    """Shuffled pool whose unused slots hold NaN, page size 1: the 64-dim
    tiles' padding columns lie in the next rows of the pool, so reading them
    (instead of zero-filling) would put NaN into the scores."""
    case = make_case(4, 8, 2, D, "self", dtype, "paged", 1500 + D)
    outs, _ = run_case(case, "paged", True, shuffled=True, seed=D, page=1)
    assert not any(torch.isnan(o).any() for o in outs)
    check_all(case, "paged", True, outs)


@pytest.mark.parametrize("L", [100, 300, 640, 1000])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mask", ["none", "top_left", "bottom_right"])
def test_mha_dense_qblock_pairs(L, D, dtype, mask):
    """MHA runs the two-head kernel with a pair of q-blocks of one head per
    unit (odd q-block counts leave group 1 without rows in the last pair);
    bottom-right uses a longer KV."""
    causal = mask != "none"
    align = "bottom_right" if mask == "bottom_right" else "top_left"
    kvL = L + 77 if mask != "top_left" else L
    case = make_case(2, 4, 4, D, "self" if kvL == L else "cross", dtype, "dense", 1600 + L + D,
                     dense_q_range=(L, L), dense_kv_range=(kvL, kvL))
    outs, _ = run_case(case, "dense", causal, alignment=align)
    check_all(case, "dense", causal, outs, alignment=align)


@pytest.mark.parametrize("layout", ["ragged", "paged"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("mask", ["none", "top_left", "bottom_right"])
def test_mha_ragged_paged_qblock_pairs(layout, D, mask):
    """Ragged / paged MHA whose sequences average >= 4 q-blocks run the
    two-head kernel on q-block pairs (some sequences with an odd count)."""
    causal = mask != "none"
    align = "bottom_right" if mask == "bottom_right" else "top_left"
    if layout == "ragged":
        ql = [640, 1000, 300, 777]
        kl = ql if mask == "top_left" else [n + 50 for n in ql]
    else:
        ql = [600] * 3
        kl = [600, 1500, 700] if mask != "top_left" else [600] * 3
    case = make_case(len(ql), 4, 4, D, "cross", torch.bfloat16, layout, 1650 + D,
                     q_lens=ql, kv_lens=kl)
    outs, _ = run_case(case, layout, causal, alignment=align, shuffled=layout == "paged", seed=D)
    check_all(case, layout, causal, outs, alignment=align)


EDGE_LENS = [1, 63, 64, 65, 127, 128, 129, 255, 257]


@pytest.mark.parametrize("layout", ["ragged", "paged"])
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
def test_tile_boundary_lengths(layout, causal):
    case = make_case(len(EDGE_LENS), 4, 2, 64, "self", torch.bfloat16, layout, 400,
                     q_lens=EDGE_LENS, kv_lens=EDGE_LENS)
    outs, _ = run_case(case, layout, causal)
    check_all(case, layout, causal, outs)


@pytest.mark.parametrize("L", [1, 2, 63, 65, 129, 200])
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
def test_dense_odd_lengths(L, causal):
    case = make_case(2, 4, 4, 64, "self", torch.float16, "dense", 500 + L,
                     dense_q_range=(L, L))
    outs, _ = run_case(case, "dense", causal)
    check_all(case, "dense", causal, outs)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
@pytest.mark.parametrize("page", [16, 8, 32, 5])
def test_paged_shuffled_pool(dtype, causal, page):
    """Shuffled pool, -1 padded tables, separate K and V page orders; unused
    pool slots hold NaN so any read outside the table poisons the output."""
    case = make_case(5, 8, 2, 64, "self", dtype, "paged", 600 + page)
    outs, _ = run_case(case, "paged", causal, shuffled=True, seed=page, page=page)
    assert not any(torch.isnan(o).any() for o in outs)
    check_all(case, "paged", causal, outs)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("splits", [2, 3, 7])
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
def test_forced_split_kv(layout, splits, causal):
    case = make_case(3, 8, 2, 64, "self" if causal else "cross", torch.bfloat16, layout,
                     700 + splits, kv_range=(100, 600), dense_kv_range=(300, 600))
    outs, _ = run_case(case, layout, causal, num_splits=splits)
    check_all(case, layout, causal, outs)
    base, _ = run_case(case, layout, causal, num_splits=1)
    for a, b in zip(outs, base):
        torch.testing.assert_close(a.float(), b.float(), atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_bottom_right_causal(layout, dtype):
    ql = [40, 40, 40] if layout == "paged" else None
    case = make_case(3, 8, 2, 64, "cross", dtype, layout, 800, q_range=(1, 150),
                     kv_range=(1, 300), dense_q_range=(90, 90), dense_kv_range=(200, 300),
                     q_lens=ql, kv_lens=[1, 150, 300] if layout != "dense" else None)
    outs, _ = run_case(case, layout, True, alignment="bottom_right")
    check_all(case, layout, True, outs, alignment="bottom_right")


def test_paged_zero_length_sequence_gives_nan_rows():
    """A sequence with no KV (length 0) has no visible key: 0/0 = NaN, as the
    reference's merge (attention.py:712,724)."""
    case = make_case(3, 4, 2, 64, "cross", torch.bfloat16, "paged", 900, q_lens=[8, 8, 8],
                     kv_lens=[20, 1, 33])
    q, k, v, kw = pack(case, "paged", device=DEV)
    kw["kv_indptr"] = torch.tensor([20, 0, 33], dtype=torch.int32, device=DEV)
    out = fa2()(q, k, v, is_causal=False, **kw).cpu()
    assert torch.isnan(out[1]).all()
    assert not torch.isnan(out[0]).any() and not torch.isnan(out[2]).any()


def test_empty_inputs():
    q = torch.zeros((0, 4, 64), dtype=torch.bfloat16, device=DEV)
    k = torch.zeros((0, 2, 64), dtype=torch.bfloat16, device=DEV)
    ip = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = fa2()(q, k, k, q_indptr=ip, kv_indptr=ip)
    assert out.shape == q.shape


def test_deterministic():
    case = make_case(6, 8, 2, 64, "self", torch.bfloat16, "ragged", 1000, q_range=(50, 400))
    a, _ = run_case(case, "ragged", True)
    b, _ = run_case(case, "ragged", True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_layout_equivalence_on_gpu():
    """The same sequences as ragged and as (shuffled) paged give identical rows:
    each (row, head) sees the same keys through the same tile schedule."""
    case = make_case(4, 8, 2, 64, "self", torch.bfloat16, "ragged", 1100, q_range=(20, 300))
    r, _ = run_case(case, "ragged", True, num_splits=1)
    p, _ = run_case(case, "paged", True, shuffled=True, num_splits=1)
    for x, y in zip(r, p):
        assert torch.equal(x, y)


@pytest.mark.parametrize("hkv", [4, 1])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("key", [0, 5, 37, 63, 64, 100, 190])
def test_dominant_key_selects_its_value(D, dtype, key, hkv):
    """All probability mass on one key: the output row is that key's V row.
    Each key sits in one lane half of the score fragment, so a wrong
    cross-lane max/sum exchange shows up as a factor-of-two error here.
    hkv=1 shares one K/V head among the 4 query heads (two-head kernel)."""
    g = torch.Generator().manual_seed(key)
    B, H, L = 1, 4, 200
    u = torch.randn(hkv, D, generator=g)
    u = u / u.norm(dim=-1, keepdim=True)
    q = (8.0 * u).repeat_interleave(H // hkv, 0)[None, :, None, :].expand(B, H, 96, D)
    q = q.contiguous()
    k = 0.05 * torch.randn(B, hkv, L, D, generator=g)
    k[:, :, key] = 4.0 * (D ** 0.5) * u
    v = torch.randn(B, hkv, L, D, generator=g)
    out = fa2()(q.to(dtype).to(DEV), k.to(dtype).to(DEV), v.to(dtype).to(DEV)).float().cpu()
    want = v[:, :, key:key + 1, :].to(dtype).float().repeat_interleave(H // hkv, 1)
    torch.testing.assert_close(out, want.expand_as(out), atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("group", [2, 4, 3])
@pytest.mark.parametrize("splits", [1, 3])
def test_grouped_equals_expanded_heads(layout, D, group, splits):
    """Grouped heads (two query heads per workgroup) and the same problem with
    K/V repeated per query head (one head per workgroup) run the same
    per-row arithmetic over the same tiles: the outputs are identical."""
    case = make_case(3, 2 * group, 2, D, "self", torch.bfloat16, layout, 1300 + group,
                     q_range=(30, 400), dense_q_range=(300, 300))
    q, k, v, kw = pack(case, layout, device=DEV, shuffled_pages=True, seed=1)
    out = fa2()(q, k, v, is_causal=True, num_splits=splits, **kw)
    ke = k.repeat_interleave(group, dim=1)  # the head dim of every k/v layout
    ve = v.repeat_interleave(group, dim=1)
    ref = fa2()(q, ke, ve, is_causal=True, num_splits=splits, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), ref.cpu())


@pytest.mark.parametrize("layout", LAYOUTS)
def test_constant_v_gives_constant_rows(layout):
    case = make_case(3, 8, 2, 128, "self", torch.bfloat16, layout, 1200)
    row = (torch.arange(128) % 7 - 3).to(torch.bfloat16)
    for v in case.vs:
        v[:] = row
    outs, _ = run_case(case, layout, True)
    for o in outs:
        assert torch.equal(o.float(), row.float().expand_as(o))


def test_non_contiguous_inputs():
    """[B,S,H,D] storage viewed as [B,H,S,D] (last dim still contiguous)."""
    g = torch.Generator().manual_seed(5)
    B, H, S, D = 2, 4, 100, 64
    base = torch.randn((B, S, H, D), generator=g).to(torch.bfloat16)
    q = base.to(DEV).transpose(1, 2)
    k = torch.randn((B, S, H, D), generator=g).to(torch.bfloat16).to(DEV).transpose(1, 2)
    v = torch.randn((B, S, H, D), generator=g).to(torch.bfloat16).to(DEV).transpose(1, 2)
    out = fa2()(q, k, v, is_causal=True)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.float().cpu(), k.float().cpu(), v.float().cpu(), is_causal=True)
    torch.testing.assert_close(out.float().cpu(), ref, **oracle.attn_tolerances(torch.bfloat16, S))
    contig = fa2()(q.contiguous(), k.contiguous(), v.contiguous(), is_causal=True)
    assert torch.equal(out.cpu(), contig.cpu())


# ---------------------------------------------------------------------------
# golden fixtures
# ---------------------------------------------------------------------------

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("name", sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz")))
def test_golden(name):
    from test_oracle import golden_inputs, load_golden
    z, meta = load_golden(name)
    q, k, v, kw, dt = golden_inputs(z, meta)
    want = torch.from_numpy(z["out"])
    valid = torch.from_numpy(z["valid"]).bool()
    kwd = {n: (t.to(DEV) if isinstance(t, torch.Tensor) else t) for n, t in kw.items()}
    out = fa2()(q.to(DEV), k.to(DEV), v.to(DEV), **kwd).float().cpu()
    r = oracle.mma_round_for(dt)
    emul = oracle.oracle_attention(q, k, v, operand_round=r, p_round=r, **kw)
    got, ref, em = out[valid], want[valid], emul[valid]
    N = int(k.shape[0] if k.dim() == 3 else k.shape[2])
    fin = ~torch.isnan(ref)
    assert torch.equal(torch.isnan(got), ~fin)
    torch.testing.assert_close(got[fin], ref[fin], **oracle.attn_tolerances(dt, N))
    strict_check([got[fin]], [em[fin]], [ref[fin].double()], dt)


# ---------------------------------------------------------------------------
# assertion parity with the reference wrapper (attention.py:762-834)
# ---------------------------------------------------------------------------

def _dense(B=1, H=2, S=8, D=64, dt=torch.float16):
    return torch.zeros((B, H, S, D), dtype=dt, device=DEV)


@pytest.mark.parametrize("bad", [
    "dtype", "q3d_dense", "batch", "kv_heads", "seq_kv", "head_dim", "heads_div",
    "ragged_k4d", "ragged_total", "ragged_no_kv_indptr", "paged_q3d", "paged_no_page",
    "paged_no_lens", "paged_no_vtable", "paged_heads"])
def test_assertions_match_reference(bad):
    f = fa2()
    q, k, v = _dense(), _dense(), _dense()
    ip = torch.tensor([0, 8], dtype=torch.int32, device=DEV)
    tbl = torch.zeros((1, 1), dtype=torch.int32, device=DEV)
    cache = torch.zeros((16, 2, 64), dtype=torch.float16, device=DEV)
    lens = torch.tensor([8], dtype=torch.int32, device=DEV)
    calls = {
        "dtype": lambda: f(q, k.to(torch.bfloat16), v),
        "q3d_dense": lambda: f(q[0], k, v),
        "batch": lambda: f(q, _dense(B=2), _dense(B=2)),
        "kv_heads": lambda: f(q, _dense(H=2), _dense(H=1)),
        "seq_kv": lambda: f(q, _dense(S=8), _dense(S=9)),
        "head_dim": lambda: f(q, _dense(D=128), _dense(D=128)),
        "heads_div": lambda: f(_dense(H=3), _dense(H=2), _dense(H=2)),
        "ragged_k4d": lambda: f(q[0].transpose(0, 1), k, v, q_indptr=ip, kv_indptr=ip),
        "ragged_total": lambda: f(q[0].transpose(0, 1), k[0].transpose(0, 1),
                                  v[0, :, :4].transpose(0, 1), q_indptr=ip, kv_indptr=ip),
        "ragged_no_kv_indptr": lambda: f(q[0].transpose(0, 1), k[0].transpose(0, 1),
                                         v[0].transpose(0, 1), q_indptr=ip),
        "paged_q3d": lambda: f(q[0], cache, cache, kv_indptr=lens, k_block_table=tbl,
                               v_block_table=tbl, kv_page_size=16),
        "paged_no_page": lambda: f(q, cache, cache, kv_indptr=lens, k_block_table=tbl,
                                   v_block_table=tbl),
        "paged_no_lens": lambda: f(q, cache, cache, k_block_table=tbl, v_block_table=tbl,
                                   kv_page_size=16),
        "paged_no_vtable": lambda: f(q, cache, cache, kv_indptr=lens, k_block_table=tbl,
                                     kv_page_size=16),
        "paged_heads": lambda: f(_dense(H=3), cache, cache, kv_indptr=lens, k_block_table=tbl,
                                 v_block_table=tbl, kv_page_size=16),
    }
    with pytest.raises(AssertionError):
        calls[bad]()


def test_unsupported_head_dim_raises():
    q = torch.zeros((1, 2, 8, 48), dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError):
        fa2()(q, q, q)
