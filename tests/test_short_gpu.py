"""GPU parity of the short-problem kernel (fa2_fwd_short_kernel).

Calls too small to fill the GPU split each 32-row query block's KV tiles over
the 4 waves of one workgroup and merge the waves' (max, sum, O) states in
LDS.  ``kernel="short"`` forces it on every fp16/bf16 call at head_dim 64 or
128; these tests run the reference matrix (tests/test_attention.py:137-251)
and the edge cases of test_attention_gpu.py through it: tile-boundary and
length-1 sequences, more tiles than waves, shuffled NaN-poisoned page pools
of several page sizes, bottom-right rows with no visible key, zero-length
sequences, against the reference tolerance and the strict bar.  They also
check which kernel the automatic choice takes.
"""

import pytest
import torch

from attn_cases import (ATTN_TYPES, CAUSAL_FLAGS, LAYOUTS, TOPOLOGIES, make_case, pack,
                        topology_heads, unpack)
from test_attention_gpu import check_all, fa2, run_case

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES16 = [torch.float16, torch.bfloat16]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X")
    from kernels import _fa2
    _fa2.lib()
    yield


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("attn_type", ATTN_TYPES)
@pytest.mark.parametrize("topology", TOPOLOGIES)
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
@pytest.mark.parametrize("dtype", DTYPES16)
def test_short_reference_matrix(layout, attn_type, topology, causal, dtype):
    if causal and attn_type == "cross":
        pytest.skip("reference skips causal cross-attention (tests/test_attention.py:145-146)")
    QH, KVH = topology_heads(topology)
    s = 3000 + 17 * LAYOUTS.index(layout) + 5 * TOPOLOGIES.index(topology) + \
        3 * ATTN_TYPES.index(attn_type) + int(causal) + 7 * DTYPES16.index(dtype)
    case = make_case(4, QH, KVH, 64, attn_type, dtype, layout, s)
    print(f"short layout={layout} {attn_type} {topology} causal={causal} {dtype} seed={s}",
          flush=True)
    outs, _ = run_case(case, layout, causal, kernel="short")
    check_all(case, layout, causal, outs)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
def test_short_long_kv(layout, D, causal):
    """More KV tiles than waves (up to ~40 tiles, ~10 per wave): the per-wave
    loop with its next-tile loads, and rows whose tiles end on different
    waves."""
    case = make_case(3, 8, 2, D, "self" if causal else "cross", torch.bfloat16, layout,
                     3100 + D + int(causal), q_range=(100, 600), kv_range=(1500, 2600),
                     dense_q_range=(300, 300), dense_kv_range=(2500, 2500))
    outs, _ = run_case(case, layout, causal, kernel="short")
    check_all(case, layout, causal, outs)


EDGE_LENS = [1, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 257]


@pytest.mark.parametrize("layout", ["ragged", "paged"])
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
def test_short_tile_boundary_lengths(layout, causal):
    """Lengths around the 32-row blocks, the 64-key tiles and the 128-row
    work items."""
    case = make_case(len(EDGE_LENS), 4, 2, 64, "self", torch.bfloat16, layout, 3200,
                     q_lens=EDGE_LENS, kv_lens=EDGE_LENS)
    outs, _ = run_case(case, layout, causal, kernel="short")
    check_all(case, layout, causal, outs)


@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
@pytest.mark.parametrize("page", [16, 8, 32, 5, 64])
def test_short_paged_shuffled_pool(dtype, causal, page):
    """Shuffled pool, -1 padded tables, separate K and V page orders; unused
    pool slots hold NaN, so a read outside the table poisons the output.
    Page 64 takes one table read per tile of a wave."""
    case = make_case(5, 8, 2, 128, "self", dtype, "paged", 3300 + page)
    outs, _ = run_case(case, "paged", causal, shuffled=True, seed=page, page=page,
                       kernel="short")
    assert not any(torch.isnan(o).any() for o in outs)
    check_all(case, "paged", causal, outs)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("dtype", DTYPES16)
def test_short_bottom_right_causal(layout, dtype):
    """Bottom-right alignment, with query blocks whose rows see no key (NaN
    rows: every wave's state is empty and the merge gives 0/0)."""
    ql = [40, 40, 40] if layout == "paged" else None
    case = make_case(3, 8, 2, 64, "cross", dtype, layout, 3400, q_range=(1, 150),
                     kv_range=(1, 300), dense_q_range=(90, 90), dense_kv_range=(200, 300),
                     q_lens=ql, kv_lens=[1, 150, 300] if layout != "dense" else None)
    outs, _ = run_case(case, layout, True, alignment="bottom_right", kernel="short")
    check_all(case, layout, True, outs, alignment="bottom_right")


def test_short_zero_length_sequence_gives_nan_rows():
    case = make_case(3, 4, 2, 64, "cross", torch.bfloat16, "paged", 3500, q_lens=[8, 8, 8],
                     kv_lens=[20, 1, 33])
    q, k, v, kw = pack(case, "paged", device=DEV)
    kw["kv_indptr"] = torch.tensor([20, 0, 33], dtype=torch.int32, device=DEV)
    out = fa2()(q, k, v, is_causal=False, kernel="short", **kw).cpu()
    assert torch.isnan(out[1]).all()
    assert not torch.isnan(out[0]).any() and not torch.isnan(out[2]).any()


def test_short_dominant_key_in_each_wave():
    """All probability mass on one key, placed in each of the 4 waves' tiles
    in turn: the merge must take that wave's value with weight 1 and the
    others' with weight ~0."""
    g = torch.Generator().manual_seed(3600)
    B, H, L, D = 1, 4, 512, 64
    for key in (3, 70, 130, 200, 260, 400, 511):
        u = torch.randn(1, D, generator=g)
        u = u / u.norm(dim=-1, keepdim=True)
        q = (8.0 * u)[None, :, None, :].expand(B, H, 64, D).contiguous()
        k = 0.05 * torch.randn(B, 1, L, D, generator=g)
        k[:, :, key] = 4.0 * (D ** 0.5) * u
        v = torch.randn(B, 1, L, D, generator=g)
        out = fa2()(q.bfloat16().to(DEV), k.bfloat16().to(DEV), v.bfloat16().to(DEV),
                    kernel="short").float().cpu()
        want = v[:, :, key:key + 1, :].bfloat16().float().expand(B, H, 64, D)
        torch.testing.assert_close(out, want, atol=2e-2, rtol=2e-2)


def test_auto_choice():
    """The automatic choice: a c1-sized call (16 units of the regular kernel)
    runs the short-problem kernel, a call that fills the GPU does not.  Each
    is compared bit for bit with the forced choices."""
    g = torch.Generator().manual_seed(3700)

    def run(B, H, L, D, kernel, t):
        q, k, v = t
        return fa2()(q, k, v, is_causal=True, kernel=kernel).cpu()

    small = [torch.randn(1, 8, 512, 64, generator=g).half().to(DEV) for _ in range(3)]
    a = run(1, 8, 512, 64, "auto", small)
    s = run(1, 8, 512, 64, "short", small)
    assert torch.equal(a.view(torch.int16), s.view(torch.int16))
    big = [torch.randn(2, 32, 2048, 128, generator=g).bfloat16().to(DEV) for _ in range(3)]
    a = run(2, 32, 2048, 128, "auto", big)
    r = run(2, 32, 2048, 128, "regular", big)
    assert torch.equal(a.view(torch.int16), r.view(torch.int16))


def test_short_matches_regular_within_rounding():
    """The two kernels sum in different orders: the same inputs agree to
    within a few bf16 ulps."""
    case = make_case(4, 8, 2, 128, "self", torch.bfloat16, "ragged", 3800, q_range=(50, 700))
    s, _ = run_case(case, "ragged", True, kernel="short")
    r, _ = run_case(case, "ragged", True, kernel="regular")
    for a, b in zip(s, r):
        torch.testing.assert_close(a.float(), b.float(), atol=2e-2, rtol=2e-2)
