"""Pinning of the C restatement of decode_attention / speculative_decode_attention
(oracle.oracle_decode, oracle/fa2_oracle.c:fa2o_decode) - CPU only.

The reference suites hold no golden vectors for these paths
(tests/test_decode.py, tests/test_speculative_decode.py compare against
per-sequence SDPA only), so the restatement is pinned by:
  * fp64 SDPA, built exactly as those suites build their oracle, on every
    layout x topology (x M x causal for the speculative kernel);
  * an independent restatement: speculative causal decode equals the
    flash_attention_v2 restatement with a bottom-right mask over dense q;
  * closed forms (constant V, one key, equal keys, a dominant key, an empty
    sequence -> NaN) and invariances (split factor, block size, page order,
    4-D page cache);
  * planted mistakes, each of which one of these checks must catch.
"""

import math

import pytest
import torch

import oracle
from decode_cases import (LAYOUTS, M_VALUES, TOPOLOGIES, make_decode_case, pack_decode, truth)
from attn_cases import topology_heads


def run_oracle(case, layout, squeeze=False, **kw):
    q, k, v, pk = pack_decode(case, layout, squeeze_m=squeeze, shuffled=kw.pop("shuffled", False),
                              cache4d=kw.pop("cache4d", False), page=kw.pop("page", 16))
    out = oracle.oracle_decode(q, k, v, causal=case.causal, **pk, **kw)
    if squeeze:
        out = out.unsqueeze(2)
    return [out[b] for b in range(len(case.qs))]


def max_err(outs, refs):
    return max((o.double() - r.double()).abs().max().item() for o, r in zip(outs, refs))


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("topology", TOPOLOGIES)
def test_decode_vs_fp64_sdpa(layout, topology):
    QH, KVH = topology_heads(topology)
    case = make_decode_case(4, QH, KVH, 64, 1, torch.float32, layout, seed=11)
    outs = run_oracle(case, layout, squeeze=True, block_n=32, split_k=3)
    assert max_err(outs, truth(case)) < 2e-5


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("topology", TOPOLOGIES)
@pytest.mark.parametrize("M", [2, 5, 16])
@pytest.mark.parametrize("causal", [False, True])
def test_speculative_vs_fp64_sdpa(layout, topology, M, causal):
    QH, KVH = topology_heads(topology)
    case = make_decode_case(3, QH, KVH, 64, M, torch.float32, layout, seed=13 + M,
                            causal=causal)
    outs = run_oracle(case, layout, block_n=32, split_k=2)
    assert max_err(outs, truth(case)) < 2e-5


@pytest.mark.parametrize("M", [1, 4, 16])
def test_speculative_equals_bottom_right_prefill_restatement(M):
    """Two independent restatements (decode kernel vs flash_attention_v2
    partial kernel with a bottom-right mask) agree on dense inputs."""
    case = make_decode_case(2, 8, 2, 64, M, torch.float32, "dense", seed=17, causal=True)
    q, k, v, _ = pack_decode(case, "dense")
    a = oracle.oracle_decode(q, k, v, causal=True, block_n=64, split_k=1)
    b = oracle.oracle_attention(q, k, v, is_causal=True, causal_alignment="bottom_right",
                                operand_round="none", p_round="none", block_m=64, block_n=64)
    assert (a - b).abs().max().item() < 1e-5


def test_split_and_block_invariance():
    case = make_decode_case(3, 8, 2, 64, 4, torch.float32, "ragged", seed=19, causal=True,
                            kv_range=(100, 300))
    base = run_oracle(case, "ragged", block_n=64, split_k=1)
    for bn, sk in ((32, 1), (32, 5), (128, 2), (16, 8)):
        assert max_err(run_oracle(case, "ragged", block_n=bn, split_k=sk), base) < 2e-6


def test_page_order_and_4d_cache_invariance():
    case = make_decode_case(3, 8, 1, 64, 1, torch.float32, "paged", seed=23)
    base = run_oracle(case, "paged", squeeze=True)
    assert max_err(run_oracle(case, "paged", squeeze=True, shuffled=True), base) == 0.0
    assert max_err(run_oracle(case, "paged", squeeze=True, cache4d=True), base) == 0.0
    assert max_err(run_oracle(case, "paged", squeeze=True, page=5), base) == 0.0


def test_closed_forms():
    D = 64
    # constant V -> every output is that constant
    case = make_decode_case(2, 4, 2, D, 3, torch.float32, "ragged", seed=29, causal=True)
    for t in case.ctx_v + case.draft_v:
        t.fill_(0.75)
    for o in run_oracle(case, "ragged"):
        assert torch.allclose(o, torch.full_like(o, 0.75), atol=1e-6)
    # one key -> its value; equal keys -> mean of the visible values
    case = make_decode_case(1, 2, 1, D, 1, torch.float32, "dense", seed=31, ctx_lens=[1])
    o = run_oracle(case, "dense", squeeze=True)[0]
    assert torch.allclose(o[:, 0], case.ctx_v[0][0, 0].expand(2, D), atol=1e-6)
    case = make_decode_case(1, 2, 1, D, 4, torch.float32, "dense", seed=37, causal=True,
                            ctx_lens=[10])
    k0 = case.ctx_k[0][0].clone()
    for t in case.ctx_k + case.draft_k:
        t.copy_(k0.expand_as(t))
    o = run_oracle(case, "dense")[0]
    vals = case.vs[0][:, 0]
    for m in range(4):
        assert torch.allclose(o[0, m], vals[: 10 + m + 1].mean(0), atol=1e-5)
    # a dominant key -> its value
    case = make_decode_case(1, 4, 1, D, 1, torch.float32, "ragged", seed=41, ctx_lens=[50])
    case.ctx_k[0][17] = case.qs[0][0, 0] * 40.0
    o = run_oracle(case, "ragged", squeeze=True)[0]
    assert torch.allclose(o[0, 0], case.ctx_v[0][17, 0], atol=1e-4)


def test_empty_sequence_is_nan():
    """The reference's merge divides 0 by 0 when no split saw a key
    (decode.py:192-197)."""
    case = make_decode_case(2, 4, 2, 64, 1, torch.float32, "paged", seed=43, ctx_lens=[0, 9])
    q, k, v, pk = pack_decode(case, "paged", squeeze_m=True)
    out = oracle.oracle_decode(q, k, v, **pk, split_k=2)
    assert torch.isnan(out[0]).all() and not torch.isnan(out[1]).any()


MUTATIONS = {
    "no_rescale": 1, "causal_off1": 2, "head_map": 3, "k_as_v": 4, "no_scale": 5,
    "page_offset": 6,
}


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_planted_mistakes_are_caught(name):
    """Each plausible bug makes the fp64-SDPA comparison fail."""
    layout = "paged" if name == "page_offset" else "ragged"
    case = make_decode_case(3, 8, 2, 64, 4, torch.float32, layout, seed=47, causal=True,
                            kv_range=(40, 200))
    ref = truth(case)
    good = run_oracle(case, layout, block_n=16, split_k=1)
    assert max_err(good, ref) < 2e-5
    bad = run_oracle(case, layout, block_n=16, split_k=1, mutation=MUTATIONS[name])
    err = max_err(bad, ref)
    assert math.isnan(err) or err > 1e-2, (name, err)


def test_rounding_emulation_error_is_small_but_nonzero():
    """bf16 P rounding (this build's MFMA) moves the result by ~1e-3, far
    inside the reference tolerance - the floor the strict GPU bar scales."""
    case = make_decode_case(2, 8, 2, 128, 1, torch.bfloat16, "dense", seed=53,
                            dense_kv_range=(500, 500))
    ref = truth(case)
    exact = run_oracle(case, "dense", squeeze=True)
    emul = run_oracle(case, "dense", squeeze=True, p_round="bf16")
    e0, e1 = max_err(exact, ref), max_err(emul, ref)
    assert e0 < 1e-5 < e1 < oracle.attn_tolerances(torch.bfloat16, 500)["atol"] / 10
