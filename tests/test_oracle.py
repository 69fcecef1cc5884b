"""Pins the CPU oracle (oracle/fa2_oracle.c) before anything is checked against it.

Checks, each chosen so that a plausible mistake fails at least one of them
(test_planted_mistakes_are_caught proves that for six planted bugs):

* rounding helpers == torch's own fp16/bf16 casts, bit for bit;
* oracle with exact arithmetic == fp64 SDPA (library routine) on every
  layout x mask x head topology of the reference matrix;
* oracle with the reference's fp16 rounding passes the reference test's
  tolerance against fp32 SDPA (tests/test_attention.py:246-251);
* committed golden fixtures (tests/golden/, written by torch SDPA);
* closed forms: constant V, a single key, identical keys (prefix means),
  one dominant logit;
* invariances: dense == ragged == paged (also shuffled pools), split-K,
  key permutation (non-causal), GQA == MHA with repeated KV heads.
"""

import math
import os
import zlib

import numpy as np
import pytest
import torch

import oracle
from attn_cases import (ATTN_TYPES, CAUSAL_FLAGS, LAYOUTS, TOPOLOGIES, make_case, pack,
                        topology_heads, unpack)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def run_oracle(case, layout, causal, alignment="top_left", rounding=None, shuffled=False,
               **kw):
    q, k, v, lk = pack(case, layout, shuffled_pages=shuffled)
    r = rounding or "none"
    out = oracle.oracle_attention(q, k, v, is_causal=causal, causal_alignment=alignment,
                                  operand_round=r, p_round=r, **lk, **kw)
    return unpack(case, layout, out, lk)


def sdpa64(case, causal, alignment="top_left"):
    if causal and alignment == "bottom_right":
        return oracle.sdpa_reference_bottom_right(case.qs, case.ks, case.vs, case.QH, case.KVH,
                                                  dtype=torch.float64)
    return oracle.sdpa_reference(case.qs, case.ks, case.vs, case.QH, case.KVH, causal,
                                 dtype=torch.float64)


def max_err(outs, refs):
    e = 0.0
    for o, r in zip(outs, refs):
        e = max(e, (o.double() - r.double()).abs().max().item())
    return e


# ---------------------------------------------------------------------------
# rounding helpers
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("mode,dt", [("f16", torch.float16), ("bf16", torch.bfloat16)])
def test_rounding_matches_torch_casts(mode, dt):
    g = torch.Generator().manual_seed(1)
    vals = torch.cat([
        torch.randn(2000, generator=g) * 10.0 ** torch.randint(-9, 6, (2000,), generator=g),
        torch.tensor([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e-8, 6e-8, 3e-8, 2.98e-8,
                      6.1e-5, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 1.0 + 2 ** -8,
                      1.0 + 3 * 2 ** -8, float("inf"), -float("inf")]),
    ])
    want = vals.to(dt).float()
    got = torch.tensor([oracle.round_scalar(float(x), mode) for x in vals])
    assert torch.equal(got, want)


# ---------------------------------------------------------------------------
# exact arithmetic vs fp64 SDPA, full reference matrix (small sizes)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("attn_type", ATTN_TYPES)
@pytest.mark.parametrize("topology", TOPOLOGIES)
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
def test_oracle_exact_vs_sdpa64(layout, attn_type, topology, causal):
    if causal and attn_type == "cross":
        pytest.skip("reference skips causal cross-attention (tests/test_attention.py:145-146)")
    QH, KVH = topology_heads(topology)
    seed = zlib.crc32(f"{layout}-{attn_type}-{topology}-{causal}".encode()) % 10000
    case = make_case(3, QH, KVH, 32, attn_type, torch.float32, layout, seed,
                     q_range=(1, 70), kv_range=(1, 140), dense_q_range=(16, 70),
                     dense_kv_range=(16, 140))
    outs = run_oracle(case, layout, causal)
    assert max_err(outs, sdpa64(case, causal)) < 2e-5


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("D", [16, 256])
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
def test_oracle_exact_vs_sdpa64_head_dims(layout, D, causal):
    """The restatement at the smallest and largest head dims the kernels take."""
    case = make_case(2, 4, 2, D, "self", torch.float32, layout, 40 + D + int(causal),
                     q_range=(1, 70), kv_range=(1, 70), dense_q_range=(30, 70))
    assert max_err(run_oracle(case, layout, causal), sdpa64(case, causal)) < 2e-5


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_oracle_reference_rounding_within_reference_tolerance(layout, dtype):
    case = make_case(3, 8, 2, 64, "self", dtype, layout, 11)
    outs = run_oracle(case, layout, True, rounding="f16")
    refs = oracle.sdpa_reference(case.qs, case.ks, case.vs, 8, 2, True)
    for o, r in zip(outs, refs):
        torch.testing.assert_close(o.float(), r, **oracle.attn_tolerances(dtype, max(case.kv_lens)))


@pytest.mark.parametrize("layout", LAYOUTS)
def test_oracle_bottom_right_vs_sdpa64(layout):
    # paged q is dense [B,Hq,M,D]: every sequence has M query rows, so the
    # bottom-right diagonal is placed by M (uniform q lengths here)
    ql = [23, 23, 23, 23] if layout == "paged" else None
    case = make_case(4, 4, 2, 32, "cross", torch.float32, layout, 5, q_range=(1, 40),
                     kv_range=(1, 150), dense_q_range=(20, 40), dense_kv_range=(50, 150),
                     q_lens=ql)
    outs = run_oracle(case, layout, True, alignment="bottom_right")
    refs = sdpa64(case, True, "bottom_right")
    for o, r in zip(outs, refs):
        nan_r = torch.isnan(r)
        assert torch.equal(torch.isnan(o), nan_r)  # rows with no key -> NaN
        assert (o[~nan_r].double() - r[~nan_r]).abs().max().item() < 2e-5 if (~nan_r).any() else True


# ---------------------------------------------------------------------------
# golden fixtures (tests/golden/*.npz written by make_golden.py from torch SDPA)
# ---------------------------------------------------------------------------

def golden_files():
    if not os.path.isdir(GOLDEN):
        return []
    return sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))


def load_golden(name):
    z = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    meta = {k[5:]: z[k] for k in z.files if k.startswith("meta_")}
    return z, meta


def golden_inputs(z, meta):
    """Inputs of a fixture: 16-bit tensors are stored as their bit patterns."""
    dt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[str(meta["dtype"])]

    def tensor(name):
        t = torch.from_numpy(z[name].copy())
        return t.view(dt) if dt != torch.float32 else t

    q, k, v = tensor("q"), tensor("k"), tensor("v")
    kw = dict(is_causal=bool(meta["causal"]))
    if str(meta["alignment"]) != "top_left":
        kw["causal_alignment"] = str(meta["alignment"])
    for n in ("q_indptr", "kv_indptr", "k_block_table", "v_block_table"):
        if n in z.files:
            kw[n] = torch.from_numpy(z[n].copy())
    if "page_size" in meta:
        kw["kv_page_size"] = int(meta["page_size"])
    return q, k, v, kw, dt


@pytest.mark.parametrize("name", golden_files())
def test_oracle_matches_golden(name):
    z, meta = load_golden(name)
    q, k, v, kw, dt = golden_inputs(z, meta)
    out = oracle.oracle_attention(q, k, v, operand_round="none", p_round="none", **kw)
    want = torch.from_numpy(z["out"])
    valid = torch.from_numpy(z["valid"]).bool()  # rows that exist (padding excluded)
    got = out[valid]
    ref = want[valid]
    assert torch.equal(torch.isnan(got), torch.isnan(ref))
    fin = ~torch.isnan(ref)
    assert (got[fin].double() - ref[fin].double()).abs().max().item() < 2e-5


def test_golden_fixtures_present():
    assert len(golden_files()) >= 6


# ---------------------------------------------------------------------------
# closed forms
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("layout", LAYOUTS)
def test_constant_v_gives_constant_output(layout):
    case = make_case(3, 4, 2, 32, "self", torch.float32, layout, 3)
    for v in case.vs:
        v.fill_(0.0)
        v[..., :] = torch.arange(32, dtype=torch.float32) * 0.25 - 3.0
    outs = run_oracle(case, layout, True)
    for o in outs:
        assert torch.allclose(o, torch.arange(32, dtype=torch.float32) * 0.25 - 3.0, atol=1e-5)


def test_single_key_returns_its_value():
    case = make_case(2, 4, 4, 32, "cross", torch.float32, "ragged", 9, q_lens=[5, 9],
                     kv_lens=[1, 1])
    outs = run_oracle(case, "ragged", False)
    for o, v in zip(outs, case.vs):
        assert torch.allclose(o, v[0].unsqueeze(0).expand_as(o), atol=1e-6)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_identical_keys_give_prefix_means(layout):
    case = make_case(2, 2, 2, 32, "self", torch.float32, layout, 4, q_range=(60, 130),
                     dense_q_range=(60, 130))
    for k in case.ks:
        k[:] = k[0:1]
    outs = run_oracle(case, layout, True)
    for o, v in zip(outs, case.vs):
        L = v.shape[0]
        csum = torch.cumsum(v.double(), 0) / torch.arange(1, L + 1, dtype=torch.float64)[:, None, None]
        assert (o.double() - csum).abs().max().item() < 1e-5


def test_dominant_logit_selects_one_value():
    case = make_case(1, 2, 2, 32, "cross", torch.float32, "dense", 6, dense_q_range=(8, 8),
                     dense_kv_range=(40, 40))
    u = torch.randn(2, 32, generator=torch.Generator().manual_seed(8))
    u = u / u.norm(dim=-1, keepdim=True)
    case.qs[0][:] = 8.0 * u           # every query along u (per head)
    case.ks[0][17] = 40.0 * u         # key 17 along u: logit ~ 56 vs ~ 4 for the rest
    outs = run_oracle(case, "dense", False)
    want = case.vs[0][17].unsqueeze(0).expand_as(outs[0])
    assert torch.allclose(outs[0], want, atol=1e-4)


# ---------------------------------------------------------------------------
# invariances
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
def test_layout_equivalence(causal):
    base = make_case(3, 4, 2, 32, "self", torch.float32, "ragged", 21)
    outs = {lay: run_oracle(base, lay, causal) for lay in ("ragged", "paged")}
    outs["paged_shuffled"] = run_oracle(base, "paged", causal, shuffled=True)
    for b in range(3):
        assert torch.equal(outs["ragged"][b], outs["paged"][b])
        assert torch.equal(outs["ragged"][b], outs["paged_shuffled"][b])


def test_dense_equals_ragged_for_uniform_lengths():
    case = make_case(3, 4, 1, 32, "self", torch.float32, "dense", 22)
    d = run_oracle(case, "dense", True)
    r = run_oracle(case, "ragged", True)
    for x, y in zip(d, r):
        assert torch.equal(x, y)


@pytest.mark.parametrize("split_k,block_n", [(2, 64), (3, 64), (5, 16)])
def test_split_k_invariance_non_causal(split_k, block_n):
    case = make_case(2, 4, 2, 32, "cross", torch.float32, "ragged", 23, kv_range=(60, 250))
    a = run_oracle(case, "ragged", False)
    b = run_oracle(case, "ragged", False, split_k=split_k, block_n=block_n)
    assert max_err(a, b) < 1e-5


def test_reference_split_k_nan_defect_is_restated():
    """The reference's split kernel visits, for rows 0..31 of q-block 0 under a
    causal mask with BLOCK_N=32 and SPLIT_K=2, a key block that is entirely
    masked while the running max is still -inf: exp(-inf - -inf) = NaN
    (attention.py:600-611), and the merge keeps it (0 * NaN).  The oracle
    restates that; the HIP kernels do not reproduce it (their outputs match
    SDPA for every row with a visible key)."""
    case = make_case(1, 2, 2, 32, "self", torch.float32, "dense", 24, dense_q_range=(64, 64))
    out = run_oracle(case, "dense", True, split_k=2, block_n=32)[0]
    assert torch.isnan(out[:32]).all()
    assert not torch.isnan(out[32:]).any()


def test_key_permutation_invariance():
    case = make_case(2, 4, 2, 32, "cross", torch.float32, "ragged", 25)
    a = run_oracle(case, "ragged", False)
    g = torch.Generator().manual_seed(3)
    for i in range(2):
        perm = torch.randperm(case.ks[i].shape[0], generator=g)
        case.ks[i] = case.ks[i][perm]
        case.vs[i] = case.vs[i][perm]
    b = run_oracle(case, "ragged", False)
    assert max_err(a, b) < 1e-5


def test_gqa_equals_mha_with_repeated_heads():
    case = make_case(2, 8, 2, 32, "self", torch.float32, "ragged", 26)
    a = run_oracle(case, "ragged", True)
    rep = make_case(2, 8, 8, 32, "self", torch.float32, "ragged", 26)
    rep.qs = case.qs
    rep.ks = [k.repeat_interleave(4, dim=1) for k in case.ks]
    rep.vs = [v.repeat_interleave(4, dim=1) for v in case.vs]
    b = run_oracle(rep, "ragged", True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


# ---------------------------------------------------------------------------
# planted mistakes: every one must fail at least one of the checks above
# ---------------------------------------------------------------------------

MUTATIONS = {1: "no_rescale", 2: "causal_off_by_one", 3: "head_map", 4: "k_as_v",
             5: "no_scale", 6: "page_offset"}


@pytest.mark.parametrize("mutation", sorted(MUTATIONS))
def test_planted_mistakes_are_caught(mutation):
    QH, KVH = 8, 2
    caught = []
    for layout in ("dense", "paged"):
        for causal in (False, True):
            case = make_case(2, QH, KVH, 32, "self", torch.float32, layout, 40 + mutation,
                             q_range=(70, 130), dense_q_range=(70, 130))
            q, k, v, lk = pack(case, layout, shuffled_pages=True)
            out = oracle.oracle_attention(q, k, v, is_causal=causal, operand_round="none",
                                          p_round="none", mutation=mutation, **lk)
            outs = unpack(case, layout, out, lk)
            refs = sdpa64(case, causal)
            err = max(((o.double() - r).abs().max().item() if not torch.isnan(o).any()
                       else math.inf) for o, r in zip(outs, refs))
            caught.append(err > 1e-3)
    assert any(caught), MUTATIONS[mutation]


# ---------------------------------------------------------------------------
# flash_attention_v1's arithmetic (oracle.oracle_v1)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
def test_oracle_v1_is_fp32_attention(layout, causal):
    """fp32 inputs: the v1 restatement is within fp32 rounding of fp64 SDPA
    (far tighter than the fp16-operand v2 restatement), on every layout."""
    case = make_case(4, 8, 2, 64, "self", torch.float32, layout, 900 + int(causal))
    q, k, v, lk = pack(case, layout)
    v1 = unpack(case, layout, oracle.oracle_v1(q, k, v, is_causal=causal, **lk), lk)
    v2 = run_oracle(case, layout, causal, rounding="f16")
    truth = sdpa64(case, causal)
    e1, e2 = max_err(v1, truth), max_err(v2, truth)
    assert e1 < 2e-6, e1
    assert e2 > 50 * e1, (e1, e2)


def test_oracle_v1_keeps_fp32_range():
    """Values past fp16's range: v1's arithmetic stays finite and exact to fp32,
    v2's fp16 operands overflow (the reference's .to(float16) casts)."""
    case = make_case(2, 4, 4, 64, "self", torch.float32, "dense", 950)
    case.vs = [x * 1.0e5 for x in case.vs]
    q, k, v, lk = pack(case, "dense")
    v1 = unpack(case, "dense", oracle.oracle_v1(q, k, v, is_causal=True, **lk), lk)
    truth = sdpa64(case, True)
    assert all(torch.isfinite(o).all() for o in v1)
    rel = max_err(v1, truth) / max(t.abs().max().item() for t in truth)
    assert rel < 2e-6, rel
    v2 = run_oracle(case, "dense", True, rounding="f16")
    assert not all(torch.isfinite(o).all() for o in v2)
