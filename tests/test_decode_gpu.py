"""GPU parity of the HIP decode_attention / speculative_decode_attention
(fa2_decode_fwd, called through the C ABI).

Mirrors the reference acceptance matrices - tests/test_decode.py:133-244
(layout x MHA/GQA/MQA x fp16/bf16/fp32) and
tests/test_speculative_decode.py:129-331 (the same x M in {2..16} x causal) -
with explicit seeds, and adds what they leave open: head_dim 128, long
contexts across many key tiles, 32 query heads per kv head (units of up to
512 rows), shuffled NaN-poisoned page pools with distinct K/V tables, page
sizes 5/8/32, 4-D page caches, forced split factors (including more splits
than tiles), empty sequences (NaN rows, the reference's 0/0), non-contiguous
queries, determinism, and assertion parity.  Every numeric case is checked
against the reference suites' own tolerance and the strict bar of
tests/parity.py.
"""

import pytest
import torch

import oracle
from attn_cases import topology_heads
from decode_cases import (DTYPES, LAYOUTS, M_VALUES, TOPOLOGIES, make_decode_case, pack_decode,
                          truth)
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


def reference_rounding(dtype):
    """Operand / P rounding of the reference decode kernels: none - they load
    every dtype into fp32 and compute in fp32 (kernels/decode.py:84, 92-160;
    kernels/speculative_decode.py:91, 150-175).  The strict bar measures the
    HIP kernels against that arithmetic: fp32 tensors run in fp32 there too,
    fp16/bf16 tensors round P for the P.V MFMA (within the bar's 4x / 2x)."""
    return "none", "none"


def run(case, layout, decode=False, num_splits=0, **pk):
    from kernels import decode_attention, speculative_decode_attention
    q, k, v, kw = pack_decode(case, layout, device=DEV, squeeze_m=decode, **pk)
    if decode:
        out = decode_attention(q, k, v, **kw, num_splits=num_splits).unsqueeze(2)
    else:
        out = speculative_decode_attention(q, k, v, causal=case.causal, **kw,
                                           num_splits=num_splits)
    torch.cuda.synchronize()
    out = out.cpu()
    return [out[b] for b in range(len(case.qs))]


def check(case, layout, outs):
    dt = case.dtype
    N = max(case.kv_lens)
    fin = [~torch.isnan(t) for t in truth(case, torch.float64)]
    ref32 = truth(case, torch.float32)
    reference_check([o[f] for o, f in zip(outs, fin)], [r[f] for r, f in zip(ref32, fin)], dt, N)
    opr, prd = reference_rounding(dt)
    q, k, v, kw = pack_decode(case, layout)
    emul = oracle.oracle_decode(q, k, v, causal=case.causal, **kw, operand_round=opr,
                                p_round=prd)
    return strict_check(outs, [emul[b] for b in range(len(case.qs))], truth(case, torch.float64),
                        dt)


# ---- the reference matrices -------------------------------------------------

@pytest.mark.parametrize("seed", [0, 1])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("topology", TOPOLOGIES)
@pytest.mark.parametrize("layout", LAYOUTS)
def test_decode_reference_matrix(layout, topology, dtype, seed):
    QH, KVH = topology_heads(topology)
    case = make_decode_case(4, QH, KVH, 64, 1, dtype, layout, seed=1000 + seed)
    check(case, layout, run(case, layout, decode=True))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("M", M_VALUES)
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("topology", TOPOLOGIES)
@pytest.mark.parametrize("layout", LAYOUTS)
def test_speculative_reference_matrix(layout, topology, dtype, M, causal):
    QH, KVH = topology_heads(topology)
    case = make_decode_case(4, QH, KVH, 64, M, dtype, layout, seed=2000 + M, causal=causal)
    check(case, layout, run(case, layout))


# ---- beyond the reference matrices -----------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=str)
@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("heads", [(32, 8), (32, 1), (8, 8)])
def test_decode_d128_long_context(layout, heads, dtype):
    QH, KVH = heads
    case = make_decode_case(5, QH, KVH, 128, 1, dtype, layout, seed=3001, kv_range=(700, 3000),
                            dense_kv_range=(1500, 3000))
    check(case, layout, run(case, layout, decode=True))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("heads,M", [((32, 8), 16), ((32, 1), 16), ((32, 1), 5), ((4, 4), 7)])
def test_speculative_d128_many_rows(layout, heads, M, causal):
    """32 query heads per kv head x 16 drafts = 512 rows: four q-blocks per unit."""
    QH, KVH = heads
    case = make_decode_case(3, QH, KVH, 128, M, torch.bfloat16, layout, seed=3100 + M,
                            causal=causal, kv_range=(200, 1200), dense_kv_range=(300, 900))
    check(case, layout, run(case, layout))


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("D", [16, 32, 256])
def test_decode_other_head_dims(layout, D, dtype):
    """Head dims 16, 32 and 256 run the register-staged kernel in packed mode."""
    case = make_decode_case(4, 8, 2, D, 1, dtype, layout, seed=3500 + D)
    check(case, layout, run(case, layout, decode=True))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("D", [32, 256])
def test_speculative_other_head_dims(layout, D, causal):
    case = make_decode_case(3, 8, 2, D, 4, torch.bfloat16, layout, seed=3600 + D, causal=causal,
                            kv_range=(40, 400))
    check(case, layout, run(case, layout))


@pytest.mark.parametrize("page", [5, 8, 16, 32])
@pytest.mark.parametrize("cache4d", [False, True])
def test_paged_pools(page, cache4d):
    """Shuffled, NaN-poisoned pools with -1 padding and distinct K/V tables."""
    case = make_decode_case(6, 8, 2, 128, 4, torch.bfloat16, "paged", seed=3200 + page,
                            causal=True, kv_range=(1, 700))
    check(case, "paged", run(case, "paged", shuffled=True, page=page, cache4d=cache4d))


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 64])
@pytest.mark.parametrize("layout", LAYOUTS)
def test_forced_splits(layout, splits):
    """Any split factor, including more splits than key tiles (empty splits)."""
    case = make_decode_case(3, 8, 2, 64, 3, torch.float16, layout, seed=3300, causal=True,
                            kv_range=(1, 400), dense_kv_range=(200, 300))
    check(case, layout, run(case, layout, num_splits=splits))


@pytest.mark.parametrize("B", [255, 256, 257, 700])
@pytest.mark.parametrize("layout", ["ragged", "paged"])
def test_batch_sizes_around_the_plan_fast_path(layout, B):
    """The device plan ranks up to 256 sequences directly and counting-sorts
    larger batches: either order must cover every sequence exactly once."""
    case = make_decode_case(B, 4, 2, 64, 1, torch.bfloat16, layout, seed=3600 + B,
                            kv_range=(1, 80))
    check(case, layout, run(case, layout, decode=True))


@pytest.mark.parametrize("layout", ["ragged", "paged"])
def test_empty_and_single_key_sequences(layout):
    """A sequence without keys gives NaN (the reference's 0/0,
    decode.py:192-197); one with a single key gives that key's value."""
    case = make_decode_case(4, 8, 2, 128, 1, torch.bfloat16, layout, seed=3400,
                            ctx_lens=[0, 1, 300, 0])
    outs = run(case, layout, decode=True)
    assert torch.isnan(outs[0]).all() and torch.isnan(outs[3]).all()
    assert not torch.isnan(outs[1]).any() and not torch.isnan(outs[2]).any()
    v1 = case.ctx_v[1][0].float()  # [KVH, D]
    assert torch.equal(outs[1][:, 0].float(), v1.repeat_interleave(4, 0))
    check(case, layout, outs)


def test_noncontiguous_query_and_determinism():
    from kernels import speculative_decode_attention
    case = make_decode_case(3, 8, 2, 128, 6, torch.bfloat16, "ragged", seed=3500, causal=True,
                            kv_range=(50, 900))
    q, k, v, kw = pack_decode(case, "ragged", device=DEV)
    # the same values through a [B, M, QH, D] buffer viewed as [B, QH, M, D]
    qt = q.transpose(1, 2).contiguous().transpose(1, 2)
    a = speculative_decode_attention(q, k, v, causal=True, **kw)
    b = speculative_decode_attention(qt, k, v, causal=True, **kw)
    c = speculative_decode_attention(q, k, v, causal=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(a, c)


def test_decode_equals_speculative_m1():
    from kernels import decode_attention, speculative_decode_attention
    case = make_decode_case(4, 16, 4, 128, 1, torch.float16, "paged", seed=3600,
                            kv_range=(10, 2000))
    q, k, v, kw = pack_decode(case, "paged", device=DEV, shuffled=True)
    a = decode_attention(q[:, :, 0], k, v, **kw)
    b = speculative_decode_attention(q, k, v, **kw)
    torch.cuda.synchronize()
    assert torch.equal(a, b[:, :, 0])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_flash_attention_v1_is_v2_on_16_bit(dtype):
    """fp16/bf16 tensors: v1 runs v2's kernels (their operands are exact in
    fp32), so the two agree bit for bit; fp32 tensors differ by design (v1 in
    fp32, v2 with fp16 operands; tests/test_v1_gpu.py)."""
    from kernels import flash_attention_v1, flash_attention_v2
    g = torch.Generator().manual_seed(3700)
    q = torch.randn((2, 8, 300, 64), generator=g).to(dtype).to(DEV)
    k = torch.randn((2, 2, 300, 64), generator=g).to(dtype).to(DEV)
    v = torch.randn((2, 2, 300, 64), generator=g).to(dtype).to(DEV)
    for causal in (False, True):
        a = flash_attention_v1(q, k, v, is_causal=causal)
        b = flash_attention_v2(q, k, v, is_causal=causal)
        torch.cuda.synchronize()
        assert torch.equal(a, b)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_fp32_decode_beyond_fp16_range(layout):
    """fp32 tensors are computed in fp32 as the reference does: values past
    fp16's range (65504) stay finite and match fp64 attention (an fp16
    operand path would give inf/NaN)."""
    case = make_decode_case(3, 8, 2, 64, 4, torch.float32, layout, 3800, causal=True,
                            kv_range=(50, 700))
    scale_q, scale_kv = 1.0e3, 2.0e5
    case.qs = [q * scale_q for q in case.qs]
    case.ctx_k = [k * 1e-3 for k in case.ctx_k]
    case.draft_k = [k * 1e-3 for k in case.draft_k]
    case.ctx_v = [v * scale_kv for v in case.ctx_v]
    case.draft_v = [v * scale_kv for v in case.draft_v]
    outs = run(case, layout)
    assert all(torch.isfinite(o).all() for o in outs)
    assert max(o.abs().max().item() for o in outs) > 65504
    check(case, layout, outs)


def test_assertions_match_reference():
    """Assertion messages and order of decode.py:236-274 and
    speculative_decode.py:262-297."""
    from kernels import decode_attention, speculative_decode_attention
    q = torch.randn((2, 4, 64), device=DEV, dtype=torch.float16)
    k = torch.randn((2, 2, 10, 64), device=DEV, dtype=torch.float16)
    with pytest.raises(AssertionError, match="same dtype"):
        decode_attention(q, k.float(), k)
    with pytest.raises(AssertionError, match="same device"):
        decode_attention(q, k.cpu(), k)
    with pytest.raises(AssertionError, match="CUDA device"):
        decode_attention(q.cpu(), k.cpu(), k.cpu())
    kc = torch.randn((32, 2, 64), device=DEV, dtype=torch.float16)
    tbl = torch.zeros((2, 2), dtype=torch.int32, device=DEV)
    lens = torch.tensor([5, 7], dtype=torch.int32, device=DEV)
    with pytest.raises(AssertionError):
        decode_attention(q, kc, kc, k_block_table=tbl, kv_indptr=lens, kv_page_size=16)
    with pytest.raises(AssertionError):
        decode_attention(q, kc, kc, k_block_table=tbl, v_block_table=tbl, kv_indptr=lens)
    with pytest.raises(AssertionError, match="context lengths"):
        decode_attention(q, kc, kc, k_block_table=tbl, v_block_table=tbl, kv_page_size=16)
    q17 = torch.randn((2, 4, 17, 64), device=DEV, dtype=torch.float16)
    with pytest.raises(AssertionError, match="M <= 16"):
        speculative_decode_attention(q17, k, k)
    # beyond the reference: checks that keep the device grid in bounds
    with pytest.raises(ValueError):
        decode_attention(q, k[:1], k[:1])
    with pytest.raises(ValueError):
        decode_attention(q, torch.randn((2, 3, 10, 64), device=DEV, dtype=torch.float16),
                         torch.randn((2, 3, 10, 64), device=DEV, dtype=torch.float16))


@pytest.mark.parametrize("fill", ["zeros", "ones", "random", "reused"])
def test_split_merge_words_need_no_clearing(fill):
    """A split decode call merges its splits inside the kernel: the last
    split of a unit to finish combines the partials, counted in one 64-bit
    word per unit of the workspace that holds a per-call tag.  Whatever the
    workspace held before (never cleared: zeros, all ones, random bytes, the
    words a previous call left), the output must equal that of a call on a
    fresh workspace bit for bit, and so must a second call on the same one."""
    from kernels import _fa2
    from kernels.decode import _run_decode
    g = torch.Generator(device=DEV).manual_seed(4242)
    B, QH, KVH, D, N = 4, 16, 2, 128, 3000  # 8 units of 47 tiles: 5 automatic splits
    q = torch.randn(B, QH, D, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, KVH, N, D, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(B, KVH, N, D, generator=g, device=DEV).to(torch.bfloat16)
    print(f"split merge words, workspace {fill}", flush=True)

    def call(ws):
        out = torch.empty_like(q)
        _run_decode("decode_attention", q.unsqueeze(2), k, v, out.unsqueeze(2),
                    layout=_fa2.LAYOUT_DENSE, causal=False, batch=B, q_heads=QH, kv_heads=KVH,
                    head_dim=D, kv_indptr=None, k_block_table=None, v_block_table=None,
                    kv_page_size=None, workspace=ws)
        torch.cuda.synchronize()
        return out

    n = 64 << 20
    ref = call(torch.zeros(n, dtype=torch.uint8, device=DEV))
    assert torch.isfinite(ref).all()
    ws = torch.zeros(n, dtype=torch.uint8, device=DEV)
    if fill == "ones":
        ws.fill_(255)
    elif fill == "random":
        ws.copy_(torch.randint(0, 256, (n,), generator=g, device=DEV, dtype=torch.uint8))
    elif fill == "reused":
        call(ws)
    assert torch.equal(call(ws), ref)
    assert torch.equal(call(ws), ref)
    # and the merged output is the attention (the reference suite's bar)
    expect = oracle.sdpa_reference([q[b].unsqueeze(0).cpu() for b in range(B)],
                                   [k[b].transpose(0, 1).cpu() for b in range(B)],
                                   [v[b].transpose(0, 1).cpu() for b in range(B)],
                                   QH, KVH, False)
    reference_check([ref.cpu()], [torch.stack([e[0] for e in expect])],
                    torch.bfloat16, N)


@pytest.mark.parametrize("splits", [1, 4])
def test_bounded_wait_giveup_is_never_silent(splits):
    """The decode kernel's producer/consumer ring waits are bounded; a wait
    that gives up must show.  Forced from the host with decode_spin_cap = 1
    (one poll), every workgroup whose waits gave up writes NaN rows (or NaN
    partials, which the in-kernel merge turns into NaN rows) and is counted
    by fa2_decode_wait_giveups; the others stay equal to the normal call.
    With the library's bound no wait gives up and the count stays 0."""
    from kernels import _fa2
    from kernels.decode import _run_decode
    g = torch.Generator(device=DEV).manual_seed(777)
    B, QH, KVH, D, N = 4, 16, 2, 128, 4096
    q = torch.randn(B, QH, D, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, KVH, N, D, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(B, KVH, N, D, generator=g, device=DEV).to(torch.bfloat16)

    def call(cap):
        out = torch.empty_like(q)
        _run_decode("decode_attention", q.unsqueeze(2), k, v, out.unsqueeze(2),
                    layout=_fa2.LAYOUT_DENSE, causal=False, batch=B, q_heads=QH, kv_heads=KVH,
                    head_dim=D, kv_indptr=None, k_block_table=None, v_block_table=None,
                    kv_page_size=None, num_splits=splits, decode_spin_cap=cap)
        torch.cuda.synchronize()
        return out

    _fa2.decode_wait_giveups(reset=True)
    ref = call(0)
    assert _fa2.decode_wait_giveups(reset=True) == 0
    assert torch.isfinite(ref).all()
    forced = call(1)
    n = _fa2.decode_wait_giveups(reset=True)
    # one workgroup per (sequence, kv head) here: its QH / KVH query heads
    units = forced.view(B, KVH, QH // KVH, D)
    nan_units = units.isnan().flatten(2).all(-1)
    finite_units = torch.isfinite(units).flatten(2).all(-1)
    assert n >= 1, "one poll never gave up: the forced path did not run"
    if splits == 1:
        assert int(nan_units.sum()) == n
    else:  # a unit is NaN when any of its splits gave up
        assert 1 <= int(nan_units.sum()) <= n
    assert bool((nan_units | finite_units).all())
    same = ref.view(B, KVH, QH // KVH, D)[finite_units]
    assert torch.equal(units[finite_units], same)
    assert torch.isfinite(call(0)).all() and _fa2.decode_wait_giveups() == 0
