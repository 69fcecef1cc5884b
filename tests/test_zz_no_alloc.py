"""fa2_fwd_noalloc (the C entry point that allocates nothing; its work list
and split partials live in the library's static per-device scratch) against
fa2_fwd with a workspace from the caller, through the C ABI.

Each case runs two calls in a row through fa2_fwd_noalloc, the second with a
smaller input, so the second call finds the first call's contents in the
scratch; both must equal fa2_fwd's outputs bit for bit (same plan, same
arithmetic).  A call whose automatic split would not fit the scratch runs
with fewer splits: it is checked against the oracle instead.
"""

import pytest
import torch

from attn_cases import make_case, pack, unpack
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


def call(q, k, v, kw, causal, layout, noalloc, num_splits=0, alignment="top_left",
         max_workgroups=0):
    """One forward call through the C ABI: fa2_fwd (workspace from torch) or
    fa2_fwd_noalloc, with the parameter block flash_attention_v2 builds."""
    from kernels import _fa2
    from kernels._launch import enqueue, index_tensor, strides, table
    out = torch.empty_like(q)
    mask = (_fa2.MASK_NONE if not causal else
            _fa2.MASK_TOP_LEFT if alignment == "top_left" else _fa2.MASK_BOTTOM_RIGHT)
    lay = {"dense": _fa2.LAYOUT_DENSE, "ragged": _fa2.LAYOUT_RAGGED,
           "paged": _fa2.LAYOUT_PAGED}[layout]
    ex = {}
    if layout == "dense":
        B, Hq, M, D = q.shape
        Hkv, N = k.shape[1], k.shape[2]
    elif layout == "ragged":
        M, Hq, D = q.shape
        N, Hkv = k.shape[0], k.shape[1]
        B = kw["q_indptr"].numel() - 1
        ex = dict(qi=index_tensor(kw["q_indptr"], q.device),
                  kvi=index_tensor(kw["kv_indptr"], q.device))
    else:
        B, Hq, M, D = q.shape
        N, Hkv = k.shape[0], k.shape[1]
        ex = dict(kvi=index_tensor(kw["kv_indptr"], q.device),
                  kt=table(kw["k_block_table"], q.device),
                  vt=table(kw["v_block_table"], q.device), page_size=kw["kv_page_size"],
                  kv_len_max=kw["k_block_table"].shape[1] * kw["kv_page_size"])
    enqueue(decode=False, layout=lay, mask=mask, num_splits=num_splits, batch=B, q_heads=Hq,
            kv_heads=Hkv, head_dim=D, q_len=M, kv_len=N, q=q, k=k, v=v, out=out,
            q_strides=strides(q), o_strides=strides(out), noalloc=noalloc,
            max_workgroups=max_workgroups, **ex)
    torch.cuda.synchronize()
    return out.cpu()


def same_bits(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


# (layout, causal, alignment, splits, q heads, kv heads, dtype, first, second)
# first / second: (sequences, q length range, kv length range)
CASES = [
    ("ragged", True, "top_left", 0, 8, 2, torch.bfloat16, (6, (200, 900)), (2, (1, 300))),
    ("paged", True, "bottom_right", 0, 8, 2, torch.bfloat16, (5, (128, 128)), (2, (64, 64))),
    ("paged", False, "top_left", 3, 8, 1, torch.float16, (4, (100, 300)), (2, (1, 100))),
    ("dense", False, "top_left", 4, 8, 8, torch.bfloat16, (3, (200, 400)), (1, (20, 60))),
    ("dense", True, "top_left", 2, 6, 2, torch.float32, (2, (100, 300)), (1, (10, 50))),
    ("ragged", False, "top_left", 5, 4, 4, torch.float16, (5, (50, 400)), (3, (1, 64))),
]


@pytest.mark.parametrize("case_id", range(len(CASES)))
def test_noalloc_matches_fa2_fwd(case_id):
    layout, causal, align, splits, qh, kvh, dt, first, second = CASES[case_id]
    print(f"noalloc case {case_id}: {layout} causal={causal} {align} splits={splits} "
          f"{qh}/{kvh} {dt}", flush=True)
    results = []
    for n, (B, (lo, hi)) in enumerate((first, second)):
        attn = "cross" if align == "bottom_right" else "self"
        kvr = (hi + 50, hi + 700) if attn == "cross" else (lo, hi)
        case = make_case(B, qh, kvh, 128, attn, dt, layout, 6000 + 10 * case_id + n,
                         q_range=(lo, hi), kv_range=kvr, dense_q_range=(lo, hi),
                         dense_kv_range=kvr)
        q, k, v, kw = pack(case, layout, device=DEV, shuffled_pages=layout == "paged", seed=n)
        ref = call(q, k, v, kw, causal, layout, False, splits, align)
        out = call(q, k, v, kw, causal, layout, True, splits, align)
        assert same_bits(out, ref), (case_id, n)
        results.append((case, kw, out))
    # the second (smaller) call is also right on its own terms
    case, kw, out = results[1]
    check_all(case, layout, causal, unpack(case, layout, out, kw), alignment=align)


def test_noalloc_reduces_splits_to_fit():
    """32 query rows of 2 heads over 64K keys: the automatic split (64 ways
    over 8 partial slots of 128 rows) needs ~34 MB of partials, more than the
    32 MiB scratch; the call runs with fewer splits and is checked against the
    oracle."""
    from kernels import _fa2
    case = make_case(1, 2, 2, 128, "cross", torch.bfloat16, "dense", 6100, dense_q_range=(32, 32),
                     dense_kv_range=(65536, 65536))
    q, k, v, kw = pack(case, "dense", device=DEV)
    p_ws = _workspace_bytes(q, k)
    assert p_ws > _fa2.NOALLOC_SCRATCH_BYTES
    out = call(q, k, v, kw, False, "dense", True)
    check_all(case, "dense", False, unpack(case, "dense", out, kw))


def test_noalloc_paged_runs_whole_units():
    """40 paged sequences of one q-block over 128-1800 keys, Hq16/Hkv4: 320
    two-head units, more than the CUs, so fa2_fwd takes the balanced walk
    (units cut into pieces, whose partial slots need ~68 MB of workspace).
    That does not fit the scratch: fa2_fwd_noalloc runs rounds of whole units,
    which fa2_fwd runs when the grid is capped at the CU count.  Both must
    give the same bits, twice in a row, the second on 24 sequences."""
    import random
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    rng = random.Random(61)
    for n, B in enumerate((40, 24)):
        kv = [rng.randint(128, 1800) for _ in range(B)]
        case = make_case(B, 16, 4, 128, "cross", torch.bfloat16, "paged", 6200 + n,
                         q_lens=[128] * B, kv_lens=kv)
        q, k, v, kw = pack(case, "paged", device=DEV, shuffled_pages=True, seed=n)
        print(f"noalloc paged whole units B{B}", flush=True)
        out = call(q, k, v, kw, True, "paged", True, alignment="bottom_right")
        rounds = call(q, k, v, kw, True, "paged", False, alignment="bottom_right",
                      max_workgroups=cus)
        assert same_bits(out, rounds), B


def _workspace_bytes(q, k):
    """fa2_fwd's workspace for a dense non-causal call with automatic splits."""
    from kernels import _fa2
    from kernels._launch import strides
    p = _fa2.Fa2Params()
    p.layout, p.dtype, p.mask, p.num_splits = _fa2.LAYOUT_DENSE, _fa2.DTYPE_BF16, 0, 0
    p.batch, p.q_heads, p.q_len, p.head_dim = q.shape
    p.kv_heads, p.kv_len = k.shape[1], k.shape[2]
    p.q_sb, p.q_sh, p.q_ss = strides(q)
    p.k_sb, p.k_sh, p.k_ss = strides(k)
    p.v_sb, p.v_sh, p.v_ss = strides(k)
    p.o_sb, p.o_sh, p.o_ss = strides(q)
    p.softmax_scale = 1.0
    p.q = p.k = p.v = p.o = 16
    with torch.cuda.device(q.device):
        return _fa2.workspace_size(p)
