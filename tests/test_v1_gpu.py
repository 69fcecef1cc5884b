"""GPU parity of ``flash_attention_v1`` against its own contract.

The reference's v1 (kernels/attention.py:164-364) has v2's signature,
assertions, layouts and top-left mask, but computes in fp32: q, k, v are cast
to fp32 (:177, :196-197, :228) and the softmax weights stay fp32 for the P.V
product (:225-240).  Here fp32 tensors run the fp32-MFMA kernel
(fa2_kernel_f32.h); fp16/bf16 tensors run v2's kernels, whose operands are
exact and whose P is rounded to the tensor type.  Every case is checked
against the reference suite's bar (fp32 SDPA, tests/test_attention.py:80-98,
246-251) and the strict bar against ``oracle.oracle_v1`` - the C
restatement with fp32 operands and fp32 P, i.e. v1's arithmetic.
"""

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
    _fa2.lib()
    yield


def run_v1(case, layout, causal, shuffled=False, page=16, seed=0):
    from kernels import flash_attention_v1
    q, k, v, kw = pack(case, layout, device=DEV, shuffled_pages=shuffled, seed=seed, page=page)
    out = flash_attention_v1(q, k, v, is_causal=causal, **kw)
    torch.cuda.synchronize()
    assert out.dtype == case.dtype
    return unpack(case, layout, out.cpu(), kw)


def check_v1(case, layout, causal, outs):
    truth = oracle.sdpa_reference(case.qs, case.ks, case.vs, case.QH, case.KVH, causal,
                                  dtype=torch.float64)
    ref32 = oracle.sdpa_reference(case.qs, case.ks, case.vs, case.QH, case.KVH, causal)
    reference_check(outs, ref32, case.dtype, max(case.kv_lens))
    q, k, v, kw = pack(case, layout)
    emul = unpack(case, layout, oracle.oracle_v1(q, k, v, is_causal=causal, **kw), kw)
    return strict_check(outs, emul, truth, case.dtype)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("attn_type", ATTN_TYPES)
@pytest.mark.parametrize("topology", TOPOLOGIES)
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_v1_reference_matrix(layout, attn_type, topology, causal, dtype):
    if causal and attn_type == "cross":
        pytest.skip("reference skips causal cross-attention (tests/test_attention.py:145-146)")
    QH, KVH = topology_heads(topology)
    s = 7000 + 17 * LAYOUTS.index(layout) + 5 * TOPOLOGIES.index(topology) + \
        3 * ATTN_TYPES.index(attn_type) + int(causal) + 7 * DTYPES.index(dtype)
    case = make_case(4, QH, KVH, 64, attn_type, dtype, layout, s)
    print(f"v1 {layout} {attn_type} {topology} causal={causal} {dtype} seed={s}", flush=True)
    check_v1(case, layout, causal, run_v1(case, layout, causal))


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("causal", CAUSAL_FLAGS)
def test_v1_fp32_head_dims(layout, D, causal):
    """Every head dim on the fp32 kernel: 16 and 32 on 64-dim tiles (padding
    dims zero-filled, never read), 256 with one workgroup per CU."""
    case = make_case(3, 8, 2, D, "self", torch.float32, layout, 7100 + D + int(causal),
                     q_range=(1, 300))
    check_v1(case, layout, causal, run_v1(case, layout, causal))


@pytest.mark.parametrize("page", [16, 8, 5, 1])
@pytest.mark.parametrize("D", [32, 128])
def test_v1_fp32_shuffled_pools(page, D):
    """fp32 rows through shuffled NaN-poisoned pools: page sizes on every
    loader path (one table read per wave, per instruction, per lane)."""
    case = make_case(4, 8, 2, D, "self", torch.float32, "paged", 7200 + page + D)
    check_v1(case, "paged", True, run_v1(case, "paged", True, shuffled=True, page=page, seed=page))


@pytest.mark.parametrize("layout", LAYOUTS)
def test_v1_fp32_long_kv_split(layout):
    """Few units over long KV: the automatic split-KV with the combine kernel."""
    case = make_case(2, 8, 8, 128, "cross", torch.float32, layout, 7300 + LAYOUTS.index(layout),
                     q_range=(20, 100), kv_range=(3000, 6000), dense_q_range=(20, 100),
                     dense_kv_range=(3000, 6000))
    check_v1(case, layout, False, run_v1(case, layout, False))


def test_v1_fp32_beyond_fp16_range():
    """Values past fp16's range stay finite and exact to fp32 (v1's fp32
    arithmetic); v2 on the same fp32 tensors follows the reference's fp16
    casts and overflows."""
    from kernels import flash_attention_v2
    case = make_case(2, 8, 2, 128, "self", torch.float32, "dense", 7400,
                     dense_q_range=(200, 300))
    case.vs = [x * 1.0e5 for x in case.vs]
    outs = run_v1(case, "dense", True)
    assert all(torch.isfinite(o).all() for o in outs)
    assert max(o.abs().max().item() for o in outs) > 65504
    check_v1(case, "dense", True, outs)
    q, k, v, kw = pack(case, "dense", device=DEV)
    o2 = flash_attention_v2(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    assert not torch.isfinite(o2).all()


@pytest.mark.parametrize("page", [16, 5])
def test_v1_fp32_pool_over_2gib(page):
    """The fp32 kernel over a pool past 2 GiB (its BUF = false instantiation)."""
    from kernels import flash_attention_v1
    from test_large_gpu import GIB2, big_pool
    case = make_case(3, 8, 2, 128, "self", torch.float32, "paged", 7500 + page, q_range=(50, 400))
    kc, kt = big_pool(case.ks, page, GIB2 + (64 << 20), 5)
    vc, vt = big_pool(case.vs, page, GIB2 + (64 << 20), 6)
    q = pack(case, "paged")[0].to(DEV)
    kw = dict(kv_indptr=torch.tensor(case.kv_lens, dtype=torch.int32, device=DEV),
              k_block_table=kt, v_block_table=vt, kv_page_size=page)
    out = flash_attention_v1(q, kc, vc, is_causal=True, **kw)
    torch.cuda.synchronize()
    check_v1(case, "paged", True, unpack(case, "paged", out.cpu(), kw))
    del kc, vc
    torch.cuda.empty_cache()
