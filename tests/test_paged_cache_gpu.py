"""GPU parity of the paged KV-cache writer (kernels.paged_cache, fa2_kv_append
through the C ABI) against the CPU restatement of the reference's cache
builders (oracle/paged_cache.py).  Writes are copies, so every check is
bitwise: the device-built caches and tables equal the reference helpers',
appends through shuffled tables equal the restated appends, rows outside the
table or the cache are never written, and attention over a cache grown by
appends equals attention over the reference-built cache.
"""

import pytest
import torch

import workloads as W
from oracle import paged_cache as PC

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.float16, torch.bfloat16, torch.float32]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X")
    from kernels import _fa2
    _fa2.lib()
    yield


def seqs(lens, H, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn((n, H, D), generator=g).to(dtype) for n in lens]


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("page", [1, 5, 16, 32])
@pytest.mark.parametrize("D", [64, 128])
def test_allocate_paged_cache_matches_reference_helper(dtype, page, D):
    from kernels.paged_cache import allocate_paged_cache
    lens = [1, 37, 16, 200, 3]
    xs = seqs(lens, 4, D, dtype, seed=page + D)
    cache, tbl = allocate_paged_cache([x.to(DEV) for x in xs], lens, 4, D, page)
    torch.cuda.synchronize()
    ref_cache, ref_tbl = PC.allocate_paged_cache(xs, lens, 4, D, page)
    assert torch.equal(cache.cpu(), ref_cache) and torch.equal(tbl.cpu(), ref_tbl)


def test_build_paged_cache_matches_benchmark_helper():
    from kernels.paged_cache import build_paged_cache
    xs = seqs([9, 64, 1, 100], 8, 128, torch.bfloat16, seed=5)
    cache, lengths, tbl = build_paged_cache([x.to(DEV) for x in xs], 16)
    torch.cuda.synchronize()
    rc, rl, rt = PC.build_paged_cache(xs, 16)
    assert torch.equal(cache.cpu(), rc) and torch.equal(lengths.cpu(), rl)
    assert torch.equal(tbl.cpu(), rt)


@pytest.mark.parametrize("page", [8, 16])
@pytest.mark.parametrize("cache4d", [False, True])
def test_append_through_shuffled_tables(page, cache4d):
    """K and V with independent shuffled tables, appends at non-zero start
    positions (a decode step of several tokens per sequence)."""
    from kernels.paged_cache import paged_kv_append
    lens, add = [5, 0, 40, 17, 1], [1, 3, 8, 0, 20]
    H, D, dt = 8, 128, torch.bfloat16
    g = torch.Generator().manual_seed(11)
    full_k = [torch.cat(p, 0) for p in zip(seqs(lens, H, D, dt, 1), seqs(add, H, D, dt, 2))]
    full_v = [torch.cat(p, 0) for p in zip(seqs(lens, H, D, dt, 3), seqs(add, H, D, dt, 4))]
    kc, kt = W.paged_cache_shuffled(full_k, page, 4, g, fill=0.0)
    vc, vt = W.paged_cache_shuffled(full_v, page, 4, g, fill=0.0)
    new_k = torch.cat([k[n:] for k, n in zip(full_k, lens)], 0)
    new_v = torch.cat([v[n:] for v, n in zip(full_v, lens)], 0)
    ip = W.indptr(add)
    start = torch.tensor(lens, dtype=torch.int32)
    # the caches before the append: the new rows' slots hold stale data (7.0)
    kc0 = PC.append(kc, kt, torch.full_like(new_k, 7.0), ip, page, start)
    vc0 = PC.append(vc, vt, torch.full_like(new_v, 7.0), ip, page, start)
    dk, dv = kc0.to(DEV), vc0.to(DEV)
    if cache4d:
        dk, dv = dk.view(-1, page, H, D), dv.view(-1, page, H, D)
    paged_kv_append(dk, dv, kt.to(DEV), vt.to(DEV), new_k.to(DEV), new_v.to(DEV), ip.to(DEV),
                    page, start_pos=start.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(dk.reshape(kc.shape).cpu(), kc) and torch.equal(dv.reshape(vc.shape).cpu(), vc)


def test_rows_outside_table_or_cache_are_not_written():
    from kernels.paged_cache import paged_kv_append
    page = 4
    tbl = torch.tensor([[0, -1, 7], [2, 1, 3]], dtype=torch.int32)
    new = torch.arange(1, 1 + 26 * 64, dtype=torch.float32).reshape(26, 1, 64)
    ip = torch.tensor([0, 12, 25], dtype=torch.int32)
    cache = torch.zeros((3 * page, 1, 64))
    dc = cache.to(DEV)
    paged_kv_append(dc, None, tbl.to(DEV), None, new.to(DEV), None, ip.to(DEV), page)
    torch.cuda.synchronize()
    assert torch.equal(dc.cpu(), PC.append(cache, tbl, new, ip, page))


def test_decode_over_appended_cache_equals_reference_built_cache():
    """Grow a cache token by token with paged_kv_append (the serving loop),
    then decode_attention over it equals decode over the cache the
    reference's helper builds from the whole sequences (bitwise)."""
    from kernels import decode_attention
    from kernels.paged_cache import paged_kv_append
    page, H, QH, D, dt = 16, 2, 8, 128, torch.float16
    lens = [30, 47, 5]
    ks = seqs(lens, H, D, dt, 21)
    vs = seqs(lens, H, D, dt, 22)
    ref_k, tbl = PC.allocate_paged_cache(ks, lens, H, D, page)
    ref_v, _ = PC.allocate_paged_cache(vs, lens, H, D, page)
    kc = torch.zeros_like(ref_k).to(DEV)
    vc = torch.zeros_like(ref_v).to(DEV)
    t = tbl.to(DEV)
    cur = [0, 0, 0]
    while any(c < n for c, n in zip(cur, lens)):  # up to 8 tokens per step
        add = [min(8, n - c) for c, n in zip(cur, lens)]
        nk = torch.cat([k[c:c + a] for k, c, a in zip(ks, cur, add)], 0).to(DEV)
        nv = torch.cat([v[c:c + a] for v, c, a in zip(vs, cur, add)], 0).to(DEV)
        paged_kv_append(kc, vc, t, t, nk, nv, W.indptr(add).to(DEV), page,
                        start_pos=torch.tensor(cur, dtype=torch.int32, device=DEV))
        cur = [c + a for c, a in zip(cur, add)]
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu(), ref_k) and torch.equal(vc.cpu(), ref_v)
    q = torch.randn((3, QH, D), generator=torch.Generator().manual_seed(23)).to(dt).to(DEV)
    lengths = torch.tensor(lens, dtype=torch.int32, device=DEV)
    a = decode_attention(q, kc, vc, kv_indptr=lengths, k_block_table=t, v_block_table=t,
                         kv_page_size=page)
    b = decode_attention(q, ref_k.to(DEV), ref_v.to(DEV), kv_indptr=lengths, k_block_table=t,
                         v_block_table=t, kv_page_size=page)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
