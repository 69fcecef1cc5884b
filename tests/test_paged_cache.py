"""CPU checks of the paged-cache writer's oracle (oracle/paged_cache.py) and
of the ``fa2_kv_append`` C ABI's validation (no kernel is launched).

The reference holds no fixtures for its cache builders; the restatement is
pinned by round trips (write, then read back through the table with the
attention kernels' addressing), by agreement with the independently written
page-pool helpers of workloads.py, by the padding and length conventions of
tests/test_attention.py:101-134 and benchmarks/attention.py:351-431, and by
appends that must equal the concatenated sequences.
"""

import ctypes

import pytest
import torch

import workloads as W
from oracle import paged_cache as PC
from kernels import _fa2


def seqs(lens, H=2, D=8, seed=0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn((n, H, D), generator=g).to(dtype) for n in lens]


@pytest.mark.parametrize("page", [1, 5, 16])
def test_allocate_round_trip_and_format(page):
    lens = [7, 1, 33, 16]
    xs = seqs(lens)
    cache, tbl = PC.allocate_paged_cache(xs, lens, 2, 8, page)
    nb = [(n + page - 1) // page for n in lens]
    assert cache.shape == (sum(nb) * page, 2, 8)
    assert tbl.shape == (4, max(nb)) and tbl.dtype == torch.int32
    cur = 0
    for b, n in enumerate(nb):  # pages in sequence order, padding 0
        assert tbl[b, :n].tolist() == list(range(cur, cur + n))
        assert (tbl[b, n:] == 0).all()
        cur += n
    for b, n in enumerate(lens):
        assert torch.equal(PC.gather(cache, tbl, b, n, page), xs[b])
    ref_cache, ref_tbl = W.paged_cache_contiguous(xs, page)
    assert torch.equal(cache, ref_cache) and torch.equal(tbl, ref_tbl)


def test_build_paged_cache_conventions():
    lens = [5, 20, 3]
    xs = seqs(lens, seed=1)
    cache, lengths, tbl = PC.build_paged_cache(xs, 8)
    assert lengths.tolist() == lens and lengths.dtype == torch.int32
    assert tbl[0, 1].item() == -1 and tbl[2, 1].item() == -1  # -1 padding
    for b, n in enumerate(lens):
        assert torch.equal(PC.gather(cache, tbl, b, n, 8), xs[b])
    # every page tail past a sequence's end is zero
    assert (cache[5:8] == 0).all()


def test_append_equals_concatenation():
    page, lens, add = 4, [3, 0, 9], [2, 5, 1]
    old = seqs(lens, seed=2)
    new = seqs(add, seed=3)
    g = torch.Generator().manual_seed(4)
    full = [torch.cat([o, n], 0) for o, n in zip(old, new)]
    # a shuffled pool large enough for the final lengths
    cache, tbl = W.paged_cache_shuffled(full, page, 3, g, fill=0.0)
    for b, n in enumerate(add):  # blank the rows about to be appended
        for j in range(lens[b], lens[b] + n):
            cache[int(tbl[b, j // page]) * page + j % page] = 0
    ip = W.indptr(add)
    out = PC.append(cache, tbl, torch.cat(new, 0), ip, page,
                    start=torch.tensor(lens, dtype=torch.int32))
    for b in range(3):
        assert torch.equal(PC.gather(out, tbl, b, lens[b] + add[b], page), full[b])


def test_append_skips_rows_outside_the_table_or_cache():
    page = 4
    cache = torch.zeros((3 * page, 1, 4))
    # -1, 7 and 3 are not pages of a 3-page cache
    tbl = torch.tensor([[0, -1, 7], [2, 1, 3]], dtype=torch.int32)
    new = torch.arange(1, 1 + 2 * 13 * 4, dtype=torch.float32).reshape(26, 1, 4)
    ip = torch.tensor([0, 12, 25], dtype=torch.int32)  # sequence 1: 13 rows, 4 pages
    out = PC.append(cache, tbl, new, ip, page)
    assert torch.equal(out[0:4], new[0:4])        # seq 0, logical page 0 -> page 0
    assert torch.equal(out[8:12], new[12:16])     # seq 1, logical page 0 -> page 2
    assert torch.equal(out[4:8], new[16:20])      # seq 1, logical page 1 -> page 1
    # nothing else was written: seq 0's pages 1, 2, seq 1's page 2 (entry 3)
    # and its 13th row (logical page 3, past the table width)
    assert out.count_nonzero() == 3 * 4 * 4


# ---- fa2_kv_append validation (returns before any device work) -------------

def params(**kw):
    p = _fa2.KvAppendParams()
    p.dtype, p.batch, p.kv_heads, p.head_dim, p.num_rows = 1, 2, 2, 64, 10
    p.page_size, p.num_pages, p.table_width = 16, 4, 2
    p.k_table_stride = p.v_table_stride = 2
    p.new_ts, p.new_hs, p.cache_ts, p.cache_hs = 128, 64, 128, 64
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def rc(p):
    return _fa2.lib().fa2_kv_append(ctypes.byref(p), None)


def test_kv_append_struct_and_validation():
    assert _fa2.lib().fa2_kv_append_params_size() == ctypes.sizeof(_fa2.KvAppendParams)
    assert rc(params(dtype=5)) == 3
    assert rc(params(page_size=0)) == 5
    assert rc(params(kv_heads=0)) == 5
    assert rc(params()) == 1                          # pointers missing
    assert rc(params(num_rows=0)) == 0                # nothing to write
    assert rc(params(batch=0)) == 0
    p = params(k_new=16, k_cache=16, new_indptr=16, k_block_table=16, head_dim=4)
    assert rc(p) == 7                                 # 8-byte rows
    p = params(k_new=16, k_cache=16, new_indptr=16, k_block_table=16, v_new=16)
    assert rc(p) == 1                                 # V half given
    p = params(k_new=16, k_cache=16, new_indptr=16, k_block_table=16, cache_hs=60)
    assert rc(p) == 7                                 # misaligned head stride
