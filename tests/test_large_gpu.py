"""GPU parity where K/V addresses leave the 32-bit range.

Tiles are read through buffer descriptors whose 32-bit offsets cover a few
rows from a 64-bit base: per tile for dense and ragged K/V, per page (or per
DMA instruction) for paged caches whose page size is a multiple of 16 (or 4
at head_dim 128, 8 at 64) rows.  Other page sizes, and the register-staged
fp32 kernel, address pool rows by 32-bit offsets from the pool base when
the pool fits them and through 64-bit addresses (the BUF = false kernels)
otherwise, or when the pool's size is not given (``kv_len = 0`` in
``fa2_params``).  These tests put sequences past the 2 GiB mark of real
pools and tensors, and run the whole paged matrix with an unknown pool size,
each against the C oracle and the reference tolerance.
"""

import math

import pytest
import torch

import workloads as W
from attn_cases import make_case, pack, unpack
from decode_cases import make_decode_case, pack_decode
from test_attention_gpu import check_all
from test_decode_gpu import check as check_decode

pytestmark = pytest.mark.gpu

DEV = "cuda"
GIB2 = 2 ** 31


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X")
    from kernels import _fa2
    _fa2.lib()
    yield


def big_pool(seqs, page, min_bytes, seed):
    """A NaN-filled pool of at least ``min_bytes`` on the GPU whose used pages
    all start past the 2 GiB mark, in a random order; table padded with -1."""
    H, D = seqs[0].shape[1], seqs[0].shape[2]
    row_bytes = H * D * seqs[0].element_size()
    first = math.ceil(GIB2 / (row_bytes * page))           # first page past 2 GiB
    nb = [(s.shape[0] + page - 1) // page for s in seqs]
    pages = max(math.ceil(min_bytes / (row_bytes * page)), first + sum(nb) + 7)
    cache = torch.full((pages * page, H, D), float("nan"), dtype=seqs[0].dtype, device=DEV)
    g = torch.Generator().manual_seed(seed)
    perm = first + torch.randperm(pages - first, generator=g)[: sum(nb)]
    table = torch.full((len(seqs), max(nb)), -1, dtype=torch.int32)
    cur = 0
    for b, s in enumerate(seqs):
        for j in range(nb[b]):
            pg = int(perm[cur])
            cur += 1
            table[b, j] = pg
            chunk = s[j * page: (j + 1) * page].to(DEV)
            cache[pg * page: pg * page + chunk.shape[0]] = chunk
            cache[pg * page + chunk.shape[0]: (pg + 1) * page] = 0
    assert int(table[table >= 0].min()) * page * row_bytes >= GIB2
    return cache, table.to(DEV)


# (q heads, kv heads, dtype, kernel choice): the two-head kernel (even
# groups), the one-head LDS kernel (odd groups), the register-staged fp32
# kernel and the short-problem kernel
KERNELS = [(8, 2, torch.bfloat16, "regular"), (6, 2, torch.float16, "regular"),
           (8, 2, torch.float32, "regular"), (8, 2, torch.bfloat16, "short")]
KERNEL_IDS = ["pp", "lds", "f32", "short"]


@pytest.mark.parametrize("qh,kvh,dtype,kernel", KERNELS, ids=KERNEL_IDS)
@pytest.mark.parametrize("page", [16, 5])
@pytest.mark.parametrize("causal", [False, True])
def test_paged_pool_over_2gib(qh, kvh, dtype, kernel, page, causal):
    from kernels.attention import flash_attention_v2
    case = make_case(3, qh, kvh, 128, "self", dtype, "paged", 5000 + page + int(causal) + qh,
                     q_range=(50, 400))
    print(f"pool>2GiB {qh}/{kvh} {dtype} page={page} causal={causal}", flush=True)
    kc, kt = big_pool(case.ks, page, GIB2 + (64 << 20), 1)
    vc, vt = big_pool(case.vs, page, GIB2 + (64 << 20), 2)
    q = pack(case, "paged")[0].to(DEV)
    kw = dict(kv_indptr=torch.tensor(case.kv_lens, dtype=torch.int32, device=DEV),
              k_block_table=kt, v_block_table=vt, kv_page_size=page)
    out = flash_attention_v2(q, kc, vc, is_causal=causal, kernel=kernel, **kw)
    torch.cuda.synchronize()
    check_all(case, "paged", causal, unpack(case, "paged", out.cpu(), kw))
    del kc, vc
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("page", [16, 5])
def test_decode_pool_over_2gib(dtype, page):
    """speculative_decode_attention (the decode kernel; fp32: the
    register-staged kernel in packed mode) over a pool past 2 GiB."""
    from kernels import speculative_decode_attention
    case = make_decode_case(3, 8, 2, 128, 4, dtype, "paged", 5100 + page, causal=True,
                            kv_range=(100, 900))
    kc, kt = big_pool(case.ks, page, GIB2 + (64 << 20), 3)
    vc, vt = big_pool(case.vs, page, GIB2 + (64 << 20), 4)
    q = torch.stack(case.qs).to(DEV)
    out = speculative_decode_attention(
        q, kc, vc, causal=True, kv_indptr=torch.tensor(case.kv_lens, dtype=torch.int32,
                                                       device=DEV),
        k_block_table=kt, v_block_table=vt, kv_page_size=page)
    torch.cuda.synchronize()
    out = out.cpu()
    check_decode(case, "paged", [out[b] for b in range(3)])
    del kc, vc
    torch.cuda.empty_cache()


def test_ragged_kv_over_2gib():
    """Ragged K/V of more than 2 GiB: sequence 0 holds ~4.3M keys (its 64
    queries see only the first keys under the causal mask), so sequences 1 and
    2 start past the 2 GiB mark."""
    from kernels.attention import flash_attention_v2
    H, D, dt = 2, 128, torch.bfloat16
    n0 = GIB2 // (H * D * 2) + 1000
    small = make_case(2, 8, H, D, "self", dt, "ragged", 5200, q_range=(100, 700))
    g = torch.Generator().manual_seed(5201)
    q0 = torch.randn((64, 8, D), generator=g).to(dt)
    k0 = torch.randn((64, H, D), generator=g).to(dt)
    v0 = torch.randn((64, H, D), generator=g).to(dt)
    q_lens = [64] + small.q_lens
    kv_lens = [n0] + small.kv_lens
    k = torch.zeros((sum(kv_lens), H, D), dtype=dt, device=DEV)
    v = torch.zeros_like(k)
    k[:64], v[:64] = k0.to(DEV), v0.to(DEV)
    off = n0
    for ks, vs in zip(small.ks, small.vs):
        k[off: off + ks.shape[0]] = ks.to(DEV)
        v[off: off + vs.shape[0]] = vs.to(DEV)
        off += ks.shape[0]
    q = torch.cat([q0] + small.qs, 0).to(DEV)
    qi, ki = W.indptr(q_lens, DEV), W.indptr(kv_lens, DEV)
    out = flash_attention_v2(q, k, v, is_causal=True, q_indptr=qi, kv_indptr=ki).cpu()
    # sequence 0 (top-left causal: its rows see the first 64 keys at most)
    from attn_cases import Case
    c0 = Case([q0], [k0], [v0], [64], [64], 8, H, D, dt)
    check_all(c0, "ragged", True, [out[:64]])
    check_all(small, "ragged", True, [out[64: 64 + q_lens[1]], out[64 + q_lens[1]:]])
    del k, v
    torch.cuda.empty_cache()


def unknown_pool_fwd(q, k, v, kw, causal, alignment="top_left", num_splits=0, kernel="auto"):
    """flash_attention_v2's paged call with kv_len = 0 in fa2_params (the
    pool size unknown to the library; kv_len_max as the wrapper passes it,
    so that the split factor, and with it the arithmetic, is the same)."""
    from kernels import _fa2
    from kernels._launch import enqueue, index_tensor, strides, table
    out = torch.empty_like(q)
    mask = (_fa2.MASK_NONE if not causal else
            _fa2.MASK_TOP_LEFT if alignment == "top_left" else _fa2.MASK_BOTTOM_RIGHT)
    enqueue(decode=False, layout=_fa2.LAYOUT_PAGED, mask=mask, num_splits=num_splits,
            batch=q.shape[0], q_heads=q.shape[1], kv_heads=k.shape[1], head_dim=q.shape[3],
            q_len=q.shape[2], kv_len=0, q=q, k=k, v=v, out=out, q_strides=strides(q),
            o_strides=strides(out), kvi=index_tensor(kw["kv_indptr"], q.device),
            kt=table(kw["k_block_table"], q.device), vt=table(kw["v_block_table"], q.device),
            page_size=kw["kv_page_size"],
            kv_len_max=kw["k_block_table"].shape[1] * kw["kv_page_size"],
            kernel={"auto": _fa2.KERNEL_AUTO, "regular": _fa2.KERNEL_REGULAR,
                    "short": _fa2.KERNEL_SHORT}[kernel])
    return out


@pytest.mark.parametrize("qh,kvh,dtype,kernel", KERNELS + [(8, 1, torch.float16, "regular")],
                         ids=KERNEL_IDS + ["mqa"])
@pytest.mark.parametrize("page", [16, 8, 5, 1])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("splits", [0, 3])
def test_paged_unknown_pool_size(qh, kvh, dtype, kernel, page, causal, splits):
    """kv_len = 0: the BUF = false kernels (per-page descriptors, or 64-bit
    row addresses for page sizes that are not a multiple of 4/8 rows), against
    the oracle and bitwise against the call with the pool size."""
    from kernels.attention import flash_attention_v2
    case = make_case(3, qh, kvh, 64 if page == 8 else 128, "self", dtype, "paged",
                     5300 + page + 2 * int(causal) + qh, q_range=(1, 300))
    q, k, v, kw = pack(case, "paged", device=DEV, shuffled_pages=True, seed=page, page=page)
    if kernel == "short" and splits > 1:
        pytest.skip("the short-problem kernel does not split across workgroups")
    out = unknown_pool_fwd(q, k, v, kw, causal, num_splits=splits, kernel=kernel)
    ref = flash_attention_v2(q, k, v, is_causal=causal, num_splits=splits, kernel=kernel, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu().view(torch.int16), ref.cpu().view(torch.int16))
    check_all(case, "paged", causal, unpack(case, "paged", out.cpu(), kw))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("page", [16, 5])
def test_decode_unknown_pool_size(dtype, page):
    """decode with kv_len = 0 through the ABI (the decode kernel's BUF = false
    instantiation), bitwise against the call with the pool size."""
    from kernels import _fa2, decode_attention
    from kernels._launch import enqueue, index_tensor, table
    case = make_decode_case(4, 8, 2, 128, 1, dtype, "paged", 5400 + page, kv_range=(1, 900))
    q, k, v, kw = pack_decode(case, "paged", device=DEV, shuffled=True, seed=page, page=page,
                              squeeze_m=True)
    ref = decode_attention(q, k, v, **kw)
    out = torch.empty_like(q)
    q4, o4 = q.unsqueeze(2), out.unsqueeze(2)
    ab = lambda t: (t.stride(0), t.stride(1), t.stride(1))  # noqa: E731 (M = 1)
    enqueue(decode=True, layout=_fa2.LAYOUT_PAGED, mask=_fa2.MASK_NONE, num_splits=0,
            batch=4, q_heads=8, kv_heads=2, head_dim=128, q_len=1, kv_len=0, q=q4, k=k, v=v,
            out=o4, q_strides=ab(q4), o_strides=ab(o4),
            kvi=index_tensor(kw["kv_indptr"], q.device), kt=table(kw["k_block_table"], q.device),
            vt=table(kw["v_block_table"], q.device), page_size=page,
            kv_len_max=kw["k_block_table"].shape[1] * page)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu().view(torch.int16), ref.cpu().view(torch.int16))
    o = out.cpu().unsqueeze(2)
    check_decode(case, "paged", [o[b] for b in range(4)])
