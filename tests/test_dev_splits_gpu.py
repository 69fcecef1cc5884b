"""GPU checks of the automatic split count that the plan kernel lowers.

With automatic splits the host sizes the split count from the longest KV
sweep a sequence can have.  For ragged K/V the host knows only the total of
all sequences; for paged K/V it knows the block table's width.  The plan
kernel knows the longest sweep of the call and lowers the count
(csrc/fa2_device.h, fa2_plan_kernel): the forward kernels run that many
splits out of a grid sized for the host's count, and the combine kernel
exits at once when one split remains.  (A ragged launch whose workgroups
all fit on the GPU at once skips the plan kernel: each workgroup derives
the same split count itself, and the forward kernel merges the splits.)
Each split count gives the same
arithmetic wherever it is decided, so an automatic call must equal, bit for
bit, the call that forces the count the plan kernel chose.  It must also
pass the oracle bars.
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


def run(case, layout, causal, num_splits, kernel="regular", **extra):
    from kernels.attention import flash_attention_v2
    q, k, v, kw = pack(case, layout, device=DEV)
    kw.update(extra)
    out = flash_attention_v2(q, k, v, is_causal=causal, num_splits=num_splits, kernel=kernel,
                             **kw)
    torch.cuda.synchronize()
    return out.cpu(), kw


def same(a, b):
    if a.dtype == torch.float32:
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("heads", [(8, 2), (8, 8)], ids=["gqa", "mha"])
@pytest.mark.parametrize("causal", [False, True])
def test_short_ragged_sequences_run_unsplit(heads, causal):
    """The reference benchmark's small ragged point (B16, q = kv = 128): the
    host's bound is 2048 keys (32 tiles, 2 splits); every sweep is 2 tiles."""
    QH, KVH = heads
    n = 16
    case = make_case(n, QH, KVH, 128, "self", torch.bfloat16, "ragged", 5000 + QH + int(causal),
                     q_lens=[128] * n, kv_lens=[128] * n)
    print(f"dev splits ragged B16 L128 {QH}/{KVH} causal={causal}", flush=True)
    auto, kw = run(case, "ragged", causal, 0)
    one, _ = run(case, "ragged", causal, 1)
    assert same(auto, one)
    check_all(case, "ragged", causal, unpack(case, "ragged", auto, kw))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=str)
def test_ragged_split_count_lowered_not_removed(dtype):
    """16 sequences of 64 queries over 1100 keys and one over 2100: the
    host's bound (18600 keys) gives 3 splits, the longest sweep (33 tiles)
    2.  The automatic call equals the call forced to 2 splits, and the
    combine merges them."""
    n = 16
    kl = [2100] + [1100] * (n - 1)
    D = 128 if dtype != torch.float32 else 64
    case = make_case(n, 8, 2, D, "cross", dtype, "ragged", 5100, q_lens=[64] * n, kv_lens=kl)
    print(f"dev splits ragged lowered 3 -> 2 {dtype}", flush=True)
    auto, kw = run(case, "ragged", False, 0)
    two, _ = run(case, "ragged", False, 2)
    assert same(auto, two)
    check_all(case, "ragged", False, unpack(case, "ragged", auto, kw))


def test_paged_wide_table_short_sequences():
    """A block table wider than the sequences (2048 keys of pages, 100-300
    used): the host bound gives 2 splits, the sweeps need one."""
    n = 16
    kl = [100 + 13 * b for b in range(n)]
    case = make_case(n, 8, 2, 128, "cross", torch.bfloat16, "paged", 5200, q_lens=[64] * n,
                     kv_lens=kl)
    q, k, v, kw = pack(case, "paged", device=DEV)
    # widen the tables with -1 padding to 2048 keys (128 pages of 16)
    for name in ("k_block_table", "v_block_table"):
        t = kw[name]
        wide = torch.full((t.shape[0], 2048 // kw["kv_page_size"]), -1, dtype=t.dtype,
                          device=t.device)
        wide[:, : t.shape[1]] = t
        kw[name] = wide
    from kernels.attention import flash_attention_v2
    print("dev splits paged wide table", flush=True)
    auto = flash_attention_v2(q, k, v, is_causal=False, num_splits=0, kernel="regular", **kw)
    one = flash_attention_v2(q, k, v, is_causal=False, num_splits=1, kernel="regular", **kw)
    auto, one = auto.cpu(), one.cpu()
    assert same(auto, one)
    check_all(case, "paged", False, unpack(case, "paged", auto, kw))


def test_long_sequence_keeps_host_splits():
    """One sequence long enough for the host's count (8 splits: 24 units for
    512 slots, 8492 keys of bound) sweeps 128 tiles: nothing is lowered."""
    case = make_case(2, 8, 2, 128, "cross", torch.bfloat16, "ragged", 5300, q_lens=[64, 64],
                     kv_lens=[8192, 300])
    print("dev splits ragged long", flush=True)
    auto, kw = run(case, "ragged", False, 0)
    eight, _ = run(case, "ragged", False, 8)
    assert same(auto, eight)
    check_all(case, "ragged", False, unpack(case, "ragged", auto, kw))


@pytest.mark.parametrize("heads", [(8, 2), (8, 8)], ids=["gqa", "mha"])
@pytest.mark.parametrize("causal,splits", [(False, 0), (False, 1), (False, 3), (True, 0),
                                           (True, 2)])
def test_inline_plan_equals_plan_kernel(heads, causal, splits):
    """A ragged launch whose workgroups all fit on the GPU at once runs
    without the plan kernel: each workgroup derives the item list and the
    split count from the sequence lengths, and the forward kernel merges its
    own splits (no combine launch).  max_workgroups > 0 keeps the plan
    kernel and the combine kernel.  Both must give the same output bit for
    bit (each unit's arithmetic does not depend on where it runs), and pass
    the oracle bars."""
    QH, KVH = heads
    lens = [64, 200, 1, 130, 17, 300]
    kv = lens if causal else [300, 900, 50, 1200, 10, 640]
    case = make_case(len(lens), QH, KVH, 128, "self" if causal else "cross", torch.bfloat16,
                     "ragged", 5400 + QH + 10 * int(causal) + splits, q_lens=lens, kv_lens=kv)
    print(f"inline plan {QH}/{KVH} causal={causal} splits={splits}", flush=True)
    inline, kw = run(case, "ragged", causal, splits)
    planned, _ = run(case, "ragged", causal, splits, max_workgroups=1 << 20)
    assert same(inline, planned)
    check_all(case, "ragged", causal, unpack(case, "ragged", inline, kw))


@pytest.mark.parametrize("layout", ["dense", "paged"])
@pytest.mark.parametrize("causal", [False, True])
def test_kernel_choice_by_grid_fill_keeps_bits(layout, causal):
    """B16 Hq8/Hkv2 q128 (the reference benchmark's small GQA point): the
    two-head grid (64 workgroups) would not cover the CUs, so the call runs
    the one-head kernel; max_workgroups = CUs keeps the two-head kernel.
    Both kernels compute the same arithmetic, so the outputs are equal bit
    for bit, and they pass the oracle bars."""
    n = 16
    case = make_case(n, 8, 2, 128, "cross", torch.bfloat16, layout, 5500 + int(causal),
                     dense_q_range=(128, 128), dense_kv_range=(512, 512), q_lens=[128] * n,
                     kv_lens=[512] * n)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    print(f"kernel choice {layout} causal={causal}", flush=True)
    one, kw = run(case, layout, causal, 0)
    two, _ = run(case, layout, causal, 0, max_workgroups=cus)
    assert same(one, two)
    check_all(case, layout, causal, unpack(case, layout, one, kw))
