"""C ABI checks that need no GPU: the library loads, exports every symbol
include/fa2.h declares, its struct layout matches the ctypes mirror, and
every validation error is reported before any device work."""

import ctypes
import os
import re

import pytest
import torch

from kernels import _fa2

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fa2.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(fa2_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_fa2.LIB_PATH)
    names = declared_functions()
    assert set(names) == set(_fa2.EXPORTS), names
    for n in names:
        assert hasattr(lib, n), n


def test_struct_layout_matches():
    assert _fa2.lib().fa2_params_size() == ctypes.sizeof(_fa2.Fa2Params)
    assert _fa2.lib().fa2_abi_version() == _fa2.ABI_VERSION == 7


def test_strerror_for_every_code():
    seen = set()
    for code in range(16):
        msg = _fa2.lib().fa2_strerror(code).decode()
        assert msg and "unknown" not in msg
        seen.add(msg)
    assert len(seen) == 16
    assert "unknown" in _fa2.lib().fa2_strerror(999).decode()


def dense_params(**kw):
    p = _fa2.Fa2Params()
    p.layout, p.dtype, p.mask, p.num_splits = 0, 1, 1, 1
    p.batch, p.q_heads, p.kv_heads, p.head_dim, p.q_len, p.kv_len = 2, 8, 2, 128, 300, 300
    p.q_sb, p.q_sh, p.q_ss = 8 * 300 * 128, 300 * 128, 128
    p.k_sb, p.k_sh, p.k_ss = 2 * 300 * 128, 300 * 128, 128
    p.v_sb, p.v_sh, p.v_ss = p.k_sb, p.k_sh, p.k_ss
    p.o_sb, p.o_sh, p.o_ss = p.q_sb, p.q_sh, p.q_ss
    p.softmax_scale = 128 ** -0.5
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def rc_ws(p):
    n = ctypes.c_size_t(0)
    return _fa2.lib().fa2_fwd_workspace_size(ctypes.byref(p), ctypes.byref(n)), n.value


def rc_fwd(p):
    return _fa2.lib().fa2_fwd(ctypes.byref(p), None)


@pytest.mark.parametrize("field,value,code", [
    ("layout", 3, 2), ("dtype", 7, 3), ("mask", 5, 4), ("q_heads", 7, 5), ("batch", -1, 5),
    ("head_dim", 96, 6), ("q_ss", 100, 7), ("num_splits", 65, 11), ("num_splits", -1, 11),
    ("max_workgroups", -1, 5), ("kv_len_max", -1, 5), ("arith", 2, 3), ("arith", -1, 3),
    ("decode_spin_cap", -1, 5), ("kernel", 3, 5), ("kernel", -1, 5),
    ("k_ss", (1 << 24) + 8, 13),  # a 32 MiB+ row stride: tile offsets leave 32 bits
    ("q_ss", (1 << 24) + 8, 13),  # the same for the q-block offsets of the short kernel
    ("q_ss", 1 << 26, 13),  # 128 MiB: uint32(q_ss * 2) alone would wrap to 0
])
def test_validation_errors(field, value, code):
    p = dense_params(**{field: value})
    assert rc_ws(p)[0] == code
    assert rc_fwd(p) == code  # reported before any HIP call


def test_null_params():
    assert _fa2.lib().fa2_fwd(None, None) == 1
    n = ctypes.c_size_t(0)
    assert _fa2.lib().fa2_fwd_workspace_size(None, ctypes.byref(n)) == 1


def test_ragged_and_paged_argument_checks():
    p = dense_params(layout=1)
    assert rc_ws(p)[0] == 9  # ragged without indptr
    p = dense_params(layout=2, kv_indptr=16, k_block_table=16, v_block_table=16, page_size=0)
    assert rc_ws(p)[0] == 8
    p = dense_params(layout=2, kv_indptr=16, k_block_table=16, page_size=16)
    assert rc_ws(p)[0] == 8


def test_null_tensor_pointers_rejected_before_launch():
    p = dense_params()
    assert rc_fwd(p) == 1  # q/k/v/o NULL


def test_workspace_sizes():
    # dense, no split: nothing
    assert rc_ws(dense_params()) == (0, 0)
    # dense split 4: (m,l) + O partials for grid_x = ceil(300/128) * 2 * 8 workgroups
    rc, n = rc_ws(dense_params(num_splits=4))
    grid = 3 * 2 * 8
    assert rc == 0 and n >= 4 * grid * 128 * (2 + 128) * 4
    # ragged: work list of ceil(Tq/128) + B entries of 8 bytes + counter
    p = dense_params(layout=1, q_indptr=16, kv_indptr=16, batch=5, q_len=1000, kv_len=1000)
    rc, n = rc_ws(p)
    assert rc == 0 and n >= (8 + 5) * 8 + 4
    # empty problem: no workspace
    assert rc_ws(dense_params(batch=0)) == (0, 0)


def c4_paged_params(**kw):
    """c4's shape: 32 paged sequences of one 128-row q-block, Hq32/Hkv8 D128
    bf16, bottom-right causal, page 16, pool of 9042 pages."""
    H, KH, D, M, rows = 32, 8, 128, 128, 9042 * 16
    p = _fa2.Fa2Params()
    p.layout, p.dtype, p.mask, p.num_splits = (_fa2.LAYOUT_PAGED, _fa2.DTYPE_BF16,
                                               _fa2.MASK_BOTTOM_RIGHT, 0)
    p.batch, p.q_heads, p.kv_heads, p.head_dim, p.q_len, p.kv_len = 32, H, KH, D, M, rows
    p.q_sb, p.q_sh, p.q_ss = H * M * D, M * D, D
    p.k_sb, p.k_sh, p.k_ss = 0, D, KH * D
    p.v_sb, p.v_sh, p.v_ss = 0, D, KH * D
    p.o_sb, p.o_sh, p.o_ss = p.q_sb, p.q_sh, p.q_ss
    p.page_size, p.kv_len_max, p.k_table_stride, p.v_table_stride = 16, 8192, 512, 512
    p.q = p.k = p.v = p.o = p.kv_indptr = p.k_block_table = p.v_block_table = 16
    p.softmax_scale = D ** -0.5
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_paged_balanced_walk_workspace():
    """More two-head units (512) than CUs, one q-block per sequence: the plan
    takes the balanced walk, whose part slots (4 per workgroup of 128 rows
    of (m, l) and D floats) set the workspace.  A capped grid keeps rounds of
    whole units and needs only the work list."""
    rc, n = rc_ws(c4_paged_params())
    assert rc == 0 and n >= 4 * 256 * 128 * (2 + 128) * 4
    rc, n = rc_ws(c4_paged_params(max_workgroups=256))
    assert rc == 0 and n < 1 << 20
    # forced splits and fewer units than CUs (16 sequences: 256 units) run whole units too
    assert rc_ws(c4_paged_params(num_splits=1))[1] < 1 << 20
    assert rc_ws(c4_paged_params(batch=16))[1] < 1 << 20


def test_fp32_workspace_holds_fp16_copies():
    """fp32 tensors with the reference's fp16 rounding (flash_attention_v2)
    at head_dim 64/128, dense or ragged: fp16 copies of q, k and v plus one
    split's fp32 partials.  fp32 arithmetic (v1), other head dims and paged
    pools need neither."""
    q_el, kv_el = 2 * 8 * 300 * 128, 2 * 2 * 300 * 128
    parts = 1 * (3 * 2 * 8) * 128 * (2 + 128) * 4  # 24 one-head units of 128 rows
    rc, n = rc_ws(dense_params(dtype=2))
    assert rc == 0 and n >= 2 * (q_el + 2 * kv_el) + parts
    assert rc_ws(dense_params(dtype=2, arith=1)) == (0, 0)
    rc, n = rc_ws(dense_params(dtype=2, head_dim=32, q_sh=300 * 32, q_ss=32, q_sb=8 * 300 * 32,
                               k_sb=2 * 300 * 32, k_sh=300 * 32, k_ss=32, v_sb=2 * 300 * 32,
                               v_sh=300 * 32, v_ss=32, o_sb=8 * 300 * 32, o_sh=300 * 32, o_ss=32))
    assert (rc, n) == (0, 0)


def test_workspace_too_small_is_rejected():
    p = dense_params(num_splits=2, q=16, k=16, v=16, o=16)
    rc, n = rc_ws(p)
    assert rc == 0 and n > 0
    p.workspace, p.workspace_bytes = 16, n - 1
    assert rc_fwd(p) == 10


def test_wrapper_asserts_is_cuda_on_cpu_tensors():
    from kernels.attention import flash_attention_v2
    q = torch.zeros((1, 2, 8, 64), dtype=torch.float16)
    with pytest.raises(AssertionError):
        flash_attention_v2(q, q, q)
    with pytest.raises(AssertionError):
        flash_attention_v2(q, q.to(torch.bfloat16), q)


def test_product_path_does_not_import_the_oracle():
    pkg = os.path.join(ROOT, "triton-kernels_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "from oracle" not in text, f
                assert "fa2_oracle" not in text, f


# ---- decode / speculative decode entry points ------------------------------

def decode_params(M=1, **kw):
    """q/o [B=2, Hq=8, M, D=128] over a dense K/V [2, 2, 4096, 128]."""
    p = dense_params(mask=0, num_splits=0, q_len=M, kv_len=4096, k_sb=2 * 4096 * 128,
                     k_sh=4096 * 128, v_sb=2 * 4096 * 128, v_sh=4096 * 128)
    p.q_sb, p.q_sh, p.q_ss = 8 * M * 128, M * 128, 128 if M > 1 else M * 128
    p.o_sb, p.o_sh, p.o_ss = p.q_sb, p.q_sh, p.q_ss
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def rc_dec(p):
    n = ctypes.c_size_t(0)
    r1 = _fa2.lib().fa2_decode_workspace_size(ctypes.byref(p), ctypes.byref(n))
    r2 = _fa2.lib().fa2_decode_fwd(ctypes.byref(p), None)
    return r1, r2, n.value


@pytest.mark.parametrize("M", [1, 4, 16])
def test_decode_workspace_ok(M):
    r1, _, n = rc_dec(decode_params(M, q=0))
    assert r1 == 0
    # 8 query heads share 2 kv heads: 4 units of 64 key tiles, so the KV sweep is split
    assert n > 0


@pytest.mark.parametrize("field,value,code", [
    ("mask", 1, 4),     # top-left causal has no decode meaning
    ("mask", 3, 4),
    ("q_sh", 256, 14),  # heads of a group are not one run of rows
    ("o_ss", 64, 14),
    ("head_dim", 96, 6),
    ("num_splits", 65, 11),
])
def test_decode_validation_errors(field, value, code):
    r1, r2, _ = rc_dec(decode_params(4, **{field: value}))
    assert r1 == code and r2 == code


def test_decode_ragged_needs_only_kv_indptr():
    p = decode_params(1, layout=1)
    assert rc_dec(p)[0] == 9           # kv_indptr missing
    p.kv_indptr = 0x1000               # never dereferenced on the host
    assert rc_dec(p)[0] == 0           # q_indptr is not needed


def test_decode_mqa_m1_any_head_stride():
    """One query head per kv head: the group is one row, any head stride."""
    p = decode_params(1, kv_heads=8, q_sh=256, q_ss=128, o_sh=256, o_ss=128,
                      k_sb=8 * 300 * 128, v_sb=8 * 300 * 128)
    assert rc_dec(p)[0] == 0


def paged_params(ctx_rows, **kw):
    """Paged B1 Hq8 Hkv8 q128 D128 over a pool of ctx_rows rows, page 16."""
    p = dense_params(layout=2, mask=0, num_splits=0, batch=1, q_heads=8, kv_heads=8, q_len=128,
                     kv_len=ctx_rows, kv_indptr=16, k_block_table=16, v_block_table=16,
                     page_size=16, k_table_stride=64, v_table_stride=64)
    p.q_sb, p.q_sh, p.q_ss = 8 * 128 * 128, 128 * 128, 128
    p.o_sb, p.o_sh, p.o_ss = p.q_sb, p.q_sh, p.q_ss
    p.k_sb, p.k_sh, p.k_ss = 0, 128, 8 * 128
    p.v_sb, p.v_sh, p.v_ss = 0, 128, 8 * 128
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_paged_split_bounded_by_pool_and_table():
    """A short paged context is not split (no partials workspace): the split
    count is bounded by the pool's rows, or by kv_len_max (table width x page
    size), as dense and ragged calls are bounded by their KV length."""
    rc, n = rc_ws(paged_params(208))
    assert rc == 0 and n < 4096           # work list only
    rc, n = rc_ws(paged_params(0, kv_len_max=208))
    assert rc == 0 and n < 4096
    rc, n = rc_ws(paged_params(1 << 20, kv_len_max=256))
    assert rc == 0 and n < 4096
    # an unknown bound keeps the old behaviour (split for parallelism)
    rc, n = rc_ws(paged_params(0))
    assert rc == 0 and n > (1 << 20)


def test_noalloc_rejects_before_any_launch():
    """fa2_fwd_noalloc: validation errors, and a forced split whose partials
    exceed the static scratch, are reported before any HIP call."""
    lib = _fa2.lib()
    assert lib.fa2_fwd_noalloc(None, None) == 1
    assert lib.fa2_fwd_noalloc(ctypes.byref(dense_params(head_dim=96)), None) == 6
    # 64 splits of B2 Hq8 Lq300: 64 * 48 workgroups * 128 rows * 130 floats > 32 MiB
    p = dense_params(num_splits=64, q=16, k=16, v=16, o=16)
    assert rc_ws(p)[1] > _fa2.NOALLOC_SCRATCH_BYTES
    assert lib.fa2_fwd_noalloc(ctypes.byref(p), None) == 15


def test_launch_extension_loads_and_shares_the_library():
    """The PyTorch-ROCm launch extension (csrc/fa2_torch.cpp) is built next to
    libfa2.so, links it by soname, and the process maps one copy of it
    whichever of ctypes and the extension loads it first."""
    from kernels import _launch
    x = _launch.ext()
    assert x is not None, _launch._EXT_ERROR
    assert callable(x.fwd)
    _fa2.lib()
    maps = [l for l in open("/proc/self/maps") if l.rstrip().endswith("libfa2.so")]
    assert len({l.split()[-1] for l in maps}) == 1
