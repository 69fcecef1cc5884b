"""The two launch paths of flash_attention_v2 enqueue the same libfa2.so
entry point with the same parameter block: the C++ extension
(csrc/fa2_torch.cpp, the default) and the ctypes path (kernels/_launch.py).
Their outputs are compared bit for bit over every layout, fp32, forced
splits, bottom-right masks, the kernel choices and non-contiguous inputs."""

import pytest
import torch

from attn_cases import make_case, pack

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X")
    from kernels import _launch
    assert _launch.ext() is not None, _launch._EXT_ERROR
    yield


def both(q, k, v, **kw):
    import kernels.attention as A
    A.USE_EXT = True
    a = A.flash_attention_v2(q, k, v, **kw)
    A.USE_EXT = False
    try:
        b = A.flash_attention_v2(q, k, v, **kw)
    finally:
        A.USE_EXT = True
    torch.cuda.synchronize()
    return a.cpu(), b.cpu()


def same(a, b):
    if a.dtype == torch.float32:
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("layout", ["dense", "ragged", "paged"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("extra", [{}, {"num_splits": 3}, {"kernel": "short"},
                                   {"kernel": "regular"},
                                   {"causal_alignment": "bottom_right"}],
                         ids=["auto", "split3", "short", "regular", "bottom_right"])
def test_extension_equals_ctypes_path(layout, dtype, extra):
    case = make_case(3, 8, 2, 128, "self", dtype, layout, 7000 + len(extra),
                     q_range=(30, 500), dense_q_range=(300, 300))
    q, k, v, kw = pack(case, layout, device=DEV, shuffled_pages=True, seed=2)
    a, b = both(q, k, v, is_causal=True, **kw, **extra)
    assert same(a, b)


def test_extension_non_contiguous_and_v1():
    from kernels.attention import flash_attention_v1
    case = make_case(2, 4, 4, 64, "self", torch.bfloat16, "dense", 7100,
                     dense_q_range=(200, 200))
    q, k, v, kw = pack(case, "dense", device=DEV)
    qt = q.transpose(1, 2).contiguous().transpose(1, 2)  # heads-inner strides
    a, b = both(qt, k, v, is_causal=True, **kw)
    assert same(a, b)
    import kernels.attention as A
    x = flash_attention_v1(q.float(), k.float(), v.float(), is_causal=True)
    A.USE_EXT = False
    try:
        y = flash_attention_v1(q.float(), k.float(), v.float(), is_causal=True)
    finally:
        A.USE_EXT = True
    torch.cuda.synchronize()
    assert same(x.cpu(), y.cpu())
