"""The attention entry points under HIP graph capture (torch.cuda.CUDAGraph).

A serving loop captures the forward once and replays it: every launch of
the path must be capturable (kernel launches on the current stream, the
workspace from torch's caching allocator, no memset, no host sync), and each
replay must read the live inputs.  Each case captures one call, then
replays it several times with eager work and synchronisations in between,
refilling the inputs before some replays.  Every replay must equal an
eager call on the same inputs bit for bit.  The eager results themselves
are held to the reference tolerances by the other GPU tests.
"""

import pytest
import torch

from attn_cases import make_case, pack

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X")
    from kernels import _fa2
    _fa2.lib()
    yield


def _replay_matches(fn, inputs, refills):
    """Capture fn(*inputs), then for each refill (a list of tensors copied
    into the inputs, or None) replay and compare with an eager call."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        for _ in range(2):
            fn(*inputs)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn(*inputs)
    for i, refill in enumerate(refills):
        if refill is not None:
            for dst, src in zip(inputs, refill):
                dst.copy_(src)
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        # eager work between replays: the same call, and an unrelated kernel
        want = fn(*inputs)
        torch.randn(1 << 20, device=DEV).sum()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i} differs from the eager call"
        assert torch.isfinite(want).all()


def _perturbed(ts, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return [torch.randn(t.shape, generator=g, device=DEV).to(t.dtype) if t.is_floating_point()
            else t.clone() for t in ts]


@pytest.mark.parametrize("layout", ["dense", "ragged", "paged"])
@pytest.mark.parametrize("topology", [(8, 2), (8, 8)])
def test_flash_attention_v2_graph(layout, topology):
    from kernels import flash_attention_v2
    QH, KVH = topology
    case = make_case(3, QH, KVH, 128, "self", torch.bfloat16, layout, 9100 + QH + KVH,
                     q_range=(100, 700), dense_q_range=(500, 500))
    q, k, v, kw = pack(case, layout, device=DEV)
    print(f"graph v2 {layout} QH={QH} KVH={KVH}", flush=True)

    def fn(q, k, v):
        return flash_attention_v2(q, k, v, is_causal=True, **kw)

    _replay_matches(fn, [q, k, v], [None, _perturbed([q, k, v], 1), None, _perturbed([q, k, v], 2)])


def test_split_and_combine_graph():
    """Forced split: the forward kernel and the combine kernel in one graph."""
    from kernels import flash_attention_v2
    case = make_case(2, 8, 2, 128, "cross", torch.float16, "dense", 9200,
                     dense_q_range=(64, 64), dense_kv_range=(4000, 4000))
    q, k, v, kw = pack(case, "dense", device=DEV)
    print("graph split dense", flush=True)

    def fn(q, k, v):
        return flash_attention_v2(q, k, v, is_causal=False, num_splits=4, **kw)

    _replay_matches(fn, [q, k, v], [None, _perturbed([q, k, v], 3), None])


def test_v1_fp32_graph():
    from kernels import flash_attention_v1
    case = make_case(2, 8, 2, 64, "self", torch.float32, "paged", 9300, q_range=(50, 300))
    q, k, v, kw = pack(case, "paged", device=DEV)
    print("graph v1 fp32 paged", flush=True)

    def fn(q, k, v):
        return flash_attention_v1(q, k, v, is_causal=True, **kw)

    _replay_matches(fn, [q, k, v], [None, _perturbed([q, k, v], 4)])


@pytest.mark.parametrize("layout", ["dense", "ragged"])
def test_v2_fp32_graph(layout):
    """fp32 tensors of flash_attention_v2: the fp16 conversion, the 16-bit
    forward writing partials and the fp32 combine, in one graph."""
    from kernels import flash_attention_v2
    case = make_case(3, 8, 2, 128, "self", torch.float32, layout, 9350, q_range=(100, 700),
                     dense_q_range=(400, 400))
    q, k, v, kw = pack(case, layout, device=DEV)
    print(f"graph v2 fp32 {layout}", flush=True)

    def fn(q, k, v):
        return flash_attention_v2(q, k, v, is_causal=True, **kw)

    _replay_matches(fn, [q, k, v], [None, _perturbed([q, k, v], 6), None])


@pytest.mark.parametrize("spec", [False, True])
def test_decode_graph(spec):
    from kernels import decode_attention, speculative_decode_attention
    g = torch.Generator(device=DEV).manual_seed(9400 + int(spec))
    B, Hq, Hkv, D, L = 4, 16, 2, 128, 3000
    M = 4 if spec else 1
    q = torch.randn((B, Hq, M, D) if spec else (B, Hq, D), generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, Hkv, L, D, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(B, Hkv, L, D, generator=g, device=DEV).to(torch.bfloat16)
    print(f"graph decode spec={spec}", flush=True)

    def fn(q, k, v):
        if spec:
            return speculative_decode_attention(q, k, v, causal=True)
        return decode_attention(q, k, v)

    _replay_matches(fn, [q, k, v], [None, _perturbed([q, k, v], 5), None])
