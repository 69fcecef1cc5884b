"""Writes the golden fixtures tests/golden/*.npz.

Each fixture holds seeded inputs of one ``flash_attention_v2`` call (16-bit
tensors as their int16 bit patterns, index tensors as int32) and the
expected output from fp64 ``torch.nn.functional.scaled_dot_product_attention``
run per sequence with repeat_interleaved KV heads - the reference test
suite's oracle (tests/test_attention.py:80-98) at higher precision - plus a
``valid`` mask of the output rows that exist (dense/paged padding rows are
excluded).  Rows that see no key are NaN (the reference's 0/0).

The reference itself is not run: its kernels need a CUDA device and Triton.

Run from the repository root:  python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from attn_cases import make_case, pack  # noqa: E402

DT = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}

CASES = [
    # name, B, QH, KVH, D, attn, dtype, layout, causal, alignment, seed, extra
    ("dense_causal_gqa_f16_d64", 2, 4, 2, 64, "self", torch.float16, "dense", True, "top_left", 101, {}),
    ("dense_cross_mqa_bf16_d64", 2, 4, 1, 64, "cross", torch.bfloat16, "dense", False, "top_left", 102, {}),
    ("ragged_causal_gqa_bf16_d64", 3, 4, 2, 64, "self", torch.bfloat16, "ragged", True, "top_left", 103,
     dict(q_lens=[1, 64, 129], kv_lens=[1, 64, 129])),
    ("ragged_cross_mha_f32_d64", 2, 2, 2, 64, "cross", torch.float32, "ragged", False, "top_left", 104,
     dict(q_lens=[5, 70], kv_lens=[200, 3])),
    ("paged_causal_gqa_f16_d64_shuffled", 3, 4, 2, 64, "self", torch.float16, "paged", True, "top_left", 105,
     dict(q_lens=[17, 50, 65], kv_lens=[17, 50, 65])),
    ("paged_bottom_right_bf16_d64", 2, 4, 2, 64, "cross", torch.bfloat16, "paged", True, "bottom_right", 106,
     dict(q_lens=[16, 16], kv_lens=[40, 100])),
    ("dense_causal_mha_bf16_d128", 1, 2, 2, 128, "self", torch.bfloat16, "dense", True, "top_left", 107, {}),
    ("paged_cross_mqa_f16_d128_page8", 2, 4, 1, 128, "cross", torch.float16, "paged", False, "top_left", 108,
     dict(q_lens=[9, 30], kv_lens=[77, 5], page=8)),
]


def main():
    for (name, B, QH, KVH, D, attn, dt, layout, causal, align, seed, extra) in CASES:
        extra = dict(extra)
        page = extra.pop("page", 16)
        case = make_case(B, QH, KVH, D, attn, dt, layout, seed, dense_q_range=(20, 70),
                         dense_kv_range=(30, 90), **extra)
        q, k, v, kw = pack(case, layout, shuffled_pages=(layout == "paged"), seed=seed, page=page)
        if causal and align == "bottom_right":
            refs = oracle.sdpa_reference_bottom_right(case.qs, case.ks, case.vs, QH, KVH,
                                                      dtype=torch.float64)
        else:
            refs = oracle.sdpa_reference(case.qs, case.ks, case.vs, QH, KVH, causal,
                                         dtype=torch.float64)
        out = torch.zeros(q.shape, dtype=torch.float32)
        valid = torch.zeros(q.shape[:-1], dtype=torch.uint8)
        if layout == "ragged":
            ip = kw["q_indptr"]
            for b in range(B):
                out[int(ip[b]): int(ip[b + 1])] = refs[b].float()
                valid[int(ip[b]): int(ip[b + 1])] = 1
        else:
            for b in range(B):
                out[b, :, : case.q_lens[b]] = refs[b].float().transpose(0, 1)
                valid[b, :, : case.q_lens[b]] = 1

        def arr(t):
            return t.view(torch.int16).numpy() if t.dtype != torch.float32 else t.numpy()

        data = dict(q=arr(q), k=arr(k), v=arr(v), out=out.numpy(), valid=valid.numpy())
        for n in ("q_indptr", "kv_indptr", "k_block_table", "v_block_table"):
            if n in kw:
                data[n] = kw[n].numpy().astype(np.int32)
        data["meta_dtype"] = np.array(DT[dt])
        data["meta_causal"] = np.array(causal)
        data["meta_alignment"] = np.array(align)
        if layout == "paged":
            data["meta_page_size"] = np.array(page)
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **data)
        print(f"{path}: {os.path.getsize(path) / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
