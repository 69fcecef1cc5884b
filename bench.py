"""Throughput of the MI355X flash_attention_v2 on the BASELINE.json configs.

Default: config c2 (dense causal GQA, B2 Hq32 Hkv8 L2048 D128, bf16), the
configuration BASELINE.json's metric is quoted on.  A "step" is one
``flash_attention_v2`` call over the whole batch with inputs already
resident in HBM.  Prints ONE JSON line (rank 0, N=1):

  value       algorithmic TFLOP/s of the whole step (host wall clock over K
              back-to-back steps, bracketed by torch.cuda.synchronize());
  roofline    achieved TFLOP/s per launch: the K back-to-back steps run in
              --windows windows with one pair of HIP events each on the
              stream the kernels run on; `achieved` uses the median of the
              windows' mean step times; against the dense bf16/fp16 MFMA peak
              (256 CU x 4096 FLOP/clk x 2.4 GHz); `traffic` = HBM bytes per
              launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
              summary of the same workload (profiles/hbm_traffic.json), null
              if there is none;
  cpu_baseline  the reference test suite's oracle (fp32 SDPA per sequence,
              oracle.sdpa_reference) on the host CPU, on a bounded sample.

  python bench.py [--steps K] [--warmup W] [--config c2] [--dtype bf16]
                  [--no-cpu] [--flush] [--windows 5]
  python bench.py --sweep [--sweep-out FILE] [--sweep-only TERMS]   # the
                  reference benchmark's shapes (benchmarks/attention.py), one
                  table row per point
  python bench.py --config c1 --host-cost 2000   # host us per call
  python bench.py --config c1 --graph 200        # HIP-graph replays vs eager

``--gpus N`` with N > 1 exits: this build measures one GPU.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "triton-kernels_amd"))

import workloads as W  # noqa: E402

PEAK_TFLOPS = 256 * 4096 * 2.4e9 / 1e12  # 2516.6 dense bf16/fp16 MFMA
PEAK_HBM_GBS = 8000.0
METRIC = "TFLOP/s + % of bf16 MFMA peak, flash_attention_v2 causal GQA seq2048 d128"
DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "f16": torch.float16,
          "fp32": torch.float32, "f32": torch.float32}
DTYPE_NAME = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}
METRIC_HBM = "GB/s of HBM (algorithmic bytes), {kind} {config}"
DESCR = {
    "d1": "d1 paged decode B16 QH8 KVH8 N8192 D64 page16",
    "d2": "d2 paged decode 64 seqs ctx~U[512,8192] page16 Hq32 Hkv8 D128",
    "s1": "s1 paged speculative decode causal M8 B16 QH8 KVH8 N8192+8 D64 page16",
    "s2": "s2 paged speculative decode causal M8 64 seqs ctx~U[512,8192]+8 page16 Hq32 Hkv8 D128",
    "a1": "a1 paged_kv_append of c4's context (140567 rows x Hkv8 x D128) into shuffled pools",
    "c1": "c1 dense causal MHA B1 H8 L512 D64",
    "c2": "c2 dense causal GQA B2 Hq32 Hkv8 L2048 D128",
    "c3": "c3 ragged causal self 16 seqs L~U[128,4096] Hq32 Hkv8 D128",
    "c4": "c4 paged chunked prefill 32 seqs ctx~U[512,8192] page16 q=last128 Hq32 Hkv8 D128",
    "c5": "c5 non-causal MQA cross B4 Hq32 Hkv1 q1024 kv16384 D128",
}


def cpu_baseline(w: W.Workload, budget_s: float = 20.0):
    """fp32 SDPA per sequence on host cores (oracle.sdpa_reference, i.e. the
    reference suite's oracle, tests/test_attention.py:80-98), 1 warmup + 3
    timed reps, median; sample = as many whole (sequence, kv-head group)
    units as fit the budget."""
    import oracle

    affinity = len(os.sched_getaffinity(0))
    cores = cpu_threads()
    torch.set_num_threads(cores)
    qs, ks, vs = W.sequences(w)
    g = w.q_heads // w.kv_heads
    units = [(b, kh) for b in range(len(qs)) for kh in range(w.kv_heads)]

    def unit_call(b, kh):
        q = qs[b][:, kh * g:(kh + 1) * g]
        k = ks[b][:, kh:kh + 1]
        v = vs[b][:, kh:kh + 1]
        if w.is_causal and w.causal_alignment == "bottom_right":
            return oracle.sdpa_reference_bottom_right([q], [k], [v], g, 1)
        return oracle.sdpa_reference([q], [k], [v], g, 1, w.is_causal)

    def unit_flops(b):
        return 4.0 * w.head_dim * g * W.visible_pairs(w.q_lens[b], w.kv_lens[b], w.is_causal,
                                                       w.causal_alignment)

    es = torch.tensor([], dtype=w.dtype).element_size()

    def unit_bytes(b):  # q, o of the group's heads; k, v of one kv head
        return es * w.head_dim * (2 * w.q_lens[b] * g + 2 * w.kv_lens[b])

    # time one unit to size the sample
    t0 = time.perf_counter()
    unit_call(*units[0])
    one = max(time.perf_counter() - t0, 1e-4)
    n = max(1, min(len(units), int(budget_s / 4 / one)))
    step = max(1, len(units) // n)
    sample = units[::step][:n]
    fl = sum(unit_flops(b) for b, _ in sample)
    nb = sum(unit_bytes(b) for b, _ in sample)
    for b, kh in sample[:1]:
        unit_call(b, kh)  # warmup
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        for b, kh in sample:
            unit_call(b, kh)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[1]
    if w.kind != "prefill":
        value, unit, amount = nb / med / 1e9, "GB/s", f"{nb / 1e6:.1f} MB"
    else:
        value, unit, amount = fl / med / 1e12, "TFLOP/s", f"{fl / 1e9:.1f} GFLOP"
    return {
        "value": round(value, 4),
        "unit": unit,
        "cores": cores,
        "kind": "port",
        "sample": f"{len(sample)} of {len(units)} (sequence, kv-head group) units of "
                  f"{w.name}, fp32 SDPA per sequence with repeat_interleaved KV heads, "
                  f"{amount} per rep, median of 3; {cores} threads of the "
                  f"{affinity} cores in this process's affinity mask",
    }


def cpu_threads() -> int:
    """Threads for the CPU baseline: every core of the affinity mask, capped by
    the host's CPU share for this job when the environment states one
    (OMP_NUM_THREADS; the GPU boxes give one GPU's job 16 cores)."""
    n = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS", "")
    if share.isdigit() and int(share) > 0:
        n = min(n, int(share))
    return n


def time_steps(step, steps: int, windows: int, stream):
    """Run `steps` back-to-back steps in `windows` windows, one HIP event pair
    per window on `stream`; returns (wall seconds, per-window mean ms)."""
    windows = max(1, min(windows, steps))
    sizes = [steps // windows + (1 if i < steps % windows else 0) for i in range(windows)]
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in sizes]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for (a, b), n in zip(ev, sizes):
        a.record(stream)
        for _ in range(n):
            step()
        b.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, [a.elapsed_time(b) / n for (a, b), n in zip(ev, sizes)]


def median(xs):
    xs = sorted(xs)
    m = len(xs) // 2
    return xs[m] if len(xs) % 2 else 0.5 * (xs[m - 1] + xs[m])


def sweep(args) -> int:
    """Time flash_attention_v2 (and v1) on every point of the reference
    benchmark's sweep (workloads.sweep_points): one table row per point on
    stdout, JSON lines to --sweep-out."""
    from kernels.attention import flash_attention_v1, flash_attention_v2

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    out = open(args.sweep_out, "w") if args.sweep_out else None
    print(f"{'layout':8}{'type':7}{'topo':6}{'mask':8}{'dtype':10}{'Q':>6}{'KV':>6}"
          f"{'v2 us':>10}{'v2 TFLOP/s':>12}{'v1 us':>10}", flush=True)
    terms = [t for t in (args.sweep_only or "").split(",") if t]
    for pt in W.sweep_points():
        layout, attn, topo, dt, causal, ql, kl = pt
        desc = {layout, attn, topo, DTYPE_NAME[dt], "causal" if causal else "full",
                f"q{ql}", f"kv{ql if attn == 'self' else kl}"}
        if any(t not in desc for t in terms):
            continue
        w = W.make_sweep(*pt).to(dev)
        kw = w.kwargs()
        res = {}
        for name, fn in (("v2", flash_attention_v2), ("v1", flash_attention_v1)):
            def step():
                return fn(w.q, w.k, w.v, **kw)
            for _ in range(args.warmup):
                step()
            _, win = time_steps(step, args.steps, args.windows, stream)
            res[name] = median(win)
        fl = W.flops(w)
        layout, attn, topo, dt, causal, ql, kl = pt
        tf = fl / (res["v2"] * 1e-3) / 1e12
        print(f"{layout:8}{attn:7}{topo:6}{'causal' if causal else 'full':8}"
              f"{DTYPE_NAME[dt]:10}{ql:>6}{w.kv_lens[0]:>6}{res['v2'] * 1e3:>10.1f}{tf:>12.1f}"
              f"{res['v1'] * 1e3:>10.1f}", flush=True)
        if out:
            out.write(json.dumps({"layout": layout, "attn": attn, "topology": topo,
                                  "dtype": DTYPE_NAME[dt], "causal": causal, "q_len": ql,
                                  "kv_len": w.kv_lens[0], "batch": W.SWEEP_BATCH,
                                  "head_dim": W.SWEEP_D, "gflop": round(fl / 1e9, 4),
                                  "v2_ms": round(res["v2"], 5), "v1_ms": round(res["v1"], 5),
                                  "v2_tflops": round(tf, 2)}) + "\n")
        del w
    if out:
        out.close()
    return 0


def host_cost(args, w, step, stream) -> int:
    """Host microseconds per call of N back-to-back calls (the time the
    Python wrapper and the launch take before the loop can issue the next
    call; the GPU keeps running the queued kernels), through the launch
    extension and through the ctypes path of flash_attention_v2 (the same
    entry point and parameter block), with the GPU time per call of each."""
    from kernels import attention

    n = args.host_cost
    res = {}
    paths = [("extension", True), ("ctypes", False)] if w.kind == "prefill" else [("ctypes", None)]
    for name, use_ext in paths:
        prev = attention.USE_EXT
        if use_ext is not None:
            attention.USE_EXT = use_ext
        try:
            for _ in range(args.warmup):
                step()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            t0 = time.perf_counter()
            for _ in range(n):
                step()
            t1 = time.perf_counter()
            b.record(stream)
            torch.cuda.synchronize()
        finally:
            attention.USE_EXT = prev
        res[name] = {"host_us_per_call": round((t1 - t0) * 1e6 / n, 2),
                     "gpu_us_per_call": round(a.elapsed_time(b) * 1e3 / n, 2)}
    print(json.dumps({"mode": "host_cost", "config": DESCR[args.config],
                      "dtype": DTYPE_NAME[w.dtype], "calls": n, "paths": res}))
    return 0


def graph_replay(args, w, step, stream) -> int:
    """GPU microseconds per call of N replays of one captured step (HIP graph:
    no host cost per call) and of N eager back-to-back calls, one event pair
    around each run; replays are checked against an eager call bit for bit."""
    n = args.graph
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    stream.wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = step()

    def run(fn):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(n):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / n

    run(g.replay)
    replay_us = run(g.replay)
    eager_us = run(step)
    same = bool(torch.equal(out, step()))
    print(json.dumps({"mode": "graph_replay", "config": DESCR[args.config],
                      "dtype": DTYPE_NAME[w.dtype], "calls": n,
                      "graph_us_per_call": round(replay_us, 2),
                      "eager_us_per_call": round(eager_us, 2),
                      "replay_equals_eager": same}))
    return 0 if same else 1


def hbm_traffic(config: str, dtype: str):
    """HBM bytes per launch of the workload's forward kernel, from the
    committed counter summary (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE,
    KiB per dispatch, each scaled by the factor the same counter shows for a
    plain device copy of known size); None when not profiled."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            table = json.load(f)
    except (OSError, ValueError):
        return None
    e = table.get("workloads", {}).get(f"{config}_{dtype}")
    if not e:
        return None
    sc = table["copy_calibration"]
    return int(round((e["fetch_kib"] * sc["fetch_scale"] + e["write_kib"] * sc["write_scale"])
                     * 1024))


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2", choices=W.CONFIGS)
    ap.add_argument("--dtype", default=None, choices=sorted(DTYPES))
    ap.add_argument("--alignment", default=None, choices=["top_left", "bottom_right"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--flush", action="store_true",
                    help="write 512 MiB between steps (outside the events) to flush L2/MALL")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--windows", type=int, default=5,
                    help="event-pair windows over the timed steps (median of their means)")
    ap.add_argument("--pool-gib", type=float, default=0.0,
                    help="paged configs: move the pages into K and V pools of at least this "
                         "many GiB each (pages near the top, past 2 GiB from 3.2 GiB on for c4); "
                         "the output is checked "
                         "bitwise against the compact pool's")
    ap.add_argument("--sweep", action="store_true",
                    help="time the reference benchmark's sweep of shapes instead")
    ap.add_argument("--sweep-out", default=None, help="JSON lines of the sweep")
    ap.add_argument("--sweep-only", default=None, metavar="TERMS",
                    help="comma-separated terms (e.g. 'ragged,bf16,q128,kv128'): run only the "
                         "sweep points whose description holds every term")
    ap.add_argument("--kernel", default="auto", choices=["auto", "regular", "short"],
                    help="prefill configs: flash_attention_v2's kernel choice (fa2_params.kernel)")
    ap.add_argument("--host-cost", type=int, default=0, metavar="N",
                    help="only time the host side of N back-to-back calls of the config's "
                         "step (launch extension and ctypes paths), with their GPU time")
    ap.add_argument("--graph", type=int, default=0, metavar="N",
                    help="only time N replays of one captured step (HIP graph) against N "
                         "eager calls, GPU time per call")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (5 times) to calibrate "
                         "the FETCH_SIZE / WRITE_SIZE counters against known bytes")
    ap.add_argument("--gemm-calibration", type=int, default=0, metavar="N",
                    help="only time torch.matmul (hipBLASLt) bf16 N x N x N, --warmup + --steps "
                         "back-to-back: the MFMA rate a library GEMM sustains on this GPU")
    args = ap.parse_args(argv)

    if args.gemm_calibration:
        n = args.gemm_calibration
        g = torch.Generator(device="cuda:0").manual_seed(0)
        a = torch.randn((n, n), device="cuda:0", generator=g).to(torch.bfloat16)
        b = torch.randn((n, n), device="cuda:0", generator=g).to(torch.bfloat16)
        c = torch.empty((n, n), device="cuda:0", dtype=torch.bfloat16)
        for _ in range(args.warmup):
            torch.matmul(a, b, out=c)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            torch.matmul(a, b, out=c)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        tf = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
        print(json.dumps({"gemm_calibration": f"bf16 {n}x{n}x{n} torch.matmul",
                          "steps": args.steps, "warmup": args.warmup, "ms_per_gemm": round(ms, 5),
                          "tflops": round(tf, 1), "frac_of_peak": round(tf / PEAK_TFLOPS, 4)}),
              flush=True)
        return 0

    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "copies": 5}), flush=True)
        return 0

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the flash_attention_v2 hot path has no "
              "multi-GPU component in this build (it would shard by (sequence, kv head) "
              "with no communication, or over the keys with one log-sum-exp merge of "
              "the per-row partials)", file=sys.stderr)
        return 2

    from kernels import _fa2, decode_attention, speculative_decode_attention
    from kernels.attention import flash_attention_v2

    _fa2.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.sweep:
        return sweep(args)
    dt = DTYPES[args.dtype] if args.dtype else None
    w_cpu = W.make(args.config, dtype=dt, causal_alignment=args.alignment)
    pool_check = None
    if args.pool_gib > 0:
        if w_cpu.layout != "paged":
            print("bench.py: --pool-gib applies to paged configs only", file=sys.stderr)
            return 2
        compact = w_cpu.to(dev)
        fn0 = {"prefill": flash_attention_v2, "decode": decode_attention,
               "speculative": speculative_decode_attention}[compact.kind]
        ref_out = fn0(compact.q, compact.k, compact.v, **compact.kwargs()).cpu()
        del compact
        torch.cuda.empty_cache()
        w_cpu = W.spread_pool(w_cpu, args.pool_gib)
    w = w_cpu.to(dev)
    kw = w.kwargs()
    if args.kernel != "auto":
        if w.kind != "prefill":
            print("bench.py: --kernel applies to prefill configs only", file=sys.stderr)
            return 2
        kw["kernel"] = args.kernel
    fl = W.flops(w)
    nbytes = W.hbm_bytes(w)
    flush_buf = torch.empty(512 << 20, dtype=torch.uint8, device=dev) if args.flush else None

    if w.kind == "append":
        from kernels.paged_cache import paged_kv_append as fn

        def step():
            return fn(w.k, w.v, w.k_block_table, w.v_block_table, w.k_new, w.v_new,
                      w.new_indptr, w.kv_page_size)
    else:
        fn = {"prefill": flash_attention_v2, "decode": decode_attention,
              "speculative": speculative_decode_attention}[w.kind]

        def step():
            return fn(w.q, w.k, w.v, **kw)

    if args.pool_gib > 0:
        out = step()
        torch.cuda.synchronize()
        pool_check = {"pool_gib_each": round(w.k.numel() * w.k.element_size() / 2**30, 3),
                      "pages_past_2gib": int(((w.k_block_table.long() * w.kv_page_size *
                                               w.k[0].numel() * w.k.element_size())
                                              >= 2**31).sum().item()),
                      "output_equals_compact_pool": bool(torch.equal(out.cpu(), ref_out))}
        del out
    print(f"bench: {DESCR[args.config]} {DTYPE_NAME[w.dtype]} warmup={args.warmup} "
          f"steps={args.steps}", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)
    if args.host_cost:
        return host_cost(args, w, step, stream)
    if args.graph:
        return graph_replay(args, w, step, stream)
    if flush_buf is None:
        # back-to-back steps; one event pair per window on the kernels' stream
        wall, win = time_steps(step, args.steps, args.windows, stream)
        kern_avg = median(win)
        kern_mean = sum(win) / len(win)
        ms_per_step = wall * 1e3 / args.steps
    else:
        # cold caches: a flush between steps, each step between its own events
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)]
        torch.cuda.synchronize()
        for i in range(args.steps):
            flush_buf.fill_(i & 0xFF)
            ev[i][0].record(stream)
            step()
            ev[i][1].record(stream)
        torch.cuda.synchronize()
        per = [a.elapsed_time(b) for a, b in ev]
        kern_avg = median(per)
        kern_mean = sum(per) / len(per)
        win = per
        ms_per_step = kern_mean  # wall clock would include the flush writes
    bound = "mfma" if fl / nbytes > (PEAK_TFLOPS * 1e12) / (PEAK_HBM_GBS * 1e9) else "hbm"
    if bound == "mfma":
        metric, unit, peak, work = METRIC, "TFLOP/s", PEAK_TFLOPS, fl / 1e12
    else:
        metric = METRIC_HBM.format(kind=fn.__name__, config=args.config)
        unit, peak, work = "GB/s", PEAK_HBM_GBS, nbytes / 1e9
    value = work / (ms_per_step * 1e-3)
    achieved = work / (kern_avg * 1e-3)

    line = {
        "metric": metric,
        "value": round(value, 2),
        "unit": unit,
        "pct_of_peak": round(100.0 * value / peak, 2),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_NAME[w.dtype],
        "data": "synthetic (seeded randn, CPU generator, seed 0)",
        "config": {
            "workload": DESCR[args.config],
            "layout": w.layout,
            "causal": w.is_causal,
            "causal_alignment": w.causal_alignment if w.is_causal else None,
            "gflop_per_step": round(fl / 1e9, 3),
            "algorithmic_mb_per_step": round(nbytes / 1e6, 2),
            "l2_mall_flushed": bool(args.flush),
            **({"large_pool": pool_check} if pool_check else {}),
            **({"kernel": args.kernel} if args.kernel != "auto" else {}),
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": bound,
            "achieved": round(achieved, 2),
            "peak": round(peak, 1),
            "unit": unit,
            "frac": round(achieved / peak, 4),
            "traffic": hbm_traffic(args.config, DTYPE_NAME[w.dtype]),
            "kernel_ms_median": round(kern_avg, 5),
            "kernel_ms_mean": round(kern_mean, 5),
            "timing": (f"median of {len(win)} event-pair windows over {args.steps} "
                       "back-to-back steps" if flush_buf is None else
                       f"median of {len(win)} per-step event pairs, caches flushed between "
                       "steps") + "; shader clock not pinned (short runs boost higher)",
            "hbm_gbs_algorithmic": round(nbytes / (kern_avg * 1e-3) / 1e9, 1),
            "tflops_algorithmic": round(fl / (kern_avg * 1e-3) / 1e12, 2),
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu and w.kind != "append":
        print("bench: timing the CPU baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(w_cpu, args.cpu_budget)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
