#!/usr/bin/env python3
"""Benchmark of the MI355X fp8 block-scale MoE operator (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload decode_t16]

A step is one call of the operator (routing -> permutation -> GEMM1+SwiGLU ->
GEMM2 -> combine) on one batch of synthetic tokens, all inputs resident in HBM.
Each timed step starts cold: a 768 MiB buffer is *read* before it (outside the
timed interval), which evicts the 256 MB Infinity Cache with clean lines.  (A
write flush would leave ~256 MB of dirty lines whose write-back the timed call
would pay for.)  Per-step device time comes from two HIP events recorded around
the C-ABI call.  A second pass records one event between consecutive kernels
(the library's ``stage_events`` argument): every kernel's device time, live, on
the stream it runs on; its sum is slightly above the per-step time because the
extra event packets sit between the kernels.  A third pass times the drop-in
``moe_fp8.run(...)`` itself (argument checks, output and workspace allocation,
ctypes) the way the reference's harness times a solution (flush, event, call,
event, back to back): ``run_us_per_call``; ``run_host_us_per_call`` is the host
time of one call.  A fourth pass replays the call captured in a HIP graph, cold like the
others (``graph_us_per_call``), as a serving loop that captures its decode step runs it.

Prints ONE JSON line.  Headline: T=16 decode (H=7168, I=2048, 32 local experts),
in us/call; the T=8192 large-prefill line and the other synthetic workloads
are reported inside the same object.  ``cpu_baseline`` times the CPU oracle
(fp32 torch, all local experts dequantised up front like the contest reference)
on the host cores: one warmup call and five timed calls of the headline workload,
median with min / max, on the affine cores (capped at OMP_NUM_THREADS when set).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "rocm-flashinfer-contest_amd"))

HBM_PEAK = 8.0e12          # B/s, MI355X HBM3E
FP8_PEAK = 5.0e15          # dense fp8 MFMA FLOP/s, MI355X
FLUSH_BYTES = 768 << 20


class StageEvents:
    """HIP events owned by torch (same HIP runtime as the library); their raw
    hipEvent_t handles are passed to the library, which records them between kernels."""

    def __init__(self, n):
        import torch
        self.events = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
        for e in self.events:
            e.record()                      # materialise the underlying hipEvent_t
        torch.cuda.synchronize()
        self.arr = (ctypes.c_void_p * n)(*[e.cuda_event for e in self.events])

    def ptr(self, first):
        return ctypes.addressof(self.arr) + first * ctypes.sizeof(ctypes.c_void_p)

    def ms(self, a, b):
        return float(self.events[a].elapsed_time(self.events[b]))


def work_counts(expert_offsets, T, H, I):
    """Algorithmic HBM bytes and fp8 flops of one call from the routing counts (A active local
    experts, P local pairs): every active expert's weights and block scales read once, every
    token's logits, hidden row and scales read once and its bf16 output row written once.  Per
    GEMM launch the same accounting: GEMM1 reads W13 (+ scales) of the active experts and the
    hidden rows; GEMM2 reads W2 (+ scales).  The intermediates between the kernels (C, the
    per-pair output rows) are not algorithmic bytes; what the kernels really move is the
    ``traffic`` figure."""
    counts = [int(expert_offsets[i + 1] - expert_offsets[i]) for i in range(len(expert_offsets) - 1)]
    A = sum(1 for c in counts if c > 0)
    P = sum(counts)
    w13 = 2 * I * H + (2 * I // 128) * (H // 128) * 4
    w2 = H * I + (H // 128) * (I // 128) * 4
    hidden = H + (H // 128) * 4
    per_token = hidden + 256 * 4 + H * 2
    return dict(active_experts=A, pairs=P, bytes=A * (w13 + w2) + T * per_token + 512,
                flops=P * (2 * H * 2 * I + 2 * I * H),
                gemm1_bytes=A * w13 + T * hidden, gemm1_flops=P * 2 * H * 2 * I,
                gemm2_bytes=A * w2, gemm2_flops=P * 2 * I * H)


def measure(wl, weights, steps, warmup, flush):
    import torch
    from moe_fp8 import workloads as W
    from moe_fp8._abi import NUM_STAGE_EVENTS, STAGES
    from moe_fp8.main import Runner

    act = W.make_activations(wl, device="cuda")
    dbg = {}
    runner = Runner(*act, *weights, 0, W.RSF, debug=dbg)
    runner()
    torch.cuda.synchronize()
    eo = dbg["expert_offsets"].cpu().tolist()
    runner.args.topk_ids = runner.args.topk_weights = runner.args.expert_offsets = runner.args.permuted_tokens = None
    sink = torch.empty(1, dtype=torch.int64, device="cuda")
    flush64 = flush.view(torch.int64)

    def evict():
        torch.sum(flush64, dim=0, keepdim=True, out=sink)     # read-only flush: clean lines

    for _ in range(warmup):
        evict()
        runner()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        evict()
        starts[i].record()
        runner()
        ends[i].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_step = [starts[i].elapsed_time(ends[i]) * 1e3 for i in range(steps)]
    ev = StageEvents(steps * NUM_STAGE_EVENTS)
    for i in range(steps):
        evict()
        runner(stage_events=ev.ptr(i * NUM_STAGE_EVENTS))
    torch.cuda.synchronize()
    stages = {s: [] for s in STAGES}
    for i in range(steps):
        b = i * NUM_STAGE_EVENTS
        for j, s in enumerate(STAGES):
            stages[s].append(ev.ms(b + j, b + j + 1) * 1e3)
    # a second column half (when the call runs one) counts towards its kernel's stage; otherwise
    # its two stages bracket nothing (event overhead only) and are dropped
    from moe_fp8 import _abi
    two_passes = _abi.load().moefp8_output_passes(wl.T, W.E_LOCAL_FULL, W.H_FULL, W.I_FULL, eo[-1]) == 2
    for s in ("gemm2", "combine"):
        extra = stages.pop(s + "_b")
        if two_passes:
            stages[s] = [x + y for x, y in zip(stages[s], extra)]
    # warm back-to-back (no flush), for reference
    torch.cuda.synchronize()
    e_a, e_b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e_a.record()
    for _ in range(steps):
        runner()
    e_b.record()
    torch.cuda.synchronize()
    warm_us = e_a.elapsed_time(e_b) * 1e3 / steps
    # the same call captured once in a HIP graph and replayed cold (flush, event, replay, event),
    # as a serving loop runs its decode step: the launches leave as one graph instead of one
    # stream packet each.  Reported beside the eager figure, which stays the per-call time.
    # A capture that the runtime refuses leaves the figure null instead of ending the bench.
    graph_us = None
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            runner()
        torch.cuda.synchronize()
    except RuntimeError as exc:
        print(f"[bench] {wl.name}: graph capture failed ({exc}); graph_us_per_call null", file=sys.stderr)
    else:
        gs = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
        ge = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
        for i in range(steps):
            evict()
            gs[i].record()
            graph.replay()
            ge[i].record()
        torch.cuda.synchronize()
        graph_us = statistics.median(gs[i].elapsed_time(ge[i]) * 1e3 for i in range(steps))
        del graph
    # the drop-in entry point itself, as the reference's harness times a solution's run()
    # (flush, event, run(...), event, back to back without host synchronisation; its argument
    # checks, output allocation and ctypes call overlap the flush still running on the device),
    # and separately the host time one run() call takes
    import moe_fp8
    run_args = (*act, *weights, 0, W.RSF)
    moe_fp8.run(*run_args)
    torch.cuda.synchronize()
    rs = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    re_ = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    host = []
    for i in range(steps):
        evict()
        rs[i].record()
        h0 = time.perf_counter()
        moe_fp8.run(*run_args)
        host.append((time.perf_counter() - h0) * 1e6)
        re_[i].record()
    torch.cuda.synchronize()
    run_us = statistics.median(rs[i].elapsed_time(re_[i]) * 1e3 for i in range(steps))
    run_host_us = statistics.median(host)
    T = wl.T
    H, I = W.H_FULL, W.I_FULL
    wk = work_counts(eo, T, H, I)
    us = statistics.median(per_step)
    st = {s: statistics.median(v) for s, v in stages.items()}
    res = dict(workload=wl.name, T=T, us_per_call=us, us_min=min(per_step), us_max=max(per_step),
               us_mean=statistics.fmean(per_step), warm_us_per_call=warm_us, host_wall_s=wall,
               run_us_per_call=run_us, run_host_us_per_call=run_host_us, graph_us_per_call=graph_us,
               stages_us=st, **wk)
    res["tflops"] = wk["flops"] / (us * 1e-6) / 1e12
    res["gbps"] = wk["bytes"] / (us * 1e-6) / 1e9
    res["hbm_frac"] = wk["bytes"] / (us * 1e-6) / HBM_PEAK
    res["mfma_frac"] = wk["flops"] / (us * 1e-6) / FP8_PEAK
    t_roof = max(wk["bytes"] / HBM_PEAK, wk["flops"] / FP8_PEAK)
    res["roofline_frac"] = t_roof / (us * 1e-6)
    # dominant kernel and its own roofline: bound by whichever of its algorithmic bytes at 8 TB/s
    # or its fp8 flops at 5 PFLOP/s takes longer
    dom = max(("gemm1", "gemm2"), key=lambda s: st[s])
    k_us = st[dom]
    k_bytes, k_flops = wk[f"{dom}_bytes"], wk[f"{dom}_flops"]
    hbm_bound = k_bytes / HBM_PEAK >= k_flops / FP8_PEAK
    if hbm_bound:
        ach = k_bytes / (k_us * 1e-6) / 1e9
        roof = dict(bound="hbm", achieved=ach, peak=HBM_PEAK / 1e9, unit="GB/s", frac=ach / (HBM_PEAK / 1e9))
    else:
        ach = k_flops / (k_us * 1e-6) / 1e12
        roof = dict(bound="mfma", achieved=ach, peak=FP8_PEAK / 1e12, unit="TFLOP/s", frac=ach / (FP8_PEAK / 1e12))
    kernel = STAGE_KERNELS[(dom, "decode" if T <= 64 else "large")]
    tr = traced_us(kernel, wl.name)
    roof.update(kernel=kernel, kernel_us=k_us, algorithmic_bytes=k_bytes, algorithmic_flops=k_flops,
                traffic=measured_traffic(kernel, wl.name), trace_us=tr,
                frac_at_trace_us=(roof["frac"] * k_us / tr) if tr else None)
    # both GEMM launches' fractions of their own bounds, from the event-bracketed stage times
    res["gemm_fracs"] = {g: dict(us=st[g], hbm_frac=wk[f"{g}_bytes"] / (st[g] * 1e-6) / HBM_PEAK,
                                 mfma_frac=wk[f"{g}_flops"] / (st[g] * 1e-6) / FP8_PEAK)
                         for g in ("gemm1", "gemm2") if st[g] > 0}
    res["roofline"] = roof
    del runner
    return res


# The library's kernel names per bench stage ("gemm1" / "gemm2"), by path: decode (T <= 64), and
# the 128-row grouped GEMMs of the large path.
STAGE_KERNELS = {("gemm1", "decode"): "gemm1_decode_kernel", ("gemm2", "decode"): "gemm2_decode_kernel",
                 ("gemm1", "large"): "gemm1_big_kernel", ("gemm2", "large"): "gemm2_big_kernel"}
PROFILES = ROOT / "profiles"


def _current_record(path, **match):
    """A profiles/ record line, only if it was taken with the current kernel sources."""
    from moe_fp8 import build
    from moe_fp8.profiling import read_record
    rec = read_record(path, **match)
    if rec is None or rec.get("source") != build.source_hash():
        return None
    return rec


def _r2(x):
    return None if x is None else round(x, 2)


def measured_traffic(kernel, workload):
    """HBM bytes per launch of the kernel on this workload, from the rocprofv3 FETCH_SIZE and
    WRITE_SIZE readings recorded in profiles/traffic_<kernel>_<workload>.txt, each divided by
    what the same counter reads per byte for a plain device copy (profiles/traffic_copy.txt);
    None when not recorded with the current kernel sources."""
    from moe_fp8.profiling import copy_calibration
    rec = _current_record(PROFILES / f"traffic_{kernel}_{workload}.txt", kernel=kernel)
    cal = PROFILES / "traffic_copy.txt"
    if rec is None or not cal.exists():
        return None
    fetch_per_byte, write_per_byte = copy_calibration(cal)
    return round(float(rec["fetch_kib"]) * 1024 / fetch_per_byte + float(rec["write_kib"]) * 1024 / write_per_byte)


def traced_us(kernel, workload):
    """The kernel's mean cold-call duration in the committed rocprofv3 kernel trace of this workload
    (profiles/moe_fp8_kernels_<workload>.md), if taken with the current kernel sources."""
    rec = _current_record(PROFILES / f"moe_fp8_kernels_{workload}.md", kernel=kernel)
    return float(rec["cold_us"]) if rec else None


def copy_calibration():
    """A plain 256 MiB device-to-device copy, three times: the reference kernel for scaling the
    FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import torch
    n = 256 << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"# copy calibration: {n} bytes per copy", file=sys.stderr)
    return 0


def cpu_baseline(wl, weights_cpu, threads, affinity, reps=5):
    """The CPU oracle on the host cores: one warmup call, then `reps` timed calls of the headline
    workload; value = median, with min / max.  `threads` = torch's intra-op threads used."""
    import torch
    sys.path.insert(0, str(ROOT / "oracle"))
    import moe_oracle
    from moe_fp8 import workloads as W

    torch.set_num_threads(threads)
    act = W.make_activations(wl, device="cpu")
    moe_oracle.moe_forward(*act, *weights_cpu, 0, W.RSF, dequant_all_upfront=True)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        moe_oracle.moe_forward(*act, *weights_cpu, 0, W.RSF, dequant_all_upfront=True)
        times.append((time.perf_counter() - t0) * 1e6)
    return dict(value=statistics.median(times), unit="us/call", cores=threads, kind="port",
                median=statistics.median(times), min=min(times), max=max(times), reps=reps, warmup=1,
                affinity_cores=affinity,
                sample=f"{reps} calls of {wl.name} (T={wl.T}, H=7168, I=2048, 32 local experts) after 1 warmup call: "
                       f"fp32 torch-CPU oracle, all 32 experts dequantised up front as in the contest reference "
                       f"(~11 GB of fp32 weights); {threads} intra-op threads of {affinity} affine cores")


def measure_quantize(T, steps, flush, H=7168):
    """Per-token 1x128 quantization of bf16 activations [T, H] (moe_fp8.quantize_hidden), cold
    cache per call: bytes = T*H*2 read + T*H + T*H/128*4 written."""
    import torch
    import moe_fp8
    g = torch.Generator(device="cuda").manual_seed(T)
    x = torch.randn(T, H, generator=g, device="cuda").to(torch.bfloat16)
    sink = torch.empty(1, dtype=torch.int64, device="cuda")
    flush64 = flush.view(torch.int64)
    for _ in range(3):
        moe_fp8.quantize_hidden(x)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    for i in range(steps):
        torch.sum(flush64, dim=0, keepdim=True, out=sink)
        starts[i].record()
        moe_fp8.quantize_hidden(x)
        ends[i].record()
    torch.cuda.synchronize()
    us = sorted(starts[i].elapsed_time(ends[i]) * 1e3 for i in range(steps))[steps // 2]
    nbytes = T * H * 2 + T * H + T * (H // 128) * 4
    return {"T": T, "us_per_call": round(us, 2), "bytes": nbytes, "gbps": round(nbytes / us / 1e3, 1),
            "hbm_frac": round(nbytes / us / 1e3 / 8000.0, 4)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="decode_t16")
    ap.add_argument("--secondary", default="large_t8192")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 256 MiB device copy (counter calibration under rocprofv3)")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the operator runs all 32 local experts of one expert-parallel rank on a "
              f"single MI355X; --gpus {args.gpus} is not supported", file=sys.stderr)
        return 2

    import torch
    from moe_fp8 import workloads as W

    torch.cuda.set_device(0)
    wls = W.workloads()
    weights = W.make_weights(device="cuda")
    flush = torch.ones(FLUSH_BYTES, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    head = measure(wls[args.workload], weights, args.steps, args.warmup, flush)
    print(f"# {args.workload}: {head['us_per_call']:.1f} us/call", file=sys.stderr, flush=True)
    sweep = {}
    if not args.no_sweep:
        for name, wl in wls.items():
            if name == args.workload:
                continue
            r = measure(wl, weights, args.steps, args.warmup, flush)
            print(f"# {name}: {r['us_per_call']:.1f} us/call", file=sys.stderr, flush=True)
            sweep[name] = r
    sec = sweep.get(args.secondary)
    quant = None
    if not args.no_sweep:
        quant = {f"t{T}": measure_quantize(T, args.steps, flush) for T in (16, 8192)}
        print(f"# quantize_hidden: T=16 {quant['t16']['us_per_call']} us, T=8192 {quant['t8192']['us_per_call']} us "
              f"({quant['t8192']['hbm_frac']:.2f} of HBM)", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu_baseline:
        # the process's CPU share: the affine cores, capped at OMP_NUM_THREADS where the environment
        # sets it (16 per GPU on the measurement boxes, whatever the affinity mask shows)
        affinity = len(os.sched_getaffinity(0))
        cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
        threads = max(1, min(affinity, cap) if cap > 0 else affinity)
        weights_cpu = tuple(x.cpu() for x in weights)
        cpu = cpu_baseline(wls[args.workload], weights_cpu, threads, affinity)
        print(f"# cpu baseline: median {cpu['median']:.0f} us/call (min {cpu['min']:.0f}, max {cpu['max']:.0f}, "
              f"{cpu['reps']} reps) on {threads} threads of {affinity} affine cores", file=sys.stderr, flush=True)

    line = {
        "metric": f"moe_fp8 block-scale MoE latency, {args.workload} (T={head['T']}, H=7168, I=2048, 32 local experts)",
        "value": round(head["us_per_call"], 3),
        "unit": "us/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_mean"] / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3",
        "data": "synthetic",
        "config": {"workload": args.workload, "T": head["T"], "H": 7168, "I": 2048, "E_local": 32,
                   "top_k": 8, "n_group": 8, "topk_group": 4, "local_expert_offset": 0, "routed_scaling": 2.5,
                   "active_experts": head["active_experts"], "pairs": head["pairs"], "cold_cache": True},
        "tflops": round(head["tflops"], 3),
        "gbps": round(head["gbps"], 1),
        "hbm_frac": round(head["hbm_frac"], 4),
        "mfma_frac": round(head["mfma_frac"], 5),
        "roofline_frac": round(head["roofline_frac"], 4),
        "stages_us": {k: round(v, 2) for k, v in head["stages_us"].items()},
        "warm_us_per_call": round(head["warm_us_per_call"], 2),
        "run_us_per_call": round(head["run_us_per_call"], 2),
        "run_host_us_per_call": round(head["run_host_us_per_call"], 2),
        "graph_us_per_call": _r2(head["graph_us_per_call"]),
        "gemm_fracs": head["gemm_fracs"],
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
    }
    if sec is not None:
        line["t8192"] = {k: sec[k] for k in ("us_per_call", "tflops", "gbps", "hbm_frac", "mfma_frac", "roofline_frac",
                                           "active_experts", "pairs", "stages_us", "gemm_fracs", "roofline",
                                           "run_us_per_call", "run_host_us_per_call", "graph_us_per_call")}
    if quant is not None:
        line["quantize_hidden"] = quant
    if sweep:
        line["sweep"] = {k: {"us_per_call": round(v["us_per_call"], 2), "tflops": round(v["tflops"], 2),
                             "gbps": round(v["gbps"], 1), "roofline_frac": round(v["roofline_frac"], 4),
                             "hbm_frac": round(v["hbm_frac"], 4), "mfma_frac": round(v["mfma_frac"], 4),
                             "run_us_per_call": round(v["run_us_per_call"], 2),
                             "run_host_us_per_call": round(v["run_host_us_per_call"], 2),
                             "graph_us_per_call": _r2(v["graph_us_per_call"]),
                             "P": v["pairs"], "A": v["active_experts"],
                             "stages_us": {s: round(x, 1) for s, x in v["stages_us"].items()}}
                         for k, v in sweep.items()}
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
