#!/usr/bin/env python3
"""MatMulNBits INT4 on one MI355X: decode GEMV HBM GB/s at 7B shapes, prefill TFLOP/s.

A step is one pass of a 7B-class decoder layer's INT4 projections at M=1
(q, k, v, o, gate, up, down; hidden 3584, intermediate 18944, 28 query / 4 KV
heads of dim 128; block size 32 with packed zero points). Weights, activations
and outputs are resident in HBM before timing starts. Every step uses a
different copy of the layer's weights, activations and outputs, rotating over
enough copies to touch >= 1 GiB, so no op is served from the 256 MiB MALL.
The steps are enqueued eagerly on one stream, one C batch call per step
(--warmup untimed steps, then exactly --steps timed ones, after the per-launch
graph timings so that the GPU runs at its sustained clock) and timed with HIP
events on that stream; the same rotation replayed as a HIP graph is reported
beside it.

Prints one JSON line. value = algorithmic bytes per step / time per step
(weights + fp32 A + fp32 Y, each once). Beside it:
  roofline      the gate/up GEMV launch (K=3584, N=18944): bytes per launch /
                mean launch time, against 8 TB/s;
  prefill       M=2048 on the Llama-2-7B MLP shapes (the MFMA kernel), TFLOP/s
                against the 2.5 PFLOP/s dense fp16 peak;
  cpu_baseline  the CPU oracle (a C++-style C restatement of the reference's
                managed MatMulNBitsKernel) on the host's cores and on one thread,
                one bounded sample per workload; value = the 7B decode layer.
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import math
import statistics
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "MatMulNBits INT4 M=1 GEMV HBM GB/s at 7B shapes; M=2048 prefill TFLOP/s"
# Projections of the 7B decode layer that read the same input, by index into DECODE_7B;
# a batch call runs each group as one launch.
GROUPS = {"qkv": [0, 1, 2], "gate_up": [4, 5]}
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
# Untimed GPU time before each secondary measurement (per-op, grouped, prefill).
WARM_MS = 20.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Rotation:
    """R device-resident copies of a set of ops: weights handles, A and Y."""

    def __init__(self, ops, M, copies, seed, kind="normal", share=None):
        """share[i] = the op whose activation buffer op i reads (default: its own), as the
        projections of one input share it in a decoder layer."""
        import torch
        from modelsharp_amd import native, workloads
        self.ops, self.M, self.copies = ops, M, copies
        share = list(range(len(ops))) if share is None else share
        host = [workloads.make_weights(op, seed + i) for i, op in enumerate(ops)]
        self.handles = [[native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
                         for (b, s, z), op in zip(host, ops)] for _ in range(copies)]
        own = [{i: torch.from_numpy(workloads.make_activations(M, ops[i].K, seed + 100 * r + i, kind)).cuda()
                for i in set(share)} for r in range(copies)]
        self.A = [[own[r][share[i]] for i in range(len(ops))] for r in range(copies)]
        self.Y = [[torch.empty((M, op.N), dtype=torch.float32, device="cuda") for op in ops] for _ in range(copies)]
        self.host = host

    def enqueue(self, r, stream, only=None):
        """One batch call over copy r's ops (or the op index / list of indices `only`)."""
        from modelsharp_amd import native
        idx = range(len(self.ops)) if only is None else ([only] if isinstance(only, int) else list(only))
        native.gemm_dev_batch([self.handles[r][i] for i in idx], [self.A[r][i].data_ptr() for i in idx],
                              [self.Y[r][i].data_ptr() for i in idx], self.M, stream)

    def close(self):
        for row in self.handles:
            for h in row:
                h.close()


def graph_of(fn):
    """Captures fn(stream_handle) into a torch CUDA (HIP) graph."""
    import torch
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(side.cuda_stream)   # warm: first launches outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        fn(torch.cuda.current_stream().cuda_stream)
    return g


def time_graph(g, replays, warmup, warm_ms=WARM_MS):
    """Mean ms per replay, HIP events on the stream the graph is launched on. Untimed
    replays run first: `warmup` of them, and more until about `warm_ms` of GPU time has
    passed, since the first milliseconds of a burst of work run at lower clocks (a
    freshly captured M=2048 prefill graph measures 10-15% slow over its first 10
    replays)."""
    import torch
    for _ in range(warmup):
        g.replay()
    if warm_ms > 0:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        e1.synchronize()
        for _ in range(min(10000, math.ceil(warm_ms / max(e0.elapsed_time(e1), 1e-3)))):
            g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    end.synchronize()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / replays


TRAFFIC_PROFILE = "profiles/gemv_w4_gate_up_7b_hbm_traffic.json"


# The device sources of the roofline kernel (gemv_w4): a traffic profile is used only
# for the code it measured (its launch shape is checked separately).
GEMV_SOURCES = ("gemv_w4.h", "nbits_device.h")


def kernel_source_digest() -> str:
    """sha256 over the roofline kernel's device sources."""
    import hashlib
    h = hashlib.sha256()
    for name in GEMV_SOURCES:
        f = ROOT / "modelsharp_amd" / "csrc" / name
        h.update(name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def measured_traffic(launch):
    """HBM bytes per gate+up launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (scaled by a plain copy's counters), used only when that
    profile was taken on the same kernel sources and launch configuration."""
    path = ROOT / TRAFFIC_PROFILE
    if not path.is_file():
        return None
    prof = json.loads(path.read_text())
    same = prof.get("source_digest") == kernel_source_digest() and \
        all(prof.get(k) == launch.get(k) for k in ("kernel", "lanes_per_row", "grid", "block"))
    return prof["traffic_bytes"] if same else None


def cpu_description() -> dict:
    """CPU model and the SIMD extensions the restatement can use (from /proc/cpuinfo)."""
    model, flags = "unknown", set()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            elif line.startswith("flags") and not flags:
                flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    isa = [f for f in ("avx2", "fma", "f16c", "avx512f", "avx512bw", "avx512vl", "avx512_vnni", "avx512_bf16")
           if f in flags]
    return {"model": model, "isa": isa, "threads_available": os.cpu_count()}


def _median_call(fn, budget_s, reps=5):
    """Seconds per call of fn(): `reps` repetitions, each calling fn at least once and until
    budget_s / reps has passed; returns (median, min, max) of the repetitions' per-call times."""
    fn()   # warm
    per = []
    for _ in range(reps):
        calls, t0 = 0, time.perf_counter()
        while True:
            fn()
            calls += 1
            el = time.perf_counter() - t0
            if el >= budget_s / reps:
                break
        per.append(el / calls)
    return statistics.median(per), min(per), max(per)


def cpu_baseline(budget_s):
    """The oracle (kind "port": a C restatement of MatMulNBitsKernel.Execute's default
    path, column-parallel over N as MatMulParallel.For) on every workload, on all the
    host's cores and on one thread: each figure the median of 5 repetitions of a bounded
    sample (the budget shared over the figures)."""
    import oracle
    from modelsharp_amd import workloads
    nthreads = oracle.threads()
    nfig = 2 * (3 + len(workloads.LLAMA7B_SMALLM_M) + 3 * len(workloads.LLAMA7B_PREFILL_OPS))
    per = max(0.25, budget_s / nfig)

    def timed(fn):
        med, lo, hi = _median_call(fn, per)
        return {"ms_per_call": round(med * 1e3, 3), "ms_min": round(lo * 1e3, 3), "ms_max": round(hi * 1e3, 3)}

    def decode_set(name, ops, M, seed, bs_note):
        host = [workloads.make_weights(op, seed + i) for i, op in enumerate(ops)]
        acts = [workloads.make_activations(M, op.K, seed + 50 + i) for i, op in enumerate(ops)]
        nbytes = sum(workloads.algorithmic_bytes(op, M) for op in ops)

        def run(nt):
            for (b, s, z), a, op in zip(host, acts, ops):
                oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, op.block_size, nthreads=nt)
        row = {"workload": name, "sample": f"{'+'.join(op.name for op in ops)} at M={M}, {bs_note}",
               "bytes_per_call": nbytes}
        for nt, key in ((nthreads, "all_cores"), (1, "one_thread")):
            t = timed(lambda: run(nt))
            row[key] = {"threads": nt, **t, "GBs": round(nbytes / (t["ms_per_call"] * 1e-3) / 1e9, 3)}
        return row

    rows = []
    rows.append(decode_set("qwen05b_up", [workloads.QWEN05B_UP], 1, 100, "K=896 N=4864 bs=32 zp"))
    rows.append(decode_set("qwen05b_decode", workloads.QWEN05B_DECODE, 1, 200, "8 projections, bs=32 zp"))
    rows.append(decode_set("7b_decode", workloads.DECODE_7B, 1, 300, "7 projections, bs=32 zp"))
    for M in workloads.LLAMA7B_SMALLM_M:
        rows.append(decode_set(f"llama7b_smallm_M{M}", workloads.LLAMA7B_SMALLM_OPS, M, 400,
                               "bs=128, no zp"))
    # prefill: a sample of output columns (a full M=2048 call is ~10^2 s of CPU work); the
    # columns are independent, so GFLOP/s over a sample is the call's rate
    for i, op in enumerate(workloads.LLAMA7B_PREFILL_OPS):
        b, s, z = workloads.make_weights(op, 500 + i)
        for M in (128, 512, 2048):
            a = workloads.make_activations(M, op.K, 501 + i, kind="rmsnorm")
            prow = {"workload": f"llama7b_prefill_K{op.K}_N{op.N}_M{M}",
                    "sample": f"M={M} K={op.K} N={op.N}, bs=32 zp, output columns sampled"}
            for nt, key in ((nthreads, "all_cores"), (1, "one_thread")):
                cols = max(8, min(op.N, (128 if nt > 1 else 8) * 2048 // M))
                bc, sc = b[:cols], s.reshape(op.N, -1)[:cols]
                zc = None if z is None else z[:cols]
                t = timed(lambda: oracle.matmul_nbits(a, bc, sc, zc, cols, op.K, 4, 32, nthreads=nt))
                fl = 2.0 * M * cols * op.K
                prow[key] = {"threads": nt, "columns": cols, **t,
                             "GFLOPs": round(fl / (t["ms_per_call"] * 1e-3) / 1e9, 3)}
            rows.append(prow)

    head = next(r for r in rows if r["workload"] == "7b_decode")
    out = {"value": head["all_cores"]["GBs"], "unit": "GB/s", "cores": nthreads, "kind": "port",
           "sample": f"7B decode layer ({head['sample']}), {head['all_cores']['ms_per_call']} ms per layer on "
                     f"{nthreads} threads; C++-style restatement of the managed MatMulNBitsKernel (the reference's "
                     f"C# runtime is not available), column-parallel like MatMulParallel.For",
           "cpu": cpu_description(), "rows": rows}
    if oracle.ref_lib() is not None:
        # The reference's own native ms_qgemm_nbits (qgemm.cpp, built from its sources), on
        # the 7B gate projection, all threads (its OpenMP default).
        gate = next(o for o in workloads.DECODE_7B if o.name == "gate")
        b, s, z = workloads.make_weights(gate, 600)
        a = workloads.make_activations(1, gate.K, 601)
        med, _, _ = _median_call(lambda: oracle.ref_qgemm_nbits(a, b, s, z, 1, gate.N, gate.K, 4, 32), per)
        out["reference_native_gate_GBs"] = round(workloads.algorithmic_bytes(gate, 1) / med / 1e9, 3)
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed decode-layer steps")
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--rotate-mib", type=int, default=1024, help="bytes the weight rotation touches")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline budget (0 = skip)")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-layer", action="store_true", help="skip the device-resident decoder layer")
    ap.add_argument("--detail", default="", help="also write per-op results of every workload to this JSON file")
    ap.add_argument("--op", default="", help="profiling mode: launch only this 7B decode op (q,k,v,o,gate,up,down), "
                                             "a grouped launch (qkv, gate_up), prefill_up / prefill_down or the "
                                             "block-size-128 small-batch smallm_up / smallm_down (M from --m), "
                                             "eagerly over the rotation, then a plain copy of --copy-mib; or "
                                             "decoder_layer (--calls steps of the device-resident 7B layer) or "
                                             "attention_prefill (--calls launches); no JSON line")
    ap.add_argument("--calls", type=int, default=64, help="launches in --op mode")
    ap.add_argument("--m", type=int, default=2048, help="rows of A for prefill_* and smallm_* in --op mode")
    ap.add_argument("--copy-mib", type=int, default=256, help="size of the calibration copy in --op mode")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this MatMulNBits build measures one GPU; the op shards by columns or by "
                                   "K-blocks across GPUs (see the design notes), but no multi-GPU figure is "
                                   "produced", "n_gpus": args.gpus}), flush=True)
        return 2

    import torch
    from modelsharp_amd import native, workloads
    if not (ROOT / "modelsharp_amd" / "lib" / native.LIB_NAME).is_file():
        import __graft_entry__
        __graft_entry__.build()
    if not native.available():
        raise SystemExit("no gfx950 device: " + native.last_error())
    torch.cuda.set_device(0)
    log(f"device: {native.device_name()}")
    if args.op:
        return profile_op(args)

    # ---- 7B decode layer, M=1 -------------------------------------------------------------
    ops = workloads.DECODE_7B
    step_bytes = sum(workloads.algorithmic_bytes(op, 1) for op in ops)
    copies = workloads.rotation_copies(step_bytes, args.rotate_mib << 20)
    log(f"7b decode layer: {step_bytes / 1e6:.2f} MB/step, {copies} rotating copies")
    rot = Rotation(ops, 1, copies, seed=7, share=workloads.DECODE_7B_SHARE)

    def layer_rotation(stream):
        for r in range(copies):
            rot.enqueue(r, stream)

    # the same rotation replayed as a HIP graph
    g = graph_of(layer_rotation)
    replays = max(2, math.ceil(200 / copies))
    ms_step_graph = time_graph(g, replays, 2) / copies
    log(f"graph: {ms_step_graph * 1e3:.2f} us/step")

    # the same step with every op in a launch of its own (no grouping of shared inputs)
    gu = graph_of(lambda stream: [rot.enqueue(r, stream, only=i) for r in range(copies) for i in range(len(ops))])
    ms_step_ungrouped = time_graph(gu, replays, 2) / copies
    log(f"ungrouped: {ms_step_ungrouped * 1e3:.2f} us/step  {step_bytes / (ms_step_ungrouped * 1e-3) / 1e9:.1f} GB/s")
    del gu

    # per-op launch times (graph of one op over all copies)
    per_op = {}
    for i, op in enumerate(ops):
        gi = graph_of(lambda stream, i=i: [rot.enqueue(r, stream, only=i) for r in range(copies)])
        ms = time_graph(gi, max(4, 2 * replays), 2) / copies
        nbytes = workloads.algorithmic_bytes(op, 1)
        per_op[op.name] = {"K": op.K, "N": op.N, "us": round(ms * 1e3, 3),
                           "GBs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                           "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                           "kernel": rot.handles[0][i].launch_info(1)}
        log(f"  {op.name:5s} K={op.K:6d} N={op.N:6d}: {ms * 1e3:7.2f} us  {per_op[op.name]['GBs']:7.1f} GB/s")
    # grouped launches as the step runs them (projections of one input in one launch)
    groups = {}
    for gname, idx in GROUPS.items():
        gg = graph_of(lambda stream, idx=idx: [rot.enqueue(r, stream, only=idx) for r in range(copies)])
        ms = time_graph(gg, max(4, 2 * replays), 2) / copies
        nbytes = workloads.algorithmic_bytes_group([ops[i] for i in idx], 1)
        info = native.batch_launch_info([rot.handles[0][i] for i in idx], [rot.A[0][i].data_ptr() for i in idx], 1)
        groups[gname] = {"ops": [ops[i].name for i in idx], "us": round(ms * 1e3, 3),
                         "bytes": nbytes, "GBs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                         "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "kernel": info}
        log(f"  {gname:8s} one launch ({info['calls']} ops): {ms * 1e3:7.2f} us  {groups[gname]['GBs']:7.1f} GB/s")
        del gg
    # The headline, after the graph timings above (so the step runs at the clock a
    # sustained decode loop runs at: a cold burst of 20 steps measured 45.2-47.3 us per step
    # whether issued eagerly or as one pre-instantiated graph of the 20 steps, against
    # 44.3 us for 200 steps either way): exactly --warmup untimed steps, then exactly
    # --steps timed steps, each step one batch call (one C call, 4 launches) over the next
    # copy of the rotation, on one stream; HIP events on that stream around the timed
    # steps, device synchronisation on both sides.
    s = torch.cuda.current_stream().cuda_stream
    steps, warm = max(1, args.steps), max(0, args.warmup)
    torch.cuda.synchronize()
    for i in range(warm):
        rot.enqueue(i % copies, s)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        rot.enqueue((warm + i) % copies, s)
    e1.record()
    e1.synchronize()
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / steps
    value = step_bytes / (ms_step * 1e-3) / 1e9
    log(f"{steps} steps: {ms_step * 1e3:.2f} us/step  {value:.1f} GB/s")

    dom = groups["gate_up"]
    gate = next(op for op in ops if op.name == "gate")   # the CPU baseline's sample

    # host-pointer entry (ms_hip_nbits_gemm): A through the handle's pinned staging and a
    # DMA copy, the kernel storing Y straight into pinned host memory (calls of up to 1 MB
    # of A and Y), synchronous; rotating over the weight copies. Reported, never `value`.
    # Each call is timed on its own: the first few hundred calls of a process include one
    # stall of tens of milliseconds in the runtime (measured: one call of 43 ms among 256
    # whose median was 42 us), so a full untimed series goes first and the median is reported
    # beside the mean and the maximum.
    gi = ops.index(gate)
    a_host = workloads.make_activations(1, gate.K, 99)
    calls = 32 * copies
    for c in range(calls):
        rot.handles[c % copies][gi].gemm(a_host)
    per_call = []
    for c in range(calls):
        t0 = time.perf_counter()
        rot.handles[c % copies][gi].gemm(a_host)
        per_call.append((time.perf_counter() - t0) * 1e6)
    host_us = statistics.median(per_call)
    host = {"op": "gate", "K": gate.K, "N": gate.N, "M": 1, "us_per_call": round(host_us, 2),
            "mean_us": round(statistics.mean(per_call), 2), "max_us": round(max(per_call), 1), "calls": calls,
            "GBs": round(workloads.algorithmic_bytes(gate, 1) / (host_us * 1e-6) / 1e9, 1),
            "path": "ms_hip_nbits_gemm: host A -> pinned staging -> H2D copy, kernel storing Y into pinned "
                    "host memory -> host Y, synchronous; median of per-call times"}
    log(f"  host-pointer gate call: median {host_us:.2f} us, mean {host['mean_us']} us, max {host['max_us']} us "
        f"({host['GBs']} GB/s, PCIe copies included)")
    traffic = measured_traffic(dom["kernel"])
    rot.close()
    del rot, g
    torch.cuda.empty_cache()

    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps,
        "warmup": warm, "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "7b_decode_layer", "ops": {op.name: [op.K, op.N] for op in ops}, "M": 1,
                   "bits": 4, "block_size": 32, "zero_points": "packed uint4", "rotating_copies": copies,
                   "bytes_per_step": step_bytes,
                   "timing": "eager batch calls (one C call per step) on one stream, HIP events, "
                             "after the per-launch graph timings"},
        "ms_per_step_graph": round(ms_step_graph, 5),
        "ms_per_step_ungrouped": round(ms_step_ungrouped, 5),
        "per_op": per_op,
        "groups": groups,
        "host_pointer": host,
        "roofline": {"bound": "hbm", "kernel": "gemv_w4, gate+up in one launch (K=3584, 2 x N=18944, M=1)",
                     "achieved": dom["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["GBs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": TRAFFIC_PROFILE if traffic else None,
                     "algorithmic_bytes_per_launch": dom["bytes"]},
    }

    # ---- the whole decoder layer on the device ------------------------------------------
    if not args.no_layer:
        result["decoder_layer"] = decoder_layer(args)

    # ---- prefill, M=2048 ----------------------------------------------------------------
    if not args.no_prefill:
        pre = {}
        total_flops, total_ms = 0, 0.0
        for op in workloads.LLAMA7B_PREFILL_OPS:
            M = 2048
            prot = Rotation([op], M, 2, seed=11, kind="rmsnorm")
            gp = graph_of(lambda stream: [prot.enqueue(r, stream) for r in range(2)])
            ms = time_graph(gp, 10, 2) / 2
            fl = workloads.flops(op, M)
            pre[f"K{op.K}_N{op.N}"] = {"us": round(ms * 1e3, 2), "TFLOPs": round(fl / (ms * 1e-3) / 1e12, 1),
                                       "frac_fp16_peak": round(fl / (ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4)}
            log(f"  prefill M={M} K={op.K} N={op.N}: {ms * 1e3:.1f} us  {pre[f'K{op.K}_N{op.N}']['TFLOPs']} TFLOP/s")
            total_flops += fl
            total_ms += ms
            prot.close()
            del prot, gp
            torch.cuda.empty_cache()
        tf = total_flops / (total_ms * 1e-3) / 1e12
        # The MLP's gate and up projections as an engine issues them: one batch call on the
        # shared input, which converts it to fp16 once (reported beside the per-op line).
        op = workloads.LLAMA7B_PREFILL_OPS[0]
        M = 2048
        prot = Rotation([op, op], M, 2, seed=11, kind="rmsnorm", share=[0, 0])
        gp = graph_of(lambda stream: [prot.enqueue(r, stream) for r in range(2)])
        ms = time_graph(gp, 10, 2) / 2
        fl = 2 * workloads.flops(op, M)
        gate_up = {"ops": f"gate + up, K={op.K}, 2 x N={op.N}, M={M}, one batch call", "us": round(ms * 1e3, 2),
                   "TFLOPs": round(fl / (ms * 1e-3) / 1e12, 1),
                   "frac_fp16_peak": round(fl / (ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4)}
        log(f"  prefill gate+up batch M={M}: {ms * 1e3:.1f} us  {gate_up['TFLOPs']} TFLOP/s")
        prot.close()
        del prot, gp
        torch.cuda.empty_cache()
        # The other prefill sizes of the workload (reported, not aggregated): each op with
        # the kernel the library picks for it.
        smaller = {}
        for M in (128, 512):
            for op in workloads.LLAMA7B_PREFILL_OPS:
                prot = Rotation([op], M, 2, seed=11, kind="rmsnorm")
                gp = graph_of(lambda stream: [prot.enqueue(r, stream) for r in range(2)])
                ms = time_graph(gp, 10, 2) / 2
                fl = workloads.flops(op, M)
                smaller[f"M{M}_K{op.K}_N{op.N}"] = {
                    "us": round(ms * 1e3, 2), "TFLOPs": round(fl / (ms * 1e-3) / 1e12, 1),
                    "frac_fp16_peak": round(fl / (ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4),
                    "kernel": prot.handles[0][0].launch_info(M)["kernel"]}
                log(f"  prefill M={M} K={op.K} N={op.N}: {ms * 1e3:.1f} us ({smaller[f'M{M}_K{op.K}_N{op.N}']['kernel']})")
                prot.close()
                del prot, gp
                torch.cuda.empty_cache()
        # The same shapes with 8-bit codes (reported, not aggregated).
        bits8 = {}
        for op4 in workloads.LLAMA7B_PREFILL_OPS:
            op = dataclasses.replace(op4, name=op4.name + "_8bit", bits=8)
            M = 2048
            prot = Rotation([op], M, 2, seed=13, kind="rmsnorm")
            gp = graph_of(lambda stream: [prot.enqueue(r, stream) for r in range(2)])
            ms = time_graph(gp, 10, 2) / 2
            fl = workloads.flops(op, M)
            bits8[f"K{op.K}_N{op.N}"] = {"us": round(ms * 1e3, 2), "TFLOPs": round(fl / (ms * 1e-3) / 1e12, 1),
                                         "frac_fp16_peak": round(fl / (ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4),
                                         "kernel": prot.handles[0][0].launch_info(M)["kernel"]}
            log(f"  prefill 8-bit M={M} K={op.K} N={op.N}: {ms * 1e3:.1f} us ({bits8[f'K{op.K}_N{op.N}']['kernel']})")
            prot.close()
            del prot, gp
            torch.cuda.empty_cache()
        result["prefill"] = {"workload": "llama7b_prefill M=2048, (K,N)=(4096,11008),(11008,4096), bs=32, zp",
                             "per_op": pre, "TFLOPs": round(tf, 1), "peak_TFLOPs": FP16_PEAK_TFLOPS,
                             "frac": round(tf / FP16_PEAK_TFLOPS, 4), "bound": "mfma",
                             "gate_up_batch": gate_up, "smaller_m": smaller, "bits8_m2048": bits8}

    if args.detail:
        result_detail = detail_workloads(args)
        pathlib.Path(args.detail).write_text(json.dumps(result_detail, indent=1))

    if args.cpu_seconds > 0:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    else:
        result["cpu_baseline"] = None

    print(json.dumps(result), flush=True)
    return 0


class LayerRotation:
    """R copies of one 7B decoder layer held on the device (the seven INT4 projections, two
    RMSNorm weights, a KV cache of `capacity` rows per kv head already holding `past` rows,
    rotary caches) and the activation buffers of a step at M = 1."""
    HID, H, KH, D, INTER = 3584, 28, 4, 128, 18944

    def __init__(self, copies, past, seed):
        import torch
        from modelsharp_amd import native, workloads
        self.copies, self.past, self.capacity = copies, past, past + 1
        ops = workloads.DECODE_7B
        host = [workloads.make_weights(op, seed + i) for i, op in enumerate(ops)]
        self.h = [[native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
                   for (b, s, z), op in zip(host, ops)] for _ in range(copies)]
        g = torch.Generator(device="cpu").manual_seed(seed)
        dev = lambda *shape: torch.randn(*shape, generator=g).cuda()   # noqa: E731
        HID, KH, D = self.HID, self.KH, self.D
        self.g1 = [torch.rand(HID, generator=g).cuda() + 0.5 for _ in range(copies)]
        self.g2 = [torch.rand(HID, generator=g).cuda() + 0.5 for _ in range(copies)]
        self.kc = [dev(1, KH, self.capacity, D) for _ in range(copies)]
        self.vc = [dev(1, KH, self.capacity, D) for _ in range(copies)]
        ang = torch.outer(torch.arange(self.capacity, dtype=torch.float64),
                          1.0 / 10000 ** (torch.arange(D // 2, dtype=torch.float64) / (D // 2)))
        self.cos, self.sin = torch.cos(ang).float().cuda(), torch.sin(ang).float().cuda()
        self.x = [dev(1, HID) for _ in range(copies)]
        self.resid = [dev(1, HID) for _ in range(copies)]
        self.resid2 = [torch.empty(1, HID, device="cuda") for _ in range(copies)]   # the fused norms' sums
        e = lambda n: torch.empty(1, n, device="cuda")   # noqa: E731
        self.n1, self.q, self.k, self.v, self.attn, self.o = e(HID), e(HID), e(KH * D), e(KH * D), e(HID), e(HID)
        self.n2, self.gt, self.up, self.act, self.y = e(HID), e(self.INTER), e(self.INTER), e(self.INTER), e(HID)
        self.desc = native.GqaDesc(batch=1, q_seq=1, kv_seq=1, num_heads=self.H, kv_num_heads=KH, head_dim=D,
                                   packed_qkv=0, past_seq=past, past_in_present=1, present_capacity=self.capacity,
                                   do_rotary=1, rotary_interleaved=0, cos_rows=self.capacity, cos_cols=D // 2,
                                   local_window_size=-1, scale=0.0, seqlens_len=0)
        self.ws_bytes = native.gqa_workspace_size(self.desc)
        self.ws = torch.empty(max(1, (self.ws_bytes + 3) // 4), device="cuda")

    def stage(self, r, name, stream):
        """One stage of copy r's step on `stream` (the residual stream updated in place)."""
        from modelsharp_amd import native
        h, HID, eps = self.h[r], self.HID, 1e-6
        if name == "norm1":
            native.skip_rmsnorm(self.x[r].data_ptr(), self.resid[r].data_ptr(), self.g1[r].data_ptr(), None, None,
                                self.n1.data_ptr(), self.resid[r].data_ptr(), None, 1, HID, eps, stream)
        elif name == "qkv":
            native.gemm_dev_batch(h[0:3], [self.n1.data_ptr()] * 3,
                                  [self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr()], 1, stream)
        elif name == "attention":
            native.gqa(self.desc, self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), None, None, None,
                       self.cos.data_ptr(), self.sin.data_ptr(), self.attn.data_ptr(),
                       self.kc[r].data_ptr(), self.vc[r].data_ptr(), self.ws.data_ptr(), self.ws_bytes, stream)
        elif name == "o":
            h[3].gemm_dev(self.attn.data_ptr(), self.o.data_ptr(), 1, stream)
        elif name == "norm2":
            native.skip_rmsnorm(self.o.data_ptr(), self.resid[r].data_ptr(), self.g2[r].data_ptr(), None, None,
                                self.n2.data_ptr(), self.resid[r].data_ptr(), None, 1, HID, eps, stream)
        elif name == "gate_up":
            native.gemm_dev_batch(h[4:6], [self.n2.data_ptr()] * 2, [self.gt.data_ptr(), self.up.data_ptr()], 1,
                                  stream)
        elif name == "silu_mul":
            native.silu_mul(self.gt.data_ptr(), self.up.data_ptr(), self.act.data_ptr(), self.INTER, stream)
        elif name == "gate_up_silu":   # gate, up and SiLU-Mul in one launch
            native.gemm_dev_swiglu(h[4], h[5], self.n2.data_ptr(), self.act.data_ptr(), 1, stream)
        elif name == "down":
            h[6].gemm_dev(self.act.data_ptr(), self.x[r].data_ptr(), 1, stream)
        elif name == "norm1_qkv":   # SkipRMSNorm computed in the q/k/v launch's staging
            native.gemm_dev_skipnorm(h[0:3], self.x[r].data_ptr(), self.resid[r].data_ptr(), self.g1[r].data_ptr(),
                                     eps, self.n1.data_ptr(), self.resid2[r].data_ptr(),
                                     [self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr()], 1, stream)
        elif name == "norm2_gate_up_silu":   # SkipRMSNorm, gate, up and SiLU-Mul in one launch
            native.gemm_dev_skipnorm_swiglu(h[4], h[5], self.o.data_ptr(), self.resid2[r].data_ptr(),
                                            self.g2[r].data_ptr(), eps, self.n2.data_ptr(), self.resid[r].data_ptr(),
                                            self.act.data_ptr(), 1, stream)

    # the norms in the launches of the projections that read them (the residual stream
    # alternates between two buffers: a fused norm's sum may not overwrite its skip input)
    STAGES = ("norm1_qkv", "attention", "o", "norm2_gate_up_silu", "down")
    # the norms as launches of their own
    NORMS_APART = ("norm1", "qkv", "attention", "o", "norm2", "gate_up_silu", "down")
    # and gate+up and SiLU-Mul as two launches too
    UNFUSED = ("norm1", "qkv", "attention", "o", "norm2", "gate_up", "silu_mul", "down")

    def close(self):
        for row in self.h:
            for w in row:
                w.close()


class AttentionPrefill:
    """GroupQueryAttention at prefill on the 7B layer's heads: 2048 query rows over
    themselves (causal), rotary (half-split, base 10000), past 0, random q/k/v."""
    S = 2048

    def __init__(self):
        import torch
        from modelsharp_amd import native
        S, H, KH, D = self.S, LayerRotation.H, LayerRotation.KH, LayerRotation.D
        gen = torch.Generator(device="cpu").manual_seed(5)
        self.q = torch.randn(1, S, H * D, generator=gen).cuda()
        self.k = torch.randn(1, S, KH * D, generator=gen).cuda()
        self.v = torch.randn(1, S, KH * D, generator=gen).cuda()
        ang = torch.outer(torch.arange(S, dtype=torch.float64),
                          1.0 / 10000 ** (torch.arange(D // 2, dtype=torch.float64) / (D // 2)))
        self.cos, self.sin = torch.cos(ang).float().cuda(), torch.sin(ang).float().cuda()
        self.pk, self.pv = torch.empty(1, KH, S, D, device="cuda"), torch.empty(1, KH, S, D, device="cuda")
        self.o = torch.empty(1, S, H * D, device="cuda")
        self.d = native.GqaDesc(batch=1, q_seq=S, kv_seq=S, num_heads=H, kv_num_heads=KH, head_dim=D, packed_qkv=0,
                                past_seq=0, past_in_present=0, present_capacity=S, do_rotary=1, rotary_interleaved=0,
                                cos_rows=S, cos_cols=D // 2, local_window_size=-1, scale=0.0, seqlens_len=0)
        self.wsb = native.gqa_workspace_size(self.d)
        self.ws = torch.empty(max(1, (self.wsb + 3) // 4), device="cuda")
        self.flops = 2 * 2 * H * D * S * (S + 1) / 2   # q.k and p.v over the causal half

    def launch(self, stream):
        from modelsharp_amd import native
        native.gqa(self.d, self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), None, None, None,
                   self.cos.data_ptr(), self.sin.data_ptr(), self.o.data_ptr(), self.pk.data_ptr(), self.pv.data_ptr(),
                   self.ws.data_ptr(), self.wsb, stream)


def decoder_layer(args):
    """The 7B decoder layer at decode on the device: SkipSimplifiedLayerNormalization ->
    q/k/v (one grouped launch) -> GroupQueryAttention (28 query / 4 kv heads of 128, rotary,
    past 2047 rows appended in place) -> o -> SkipSimplifiedLayerNormalization -> gate/up
    and SiLU*Mul (one launch) -> down, device pointers throughout; rotating copies of the
    layer (weights and KV cache) over >= 1 GiB; the same step with gate/up and SiLU*Mul as
    two launches beside it. Then GroupQueryAttention at prefill (2048 query rows, past 0)."""
    import torch
    from modelsharp_amd import native, workloads
    past = 2047
    per_copy = sum(workloads.algorithmic_bytes(op, 1) for op in workloads.DECODE_7B) + 2 * 4 * (past + 1) * 128 * 4
    copies = workloads.rotation_copies(per_copy, args.rotate_mib << 20)
    lay = LayerRotation(copies, past, seed=21)
    g = graph_of(lambda st: [lay.stage(r, n, st) for r in range(copies) for n in LayerRotation.STAGES])
    ms = time_graph(g, max(4, math.ceil(200 / copies)), 2) / copies
    del g
    g = graph_of(lambda st: [lay.stage(r, n, st) for r in range(copies) for n in LayerRotation.NORMS_APART])
    ms_norms = time_graph(g, max(4, math.ceil(200 / copies)), 2) / copies
    del g
    g = graph_of(lambda st: [lay.stage(r, n, st) for r in range(copies) for n in LayerRotation.UNFUSED])
    ms_unfused = time_graph(g, max(4, math.ceil(200 / copies)), 2) / copies
    del g
    stages = {}
    for n in dict.fromkeys(LayerRotation.STAGES + LayerRotation.NORMS_APART + LayerRotation.UNFUSED):
        gs = graph_of(lambda st, n=n: [lay.stage(r, n, st) for r in range(copies)])
        stages[n] = round(time_graph(gs, max(4, math.ceil(200 / copies)), 2) / copies * 1e3, 3)
        del gs
    finite = bool(torch.isfinite(lay.x[0]).all())
    log(f"decoder layer step (past {past}): {ms * 1e3:.2f} us ({ms_norms * 1e3:.2f} us with the norms as launches "
        f"of their own, {ms_unfused * 1e3:.2f} us with gate+up and SiLU-Mul apart too); stages {stages}; "
        f"finite output {finite}")
    out = {"workload": "7B decoder layer at decode, M=1, past 2047, device-resident (hidden 3584, 28/4 heads of "
                       "128, intermediate 18944, bs 32 zp)", "rotating_copies": copies,
           "us_per_step": round(ms * 1e3, 3), "stages": list(LayerRotation.STAGES),
           "us_per_step_norms_apart": round(ms_norms * 1e3, 3),
           "us_per_step_gate_up_and_silu_apart": round(ms_unfused * 1e3, 3), "stage_us": stages,
           "bytes_per_step": per_copy, "GBs": round(per_copy / (ms * 1e-3) / 1e9, 1), "finite": finite}
    lay.close()
    del lay
    torch.cuda.empty_cache()
    # attention at prefill: 2048 query rows over themselves (causal), rotary, past 0
    att = AttentionPrefill()
    gp = graph_of(att.launch)
    msp = time_graph(gp, 5, 1)
    out["attention_prefill"] = {"q_seq": att.S, "past": 0, "us": round(msp * 1e3, 1),
                                "TFLOPs": round(att.flops / (msp * 1e-3) / 1e12, 2)}
    log(f"attention prefill S={att.S}: {msp * 1e3:.1f} us")
    del gp, att
    torch.cuda.empty_cache()
    return out


def profile_op(args) -> int:
    """Eager launches of one decode op over the rotation (for per-dispatch
    hardware counters), then a device-to-device copy of known size whose
    counters calibrate the byte counts."""
    import torch
    from modelsharp_amd import workloads
    from modelsharp_amd import native
    if args.op in ("decoder_layer", "attention_prefill"):
        stream = torch.cuda.current_stream().cuda_stream
        if args.op == "attention_prefill":
            att = AttentionPrefill()
            for _ in range(args.calls):
                att.launch(stream)
            what = f"GroupQueryAttention, {att.S} queries, past 0, 28/4 heads of 128 ({att.flops:.4g} flops each)"
        else:
            copies = 4
            lay = LayerRotation(copies, 2047, seed=21)
            for i in range(args.calls):
                for n in LayerRotation.STAGES:
                    lay.stage(i % copies, n, stream)
            what = f"7B decoder layer steps at past 2047 ({copies} rotating copies), stages {LayerRotation.STAGES}"
        torch.cuda.synchronize()
        log(f"{args.calls} launches of {args.op}: {what}; kernel sources {kernel_source_digest()}")
        return 0
    if args.op.startswith("prefill_"):
        ops = [next(o for o in workloads.LLAMA7B_PREFILL_OPS if o.name == args.op[len("prefill_"):])]
        M, kind = args.m, "rmsnorm"
        copies = max(2, workloads.rotation_copies(workloads.algorithmic_bytes_group(ops, M), args.rotate_mib << 20))
    elif args.op.startswith("smallm_"):
        ops = [next(o for o in workloads.LLAMA7B_SMALLM_OPS if o.name == args.op[len("smallm_"):])]
        M, kind = args.m, "normal"
        copies = workloads.rotation_copies(workloads.algorithmic_bytes_group(ops, M), args.rotate_mib << 20)
    else:
        ops = ([workloads.DECODE_7B[i] for i in GROUPS[args.op]] if args.op in GROUPS else
               [next(o for o in workloads.DECODE_7B if o.name == args.op)])
        M, kind = 1, "normal"
    fp = workloads.algorithmic_bytes_group(ops, M)
    if M == 1 and not args.op.startswith("smallm_"):
        copies = workloads.rotation_copies(fp, args.rotate_mib << 20)
    rot = Rotation(ops, M, copies, seed=7, kind=kind, share=[0] * len(ops))
    stream = torch.cuda.current_stream().cuda_stream
    for i in range(args.calls):
        rot.enqueue(i % copies, stream)
    torch.cuda.synchronize()
    launch = native.batch_launch_info(rot.handles[0], [a.data_ptr() for a in rot.A[0]], M)
    log(f"{args.calls} launches of {args.op} (M={M}, K={ops[0].K}, N={'+'.join(str(o.N) for o in ops)}, "
        f"{fp} algorithmic bytes, {sum(workloads.flops(o, M) for o in ops)} flops each), {copies} rotating copies; "
        f"launch {launch}; kernel sources {kernel_source_digest()}")
    src = torch.empty(args.copy_mib << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"4 copies of {args.copy_mib << 20} bytes (read {args.copy_mib << 20}, write {args.copy_mib << 20} each)")
    rot.close()
    return 0


def detail_workloads(args):
    """Per-op results for the other workloads (parity-test sizes; not the bench line)."""
    import torch
    from modelsharp_amd import workloads
    out = {}
    groups = [("qwen05b_up", [workloads.QWEN05B_UP], [1]),
              ("qwen05b_decode", workloads.QWEN05B_DECODE, [1]),
              ("llama7b_smallm", workloads.LLAMA7B_SMALLM_OPS, workloads.LLAMA7B_SMALLM_M),
              ("llama7b_prefill", workloads.LLAMA7B_PREFILL_OPS, workloads.LLAMA7B_PREFILL_M)]
    for name, ops, Ms in groups:
        for M in Ms:
            for op in ops:
                fp = workloads.algorithmic_bytes(op, M)
                copies = min(workloads.rotation_copies(fp, args.rotate_mib << 20), 64)
                if M >= 128:
                    copies = 2
                rot = Rotation([op], M, copies, seed=3, kind="rmsnorm" if M >= 128 else "normal")
                g = graph_of(lambda stream: [rot.enqueue(r, stream) for r in range(copies)])
                ms = time_graph(g, 10 if M >= 128 else 50, 2) / copies
                out[f"{name}/{op.name}/M{M}"] = {
                    "K": op.K, "N": op.N, "M": M, "us": round(ms * 1e3, 3),
                    "GBs": round(fp / (ms * 1e-3) / 1e9, 1),
                    "TFLOPs": round(workloads.flops(op, M) / (ms * 1e-3) / 1e12, 2),
                    "kernel": rot.handles[0][0].launch_info(M)}
                log(f"  {name}/{op.name}/M{M}: {out[f'{name}/{op.name}/M{M}']}")
                rot.close()
                del rot, g
                torch.cuda.empty_cache()
    # Qwen2.5-0.5B decode token: the 8 projections in one batch call with the inputs shared
    # as in the model (q/k/v one input, gate/up another), against the sum of single launches.
    ops = workloads.QWEN05B_DECODE
    fp = sum(workloads.algorithmic_bytes(op, 1) for op in ops)
    copies = min(workloads.rotation_copies(fp, args.rotate_mib << 20), 64)
    rot = Rotation(ops, 1, copies, seed=3, share=workloads.QWEN05B_DECODE_SHARE)
    g = graph_of(lambda stream: [rot.enqueue(r, stream) for r in range(copies)])
    ms = time_graph(g, 50, 2) / copies
    single = sum(v["us"] for k, v in out.items() if k.startswith("qwen05b_decode/"))
    out["qwen05b_decode/per_token"] = {"bytes": fp, "us_grouped": round(ms * 1e3, 3),
                                       "GBs_grouped": round(fp / (ms * 1e-3) / 1e9, 1),
                                       "us_sum_of_single_launches": round(single, 3)}
    log(f"  qwen05b_decode/per_token: {out['qwen05b_decode/per_token']}")
    rot.close()
    del rot, g
    torch.cuda.empty_cache()
    return out


if __name__ == "__main__":
    sys.exit(main())
