#!/usr/bin/env python3
"""Benchmark of the full verify step at serving shape on one MI355X.

Workload (the headline configuration): 64 requests x 17 rows x 151936 vocab bf16 logits,
per-request temperature {0, 0.6, 1.0}, top-k {off, 20}, top-p {1.0, 0.95}, presence/repetition
penalties over a 512-token history, sparse draft q [64, 16, 16], int32 page table.  One step =
logit adjustments -> target distribution -> chain rejection -> residual resample -> accepted-prefix
compaction + KV-slot gather, on inputs already resident in HBM.  K steps are timed as plain stream
launches and as HIP-graph replays (each bracketed by device synchronisation); the faster is the
step time.

Prints ONE JSON line (metric: verified rows/s) with the roofline of the dominant kernel -- the
chunk pass k_chunk, which reads every logit once; its launches are bracketed by HIP events on
their stream (dsv_profile_events) over a run of full steps -- and the CPU oracle timed on the
host.  The HBM traffic figure comes from the committed rocprofv3 counter summary of that kernel
(profiles/k_chunk_serving_traffic.txt) when it is present.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "verify rows/sec at B=64x17x151936 bf16; achieved HBM GB/s vs peak"
PEAK_GBPS = 8000.0  # MI355X HBM3E


def algorithmic_bytes(bs, T, V, K, hist_len):
    """(whole step, chunk pass) algorithmic HBM bytes.  The step: one read of every verified
    logit row plus the small per-request inputs and outputs.  The chunk pass k_chunk: the
    logits (2 bytes per value) and each request's history bitmap (V/8 bytes, read once per
    request; its rows find it in L2) -- its per-chunk statistics, candidates and value counts
    are workspace it writes for the merge (counted in the traffic figure, not here)."""
    logits = bs * T * V * 2
    small_in = (bs * hist_len * 4 + bs * (T - 1) * K * (8 + 4) + bs * T * 8 + bs * (T - 1) * 4 + bs * 4
                + bs * 4 * 4 + bs * 4 + bs * T * 4)
    outputs = bs * (4 + 4 + 8 + 4) + bs * T * 8 + bs * T * 4
    chunk_pass = logits + bs * ((V + 31) // 32) * 4
    return logits + small_in + outputs, chunk_pass


def committed_traffic():
    """HBM bytes per k_chunk launch from the committed counter summary, or None."""
    path = os.path.join(ROOT, "profiles", "k_chunk_serving_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch"):
            return float(line.split("=", 1)[1].split()[0])
    return None


def time_kernel_events(step, steps, lib, torch):
    """Average k_chunk duration over `steps` eager steps: HIP events recorded by the library right
    before and after the kernel launch, on the stream it is launched on."""
    pairs = []
    for _ in range(steps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        e.record()  # creates both events; the library re-records them around the kernel
        lib.dsv_profile_events(s.cuda_event, e.cuda_event)
        step()
        pairs.append((s, e))
    lib.dsv_profile_events(None, None)
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in pairs) / steps


def time_graph(step, steps, warmup, torch):
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, g


def cpu_baseline(batch, min_seconds=10.0, max_seconds=30.0):
    """The CPU oracle (torch on the host) on a bounded sample of the same workload: passes over
    the requests, one request per call, until at least ``min_seconds`` of work (capped at
    ``max_seconds``)."""
    import numpy as np
    import torch

    import oracle.verify_oracle as O

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    bs, T = batch["candidates"].shape
    calls, rows, t0 = 0, 0, time.perf_counter()
    done = False
    while not done:
        for b in range(bs):
            O.verify_step(
                batch["logits"], batch["info"], candidates=batch["candidates"].numpy(),
                q_ids=batch["q_ids"].numpy(), q_values=batch["q_values"].numpy(),
                verify_lens=np.full(bs, T), uniforms=batch["uniforms"].numpy(),
                uniform_final=batch["uniform_final"].numpy(), prefix_lens=batch["prefix_lens"].numpy(),
                hist_ids=batch["hist_ids"], presence=batch["presence"], repetition=batch["repetition"],
                page_table=batch["page_table"], requests=[b])
            calls += 1
            rows += T
            if time.perf_counter() - t0 > max_seconds:
                done = True
                break
        if time.perf_counter() - t0 >= min_seconds:
            done = True
    dt = time.perf_counter() - t0
    return {"value": rows / dt, "unit": "rows/s", "cores": n, "kind": "port",
            "sample": f"{calls} request verifications ({calls / bs:.2f} passes over the {bs} requests, "
                      f"{rows} rows x 151936) of the same workload, one request per oracle call, {dt:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain 256 MiB device copy (the reference for HBM byte counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if args.calibrate_copy:
        n = 256 << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": n, "calibrate_copy_bytes_written": n, "launches": 5}))
        return

    from dspine_amd import workloads as W
    from dspine_amd.verify import History, Workspace, new_outputs, verify_step

    dev = torch.device("cuda:0")
    t0 = time.perf_counter()
    batch = W.serving_round()
    d = W.to_device(batch, dev)
    print(f"[bench] workload ready in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    bs, T = batch["candidates"].shape
    V = batch["logits"].shape[1]
    K = batch["q_ids"].shape[2]
    H = batch["hist_ids"].shape[1]
    outs, kv = new_outputs(bs, T, dev)
    ws = Workspace()
    hist = History(d["hist_ids"], d["presence"], d["repetition"])
    info = d["info"]
    info.temperatures = info.temperatures.reshape(-1).contiguous()

    def step(stages=0):
        verify_step(logits=d["logits"], sampling_info=info, candidates=d["candidates"],
                    q_ids=d["q_ids"], q_values=d["q_values"], uniforms=d["uniforms"],
                    uniform_final=d["uniform_final"], prefix_lens=d["prefix_lens"], history=hist,
                    page_table=d["page_table"], outputs=outs, kv_slots=kv, workspace=ws,
                    _stages=stages)

    # eager timing: K steps bracketed by device synchronisation
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / args.steps
    # graph replay; the step's time is the faster of the two launch modes (the same work either way)
    graph_ms, _g = time_graph(step, args.steps, args.warmup, torch)
    ms = min(graph_ms, eager_ms)
    mode = "graph" if graph_ms <= eager_ms else "eager"
    # the dominant kernel: k_chunk inside full steps, HIP events on its launch stream
    from dspine_amd import _lib

    kern_ms = time_kernel_events(step, args.steps, _lib.load(), torch)
    total_bytes, chunk_bytes = algorithmic_bytes(bs, T, V, K, H)
    acc = outs[0].float().mean().item()
    print(f"[bench] graph {graph_ms * 1e3:.1f} us/step, eager {eager_ms * 1e3:.1f} us/step, k_chunk "
          f"{kern_ms * 1e3:.1f} us, mean accept {acc:.2f}, step {total_bytes / (ms * 1e-3) / 1e9:.0f} GB/s",
          file=sys.stderr, flush=True)
    achieved = chunk_bytes / (kern_ms * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": bs * T / (ms * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "full verify step (penalties, temperature softmax, top-k/top-p filter, chain "
                        "rejection with sparse q, residual resample, compaction + KV slots)",
            "requests": bs, "rows_per_request": T, "vocab": V, "q_width": K, "history": H,
            "logits_dtype": "bf16", "timed_launch": mode, "eager_ms_per_step": eager_ms,
            "graph_ms_per_step": graph_ms,
            "step_GBps_algorithmic": total_bytes / (ms * 1e-3) / 1e9,
        },
        "roofline": {
            "bound": "hbm", "achieved": achieved, "peak": PEAK_GBPS, "unit": "GB/s",
            "frac": achieved / PEAK_GBPS, "traffic": committed_traffic(),
            "kernel": "k_chunk (chunk pass: 1088 rows x 8 chunks of 20480 bf16)",
            "kernel_us": kern_ms * 1e3, "algorithmic_bytes": chunk_bytes,
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(batch)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
