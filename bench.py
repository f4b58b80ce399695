#!/usr/bin/env python3
"""Benchmark of the verification hot path on one MI355X.

Default workload (the headline configuration, ``--config 4``): the full verify step at serving
shape -- 64 requests x 17 rows x 151936 vocab bf16 logits, per-request temperature {0, 0.6,
1.0}, top-k {off, 20}, top-p {1.0, 0.95}, presence/repetition penalties over a 512-token
history, sparse draft q [64, 16, 16], int32 page table.  One step = logit adjustments -> target
distribution -> chain rejection -> residual resample -> accepted-prefix compaction + KV-slot
gather, on inputs already resident in HBM.

Other workloads (parity cases of the same path, timed the same way):
  --config 2   top-k only: [1088, 151936] bf16 with planted peaks and duplicates, --k {1,20,64}
  --config 3   rejection: 32 x 17 x 151936 fp32, top-k 20, top-p 0.95, sparse q (--sigma)
  --config 5   ragged: 32 requests x U{4..16} rows x 262144 bf16 Student-t, top-p 0.9

  --config 1   greedy: 1 x 17 x 151936 fp32, argmax acceptance with one seeded mismatch
  --config 4 --accept deep   the serving step with a planted likely token per row, so that a
               mean of ~6.5 of the 16 drafts is accepted

The logits of each step come from one of several identical copies in turn (together >= 661 MB,
so no step reads data the previous steps left in the 256 MB Infinity Cache).  One HIP graph per
copy holds one step; the step time is the median of K single-step replays (each bracketed by its
own HIP events, the K bracketed by device synchronisation), reported with p90.  All K steps in
one graph and K plain stream launches are reported beside it as labelled fields.

Prints ONE JSON line (metric: verified rows/s) with the roofline of the dominant kernel -- the
chunk pass k_chunk, which reads every logit once; its launches are bracketed by HIP events on
their stream (dsv_profile_events) over a run of full steps -- the step's own fraction of peak
(``step_frac``) and the CPU oracle timed on the host.  The HBM traffic figure comes from the
committed rocprofv3 counter summary of that kernel (profiles/k_chunk_<workload>_traffic.txt)
when one is present.
"""

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "verify rows/sec at B=64x17x151936 bf16; achieved HBM GB/s vs peak"
DEEP_PEAK = 16.0  # the planted logit of --accept deep (mean accepted length ~6.5 of 16)
PEAK_GBPS = 8000.0  # MI355X HBM3E
ROTATE_BYTES = 661 << 20  # logits copies read in turn: more than twice the 256 MB Infinity Cache


def verify_bytes(bs, T, V, K, hist_len, esize, rows=None):
    """(whole step, chunk pass) algorithmic HBM bytes of a fused verify step.  The step: one
    read of every verified logit row plus the small per-request inputs and outputs.  The chunk
    pass k_chunk: the logits and each request's history ids (read once per request; the
    request's other chunks find them in L2) -- its per-chunk statistics, candidates, value
    counts and the requests' history bitmaps are workspace it writes for the later kernels
    (counted in the traffic figure, not here)."""
    rows = bs * T if rows is None else rows
    logits = rows * V * esize
    small_in = (bs * hist_len * 4 + bs * (T - 1) * K * (8 + 4) + bs * T * 8 + bs * (T - 1) * 4 + bs * 4
                + bs * 4 * 4 + bs * 4 + bs * T * 4)
    outputs = bs * (4 + 4 + 8 + 4) + bs * T * 8 + bs * T * 4
    chunk_pass = logits + bs * hist_len * 4
    return logits + small_in + outputs, chunk_pass


def committed_traffic(workload):
    """HBM bytes per k_chunk launch from the committed counter summary, or None."""
    path = os.path.join(ROOT, "profiles", f"k_chunk_{workload}_traffic.txt")
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
    for i in range(steps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        e.record()  # creates both events; the library re-records them around the kernel
        lib.dsv_profile_events(s.cuda_event, e.cuda_event)
        step(i)
        pairs.append((s, e))
    lib.dsv_profile_events(None, None)
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in pairs) / steps


def time_eager(step, steps, warmup, torch):
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def time_replays(step, steps, warmup, nbuf, torch):
    """Per-step latency as a serving loop pays it: one HIP graph per logits copy, each holding
    one step, replayed in turn `steps` times after `warmup` untimed replays; every replay is
    bracketed by its own HIP events on the replay stream.  Returns the per-step times (ms)."""
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    graphs = []
    for i in range(nbuf):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(i)
        graphs.append(g)
    for i in range(max(warmup, nbuf)):
        graphs[i % nbuf].replay()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i, (s, e) in enumerate(ev):
        s.record()
        graphs[i % nbuf].replay()
        e.record()
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in ev], graphs


def time_one_graph(step, steps, nbuf, torch):
    """All `steps` steps captured in one graph (the logits copies in turn), replayed once untimed
    and once timed: the device-side floor of back-to-back steps without a replay boundary."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            step(i % nbuf)
    g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def percentile(xs, q):
    xs = sorted(xs)
    i = min(len(xs) - 1, max(0, int(math.ceil(q * len(xs))) - 1))
    return xs[i]


def copies(t, torch):
    """Identical copies of `t` at distinct addresses, together >= ROTATE_BYTES."""
    n = max(2, math.ceil(ROTATE_BYTES / (t.numel() * t.element_size())))
    return [t] + [t.clone() for _ in range(n - 1)]


def _cpu_median(run, runs=10, warm=2):
    """Median wall time (s) of `runs` calls of run() after `warm` untimed ones, on every core this
    process may use (torch.set_num_threads), and that thread count."""
    import torch

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    for _ in range(warm):
        run()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2], n, times


def cpu_verify_baseline(batch, requests=32, sparse_joint=False, backend="pytorch"):
    """The CPU oracle (torch on the host) on a bounded sample of the same workload: the first
    `requests` requests verified in one oracle call (about a second a call on the serving
    workload), median of 10 calls after 2 warm-ups."""
    import numpy as np

    import oracle.verify_oracle as O

    bs, T = batch["candidates"].shape
    lens = batch.get("verify_lens")
    lens = np.full(bs, T) if lens is None else lens.numpy()
    offs = batch.get("row_offsets")
    V = batch["logits"].shape[1]
    sub = list(range(min(requests, bs)))
    rows = int(sum(int(lens[b]) for b in sub))

    def run():
        O.verify_step(
            batch["logits"], batch["info"], candidates=batch["candidates"].numpy(),
            q_ids=batch["q_ids"].numpy(), q_values=batch["q_values"].numpy(), verify_lens=lens,
            uniforms=batch["uniforms"].numpy(), uniform_final=batch["uniform_final"].numpy(),
            prefix_lens=batch["prefix_lens"].numpy(), hist_ids=batch.get("hist_ids"),
            presence=batch.get("presence"), repetition=batch.get("repetition"),
            page_table=batch.get("page_table"), row_offsets=None if offs is None else offs.numpy(),
            sampling_backend=backend, requests=sub, sparse_joint=sparse_joint)

    med, n, times = _cpu_median(run)
    return {"value": rows / med, "unit": "rows/s", "cores": n, "kind": "port", "ms_per_sample": med * 1e3,
            "sample": f"requests 0..{len(sub) - 1} of the same workload ({rows} rows x {V}) in one oracle call, "
                      f"median of {len(times)} calls after 2 warm-ups ({sum(times):.1f} s timed)"}


def cpu_topk_baseline(x, k, rows=1088):
    """The CPU oracle's top-k (stable descending sort) on the first `rows` rows (every row of the
    workload by default), median of 10."""
    import oracle.verify_oracle as O

    sl = x[:rows].float()
    med, n, times = _cpu_median(lambda: O.topk(sl, k))
    return {"value": rows / med, "unit": "rows/s", "cores": n, "kind": "port", "ms_per_sample": med * 1e3,
            "sample": f"rows 0..{rows - 1} x {x.shape[1]}, k={k}, median of {len(times)} calls after 2 warm-ups "
                      f"({sum(times):.1f} s timed)"}


def cpu_greedy_baseline(batch):
    """The CPU oracle's greedy verify (argmax + first mismatch) of the whole 1 x 17 round,
    median of 10 after 2 warm-ups."""
    import oracle.verify_oracle as O

    bs, T = batch["candidates"].shape

    def run():
        top1 = O.argmax_rows(batch["logits"])
        O.greedy_accept(top1, batch["candidates"].numpy(), [T] * bs, batch["prefix_lens"].numpy())

    med, n, times = _cpu_median(run)
    return {"value": bs * T / med, "unit": "rows/s", "cores": n, "kind": "port", "ms_per_sample": med * 1e3,
            "sample": f"the whole round ({bs * T} rows x {batch['logits'].shape[1]} fp32), median of {len(times)} "
                      f"calls after 2 warm-ups"}


def setup_verify(config, args, torch, dev):
    """(step(i), workload facts) of a fused verify workload."""
    from dspine_amd import workloads as W
    from dspine_amd.verify import History, Workspace, new_outputs, verify_step

    if config == 4:
        deep = args.accept == "deep"
        batch = W.serving_round(peak=DEEP_PEAK if deep else None)
        name = "serving_deep" if deep else "serving"
        workload = ("full verify step (penalties, temperature softmax, top-k/top-p filter, chain rejection with "
                    "sparse q, residual resample, compaction + KV slots)"
                    + (f"; one planted logit per row at {DEEP_PEAK:g} +- 1 (deep acceptance)" if deep else ""))
    elif config == 3:
        batch = W.rejection_round(sigma_draft=args.sigma)
        name, workload = "rejection", (f"verify step, fp32 target, T=1, top-k 20, top-p 0.95, sparse q from "
                                       f"draft logits + N(0, {args.sigma}^2)")
    else:
        batch = W.ragged_round()
        name, workload = "ragged", ("ragged verify step, compact rows (verify lengths U{4..16}), T=1, top-p 0.9, "
                                    "heavy-tailed logits")
    d = W.to_device(batch, dev)
    bs, T = batch["candidates"].shape
    V = batch["logits"].shape[1]
    K = batch["q_ids"].shape[2]
    H = batch["hist_ids"].shape[1] if "hist_ids" in batch else 0
    rows = batch["logits"].shape[0]
    esize = batch["logits"].element_size()
    outs, kv = new_outputs(bs, T, dev)
    ws = Workspace()
    hist = History(d["hist_ids"], d["presence"], d["repetition"]) if H else None
    info = d["info"]
    info.temperatures = info.temperatures.reshape(-1).contiguous()
    bufs = copies(d["logits"], torch)

    def step(i):
        verify_step(logits=bufs[i % len(bufs)], sampling_info=info, candidates=d["candidates"],
                    q_ids=d["q_ids"], q_values=d["q_values"], uniforms=d["uniforms"],
                    uniform_final=d["uniform_final"], prefix_lens=d["prefix_lens"],
                    verify_lens=d.get("verify_lens"), row_offsets=d.get("row_offsets"), history=hist,
                    page_table=d.get("page_table"), outputs=outs, kv_slots=kv if "page_table" in d else None,
                    workspace=ws)

    total, chunk = verify_bytes(bs, T, V, K, H, esize, rows=rows)
    C = math.ceil(V / (20480 if esize == 2 else 12288))
    facts = dict(name=name, batch=batch, rows=rows, total=total, chunk=chunk, dtype="bf16" if esize == 2 else "f32",
                 kernel=f"k_chunk (chunk pass: {rows} rows x {C} chunks of {20480 if esize == 2 else 12288} "
                        f"{'bf16' if esize == 2 else 'fp32'})",
                 config={"workload": workload, "requests": bs, "rows_per_request": T, "rows": rows, "vocab": V,
                         "q_width": K, "history": H, "logits_dtype": "bf16" if esize == 2 else "fp32",
                         "logits_copies": len(bufs)},
                 accept=lambda: outs[0].float().mean().item())
    return step, facts


def setup_greedy(args, torch, dev):
    """Greedy verify of the 1 x 17 x 151936 fp32 round (argmax acceptance, capped at 17)."""
    from dspine_amd import workloads as W
    from dspine_amd.verification.caps import accept_greedy

    batch = W.greedy_round()
    rows, V = batch["logits"].shape
    cand = batch["candidates"].to(dev)
    prefix = batch["prefix_lens"].to(dev)
    bufs = copies(batch["logits"].to(dev), torch)
    outs = (torch.empty(1, device=dev, dtype=torch.int32), torch.empty(1, device=dev, dtype=torch.int32),
            torch.empty(1, device=dev, dtype=torch.int64), torch.empty((1, rows), device=dev, dtype=torch.int64),
            torch.empty(1, device=dev, dtype=torch.int32))

    def step(i):
        accept_greedy(candidates=cand, next_token_logits=bufs[i % len(bufs)], prefix_lens=prefix, cap=rows,
                      outputs=outs)

    logits = rows * V * 4
    small = rows * 8 + 4 + (4 + 4 + 8 + rows * 8 + 4)
    facts = dict(name="greedy", batch=batch, rows=rows, total=logits + small, chunk=logits, dtype="f32",
                 kernel=f"k_chunk (greedy pass: {rows} rows x {math.ceil(V / 12288)} chunks of 12288 fp32)",
                 config={"workload": "greedy verify (argmax acceptance), temperature 0, one seeded mismatch",
                         "requests": 1, "rows_per_request": rows, "rows": rows, "vocab": V, "logits_dtype": "fp32",
                         "logits_copies": len(bufs)},
                 accept=lambda: outs[0].float().mean().item())
    return step, facts


def setup_topk(args, torch, dev):
    from dspine_amd import workloads as W
    from dspine_amd.kernels.dspine import topk

    x = W.topk_rows()["logits"]
    rows, V = x.shape
    k = args.k
    vals = torch.empty((rows, k), dtype=torch.float32, device=dev)
    ids = torch.empty((rows, k), dtype=torch.int64, device=dev)
    bufs = copies(x.to(dev), torch)

    def step(i):
        topk(bufs[i % len(bufs)], k, vals, ids)

    logits = rows * V * 2
    facts = dict(name="topk", x=x, rows=rows, total=logits + rows * k * 12, chunk=logits, dtype="bf16",
                 kernel=f"k_chunk (candidate pass: {rows} rows x {math.ceil(V / 20480)} chunks of 20480 bf16)",
                 config={"workload": f"top-k only, k={k}, (value desc, id asc) order, planted peaks and ~1% "
                                     f"duplicates", "rows": rows, "vocab": V, "k": k, "logits_dtype": "bf16",
                         "logits_copies": len(bufs)},
                 accept=None)
    return step, facts


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=4, choices=(1, 2, 3, 4, 5),
                    help="workload: 4 = the serving verify step (default); 1 greedy, 2 top-k, 3 rejection, 5 ragged")
    ap.add_argument("--accept", default="low", choices=("low", "deep"),
                    help="drafts of --config 4: low (the seeded workload as generated) or deep (a planted likely "
                         "token per row: a mean accepted length near 6.5)")
    ap.add_argument("--k", type=int, default=64, choices=(1, 20, 64), help="top-k of --config 2")
    ap.add_argument("--sigma", type=float, default=0.5, choices=(0.5, 1.5), help="draft noise of --config 3")
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

    from dspine_amd import _lib

    dev = torch.device("cuda:0")
    t0 = time.perf_counter()
    if args.config == 1:
        step, f = setup_greedy(args, torch, dev)
    elif args.config == 2:
        step, f = setup_topk(args, torch, dev)
    else:
        step, f = setup_verify(args.config, args, torch, dev)
    nbuf = f["config"]["logits_copies"]
    print(f"[bench] config {args.config} ready in {time.perf_counter() - t0:.1f} s ({nbuf} logits copies)",
          file=sys.stderr, flush=True)

    # the headline: the median of `steps` single-step graph replays
    times, _graphs = time_replays(step, args.steps, args.warmup, nbuf, torch)
    ms = statistics.median(times)
    p90 = percentile(times, 0.9)
    # labelled side figures: every step in one graph (no replay boundary), and plain launches
    one_graph_ms = time_one_graph(step, args.steps, nbuf, torch)
    eager_ms = time_eager(step, args.steps, args.warmup, torch)
    kern_ms = time_kernel_events(step, args.steps, _lib.load(), torch)
    total_bytes, chunk_bytes = f["total"], f["chunk"]
    achieved = chunk_bytes / (kern_ms * 1e-3) / 1e9
    step_gbps = total_bytes / (ms * 1e-3) / 1e9
    acc = f["accept"]() if f["accept"] else None
    print(f"[bench] step p50 {ms * 1e3:.1f} us, p90 {p90 * 1e3:.1f} us ({args.steps} single-step graph replays); "
          f"one graph of all steps {one_graph_ms * 1e3:.1f} us/step, eager {eager_ms * 1e3:.1f} us/step; k_chunk "
          f"{kern_ms * 1e3:.1f} us ({achieved / PEAK_GBPS:.3f} of peak), step {step_gbps:.0f} GB/s "
          f"({step_gbps / PEAK_GBPS:.3f} of peak)" + (f", mean accept {acc:.2f}" if acc is not None else ""),
          file=sys.stderr, flush=True)
    cfg = dict(f["config"])
    cfg.update({"timed_launch": "median of single-step graph replays", "p50_ms": ms, "p90_ms": p90,
                "min_ms": min(times), "one_graph_ms_per_step": one_graph_ms, "eager_ms_per_step": eager_ms,
                "step_GBps_algorithmic": step_gbps, "step_algorithmic_bytes": total_bytes})
    if acc is not None:
        cfg["mean_accept"] = acc
    line = {
        "metric": METRIC,
        "value": f["rows"] / (ms * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f["dtype"],
        "data": "synthetic",
        "config": cfg,
        "roofline": {
            "bound": "hbm", "achieved": achieved, "peak": PEAK_GBPS, "unit": "GB/s",
            "frac": achieved / PEAK_GBPS, "traffic": committed_traffic(f["name"]),
            "kernel": f["kernel"], "kernel_us": kern_ms * 1e3, "algorithmic_bytes": chunk_bytes,
            "step_frac": step_gbps / PEAK_GBPS,
        },
    }
    if not args.no_cpu_baseline:
        if args.config == 1:
            line["cpu_baseline"] = cpu_greedy_baseline(f["batch"])
        elif args.config == 2:
            line["cpu_baseline"] = cpu_topk_baseline(f["x"], args.k)
        else:
            line["cpu_baseline"] = cpu_verify_baseline(f["batch"])
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
