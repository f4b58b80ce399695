"""Timing of the path's other entry points at the serving shape on one GPU: 64 requests x 17
rows x 151936 (the verify step's batch, bf16 logits), each entry point called on its own
inputs of that shape.  Prints one JSON line per entry point: microseconds per call (HIP events
over the calls on the current stream), and for the HBM-bound ones the algorithmic bytes per call
and their fraction of MI355X's 8 TB/s.

    python -m dspine_amd.entry_bench [--calls N]

Algorithmic bytes (the least any implementation moves):
  target_probs     logits read once + P written: 2 + 4 bytes per bf16 logit
  filter_target_probs  the given P read once + the filtered P written: 4 + 4 bytes per element
  compress_probs   the P a row's result depends on, 4 bytes per element: the whole row when it
                   keeps at most `capacity` ids (every value is checked for negative, NaN or
                   infinite p), else up to its (capacity + 1)-th kept id, where the row is known
                   to overflow (counted from the P of the run, to the pass's 4096-id tile)
  adjust_logits    logits read and written: 2 + 2 bytes per logit, plus one float32 penalty row
                   per request (read once, reused by the request's rows)
  chain_on_probs   P of the accepted row read once for the bonus draw (4 bytes per element);
                   the draft tests read one value a row
Two torch references give this part's practical rates: a fill of P (write only) and a copy of
the logits (read + write).
The planner, the commit, the uniforms and the window index move KBs and are timed only.
"""

import argparse
import json
from types import SimpleNamespace

import torch

PEAK_GBPS = 8000.0


def timed(fn, calls, warm=3):
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(calls):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / calls * 1e3


def line(name, us, nbytes=None, **extra):
    rec = {"entry": name, "us_per_call": round(us, 2)}
    if nbytes is not None:
        gbps = nbytes / (us * 1e-6) / 1e9
        rec.update(algorithmic_bytes=int(nbytes), GBps=round(gbps, 1), frac=round(gbps / PEAK_GBPS, 3))
    rec.update(extra)
    print(json.dumps(rec), flush=True)


def main():
    from dspine_amd import workloads as W
    from dspine_amd.runtime.worker import SoftmaxTemp, chain_on_probs, commit_accept, filter_probs
    from dspine_amd.sampling.compact import adjust_history, adjust_logits
    from dspine_amd.sampling.random import seeded_uniforms
    from dspine_amd.sampling.sparse.accept import compress_probs
    from dspine_amd.verification.sps import allocate_verify_lens, window_index
    from dspine_amd.verify import new_outputs, target_probs

    ap = argparse.ArgumentParser()
    ap.add_argument("--calls", type=int, default=20)
    args = ap.parse_args()
    dev = torch.device("cuda:0")
    batch = W.serving_round()
    d = W.to_device(batch, dev)
    info = d["info"]
    info.temperatures = info.temperatures.reshape(-1).contiguous()
    logits = d["logits"]
    bs, T = batch["candidates"].shape
    rows, V = logits.shape
    n_logits = rows * V

    # a1: dense target P
    P = torch.empty((rows, V), device=dev, dtype=torch.float32)
    us = timed(lambda: target_probs(logits, info, bs=bs, T=T, out=P), args.calls)
    line("target_probs", us, n_logits * 6, shape=[rows, V], logits="bf16")

    # the write rate of this part for reference: a plain fill of P (torch), and the dense P of
    # an all-greedy batch (one-hot rows: the writes of k_dense_p alone)
    us = timed(lambda: P.zero_(), args.calls)
    line("fill_P_reference", us, n_logits * 4, shape=[rows, V])
    g_info = W.info_to(W.sampling_info([0.0] * bs, [0] * bs, [1.0] * bs), dev)
    g_info.temperatures = g_info.temperatures.reshape(-1).contiguous()
    us = timed(lambda: target_probs(logits, g_info, bs=bs, T=T, out=P), args.calls)
    line("target_probs_greedy_rows", us, n_logits * 4 + n_logits * 2, shape=[rows, V])

    # a2: the backend filter on given probabilities (runtime/worker.py:473-508): the softmax of
    # the same logits (temperatures at least 0.5), filtered with the requests' top-k / top-p
    temps = torch.repeat_interleave(info.temperatures.clamp_min(0.5), T)
    probs = SoftmaxTemp.execute(logits=logits, temperatures=temps, rows_per_request=1)
    F = torch.empty_like(P)
    us = timed(lambda: filter_probs(probs, info, bs=bs, T=T, sampling_backend="pytorch", out=F), args.calls)
    line("filter_target_probs", us, n_logits * 8, shape=[rows, V], probs="float32")
    del probs, F
    target_probs(logits, info, bs=bs, T=T, out=P)

    # a9: p > 0 compaction of that P
    cap = 64
    us = timed(lambda: compress_probs(torch, P, cap), args.calls)
    kept = (P > 0).to(torch.int32).cumsum(1, dtype=torch.int32)
    over = kept[:, -1] > cap
    at = (kept > cap).to(torch.int8).argmax(1)  # the (capacity + 1)-th kept id of an overflowing row
    need = torch.where(over, torch.clamp((at // 4096 + 1) * 4096, max=V), torch.full_like(at, V))
    del kept
    line("compress_probs", us, int(need.sum()) * 4, shape=[rows, V], capacity=cap,
         rows_overflowing=int(over.sum()), full_read_frac=round(n_logits * 4 / (us * 1e-6) / 1e9 / PEAK_GBPS, 3))

    # a5: chain rejection with the draft's sparse q against that P
    outs, _ = new_outputs(bs, T, dev, kv_slots=False)
    vl = torch.full((bs,), T, device=dev, dtype=torch.int32)

    def chain():
        chain_on_probs(candidates=d["candidates"], probs=P, q_ids=d["q_ids"], q_values=d["q_values"],
                       verify_lens=vl, uniforms=d["uniforms"], uniform_final=d["uniform_final"],
                       prefix_lens=d["prefix_lens"], outputs=outs)

    us = timed(chain, args.calls)
    line("chain_on_probs", us, bs * V * 4, requests=bs, mean_accept=round(float(outs[0].float().mean()), 2))

    # a14: an additive penalty row per request applied to the logits in place (on a copy): the
    # full block as [bs, T, V] (sampling/compact.py:116) and compact rows with a row map (:99)
    work = logits.clone()
    pen = torch.randn((bs, V), device=dev) * 0.1
    info_pen = SimpleNamespace(acc_additive_penalties=pen)
    us = timed(lambda: adjust_logits(work.view(bs, T, V), info_pen, None), args.calls)
    line("adjust_logits", us, n_logits * 4 + bs * V * 4, shape=[bs, T, V], op="additive")
    # the read + write rate of this part for reference: torch's copy of the same logits
    us = timed(lambda: work.copy_(logits), args.calls)
    line("copy_logits_reference", us, n_logits * 4, shape=[rows, V], logits="bf16")
    rtr = torch.arange(rows, device=dev) // T
    us = timed(lambda: adjust_logits(work, info_pen, rtr), args.calls)
    line("adjust_logits_row_map", us, n_logits * 4 + bs * V * 4, shape=[rows, V], op="additive")

    us = timed(lambda: adjust_history(work, d["hist_ids"], d["presence"], d["repetition"], rtr), args.calls)
    line("adjust_history", us, None, history=int(d["hist_ids"].shape[1]))

    # a13 / a16 / f2 / f3: KB-sized work, timed only
    seeds = torch.randint(0, 1 << 62, (bs,), device=dev)
    pos = torch.randint(0, 4096, (bs,), device=dev)
    us = timed(lambda: seeded_uniforms(seeds, pos, T - 1, 0), args.calls)
    line("seeded_uniforms", us, None, n=bs, width=T - 1)

    lens = torch.randint(1, T + 1, (bs,), device=dev, dtype=torch.int32)
    qo = torch.zeros(bs + 1, device=dev, dtype=torch.int32)
    qo[1:] = lens.cumsum(0)
    total = int(qo[-1])
    us = timed(lambda: window_index(qo, T, total), args.calls)
    line("window_index", us, None, requests=bs, total=total)

    g = torch.Generator(device=dev).manual_seed(3)
    raw = torch.rand((bs, T - 1), generator=g, device=dev)
    table = torch.rand((T - 1, 64), generator=g, device=dev)
    depth = torch.arange(T - 1, device=dev)
    budget = bs * 6
    us = timed(lambda: allocate_verify_lens(raw, table, depth, budget), args.calls)
    line("allocate_verify_lens", us, None, requests=bs, positions=T - 1, budget=budget)

    pool, cols = bs + 8, 8192
    req_to_token = torch.zeros((pool, cols), device=dev, dtype=torch.int32)
    ocl = torch.randperm(1 << 20, device=dev)[: bs * T].to(torch.int64)
    seq = torch.zeros(pool, device=dev, dtype=torch.int64)
    accept = torch.randint(0, T, (bs,), device=dev, dtype=torch.int32)
    c_outs = (accept, None, None, torch.empty((bs, T), device=dev, dtype=torch.int64), None)
    req_rows = torch.randperm(pool, device=dev)[:bs]
    us = timed(lambda: commit_accept(c_outs, prefix_lens=d["prefix_lens"], req_pool_indices=req_rows,
                                     req_to_token=req_to_token, out_cache_loc=ocl, verify_lens=None,
                                     seq_lens=seq), args.calls)
    line("commit_accept", us, None, requests=bs, T=T)


if __name__ == "__main__":
    main()
