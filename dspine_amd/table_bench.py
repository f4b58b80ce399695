"""Timing of the draft-side sampling table at a serving shape on one GPU: bs 64 requests x T 16
(n = 960 block rows), K 16 lanes, H 4096, R 512, C 1024, V 151936, random bf16 / float32 inputs
of those shapes (no checkpoint).  Prints one JSON line: microseconds per call and the matrix-core
rate against MI355X's dense peak -- serial_rs_table in float32 (157.3 TFLOP/s), or with
``--factor`` the factorized table in float64 (78.6 TFLOP/s; vocabulary 32768 there, the one-time
cache build timed and reported beside it).

    python -m dspine_amd.table_bench [--calls N] [--factor]
"""

import argparse
import json
import math

import torch

PEAK_TFLOPS = 157.3
PEAK_F64_TFLOPS = 78.6


def flops(n, K, H, R, C):
    """2 x multiply-adds of the three products: senders x [pg; pv], msg x write_w, and the dot
    products with the candidates' head rows."""
    Ns = n * K
    return 2.0 * (Ns * C * 2 * R + Ns * R * H + n * K * K * H)


def factor_flops(n, K, H, R):
    """2 x multiply-adds of the float64 matrix-core products of the factorized table: x W,
    m Gram and m . TG (the base dot products and messages run on the vector units)."""
    return 2.0 * n * (H * R + K * R * R + K * K * R)


def main():
    from dspine_amd.kernels.dspine import serial_rs_table

    ap = argparse.ArgumentParser()
    ap.add_argument("--calls", type=int, default=50)
    ap.add_argument("--factor", action="store_true", help="time the factorized float64 table instead")
    args = ap.parse_args()
    dev = torch.device("cuda:0")
    # (the factorized table's per-round cost does not depend on the vocabulary, only its one-time
    # cache build does: 32768 rows keep that build short)
    bs, T, K, H, R, C, V = 64, 16, 16, 4096, 512, 1024, 32768 if args.factor else 151936
    m, n = bs * T, bs * (T - 1)
    g = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16

    def rnd(*shape, scale=1.0, dtype=bf):
        return (torch.randn(*shape, generator=g, device=dev) * scale).to(dtype)

    raw, packed = rnd(m, H), rnd(m, 3 * R)
    rms = torch.rand(m, generator=g, device=dev) + 0.5
    codebook = rnd(V, C, scale=1 / math.sqrt(C))
    pg, pv = rnd(R, C, scale=1 / math.sqrt(C), dtype=torch.float32), rnd(R, C, scale=1 / math.sqrt(C), dtype=torch.float32)
    gb = rnd(R, scale=0.1, dtype=torch.float32)
    w_last = rnd(H, R, scale=1 / math.sqrt(R), dtype=torch.float32)
    norm_w = 1 + rnd(H, scale=0.1, dtype=torch.float32)
    lm = rnd(V, H, scale=1 / math.sqrt(H))
    cand = torch.randint(0, V, (n, K), generator=g, device=dev).sort(-1).values
    anchors = torch.randint(0, V, (bs,), generator=g, device=dev)
    out = torch.empty((n, K, K), device=dev)
    if args.factor:
        factor_main(args, raw, rms, packed, anchors, cand, codebook, pg, pv, gb, w_last, norm_w, lm, out, T)
        return

    def call():
        serial_rs_table(raw, rms, packed, anchors, cand, codebook, pg, pv, gb, w_last, norm_w, lm, 1e-6, T, out=out)

    for _ in range(3):
        call()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.calls):
        call()
    e.record()
    torch.cuda.synchronize()
    us = s.elapsed_time(e) * 1e3 / args.calls
    f = flops(n, K, H, R, C)
    print(json.dumps({"workload": "serial_rs_table bs 64 x T 16, K 16, H 4096, R 512, C 1024, V 151936",
                      "us_per_call": us, "gflop": f / 1e9, "tflops": f / (us * 1e-6) / 1e12,
                      "peak_tflops": PEAK_TFLOPS, "frac": f / (us * 1e-6) / 1e12 / PEAK_TFLOPS}))


def factor_main(args, raw, rms, packed, anchors, cand, codebook, pg, pv, gb, w_last, norm_w, lm, out, T):
    from dspine_amd.sampling.factorized.kernels import Workspace, build_cache, factor_table

    dev = raw.device
    n, K = cand.shape
    H, R = raw.shape[1], pg.shape[0]
    query = packed[:, :R].contiguous()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    cache = build_cache(codebook, pg, pv, gb, w_last, norm_w, lm)
    e.record()
    torch.cuda.synchronize()
    build_ms = s.elapsed_time(e)
    base = torch.empty((n, K), device=dev, dtype=torch.float64)
    ws = Workspace.allocate(n, K, H, R, dev)

    def call():
        factor_table(raw, rms, query, anchors, cand, cache, 1e-6, T, out, base, ws)

    for _ in range(3):
        call()
    torch.cuda.synchronize()
    s.record()
    for _ in range(args.calls):
        call()
    e.record()
    torch.cuda.synchronize()
    us = s.elapsed_time(e) * 1e3 / args.calls
    f = factor_flops(n, K, H, R)
    print(json.dumps({"workload": f"factor_table (float64) bs {n // (T - 1)} x T {T}, K {K}, H {H}, R {R}, "
                                  f"V {lm.shape[0]}", "us_per_call": us, "gflop": f / 1e9,
                      "tflops": f / (us * 1e-6) / 1e12, "peak_tflops": PEAK_F64_TFLOPS,
                      "frac": f / (us * 1e-6) / 1e12 / PEAK_F64_TFLOPS, "cache_build_ms": build_ms,
                      "unsafe_entries": int((~ws.safe).sum())}))


if __name__ == "__main__":
    main()
