"""Timing of the draft-side sampling table (serial_rs_table) at a serving shape on one GPU:
bs 64 requests x T 16 (n = 960 block rows), K 16 lanes, H 4096, R 512, C 1024, V 151936, random
bf16 / float32 inputs of those shapes (no checkpoint).  Prints one JSON line: microseconds per
call and the float32 matrix-core rate against MI355X's dense fp32 MFMA peak (157.3 TFLOP/s).

    python -m dspine_amd.table_bench [--calls N]
"""

import argparse
import json
import math

import torch

PEAK_TFLOPS = 157.3


def flops(n, K, H, R, C):
    """2 x multiply-adds of the three products: senders x [pg; pv], msg x write_w, and the dot
    products with the candidates' head rows."""
    Ns = n * K
    return 2.0 * (Ns * C * 2 * R + Ns * R * H + n * K * K * H)


def main():
    from dspine_amd.kernels.dspine import serial_rs_table

    ap = argparse.ArgumentParser()
    ap.add_argument("--calls", type=int, default=50)
    args = ap.parse_args()
    dev = torch.device("cuda:0")
    bs, T, K, H, R, C, V = 64, 16, 16, 4096, 512, 1024, 151936
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


if __name__ == "__main__":
    main()
