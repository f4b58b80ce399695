"""Write the golden verification fixtures: the five benchmark workloads at reduced size
(V = 1031, a few requests), their inputs and the oracle's outputs, as .npz files beside this
script (loaded with allow_pickle=False).

    python tests/golden/make_golden.py

Inputs come from the seeded generators of dspine_amd.workloads; expected outputs from
oracle/verify_oracle.py (exact float64 softmax for the sampled cases).  bf16 logits are stored
as their 16-bit patterns.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from dspine_amd import workloads as W  # noqa: E402
import oracle.verify_oracle as O  # noqa: E402

V = 1031


def logits_arrays(x):
    if x.dtype == torch.bfloat16:
        return {"logits_bits": x.contiguous().view(torch.int16).numpy(), "logits_dtype": np.array("bf16")}
    return {"logits_f32": x.float().numpy(), "logits_dtype": np.array("f32")}


def info_arrays(info):
    return {"temperatures": info.temperatures.reshape(-1).numpy(), "top_ks": info.top_ks.numpy(),
            "top_ps": info.top_ps.numpy(), "min_ps": info.min_ps.numpy(),
            "flags": np.array([info.need_top_k_sampling, info.need_top_p_sampling, info.need_min_p_sampling,
                               info.is_any_greedy], dtype=np.int32),
            "max_top_k": np.array(info.max_top_k, dtype=np.int64)}


def sampled_case(batch, name):
    bs, T = batch["candidates"].shape
    lens = batch.get("verify_lens")
    lens = np.full(bs, T, np.int32) if lens is None else lens.numpy()
    offs = batch.get("row_offsets")
    ref = O.verify_step(batch["logits"], batch["info"], candidates=batch["candidates"].numpy(),
                        q_ids=batch["q_ids"].numpy(), q_values=batch["q_values"].numpy(), verify_lens=lens,
                        uniforms=batch["uniforms"].numpy(), uniform_final=batch["uniform_final"].numpy(),
                        prefix_lens=batch["prefix_lens"].numpy(), hist_ids=batch.get("hist_ids"),
                        presence=batch.get("presence"), repetition=batch.get("repetition"),
                        page_table=batch.get("page_table"), row_offsets=None if offs is None else offs.numpy(),
                        exact_softmax=True)
    arrays = {"kind": np.array("sampled"), **logits_arrays(batch["logits"]), **info_arrays(batch["info"]),
              "candidates": batch["candidates"].numpy(), "q_ids": batch["q_ids"].numpy(),
              "q_values": batch["q_values"].numpy(), "uniforms": batch["uniforms"].numpy(),
              "uniform_final": batch["uniform_final"].numpy(), "prefix_lens": batch["prefix_lens"].numpy(),
              "verify_lens": lens.astype(np.int32)}
    if offs is not None:
        arrays["row_offsets"] = offs.numpy()
    for key in ("hist_ids", "presence", "repetition", "page_table"):
        if batch.get(key) is not None:
            arrays[key] = batch[key].numpy()
    for key in ("accept", "commit", "bonus", "output", "new_seq", "margins"):
        arrays["expect_" + key] = ref[key]
    if ref["kv_slots"] is not None:
        arrays["expect_kv_slots"] = ref["kv_slots"]
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)


def main():
    torch.manual_seed(0)
    # 1. greedy verification, 1 x 17 rows fp32 N(0, 3^2), one forced mismatch
    g = W.greedy_round(V=V, seed=1)
    top1 = O.argmax_rows(g["logits"])
    out = O.greedy_accept(top1, g["candidates"].numpy(), [17], g["prefix_lens"].numpy())
    np.savez_compressed(os.path.join(HERE, "greedy_1x17.npz"), kind=np.array("greedy"), **logits_arrays(g["logits"]),
                        candidates=g["candidates"].numpy(), prefix_lens=g["prefix_lens"].numpy(),
                        expect_accept=out[0], expect_commit=out[1], expect_bonus=out[2], expect_output=out[3],
                        expect_new_seq=out[4])
    # 2. top-k rows: bf16 with planted peaks and exact duplicates, k in {1, 20, 64}
    t = W.topk_rows(rows=24, V=V, seed=2, peaks=32, dup_frac=0.05)
    arrays = {"kind": np.array("topk"), **logits_arrays(t["logits"])}
    for k in (1, 20, 64):
        vals, ids = O.topk(t["logits"].float(), k)
        arrays[f"expect_ids_{k}"] = ids.numpy()
        arrays[f"expect_values_{k}"] = vals.numpy()
    np.savez_compressed(os.path.join(HERE, "topk_24rows.npz"), **arrays)
    # 3. stochastic rejection, fp32, T=1, top-k 20, top-p 0.95, sigma 0.5 and 1.5
    for sigma in (0.5, 1.5):
        sampled_case(W.rejection_round(bs=4, V=V, sigma_draft=sigma, seed=3), f"rejection_sigma{sigma}")
    # 4. serving mix: bf16, temperatures {0, 0.6, 1}, top-k {off, 20}, top-p {1, 0.95}, penalties
    sampled_case(W.serving_round(bs=6, V=V, seed=10, hist_len=64), "serving_6x17")
    # 5. ragged, heavy-tailed bf16, top-p 0.9, verify lengths 4..16
    sampled_case(W.ragged_round(bs=5, V=V, seed=5), "ragged_5")
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
