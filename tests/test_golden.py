"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py):
the five benchmark workloads at reduced size with their expected outputs.  On the CPU the
oracle must still produce them; on the GPU the HIP path must (integer outputs bit-exact; a
request whose recorded decision margin is below MARGIN may differ)."""

import glob
import os
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import parity
from parity import MARGIN

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = sorted(os.path.basename(f)[:-4] for f in glob.glob(os.path.join(HERE, "*.npz")))


def load(name):
    z = np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False)
    return {k: z[k] for k in z.files}


def logits_of(z):
    if str(z["logits_dtype"]) == "bf16":
        return torch.from_numpy(z["logits_bits"]).view(torch.bfloat16)
    return torch.from_numpy(z["logits_f32"])


def info_of(z):
    f = z["flags"]
    return SimpleNamespace(temperatures=torch.from_numpy(z["temperatures"]).view(-1, 1),
                           top_ks=torch.from_numpy(z["top_ks"]), top_ps=torch.from_numpy(z["top_ps"]),
                           min_ps=torch.from_numpy(z["min_ps"]), need_top_k_sampling=bool(f[0]),
                           need_top_p_sampling=bool(f[1]), need_min_p_sampling=bool(f[2]), is_any_greedy=bool(f[3]),
                           is_all_greedy=False, max_top_k=int(z["max_top_k"]))


def oracle_outputs(z):
    import oracle.verify_oracle as O

    kind = str(z["kind"])
    x = logits_of(z)
    if kind == "greedy":
        out = O.greedy_accept(O.argmax_rows(x), z["candidates"], [z["candidates"].shape[1]], z["prefix_lens"])
        return dict(zip(("accept", "commit", "bonus", "output", "new_seq"), out))
    if kind == "topk":
        res = {}
        for k in (1, 20, 64):
            vals, ids = O.topk(x.float(), k)
            res[f"ids_{k}"], res[f"values_{k}"] = ids.numpy(), vals.numpy()
        return res
    return O.verify_step(x, info_of(z), candidates=z["candidates"], q_ids=z["q_ids"], q_values=z["q_values"],
                         verify_lens=z["verify_lens"], uniforms=z["uniforms"], uniform_final=z["uniform_final"],
                         prefix_lens=z["prefix_lens"], hist_ids=_t(z, "hist_ids"), presence=_t(z, "presence"),
                         repetition=_t(z, "repetition"), page_table=_t(z, "page_table"),
                         row_offsets=z.get("row_offsets"), exact_softmax=True)


def _t(z, key):
    return torch.from_numpy(z[key]) if key in z else None


def test_golden_fixtures_present():
    assert {"greedy_1x17", "topk_24rows", "rejection_sigma0.5", "rejection_sigma1.5", "serving_6x17",
            "ragged_5"} <= set(CASES)


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_golden(name):
    z = load(name)
    got = oracle_outputs(z)
    for key, want in z.items():
        if not key.startswith("expect_"):
            continue
        k = key[len("expect_"):]
        assert np.array_equal(np.asarray(got[k]), want), (name, k)


def _compare(name, z, got, names):
    margins = z.get("expect_margins")
    n = z["expect_" + names[0]].shape[0]
    differing = []
    for b in range(n):
        same = all(np.array_equal(got[k][b], z["expect_" + k][b]) for k in names)
        if not same:
            assert margins is not None and margins[b] < MARGIN, (name, b, {k: got[k][b] for k in names},
                                                                 {k: z["expect_" + k][b] for k in names})
            differing.append((b, float(margins[b])))
    near = 0 if margins is None else int((margins < MARGIN).sum())
    parity.record(f"golden {name}", n, near, differing)


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_hip_matches_golden(device, name):
    z = load(name)
    kind = str(z["kind"])
    x = logits_of(z).to(device)
    if kind == "topk":
        from dspine_amd.kernels.dspine import topk

        for k in (1, 20, 64):
            vals, ids = topk(x, k)
            torch.cuda.synchronize()
            assert np.array_equal(ids.cpu().numpy(), z[f"expect_ids_{k}"]), k
            assert np.array_equal(vals.cpu().numpy(), z[f"expect_values_{k}"]), k
        return
    names = ("accept", "commit", "bonus", "output", "new_seq")
    if kind == "greedy":
        from dspine_amd.verification.caps import accept_greedy

        outs = accept_greedy(candidates=torch.from_numpy(z["candidates"]).to(device), next_token_logits=x,
                             prefix_lens=torch.from_numpy(z["prefix_lens"]).to(device))
        torch.cuda.synchronize()
        _compare(name, z, {n: t.cpu().numpy() for n, t in zip(names, outs)}, names)
        return
    from dspine_amd import workloads as W
    from dspine_amd.verify import History, verify_step

    dev = lambda key: torch.from_numpy(z[key]).to(device) if key in z else None  # noqa: E731
    hist = None
    if "hist_ids" in z:
        hist = History(dev("hist_ids"), dev("presence"), dev("repetition"))
    outs, kv = verify_step(logits=x, sampling_info=W.info_to(info_of(z), device), candidates=dev("candidates"),
                           q_ids=dev("q_ids"), q_values=dev("q_values"), uniforms=dev("uniforms"),
                           uniform_final=dev("uniform_final"), prefix_lens=dev("prefix_lens"),
                           verify_lens=dev("verify_lens"), row_offsets=dev("row_offsets"), history=hist,
                           page_table=dev("page_table"))
    torch.cuda.synchronize()
    got = {n: t.cpu().numpy() for n, t in zip(names, outs)}
    if kv is not None and "expect_kv_slots" in z:
        got["kv_slots"] = kv.cpu().numpy()
        names = names + ("kv_slots",)
    _compare(name, z, got, names)
