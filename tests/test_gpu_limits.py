"""The fused verify step at the edges of its contract: one-row blocks (no drafts), the largest
vocabularies the row kernels take, the widest sparse q, and requests just past each limit
(refused before any launch).  Integer outputs must equal the oracle's (tests/parity.py for
near-margin requests)."""

import numpy as np
import pytest
import torch

import parity
from dspine_amd import workloads as W

pytestmark = pytest.mark.gpu

NAMES = ("accept", "commit", "bonus", "output", "new_seq")


def _gpu(batch, device, **kw):
    from dspine_amd.verify import History, verify_step

    d = W.to_device(batch, device)
    hist = History(d["hist_ids"], d["presence"], d["repetition"]) if "hist_ids" in d else None
    outs, kv = verify_step(
        logits=d["logits"], sampling_info=d["info"], candidates=d["candidates"], q_ids=d["q_ids"],
        q_values=d["q_values"], uniforms=d["uniforms"], uniform_final=d["uniform_final"],
        prefix_lens=d["prefix_lens"], verify_lens=d.get("verify_lens"), history=hist,
        page_table=d.get("page_table"), **kw)
    torch.cuda.synchronize()
    res = {n: t.cpu().numpy() for n, t in zip(NAMES, outs)}
    res["kv_slots"] = kv.cpu().numpy() if kv is not None else None
    return res


def _oracle(batch):
    import oracle.verify_oracle as O

    bs, T = batch["candidates"].shape
    lens = batch.get("verify_lens")
    return O.verify_step(
        batch["logits"], batch["info"], candidates=batch["candidates"].numpy(), q_ids=batch["q_ids"].numpy(),
        q_values=batch["q_values"].numpy(), verify_lens=np.full(bs, T) if lens is None else lens.numpy(),
        uniforms=batch["uniforms"].numpy(), uniform_final=batch["uniform_final"].numpy(),
        prefix_lens=batch["prefix_lens"].numpy(), hist_ids=batch.get("hist_ids"), presence=batch.get("presence"),
        repetition=batch.get("repetition"), page_table=batch.get("page_table"), exact_softmax=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_verify_one_row_blocks(device, dtype):
    """T = 1: every request is its anchor row alone (empty q and coins), so the accepted length
    is 0 and the bonus is drawn from the row's full target distribution (greedy, top-k, nucleus
    and unfiltered requests)."""
    batch = W.serving_round(bs=12, T=1, V=20011, seed=5, hist_len=24, dtype=dtype)
    got = _gpu(batch, device)
    ref = _oracle(batch)
    assert (ref["accept"] == 0).all()
    parity.compare_requests(got, ref, range(12), f"one-row blocks {dtype}")


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 655360), (torch.float32, 393216)])
def test_verify_largest_vocab(device, dtype, V):
    """The largest vocabulary of the row kernels (32 chunks a row: 655360 bf16 / 393216 float32
    values), mixed requests with penalties and KV slots."""
    batch = W.serving_round(bs=4, T=3, V=V, seed=6, K=8, hist_len=32, dtype=dtype)
    got = _gpu(batch, device)
    ref = _oracle(batch)
    parity.compare_requests(got, ref, range(4), f"largest vocab {V} {dtype}")


def test_verify_widest_q(device):
    """64 sparse-q lanes a draft (the widest the kernels take) on the serving mix's shape."""
    batch = W.serving_round(bs=6, T=5, V=30011, seed=7, K=64, hist_len=16)
    got = _gpu(batch, device)
    ref = _oracle(batch)
    parity.compare_requests(got, ref, range(6), "widest q (K 64)")


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 655361), (torch.float32, 393217)])
def test_verify_vocab_past_the_limit(device, dtype, V):
    """One value past the largest vocabulary: refused with NotImplementedError before a launch."""
    batch = W.serving_round(bs=2, T=2, V=V, seed=8, K=4, hist_len=8, dtype=dtype)
    with pytest.raises(NotImplementedError):
        _gpu(batch, device)


def test_verify_q_past_the_limit(device):
    """65 q lanes: refused with ValueError before a launch."""
    batch = W.serving_round(bs=2, T=3, V=4099, seed=9, K=65, hist_len=8)
    with pytest.raises(ValueError):
        _gpu(batch, device)
