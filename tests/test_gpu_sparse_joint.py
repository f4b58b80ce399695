"""The sparse joint target inside the fused verify step, against the oracle routed as the
reference routes.

For flashinfer batches that ``build_sparse_target`` accepts (no min-p, no greedy rows, a
host-known max top-k <= 32) with the reference's 16 q lanes, ``TargetDistribution.sample_prefix``
verifies against the sparse joint target (sampling/target.py:53-66, sampling/sparse/target.py:
95-178): every value tied with the k-th is kept, the nucleus tests the mass of the strictly
larger p, and a row keeping more than 32 values becomes the dense row of every p >= p_(k).  bf16
logits tie at the k-th value on most top-k rows, and the integer-valued rows of the workload keep
hundreds (dense rows).  Integer outputs must equal the oracle's (tests/parity.py for
near-margin requests).
"""

import numpy as np
import pytest
import torch

import parity
from dspine_amd import workloads as W

pytestmark = pytest.mark.gpu

NAMES = ("accept", "commit", "bonus", "output", "new_seq")


def _O():
    import oracle.verify_oracle as O

    return O


def _gpu(batch, device, sparse_joint=True, backend="flashinfer"):
    from dspine_amd.verify import History, verify_step

    d = W.to_device(batch, device)
    hist = History(d["hist_ids"], d["presence"], d["repetition"]) if "hist_ids" in d else None
    outs, _ = verify_step(
        logits=d["logits"], sampling_info=d["info"], candidates=d["candidates"], q_ids=d["q_ids"],
        q_values=d["q_values"], uniforms=d["uniforms"], uniform_final=d["uniform_final"],
        prefix_lens=d["prefix_lens"], verify_lens=d.get("verify_lens"), row_offsets=d.get("row_offsets"),
        history=hist, sampling_backend=backend, sparse_joint=sparse_joint)
    torch.cuda.synchronize()
    return {n: t.cpu().numpy() for n, t in zip(NAMES, outs)}


def _oracle(batch, sparse_joint=True, exact_softmax=True):
    O = _O()
    bs, T = batch["candidates"].shape
    lens = batch.get("verify_lens")
    lens = np.full(bs, T) if lens is None else lens.numpy()
    return O.verify_step(
        batch["logits"], batch["info"], candidates=batch["candidates"].numpy(), q_ids=batch["q_ids"].numpy(),
        q_values=batch["q_values"].numpy(), verify_lens=lens, uniforms=batch["uniforms"].numpy(),
        uniform_final=batch["uniform_final"].numpy(), prefix_lens=batch["prefix_lens"].numpy(),
        hist_ids=batch.get("hist_ids"), presence=batch.get("presence"), repetition=batch.get("repetition"),
        row_offsets=None if batch.get("row_offsets") is None else batch["row_offsets"].numpy(),
        sampling_backend="flashinfer", exact_softmax=exact_softmax, sparse_joint=sparse_joint)


def _tie_stats(ref, batch):
    """(rows tied at the k-th value, dense rows: more than 32 kept) of the oracle's verified rows."""
    info = batch["info"]
    T = batch["candidates"].shape[1]
    offs = None if batch.get("row_offsets") is None else batch["row_offsets"].numpy()
    tied = 0
    for r in ref["probs"]:
        b = r // T if offs is None else int(np.searchsorted(offs, r, side="right") - 1)
        k = int(info.top_ks[b])
        top = np.sort(ref["adjusted"][r].float().numpy())[::-1]
        tied += int((top == top[k - 1]).sum() > 1)
    dense = int(np.asarray(ref["packed"][3]).sum())
    return tied, dense


def test_sparse_joint_full_vocab(device):
    """24 requests x 16 rows x 151936 bf16 (the reference's block and q width), top-k {8, 20,
    32}, top-p {1, 0.95, 0.6}, penalties; a quarter of the requests with integer-valued logits
    (dense rows).  Every request against the oracle's sparse route."""
    batch = W.sparse_round()
    bs = batch["candidates"].shape[0]
    assert _O().sparse_route(batch["info"], "flashinfer", batch["logits"].shape[1], batch["q_ids"].shape[-1])
    ref = _oracle(batch)
    tied, dense = _tie_stats(ref, batch)
    assert tied > 100 and dense > 20, (tied, dense)  # the case exercises both
    got = _gpu(batch, device)
    tag = f"sparse joint 24x16x151936 bf16 (tied rows {tied}, dense {dense})"
    parity.compare_requests(got, ref, range(bs), tag, extra=())
    parity.compare_literal(got, _oracle(batch, exact_softmax=False), ref, range(bs), tag)
    # the route matters: the rank-based flashinfer filter differs on some of these requests
    rank = _oracle(batch, sparse_joint=False)
    assert any(not np.array_equal(rank[n], ref[n]) for n in ("accept", "bonus")), "the case should tell the routes apart"


def test_sparse_joint_full_vocab_f32(device):
    """The same route on float32 logits at the full vocabulary (12 requests x 16 rows x 151936,
    13 chunks a row), a third of the requests integer-valued: every request against the oracle,
    exact and literal softmax."""
    batch = W.sparse_round(bs=12, seed=8, coarse_every=3, dtype=torch.float32)
    bs = batch["candidates"].shape[0]
    assert _O().sparse_route(batch["info"], "flashinfer", batch["logits"].shape[1], batch["q_ids"].shape[-1])
    ref = _oracle(batch)
    tied, dense = _tie_stats(ref, batch)
    assert dense > 10, (tied, dense)
    got = _gpu(batch, device)
    tag = f"sparse joint 12x16x151936 fp32 (tied rows {tied}, dense {dense})"
    parity.compare_requests(got, ref, range(bs), tag, extra=())
    parity.compare_literal(got, _oracle(batch, exact_softmax=False), ref, range(bs), tag)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("seed", [1, 2])
def test_sparse_joint_small(device, dtype, seed):
    """Shorter rows (V 20011, several chunks), both logit types, T 16 and verify lengths."""
    batch = W.sparse_round(bs=16, V=20011, seed=20 + seed, coarse_every=3, dtype=dtype)
    g = torch.Generator().manual_seed(seed)
    batch["verify_lens"] = torch.randint(1, 17, (16,), generator=g, dtype=torch.int64).to(torch.int32)
    ref = _oracle(batch)
    got = _gpu(batch, device)
    parity.compare_requests(got, ref, range(16), f"sparse joint small {dtype} seed={seed}", extra=())


def test_sparse_joint_ragged(device):
    """Compact rows with row offsets (verify lengths 1..16), bf16, V 151936."""
    full = W.sparse_round(bs=12, seed=31, coarse_every=3)
    bs, T = full["candidates"].shape
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(1, T + 1, (bs,), generator=g, dtype=torch.int64)
    offs = torch.cat((torch.zeros(1, dtype=torch.int64), lens.cumsum(0)))[:-1]
    rows = torch.cat([full["logits"][b * T: b * T + int(lens[b])] for b in range(bs)])
    batch = dict(full, logits=rows, verify_lens=lens.to(torch.int32), row_offsets=offs)
    ref = _oracle(batch)
    got = _gpu(batch, device)
    parity.compare_requests(got, ref, range(bs), "sparse joint ragged bf16", extra=())


def test_sparse_joint_through_target_distribution(device):
    """TargetDistribution.sample_prefix takes the route by itself (flashinfer worker, 16 q lanes)."""
    from dspine_amd.runtime import worker as Wk
    from dspine_amd.sampling.random import RequestRNG

    O = _O()
    batch = W.sparse_round(bs=8, V=30011, seed=41, coarse_every=4)
    bs, T = batch["candidates"].shape
    seeds = torch.arange(bs, dtype=torch.int64) * 7919 + 5
    positions = batch["prefix_lens"].to(torch.int64) + 2
    rng = RequestRNG()
    rng.stage(seeds.to(device), positions.to(device))
    wk = Wk.VerifyWorker(T, device, k=16, sampling_backend="flashinfer", random=rng)
    wk._dspine_sampler.stage(batch["q_ids"].to(device), batch["q_values"].to(device))
    logits = batch["logits"].clone()
    outs = wk.target_distribution.sample_prefix(
        candidates=batch["candidates"].to(device), next_token_logits=logits.to(device),
        sampling_info=W.info_to(batch["info"], device), prefix_lens=batch["prefix_lens"].to(device), bs=bs,
        verify_lens=torch.full((bs,), T, dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    got = {n: t.cpu().numpy() for n, t in zip(NAMES, outs)}
    u_acc = O.seeded_uniforms(seeds.numpy(), positions.numpy(), T - 1, O.ACCEPT)
    u_fin = O.seeded_uniforms(seeds.numpy(), positions.numpy(), 1, O.BONUS).reshape(-1)
    ref = O.verify_step(logits, batch["info"], candidates=batch["candidates"].numpy(),
                        q_ids=batch["q_ids"].numpy(), q_values=batch["q_values"].numpy(),
                        verify_lens=np.full(bs, T), uniforms=u_acc, uniform_final=u_fin,
                        prefix_lens=batch["prefix_lens"].numpy(), sampling_backend="flashinfer",
                        exact_softmax=True, sparse_joint=True)
    parity.compare_requests(got, ref, range(bs), "sparse joint via TargetDistribution", extra=())


def test_sparse_joint_contract(device):
    """The C ABI refuses the sparse joint target outside its batches (ValueError before launch)."""
    batch = W.sparse_round(bs=4, V=4099, seed=7)
    for info in (W.sampling_info([1.0] * 4, [20, 8, 0, 8], [0.9] * 4),          # top-k off
                 W.sampling_info([1.0, 0.0, 1.0, 1.0], [20, 8, 8, 8], [0.9] * 4)):  # a greedy row
        with pytest.raises(ValueError, match="sparse joint"):
            _gpu(dict(batch, info=info), device)
    with pytest.raises(ValueError, match="sparse joint"):
        _gpu(batch, device, backend="pytorch")
