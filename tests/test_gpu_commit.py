"""The commit of an accepted round on the GPU (``dsv_commit_accept``) against the oracle's
closed form, and the worker's double-buffered accept buffers around it: a round's outputs stay
intact while the next round is verified into the other buffer set (the discipline of the
reference's tests/test_tp_accept.py:155-180)."""

import numpy as np
import pytest
import torch

from dspine_amd import workloads as W

pytestmark = pytest.mark.gpu


def _O():
    import oracle.verify_oracle as O

    return O


@pytest.mark.parametrize("mode", ["window_slots", "in_table", "compact_slots"])
@pytest.mark.parametrize("bs", [1, 37, 3000])
def test_commit_matches_oracle(device, mode, bs):
    from dspine_amd.runtime.worker import commit_accept

    O = _O()
    T = 17
    g = torch.Generator().manual_seed(bs)
    acc = torch.randint(0, T, (bs,), generator=g, dtype=torch.int64).to(torch.int32)
    lens = torch.randint(1, T + 1, (bs,), generator=g, dtype=torch.int64).to(torch.int32)
    prefix = torch.randint(0, 200, (bs,), generator=g, dtype=torch.int64)
    prefix[0] = 210  # positions past the table's columns are not written
    pool = bs + 5
    rows = torch.randperm(pool, generator=g)[:bs]
    cols = 224
    ocl = torch.randperm(1 << 20, generator=g)[: bs * T].to(torch.int64)
    table = torch.randint(0, 1 << 20, (pool, cols), generator=g, dtype=torch.int64).to(torch.int32)
    offs = None
    if mode == "compact_slots":
        offs = torch.cat((torch.zeros(1, dtype=torch.int64), lens.to(torch.int64).cumsum(0)))[:-1]
        ocl = ocl[: int(lens.sum())].contiguous()
    if mode == "in_table":
        for b in range(min(bs, 64)):
            p = int(prefix[b])
            table[rows[b], p: min(cols, p + T)] = ocl[b * T: b * T + min(T, cols - p)].to(torch.int32)
    ref_table = table.numpy().copy()
    ref_seq = np.zeros(pool, np.int64)
    freed_ref = O.commit_accept(acc.numpy(), prefix.numpy(), rows.numpy(), ref_table, T,
                                out_cache_loc=None if mode == "in_table" else ocl.numpy(), verify_lens=lens.numpy(),
                                slot_offsets=None if offs is None else offs.numpy(), seq_lens=ref_seq)
    d_table = table.to(device)
    seq = torch.zeros(pool, dtype=torch.int64, device=device)
    outs = (acc.to(device), None, None, torch.empty((bs, T), device=device, dtype=torch.int64), None)
    free, count = commit_accept(outs, prefix_lens=prefix.to(device), req_pool_indices=rows.to(device),
                                req_to_token=d_table, out_cache_loc=None if mode == "in_table" else ocl.to(device),
                                verify_lens=lens.to(device), slot_offsets=None if offs is None else offs.to(device),
                                seq_lens=seq)
    torch.cuda.synchronize()
    n = int(count.item())
    assert n == freed_ref.size
    assert np.array_equal(free[:n].cpu().numpy(), freed_ref)
    assert np.array_equal(d_table.cpu().numpy(), ref_table)
    assert np.array_equal(seq.cpu().numpy(), ref_seq)


def test_commit_with_double_buffered_rounds(device):
    """Two sampled verify rounds through the worker: the first verify's outputs (the buffers the
    commit reads) keep their values while the second is verified into the other set, and each commit
    matches the oracle's closed form on that round's accept lengths."""
    from dspine_amd.runtime import worker as Wk
    from dspine_amd.verify import verify_step

    O = _O()
    bs, T, V, K = 6, 5, 4099, 4
    wk = Wk.VerifyWorker(T, device)
    rounds = []
    for seed in (1, 2):
        batch = W.serving_round(bs=bs, T=T, V=V, seed=seed, K=K, hist_len=8)
        d = W.to_device(batch, device)
        outs = wk._next_accept_bonus_buffers(bs)
        verify_step(logits=d["logits"], sampling_info=d["info"], candidates=d["candidates"], q_ids=d["q_ids"],
                    q_values=d["q_values"], uniforms=d["uniforms"], uniform_final=d["uniform_final"],
                    prefix_lens=d["prefix_lens"], outputs=outs)
        torch.cuda.synchronize()
        rounds.append((outs, tuple(t.clone() for t in outs), batch))
    (o1, saved1, b1), (o2, _, _) = rounds
    assert all(a.data_ptr() != b.data_ptr() for a, b in zip(o1, o2))
    for live, saved in zip(o1, saved1):  # the first verify's buffers were not touched by the second
        assert torch.equal(live, saved)
    table = torch.zeros((bs, 4200), dtype=torch.int32, device=device)
    seq = torch.zeros(bs, dtype=torch.int64, device=device)
    ocl = torch.arange(bs * T, dtype=torch.int64, device=device) + 7000
    rows = torch.arange(bs, device=device)
    free, count = Wk.commit_accept(o1, prefix_lens=b1["prefix_lens"].to(device), req_pool_indices=rows,
                                   req_to_token=table, out_cache_loc=ocl, seq_lens=seq)
    ref_table = np.zeros((bs, 4200), np.int32)
    ref_seq = np.zeros(bs, np.int64)
    freed = O.commit_accept(o1[0].cpu().numpy(), b1["prefix_lens"].numpy(), np.arange(bs), ref_table, T,
                            out_cache_loc=ocl.cpu().numpy(), seq_lens=ref_seq)
    torch.cuda.synchronize()
    assert np.array_equal(table.cpu().numpy(), ref_table)
    assert np.array_equal(seq.cpu().numpy(), ref_seq)
    assert seq.cpu().tolist() == [int(p) + int(a) + 1 for p, a in zip(b1["prefix_lens"], saved1[0].cpu())]
    assert np.array_equal(free[: int(count.item())].cpu().numpy(), freed)
