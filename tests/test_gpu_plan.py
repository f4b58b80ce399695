"""The SPS planner on the GPU (verification/sps.py:35-99 through ``dsv_sps_plan``): verify
lengths, the layout's row pointer and the window index against the oracle, bit-exact, including
captured-graph replays with new confidences."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

CFG = SimpleNamespace(min_verify_len=1, survival_eps=0.0)


def _O():
    import oracle.verify_oracle as O

    return O


def _check(raw, table, depth, budget, boundaries, device, tag):
    from dspine_amd.verification.sps import allocate_verify_lens, device_plan

    O = _O()
    bs, gamma = raw.shape
    ref = O.allocate_verify_lens(raw, table, depth, budget, boundaries)
    qo_ref, idx_ref = O.sps_layout(ref.numpy(), gamma + 1)
    d = lambda t: None if t is None else t.to(device)  # noqa: E731
    lens = allocate_verify_lens(d(raw), d(table), d(depth), budget, d(boundaries))
    layout, index = device_plan(d(raw), d(table), d(depth), budget, CFG, boundaries=d(boundaries))
    torch.cuda.synchronize()
    assert torch.equal(lens.cpu(), ref), (tag, budget)
    assert torch.equal(layout.verify_lens.cpu(), ref), (tag, budget)
    assert np.array_equal(layout.qo_indptr_device.cpu().numpy(), qo_ref), (tag, budget)
    assert np.array_equal(index.cpu().numpy(), idx_ref), (tag, budget)
    assert layout.total_verify_tokens == layout.graph_num_tokens == budget


@pytest.mark.parametrize("bs", [1, 3, 9, 17, 65, 256])
def test_plan_matches_oracle_linear_bins(device, bs):
    """tests/test_sps.py:360-384's case (equal confidences on every other request) and random
    tables, at budgets from the roots only to the full block."""
    g = torch.Generator().manual_seed(714 + bs)
    raw = torch.rand((bs, 15), generator=g)
    raw[::2] = 1
    table = torch.linspace(0.1, 1.0, 16).expand(15, 16).contiguous()
    for budget in sorted({bs, bs * 7 + (bs > 1), bs * 16, bs + (bs * 15) // 3}):
        _check(raw, table, torch.arange(15), budget, None, device, f"linspace bs={bs}")
    table = torch.rand((15, 64), generator=g)
    raw = torch.rand((bs, 15), generator=g)
    depth = torch.arange(15).flip(0)  # rows of the table in another order
    for budget in sorted({bs, bs + 1, bs * 5, bs * 16 - 1, bs * 16}):
        _check(raw, table, depth, budget, None, device, f"random bs={bs}")


def test_plan_fp32_extreme_survival(device):
    """tests/test_sps.py:387-417: extreme float32 survival values, every budget."""
    bs, gamma = 4, 15
    conditional = torch.tensor([
        [1.0] * gamma,
        [1.0, 1.0 - 2**-24, 1.0 - 2**-23] * 5,
        [1e-30, 1.0, 1e-30] + [1.0] * 12,
        [1.0, torch.finfo(torch.float32).tiny, 1.0, 1e-10] + [1.0] * 11,
    ], dtype=torch.float32)
    table = conditional.T.contiguous()
    raw = torch.tensor([0.125, 0.375, 0.625, 0.875])[:, None].expand(bs, gamma).contiguous()
    for budget in range(bs, bs * (gamma + 1) + 1):
        _check(raw, table, torch.arange(gamma), budget, None, device, "extreme")


@pytest.mark.parametrize("bs", [3, 40])
def test_plan_logit_boundaries(device, bs):
    """Bins from 1023 float64 logit-grid boundaries (tests/test_sps.py:420-448), confidences at
    0, 1, 1 - 1e-6 and exactly on boundaries."""
    logits = torch.linspace(-13.815509557963773, 13.815509557963773, 1024, dtype=torch.float64)
    boundaries = ((logits[1:] + logits[:-1]) / 2).sigmoid()
    table = (0.216 * logits + 0.3).sigmoid().float().repeat(15, 1)
    g = torch.Generator().manual_seed(bs)
    raw = torch.rand((bs, 15), generator=g)
    raw[0] = 1.0
    raw[1] = 1 - 1e-6
    raw[2, :5] = 0.0
    raw[-1] = boundaries[torch.randint(0, 1023, (15,), generator=g)].float()
    for budget in sorted({bs, bs + 7, bs * 8, bs * 16}):
        _check(raw, table, torch.arange(15), budget, boundaries, device, f"boundaries bs={bs}")


def test_plan_large_batch(device):
    """2000 requests x 15 positions (30000 survival keys, several a thread), ties everywhere."""
    g = torch.Generator().manual_seed(9)
    raw = (torch.randint(0, 8, (2000, 15), generator=g).float() / 8)
    table = torch.rand((15, 8), generator=g)
    for budget in (2000, 2001, 9999, 17000, 32000):
        _check(raw, table, torch.arange(15), budget, None, device, "large")


def test_plan_graph_replays(device):
    """The plan captured once in a HIP graph and replayed with new confidences (the reference's
    tests/test_sps.py:420-448 pattern): every replay equals the oracle, with the program's own
    eager work between replays."""
    from dspine_amd.verification.sps import device_plan

    O = _O()
    bs, gamma, budget = 6, 15, 31
    g = torch.Generator().manual_seed(4)
    table = torch.rand((15, 32), generator=g).to(device)
    depth = torch.arange(gamma, device=device)
    raw = torch.rand((bs, gamma), generator=g).to(device)
    device_plan(raw, table, depth, budget, CFG)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        layout, index = device_plan(raw, table, depth, budget, CFG)
    for i in range(4):
        raw.copy_(torch.rand((bs, gamma), generator=g).to(device))
        if i == 2:
            raw[0].fill_(1.0)
        graph.replay()
        torch.cuda.synchronize()
        ref = O.allocate_verify_lens(raw.cpu(), table.cpu(), depth.cpu(), budget)
        qo_ref, idx_ref = O.sps_layout(ref.numpy(), gamma + 1)
        assert torch.equal(layout.verify_lens.cpu(), ref), i
        assert np.array_equal(layout.qo_indptr_device.cpu().numpy(), qo_ref), i
        assert np.array_equal(index.cpu().numpy(), idx_ref), i


def test_plan_tp_synchronised_lengths(device):
    """With a tensor-parallel coordinator the lengths are synchronised (here: replaced by the
    leader's) before the layout is derived from them."""
    from dspine_amd.verification.sps import device_plan

    O = _O()
    leader = torch.tensor([1, 5, 2, 16, 1, 3], dtype=torch.int32)

    class Tp:
        def sync_tensor(self, t):
            t.copy_(leader.to(t.device))

    raw = torch.rand((6, 15)).to(device)
    table = torch.rand((15, 16)).to(device)
    layout, index = device_plan(raw, table, torch.arange(15, device=device), int(leader.sum()), CFG, tp=Tp())
    torch.cuda.synchronize()
    qo_ref, idx_ref = O.sps_layout(leader.numpy(), 16)
    assert torch.equal(layout.verify_lens.cpu(), leader)
    assert np.array_equal(layout.qo_indptr_device.cpu().numpy(), qo_ref)
    assert np.array_equal(index.cpu().numpy(), idx_ref)


def test_plan_given_lengths_past_the_budget(device):
    """Given lengths (the TP-synchronised path) that sum past the budget write only the index's
    budget entries: the entries after it keep their sentinel, and qo_indptr[bs] reports the sum."""
    from dspine_amd.verification.sps import _plan

    bs, gamma, budget = 6, 7, 20
    lens = torch.tensor([8, 8, 1, 8, 8, 8], dtype=torch.int32, device=device)  # 41 > 20
    qo = torch.empty(bs + 1, dtype=torch.int32, device=device)
    store = torch.full((budget + 64,), -7, dtype=torch.int64, device=device)
    index = store[:budget]
    depth = torch.arange(1, gamma + 1, dtype=torch.int64, device=device)
    _plan(None, None, depth, budget, None, lens, qo, index)
    torch.cuda.synchronize()
    full = gamma + 1
    want = [b * full + d for b, n in enumerate(lens.tolist()) for d in range(n)][:budget]
    assert store[:budget].tolist() == want
    assert (store[budget:] == -7).all()
    assert qo.tolist() == [0, 8, 16, 17, 25, 33, 41]
