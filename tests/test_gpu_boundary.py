"""The SGLang-facing seams on the GPU, driven the way the reference's controllers drive them:
``VerifyCaps.accept`` / ``RaggedVerifyCaps.accept`` (verification/caps.py:331-379,
verification/ragged.py:282-335) on stub controllers, both branches of
``accept_sampled_prefix`` (sampling/rejection.py:156-237: the worker's TargetDistribution and
the dense target P + chain fallback), and the AROUND hook on the verify-logit adjustments
(sampling/compact.py:82-116).  Outputs are compared with the oracle on the same
request-seeded uniforms (integer outputs bit-exact; tests/parity.py for near-margin requests).
"""

from types import SimpleNamespace

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


def _case(seed, bs=8, T=6, V=30011, K=8, dtype=torch.bfloat16):
    """Logits, sampling info (greedy / list / nucleus / unfiltered rows mixed), draft q lanes
    and drafts sampled from q.  Each row has a planted peak (p near 1) that one q lane holds
    with q = 0.6, so about 0.6 of the drafts are accepted and the rest are rejected."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(bs * T, V, generator=g) * 2.5
    peak = torch.randint(0, V, (bs * T,), generator=g)
    logits[torch.arange(bs * T), peak] = 30.0
    logits = logits.to(dtype)
    temps = torch.tensor([0.0, 0.6, 1.0, 0.8])[torch.arange(bs) % 4]
    ks = torch.tensor([0, 20, 0, 64])[torch.arange(bs) % 4]
    ps = torch.tensor([1.0, 0.95, 0.9, 1.0])[torch.arange(bs) % 4]
    info = W.sampling_info(temps, ks, ps)
    q_ids = torch.stack([torch.randperm(V, generator=g)[:K] for _ in range(bs * (T - 1))]).view(bs, T - 1, K)
    q_ids[:, :, 0] = peak.view(bs, T)[:, : T - 1]
    q = torch.full((bs, T - 1, K), 0.4 / (K - 1))
    q[:, :, 0] = 0.6
    q_ids, order = q_ids.sort(-1)
    q = q.gather(-1, order)
    lanes = torch.multinomial(q.view(-1, K), 1, generator=g).view(bs, T - 1)
    cand = torch.cat((torch.zeros(bs, 1, dtype=torch.int64), q_ids.gather(2, lanes[..., None]).squeeze(-1)), 1)
    prefix = torch.randint(10, 500, (bs,), generator=g, dtype=torch.int64).to(torch.int32)
    seeds = torch.arange(bs, dtype=torch.int64) * 104729 + seed
    positions = prefix.to(torch.int64) + 3
    return dict(logits=logits, info=info, q_ids=q_ids, q=q.contiguous(), cand=cand, prefix=prefix, seeds=seeds,
                positions=positions)


def _worker(c, T, device, use_target_distribution=True):
    from dspine_amd.runtime import worker as Wk
    from dspine_amd.sampling.random import RequestRNG

    rng = RequestRNG()
    rng.stage(c["seeds"].to(device), c["positions"].to(device))
    wk = Wk.VerifyWorker(T, device, k=c["q_ids"].shape[-1], random=rng,
                         use_target_distribution=use_target_distribution)
    wk._dspine_sampler.stage(c["q_ids"].to(device), c["q"].to(device))
    return wk


def _oracle_sampled(c, lens, rows=None, row_offsets=None):
    O = _O()
    bs, T = c["cand"].shape
    u_acc = O.seeded_uniforms(c["seeds"].numpy(), c["positions"].numpy(), T - 1, O.ACCEPT)
    u_fin = O.seeded_uniforms(c["seeds"].numpy(), c["positions"].numpy(), 1, O.BONUS).reshape(-1)
    logits = c["logits"] if rows is None else rows
    return O.verify_step(logits, c["info"], candidates=c["cand"].numpy(), q_ids=c["q_ids"].numpy(),
                         q_values=c["q"].numpy(), verify_lens=np.asarray(lens), uniforms=u_acc,
                         uniform_final=u_fin, prefix_lens=c["prefix"].numpy(), row_offsets=row_offsets,
                         exact_softmax=True)


def _got(outs):
    torch.cuda.synchronize()
    return {n: t.cpu().numpy() for n, t in zip(NAMES, outs)}


def _compare(got, ref, tag):
    bs = got["accept"].shape[0]
    assert (ref["accept"] > 0).any(), "the case should accept some drafts"
    differing = parity.compare_requests(got, ref, range(bs), tag, extra=())
    assert len(differing) <= 1, differing


# ------------------------------------------------------------------------------------------
# VerifyCaps.accept
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("active", [6, 4])
def test_capped_accept_greedy(device, active):
    from dspine_amd.verification import caps

    O = _O()
    bs, T = 8, 6
    c = _case(1, bs, T)
    top1 = O.argmax_rows(c["logits"])
    c["cand"][:, 1:] = torch.as_tensor(top1).view(bs, T)[:, : T - 1]
    c["cand"][3, 2] = (c["cand"][3, 2] + 1) % c["logits"].shape[1]  # one mismatch
    wk = _worker(c, T, device)
    ctl = SimpleNamespace(worker=wk, executed_width=active, active=active, sampled_round=False, full=T)
    outs = caps.accept(ctl, candidates=c["cand"].to(device), next_token_logits=c["logits"].to(device),
                       sampling_info=W.info_to(c["info"], device), draft_input=None,
                       prefix_lens=c["prefix"].to(torch.int64).to(device), bs=bs)
    got = _got(outs)
    ref = O.greedy_accept(top1, c["cand"].numpy(), [active] * bs, c["prefix"].numpy())
    for n, r in zip(NAMES, ref):
        assert np.array_equal(got[n], r), n
    assert got["accept"][3] == min(1, active - 1)
    assert outs[0].data_ptr() == wk._buffers[wk._flip][0].data_ptr()  # the worker's double buffer


@pytest.mark.parametrize("branch", ["target_distribution", "dense_fallback"])
@pytest.mark.parametrize("active", [6, 4])
def test_capped_accept_sampled(device, branch, active):
    """Both branches of accept_sampled_prefix through VerifyCaps.accept: the fused verify of
    the worker's TargetDistribution, and (no TargetDistribution) the dense target P with
    sparse-q chain rejection; each counts one sampled execution."""
    from dspine_amd.verification import caps

    bs, T = 8, 6
    c = _case(2, bs, T)
    wk = _worker(c, T, device, use_target_distribution=branch == "target_distribution")
    ctl = SimpleNamespace(worker=wk, executed_width=active, active=active, sampled_round=True, full=T,
                          sampled_executions=0)
    outs = caps.accept(ctl, candidates=c["cand"].to(device), next_token_logits=c["logits"].to(device),
                       sampling_info=W.info_to(c["info"], device), draft_input=None,
                       prefix_lens=c["prefix"].to(device), bs=bs)
    assert ctl.sampled_executions == 1
    assert ctl._sampled_cap_lens[(bs, active)].tolist() == [active] * bs
    _compare(_got(outs), _oracle_sampled(c, [active] * bs), f"capped sampled {branch} active={active}")


def test_accept_sampled_prefix_refuses_stale_round(device):
    from dspine_amd.sampling.rejection import accept_sampled_prefix

    bs, T = 4, 6
    c = _case(3, bs, T)
    wk = _worker(c, T, device, use_target_distribution=False)
    wk._dspine_sampler.finish()
    ctl = SimpleNamespace(worker=wk, sampled_executions=0)
    with pytest.raises(RuntimeError, match="current sampled proposal"):
        accept_sampled_prefix(ctl, candidates=c["cand"].to(device), next_token_logits=c["logits"].to(device),
                              sampling_info=W.info_to(c["info"], device), prefix_lens=c["prefix"].to(device),
                              bs=bs, verify_lens=torch.full((bs,), T, device=device, dtype=torch.int32))
    assert ctl.sampled_executions == 0


# ------------------------------------------------------------------------------------------
# RaggedVerifyCaps.accept
# ------------------------------------------------------------------------------------------
def _ragged_ctl(wk, lens, device, sampled, compact=False, row_offsets=None, row_to_request=None):
    bs = len(lens)
    return SimpleNamespace(worker=wk, ragged_round=True, batch_size=bs, tokens=int(sum(lens)),
                           executed_tokens=int(sum(lens)), sampled_round=sampled, full=wk.block_size,
                           compact_round=compact, sampled_executions=0,
                           layout=SimpleNamespace(verify_lens=torch.tensor(lens, dtype=torch.int32, device=device)),
                           row_offsets=row_offsets, row_to_request=row_to_request)


def test_ragged_accept_greedy(device):
    from dspine_amd.verification import ragged

    O = _O()
    bs, T = 8, 6
    c = _case(4, bs, T)
    lens = [1, 2, 6, 3, 6, 4, 5, 2]
    # the full envelope: rows past a request's length are padding rows [0, -inf, ...]
    env = c["logits"].clone()
    for b, n in enumerate(lens):
        env[b * T + n: (b + 1) * T] = O.logits_padding(torch.empty(0, dtype=env.dtype), (T - n, env.shape[1]))
    top1 = O.argmax_rows(env)
    c["cand"][:, 1:] = torch.as_tensor(top1).view(bs, T)[:, : T - 1]
    c["cand"][4, 3] = (c["cand"][4, 3] + 1) % env.shape[1]
    wk = _worker(c, T, device)
    ctl = _ragged_ctl(wk, lens, device, sampled=False)
    outs = ragged.accept(ctl, candidates=c["cand"].to(device), next_token_logits=env.to(device),
                         sampling_info=W.info_to(c["info"], device), draft_input=None,
                         prefix_lens=c["prefix"].to(device), bs=bs)
    got = _got(outs)
    ref = O.greedy_accept(top1, c["cand"].numpy(), lens, c["prefix"].numpy())
    for n, r in zip(NAMES, ref):
        assert np.array_equal(got[n], r), n
    assert got["accept"][4] == 2


@pytest.mark.parametrize("compact", [True, False])
def test_ragged_accept_sampled(device, compact):
    """Sampled ragged rounds: compact rows [sum(lens), V] with row offsets and the
    row-to-request map, or the padded full envelope [bs*T, V]."""
    from dspine_amd.verification import ragged

    bs, T = 8, 6
    c = _case(5, bs, T)
    lens = [2, 6, 1, 3, 6, 4, 5, 6]
    offs = np.concatenate(([0], np.cumsum(lens)[:-1]))
    wk = _worker(c, T, device)
    if compact:
        rows = torch.cat([c["logits"][b * T: b * T + n] for b, n in enumerate(lens)])
        rtr = torch.repeat_interleave(torch.arange(bs), torch.tensor(lens))
        ctl = _ragged_ctl(wk, lens, device, sampled=True, compact=True,
                          row_offsets=torch.as_tensor(offs, dtype=torch.int32, device=device),
                          row_to_request=rtr.to(device))
        logits = rows
        ref = _oracle_sampled(c, lens, rows=rows, row_offsets=offs)
    else:
        ctl = _ragged_ctl(wk, lens, device, sampled=True)
        logits = c["logits"]
        ref = _oracle_sampled(c, lens)
    outs = ragged.accept(ctl, candidates=c["cand"].to(device), next_token_logits=logits.to(device),
                         sampling_info=W.info_to(c["info"], device), draft_input=None,
                         prefix_lens=c["prefix"].to(device), bs=bs)
    assert ctl.sampled_executions == 1
    _compare(_got(outs), ref, f"ragged sampled compact={compact}")


# ------------------------------------------------------------------------------------------
# the AROUND hook with real adjustments
# ------------------------------------------------------------------------------------------
class _Info(SimpleNamespace):
    def __len__(self):
        return self.bs


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_hook_adjusts_full_block_and_compact_rows(device, dtype):
    from dspine_amd.runtime import worker as Wk
    from dspine_amd.sampling.compact import around_verify_logits_adjustments

    O = _O()
    g = torch.Generator().manual_seed(8)
    bs, T, V = 5, 4, 3001
    logits = (torch.randn(bs * T, V, generator=g) * 2).to(dtype)
    info = _Info(bs=bs, acc_additive_penalties=torch.randn(bs, V, generator=g) * 0.5,
                 acc_scaling_penalties=1.0 + torch.rand(bs, V, generator=g),
                 logit_bias=torch.randn(bs, V, generator=g) * 0.1, has_custom_logit_processor=False)
    d_info = _Info(**{k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in vars(info).items()})
    original = lambda **kw: pytest.fail("the original adjustment must not run under a DSpine worker")  # noqa: E731
    prev = Wk._active_worker
    try:
        Wk.set_active_worker(SimpleNamespace(verify_caps=None))
        x = logits.to(device)
        around_verify_logits_adjustments(original, next_token_logits=x, sampling_info=d_info, draft_token_num=T)
        ref = logits.clone()
        O.adjust_logits(ref, info, torch.arange(bs).repeat_interleave(T))
        torch.cuda.synchronize()
        assert torch.equal(x.cpu(), ref)
        # compact round: the controller's packed rows and row-to-request map
        lens = [1, 4, 2, 3, 1]
        rtr = torch.repeat_interleave(torch.arange(bs), torch.tensor(lens))
        packed = torch.cat([logits[b * T: b * T + n] for b, n in enumerate(lens)]).to(device)
        ctl = SimpleNamespace(compact_round=True, compact_logits=packed, row_to_request=rtr.to(device))
        Wk.set_active_worker(SimpleNamespace(verify_caps=ctl))
        around_verify_logits_adjustments(original, next_token_logits=packed, sampling_info=d_info,
                                         draft_token_num=T)
        ref = torch.cat([logits[b * T: b * T + n] for b, n in enumerate(lens)])
        O.adjust_logits(ref, info, rtr)
        torch.cuda.synchronize()
        assert torch.equal(packed.cpu(), ref)
    finally:
        Wk.set_active_worker(prev)
