"""Capped chain rejection on explicit distributions and the sampled-prefix glue
(sampling/rejection.py of the reference)."""

from __future__ import annotations

import logging

import torch

from dspine_amd import _lib
from dspine_amd.sampling.sparse.accept import fill_chain_args

logger = logging.getLogger(__name__)


def sample_capped_chain_from_probs(*, candidates, target_probs, draft_probs, verify_lens, uniforms,
                                   uniform_final, prefix_lens, outputs):
    """Chain rejection with dense P [B, T, V] and dense draft q [B, T-1, V], both float32
    (sampling/rejection.py:99-153): accept draft s iff 0 < q <= 1 and u*q < p; the bonus is drawn
    from max(P - clamp(Q), 0) (P when every draft was accepted or the residual has no mass) in
    id order.  Writes and returns ``outputs``.  T >= 2 (the reference is fixed at T = 16)."""
    bs, width = candidates.shape
    vocab = target_probs.shape[-1]
    if width < 2 or target_probs.shape != (bs, width, vocab):
        raise ValueError(f"Sampled ragged adapter requires target [B,{width},V]")
    if draft_probs.shape != (bs, width - 1, vocab):
        raise ValueError(f"Sampled ragged adapter requires draft q [B,{width - 1},V]")
    if verify_lens.shape != (bs,) or uniforms.shape != (bs, width - 1):
        raise ValueError("Invalid cap or uniform layout")
    if uniform_final.shape != (bs,) or prefix_lens.shape != (bs,):
        raise ValueError("Invalid final uniform or prefix layout")
    if len(outputs) != 5:
        raise ValueError("Expected accept/commit/bonus/output/new_seq buffers")
    tensors = (candidates, target_probs, draft_probs, verify_lens, uniforms, uniform_final, prefix_lens, *outputs)
    if any(not t.is_contiguous() for t in tensors):
        raise ValueError("The sampled capped kernel requires contiguous tensors")
    if any(t.device != candidates.device for t in tensors):
        raise ValueError("The sampled capped kernel requires one device")
    if target_probs.dtype != torch.float32 or draft_probs.dtype != torch.float32:
        raise ValueError("target and draft distributions must be float32")
    dev = _lib.require_cuda(candidates)
    a = _lib.ChainArgs()
    keep = fill_chain_args(a, candidates=candidates, verify_lens=verify_lens, uniforms=uniforms,
                           uniform_final=uniform_final, prefix_lens=prefix_lens, outputs=outputs)
    a.vocab = vocab
    a.dense_p, a.p_stride = target_probs.data_ptr(), vocab
    a.dense_q, a.q_stride = draft_probs.data_ptr(), vocab
    if bs:
        _lib.check(_lib.load().dsv_accept_chain(a, _lib.stream_of(dev)), "dsv_accept_chain")
    del keep
    return outputs


def accept_sampled_prefix(controller, *, candidates, next_token_logits, sampling_info, prefix_lens, bs,
                          verify_lens, row_offsets=None, row_to_request=None):
    """Verify one shortened target call with this round's sampled chain q
    (sampling/rejection.py:156-237): the worker's TargetDistribution when it takes the round,
    else the full-block target P and chain rejection with the sparse q lanes."""
    from dspine_amd.runtime.worker import build_dspine_target_probs, chain_on_probs
    from dspine_amd.sampling.random import verification_uniforms

    worker = controller.worker
    if worker.target_distribution is not None:
        result = worker.target_distribution.sample_prefix(
            candidates=candidates, next_token_logits=next_token_logits, sampling_info=sampling_info,
            prefix_lens=prefix_lens, bs=bs, verify_lens=verify_lens, row_offsets=row_offsets,
            row_to_request=row_to_request)
        if result is not None:
            controller.sampled_executions += 1
            return result
    sampler = worker._dspine_sampler
    if not sampler.round_sampled or sampler.round_bs != bs:
        raise RuntimeError("Sampled caps require the current sampled proposal and q")
    width = int(worker.block_size)
    if candidates.shape != (bs, width):
        raise ValueError(f"Sampled caps require full{width} proposal storage")
    if next_token_logits.shape[0] != bs * width:
        raise ValueError(f"Target output must retain the full{width} mapped row envelope")
    target = build_dspine_target_probs(next_token_logits=next_token_logits, sampling_info=sampling_info,
                                       block_size=width, bs=bs, sampling_backend=worker.sampling_backend)
    outputs = worker._next_accept_bonus_buffers(bs)
    uniforms, final = verification_uniforms(bs, width, candidates.device, sampler.random)
    chain_on_probs(candidates=candidates, probs=target.view(bs * width, -1),
                   q_ids=sampler.candidate_out[:bs].contiguous(),
                   q_values=sampler.q_out[:bs].to(torch.float32).contiguous(), verify_lens=verify_lens,
                   uniforms=uniforms, uniform_final=final, prefix_lens=prefix_lens, outputs=outputs)
    controller.sampled_executions += 1
    if controller.sampled_executions == 1:
        logger.info("DSPine sampled capped rejection executed: batch=%d full=%d", bs, width)
    return outputs
