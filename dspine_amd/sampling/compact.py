"""Request-wise logit adjustments, in place, for verification rows (sampling/compact.py of the
reference).  Each additive / multiplicative operation is one HIP pass over the rows
(``dsv_adjust_logits``), rounded to the logits dtype once per operation as the reference's
in-place tensor ops are; a presence / repetition penalty given as a token history touches only
the history's tokens (``dsv_adjust_history``)."""

from __future__ import annotations

import torch

from dspine_amd import _lib


def can_keep_compact(info):
    """sampling/compact.py:6-11."""
    return (info is not None and not getattr(info, "has_custom_logit_processor", False)
            and getattr(info, "sampling_mask_batch_indices", None) is None)


def _rows_view(logits, row_to_request):
    """(rows, row_stride, rows_per_request) of [rows, V] (mapped) or [B, T, V] logits."""
    if logits.stride(-1) != 1:
        raise ValueError("logits rows must be contiguous")
    V = logits.shape[-1]
    if row_to_request is not None:
        if logits.ndim != 2 or row_to_request.numel() != logits.shape[0]:
            raise ValueError("row_to_request must map every row of [rows, V] logits")
        return logits.shape[0], logits.stride(0), 1
    if logits.ndim != 3:
        raise ValueError("full-block logits must be viewed as [B, T, V]")
    B, T, _ = logits.shape
    if T == 1:
        return B, logits.stride(0), 1
    if B > 1 and logits.stride(0) != T * logits.stride(1):
        raise ValueError("full-block logits rows must be evenly strided")
    return B * T, logits.stride(1), T


def _apply(logits, value, op, row_to_request):
    rows, stride, per_req = _rows_view(logits, row_to_request)
    V = logits.shape[-1]
    dev = _lib.require_cuda(logits)
    value = value.to(device=dev, dtype=torch.float32)
    if value.ndim != 2 or value.shape[1] != V:
        raise ValueError("penalty tensors must be [requests, V]")
    value = value.contiguous()
    rtr = None
    if row_to_request is not None:
        rtr = row_to_request.to(device=dev, dtype=torch.int64).contiguous()
    if rows:
        _lib.check(_lib.load().dsv_adjust_logits(
            logits.data_ptr(), _lib.dtype_code(logits), rows, V, stride, _lib.ptr(rtr), per_req,
            value.shape[0], op, value.data_ptr(), value.stride(0), _lib.stream_of(dev)), "dsv_adjust_logits")


def adjust_logits(logits, info, row_to_request):
    """Apply the request transforms to real logits in place, in the reference's order
    (sampling/compact.py:14-79): additive penalties (alias acc_linear_penalties), scaling
    penalties ``x < 0 ? x*s : x/s``, the live penalizers in orchestrator order, the grammar
    mask, then logit_bias.  Packed logits [rows, V] use ``row_to_request``; full blocks are
    [B, T, V] with no mapping."""
    if info is None:
        return

    def mapped_mask(mask):
        mask = mask.to(device=logits.device)
        return (mask.index_select(0, row_to_request) if row_to_request is not None
                else mask.repeat_interleave(logits.shape[1], dim=0))

    linear = getattr(info, "acc_additive_penalties", None)
    if linear is None:
        linear = getattr(info, "acc_linear_penalties", None)
    if linear is not None:
        _apply(logits, linear, _lib.DSV_ADJ_ADD, row_to_request)
    scaling = getattr(info, "acc_scaling_penalties", None)
    if scaling is not None:
        _apply(logits, scaling, _lib.DSV_ADJ_SCALE, row_to_request)
    penalizer = getattr(info, "penalizer_orchestrator", None)
    if penalizer is not None and penalizer.is_required:
        for penalty in penalizer.penalizers.values():
            if not penalty.is_prepared():
                continue
            if penalty.is_multiplicative:
                _apply(logits, penalty.get_scaling_penalties(), _lib.DSV_ADJ_SCALE, row_to_request)
            else:
                bias = torch.zeros((len(info), logits.shape[-1]), device=logits.device, dtype=torch.float32)
                penalty.apply(bias)
                _apply(logits, bias, _lib.DSV_ADJ_ADD, row_to_request)
    grammar = getattr(info, "grammar_mask", None)
    if grammar is not None:
        grammar.grammar.apply_vocab_mask(logits=logits.reshape(-1, logits.shape[-1]),
                                         vocab_mask=mapped_mask(grammar.vocab_mask))
    bias = getattr(info, "logit_bias", None)
    if bias is not None:
        _apply(logits, bias, _lib.DSV_ADJ_ADD, row_to_request)


def adjust_history(logits, hist_ids, presence=None, repetition=None, row_to_request=None):
    """Presence (x -= presence[req]) then repetition (x < 0 ? x*r : x/r) on each token of the
    request's history, in place: the same values as adjust_logits with SGLang's dense buffers
    additive = -presence and scaling = repetition on the history tokens, touching only those
    tokens.  hist_ids [requests, H] int32 (-1 = padding; repeats count once)."""
    rows, stride, per_req = _rows_view(logits, row_to_request)
    dev = _lib.require_cuda(logits, hist_ids)
    if hist_ids.ndim != 2:
        raise ValueError("hist_ids must be [requests, H]")
    hist = hist_ids.to(torch.int32).contiguous()
    req = hist.shape[0]
    pres = None if presence is None else presence.reshape(-1).to(device=dev, dtype=torch.float32).contiguous()
    rep = None if repetition is None else repetition.reshape(-1).to(device=dev, dtype=torch.float32).contiguous()
    for name, v in (("presence", pres), ("repetition", rep)):
        if v is not None and v.numel() != req:
            raise ValueError(f"{name} must hold one value per request")
    rtr = None if row_to_request is None else row_to_request.to(device=dev, dtype=torch.int64).contiguous()
    if rows:
        _lib.check(_lib.load().dsv_adjust_history(
            logits.data_ptr(), _lib.dtype_code(logits), rows, logits.shape[-1], stride, _lib.ptr(rtr), per_req,
            max(req, 1), hist.data_ptr(), hist.shape[1], _lib.ptr(pres), _lib.ptr(rep), _lib.stream_of(dev)),
            "dsv_adjust_history")


def around_verify_logits_adjustments(original, *, next_token_logits, sampling_info, draft_token_num):
    """The AROUND hook on SGLang's verify-logit adjustments (sampling/compact.py:82-116).

    Resolves the active worker's verification controller (``caps.active_controller``).  With
    no DSpine worker at all the original SGLang adjustment runs.  A compact round adjusts the
    packed rows of the controller with its ``row_to_request`` (the logits must be the round's
    own packed tensor).  Otherwise full blocks [bs * draft_token_num, V] are adjusted as
    [bs, draft_token_num, V]: first SGLang's custom logit processors when the batch has them
    (``sglang.srt.layers.sampler.apply_custom_logit_processor``, imported only then, as the
    reference does), then ``adjust_logits``."""
    from dspine_amd.runtime import worker
    from dspine_amd.verification.caps import active_controller

    controller = active_controller()
    if controller is None and worker._active_worker is None:
        return original(next_token_logits=next_token_logits, sampling_info=sampling_info,
                        draft_token_num=draft_token_num)
    if controller is not None and getattr(controller, "compact_round", False):
        if next_token_logits is not controller.compact_logits:
            raise RuntimeError("Packed verification logits do not belong to this round")
        return adjust_logits(next_token_logits, sampling_info, controller.row_to_request)
    if sampling_info is None:
        return
    if next_token_logits.ndim != 2 or draft_token_num <= 0:
        raise ValueError("Verification needs 2D logits and a positive draft width")
    bs = len(sampling_info)
    if next_token_logits.shape[0] != bs * draft_token_num:
        raise ValueError("Verification logits do not match the request/block layout")
    if getattr(sampling_info, "has_custom_logit_processor", False):
        from sglang.srt.layers.sampler import apply_custom_logit_processor

        apply_custom_logit_processor(next_token_logits, sampling_info, num_tokens_in_batch=draft_token_num)
    return adjust_logits(next_token_logits.view(bs, draft_token_num, -1), sampling_info, None)
