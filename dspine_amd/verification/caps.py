"""Greedy (argmax) acceptance with a verify cap (verification/caps.py of the reference).

``accept_greedy`` fuses ``torch.argmax(next_token_logits)`` with ``_accept_capped``
(caps.py:32-59) / ``_accept`` (ragged.py:51-76): a = first i < cap-1 whose proposal differs
from the row's first argmax, bonus = argmax of row a, and the output keeps the proposals after
a (they are not zeroed, unlike the sampled path).
"""

from __future__ import annotations

import torch

from dspine_amd import _lib
from dspine_amd.verify import Workspace

_ws: dict = {}


def accept_greedy(*, candidates: torch.Tensor, next_token_logits: torch.Tensor,
                  prefix_lens: torch.Tensor, cap: int | None = None,
                  verify_lens: torch.Tensor | None = None, outputs=None,
                  top1: torch.Tensor | None = None):
    """Returns the 5-tuple (accept i32, commit i32, bonus i64, output i64 [bs, T], new_seq i32).
    ``cap`` is the static verify width (caps.py) or ``verify_lens`` the per-request lengths
    (ragged.py); next_token_logits is the full [bs*T, V] envelope."""
    dev = _lib.require_cuda(candidates, next_token_logits, prefix_lens, verify_lens)
    if candidates.ndim != 2 or candidates.dtype != torch.int64 or not candidates.is_contiguous():
        raise ValueError("candidates must be contiguous int64 [bs, T]")
    bs, T = candidates.shape
    logits = next_token_logits
    if logits.ndim != 2 or logits.shape[0] != bs * T or logits.stride(1) != 1:
        raise ValueError("Greedy acceptance needs row-contiguous [bs*T, V] logits")
    if prefix_lens.shape != (bs,) or prefix_lens.dtype != torch.int32:
        raise ValueError("prefix_lens must be int32 [bs]")
    if verify_lens is None:
        cap = T if cap is None else int(cap)
        if not 1 <= cap <= T:
            raise ValueError(f"cap {cap} outside [1, {T}]")
    elif verify_lens.shape != (bs,) or verify_lens.dtype != torch.int32 or not verify_lens.is_contiguous():
        raise ValueError("verify_lens must be contiguous int32 [bs]")
    if outputs is None:
        outputs = (torch.empty(bs, device=dev, dtype=torch.int32),
                   torch.empty(bs, device=dev, dtype=torch.int32),
                   torch.empty(bs, device=dev, dtype=torch.int64),
                   torch.empty((bs, T), device=dev, dtype=torch.int64),
                   torch.empty(bs, device=dev, dtype=torch.int32))
    accept, commit, bonus, output, new_seq = outputs
    if output.shape != (bs, T):
        raise ValueError("output must be [bs, T]")
    if top1 is not None and (top1.shape != (bs, T) or top1.dtype != torch.int64):
        raise ValueError("top1 must be int64 [bs, T]")
    lib = _lib.load()
    ws = _ws.setdefault(dev, Workspace()).get(int(lib.dsv_greedy_workspace_bytes(bs * T, logits.shape[1])), dev)
    _lib.check(lib.dsv_greedy_verify(
        logits.data_ptr(), _lib.dtype_code(logits), bs * T, logits.shape[1], logits.stride(0), bs, T,
        candidates.data_ptr(), _lib.ptr(verify_lens), int(cap or 0), prefix_lens.data_ptr(),
        accept.data_ptr(), commit.data_ptr(), bonus.data_ptr(), output.data_ptr(), new_seq.data_ptr(),
        _lib.ptr(top1), ws.data_ptr(), ws.numel(), _lib.stream_of(dev)), "dsv_greedy_verify")
    return outputs


def active_controller():
    """The active worker's verification controller, or None (verification/caps.py:381-385)."""
    from dspine_amd.runtime import worker as module

    current = module._active_worker
    return getattr(current, "verify_caps", None) if current is not None else None


def _prefix_i32(prefix_lens):
    return prefix_lens if prefix_lens.dtype == torch.int32 else prefix_lens.to(torch.int32)


def accept(self, *, candidates, next_token_logits, sampling_info, draft_input, prefix_lens, bs):
    """``VerifyCaps.accept`` (verification/caps.py:331-379), written as a plain function of the
    controller so that it binds as the method (``VerifyCaps.accept = caps.accept``).

    Reads the controller state the reference reads: ``executed_width`` and ``active`` (the
    confirmed shortened target forward), ``sampled_round``, ``full``, ``worker`` (its
    ``_next_accept_bonus_buffers``) and ``_sampled_cap_lens``.  Sampled rounds verify against
    this round's q (``accept_sampled_prefix`` with every request's length = ``active``);
    greedy rounds run the fused argmax + capped acceptance (``dsv_greedy_verify``) into the
    worker's next output buffers.  Returns (accept i32, commit i32, bonus i64, output i64
    [bs, full], new_seq i32)."""
    if self.executed_width != self.active:
        raise RuntimeError("Capped acceptance requires a confirmed shortened target forward")
    if self.sampled_round:
        from dspine_amd.sampling.rejection import accept_sampled_prefix

        cache = getattr(self, "_sampled_cap_lens", None)
        if cache is None:
            cache = self._sampled_cap_lens = {}
        key = (bs, self.active)
        if key not in cache:
            cache[key] = torch.full((bs,), self.active, device=candidates.device, dtype=torch.int32)
        return accept_sampled_prefix(self, candidates=candidates, next_token_logits=next_token_logits,
                                     sampling_info=sampling_info, prefix_lens=prefix_lens, bs=bs,
                                     verify_lens=cache[key])
    if candidates.shape != (bs, self.full):
        raise ValueError(f"Capped acceptance requires full{self.full} proposal storage")
    outputs = self.worker._next_accept_bonus_buffers(bs)
    return accept_greedy(candidates=candidates, next_token_logits=next_token_logits,
                         prefix_lens=_prefix_i32(prefix_lens), cap=self.active, outputs=outputs)
