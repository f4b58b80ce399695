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
