"""Compact verify-window index (verification/sps.py of the reference, the ``_indices`` part of
``device_plan``)."""

from __future__ import annotations

import torch

from dspine_amd import _lib


def window_index(qo_indptr: torch.Tensor, block_size: int, total: int, out: torch.Tensor | None = None):
    """int64 [total]: out[qo[b] + d] = b*block_size + d for d < qo[b+1] - qo[b]
    (verification/sps.py:27-32, :87-98).  qo_indptr [bs+1] int32/int64 with qo[bs] == total;
    the KV slots of the verified rows are out_cache_loc[window_index]."""
    if qo_indptr.ndim != 1 or qo_indptr.dtype not in (torch.int32, torch.int64) or not qo_indptr.is_contiguous():
        raise ValueError("qo_indptr must be a contiguous int32/int64 vector")
    if block_size < 1 or total < 0:
        raise ValueError("invalid window layout")
    dev = _lib.require_cuda(qo_indptr)
    if out is None:
        out = torch.empty(total, device=dev, dtype=torch.int64)
    elif out.shape != (total,) or out.dtype != torch.int64 or not out.is_contiguous():
        raise ValueError("out must be a contiguous int64 [total] tensor")
    bs = qo_indptr.numel() - 1
    if bs > 0 and total > 0:
        _lib.check(_lib.load().dsv_window_index(qo_indptr.data_ptr(), int(qo_indptr.dtype == torch.int64), bs,
                                                int(block_size), out.data_ptr(), total, _lib.stream_of(dev)),
                   "dsv_window_index")
    return out
