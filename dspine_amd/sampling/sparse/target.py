"""Small-support joint target P (sampling/sparse/target.py of the reference).

Eligible batches (flashinfer backend, no min-p, no greedy rows, a host-known max top-k within
the capacity) get the softmax P, its top-(capacity+1) prefix and the packed joint support in
three HIP launches: ``dsv_target_probs`` (softmax), ``dsv_topk`` (exact top-W under
(value desc, id asc)) and ``dsv_pack_joint`` (support test, id-ordered packing, dense
renormalisation of overflow rows in place).  Probabilities in the prefix are absolute
full-vocabulary probabilities; they are not renormalised before the top-p test.  Other batches
return None and the caller keeps its dense builder.
"""

from __future__ import annotations

from dataclasses import dataclass
from types import SimpleNamespace

import torch

from dspine_amd import _lib
from dspine_amd.kernels.dspine import topk
from dspine_amd.verify import target_probs

PREFIX_MAX = 64  # top-W prefix a wave packs: capacity <= 63


@dataclass
class SparseTarget:
    packed: tuple
    dense_p: torch.Tensor
    denominator: torch.Tensor | None = None


def _row_indices(logits, info, row_to_request, row_offsets, block_size):
    """Request of each row (sparse/target.py:70-83)."""
    rows = logits.shape[0]
    if row_to_request is not None:
        if row_to_request.numel() != rows:
            raise ValueError("row_to_request must cover every target row")
        return row_to_request.reshape(-1).to(device=logits.device, dtype=torch.long)
    index = torch.arange(rows, device=logits.device, dtype=torch.long)
    if row_offsets is not None:
        return torch.bucketize(index, row_offsets[1:].contiguous(), right=True)
    bs = info.temperatures.numel()
    if rows != bs * block_size:
        raise ValueError("Compact target logits require row mapping")
    return index // block_size


def sparse_eligible(info, sampling_backend: str, vocab: int, capacity: int = 32) -> bool:
    """Whether build_sparse_target takes the batch (sparse/target.py:106-116): the flashinfer
    backend, no min-p, no greedy rows and a host-known max top-k in [1, capacity] (<= vocab)."""
    max_k = getattr(info, "max_top_k", None)
    return (sampling_backend == "flashinfer"
            and not getattr(info, "need_min_p_sampling", False)
            and not getattr(info, "is_any_greedy", False)
            and isinstance(max_k, int) and 1 <= max_k <= capacity
            and vocab >= 1 and max_k <= vocab)


def build_sparse_target(logits, info, *, row_to_request=None, row_offsets=None, verify_lens=None,
                        block_size=16, capacity=32, sampling_backend="flashinfer"):
    """SparseTarget, or None when the ordinary dense path is required (sparse/target.py:95-178).

    packed = (ids int32 [rows, capacity], values float32 [rows, capacity], lengths int32 [rows],
    overflow int32 [rows]) in compact row indexing; dense_p [rows, V] float32 is the softmax,
    whose overflow rows hold the normalised p * (p >= p[k-1]).  No host read of device tensors.
    verify_lens is accepted for the shared caller contract."""
    del verify_lens
    max_k = getattr(info, "max_top_k", None)
    if (sampling_backend != "flashinfer"
            or getattr(info, "need_min_p_sampling", False)
            or getattr(info, "is_any_greedy", False)
            or not isinstance(max_k, int) or not 1 <= max_k <= capacity):
        return None
    if logits.ndim != 2 or capacity < 1:
        raise ValueError("Expected [rows,vocab] logits and positive capacity")
    if capacity >= PREFIX_MAX:
        return None
    rows, vocab = logits.shape
    if vocab < 1 or max_k > vocab:
        return None
    dev = _lib.require_cuda(logits)
    request = _row_indices(logits, info, row_to_request, row_offsets, block_size)
    if rows == 0:
        return SparseTarget((torch.empty((0, capacity), device=dev, dtype=torch.int32),
                             torch.empty((0, capacity), device=dev, dtype=torch.float32),
                             torch.empty(0, device=dev, dtype=torch.int32),
                             torch.empty(0, device=dev, dtype=torch.int32)),
                            torch.empty((0, vocab), device=dev, dtype=torch.float32))
    temperatures = info.temperatures.reshape(-1).to(dev)[request]
    top_ks = info.top_ks.reshape(-1).to(dev)[request].to(torch.int32).contiguous()
    top_ps = info.top_ps.reshape(-1).to(dev)[request].to(torch.float32).contiguous()
    softmax_info = SimpleNamespace(temperatures=temperatures,
                                   top_ks=torch.full((rows,), 1 << 30, device=dev, dtype=torch.int32),
                                   top_ps=torch.ones(rows, device=dev))
    p = target_probs(logits, softmax_info, bs=rows, T=1)
    width = min(capacity + 1, vocab)
    top_vals, top_ids = topk(p, width)
    ids = torch.empty((rows, capacity), device=dev, dtype=torch.int32)
    values = torch.empty((rows, capacity), device=dev, dtype=torch.float32)
    lengths = torch.empty(rows, device=dev, dtype=torch.int32)
    overflow = torch.empty_like(lengths)
    _lib.check(_lib.load().dsv_pack_joint(
        top_vals.data_ptr(), top_ids.data_ptr(), rows, width, top_ks.data_ptr(), top_ps.data_ptr(), capacity,
        ids.data_ptr(), values.data_ptr(), lengths.data_ptr(), overflow.data_ptr(), p.data_ptr(), vocab,
        p.stride(0), _lib.stream_of(dev)), "dsv_pack_joint")
    return SparseTarget((ids, values, lengths, overflow), p)
