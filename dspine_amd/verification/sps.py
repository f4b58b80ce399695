"""SPS (survival-probability) verify-length planning and the compact verify-window index
(verification/sps.py of the reference).

``device_plan`` is one HIP launch (``dsv_sps_plan``): the calibration table lookup of every
draft position's confidence, prefix survival, the budget's highest-survival positions, the
per-request verify lengths, the ragged layout's row pointer and the window index.  No host
synchronisation, so the plan can be captured in a HIP graph and replayed with new confidences.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from dspine_amd import _lib


def conditional_table(data):
    """The legacy empirical table (verification/sps.py:16-24): per depth, each bin's success
    rate shrunk toward the depth's prior (itself shrunk toward 0.85), clipped to [0.05, 0.999]."""
    result = []
    for successes, counts in zip(data["success"], data["count"]):
        prior = (sum(successes) + 8 * 0.85) / (sum(counts) + 8)
        result.append([min(0.999, max(0.05, (s + 12 * prior) / (c + 12))) for s, c in zip(successes, counts)])
    return result


@dataclass
class RaggedVerifyLayout:
    """The device layout a ragged verify round runs on: per-request lengths, the row pointer
    ``qo_indptr_device`` [bs + 1] (int32, exclusive prefix of the lengths), the graph tier and
    the verified token count."""

    verify_lens: torch.Tensor
    qo_indptr_device: torch.Tensor
    graph_num_tokens: int
    total_verify_tokens: int


def _plan(raw, probabilities, depth, budget, boundaries, lens, qo, index):
    dev = _lib.require_cuda(lens, raw, probabilities, depth, boundaries, qo, index)
    bs = lens.shape[0]
    gamma = depth.shape[0] if raw is None else raw.shape[1]
    args = dict(rp=None, rs=0, pp=None, ps=0, nb=1, pr=1, dp=None, bp=None, nbd=0)
    if raw is not None:
        args.update(rp=raw.data_ptr(), rs=raw.stride(0), pp=probabilities.data_ptr(), ps=probabilities.stride(0),
                    nb=probabilities.shape[1], pr=probabilities.shape[0], dp=depth.data_ptr())
        if boundaries is not None:
            args.update(bp=boundaries.data_ptr(), nbd=boundaries.numel())
    _lib.check(_lib.load().dsv_sps_plan(
        args["rp"], args["rs"], bs, gamma, args["pp"], args["ps"], args["nb"], args["pr"], args["dp"], args["bp"],
        args["nbd"], int(budget), lens.data_ptr(), _lib.ptr(qo), _lib.ptr(index), _lib.stream_of(dev)),
        "dsv_sps_plan")


def _plan_inputs(raw, probabilities, depth, budget, boundaries):
    if raw.ndim != 2 or raw.dtype != torch.float32 or raw.stride(1) != 1:
        raise ValueError("raw confidences must be row-contiguous float32 [bs, gamma]")
    bs, gamma = raw.shape
    if not bs <= budget <= bs * (gamma + 1):
        raise ValueError("SPS budget must include every root and fit the draft block")
    if probabilities.ndim != 2 or probabilities.stride(1) != 1:
        raise ValueError("probabilities must be a row-contiguous [depths, bins] table")
    probabilities = probabilities.to(torch.float32)
    depth = depth.to(device=raw.device, dtype=torch.int64).contiguous()
    if depth.shape != (gamma,):
        raise ValueError("depth must select one table row per draft position")
    if boundaries is not None:
        boundaries = boundaries.to(device=raw.device, dtype=torch.float64).contiguous()
        if boundaries.ndim != 1 or boundaries.numel() > probabilities.shape[1] - 1:
            raise ValueError("boundaries must hold at most bins - 1 values")
    return probabilities, depth, boundaries


def allocate_verify_lens(raw, probabilities, depth, budget, boundaries=None):
    """Per-request verify lengths int32 [bs] (verification/sps.py:35-58): one root per request
    plus the ``budget - bs`` draft positions of highest prefix survival, where a position's
    conditional acceptance probability is ``probabilities[depth[d], bin(raw[b, d])]`` (bins by
    ``torch.bucketize`` against ``boundaries``, else ``trunc(raw * bins)`` clamped) and survival
    is the running minimum of the running product; ties go to the lower depth, then the lower
    request (a stable position-major order), so a descendant never precedes its ancestors."""
    probabilities, depth, boundaries = _plan_inputs(raw, probabilities, depth, budget, boundaries)
    lens = torch.empty(raw.shape[0], device=raw.device, dtype=torch.int32)
    _plan(raw, probabilities, depth, budget, boundaries, lens, None, None)
    return lens


def device_plan(raw, probabilities, depth, budget, cfg, graph_tokens=None, boundaries=None, *, tp=None):
    """(layout, window index int64 [budget]) of one SPS round (verification/sps.py:61-99).

    ``cfg`` is SGLang's DSparkScheduleConfig (duck-typed: ``min_verify_len`` must be 1 and
    ``survival_eps`` 0).  With ``tp`` the lengths are synchronised across tensor-parallel ranks
    (``tp.sync_tensor``) before the layout is derived from them."""
    if cfg.min_verify_len != 1 or cfg.survival_eps != 0.0:
        raise ValueError("DSpine SPS requires one root per request and no survival cutoff")
    if graph_tokens is None:
        graph_tokens = budget
    if graph_tokens != budget:
        raise ValueError("SPS graph tier must equal the verified token budget")
    probabilities, depth, boundaries = _plan_inputs(raw, probabilities, depth, budget, boundaries)
    bs = raw.shape[0]
    dev = raw.device
    lens = torch.empty(bs, device=dev, dtype=torch.int32)
    qo = torch.empty(bs + 1, device=dev, dtype=torch.int32)
    index = torch.empty(budget, device=dev, dtype=torch.int64)
    if tp is None:
        _plan(raw, probabilities, depth, budget, boundaries, lens, qo, index)
    else:
        _plan(raw, probabilities, depth, budget, boundaries, lens, None, None)
        tp.sync_tensor(lens)
        _plan(None, None, depth, budget, None, lens, qo, index)
    layout = RaggedVerifyLayout(verify_lens=lens, qo_indptr_device=qo, graph_num_tokens=int(graph_tokens),
                                total_verify_tokens=int(budget))
    return layout, index


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
