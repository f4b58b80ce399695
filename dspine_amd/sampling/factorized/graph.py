"""Factorized proposal logits with bounded graph and workspace storage
(sampling/factorized/graph.py of the reference).

``ProposalGraphs(sampler)`` builds the float64 cache once, captures ``factor_table`` in one HIP
graph per selected batch size (sizes at least doubling, so retained storage stays linear in the
largest) and replays the smallest captured size that covers a batch, zeroing the padding rows of
the live draft state first; batches above every captured size run eagerly on grow-only buffers.
``lookup`` refuses weights or cache tensors that changed after preparation and a stream other
than the first one it saw.
"""

from __future__ import annotations

from dataclasses import fields, replace

import torch

from dspine_amd.sampling.factorized.kernels import Workspace, factor_table
from dspine_amd.sampling.factorized.weights import build_cache


def _signature(tensor):
    if tensor is None:
        return None
    try:
        version = tensor._version
    except RuntimeError:
        version = None
    return (tensor.data_ptr(), tensor.device, tensor.dtype, tuple(tensor.shape), tuple(tensor.stride()), version)


def _capture_sizes(configured, capacity):
    """Configured batch sizes within capacity, keeping a size only when it at least doubles the
    previous kept one; the largest configured size always closes the list."""
    wanted = sorted({int(x) for x in configured if 0 < int(x) <= capacity})
    kept = []
    for size in wanted:
        if not kept or size >= 2 * kept[-1]:
            kept.append(size)
    if wanted and kept[-1] != wanted[-1]:
        kept[-1] = wanted[-1]
    return kept


class _Buffers:
    def __init__(self, bs, sampler):
        self.bs = bs
        n = bs * (sampler.block_size - 1)
        k = sampler.k
        h, r = sampler.raw.shape[1], sampler.query.shape[1]
        dev = sampler.raw.device
        self.base = torch.empty((n, k), device=dev, dtype=torch.float64)
        self.output = torch.empty((n, k, k), device=dev, dtype=torch.float32)
        self.workspace = Workspace.allocate(n, k, h, r, dev)

    def view(self, n):
        """The first n rows of every buffer (the GEMM scratch is shared whole)."""
        parts = {f.name: getattr(self.workspace, f.name)[:n] for f in fields(self.workspace)
                 if f.name not in ("fallback", "gemm")}
        parts["fallback"] = replace(self.workspace.fallback, y=self.workspace.fallback.y[:n])
        return self.output[:n], self.base[:n], replace(self.workspace, **parts)


class ProposalGraphs:
    def __init__(self, sampler):
        self.sampler = sampler
        self.entries = {}
        self.stream = None
        self.graph_buffers = self.eager_buffers = None
        bridge = sampler.draft_model.selected_prefix_bridge
        tensors = (bridge.codebook, sampler.pred_gate_f32, sampler.prev_f32, sampler.gate_b_f32, sampler.write_f32,
                   sampler.norm_f32, sampler.lm_head_weight)
        res_emb = getattr(sampler, "res_emb", None)
        res_proj = getattr(sampler, "res_proj_f32", None)
        self.source_tensors = tensors + (res_emb, res_proj)
        self.source_signature = tuple(_signature(x) for x in self.source_tensors)
        self.weights = build_cache(*tensors, res_emb=res_emb, res_proj=res_proj,
                                   tp_head=getattr(sampler, "tp_head", None))
        self.weight_signature = tuple((key, _signature(value)) for key, value in sorted(self.weights.items()))
        sizes = _capture_sizes(getattr(sampler, "capture_batch_sizes", ()), sampler.max_bs)
        if not sizes:
            return
        self.graph_buffers = _Buffers(max(sizes), sampler)
        dev = sampler.raw.device
        current = torch.cuda.current_stream(dev)
        for bs in sizes:
            stream = torch.cuda.Stream(device=dev)
            stream.wait_stream(current)
            with torch.cuda.stream(stream):
                for _ in range(3):
                    self._compute(bs, self.graph_buffers)
            current.wait_stream(stream)
            current.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                self._compute(bs, self.graph_buffers)
            current.wait_stream(stream)
            current.synchronize()
            self.entries[bs] = graph

    def _compute(self, bs, buffers):
        s = self.sampler
        t, k = s.block_size, s.k
        n = bs * (t - 1)
        output, base, workspace = buffers.view(n)
        head = getattr(s, "candidate_head", None)
        return factor_table(s.raw[: bs * t], s.rms[: bs * t], s.query[: bs * t], s.anchors[:bs],
                            s.candidate_out[:bs].view(n, k), self.weights, s.norm_eps, t, output, base, workspace,
                            candidate_head=head[:n] if head is not None else None)

    def lookup(self, bs):
        s = self.sampler
        if not 0 < bs <= s.max_bs:
            raise ValueError("Proposal batch exceeds the configured sampler capacity")
        if tuple(_signature(x) for x in self.source_tensors) != self.source_signature:
            raise RuntimeError("Proposal weights changed after cache preparation")
        if tuple((key, _signature(value)) for key, value in sorted(self.weights.items())) != self.weight_signature:
            raise RuntimeError("Factorized proposal cache changed after preparation")
        current = torch.cuda.current_stream(s.raw.device)
        stream = int(current.cuda_stream)
        if self.stream is None:
            self.stream = stream
        elif stream != self.stream:
            raise RuntimeError("Proposal buffers must stay on their inference stream")
        bucket = next((size for size in sorted(self.entries) if size >= bs), None)
        if bucket is not None:
            if bucket != bs:
                # requests are independent: finite padding rows let a larger captured size serve
                rows = slice(bs * s.block_size, bucket * s.block_size)
                s.raw[rows].zero_()
                s.rms[rows].zero_()
                s.query[rows].zero_()
                s.anchors[bs:bucket].zero_()
                s.candidate_out[bs:bucket].zero_()
            self.entries[bucket].replay()
            return self.graph_buffers.output[: bs * (s.block_size - 1)]
        buffers = self.eager_buffers
        if buffers is None or buffers.bs < bs:
            capacity = min(s.max_bs, max(bs, 2 * buffers.bs if buffers else 1))
            self.eager_buffers = buffers = _Buffers(capacity, s)
        return self._compute(bs, buffers)
