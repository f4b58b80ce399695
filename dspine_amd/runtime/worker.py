"""The verify-side runtime of the DSpine worker (runtime/worker.py of the reference, the parts
on the draft-verification path).

Target distributions come from the HIP row kernels (``dsv_target_probs``); chain rejection on
an explicit target runs ``dsv_accept_chain`` with the draft's sparse q lanes, so the
reference's dense-q scatter (and its [bs, T-1, V] buffer traffic) does not exist here; the
sampled-verify seam routes to the fused single-pass verify (``dsv_verify``) through
``TargetDistribution.sample_prefix``.  The SGLang scheduler integration around these
functions (model forward, KV pools, plugin hooks) is not part of this package: the worker
below holds only the state the verify path reads.
"""

from __future__ import annotations

import threading
from types import SimpleNamespace

import torch

from dspine_amd import _lib
from dspine_amd.sampling.random import verification_uniforms
from dspine_amd.sampling.sparse.accept import fill_chain_args, fill_sparse_q
from dspine_amd.verify import Workspace, sampling_fields, target_probs

_active_worker = None


class SoftmaxTemp:
    """softmax(logits.float() / temperature) per row, the temperature of row r being that of
    request r // rows_per_request (SGLang's SoftmaxTemp, called at runtime/worker.py:455-459)."""

    @staticmethod
    def execute(*, logits, temperatures, rows_per_request=1):
        rows = logits.shape[0]
        t = int(rows_per_request)
        if t < 1 or rows % t:
            raise ValueError("rows must be whole requests of rows_per_request rows")
        info = SimpleNamespace(temperatures=temperatures, top_ks=_full_i32(rows // t, logits.device),
                               top_ps=torch.ones(rows // t, device=logits.device))
        return target_probs(logits, info, bs=rows // t, T=t)


def _full_i32(n, device):
    return torch.full((n,), 1 << 30, device=device, dtype=torch.int32)


def build_dspine_target_probs(*, next_token_logits, sampling_info, block_size: int, bs: int,
                              sampling_backend: str) -> torch.Tensor:
    """[bs, T, V] float32 (runtime/worker.py:440-470): softmax(logits / temperature), the
    configured backend's top-k / top-p / min-p filter, renormalised; rows of requests with
    top_k <= 1 one-hot at argmax(logits) (lowest id) when ``is_any_greedy``; a batch with no
    filter flag is the plain softmax."""
    t = int(block_size)
    probs = target_probs(next_token_logits, sampling_info, bs=bs, T=t, sampling_backend=sampling_backend)
    return probs.view(bs, t, -1)


def filter_target_probs(probs, sampling_info, t, bs, sampling_backend, normalize=True):
    """runtime/worker.py:473-508 on given probabilities [bs*t, V]: the backend filter, then
    (``normalize``) renormalised; without a filter flag the input is returned as a view.

    One library call (``dsv_filter_probs``): a pre-pass writes log p and each row's float64
    mass, then the HIP row kernels filter every row as a request of its own at temperature 1
    (softmax(log p) = p / sum(p), which renormalises to the same distribution; top-k and min-p,
    a ratio to the row's top p, select the same ids).  The reference's top-p test compares the
    raw mass ranked ahead of an id with top_p (:52-67; flashinfer's joint branch likewise, its
    min-p branch renormalises over the top-k first), so those rows' top_p is divided by the
    row's mass.  With ``normalize`` False the kept entries are the input values themselves."""
    need_k = bool(getattr(sampling_info, "need_top_k_sampling", False))
    need_p = bool(getattr(sampling_info, "need_top_p_sampling", False))
    need_min_p = bool(getattr(sampling_info, "need_min_p_sampling", False))
    if not (need_k or need_p or need_min_p):
        return probs.view(bs, t, -1)
    if sampling_backend not in ("pytorch", "flashinfer"):
        raise ValueError(f"DSPINE sampled verify: unsupported sampling backend {sampling_backend!r}")
    flat = probs.reshape(bs * t, -1)
    if flat.dtype != torch.float32:
        raise ValueError("filter_target_probs expects float32 probabilities")
    if flat.stride(1) != 1:
        raise ValueError("filter_target_probs expects row-contiguous probabilities")
    out = filter_probs(flat, sampling_info, bs=bs, T=t, sampling_backend=sampling_backend, normalize=normalize,
                       top_p_over_mass=need_p and not (sampling_backend == "flashinfer" and need_min_p))
    return out.view(bs, t, -1)


def filter_probs(probs, info, *, bs: int, T: int, sampling_backend: str, normalize: bool = True,
                 top_p_over_mass: bool = True, out: torch.Tensor | None = None,
                 workspace: Workspace | None = None) -> torch.Tensor:
    """``dsv_filter_probs`` on float32 probabilities [bs*T, V] with the per-request sampling
    parameters of ``info``; returns out [bs*T, V] float32."""
    lib = _lib.load()
    dev = _lib.require_cuda(probs, out)
    if probs.ndim != 2 or probs.dtype != torch.float32 or probs.stride(1) != 1:
        raise ValueError("probabilities must be a row-contiguous float32 [rows, V] tensor")
    rows, V = probs.shape
    if bs < 1 or T < 1 or rows != bs * T:
        raise ValueError(f"probability rows {rows} != bs*T ({bs}*{T})")
    if out is None:
        out = torch.empty((rows, V), device=dev, dtype=torch.float32)
    if out.shape != (rows, V) or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError("out must be a row-contiguous float32 [rows, V] tensor")
    a = _lib.VerifyArgs()
    keep = sampling_fields(a, info, bs, dev, sampling_backend)
    ws = workspace if workspace is not None else _filter_ws.setdefault(dev, Workspace())
    wbuf = ws.get(int(lib.dsv_filter_workspace_bytes(rows, V)), dev)
    a.logits, a.logits_dtype = probs.data_ptr(), _lib.DSV_F32
    a.rows, a.vocab, a.row_stride = rows, V, probs.stride(0)
    a.bs, a.T = bs, T
    a.workspace, a.workspace_bytes = wbuf.data_ptr(), wbuf.numel()
    _lib.check(lib.dsv_filter_probs(a, probs.data_ptr(), probs.stride(0), out.data_ptr(), out.stride(0),
                                    int(bool(normalize)), int(bool(top_p_over_mass)), _lib.stream_of(dev)),
               "dsv_filter_probs")
    del keep
    return out


_filter_ws: dict = {}


def dspine_accept_sampling(*, target_probs=None, candidates, target_logits, candidate_ids, q_rows,
                           sampling_info, sampling_backend, dense_q=None, random_state=None):
    """Chain rejection sampling of a drafted block (runtime/worker.py:511-581).

    candidates [bs, T] = [anchor, T-1 drafts]; candidate_ids / q_rows [bs, T-1, K] hold the
    sparse q each draft was drawn from (lanes with distinct ids).  With ``target_probs``
    [bs, T, V] the rejection runs against it; otherwise the fused verify reads target_logits
    once.  ``dense_q`` is accepted for the reference's signature and left untouched (all
    zero): the q lanes are read directly.  Returns (accept_len int32 [bs], bonus int64 [bs])."""
    bs, block = candidates.shape
    gamma = block - 1
    if tuple(candidate_ids.shape[:2]) != (bs, gamma) or candidate_ids.shape != q_rows.shape:
        raise RuntimeError("DSPINE verify: candidate / q layout mismatch")
    device = candidates.device
    uniforms, final = verification_uniforms(bs, block, device, random_state)
    prefix = torch.zeros(bs, device=device, dtype=torch.int32)
    q_vals = q_rows.to(torch.float32).contiguous()
    q_ids = candidate_ids.contiguous()
    if target_probs is None:
        from dspine_amd.verify import verify_step

        outputs, _ = verify_step(logits=target_logits, sampling_info=sampling_info, candidates=candidates,
                                 q_ids=q_ids, q_values=q_vals, uniforms=uniforms, uniform_final=final,
                                 prefix_lens=prefix, sampling_backend=sampling_backend)
        return outputs[0], outputs[2]
    outputs = _new_outputs(bs, block, device)
    chain_on_probs(candidates=candidates, probs=target_probs.reshape(bs * block, -1), q_ids=q_ids,
                   q_values=q_vals, verify_lens=None, uniforms=uniforms, uniform_final=final,
                   prefix_lens=prefix, outputs=outputs)
    return outputs[0], outputs[2]


def chain_on_probs(*, candidates, probs, q_ids, q_values, verify_lens, uniforms, uniform_final, prefix_lens,
                   outputs, row_offsets=None):
    """Sparse-q chain rejection against dense P [rows, V] float32 (dsv_accept_chain)."""
    dev = _lib.require_cuda(candidates, probs, q_ids, q_values, uniforms, uniform_final, prefix_lens)
    if probs.ndim != 2 or probs.dtype != torch.float32 or probs.stride(1) != 1:
        raise ValueError("target probabilities must be row-contiguous float32 [rows, V]")
    bs, t = candidates.shape
    a = _lib.ChainArgs()
    keep = fill_chain_args(a, candidates=candidates, verify_lens=verify_lens, uniforms=uniforms,
                           uniform_final=uniform_final, prefix_lens=prefix_lens, outputs=outputs,
                           row_offsets=row_offsets)
    fill_sparse_q(a, q_ids, q_values, bs, t)
    a.vocab = probs.shape[1]
    a.dense_p, a.p_stride = probs.data_ptr(), probs.stride(0)
    if bs:
        _lib.check(_lib.load().dsv_accept_chain(a, _lib.stream_of(dev)), "dsv_accept_chain")
    del keep
    return outputs


def _new_outputs(bs, t, device):
    return (torch.empty(bs, device=device, dtype=torch.int32),
            torch.empty(bs, device=device, dtype=torch.int32),
            torch.empty(bs, device=device, dtype=torch.int64),
            torch.empty((bs, t), device=device, dtype=torch.int64),
            torch.empty(bs, device=device, dtype=torch.int32))


class DraftRound:
    """This round's sampled draft chain as the verifier consumes it (the fields of the
    reference's DSpineDraftSampler that verification reads, runtime/worker.py:70-438):
    candidate_out int64 [>=bs, T-1, K] and q_out float32 [>=bs, T-1, K] from
    ``serial_sample_chain``, the round's batch size, whether it ran, K and the request RNG."""

    def __init__(self, k: int = 16, random=None):
        self.k = int(k)
        self.random = random
        self.round_sampled = False
        self.round_bs = 0
        self.candidate_out = None
        self.q_out = None

    def stage(self, candidate_out, q_out):
        if candidate_out.shape != q_out.shape or candidate_out.shape[-1] != self.k:
            raise ValueError("draft round storage must be [bs, T-1, K] ids and q")
        self.candidate_out, self.q_out = candidate_out, q_out
        self.round_bs = int(candidate_out.shape[0])
        self.round_sampled = True

    def finish(self):
        self.round_sampled = False


class VerifyWorker:
    """Verify-path state of DSpineWorkerV2 (runtime/worker.py:584-1089): the block size, the
    draft round, double-buffered caller-owned output buffers, the target distribution and the
    sampling backend."""

    def __init__(self, block_size: int, device, *, k: int = 16, sampling_backend: str = "pytorch",
                 random=None, use_target_distribution: bool = True):
        from dspine_amd.sampling.target import TargetDistribution

        self.block_size = int(block_size)
        self.device = torch.device(device)
        self.sampling_backend = sampling_backend
        self._dspine_sampler = DraftRound(k, random)
        self.target_distribution = TargetDistribution(self) if use_target_distribution else None
        self.verify_caps = None  # the verification controller (caps.active_controller reads it)
        self._buffers = [None, None]
        self._flip = 0
        self._lock = threading.Lock()

    def _next_accept_bonus_buffers(self, bs: int):
        """Two alternating sets of (accept, commit, bonus, output, new_seq), grown on demand, so
        the outputs of one round stay valid while the next is verified."""
        with self._lock:
            self._flip ^= 1
            buf = self._buffers[self._flip]
            if buf is None or buf[0].numel() < bs:
                buf = _new_outputs(max(bs, 2 * (buf[0].numel() if buf else 0)), self.block_size, self.device)
                self._buffers[self._flip] = buf
        return tuple(x[:bs] for x in buf)

    def _accept_sampled_round(self, *, candidates, next_token_logits, sampling_info, max_top_k=None,
                              uniform_top_k_value=None):
        """runtime/worker.py:1016-1046: refuse a round whose sampled chain did not run."""
        sampler = self._dspine_sampler
        bs = int(candidates.shape[0])
        if not sampler.round_sampled:
            raise RuntimeError("DSPINE sampled verify reached without this round's sampled draft chain")
        if bs != sampler.round_bs:
            raise RuntimeError(
                f"DSPINE sampled verify for batch {bs} while the staged round has batch {sampler.round_bs}")
        return self._dspine_verify(candidates=candidates, next_token_logits=next_token_logits,
                                   candidate_ids=sampler.candidate_out[:bs], q_rows=sampler.q_out[:bs],
                                   sampling_info=sampling_info)

    def _dspine_verify(self, *, candidates, next_token_logits, candidate_ids, q_rows, sampling_info, **_):
        """runtime/worker.py:1048-1089."""
        bs = candidates.shape[0]
        target = None
        if self.target_distribution is not None:
            outputs = self.target_distribution.sample_prefix(
                candidates=candidates, next_token_logits=next_token_logits, sampling_info=sampling_info,
                prefix_lens=torch.zeros(bs, device=candidates.device, dtype=torch.int32), bs=bs,
                verify_lens=torch.full((bs,), self.block_size, device=candidates.device, dtype=torch.int32))
            if outputs is not None:
                return outputs[0], outputs[2]
            target = self.target_distribution.dense(next_token_logits, sampling_info, bs)
        return dspine_accept_sampling(target_probs=target, candidates=candidates, target_logits=next_token_logits,
                                      candidate_ids=candidate_ids, q_rows=q_rows, sampling_info=sampling_info,
                                      sampling_backend=self.sampling_backend,
                                      random_state=self._dspine_sampler.random)


def set_active_worker(worker) -> None:
    global _active_worker
    _active_worker = worker


def accept_dspine_sampled_round(*, candidates, next_token_logits, sampling_info, max_top_k=None,
                                uniform_top_k_value=None, **_dflash_only_arguments):
    """Seam C (runtime/worker.py:1092-1115): (accept_len int32 [bs], bonus int64 [bs]) of this
    round's drafts under the request's ordinary target distribution."""
    worker = _active_worker
    if worker is None:
        raise RuntimeError("DSPINE sampled verify reached before the DSpine worker exists")
    return worker._accept_sampled_round(candidates=candidates, next_token_logits=next_token_logits,
                                        sampling_info=sampling_info, max_top_k=max_top_k,
                                        uniform_top_k_value=uniform_top_k_value)


def commit_accept(outputs, *, prefix_lens, req_pool_indices, req_to_token, out_cache_loc=None,
                  verify_lens=None, slot_offsets=None, seq_lens=None, free_slots=None, free_count=None):
    """Commit one verified round (``dsv_commit_accept``): what SGLang's speculative worker does
    with the accept / bonus buffers after verification (its ``_commit_accept``, which the
    reference's tests/test_tp_accept.py:106-180 drive; SGLang itself is not part of the
    reference, so this is the closed form).

    ``outputs`` is the round's 5-tuple (only ``accept`` [bs] int32 is read; the caller keeps the
    buffers, which the worker double-buffers).  Request b verified positions
    ``prefix_lens[b] + i`` for ``i < verify_lens[b]`` (default: the block width T) and commits the
    first ``accept[b] + 1``.  With ``out_cache_loc`` (int64 window slots, ``b*T + i`` or
    ``slot_offsets[b] + i``) the committed slots are written into ``req_to_token[
    req_pool_indices[b], prefix + i]``; without it the slots are already in the table.
    ``seq_lens[req_pool_indices[b]]`` becomes ``prefix + accept + 1``; the slots of the rejected
    positions are compacted into ``free_slots`` (int64, (b, i) order) and counted in
    ``free_count[0]``.  Returns ``(free_slots, free_count)``."""
    accept, output = outputs[0], outputs[3]
    bs, T = output.shape
    dev = _lib.require_cuda(accept, prefix_lens, req_pool_indices, req_to_token, out_cache_loc, verify_lens,
                            slot_offsets, seq_lens, free_slots, free_count)
    if accept.shape != (bs,) or accept.dtype != torch.int32 or not accept.is_contiguous():
        raise ValueError("accept must be contiguous int32 [bs]")
    for name, t in (("prefix_lens", prefix_lens), ("req_pool_indices", req_pool_indices)):
        if t.shape != (bs,) or t.dtype not in (torch.int32, torch.int64) or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int32/int64 [bs] vector")
    if req_to_token.ndim != 2 or req_to_token.dtype != torch.int32 or req_to_token.stride(1) != 1:
        raise ValueError("req_to_token must be a row-contiguous int32 [pool, context] table")
    if verify_lens is not None and (verify_lens.shape != (bs,) or verify_lens.dtype != torch.int32
                                    or not verify_lens.is_contiguous()):
        raise ValueError("verify_lens must be contiguous int32 [bs]")
    if out_cache_loc is not None and (out_cache_loc.dtype != torch.int64 or not out_cache_loc.is_contiguous()):
        raise ValueError("out_cache_loc must be contiguous int64")
    if out_cache_loc is not None and slot_offsets is None and out_cache_loc.numel() < bs * T:
        raise ValueError("out_cache_loc must hold the [bs*T] window slots")
    if slot_offsets is not None and (slot_offsets.shape != (bs,) or slot_offsets.dtype != torch.int64
                                     or out_cache_loc is None):
        raise ValueError("slot_offsets must be int64 [bs] offsets into out_cache_loc")
    if seq_lens is not None and (seq_lens.dtype not in (torch.int32, torch.int64) or not seq_lens.is_contiguous()):
        raise ValueError("seq_lens must be a contiguous int32/int64 vector")
    if free_slots is None:
        free_slots = torch.empty(bs * T, device=dev, dtype=torch.int64)
    elif free_slots.dtype != torch.int64 or free_slots.numel() < bs * T or not free_slots.is_contiguous():
        raise ValueError("free_slots must be contiguous int64 with room for bs*T slots")
    if free_count is None:
        free_count = torch.empty(1, device=dev, dtype=torch.int32)
    elif free_count.dtype != torch.int32 or free_count.numel() < 1:
        raise ValueError("free_count must be int32 [1]")
    _lib.check(_lib.load().dsv_commit_accept(
        bs, T, accept.data_ptr(), _lib.ptr(verify_lens), prefix_lens.data_ptr(),
        int(prefix_lens.dtype == torch.int64), req_pool_indices.data_ptr(), int(req_pool_indices.dtype == torch.int64),
        req_to_token.data_ptr(), req_to_token.stride(0), req_to_token.shape[1], _lib.ptr(out_cache_loc),
        _lib.ptr(slot_offsets), _lib.ptr(seq_lens), int(seq_lens is not None and seq_lens.dtype == torch.int64),
        free_slots.data_ptr(), free_count.data_ptr(), _lib.stream_of(dev)), "dsv_commit_accept")
    return free_slots, free_count
