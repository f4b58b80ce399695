"""Target distributions with sparse-q chain rejection (sampling/target.py of the reference).

``sample_prefix`` verifies a round in one fused HIP pass (``dsv_verify``): the target
distribution of each verified row is computed and consumed in registers/LDS, never written to
HBM.  Batches the reference sends through ``build_sparse_target`` get its sparse joint target
(every value tied with the k-th kept, the nucleus on the strictly larger mass, rows keeping more
than 32 values dense); the others the backend filter of ``build_dspine_target_probs``.  ``dense``
materialises P for callers that need it.
"""

from __future__ import annotations

import copy

import torch

from dspine_amd.sampling.random import verification_uniforms
from dspine_amd.sampling.sparse.target import sparse_eligible
from dspine_amd.verify import Workspace, verify_step

SPARSE_Q_WIDTH = 16  # the q width of the reference's sparse-q path (sampling/target.py:53-54)


def sparse_route(info, sampling_backend: str, vocab: int, q_width: int) -> bool:
    """Whether ``sample_prefix`` verifies against the sparse joint target: the reference's
    sparse-q path (K = 16 q lanes, sampling/target.py:53-54) with a batch that
    ``build_sparse_target`` accepts (sampling/target.py:58-66, sparse/target.py:106-116).  Other
    batches use the backend filter of ``build_dspine_target_probs``."""
    return q_width == SPARSE_Q_WIDTH and sparse_eligible(info, sampling_backend, vocab)


class TargetDistribution:
    def __init__(self, worker):
        self.worker = worker
        self.scratch = Workspace()  # grow-only (sampling/target.py:94-104)

    def dense(self, logits, info, bs, row_to_request=None):
        """P [bs, T, V] float32 of full blocks, or [rows, 1, V] of compact rows mapped to their
        requests by ``row_to_request`` (sampling/target.py:15-32)."""
        from dspine_amd.runtime.worker import build_dspine_target_probs

        width = int(self.worker.block_size)
        if row_to_request is not None:
            info = copy.copy(info)
            for name in ("temperatures", "top_ks", "top_ps", "min_ps"):
                value = getattr(info, name, None)
                if value is not None:
                    setattr(info, name, value.reshape(-1).index_select(0, row_to_request))
            bs, width = logits.shape[0], 1
        return build_dspine_target_probs(next_token_logits=logits, sampling_info=info, block_size=width, bs=bs,
                                         sampling_backend=self.worker.sampling_backend)

    def sample_prefix(self, *, candidates, next_token_logits, sampling_info, prefix_lens, bs, verify_lens,
                      row_offsets=None, row_to_request=None):
        """Verify one (possibly shortened) target call against this round's sampled q
        (sampling/target.py:34-122).  Rows are ``b*T + s`` or compact ``row_offsets[b] + s``.
        Returns the worker's next output buffers.  Compact rows need their ``row_offsets``:
        ``row_to_request`` without them raises ValueError (the reference would read the compact
        rows as ``b*T + s`` there; its callers always pass both, verification/ragged.py:329-331)."""
        sampler = self.worker._dspine_sampler
        if not sampler.round_sampled or sampler.round_bs != bs:
            raise RuntimeError("Sparse rejection must consume this round's actual proposal q")
        width = int(self.worker.block_size)
        if candidates.shape != (bs, width):
            raise ValueError("Proposal storage does not match this decode batch")
        if row_to_request is not None and row_offsets is None:
            raise ValueError("Compact verification rows (row_to_request) need their row_offsets")
        outputs = self.worker._next_accept_bonus_buffers(bs)
        uniforms, final = verification_uniforms(bs, width, candidates.device, sampler.random)
        q_ids = sampler.candidate_out[:bs]
        q_values = sampler.q_out[:bs]
        if q_values.dtype != torch.float32:
            q_values = q_values.float()
        backend = self.worker.sampling_backend
        sparse = sparse_route(sampling_info, backend, next_token_logits.shape[-1], q_ids.shape[-1])
        verify_step(logits=next_token_logits, sampling_info=sampling_info, candidates=candidates,
                    q_ids=q_ids.contiguous(), q_values=q_values.contiguous(), uniforms=uniforms,
                    uniform_final=final, prefix_lens=prefix_lens.to(torch.int32), verify_lens=verify_lens,
                    row_offsets=row_offsets, outputs=outputs, sampling_backend=backend,
                    sparse_joint=sparse, workspace=self.scratch)
        return outputs
