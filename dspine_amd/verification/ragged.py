"""Acceptance for ragged (per-request length) verification (verification/ragged.py of the
reference): the ``RaggedVerifyCaps.accept`` body on this package's kernels."""

from __future__ import annotations

from dspine_amd.verification import caps


def accept(self, *, candidates, next_token_logits, sampling_info, draft_input, prefix_lens, bs):
    """``RaggedVerifyCaps.accept`` (verification/ragged.py:282-335), written as a plain function
    of the controller so that it binds as the method (``RaggedVerifyCaps.accept =
    ragged.accept``).

    A round that is not ragged takes the capped path (``caps.accept``, the parent class's
    method).  A ragged round must be the confirmed packed verification of this batch
    (``batch_size``, ``executed_tokens == tokens``).  Sampled rounds verify against this round's
    q with the layout's per-request lengths -- compact rows (``compact_round``) by their row
    offsets and row-to-request map; greedy rounds run the fused argmax + acceptance with those
    lengths (``dsv_greedy_verify``) over the full [bs*full, V] row envelope."""
    if not self.ragged_round:
        return caps.accept(self, candidates=candidates, next_token_logits=next_token_logits,
                           sampling_info=sampling_info, draft_input=draft_input, prefix_lens=prefix_lens,
                           bs=bs)
    if bs != self.batch_size or self.executed_tokens != self.tokens:
        raise RuntimeError("Ragged acceptance requires confirmed packed verification")
    if self.sampled_round:
        from dspine_amd.sampling.rejection import accept_sampled_prefix

        compact = bool(getattr(self, "compact_round", False))
        return accept_sampled_prefix(self, candidates=candidates, next_token_logits=next_token_logits,
                                     sampling_info=sampling_info, prefix_lens=prefix_lens, bs=bs,
                                     verify_lens=self.layout.verify_lens,
                                     row_offsets=self.row_offsets if compact else None,
                                     row_to_request=self.row_to_request if compact else None)
    if candidates.shape != (bs, self.full):
        raise ValueError(f"Ragged acceptance requires full{self.full} proposal storage")
    outputs = self.worker._next_accept_bonus_buffers(bs)
    return caps.accept_greedy(candidates=candidates, next_token_logits=next_token_logits,
                              prefix_lens=caps._prefix_i32(prefix_lens), verify_lens=self.layout.verify_lens,
                              outputs=outputs)
