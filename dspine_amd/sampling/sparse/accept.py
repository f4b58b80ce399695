"""Support compaction and chain rejection with sparse q on given distributions
(sampling/sparse/accept.py of the reference).

``compress_probs`` packs each row's p > 0 entries in id order (one HIP workgroup per row, a
single pass over the row); ``accept_sparse`` runs the chain rejection, residual resample and
compaction with the draft's sparse q lanes against dense, RAW (p / denominator) or packed P in
one HIP workgroup per request.  Both launch on the current stream without host
synchronisation and write caller-owned buffers.
"""

from __future__ import annotations

import torch as _torch

from dspine_amd import _lib

PACKED_MAX = 64  # largest packed capacity accept_sparse reads


def compress_probs(torch, p, capacity=64):
    """p [rows, V] float32 -> (ids int32 [rows, capacity], values float32 [rows, capacity],
    lengths int32 [rows], overflow int32 [rows]) (sparse/accept.py:422-460).

    Per row: the ids with p > 0 in ascending id order, up to ``capacity``; unused slots hold
    id -1 / value 0; lengths = min(n, capacity); overflow = n > capacity or any negative, NaN
    or infinite p."""
    del torch  # the reference passes its torch module; this build always uses its own
    if p.ndim != 2 or p.dtype != _torch.float32 or p.stride(1) != 1:
        raise ValueError("compress_probs expects a row-contiguous float32 [rows, V] tensor")
    if not isinstance(capacity, int) or capacity < 1:
        raise ValueError("compress_probs capacity must be a positive integer")
    dev = _lib.require_cuda(p)
    rows, vocab = p.shape
    ids = _torch.empty((rows, capacity), device=dev, dtype=_torch.int32)
    values = _torch.empty((rows, capacity), device=dev, dtype=_torch.float32)
    lengths = _torch.empty(rows, device=dev, dtype=_torch.int32)
    overflow = _torch.empty(rows, device=dev, dtype=_torch.int32)
    if rows:
        _lib.check(_lib.load().dsv_compress(p.data_ptr(), rows, vocab, p.stride(0), capacity, ids.data_ptr(),
                                            values.data_ptr(), lengths.data_ptr(), overflow.data_ptr(),
                                            _lib.stream_of(dev)), "dsv_compress")
    return (ids, values, lengths, overflow)


def _check_outputs(outputs, bs, t):
    if len(outputs) != 5:
        raise ValueError("Expected accept/commit/bonus/output/new_seq buffers")
    accept, commit, bonus, output, new_seq = outputs
    if (accept.dtype, commit.dtype, bonus.dtype, output.dtype, new_seq.dtype) != (
            _torch.int32, _torch.int32, _torch.int64, _torch.int64, _torch.int32):
        raise ValueError("output buffers must be (int32, int32, int64, int64, int32)")
    if accept.numel() < bs or commit.numel() < bs or bonus.numel() < bs or new_seq.numel() < bs \
            or tuple(output.shape) != (bs, t):
        raise ValueError("output buffers do not match the batch")
    if any(not x.is_contiguous() for x in outputs):
        raise ValueError("output buffers must be contiguous")


def _vec(x, name, bs, dtype):
    """A per-request vector as a contiguous tensor of the ABI dtype (a copy only when the
    caller's integer width differs)."""
    if x.shape != (bs,):
        raise ValueError(f"{name} must be a vector of batch size")
    if x.dtype != dtype:
        if x.is_floating_point() != dtype.is_floating_point:
            raise ValueError(f"{name} has dtype {x.dtype}")
        x = x.to(dtype)
    return x.contiguous()


def fill_chain_args(a, *, candidates, verify_lens, uniforms, uniform_final, prefix_lens, outputs,
                    row_offsets=None):
    """The request-side fields of ``dsv_chain_args`` (shared by every chain entry point).
    Returns the tensors that must outlive the launch."""
    bs, t = candidates.shape
    if candidates.dtype != _torch.int64 or not candidates.is_contiguous():
        raise ValueError("candidates must be contiguous int64 [bs, T]")
    if t < 2:
        raise ValueError("chain rejection needs at least one draft (T >= 2)")
    if uniforms.shape != (bs, t - 1) or uniforms.dtype != _torch.float32 or not uniforms.is_contiguous():
        raise ValueError("Invalid cap or uniform layout")
    if uniform_final.shape != (bs,) or uniform_final.dtype != _torch.float32 or not uniform_final.is_contiguous():
        raise ValueError("Invalid final uniform or prefix layout")
    keep = []
    vl = None
    if verify_lens is not None:
        vl = _vec(verify_lens, "verify_lens", bs, _torch.int32)
        keep.append(vl)
    pl = _vec(prefix_lens, "prefix_lens", bs, _torch.int32)
    keep.append(pl)
    _check_outputs(outputs, bs, t)
    if row_offsets is not None:
        if (row_offsets.shape != (bs,) or row_offsets.device != candidates.device
                or row_offsets.dtype not in (_torch.int32, _torch.int64) or not row_offsets.is_contiguous()):
            raise ValueError("row_offsets must be a contiguous device int32/int64 vector of batch size")
    a.bs, a.T = bs, t
    a.candidates = candidates.data_ptr()
    a.verify_lens = _lib.ptr(vl)
    a.uniforms, a.uniform_final = uniforms.data_ptr(), uniform_final.data_ptr()
    a.prefix_lens = pl.data_ptr()
    a.row_offsets = _lib.ptr(row_offsets)
    a.row_offsets_i64 = int(row_offsets is not None and row_offsets.dtype == _torch.int64)
    acc, com, bon, out, new = outputs
    a.accept, a.commit, a.bonus = acc.data_ptr(), com.data_ptr(), bon.data_ptr()
    a.output, a.new_seq = out.data_ptr(), new.data_ptr()
    return keep


def fill_sparse_q(a, q_ids, q_values, bs, t):
    if q_ids.ndim != 3 or tuple(q_ids.shape[:2]) != (bs, t - 1) or q_values.shape != q_ids.shape:
        raise ValueError("q_ids / q_values must be [bs, T-1, K]")
    if q_ids.dtype not in (_torch.int32, _torch.int64) or q_values.dtype != _torch.float32:
        raise ValueError("q_ids must be int32/int64 and q_values float32")
    if not (q_ids.is_contiguous() and q_values.is_contiguous()):
        raise ValueError("q_ids / q_values must be contiguous")
    a.K = q_ids.shape[2]
    a.q_ids, a.q_ids_i64 = q_ids.data_ptr(), int(q_ids.dtype == _torch.int64)
    a.q_values = q_values.data_ptr()


def accept_sparse(torch, *, candidates, dense_p, packed, q_ids, q_values, verify_lens, uniforms,
                  uniform_final, prefix_lens, outputs, scratch=None, denominator=None,
                  raw_fallback=False, row_offsets=None, vocab_size=None, overflow_read=None):
    """Chain rejection with sparse q (sparse/accept.py:463-543); writes and returns ``outputs``
    = (accept int32 [bs], commit int32 [bs], bonus int64 [bs], output int64 [bs, T],
    new_seq int32 [bs]).

    P of draft step s of request b is row ``row_offsets[b] + s`` (else ``b*T + s``) of
    ``dense_p`` [rows, V] float32 (divided by ``denominator[row]`` when ``raw_fallback``) or of
    ``packed`` = (ids, values, lengths, overflow) [rows, cap] on rows whose overflow flag is 0.
    q_ids / q_values [bs, T-1, K]: a draft's q is the sum of its lanes; the residual of a dense
    row subtracts the clamped q of the last lane with an id, that of a packed row the clamped q
    summed over the lanes with the id.  ``scratch`` is accepted for the reference's signature
    (the HIP kernel keeps its tiles in LDS).  T >= 2 and K <= 64 (the reference is fixed at
    T = K = 16).

    ``overflow_read`` (optional int32 [bs], written on the device): 1 for a request that read a
    packed row flagged overflow with no ``dense_p`` to fall back on -- where the reference stops
    on the device (sparse/accept.py:257, :291), its outputs come from the row's packed prefix --
    else 0."""
    del torch, scratch
    bs, t = candidates.shape
    if dense_p is None:
        if packed is None or type(vocab_size) is not int or vocab_size < 1:
            raise ValueError("Pure packed rejection requires packed probabilities and vocab_size")
        if raw_fallback:
            raise ValueError("Pure packed rejection requires normalized packed probabilities")
        vocab = vocab_size
    else:
        vocab = dense_p.shape[-1]
        if vocab_size is not None and vocab_size != vocab:
            raise ValueError("vocab_size differs from the dense fallback")
        if dense_p.ndim != 2 or dense_p.dtype != _torch.float32 or dense_p.stride(1) != 1:
            raise ValueError("dense_p must be a row-contiguous float32 [rows, V] tensor")
    if row_offsets is not None:
        if (row_offsets.shape != (bs,) or row_offsets.device != candidates.device
                or row_offsets.dtype not in (_torch.int32, _torch.int64) or not row_offsets.is_contiguous()):
            raise ValueError("row_offsets must be a contiguous device int32/int64 vector of batch size")
    if denominator is None and raw_fallback:
        raise ValueError("Unnormalized target probabilities require a denominator")
    dev = _lib.require_cuda(candidates, dense_p, q_ids, q_values, uniforms, uniform_final, prefix_lens,
                            verify_lens, row_offsets, denominator)
    a = _lib.ChainArgs()
    keep = fill_chain_args(a, candidates=candidates, verify_lens=verify_lens, uniforms=uniforms,
                           uniform_final=uniform_final, prefix_lens=prefix_lens, outputs=outputs,
                           row_offsets=row_offsets)
    fill_sparse_q(a, q_ids, q_values, bs, t)
    a.vocab = vocab
    if dense_p is not None:
        a.dense_p, a.p_stride = dense_p.data_ptr(), dense_p.stride(0)
        if raw_fallback:
            den = denominator.reshape(-1)
            if den.dtype != _torch.float32 or den.numel() != dense_p.shape[0] or not den.is_contiguous():
                raise ValueError("denominator must be contiguous float32 [rows]")
            a.denominator = den.data_ptr()
            keep.append(den)
    if packed is not None:
        ids, vals, lens, overflow = packed
        rows = ids.shape[0]
        if ids.ndim != 2 or vals.shape != ids.shape or lens.shape != (rows,) or overflow.shape != (rows,):
            raise ValueError("packed P must be (ids [rows, cap], values [rows, cap], lengths [rows], overflow [rows])")
        if (ids.dtype, vals.dtype, lens.dtype, overflow.dtype) != (
                _torch.int32, _torch.float32, _torch.int32, _torch.int32):
            raise ValueError("packed P must be (int32, float32, int32, int32)")
        if not all(x.is_contiguous() for x in packed):
            raise ValueError("packed P must be contiguous")
        if ids.shape[1] > PACKED_MAX:
            raise ValueError(f"packed capacity {ids.shape[1]} exceeds {PACKED_MAX}")
        _lib.require_cuda(*packed)
        a.p_ids, a.p_values, a.p_lengths = ids.data_ptr(), vals.data_ptr(), lens.data_ptr()
        a.p_overflow, a.p_cap = overflow.data_ptr(), ids.shape[1]
    if overflow_read is not None:
        if (overflow_read.shape != (bs,) or overflow_read.dtype != _torch.int32 or not overflow_read.is_contiguous()
                or overflow_read.device != candidates.device):
            raise ValueError("overflow_read must be a contiguous device int32 [bs] tensor")
        a.overflow_read = overflow_read.data_ptr()
    if bs:
        _lib.check(_lib.load().dsv_accept_chain(a, _lib.stream_of(dev)), "dsv_accept_chain")
    del keep
    return outputs
