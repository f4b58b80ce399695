"""The fused sampled-verify step on MI355X.

One call runs, on the current stream and without host synchronisation, what the reference
spreads over ``build_dspine_target_probs`` (runtime/worker.py:440-508), the dense/sparse
target builders and ``accept_sparse`` (sampling/sparse/accept.py:463-543): logit
adjustments (a presence/repetition penalty over a token history), the temperature softmax,
the top-k / top-p / min-p filter, chain rejection against the draft's sparse q, the residual
``max(p - q, 0)`` resample and the accepted-prefix compaction with the KV-slot gather.  The
target distribution is never materialised: each verified row is read once.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from dspine_amd import _lib

TOP_K_ALL = 1 << 30


@dataclass
class History:
    """Per-request penalty history: ids [bs, H] int32 (-1 = padding), presence and repetition
    [bs] float32.  Equivalent to SGLang's dense buffers ``acc_additive_penalties = -presence``
    and ``acc_scaling_penalties = repetition`` on the history tokens."""

    ids: torch.Tensor
    presence: torch.Tensor
    repetition: torch.Tensor


def new_outputs(bs: int, T: int, device, kv_slots: bool = True):
    """Caller-owned output buffers in the reference's convention
    (accept i32, commit i32, bonus i64, output i64 [bs, T], new_seq i32) + kv_slots i32."""
    outs = (
        torch.empty(bs, device=device, dtype=torch.int32),
        torch.empty(bs, device=device, dtype=torch.int32),
        torch.empty(bs, device=device, dtype=torch.int64),
        torch.empty((bs, T), device=device, dtype=torch.int64),
        torch.empty(bs, device=device, dtype=torch.int32),
    )
    kv = torch.empty((bs, T), device=device, dtype=torch.int32) if kv_slots else None
    return outs, kv


class Workspace:
    """Grow-only scratch owned by the caller (like TargetDistribution.scratch,
    sampling/target.py:94-104)."""

    def __init__(self):
        self.buf = None

    def get(self, nbytes: int, device) -> torch.Tensor:
        if self.buf is None or self.buf.device != device or self.buf.numel() < nbytes:
            size = max(nbytes, 2 * self.buf.numel() if self.buf is not None else 0)
            self.buf = torch.empty(size, dtype=torch.uint8, device=device)
        return self.buf


_default_ws: dict = {}


def _f32(t, name, n, device):
    if t is None:
        return None
    t = t.reshape(-1)
    if t.numel() != n:
        raise ValueError(f"{name} must hold {n} values, got {t.numel()}")
    return t.to(device=device, dtype=torch.float32).contiguous()


def _i32(t, name, n, device):
    if t is None:
        return None
    t = t.reshape(-1)
    if t.numel() != n:
        raise ValueError(f"{name} must hold {n} values, got {t.numel()}")
    return t.to(device=device, dtype=torch.int32).contiguous()


def _contig(t, name):
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def verify_step(*, logits: torch.Tensor, sampling_info, candidates: torch.Tensor,
                q_ids: torch.Tensor, q_values: torch.Tensor, uniforms: torch.Tensor,
                uniform_final: torch.Tensor, prefix_lens: torch.Tensor,
                verify_lens: torch.Tensor | None = None, row_offsets: torch.Tensor | None = None,
                history: History | None = None, page_table: torch.Tensor | None = None,
                outputs=None, kv_slots: torch.Tensor | None = None,
                sampling_backend: str = "pytorch", sparse_joint: bool = False,
                workspace: Workspace | None = None, _stages: int = 0):
    """Verify one round.  Returns ``(outputs, kv_slots)`` where outputs is the 5-tuple
    ``(accept, commit, bonus, output, new_seq)``.

    logits [rows, V] bf16/fp32: rows ``b*T + s`` (dense, rows == bs*T) or ``row_offsets[b] + s``
    (ragged).  candidates [bs, T] int64 (anchor + T-1 drafts); q_ids / q_values [bs, T-1, K]
    (the sparse q each draft was sampled from); uniforms [bs, T-1], uniform_final [bs] float32;
    prefix_lens [bs] int32; verify_lens [bs] int32 in [1, T] (default T).  ``sampling_info``
    supplies temperatures, top_ks (>= 2^30 = off), top_ps, min_ps and the need_* /
    is_any_greedy flags, as SGLang's SamplingBatchInfo does.  Rows of requests with top_k <= 1
    are greedy when ``is_any_greedy``.  ``sparse_joint`` selects the reference's sparse joint
    target (sampling/sparse/target.py:95-178; the flashinfer backend, no min-p, no greedy rows,
    max_top_k <= 32) in place of the backend filter.  Contract violations raise ValueError before
    any launch.
    """
    lib = _lib.load()
    dev = _lib.require_cuda(logits, candidates, q_ids, q_values, uniforms, uniform_final,
                            prefix_lens, verify_lens, row_offsets, page_table)
    if logits.ndim != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be a row-contiguous [rows, V] tensor")
    if candidates.ndim != 2 or candidates.dtype != torch.int64:
        raise ValueError("candidates must be int64 [bs, T]")
    bs, T = candidates.shape
    if T < 1 or bs < 1:
        raise ValueError("empty verification batch")
    if q_ids.ndim != 3 or tuple(q_ids.shape[:2]) != (bs, T - 1) or q_values.shape != q_ids.shape:
        raise ValueError("q_ids / q_values must be [bs, T-1, K]")
    if q_ids.dtype not in (torch.int32, torch.int64) or q_values.dtype != torch.float32:
        raise ValueError("q_ids must be int32/int64 and q_values float32")
    if uniforms.shape != (bs, T - 1) or uniforms.dtype != torch.float32:
        raise ValueError("uniforms must be float32 [bs, T-1]")
    if uniform_final.shape != (bs,) or uniform_final.dtype != torch.float32:
        raise ValueError("uniform_final must be float32 [bs]")
    if prefix_lens.shape != (bs,) or prefix_lens.dtype != torch.int32:
        raise ValueError("prefix_lens must be int32 [bs]")
    rows, V = logits.shape
    if row_offsets is None and rows != bs * T:
        raise ValueError(f"dense layout needs logits rows == bs*T ({rows} != {bs}*{T})")
    if row_offsets is not None:
        if row_offsets.shape != (bs,) or row_offsets.dtype not in (torch.int32, torch.int64):
            raise ValueError("row_offsets must be an int32/int64 vector of batch size")
        _contig(row_offsets, "row_offsets")
    if verify_lens is not None:
        if verify_lens.shape != (bs,) or verify_lens.dtype != torch.int32:
            raise ValueError("verify_lens must be int32 [bs]")
        _contig(verify_lens, "verify_lens")
    for name, t in (("candidates", candidates), ("q_ids", q_ids), ("q_values", q_values),
                    ("uniforms", uniforms), ("uniform_final", uniform_final),
                    ("prefix_lens", prefix_lens)):
        _contig(t, name)
    a = _lib.VerifyArgs()
    keep = sampling_fields(a, sampling_info, bs, dev, sampling_backend)
    if outputs is None:
        outputs, kv_new = new_outputs(bs, T, dev, kv_slots=page_table is not None)
        if kv_slots is None:
            kv_slots = kv_new
    if len(outputs) != 5:
        raise ValueError("Expected accept/commit/bonus/output/new_seq buffers")
    accept, commit, bonus, output, new_seq = outputs
    if (accept.dtype, commit.dtype, bonus.dtype, output.dtype, new_seq.dtype) != (
            torch.int32, torch.int32, torch.int64, torch.int64, torch.int32) or output.shape != (bs, T):
        raise ValueError("output buffers must be (i32 [bs], i32 [bs], i64 [bs], i64 [bs, T], i32 [bs])")
    if kv_slots is not None and (kv_slots.shape != (bs, T) or kv_slots.dtype != torch.int32):
        raise ValueError("kv_slots must be int32 [bs, T]")
    hist = pres = rep = None
    hist_len = 0
    if history is not None:
        hist = history.ids.to(device=dev, dtype=torch.int32).contiguous()
        if hist.ndim != 2 or hist.shape[0] != bs:
            raise ValueError("history ids must be [bs, H]")
        hist_len = hist.shape[1]
        pres = _f32(history.presence, "presence", bs, dev)
        rep = _f32(history.repetition, "repetition", bs, dev)
    if page_table is not None:
        if page_table.ndim != 2 or page_table.shape[0] != bs or page_table.dtype != torch.int32:
            raise ValueError("page_table must be int32 [bs, L]")
        if page_table.stride(1) != 1:
            raise ValueError("page_table rows must be contiguous")
    ws = workspace if workspace is not None else _default_ws.setdefault(dev, Workspace())
    nbytes = int(lib.dsv_verify_workspace_bytes(rows, bs, T, V))
    wbuf = ws.get(nbytes, dev)
    a.logits = logits.data_ptr()
    a.logits_dtype = _lib.dtype_code(logits)
    a.rows, a.vocab, a.row_stride = rows, V, logits.stride(0)
    a.bs, a.T = bs, T
    a.verify_lens = _lib.ptr(verify_lens)
    a.row_offsets = _lib.ptr(row_offsets)
    a.row_offsets_i64 = int(row_offsets is not None and row_offsets.dtype == torch.int64)
    a.hist_ids, a.hist_len = _lib.ptr(hist), hist_len
    a.presence, a.repetition = _lib.ptr(pres), _lib.ptr(rep)
    a.candidates = candidates.data_ptr()
    a.q_ids, a.q_ids_i64, a.K = q_ids.data_ptr(), int(q_ids.dtype == torch.int64), q_ids.shape[2]
    a.q_values = q_values.data_ptr()
    a.uniforms, a.uniform_final = uniforms.data_ptr(), uniform_final.data_ptr()
    a.prefix_lens = prefix_lens.data_ptr()
    if page_table is not None:
        a.page_table, a.page_stride, a.page_cols = page_table.data_ptr(), page_table.stride(0), page_table.shape[1]
    a.accept, a.commit, a.bonus = accept.data_ptr(), commit.data_ptr(), bonus.data_ptr()
    a.output, a.new_seq = output.data_ptr(), new_seq.data_ptr()
    a.kv_slots = _lib.ptr(kv_slots)
    a.workspace, a.workspace_bytes = wbuf.data_ptr(), wbuf.numel()
    a.stages = int(_stages)
    a.sparse_joint = int(bool(sparse_joint))
    _lib.check(lib.dsv_verify(a, _lib.stream_of(dev)), "dsv_verify")
    del keep
    return outputs, kv_slots


def sampling_fields(a, info, bs: int, dev, sampling_backend: str):
    """Fill the sampling-parameter fields of ``dsv_verify_args`` from a duck-typed
    SamplingBatchInfo (temperatures [bs] or [bs, 1], top_ks, top_ps, min_ps, the need_* and
    is_any_greedy flags, max_top_k).  Returns the converted tensors (they must outlive the
    launch)."""
    if sampling_backend not in ("pytorch", "flashinfer"):
        raise ValueError(f"unsupported sampling backend {sampling_backend!r}")
    temps = _f32(info.temperatures, "temperatures", bs, dev)
    top_ks = _i32(info.top_ks, "top_ks", bs, dev)
    top_ps = _f32(info.top_ps, "top_ps", bs, dev)
    min_ps = _f32(getattr(info, "min_ps", None), "min_ps", bs, dev)
    need_k = bool(getattr(info, "need_top_k_sampling", False))
    need_p = bool(getattr(info, "need_top_p_sampling", False))
    need_min_p = bool(getattr(info, "need_min_p_sampling", False))
    max_top_k = getattr(info, "max_top_k", None)
    if not isinstance(max_top_k, int):
        max_top_k = TOP_K_ALL  # unknown on the host: nucleus rows may occur
    a.backend = _lib.DSV_BACKEND_PYTORCH if sampling_backend == "pytorch" else _lib.DSV_BACKEND_FLASHINFER
    a.temperatures, a.top_ks, a.top_ps = _lib.ptr(temps), top_ks.data_ptr(), top_ps.data_ptr()
    a.min_ps = _lib.ptr(min_ps)
    a.filter = int(need_k or need_p or need_min_p)
    a.need_min_p = int(need_min_p)
    a.any_greedy = int(bool(getattr(info, "is_any_greedy", False)))
    a.max_top_k = int(min(max_top_k, 2**31 - 1))
    return (temps, top_ks, top_ps, min_ps)


def target_probs(logits: torch.Tensor, info, *, bs: int, T: int, sampling_backend: str = "pytorch",
                 normalize: bool = True, out: torch.Tensor | None = None,
                 workspace: Workspace | None = None) -> torch.Tensor:
    """Dense target P [rows, V] float32 of logits [rows = bs*T, V] (request b owns rows b*T ..
    b*T+T-1): softmax(logits / temperature), the backend filter, renormalised (``normalize``
    False: the filtered softmax p as is); rows of greedy requests one-hot at the argmax; an
    unfiltered batch is the plain softmax (runtime/worker.py:440-508)."""
    lib = _lib.load()
    dev = _lib.require_cuda(logits, out)
    if logits.ndim != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be a row-contiguous [rows, V] tensor")
    rows, V = logits.shape
    if bs < 1 or T < 1 or rows != bs * T:
        raise ValueError(f"logits rows {rows} != bs*T ({bs}*{T})")
    if out is None:
        out = torch.empty((rows, V), device=dev, dtype=torch.float32)
    if out.shape != (rows, V) or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError("out must be a row-contiguous float32 [rows, V] tensor")
    a = _lib.VerifyArgs()
    keep = sampling_fields(a, info, bs, dev, sampling_backend)
    ws = workspace if workspace is not None else _default_ws.setdefault(dev, Workspace())
    wbuf = ws.get(int(lib.dsv_verify_workspace_bytes(rows, bs, T, V)), dev)
    a.logits, a.logits_dtype = logits.data_ptr(), _lib.dtype_code(logits)
    a.rows, a.vocab, a.row_stride = rows, V, logits.stride(0)
    a.bs, a.T = bs, T
    a.workspace, a.workspace_bytes = wbuf.data_ptr(), wbuf.numel()
    _lib.check(lib.dsv_target_probs(a, out.data_ptr(), out.stride(0), int(bool(normalize)),
                                    _lib.stream_of(dev)), "dsv_target_probs")
    del keep
    return out
