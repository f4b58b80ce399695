"""Top-k of verification rows (kernels/dspine.py:165-207 of the reference).

The reference's two-stage Triton top-k returns the k largest ids of each row ascending by id,
with the value multiset of ``torch.topk`` and boundary ties to lower ids inside the chosen
chunks.  Here a single streaming HIP kernel selects the exact top-k under the
``(value desc, id asc)`` order of ``layers/fp8/coarse.py:19-34`` / ``sampling/tp_head.py:9-14``,
so ties at the k-th place always go to the lowest ids.  k is any value in [1, 256].
"""

from __future__ import annotations

import torch

from dspine_amd import _lib
from dspine_amd.verify import Workspace

TOPK_MAX = 256
_ws: dict = {}


def _workspace(logits: torch.Tensor, k: int) -> torch.Tensor:
    lib = _lib.load()
    nbytes = int(lib.dsv_topk_workspace_bytes(logits.shape[0], logits.shape[1], k))
    return _ws.setdefault(logits.device, Workspace()).get(nbytes, logits.device)


def _check(logits: torch.Tensor, k: int):
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("topk expects a row-contiguous [N, V] tensor")
    if not isinstance(k, int) or not 1 <= k <= min(TOPK_MAX, logits.shape[1]):
        raise ValueError(f"topk needs an integer k in [1, min({TOPK_MAX}, V)], got {k}")
    _lib.require_cuda(logits)


def topk(logits: torch.Tensor, k: int, values: torch.Tensor | None = None,
         ids: torch.Tensor | None = None):
    """(values float32 [N, k], ids int64 [N, k]) in (value desc, id asc) order."""
    _check(logits, k)
    n = logits.shape[0]
    if values is None:
        values = torch.empty((n, k), dtype=torch.float32, device=logits.device)
    if ids is None:
        ids = torch.empty((n, k), dtype=torch.int64, device=logits.device)
    if values.shape != (n, k) or ids.shape != (n, k) or values.dtype != torch.float32 \
            or ids.dtype != torch.int64 or not values.is_contiguous() or not ids.is_contiguous():
        raise ValueError("topk outputs must be contiguous float32/int64 [N, k]")
    lib = _lib.load()
    ws = _workspace(logits, k)
    _lib.check(lib.dsv_topk(logits.data_ptr(), _lib.dtype_code(logits), n, logits.shape[1],
                            logits.stride(0), k, values.data_ptr(), ids.data_ptr(), 0,
                            ws.data_ptr(), ws.numel(), _lib.stream_of(logits.device)), "dsv_topk")
    return values, ids


def topk_ids(logits: torch.Tensor, k: int, out: torch.Tensor = None) -> torch.Tensor:
    """logits [N, V] (contiguous rows) -> int64 [N, k] ids of the k largest values,
    ascending by id (kernels/dspine.py:165)."""
    _check(logits, k)
    n = logits.shape[0]
    if out is None:
        out = torch.empty((n, k), dtype=torch.int64, device=logits.device)
    elif tuple(out.shape) != (n, k) or out.dtype != torch.int64 or not out.is_contiguous():
        raise ValueError("topk_ids: out must be a contiguous int64 [N, k] tensor")
    if n == 0:
        return out
    lib = _lib.load()
    ws = _workspace(logits, k)
    _lib.check(lib.dsv_topk(logits.data_ptr(), _lib.dtype_code(logits), n, logits.shape[1],
                            logits.stride(0), k, None, out.data_ptr(), 1,
                            ws.data_ptr(), ws.numel(), _lib.stream_of(logits.device)), "dsv_topk")
    return out


def serial_sample_chain(table, inv_temp, top_k, top_p, min_p, greedy, u, cand, greedy_tok, out_tok, out_q,
                        block_size: int, *, confidence_out=None):
    """Sample every request's draft chain over its K candidate lanes (kernels/dspine.py:677-772);
    fills out_tok[:n] / out_q[:n] in place and returns (out_tok, out_q).

    table float32 [n, K, K] (n = bs*(block_size-1)); inv_temp float32 [>=bs]; top_k int32
    [>=bs] (>= 1; >= K disables it); top_p float32 [>=bs] in (0, 1]; min_p float32 [>=bs] in
    [0, 1]; greedy int32 [>=bs]; u float32 [>=n] in [0, 1); cand int64 [n, K]; greedy_tok int64
    [>=n]; out_tok int64 [>=n]; out_q float32 [>=n, K].  Row i of request b reads row ``sender``
    of its table (the lane drawn at row i-1, lane 0 first): p = softmax(table * inv_t); keep
    rank < top_k, mass ahead <= top_p, p >= min_p * max p (ties: lower lane first);
    q = w / sum w; the drawn lane is #(cdf <= u * total) clamped to the last kept lane.  Greedy
    requests emit greedy_tok with a one-hot q.  ``confidence_out`` float32 [>=n] receives max p
    (before filtering) of each row of a non-greedy request; other entries are left as they are.
    One wavefront per request walks its chain; K <= 64."""
    t = int(block_size)
    n, k = cand.shape
    if t < 2 or n % (t - 1) or tuple(table.shape) != (n, k, k) or not table.is_contiguous():
        raise ValueError("serial_sample_chain table layout mismatch")
    bs = n // (t - 1)
    staged = (inv_temp, top_k, top_p, min_p, greedy)
    if any(x.numel() < bs for x in staged) or u.numel() < n or greedy_tok.numel() < n:
        raise ValueError("serial_sample_chain staging buffers too small")
    if out_tok.numel() < n or out_q.shape[0] < n or out_q.shape[1] != k:
        raise ValueError("serial_sample_chain output buffers too small")
    if not (cand.is_contiguous() and out_q.is_contiguous()):
        raise ValueError("serial_sample_chain expects contiguous candidates and q")
    if confidence_out is not None and (confidence_out.dtype != torch.float32 or confidence_out.numel() < n
                                       or not confidence_out.is_contiguous()
                                       or confidence_out.device != table.device):
        raise ValueError("serial_sample_chain confidence needs contiguous float32 storage on the table device")
    dtypes = (table.dtype, inv_temp.dtype, top_k.dtype, top_p.dtype, min_p.dtype, greedy.dtype, u.dtype,
              cand.dtype, greedy_tok.dtype, out_tok.dtype, out_q.dtype)
    expected = (torch.float32, torch.float32, torch.int32, torch.float32, torch.float32, torch.int32,
                torch.float32, torch.int64, torch.int64, torch.int64, torch.float32)
    if dtypes != expected:
        raise ValueError(f"serial_sample_chain dtype contract violated: {dtypes}")
    if k > 64:
        raise ValueError("serial_sample_chain supports at most 64 candidate lanes")
    staged_c = [x.contiguous() for x in (inv_temp, top_k, top_p, min_p, greedy, u, greedy_tok)]
    if not out_tok.is_contiguous():
        raise ValueError("serial_sample_chain expects contiguous out_tok")
    if bs:
        dev = _lib.require_cuda(table, cand, out_tok, out_q, confidence_out, *staged_c)
        it, tk, tp, mp, gr, uu, gt = staged_c
        _lib.check(_lib.load().dsv_sample_chain(
            table.data_ptr(), n, k, t, it.data_ptr(), tk.data_ptr(), tp.data_ptr(), mp.data_ptr(), gr.data_ptr(),
            uu.data_ptr(), cand.data_ptr(), gt.data_ptr(), out_tok.data_ptr(), out_q.data_ptr(),
            _lib.ptr(confidence_out), _lib.stream_of(dev)), "dsv_sample_chain")
    return (out_tok, out_q)


_rs_ws: dict = {}


def serial_rs_table(raw, rms, query, anchors, cand, codebook, pred_gate_w, prev_w, gate_b, write_w, norm_w, lm_head_w,
                    eps: float, block_size: int, out: torch.Tensor = None, chunk_rows: int = 256,
                    res_emb: torch.Tensor = None, res_proj: torch.Tensor = None,
                    candidate_head: torch.Tensor = None):
    """float32 [n, K, K] sampling table of the serial last-write refinement
    (kernels/dspine.py:505-613), n = bs*(T-1) block rows:
    ``table[n, j, c] = normalize(x + scale * ((gate * value) @ write_w^T)) * norm_w . head[n, c]``
    with ``gate = sigmoid(q + e @ pred_gate_w^T + gate_b)``, ``value = e @ prev_w^T`` (plus
    ``res_emb[s] @ res_proj^T``), ``e = sqrt(C) * codebook[s]`` for sender ``s`` (the anchor on a
    request's first block row, else candidate j of the previous row), ``x``, ``scale``, ``q`` the
    row's pre-write state, write scale and receiver query.  Float32 on the matrix cores in three
    launches (``dsv_rs_table``); ``chunk_rows`` is accepted for the reference's signature (nothing
    is chunked: no intermediate of the size it bounds is materialised).

    raw [bs*T, H], query [bs*T, >= R], codebook [V, C], lm_head_w [V, H], candidate_head
    [n, K, H] and res_emb [V, r] are bfloat16; the weights float32, as the reference requires."""
    t = int(block_size)
    m, h = raw.shape
    bs = m // t
    n, k = cand.shape
    r = pred_gate_w.shape[0]
    if candidate_head is not None and (candidate_head.shape != (n, k, h) or candidate_head.dtype != torch.bfloat16
                                       or not candidate_head.is_contiguous()):
        raise ValueError("serial_rs_table candidate head must be contiguous BF16 [N,K,H]")
    if m % t or n != bs * (t - 1) or rms.shape != (m,) or query.shape[0] != m or query.shape[1] < r \
            or anchors.shape != (bs,):
        raise ValueError("serial_rs_table layout mismatch")
    for name, w in (("pred_gate_w", pred_gate_w), ("prev_w", prev_w), ("gate_b", gate_b), ("write_w", write_w),
                    ("norm_w", norm_w)):
        if w.dtype != torch.float32:
            raise ValueError(f"serial_rs_table: {name} must be fp32")
    if (res_emb is None) != (res_proj is None):
        raise ValueError("serial_rs_table: res_emb and res_proj go together")
    if res_proj is not None and (res_proj.dtype != torch.float32 or res_proj.shape[0] != r
                                 or res_emb.shape != (codebook.shape[0], res_proj.shape[1])):
        raise ValueError("serial_rs_table: terminal residual layout mismatch")
    if out is None:
        out = torch.empty((n, k, k), dtype=torch.float32, device=raw.device)
    elif tuple(out.shape) != (n, k, k) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("serial_rs_table: out must be a contiguous fp32 [n, K, K] tensor")
    if n == 0:
        return out
    c = codebook.shape[1]
    shapes_ok = (pred_gate_w.shape == (r, c) and prev_w.shape == (r, c) and gate_b.numel() == r
                 and write_w.shape == (h, r) and norm_w.numel() == h and lm_head_w.shape[1] == h)
    if not shapes_ok:
        raise ValueError("serial_rs_table: weight shapes do not match the state, rank and codebook widths")
    bf16 = [raw, query, codebook, lm_head_w] + [x for x in (res_emb, candidate_head) if x is not None]
    if any(x.dtype != torch.bfloat16 or x.stride(-1) != 1 for x in bf16):
        raise ValueError("serial_rs_table: raw, query, codebook, head and residual embeddings must be "
                         "row-contiguous bfloat16")
    if anchors.dtype != torch.int64 or cand.dtype != torch.int64 or not cand.is_contiguous():
        raise ValueError("serial_rs_table: anchors and candidates must be (contiguous) int64")
    dev = _lib.require_cuda(raw, rms, query, anchors, cand, codebook, pred_gate_w, prev_w, gate_b, write_w,
                            norm_w, lm_head_w, out, res_emb, res_proj, candidate_head)
    f32c = [x.contiguous() for x in (rms, pred_gate_w, prev_w, gate_b, write_w, norm_w)]
    rp = None if res_proj is None else res_proj.contiguous()
    codebook, lm_head_w = codebook.contiguous(), lm_head_w.contiguous()
    res_emb = None if res_emb is None else res_emb.contiguous()
    lib = _lib.load()
    ws = _rs_ws.setdefault(dev, Workspace()).get(int(lib.dsv_rs_table_workspace_bytes(n, k, h, r)), dev)
    head = lm_head_w if candidate_head is None else candidate_head
    _lib.check(lib.dsv_rs_table(
        raw.data_ptr(), raw.stride(0), f32c[0].data_ptr(), query.data_ptr(), query.stride(0),
        anchors.contiguous().data_ptr(), cand.data_ptr(), n, k, t, codebook.data_ptr(), c, f32c[1].data_ptr(),
        f32c[2].data_ptr(), f32c[3].data_ptr(), f32c[4].data_ptr(), h, r, f32c[5].data_ptr(), head.data_ptr(),
        int(candidate_head is not None), _lib.ptr(res_emb), _lib.ptr(rp), 0 if res_emb is None else res_emb.shape[1],
        float(eps), out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(dev)), "dsv_rs_table")
    return out
