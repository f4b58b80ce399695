"""The factorized q table's per-model cache (sampling/factorized/weights.py of the reference).

``build_cache`` makes, in float64 on the device: W = write [H, R], Gram = W^T W [R, R], norm [H],
bias [R], and per vocabulary row (in chunks of ``chunk`` rows) G = e pred^T, V = e prev^T
(+ res_emb res_proj^T) and TG = (head * norm) W, e = sqrt(C) codebook [rows, C].  The widening
and the products are the library's (``dsv_factor_widen``, ``dsv_factor_gemm`` on the float64
matrix cores).  ``head`` is kept as given (its rows are read by the per-round table).
"""

from __future__ import annotations

import math

import torch

from dspine_amd import _lib


def _widen(src, scale=1.0, mul=None, out=None):
    """float64 copy of a row-contiguous bf16 / float32 [rows, cols] (or [cols]) tensor, times
    scale (and mul[cols])."""
    t = src if src.ndim == 2 else src.reshape(1, -1)
    if t.stride(-1) != 1:
        t = t.contiguous()
    rows, cols = t.shape
    if out is None:
        out = torch.empty((rows, cols), device=t.device, dtype=torch.float64)
    _lib.check(_lib.load().dsv_factor_widen(t.data_ptr(), _lib.dtype_code(t), t.stride(0), rows, cols,
                                            float(scale), _lib.ptr(mul), out.data_ptr(), _lib.stream_of(t.device)),
               "dsv_factor_widen")
    return out if src.ndim == 2 else out.reshape(-1)


def _gemm(a, a_strides, b, b_strides, c, m, n, k, accumulate=False):
    _lib.check(_lib.load().dsv_factor_gemm(a.data_ptr(), a_strides[0], a_strides[1], b.data_ptr(), b_strides[0],
                                           b_strides[1], c.data_ptr(), m, n, k, int(accumulate),
                                           _lib.stream_of(c.device)), "dsv_factor_gemm")


def build_cache(codebook, pred, prev, bias, W, norm, head, res_emb=None, res_proj=None, chunk=4096,
                tp_head=None):
    """sampling/factorized/weights.py:34-80."""
    if (res_emb is None) != (res_proj is None):
        raise ValueError("residual pair")
    if tp_head is not None:
        raise NotImplementedError("a vocabulary-sharded head (tensor parallelism) is not built here")
    v, c = codebook.shape
    r = pred.shape[0]
    h = W.shape[0]
    if not (pred.shape == prev.shape == (r, c) and W.shape == (h, r) and head.shape == (v, h)
            and norm.shape == (h,) and bias.shape == (r,)):
        raise ValueError("build_cache: inconsistent weight shapes")
    _lib.require_cuda(codebook, pred, prev, bias, W, norm, head, res_emb, res_proj)
    dev = W.device
    wd, pd, vd = _widen(W), _widen(pred), _widen(prev)
    nd, bd = _widen(norm), _widen(bias)
    gram = torch.empty((r, r), device=dev, dtype=torch.float64)
    _gemm(wd, (1, r), wd, (r, 1), gram, r, r, h)  # W^T W: A(i, k) = W[k, i]
    cache = {"W": wd, "norm": nd, "bias": bd, "Gram": gram, "head": head}
    for key in ("G", "V", "TG"):
        cache[key] = torch.empty((v, r), device=dev, dtype=torch.float64)
    rp = None if res_proj is None else _widen(res_proj)
    step = max(1, int(chunk))
    e = torch.empty((min(step, v), c), device=dev, dtype=torch.float64)
    hn = torch.empty((min(step, v), h), device=dev, dtype=torch.float64)
    re = None if res_emb is None else torch.empty((min(step, v), res_emb.shape[1]), device=dev, dtype=torch.float64)
    for begin in range(0, v, step):
        end = min(v, begin + step)
        rows = end - begin
        eb = _widen(codebook[begin:end], scale=math.sqrt(c), out=e[:rows])
        _gemm(eb, (c, 1), pd, (1, c), cache["G"][begin:end], rows, r, c)        # e pred^T
        _gemm(eb, (c, 1), vd, (1, c), cache["V"][begin:end], rows, r, c)        # e prev^T
        if rp is not None:
            rr = res_emb.shape[1]
            rb = _widen(res_emb[begin:end], out=re[:rows])
            _gemm(rb, (rr, 1), rp, (1, rr), cache["V"][begin:end], rows, r, rr, accumulate=True)
        hb = _widen(head[begin:end], mul=nd, out=hn[:rows])                       # head * norm
        _gemm(hb, (h, 1), wd, (r, 1), cache["TG"][begin:end], rows, r, h)       # (head * norm) W
    return cache
