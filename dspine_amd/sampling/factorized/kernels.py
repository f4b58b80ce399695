"""The factorized draft q table (sampling/factorized/kernels.py of the reference), float64 on
MI355X: ``factor_table`` writes out[n, j, c] = (base[n, c] + a m[n, j] . TG[cand c]) /
sqrt(d / H + eps), d = |x|^2 + 2a (xW) . m + a^2 m Gram m, from the per-model cache of
``build_cache``, and the direct form where d cancels -- one library call (``dsv_factor_table``:
the row preparation, the messages, x W and m Gram on the float64 matrix cores, the finalize and
the direct form), on the current stream, without allocation or host synchronisation (capturable
in a graph)."""

from __future__ import annotations

from dataclasses import dataclass

import torch

from dspine_amd import _lib
from dspine_amd.sampling.factorized import cancellation as P

build_cache = P.build_cache


@dataclass
class Workspace:
    x: torch.Tensor
    scale: torch.Tensor
    first: torch.Tensor
    message: torch.Tensor
    tg: torch.Tensor
    safe: torch.Tensor
    d: torch.Tensor
    magnitude: torch.Tensor
    fallback: object
    gemm: torch.Tensor  # the float64 products x W (its parts over H) and m Gram

    @classmethod
    def allocate(cls, n, k, h, r, device):
        f = lambda shape: torch.empty(shape, device=device, dtype=torch.float64)
        words = int(_lib.load().dsv_factor_workspace_doubles(n, k, h, r))
        return cls(f((n, h)), f((n,)), f((n,)), f((n, k, r)), f((n, k, r)),
                   torch.empty((n, k), device=device, dtype=torch.bool), f((n, k)), f((n, k)),
                   P.Workspace.allocate(n, k, h, device), f((max(words, 1),)))

    def validate(self, n, k, h, r, device):
        expected = {"x": (n, h), "scale": (n,), "first": (n,), "message": (n, k, r), "tg": (n, k, r),
                    "safe": (n, k), "d": (n, k), "magnitude": (n, k)}
        for name, shape in expected.items():
            value = getattr(self, name)
            if not (value.shape == shape and value.is_contiguous() and value.device == torch.device(device)):
                raise ValueError(f"workspace {name} must be contiguous {shape} on the device")
            if value.dtype != (torch.bool if name == "safe" else torch.float64):
                raise ValueError(f"workspace {name} has dtype {value.dtype}")
        words = int(_lib.load().dsv_factor_workspace_doubles(n, k, h, r))
        if self.gemm.dtype != torch.float64 or self.gemm.numel() < words or not self.gemm.is_contiguous():
            raise ValueError(f"workspace gemm must hold {words} float64")
        self.fallback.validate(n, k, h, device)


def factor_table(raw, rms, query, anchors, cand, cache, eps, t, out, base_out, workspace, candidate_head=None):
    """Compute conditional proposal logits with float64 factors and the direct fallback
    (sampling/factorized/kernels.py:179-300).  raw [bs*t, H] and query [bs*t, R] bf16 / float32,
    rms [bs*t] float32, anchors [bs] and cand [n = bs*(t-1), K] int64; out [n, K, K] float32 and
    base_out [n, K] float64 written.  Returns ``out``."""
    n, k = cand.shape
    h = raw.shape[1]
    r = query.shape[1]
    bs = anchors.numel()
    if t < 2 or n != bs * (t - 1):
        raise ValueError("factor_table: n must be bs * (t - 1)")
    if raw.shape != (bs * t, h) or rms.shape != (bs * t,) or query.shape != (bs * t, r):
        raise ValueError("factor_table: raw / rms / query must cover bs * t state rows")
    if anchors.shape != (bs,) or anchors.dtype != torch.int64 or cand.dtype != torch.int64:
        raise ValueError("factor_table: anchors and cand must be int64")
    if not all(z.is_contiguous() for z in (raw, rms, query, anchors, cand, out, base_out)):
        raise ValueError("factor_table: contiguous operands required")
    if out.shape != (n, k, k) or out.dtype != torch.float32:
        raise ValueError("factor_table: out must be float32 [n, K, K]")
    if base_out.shape != (n, k) or base_out.dtype != torch.float64:
        raise ValueError("factor_table: base_out must be float64 [n, K]")
    if cache["W"].shape != (h, r) or cache["Gram"].shape != (r, r):
        raise ValueError("factor_table: cache does not match H / R")
    if any(cache[name].dtype != torch.float64 for name in ("W", "Gram", "G", "V", "TG", "bias", "norm")):
        raise ValueError("factor_table: cache tensors must be float64")
    if rms.dtype != torch.float32:
        raise ValueError("factor_table: rms must be float32")
    workspace.validate(n, k, h, r, raw.device)
    dev = _lib.require_cuda(raw, rms, query, anchors, cand, out, base_out)
    f = _lib.FactorArgs()
    f.n, f.K, f.T, f.H, f.R = n, k, t, h, r
    f.vocab = cache["G"].shape[0]
    f.raw, f.raw_dtype, f.raw_stride = raw.data_ptr(), _lib.dtype_code(raw), raw.stride(0)
    f.rms = rms.data_ptr()
    f.query, f.query_dtype, f.query_stride = query.data_ptr(), _lib.dtype_code(query), query.stride(0)
    f.anchors, f.cand = anchors.data_ptr(), cand.data_ptr()
    f.W, f.gram, f.G, f.Vm, f.TG = (cache[name].data_ptr() for name in ("W", "Gram", "G", "V", "TG"))
    f.bias, f.norm = cache["bias"].data_ptr(), cache["norm"].data_ptr()
    keep = P._head_args(f, cache, candidate_head, n, k, h)
    f.eps = float(eps)
    f.out, f.base_out = out.data_ptr(), base_out.data_ptr()
    ws = workspace
    f.x, f.scale, f.first = ws.x.data_ptr(), ws.scale.data_ptr(), ws.first.data_ptr()
    f.message, f.tg = ws.message.data_ptr(), ws.tg.data_ptr()
    f.safe, f.d, f.magnitude = ws.safe.data_ptr(), ws.d.data_ptr(), ws.magnitude.data_ptr()
    f.y = ws.fallback.y.data_ptr()
    f.gemm_ws, f.gemm_ws_doubles = ws.gemm.data_ptr(), ws.gemm.numel()
    _lib.check(_lib.load().dsv_factor_table(f, _lib.stream_of(dev)), "dsv_factor_table")
    del keep
    return out
