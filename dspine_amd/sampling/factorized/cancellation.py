"""The direct form of the factorized table where its factors cancel
(sampling/factorized/cancellation.py of the reference): for each (n, j) whose safe flag is 0,
y = x + a (W m), z = y / sqrt(mean(y^2) + eps) * norm, out[n, j, c] = head[cand c] . z, in float64
(``dsv_factor_direct``; the other (n, j) are left as they are)."""

from __future__ import annotations

from dataclasses import dataclass

import torch

from dspine_amd import _lib
from dspine_amd.sampling.factorized.weights import build_cache

__all__ = ["Workspace", "apply_direct_fallback", "build_cache"]


@dataclass
class Workspace:
    y: torch.Tensor

    @classmethod
    def allocate(cls, n, k, h, device):
        return cls(torch.empty((n, k, h), device=device, dtype=torch.float64))

    def validate(self, n, k, h, device):
        if not (self.y.shape == (n, k, h) and self.y.dtype == torch.float64
                and self.y.device == torch.device(device) and self.y.is_contiguous()):
            raise ValueError("fallback workspace y must be contiguous float64 [n, K, H] on the device")


def _head_args(f, cache, candidate_head, n, k, h):
    head = cache["head"] if candidate_head is None else candidate_head.reshape(n * k, h)
    if head.stride(-1) != 1:
        raise ValueError("head rows must be contiguous")
    f.head_dtype = _lib.dtype_code(head)
    f.head_stride = head.stride(0)
    if candidate_head is None:
        f.head = head.data_ptr()
    else:
        f.candidate_head = head.data_ptr()
    return head


def apply_direct_fallback(x, a, message, cand, cache, safe, out, workspace, eps, candidate_head=None):
    """sampling/factorized/cancellation.py:82-147."""
    n, k = cand.shape
    h = x.shape[-1]
    r = message.shape[-1]
    workspace.validate(n, k, h, x.device)
    if not all(z.is_contiguous() for z in (x, a, message, cand, cache["W"], cache["norm"])):
        raise ValueError("apply_direct_fallback: contiguous operands required")
    if safe.shape != (n, k) or safe.dtype != torch.bool or not safe.is_contiguous():
        raise ValueError("safe must be contiguous bool [n, K]")
    if out.shape != (n, k, k) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("out must be contiguous float32 [n, K, K]")
    dev = _lib.require_cuda(x, a, message, cand, safe, out)
    f = _lib.FactorArgs()
    f.n, f.K, f.T, f.H, f.R = n, k, 2, h, r
    f.vocab = cache["head"].shape[0]
    f.cand = cand.data_ptr()
    f.W, f.norm = cache["W"].data_ptr(), cache["norm"].data_ptr()
    keep = _head_args(f, cache, candidate_head, n, k, h)
    f.eps = float(eps)
    f.out, f.x, f.scale, f.message = out.data_ptr(), x.data_ptr(), a.data_ptr(), message.data_ptr()
    f.safe, f.y = safe.data_ptr(), workspace.y.data_ptr()
    _lib.check(_lib.load().dsv_factor_direct(f, _lib.stream_of(dev)), "dsv_factor_direct")
    del keep
    return out
