"""Neutral target rows outside each request's verified prefix (sampling/padding.py of the
reference)."""

from __future__ import annotations

import math

import torch

from dspine_amd import _lib


def logits_padding(controller, value, shape):
    """A new tensor of ``shape`` (value's dtype and device) whose rows are the one-point
    distribution [0, -inf, ..., -inf] (sampling/padding.py:4-12): normalised under any
    temperature, top-k, top-p or min-p, so unused rows cannot emit tokens."""
    del controller
    shape = tuple(int(s) for s in shape)
    if not shape or shape[-1] < 1:
        raise ValueError("padding needs a non-empty last dimension")
    dev = _lib.require_cuda(value)
    out = torch.empty(shape, device=dev, dtype=value.dtype)
    rows = math.prod(shape[:-1])
    if rows:
        _lib.check(_lib.load().dsv_logits_padding(out.data_ptr(), _lib.dtype_code(out), rows, shape[-1],
                                                  shape[-1], _lib.stream_of(dev)), "dsv_logits_padding")
    return out
