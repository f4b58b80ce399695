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
