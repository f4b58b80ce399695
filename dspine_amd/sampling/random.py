"""Request-seeded uniforms keyed by (seed, absolute position, column, draw purpose)
(sampling/random.py of the reference).  Draws come from a HIP murmur3 kernel; unseeded
verification keeps torch's device RNG stream, exactly like the reference."""

from __future__ import annotations

import torch

from dspine_amd import _lib

DRAFT, ACCEPT, BONUS, PREFILL = range(4)


def seeded_uniforms(seeds: torch.Tensor, positions: torch.Tensor, width: int, stream: int) -> torch.Tensor:
    """float32 [n, width] in [0, 1) (sampling/random.py:71-91)."""
    if seeds.ndim != 1 or positions.shape != seeds.shape:
        raise ValueError("Seeds and positions must be matching request vectors")
    if seeds.dtype != torch.int64 or positions.dtype not in (torch.int32, torch.int64):
        raise ValueError("Expected int64 seeds and integer positions")
    if seeds.device != positions.device or not 0 < width < 65536 or stream not in range(4):
        raise ValueError("Invalid seeded uniform layout")
    _lib.require_cuda(seeds)
    seeds, positions = seeds.contiguous(), positions.contiguous()
    out = torch.empty((seeds.numel(), width), device=seeds.device, dtype=torch.float32)
    lib = _lib.load()
    _lib.check(lib.dsv_uniforms(seeds.data_ptr(), positions.data_ptr(),
                                int(positions.dtype == torch.int64), seeds.numel(), width, stream,
                                out.data_ptr(), _lib.stream_of(seeds.device)), "dsv_uniforms")
    return out


class RequestRNG:
    """Staged request seeds and positions (sampling/random.py:94-104)."""

    def __init__(self, tp=None):
        self.seeds = self.positions = None
        self.tp = tp

    def stage(self, seeds, positions):
        self.seeds = seeds
        self.positions = positions.clone() if seeds is not None else None

    def draw(self, width, stream):
        return seeded_uniforms(self.seeds, self.positions, width, stream)


def verification_uniforms(bs, width, device, random_state=None):
    """ACCEPT draws [bs, width-1] and BONUS draws [bs] (sampling/random.py:107-118)."""
    if random_state is None or random_state.seeds is None:
        return (torch.rand((bs, width - 1), device=device, dtype=torch.float32),
                torch.rand((bs,), device=device, dtype=torch.float32))
    if random_state.seeds.numel() != bs:
        raise RuntimeError("Seeded verification request order was not staged")
    return random_state.draw(width - 1, ACCEPT), random_state.draw(1, BONUS).view(bs)
