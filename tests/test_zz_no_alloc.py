"""The allocation-free greedy verify (dsv_greedy_verify_noalloc, static device scratch) through
the C ABI: its outputs equal dsv_greedy_verify's (workspace entry point) on two calls in a row,
the second smaller, so the second reuses scratch the first wrote; sizes beyond the scratch are
refused before any launch."""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(seed, bs, T, V, dtype):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(bs * T, V, generator=g) * 2).to(dtype)
    logits[: T] = 0  # an all-tie request: the first id is every row's argmax
    top1 = logits.float().argmax(-1).view(bs, T)
    cand = torch.zeros(bs, T, dtype=torch.int64)
    cand[:, 1:] = top1[:, : T - 1]
    for b in range(1, bs, 3):  # a mismatch in some requests
        cand[b, 1 + (b % (T - 1))] = (cand[b, 1 + (b % (T - 1))] + 1) % V
    lens = (torch.arange(bs, dtype=torch.int32) % T) + 1
    prefix = torch.arange(bs, dtype=torch.int32) * 7 + 3
    return logits, cand, lens, prefix


def _outs(bs, T, device):
    return (torch.full((bs,), -5, device=device, dtype=torch.int32),
            torch.full((bs,), -5, device=device, dtype=torch.int32),
            torch.full((bs,), -5, device=device, dtype=torch.int64),
            torch.full((bs, T), -5, device=device, dtype=torch.int64),
            torch.full((bs,), -5, device=device, dtype=torch.int32),
            torch.full((bs, T), -5, device=device, dtype=torch.int64))


def _noalloc(lib, logits, cand, lens, cap, prefix, outs, device):
    from dspine_amd import _lib

    bs, T = cand.shape
    acc, com, bon, out, nseq, top1 = outs
    return lib.dsv_greedy_verify_noalloc(
        logits.data_ptr(), _lib.dtype_code(logits), bs * T, logits.shape[1], logits.stride(0), bs, T,
        cand.data_ptr(), _lib.ptr(lens), cap, prefix.data_ptr(), acc.data_ptr(), com.data_ptr(), bon.data_ptr(),
        out.data_ptr(), nseq.data_ptr(), top1.data_ptr(), _lib.stream_of(device))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_greedy_equals_workspace_entry(device, dtype):
    from dspine_amd import _lib
    from dspine_amd.verification.caps import accept_greedy

    lib = _lib.load()
    for seed, bs, T, V, ragged in ((1, 48, 17, 151936, False), (2, 5, 9, 70001, True)):
        logits, cand, lens, prefix = _case(seed, bs, T, V, dtype)
        d = [t.to(device) for t in (logits, cand, lens, prefix)]
        outs = _outs(bs, T, device)
        rc = _noalloc(lib, d[0], d[1], d[2] if ragged else None, 0 if ragged else T, d[3], outs, device)
        assert rc == 0, lib.dsv_last_error()
        ref_top1 = torch.empty((bs, T), device=device, dtype=torch.int64)
        ref = accept_greedy(candidates=d[1], next_token_logits=d[0], prefix_lens=d[3],
                            cap=None if ragged else T, verify_lens=d[2] if ragged else None, top1=ref_top1)
        torch.cuda.synchronize()
        for got, want in zip(outs[:5], ref):
            assert torch.equal(got.cpu(), want.cpu()), (seed, dtype)
        assert torch.equal(outs[5].cpu(), ref_top1.cpu())
        assert np.array_equal(outs[5].cpu().numpy(), logits.float().argmax(-1).view(bs, T).numpy())


def test_noalloc_refuses_oversized_input(device):
    from dspine_amd import _lib

    lib = _lib.load()
    bs, T, V = 4, 2, 20480 * 8192 + 1  # 4 * 2 rows x 8193 chunks > 65536 statistics
    outs = _outs(bs, T, device)
    cand = torch.zeros(bs, T, dtype=torch.int64, device=device)
    prefix = torch.zeros(bs, dtype=torch.int32, device=device)
    rc = lib.dsv_greedy_verify_noalloc(
        ctypes.c_void_p(16), _lib.DSV_BF16, bs * T, V, V, bs, T, cand.data_ptr(), None, T, prefix.data_ptr(),
        outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(), outs[3].data_ptr(), outs[4].data_ptr(), None,
        _lib.stream_of(device))
    assert rc == _lib.DSV_ERR_INVALID
    assert b"static" in lib.dsv_last_error()
