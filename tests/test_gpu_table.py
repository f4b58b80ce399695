"""The draft-side sampling table (kernels/dspine.py:505-613, serial_rs_table) on the matrix cores
against the oracle's float64 table, at the reference's test shapes (tests/test_cuda.py:268-292,
:335-352 and the realistic :389-445) with the tolerance the reference uses (rtol = atol = 1e-4),
and chained into the K-lane sampler (serial_sample_chain): the chain on the GPU table equals the
oracle's chain on the same table bit for bit."""

import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _O():
    import oracle.verify_oracle as O

    return O


def _inputs(seed, bs=2, T=4, H=512, R=128, C=64, V=1024, k=8, residual=False):
    """tests/test_cuda.py:268-292 (bf16 tensors; the weights are passed as float32)."""
    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16
    m, n = bs * T, bs * (T - 1)
    d = dict(
        raw=torch.randn(m, H, generator=g).to(bf),
        rms=(torch.rand(m, generator=g) + 0.5).float(),
        packed=torch.randn(m, 3 * R, generator=g).to(bf),
        codebook=(torch.randn(V, C, generator=g) / math.sqrt(C)).to(bf),
        pg=(torch.randn(R, C, generator=g) / math.sqrt(C)).to(bf).float(),
        pv=(torch.randn(R, C, generator=g) / math.sqrt(C)).to(bf).float(),
        gb=(torch.randn(R, generator=g) * 0.1).to(bf).float(),
        w_last=(torch.randn(H, R, generator=g) / math.sqrt(R)).to(bf).float(),
        norm_w=(1.0 + 0.1 * torch.randn(H, generator=g)).to(bf).float(),
        lm=(torch.randn(V, H, generator=g) / math.sqrt(H)).to(bf),
    )
    d["cand"] = torch.stack([torch.randperm(V, generator=g)[:k].sort().values for _ in range(n)]).contiguous()
    d["anchors"] = torch.randint(0, V, (bs,), generator=g)
    if residual:
        d["res_emb"] = (torch.randn(V, 32, generator=g) / 4).to(bf)
        d["res_proj"] = torch.randn(R, 32, generator=g) / math.sqrt(32)
    return d


def _gpu_table(d, T, device, candidate_head=None, eps=1e-6):
    from dspine_amd.kernels.dspine import serial_rs_table

    g = {key: v.to(device) for key, v in d.items()}
    return serial_rs_table(g["raw"], g["rms"], g["packed"], g["anchors"], g["cand"], g["codebook"], g["pg"], g["pv"],
                           g["gb"], g["w_last"], g["norm_w"], g["lm"], eps, T, res_emb=g.get("res_emb"),
                           res_proj=g.get("res_proj"),
                           candidate_head=None if candidate_head is None else candidate_head.to(device))


def _ref(d, T, candidate_head=None, eps=1e-6):
    return _O().rs_table(d["raw"], d["rms"], d["packed"], d["anchors"], d["cand"], d["codebook"], d["pg"], d["pv"],
                         d["gb"], d["w_last"], d["norm_w"], d["lm"], eps, T, res_emb=d.get("res_emb"),
                         res_proj=d.get("res_proj"), candidate_head=candidate_head)


@pytest.mark.parametrize("seed", [0, 1])
def test_table_matches_float64_reference(device, seed):
    """tests/test_cuda.py:332-357: the reference's small shapes; a request's first block row has
    the anchor as every sender, so its K table rows agree."""
    T = 4
    d = _inputs(seed, T=T)
    table = _gpu_table(d, T, device).cpu()
    torch.testing.assert_close(table.double(), _ref(d, T), rtol=1e-4, atol=1e-4)
    for b in range(2):
        first = table[b * (T - 1)]
        torch.testing.assert_close(first, first[:1].expand_as(first))


@pytest.mark.parametrize("k", [16, 32, 64, 5])
def test_table_candidate_widths(device, k):
    """K of one, two and four 16-lane blocks, and a K that leaves most of a block empty."""
    T = 5
    d = _inputs(20 + k, bs=3, T=T, H=256, R=64, C=32, V=2048, k=k)
    table = _gpu_table(d, T, device).cpu()
    torch.testing.assert_close(table.double(), _ref(d, T), rtol=1e-4, atol=1e-4)


def test_table_residual_and_candidate_head(device):
    """The terminal residual added to the value, and head rows given per candidate
    ([n, K, H] instead of lm_head gathered by id)."""
    T = 4
    d = _inputs(3, T=T, residual=True)
    n, k = d["cand"].shape
    head = (torch.randn(n, k, d["raw"].shape[1], generator=torch.Generator().manual_seed(9)) / 20).to(torch.bfloat16)
    table = _gpu_table(d, T, device, candidate_head=head).cpu()
    torch.testing.assert_close(table.double(), _ref(d, T, candidate_head=head), rtol=1e-4, atol=1e-4)


def test_table_realistic_shapes_chain(device):
    """tests/test_cuda.py:389-445's realistic shapes (H 4096, R 512, C 1024, V 4096, K 16,
    T 16), then the K-lane sampler on the table: bit-exact with the oracle's chain on the same
    table."""
    from dspine_amd.kernels.dspine import serial_sample_chain

    O = _O()
    bs, T, k = 2, 16, 16
    d = _inputs(5, bs=bs, T=T, H=4096, R=512, C=1024, V=4096, k=k)
    table = _gpu_table(d, T, device)
    torch.testing.assert_close(table.cpu().double(), _ref(d, T), rtol=1e-4, atol=1e-4)
    n = bs * (T - 1)
    g = torch.Generator().manual_seed(6)
    inv_t = torch.tensor([1 / 0.7, 1.0])
    top_k = torch.tensor([5, 16], dtype=torch.int32)
    top_p = torch.tensor([0.9, 1.0])
    min_p = torch.tensor([0.02, 0.0])
    greedy = torch.zeros(bs, dtype=torch.int32)
    u = torch.rand(n, generator=g)
    gtok = d["cand"][:, 0].clone()
    out_tok = torch.empty(n, dtype=torch.int64, device=device)
    out_q = torch.empty((n, k), device=device)
    dd = lambda x: x.to(device)  # noqa: E731
    serial_sample_chain(table, dd(inv_t), dd(top_k), dd(top_p), dd(min_p), dd(greedy), dd(u), dd(d["cand"]),
                        dd(gtok), out_tok, out_q, T)
    torch.cuda.synchronize()
    tok, q = O.sample_chain(table.cpu().numpy(), inv_t.numpy(), top_k.numpy(), top_p.numpy(), min_p.numpy(),
                            greedy.numpy(), u.numpy(), d["cand"].numpy(), gtok.numpy(), T)
    assert np.array_equal(out_tok.cpu().numpy(), tok)
    np.testing.assert_allclose(out_q.cpu().numpy(), q, rtol=1e-6, atol=1e-7)
