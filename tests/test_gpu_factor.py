"""The factorized draft q table (sampling/factorized/kernels.py:179-300, cancellation.py:82-147,
weights.py:34-80, graph.py) on the float64 matrix cores against the oracle's float64
restatement: the float32 table within one unit in the last place (float64 sums in another order
round to the same float32 almost always), the cancellation rows through the direct form, graph
replays equal to eager calls bit for bit (tests/test_dynamic_sampling.py:184-215), and the K-lane
sampler on the table equal to the oracle's chain on the same table."""

import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _O():
    import oracle.verify_oracle as O

    return O


def _inputs(seed, bs=3, T=16, H=64, R=8, C=16, V=64, k=16, f32=False, scale=0.1):
    g = torch.Generator().manual_seed(seed)
    dt = torch.float32 if f32 else torch.bfloat16
    rand = lambda *shape: torch.randn(*shape, generator=g) * scale  # noqa: E731
    m, n = bs * T, bs * (T - 1)
    return dict(raw=rand(m, H).to(dt), rms=(torch.rand(m, generator=g) + 0.5).float(), query=rand(m, R).to(dt),
                anchors=torch.randint(0, V, (bs,), generator=g),
                cand=torch.stack([torch.randperm(V, generator=g)[:k] for _ in range(n)]),
                codebook=(rand(V, C) / scale / math.sqrt(C)).bfloat16(), pred=rand(R, C) / scale / math.sqrt(C),
                prev=rand(R, C) / scale / math.sqrt(C), bias=rand(R), W=rand(H, R) / scale / math.sqrt(R),
                norm=1.0 + rand(H), head=(rand(V, H) / scale / math.sqrt(H)).bfloat16())


def _run(d, T, device, eps=1e-6):
    from dspine_amd.sampling.factorized.kernels import Workspace, build_cache, factor_table

    g = {key: v.to(device) for key, v in d.items()}
    cache = build_cache(g["codebook"], g["pred"], g["prev"], g["bias"], g["W"], g["norm"], g["head"])
    n, k = d["cand"].shape
    H, R = d["raw"].shape[1], d["query"].shape[1]
    out = torch.empty((n, k, k), device=device)
    base = torch.empty((n, k), device=device, dtype=torch.float64)
    ws = Workspace.allocate(n, k, H, R, device)
    factor_table(g["raw"], g["rms"], g["query"], g["anchors"], g["cand"], cache, eps, T, out, base, ws)
    torch.cuda.synchronize()
    return out.cpu(), base.cpu(), ws.safe.cpu(), cache


def _ref(d, T, eps=1e-6):
    O = _O()
    cache = O.factor_cache(d["codebook"], d["pred"], d["prev"], d["bias"], d["W"], d["norm"], d["head"])
    return O.factor_table(d["raw"], d["rms"], d["query"], d["anchors"], d["cand"], cache, eps, T), cache


def _ulps(a, b):
    """Distance in float32 units in the last place (same-sign values)."""
    ia = a.contiguous().view(torch.int32).long()
    ib = b.contiguous().view(torch.int32).long()
    return (ia - ib).abs()


def _check(out, ref_out, tag):
    u = _ulps(out, ref_out)
    same = int((u == 0).sum())
    assert int(u.max()) <= 1, (tag, int(u.max()))
    assert same >= 0.99 * u.numel(), (tag, same, u.numel())
    print(f"[factor] {tag}: {same} of {u.numel()} entries bit-equal, the rest within 1 ulp", flush=True)


def test_factor_cache_matches_float64(device):
    """build_cache's float64 products against the CPU's."""
    d = _inputs(3)
    _, _, _, cache = _run(d, 16, device)
    O = _O()
    ref = O.factor_cache(d["codebook"], d["pred"], d["prev"], d["bias"], d["W"], d["norm"], d["head"])
    for key in ("W", "norm", "bias", "Gram", "G", "V", "TG"):
        torch.testing.assert_close(cache[key].cpu(), ref[key], rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("bs", [1, 33])
def test_factor_table_reference_shapes(device, bs):
    """The reference test's shapes (tests/test_dynamic_sampling.py:29-51: T = K = 16, H 64, R 8,
    C 16, vocabulary 64)."""
    d = _inputs(10 + bs, bs=bs)
    out, base, safe, _ = _run(d, 16, device)
    (ref_out, ref_base, ref_safe, _), _ = _ref(d, 16)
    assert torch.equal(safe, ref_safe)
    torch.testing.assert_close(base, ref_base, rtol=1e-12, atol=1e-14)
    _check(out, ref_out, f"reference shapes bs={bs}")


def test_factor_table_serving_shape(device):
    """H 4096, R 512, C 1024 (the q-table's realistic shape), vocabulary 8192, K 16, T 16: x W is
    split over H."""
    d = _inputs(21, bs=2, T=16, H=4096, R=512, C=1024, V=8192)
    out, base, safe, _ = _run(d, 16, device)
    (ref_out, ref_base, ref_safe, _), _ = _ref(d, 16)
    assert bool(safe.all()) and bool(ref_safe.all())
    torch.testing.assert_close(base, ref_base, rtol=1e-11, atol=1e-13)
    _check(out, ref_out, "H 4096 R 512")


def test_factor_table_cancellation(device):
    """State rows that cancel one lane's write (float32 raw = -a W m): the 2^-24 test rejects
    exactly those entries, whose values come from the direct form."""
    O = _O()
    T = 5
    d = _inputs(31, bs=3, T=T, f32=True)
    cache = O.factor_cache(d["codebook"], d["pred"], d["prev"], d["bias"], d["W"], d["norm"], d["head"])
    for i, j in ((1, 3), (6, 9), (9, 0)):
        src = i // (T - 1) * T + i % (T - 1) + 1
        sid = int(d["anchors"][i // (T - 1)]) if i % (T - 1) == 0 else int(d["cand"][i - 1, j])
        m = torch.sigmoid(d["query"][src].double() + cache["G"][sid] + cache["bias"]) * cache["V"][sid]
        d["raw"][src] = (-d["rms"][src].double() * (cache["W"] @ m)).float()
    out, _, safe, _ = _run(d, T, device)
    (ref_out, _, ref_safe, ref64), _ = _ref(d, T)
    assert int((~ref_safe).sum()) == 3 and torch.equal(safe, ref_safe)
    torch.testing.assert_close(out.double(), ref64, rtol=1e-6, atol=1e-9)
    _check(out[safe], ref_out[safe], "cancellation case, safe entries")


def _sampler(bs, device, seed=61):
    """tests/test_dynamic_sampling.py:29-51's sampler (T = K = 16, H 64, R 8, C 16, vocabulary 64)."""
    g = torch.Generator().manual_seed(seed)
    t, k, h, r, c, v = 16, 16, 64, 8, 16, 64
    rand = lambda *shape: (torch.randn(*shape, generator=g) * 0.1).to(device)  # noqa: E731
    return SimpleNamespace(
        draft_model=SimpleNamespace(selected_prefix_bridge=SimpleNamespace(codebook=rand(v, c).bfloat16())),
        raw=rand(bs * t, h).bfloat16(), rms=torch.ones(bs * t, device=device), query=rand(bs * t, r).bfloat16(),
        anchors=torch.ones(bs, device=device, dtype=torch.int64),
        candidate_out=torch.arange(k, device=device).expand(bs, t - 1, k).contiguous(),
        pred_gate_f32=rand(r, c), prev_f32=rand(r, c), gate_b_f32=rand(r), write_f32=rand(h, r),
        norm_f32=torch.ones(h, device=device), lm_head_weight=rand(v, h).bfloat16(), res_emb=None,
        res_proj_f32=None, norm_eps=1e-6, max_bs=bs, block_size=t, k=k, capture_batch_sizes=[])


def test_factorized_cache_replays_and_accepts_uncaptured_batch_sizes(device):
    """tests/test_dynamic_sampling.py:184-215: graph replays (and eager calls above the captured
    sizes) equal a fresh eager factor_table bit for bit; preparation restores the live state."""
    from dspine_amd.sampling.factorized.kernels import Workspace, factor_table
    from dspine_amd.sampling.proposal import prepare

    sampler = _sampler(33, device)
    sampler.capture_batch_sizes = [1, 2, 4, 8, 16, 32]
    saved = sampler.raw.clone(), sampler.candidate_out.clone()
    cache = prepare(sampler)
    assert torch.equal(sampler.raw, saved[0]) and torch.equal(sampler.candidate_out, saved[1])
    gen = torch.Generator(device=device).manual_seed(5)
    for bs in (1, 9, 32, 17, 33, 2):
        sampler.raw.copy_((torch.randn(sampler.raw.shape, generator=gen, device=device) * 0.1).bfloat16())
        n = bs * 15
        actual = cache.lookup(bs).clone()
        expected = torch.empty_like(actual)
        factor_table(sampler.raw[: bs * 16], sampler.rms[: bs * 16], sampler.query[: bs * 16], sampler.anchors[:bs],
                     sampler.candidate_out[:bs].view(n, 16), cache.weights, sampler.norm_eps, 16, expected,
                     torch.empty((n, 16), device=device, dtype=torch.float64),
                     Workspace.allocate(n, 16, 64, 8, device))
        torch.cuda.synchronize()
        assert torch.equal(actual, expected), bs
    assert cache.eager_buffers.bs <= sampler.max_bs


def test_factor_residual_and_candidate_head(device):
    """The terminal residual added to V in the cache (weights.py:65-67), and head rows given per
    candidate ([n, K, H], the HEAD_CANDIDATES path: the base terms read them, while m . TG keeps
    the cache's vocabulary rows, so they are the gathered rows, as a vocabulary-sharded head
    supplies them)."""
    from dspine_amd.sampling.factorized.kernels import Workspace, build_cache, factor_table

    O = _O()
    T = 6
    d = _inputs(51, bs=2, T=T, H=128, R=64, C=32, V=512)
    g = torch.Generator().manual_seed(52)
    res_emb = (torch.randn(512, 24, generator=g) / 4).bfloat16()
    res_proj = torch.randn(64, 24, generator=g) / 5
    n, k = d["cand"].shape
    chead = d["head"][d["cand"]].clone()
    dv = {key: v.to(device) for key, v in d.items()}
    cache = build_cache(dv["codebook"], dv["pred"], dv["prev"], dv["bias"], dv["W"], dv["norm"], dv["head"],
                        res_emb=res_emb.to(device), res_proj=res_proj.to(device))
    ref_cache = O.factor_cache(d["codebook"], d["pred"], d["prev"], d["bias"], d["W"], d["norm"], d["head"],
                               res_emb=res_emb, res_proj=res_proj)
    torch.testing.assert_close(cache["V"].cpu(), ref_cache["V"], rtol=1e-12, atol=1e-14)
    out = torch.empty((n, k, k), device=device)
    base = torch.empty((n, k), device=device, dtype=torch.float64)
    factor_table(dv["raw"], dv["rms"], dv["query"], dv["anchors"], dv["cand"], cache, 1e-6, T, out, base,
                 Workspace.allocate(n, k, 128, 64, device), candidate_head=chead.to(device))
    torch.cuda.synchronize()
    ref_out, _, _, _ = O.factor_table(d["raw"], d["rms"], d["query"], d["anchors"], d["cand"], ref_cache, 1e-6, T,
                                      candidate_head=chead)
    _check(out.cpu(), ref_out, "residual + candidate head")
    direct = O.rs_table(d["raw"], d["rms"], d["query"], d["anchors"], d["cand"], d["codebook"], d["pred"], d["prev"],
                        d["bias"], d["W"], d["norm"], d["head"], 1e-6, T, res_emb=res_emb, res_proj=res_proj,
                        candidate_head=chead)
    torch.testing.assert_close(out.cpu().double(), direct, rtol=1e-6, atol=1e-7)


def test_factor_table_chained_into_sampler(device):
    """The K-lane sampler (serial_sample_chain) on the factorized table equals the oracle's chain
    on the same table bit for bit."""
    from dspine_amd.kernels.dspine import serial_sample_chain

    O = _O()
    bs, T, k = 4, 16, 16
    d = _inputs(41, bs=bs, T=T, H=256, R=64, C=32, V=2048)
    table, _, _, _ = _run(d, T, device)
    n = bs * (T - 1)
    g = torch.Generator().manual_seed(6)
    inv_t = torch.tensor([1 / 0.7, 1.0, 2.0, 1.0])
    top_k = torch.tensor([5, 16, 8, 3], dtype=torch.int32)
    top_p = torch.tensor([0.9, 1.0, 0.8, 0.95])
    min_p = torch.tensor([0.02, 0.0, 0.0, 0.1])
    greedy = torch.tensor([0, 0, 1, 0], dtype=torch.int32)
    u = torch.rand(n, generator=g)
    gtok = d["cand"][:, 0].clone()
    out_tok = torch.empty(n, dtype=torch.int64, device=device)
    out_q = torch.empty((n, k), device=device)
    dd = lambda x: x.to(device)  # noqa: E731
    serial_sample_chain(dd(table), dd(inv_t), dd(top_k), dd(top_p), dd(min_p), dd(greedy), dd(u), dd(d["cand"]),
                        dd(gtok), out_tok, out_q, T)
    torch.cuda.synchronize()
    tok, q = O.sample_chain(table.numpy(), inv_t.numpy(), top_k.numpy(), top_p.numpy(), min_p.numpy(),
                            greedy.numpy(), u.numpy(), d["cand"].numpy(), gtok.numpy(), T)
    assert np.array_equal(out_tok.cpu().numpy(), tok)
    np.testing.assert_allclose(out_q.cpu().numpy(), q, rtol=1e-6, atol=1e-7)
