"""Parity of the explicit-distribution entry points (through the C ABI) with the CPU oracle:
support compaction, chain rejection on dense / RAW / packed P with dense or sparse q, the
target-distribution builders, the sparse joint target, logit adjustments, padding rows, the
window index and the draft-side K-lane chain.

Integer outputs are compared bit-exactly; a request may differ only where the oracle reports
a decision margin below MARGIN.  Float outputs carry the tolerance written at each check.
"""

import numpy as np
import pytest
import torch

import parity
from dspine_amd import workloads as W
from parity import MARGIN

pytestmark = pytest.mark.gpu


def _O():
    import oracle.verify_oracle as O

    return O


def _outputs(bs, T, device):
    return (torch.full((bs,), -7, device=device, dtype=torch.int32),
            torch.full((bs,), -7, device=device, dtype=torch.int32),
            torch.full((bs,), -7, device=device, dtype=torch.int64),
            torch.full((bs, T), -7, device=device, dtype=torch.int64),
            torch.full((bs,), -7, device=device, dtype=torch.int32))


def _check_chain(outs, ref, tag, max_near=0):
    names = ("accept", "commit", "bonus", "output", "new_seq")
    got = [t.cpu().numpy() for t in outs]
    near = []
    for b in range(got[0].shape[0]):
        same = all(np.array_equal(g[b], r[b]) for g, r in zip(got, ref[:5]))
        if not same:
            assert ref[5][b] < MARGIN, (tag, b, {n: g[b] for n, g in zip(names, got)},
                                        {n: r[b] for n, r in zip(names, ref)}, ref[5][b])
            near.append(b)
    parity.record(tag, got[0].shape[0], int((np.asarray(ref[5]) < MARGIN).sum()),
                  [(b, float(ref[5][b])) for b in near])
    assert len(near) <= max_near, (tag, near)


# ------------------------------------------------------------------------------------------
# compress_probs (sampling/sparse/accept.py:7-78,422-460)
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("vocab,capacity", [(257, 32), (4096, 64), (9001, 32), (151936, 32), (5, 8)])
def test_compress_probs_bitexact(device, vocab, capacity):
    from dspine_amd.sampling.sparse.accept import compress_probs

    O = _O()
    g = torch.Generator().manual_seed(vocab + capacity)
    rows = 12
    p = torch.zeros(rows, vocab)
    for r in range(rows):
        n = [0, 1, capacity - 1, capacity, capacity + 1, 3 * capacity, vocab // 2, vocab][r % 8]
        n = min(n, vocab)
        idx = torch.randperm(vocab, generator=g)[:n]
        p[r, idx] = torch.rand(n, generator=g) + 1e-3
    p[9, 1 % vocab] = -0.25          # negative entry: overflow, not kept
    p[10, vocab - 1] = float("nan")  # NaN: overflow
    p[11, 0] = float("inf")          # inf: overflow, kept (inf > 0)
    got = compress_probs(torch, p.to(device), capacity=capacity)
    torch.cuda.synchronize()
    ref = O.compress(p, capacity)
    for name, a, b in zip(("ids", "values", "lengths", "overflow"), got, ref):
        assert torch.equal(a.cpu(), b), name
    # reference invariants (tests/test_p_distribution_reference.py:156-175): ids ascending
    ids, _, lengths, _ = (x.cpu() for x in got)
    for r in range(rows):
        n = int(lengths[r])
        assert n <= capacity and bool((ids[r, :n].diff() > 0).all())


# ------------------------------------------------------------------------------------------
# accept_sparse (sampling/sparse/accept.py:463-543)
# ------------------------------------------------------------------------------------------
def _compact_case(bs, kind, seed=713):
    """tests/test_sparse_accept_compact.py:56-105: support-7 rows, ragged caps, reversed packed
    order, an all-accepted request and a zero-residual request."""
    g = torch.Generator().manual_seed(seed)
    vocab = 257
    caps = torch.arange(bs, dtype=torch.int32) % 16 + 1
    caps[0] = 16
    offsets = torch.cat((torch.zeros(1, dtype=torch.int64), caps.long().cumsum(0)))[:-1]
    rows = int(caps.sum())
    p = torch.zeros((rows, vocab))
    support = torch.tensor([0, 2, 3, 7, 11, 13, 15])
    p[:, support] = torch.softmax(torch.randn(rows, len(support), generator=g), -1)
    qids = torch.arange(16, dtype=torch.int32).expand(bs, 15, 16).contiguous()
    qvals = torch.softmax(torch.randn((bs, 15, 16), generator=g), -1)
    cand = torch.zeros((bs, 16), dtype=torch.int64)
    cand[:, 1:] = torch.multinomial(qvals.reshape(-1, 16), 1, generator=g).reshape(bs, 15)
    u = torch.full((bs, 15), .371)
    uf = torch.linspace(.071, .917, bs)
    prefix = torch.arange(bs, dtype=torch.int32) + 8191
    cand[0, 1:] = 0
    u[0] = 0
    if bs > 1:
        lo = int(offsets[1])
        hi = lo + int(caps[1])
        same = torch.softmax(torch.arange(16, dtype=torch.float32), 0)
        p[lo:hi] = 0
        p[lo:hi, :16] = same
        qvals[1] = same
        u[1] = 1
    if kind == "overflow":
        p[::11] = torch.softmax(torch.randn((len(p[::11]), vocab), generator=g), -1)
    return dict(vocab=vocab, caps=caps, offsets=offsets, p=p, qids=qids, qvals=qvals.contiguous(), cand=cand,
                u=u.contiguous(), uf=uf.contiguous(), prefix=prefix)


@pytest.mark.parametrize("bs", [1, 9, 32, 65])
@pytest.mark.parametrize("kind", ["compact", "overflow", "pure_packed"])
def test_accept_sparse_compact_packed(device, bs, kind):
    from dspine_amd.sampling.sparse.accept import accept_sparse, compress_probs

    O = _O()
    c = _compact_case(bs, kind)
    d = {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in c.items()}
    ids, values, lengths, overflow = compress_probs(torch, d["p"], capacity=32)
    lane = torch.arange(32, device=device)[None, :]
    perm = (lengths[:, None] - 1 - lane).clamp_min(0).long()  # reversed support order
    packed = (ids.gather(1, perm).where(lane < lengths[:, None], -1).contiguous(),
              values.gather(1, perm).where(lane < lengths[:, None], 0).contiguous(), lengths, overflow)
    outs = _outputs(bs, 16, device)
    accept_sparse(torch, candidates=d["cand"], dense_p=None if kind == "pure_packed" else d["p"], packed=packed,
                  q_ids=d["qids"], q_values=d["qvals"], verify_lens=d["caps"], uniforms=d["u"],
                  uniform_final=d["uf"], prefix_lens=d["prefix"], outputs=outs, row_offsets=d["offsets"],
                  vocab_size=c["vocab"])
    torch.cuda.synchronize()
    # the spec: dense rejection on P itself (the reference test's pure-Python reference)
    ref = O.chain_accept(lambda r: c["p"][r].numpy(), c["cand"].numpy(), c["qids"].numpy(), c["qvals"].numpy(),
                         c["caps"].numpy(), c["u"].numpy(), c["uf"].numpy(), c["prefix"].numpy(),
                         row_offsets=c["offsets"].numpy())
    _check_chain(outs, ref, f"packed {kind} bs={bs}")
    if bs > 1:
        assert int(outs[0][0]) == 15  # u = 0 accepts every draft


@pytest.mark.parametrize("bs", [9, 65])
def test_accept_sparse_reports_overflow_without_dense(device, bs):
    """Packed rows flagged overflow with no dense P to fall back on (where the reference stops on
    the device, sparse/accept.py:257, :291): overflow_read marks the requests whose walk read one
    (the draft tests' rows and the bonus row); with the dense fallback nothing is marked."""
    from dspine_amd.sampling.sparse.accept import accept_sparse, compress_probs

    c = _compact_case(bs, "overflow")
    d = {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in c.items()}
    packed = compress_probs(torch, d["p"], capacity=32)
    status = torch.full((bs,), -1, dtype=torch.int32, device=device)
    for dense in (None, d["p"]):
        outs = _outputs(bs, 16, device)
        accept_sparse(torch, candidates=d["cand"], dense_p=dense, packed=packed, q_ids=d["qids"], q_values=d["qvals"],
                      verify_lens=d["caps"], uniforms=d["u"], uniform_final=d["uf"], prefix_lens=d["prefix"],
                      outputs=outs, row_offsets=d["offsets"], vocab_size=c["vocab"], overflow_read=status)
        torch.cuda.synchronize()
        acc = outs[0].cpu().tolist()
        ovf = packed[3].cpu().tolist()
        offs = c["offsets"].tolist()
        want = [int(dense is None and any(ovf[offs[b] + s] for s in range(acc[b] + 1))) for b in range(bs)]
        assert status.cpu().tolist() == want
        assert any(want) == (dense is None)


@pytest.mark.parametrize("bs", [1, 17, 65])
def test_accept_sparse_dense_compact_rows(device, bs):
    """tests/test_sparse_accept_compact.py:108-129."""
    from dspine_amd.sampling.sparse.accept import accept_sparse

    O = _O()
    g = torch.Generator().manual_seed(79)
    caps = torch.arange(bs, dtype=torch.int32) % 16 + 1
    offsets = torch.cat((torch.zeros(1, dtype=torch.int64), caps.long().cumsum(0)))[:-1]
    p = torch.softmax(torch.randn((int(caps.sum()), 97), generator=g), -1)
    qids = torch.arange(16, dtype=torch.int32).expand(bs, 15, 16).contiguous()
    qvals = torch.full((bs, 15, 16), 1 / 16)
    cand = torch.arange(16).expand(bs, 16).contiguous()
    u = torch.full((bs, 15), .413)
    uf = torch.full((bs,), .273)
    prefix = torch.zeros(bs, dtype=torch.int32)
    outs = _outputs(bs, 16, device)
    accept_sparse(torch, candidates=cand.to(device), dense_p=p.to(device), packed=None, q_ids=qids.to(device),
                  q_values=qvals.to(device), verify_lens=caps.to(device), uniforms=u.to(device),
                  uniform_final=uf.to(device), prefix_lens=prefix.to(device), outputs=outs,
                  row_offsets=offsets.to(device))
    torch.cuda.synchronize()
    ref = O.chain_accept(lambda r: p[r].numpy(), cand.numpy(), qids.numpy(), qvals.numpy(), caps.numpy(),
                         u.numpy(), uf.numpy(), prefix.numpy(), row_offsets=offsets.numpy())
    _check_chain(outs, ref, f"dense compact bs={bs}")


@pytest.mark.parametrize("T,K,vocab", [(16, 16, 151936), (17, 16, 20011), (5, 3, 4099)])
def test_accept_sparse_raw_and_duplicates(device, T, K, vocab):
    """RAW targets (p / denominator in IEEE float32) with random q lanes that repeat ids and
    hold values outside [0, 1]: q at a token is the lane sum; the dense residual subtracts the
    clamped q of the last lane with the id."""
    from dspine_amd.sampling.sparse.accept import accept_sparse

    O = _O()
    g = torch.Generator().manual_seed(T * K)
    bs = 24
    rows = bs * T
    logits = torch.randn(rows, vocab, generator=g) * 3
    w = torch.exp(logits - logits.max(-1, keepdim=True).values)
    den = w.sum(-1) * (0.5 + torch.rand(rows, generator=g))  # not the row sum: RAW != normalised
    qids = torch.randint(0, vocab, (bs, T - 1, K), generator=g, dtype=torch.int64)
    top = logits.view(bs, T, vocab)[:, : T - 1].argmax(-1)
    qids[:, :, 0] = top
    if K > 2:
        qids[:, :, 1] = top  # a repeated id
    qvals = torch.rand((bs, T - 1, K), generator=g) * 0.6
    qvals[::5, :, K - 1] = 1.5  # out of [0, 1]: clamped to 0 in the residual
    cand = torch.zeros((bs, T), dtype=torch.int64)
    lane = torch.randint(0, K, (bs, T - 1), generator=g)
    cand[:, 1:] = qids.gather(2, lane[..., None]).squeeze(-1)
    u = torch.rand((bs, T - 1), generator=g) * 0.5
    uf = torch.rand(bs, generator=g)
    caps = torch.randint(1, T + 1, (bs,), generator=g, dtype=torch.int32)
    prefix = torch.randint(0, 100, (bs,), generator=g, dtype=torch.int32)
    outs = _outputs(bs, T, device)
    accept_sparse(torch, candidates=cand.to(device), dense_p=w.to(device), packed=None, q_ids=qids.to(device),
                  q_values=qvals.to(device), verify_lens=caps.to(device), uniforms=u.to(device),
                  uniform_final=uf.to(device), prefix_lens=prefix.to(device), outputs=outs,
                  denominator=den.to(device), raw_fallback=True)
    torch.cuda.synchronize()
    ref = O.chain_accept(O.raw_prob_row(w, den), cand.numpy(), qids.numpy(), qvals.numpy(), caps.numpy(),
                         u.numpy(), uf.numpy(), prefix.numpy())
    _check_chain(outs, ref, f"raw T={T} K={K}", max_near=1)


# ------------------------------------------------------------------------------------------
# sample_capped_chain_from_probs (sampling/rejection.py:99-153): dense P and dense Q
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("vocab", [1000, 151936])
def test_capped_chain_dense_q(device, vocab):
    from dspine_amd.sampling.rejection import sample_capped_chain_from_probs

    O = _O()
    g = torch.Generator().manual_seed(vocab)
    bs, T = 6, 16
    P = torch.softmax(torch.randn(bs, T, vocab, generator=g) * 2, -1)
    Q = torch.softmax(torch.randn(bs, T - 1, vocab, generator=g) * 2 + P[:, : T - 1].log(), -1)
    Q[0, 3] = 0.0
    Q[0, 3, :10] = 0.1  # a draft row whose mass sits on 10 ids
    Q[1, :, 5] = 1.25  # out-of-range q: clamped to 0 in the residual, never accepted
    cand = torch.zeros(bs, T, dtype=torch.int64)
    cand[:, 1:] = torch.multinomial(Q.clamp(0, 1).reshape(-1, vocab), 1, generator=g).view(bs, T - 1)
    cand[1, 2] = 5
    u = torch.rand(bs, T - 1, generator=g)
    uf = torch.rand(bs, generator=g)
    caps = torch.tensor([16, 16, 1, 9, 12, 16], dtype=torch.int32)
    prefix = torch.arange(bs, dtype=torch.int32)
    outs = _outputs(bs, T, device)
    sample_capped_chain_from_probs(candidates=cand.to(device), target_probs=P.to(device), draft_probs=Q.to(device),
                                   verify_lens=caps.to(device), uniforms=u.to(device), uniform_final=uf.to(device),
                                   prefix_lens=prefix.to(device), outputs=outs)
    torch.cuda.synchronize()
    ref = O.chain_accept(lambda r: P.view(bs * T, vocab)[r].numpy(), cand.numpy(), None, None, caps.numpy(),
                         u.numpy(), uf.numpy(), prefix.numpy(), dense_q=lambda b, s: Q[b, s].numpy())
    _check_chain(outs, ref, f"dense q V={vocab}")


# ------------------------------------------------------------------------------------------
# target distributions (runtime/worker.py:440-508)
# ------------------------------------------------------------------------------------------
def _target_case(seed, bs, T, V, dtype, flags=True):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(bs * T, V, generator=g) * 2.5).to(dtype)
    temps = torch.tensor([0.6, 1.0, 1.3, 0.0])[torch.arange(bs) % 4]
    ks = torch.tensor([20, 64, 5, 1])[torch.arange(bs) % 4]
    ps = torch.tensor([0.95, 1.0, 0.8, 1.0])[torch.arange(bs) % 4]
    info = W.sampling_info(temps, ks, ps) if flags else W.sampling_info(
        torch.full((bs,), 0.8), torch.full((bs,), 1 << 30), torch.ones(bs))
    return logits, info


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("flags", [True, False])
def test_build_target_probs(device, dtype, flags):
    from dspine_amd.runtime.worker import build_dspine_target_probs

    O = _O()
    bs, T, V = 8, 3, 30011
    logits, info = _target_case(5, bs, T, V, dtype, flags)
    got = build_dspine_target_probs(next_token_logits=logits.to(device), sampling_info=W.info_to(info, device),
                                    block_size=T, bs=bs, sampling_backend="pytorch")
    torch.cuda.synchronize()
    ref = O.build_target_probs(logits, info, T, bs, "pytorch", exact_softmax=True)
    assert got.shape == (bs, T, V)
    # probabilities within 1e-5 relative of the float64-exact softmax (fp32 and bf16 logits)
    torch.testing.assert_close(got.cpu(), ref, rtol=1e-5, atol=1e-9)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_build_target_probs_nucleus(device, dtype):
    """Rows with top-k off and a top-p cut (the full-histogram path for bf16, the radix descent
    for float32), mixed with min-p and top-k > 64 rows."""
    from dspine_amd.runtime.worker import build_dspine_target_probs

    O = _O()
    bs, T, V = 6, 2, 50021
    g = torch.Generator().manual_seed(31)
    logits = (torch.randn(bs * T, V, generator=g) * 2.5).to(dtype)
    logits[2 * T:3 * T, :40] = 6.0  # a tie group straddling the cut
    info = W.sampling_info([1.0, 0.7, 1.0, 1.3, 1.0, 0.9], [0, 0, 0, 100, 200, 0],
                           [0.9, 0.5, 0.95, 0.8, 0.99, 1.0], [0.0, 0.0, 0.0, 0.0, 0.0, 0.05])
    got = build_dspine_target_probs(next_token_logits=logits.to(device), sampling_info=W.info_to(info, device),
                                    block_size=T, bs=bs, sampling_backend="pytorch")
    torch.cuda.synchronize()
    ref = O.build_target_probs(logits, info, T, bs, "pytorch", exact_softmax=True)
    torch.testing.assert_close(got.cpu(), ref, rtol=1e-5, atol=1e-9)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_nucleus_cut_inside_ties_across_chunks(device, dtype):
    """A top-p cut inside a group of 40 equal values spread over every chunk of the row (ids
    1237 apart, 85 % of the mass): the kept ties are the lowest ids, so each chunk's ties rank
    after the earlier chunks' (the counts the full-row resolver records for float32 rows).  Both
    the target distribution and the filter on the same rows' probabilities."""
    from dspine_amd.runtime.worker import build_dspine_target_probs, filter_target_probs

    O = _O()
    bs, T, V = 2, 2, 50021
    g = torch.Generator().manual_seed(41)
    logits = (torch.randn(bs * T, V, generator=g) * 2.5).to(dtype)
    ids = torch.arange(40) * 1237
    logits[:, ids] = 12.0
    info = W.sampling_info([1.0, 1.0], [0, 0], [0.5, 0.3])
    got = build_dspine_target_probs(next_token_logits=logits.to(device), sampling_info=W.info_to(info, device),
                                    block_size=T, bs=bs, sampling_backend="pytorch")
    torch.cuda.synchronize()
    ref = O.build_target_probs(logits, info, T, bs, "pytorch", exact_softmax=True)
    torch.testing.assert_close(got.cpu(), ref, rtol=1e-5, atol=1e-9)
    kept = (ref.view(bs * T, V)[:, ids] > 0).sum(-1)
    assert int(kept.min()) > 0 and int(kept.max()) < 40  # the cut splits the group in every row
    probs = O.softmax_temp(logits.float(), torch.ones(bs * T), exact=True)
    got = filter_target_probs(probs.to(device), W.info_to(info, device), T, bs, "pytorch")
    torch.cuda.synchronize()
    ref = O.filter_target_probs(probs.clone(), info, T, bs, "pytorch")
    torch.testing.assert_close(got.cpu(), ref, rtol=1e-5, atol=1e-9)
    assert torch.equal(got.cpu() > 0, ref > 0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_build_target_probs_flashinfer_min_p(device, dtype):
    """flashinfer's min-p branch on nucleus rows (top-k off or > 64): top-p on the mass
    renormalised over the top-k, then min-p against the max (tests/ref_utils.py:79-108)."""
    from dspine_amd.runtime.worker import build_dspine_target_probs

    O = _O()
    bs, T, V = 6, 2, 50021
    g = torch.Generator().manual_seed(33)
    logits = (torch.randn(bs * T, V, generator=g) * 2.5).to(dtype)
    info = W.sampling_info([1.0, 0.7, 1.0, 1.3, 1.0, 0.9], [0, 100, 1000, 0, 200, 0],
                           [0.9, 0.5, 0.95, 0.8, 0.99, 1.0], [0.05, 1e-4, 0.1, 3e-4, 0.01, 1e-5])
    got = build_dspine_target_probs(next_token_logits=logits.to(device), sampling_info=W.info_to(info, device),
                                    block_size=T, bs=bs, sampling_backend="flashinfer")
    torch.cuda.synchronize()
    ref = O.build_target_probs(logits, info, T, bs, "flashinfer", exact_softmax=True)
    torch.testing.assert_close(got.cpu(), ref, rtol=1e-5, atol=1e-9)


@pytest.mark.parametrize("normalize", [True, False])
def test_filter_target_probs(device, normalize):
    from dspine_amd.runtime.worker import filter_target_probs

    O = _O()
    bs, T, V = 8, 2, 5003
    logits, info = _target_case(6, bs, T, V, torch.float32)
    info.is_any_greedy = False
    info.top_ks[2] = 1 << 30  # a top-p only row (top-p 0.8): the float32 nucleus path
    info.max_top_k = int(info.top_ks.max())
    temps = torch.repeat_interleave(info.temperatures.view(-1).clamp_min(0.5), T)
    probs = O.softmax_temp(logits, temps, exact=True)
    got = filter_target_probs(probs.to(device), W.info_to(info, device), T, bs, "pytorch", normalize=normalize)
    torch.cuda.synchronize()
    ref = O.filter_target_probs(probs.clone(), info, T, bs, "pytorch", normalize=normalize)
    torch.testing.assert_close(got.cpu(), ref, rtol=1e-5, atol=1e-9)
    if not normalize:  # kept entries are the input values themselves
        kept = got.cpu() > 0
        assert torch.equal(got.cpu()[kept], probs.view(bs, T, V)[kept])


@pytest.mark.parametrize("backend,min_p", [("pytorch", False), ("pytorch", True), ("flashinfer", False),
                                           ("flashinfer", True)])
def test_filter_target_probs_unnormalised_rows(device, backend, min_p):
    """Rows whose mass is not 1 (runtime/worker.py:52-67, 473-508): the top-p test compares the
    raw mass ranked ahead of an id with top_p -- a row of mass 0.7 under top-p 0.6 keeps ids
    until 0.6 of raw mass (0.857 of its own) lies ahead; flashinfer's min-p branch renormalises
    over the top-k first, so there only the renormalised row matters."""
    from dspine_amd.runtime.worker import filter_target_probs

    O = _O()
    bs, T, V = 4, 2, 3001
    g = torch.Generator().manual_seed(11)
    logits = torch.randn(bs * T, V, generator=g) * 2.0
    mass = torch.tensor([0.7, 1.6, 0.35, 1.0, 0.9, 1.25, 0.5, 2.0])
    probs = torch.softmax(logits.double(), -1).float() * mass.view(-1, 1)
    # list rows (k 50), nucleus rows (no top-k; k 2000 with a cut) and the top-p values
    info = W.sampling_info([1.0] * bs, [0, 50, 0, 2000], [0.6, 0.8, 0.9, 0.95],
                           [0.0, 0.02, 0.0, 0.01] if min_p else None)
    got = filter_target_probs(probs.to(device), W.info_to(info, device), T, bs, backend)
    torch.cuda.synchronize()
    ref = O.filter_target_probs(probs.clone(), info, T, bs, backend)
    torch.testing.assert_close(got.cpu(), ref, rtol=1e-5, atol=1e-9)
    assert torch.equal(got.cpu() > 0, ref > 0)
    if not (backend == "flashinfer" and min_p):  # the raw masses decide a different support here
        unit = O.filter_target_probs((probs / probs.sum(-1, keepdim=True)).clone(), info, T, bs, backend)
        assert not torch.equal(unit > 0, ref > 0)


def test_softmax_temp(device):
    from dspine_amd.runtime.worker import SoftmaxTemp

    O = _O()
    g = torch.Generator().manual_seed(8)
    logits = torch.randn(12, 7001, generator=g) * 3
    temps = torch.tensor([[0.7], [1.0], [1.9]])
    got = SoftmaxTemp.execute(logits=logits.to(device), temperatures=temps.to(device), rows_per_request=4)
    torch.cuda.synchronize()
    ref = O.softmax_temp(logits, torch.repeat_interleave(temps.view(-1), 4), exact=True)
    torch.testing.assert_close(got.cpu(), ref, rtol=1e-5, atol=1e-9)


# ------------------------------------------------------------------------------------------
# build_sparse_target (sampling/sparse/target.py:95-178)
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("capacity", [32, 8])
def test_build_sparse_target(device, capacity):
    from dspine_amd.sampling.sparse.target import build_sparse_target

    O = _O()
    g = torch.Generator().manual_seed(capacity)
    bs, T, V = 6, 4, 20011
    logits = torch.randn(bs * T, V, generator=g) * 2.5
    logits[0, :50] = 9.0  # 50 equal top values: a tie group beyond any capacity -> overflow
    logits[5, :3] = 12.0
    temps = torch.tensor([1.0, 0.7, 1.3, 1.0, 0.9, 1.1])
    ks = torch.tensor([capacity, 5, 1, capacity, 3, 8 if capacity >= 8 else capacity])
    ps = torch.tensor([1.0, 0.9, 0.5, 0.95, 1.0, 0.3])
    info = W.sampling_info(temps, ks, ps)
    info.is_any_greedy = False
    info.max_top_k = int(ks.max())
    st = build_sparse_target(logits.to(device), W.info_to(info, device), block_size=T, capacity=capacity)
    torch.cuda.synchronize()
    assert st is not None
    rows = torch.arange(bs * T) // T
    p = O.softmax_temp(logits, temps[rows], exact=True)
    ids, vals, lens, ovf, dense = O.sparse_target(p, ks[rows], ps[rows], capacity)
    gi, gv, gl, go = (x.cpu() for x in st.packed)
    assert torch.equal(gl, lens) and torch.equal(go, ovf)
    assert torch.equal(gi, ids)
    torch.testing.assert_close(gv, vals, rtol=1e-5, atol=1e-8)
    over = ovf.bool()
    assert bool(over[0])
    torch.testing.assert_close(st.dense_p.cpu()[over], dense[over], rtol=1e-5, atol=1e-9)
    # ineligible batches keep the dense path
    info.need_min_p_sampling = True
    assert build_sparse_target(logits.to(device), W.info_to(info, device), block_size=T, capacity=capacity) is None


# ------------------------------------------------------------------------------------------
# logit adjustments (sampling/compact.py:14-79), padding, window index
# ------------------------------------------------------------------------------------------
def test_adjust_logits_known_answer(device):
    """tests/test_compact_integration.py:37-46."""
    from types import SimpleNamespace

    from dspine_amd.sampling.compact import adjust_logits

    owner = torch.tensor([0, 1, 1], device=device)
    info = SimpleNamespace(temperatures=torch.ones(2, 1), acc_scaling_penalties=torch.tensor([[2.0, 2.0], [.5, .5]]),
                           logit_bias=torch.tensor([[.5, -.5], [1.0, -1.0]]))
    actual = torch.tensor([[2.0, -2.0], [-3.0, 3.0], [4.0, -4.0]], device=device)
    adjust_logits(actual, info, owner)
    torch.cuda.synchronize()
    assert torch.equal(actual.cpu(), torch.tensor([[1.5, -4.5], [-.5, 5.0], [9.0, -3.0]]))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mapped", [True, False])
def test_adjust_logits_bitexact(device, dtype, mapped):
    from types import SimpleNamespace

    from dspine_amd.sampling.compact import adjust_history, adjust_logits

    O = _O()
    g = torch.Generator().manual_seed(17)
    bs, T, V = 5, 4, 151936
    x = (torch.randn(bs * T, V, generator=g) * 3).to(dtype)
    hist = torch.randint(-1, V, (bs, 300), generator=g, dtype=torch.int32)
    pres = torch.rand(bs, generator=g)
    rep = 1 + torch.rand(bs, generator=g)
    add, scl = O.penalties_from_history(hist, pres, rep, V)
    bias = torch.randn(bs, V, generator=g) * 0.1
    info = SimpleNamespace(acc_additive_penalties=add, acc_scaling_penalties=scl, logit_bias=bias)
    if mapped:
        owner = torch.randint(0, bs, (bs * T,), generator=g)
        ref = x.clone()
        O.adjust_logits(ref, info, owner)
        got = x.to(device)
        adjust_logits(got, info, owner.to(device))
        hist_ref = x.clone()
        O.adjust_logits(hist_ref, SimpleNamespace(acc_additive_penalties=add, acc_scaling_penalties=scl), owner)
        hist_got = x.to(device)
        adjust_history(hist_got, hist.to(device), pres.to(device), rep.to(device), row_to_request=owner.to(device))
    else:
        ref = x.clone().view(bs, T, V)
        O.adjust_logits(ref, info, None)
        got = x.to(device).view(bs, T, V)
        adjust_logits(got, info, None)
        hist_ref = x.clone().view(bs, T, V)
        O.adjust_logits(hist_ref, SimpleNamespace(acc_additive_penalties=add, acc_scaling_penalties=scl), None)
        hist_got = x.to(device).view(bs, T, V)
        adjust_history(hist_got, hist.to(device), pres.to(device), rep.to(device))
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), ref)
    assert torch.equal(hist_got.cpu(), hist_ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_adjust_logits_request_rows_padded(device, dtype):
    """The [bs, T, V] layout with 7 rows a request (a partial group of the per-request pass's
    four rows), a vocab that is a multiple of 4 but not of 8 (the rows' four-value tails; the
    value rows stay 16-byte aligned) and 16-byte aligned logits rows on a padded stride:
    bit-exact against the oracle, padding untouched."""
    from types import SimpleNamespace

    from dspine_amd.sampling.compact import adjust_logits

    O = _O()
    g = torch.Generator().manual_seed(23)
    bs, T, V, Vp = 3, 7, 50020, 50024
    full = (torch.randn(bs * T, Vp, generator=g) * 3).to(dtype)
    add = torch.randn(bs, V, generator=g) * 0.2
    scl = 1 + torch.rand(bs, V, generator=g)
    for info in (SimpleNamespace(acc_additive_penalties=add), SimpleNamespace(acc_scaling_penalties=scl)):
        ref = full.clone()
        O.adjust_logits(ref[:, :V].view(bs, T, V), info, None)
        got = full.to(device)
        adjust_logits(got[:, :V].view(bs, T, V), info, None)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_logits_padding(device, dtype):
    """tests/test_release.py:45-67: rows [0, -inf, ...]."""
    from dspine_amd.sampling.padding import logits_padding

    O = _O()
    value = torch.zeros(1, dtype=dtype, device=device)
    got = logits_padding(None, value, (3, 5, 1001))
    torch.cuda.synchronize()
    assert got.dtype == dtype
    assert torch.equal(got.cpu(), O.logits_padding(torch.zeros(1, dtype=dtype), (3, 5, 1001)))


@pytest.mark.parametrize("qdtype", [torch.int32, torch.int64])
def test_window_index(device, qdtype):
    """tests/test_sps.py:446-448: index == [b*T+d for b, n in enumerate(lens) for d < n]."""
    from dspine_amd.verification.sps import window_index

    O = _O()
    g = torch.Generator().manual_seed(3)
    for T in (16, 17):
        lens = torch.randint(1, T + 1, (64,), generator=g)
        qo = torch.cat((torch.zeros(1, dtype=torch.int64), lens.cumsum(0))).to(qdtype)
        got = window_index(qo.to(device), T, int(lens.sum()))
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), O.window_index(lens.numpy(), T))


# ------------------------------------------------------------------------------------------
# serial_sample_chain (kernels/dspine.py:616-772)
# ------------------------------------------------------------------------------------------
def _chain_inputs(bs, T, k, seed, vocab=1000):
    """tests/test_cuda.py:145-159."""
    g = torch.Generator().manual_seed(seed)
    n = bs * (T - 1)
    table = torch.randn(n, k, k, generator=g) * 3.0
    cand = torch.stack([torch.randperm(vocab, generator=g)[:k].sort().values for _ in range(n)])
    greedy_tok = cand[torch.arange(n), torch.randint(0, k, (n,), generator=g)]
    u = torch.rand(n, generator=g)
    return table.contiguous(), cand.contiguous(), greedy_tok.contiguous(), u.contiguous()


def _run_chain(device, table, staged, u, cand, greedy_tok, T, confidence=None):
    from dspine_amd.kernels.dspine import serial_sample_chain

    n, k = cand.shape
    out_tok = torch.full((n,), -1, dtype=torch.int64, device=device)
    out_q = torch.full((n, k), -1.0, dtype=torch.float32, device=device)
    serial_sample_chain(table.to(device), *[x.to(device) for x in staged], u.to(device), cand.to(device),
                        greedy_tok.to(device), out_tok, out_q, T, confidence_out=confidence)
    torch.cuda.synchronize()
    return out_tok.cpu(), out_q.cpu()


def _np(*xs):
    return [x.numpy() for x in xs]


def _staged(params):
    return (torch.tensor([1.0 / p[0] for p in params], dtype=torch.float32),
            torch.tensor([p[1] for p in params], dtype=torch.int32),
            torch.tensor([p[2] for p in params], dtype=torch.float32),
            torch.tensor([p[3] for p in params], dtype=torch.float32),
            torch.tensor([p[4] for p in params], dtype=torch.int32))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_sample_chain_matches_oracle(device, seed):
    """tests/test_cuda.py:174-210."""
    O = _O()
    T, k = 5, 8
    params = [(1.0, k, 1.0, 0.0, 0), (0.7, 3, 0.8, 0.1, 0), (1.5, k, 0.5, 0.0, 0), (1.0, k, 1.0, 0.3, 0),
              (0.3, 1, 1.0, 0.0, 0), (1.0, 1, 1.0, 0.0, 1)]
    bs = len(params)
    table, cand, greedy_tok, u = _chain_inputs(bs, T, k, seed)
    staged = _staged(params)
    n = bs * (T - 1)
    conf = torch.full((n + 3,), -0.5, device=device)
    out_tok, out_q = _run_chain(device, table, staged, u, cand, greedy_tok, T, confidence=conf)
    conf_ref = np.full(n + 3, -0.5, np.float32)
    ref_tok, ref_q = O.sample_chain(*_np(table, *staged, u, cand, greedy_tok), T, confidence=conf_ref)
    assert np.array_equal(out_tok.numpy(), ref_tok)
    torch.testing.assert_close(out_q, torch.as_tensor(ref_q), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(out_q.sum(-1), torch.ones(n), rtol=0, atol=1e-5)
    torch.testing.assert_close(conf.cpu(), torch.as_tensor(conf_ref), rtol=1e-5, atol=1e-6)
    lane = (cand == out_tok[:, None]).float().argmax(-1)
    assert bool((out_q[torch.arange(n), lane] > 0).all())


def test_sample_chain_ties_break_to_lower_lane(device):
    """tests/test_cuda.py:213-232."""
    T, k = 3, 8
    n = T - 1
    table = torch.zeros(n, k, k)
    table[:, :, 2] = 5.0
    table[:, :, 6] = 5.0
    cand = torch.arange(k, dtype=torch.int64).repeat(n, 1) + 100
    staged = (torch.ones(1), torch.tensor([1], dtype=torch.int32), torch.ones(1), torch.zeros(1),
              torch.zeros(1, dtype=torch.int32))
    out_tok, out_q = _run_chain(device, table, staged, torch.zeros(n), cand, cand[:, 0].clone(), T)
    assert out_tok.tolist() == [102, 102]
    assert out_q[:, 2].tolist() == [1.0, 1.0]


def test_sample_chain_realistic(device):
    """tests/test_cuda.py:235-262 (K = 16 lanes of a 151936 vocabulary)."""
    O = _O()
    T, k, bs = 16, 16, 8
    n = bs * (T - 1)
    g = torch.Generator().manual_seed(3)
    table = (torch.randn(n, k, k, generator=g) * 3).contiguous()
    cand = torch.stack([torch.randperm(151936, generator=g)[:k].sort().values for _ in range(n)])
    greedy_tok = cand[torch.arange(n), torch.randint(0, k, (n,), generator=g)]
    u = torch.rand(n, generator=g)
    params = list(zip([1.0, 0.6, 1.3, 1.0, 0.8, 1.0, 2.0, 1.0], [k, 4, k, 2, 16, 1, 8, 1],
                      [1.0, 0.9, 0.7, 1.0, 0.95, 1.0, 0.5, 1.0], [0.0, 0.05, 0.0, 0.0, 0.1, 0.0, 0.2, 0.0],
                      [0, 0, 0, 0, 0, 0, 0, 1]))
    staged = _staged(params)
    out_tok, out_q = _run_chain(device, table, staged, u, cand, greedy_tok, T)
    ref_tok, ref_q = O.sample_chain(*_np(table, *staged, u, cand, greedy_tok), T)
    assert np.array_equal(out_tok.numpy(), ref_tok)
    torch.testing.assert_close(out_q, torch.as_tensor(ref_q), rtol=1e-5, atol=1e-6)


def test_sample_chain_confidence_known_answers(device):
    """tests/test_sampled_confidence.py:124-196."""
    from dspine_amd.kernels.dspine import serial_sample_chain

    width, k = 4, 4
    dist = torch.tensor([[0.899, 0.099, 0.001, 0.001], [0.4, 0.3, 0.2, 0.1], [0.6, 0.2, 0.1, 0.1],
                         [0.25, 0.25, 0.25, 0.25]])
    table = dist.log().expand(width - 1, k, k).clone()
    table[0] = dist[1].log().expand(k, k)
    cand = torch.arange(10, 10 + k).expand(width - 1, k).contiguous()

    def run(draws):
        tokens = torch.empty(width - 1, device=device, dtype=torch.int64)
        q = torch.empty((width - 1, k), device=device)
        conf = torch.full((width - 1,), -1.0, device=device)
        serial_sample_chain(table.to(device), torch.ones(1, device=device),
                            torch.full((1,), k, device=device, dtype=torch.int32), torch.ones(1, device=device),
                            torch.zeros(1, device=device), torch.zeros(1, device=device, dtype=torch.int32),
                            torch.tensor(draws, device=device), cand.to(device), cand[:, 0].clone().to(device),
                            tokens, q, width, confidence_out=conf)
        torch.cuda.synchronize()
        return tokens.cpu(), q.cpu(), conf.cpu()

    first = run([0.05, 0.2, 0.4])
    changed_first = run([0.55, 0.2, 0.4])
    changed_second = run([0.05, 0.95, 0.4])
    assert first[0][0] != changed_first[0][0]
    assert first[2][0] == changed_first[2][0]
    assert first[2][1] != changed_first[2][1]
    assert first[0][1] != changed_second[0][1]
    assert first[2][1] == changed_second[2][1]
    assert first[2][2] != changed_second[2][2]

    p = torch.tensor([[0.85, 0.14, 0.009, 0.001], [0.99, 0.008, 0.001, 0.001]])
    temperature = 0.7
    table2 = (p.log() * temperature).unsqueeze(1).expand(2, k, k).contiguous()
    conf = torch.empty(2, device=device)
    q = torch.empty((2, k), device=device)
    serial_sample_chain(table2.to(device), torch.full((2,), 1 / temperature, device=device),
                        torch.full((2,), 5, device=device, dtype=torch.int32), torch.full((2,), 0.8, device=device),
                        torch.full((2,), 0.05, device=device), torch.zeros(2, device=device, dtype=torch.int32),
                        torch.tensor([0.2, 0.8], device=device), torch.arange(k).expand(2, k).contiguous().to(device),
                        torch.zeros(2, device=device, dtype=torch.int64),
                        torch.empty(2, device=device, dtype=torch.int64), q, 2, confidence_out=conf)
    torch.cuda.synchronize()
    torch.testing.assert_close(q.cpu().amax(-1), torch.ones(2))
    torch.testing.assert_close(conf.cpu(), p.amax(-1), rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------------------------------
# worker seam: accept_dspine_sampled_round / TargetDistribution / dspine_accept_sampling
# ------------------------------------------------------------------------------------------
def _seam_case(seed, bs=10, T=16, V=40009, K=16):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(bs * T, V, generator=g) * 2.5).to(torch.bfloat16)
    info = W.sampling_info(torch.tensor([0.0, 0.6, 1.0, 1.0, 0.8] * (bs // 5)),
                           torch.tensor([1 << 30, 20, 1 << 30, 20, 64] * (bs // 5)),
                           torch.tensor([1.0, 0.95, 0.95, 1.0, 0.9] * (bs // 5)))
    q_ids = torch.stack([torch.randperm(V, generator=g)[:K] for _ in range(bs * (T - 1))]).view(bs, T - 1, K)
    q_ids[:, :, 0] = logits.float().view(bs, T, V)[:, : T - 1].argmax(-1)
    q = torch.softmax(torch.randn(bs, T - 1, K, generator=g) * 2, -1)
    lanes = torch.multinomial(q.view(-1, K), 1, generator=g).view(bs, T - 1)
    cand = torch.cat((torch.zeros(bs, 1, dtype=torch.int64), q_ids.gather(2, lanes[..., None]).squeeze(-1)), 1)
    return logits, info, q_ids, q.contiguous(), cand


def test_worker_seam_fused_equals_explicit(device):
    """accept_dspine_sampled_round (fused, one pass) == dspine_accept_sampling on an explicit
    target P == the oracle, with the same request-seeded uniforms; dense_q stays zero."""
    from dspine_amd.runtime import worker as Wk
    from dspine_amd.sampling.random import RequestRNG

    O = _O()
    bs, T, V = 10, 16, 40009
    logits, info, q_ids, q, cand = _seam_case(11, bs, T, V)
    seeds = torch.arange(bs, dtype=torch.int64) * 7919 + 5
    positions = torch.arange(bs, dtype=torch.int64) + 100
    rng = RequestRNG()
    rng.stage(seeds.to(device), positions.to(device))
    wk = Wk.VerifyWorker(T, device, k=16, random=rng)
    wk._dspine_sampler.stage(q_ids.to(device), q.to(device))
    Wk.set_active_worker(wk)
    d_info = W.info_to(info, device)
    acc, bonus = Wk.accept_dspine_sampled_round(candidates=cand.to(device), next_token_logits=logits.to(device),
                                                sampling_info=d_info)
    P = Wk.build_dspine_target_probs(next_token_logits=logits.to(device), sampling_info=d_info, block_size=T, bs=bs,
                                     sampling_backend="pytorch")
    dense_q = torch.zeros((bs, T - 1, V), device=device)
    acc2, bonus2 = Wk.dspine_accept_sampling(target_probs=P, candidates=cand.to(device),
                                             target_logits=logits.to(device), candidate_ids=q_ids.to(device),
                                             q_rows=q.to(device), sampling_info=d_info, sampling_backend="pytorch",
                                             dense_q=dense_q, random_state=rng)
    torch.cuda.synchronize()
    assert int(dense_q.abs().sum()) == 0
    u_acc = O.seeded_uniforms(seeds.numpy(), positions.numpy(), T - 1, O.ACCEPT)
    u_fin = O.seeded_uniforms(seeds.numpy(), positions.numpy(), 1, O.BONUS).reshape(-1)
    ref = O.verify_step(logits, info, candidates=cand.numpy(), q_ids=q_ids.numpy(), q_values=q.numpy(),
                        verify_lens=np.full(bs, T), uniforms=u_acc, uniform_final=u_fin,
                        prefix_lens=np.zeros(bs, np.int32), exact_softmax=True)
    differing = set()
    for name, a, b in (("accept", acc, acc2), ("bonus", bonus, bonus2)):
        a, b = a.cpu().numpy(), b.cpu().numpy()
        for i in range(bs):
            if a[i] != ref[name][i] or b[i] != ref[name][i]:
                assert ref["margins"][i] < MARGIN, (name, i, a[i], b[i], ref[name][i])
                differing.add(i)
    parity.record("worker seam (fused, explicit P)", bs, int((ref["margins"] < MARGIN).sum()),
                  [(i, float(ref["margins"][i])) for i in sorted(differing)])
    assert len(differing) <= 1, differing
    Wk.set_active_worker(None)


def test_worker_seam_refuses_stale_round(device):
    from dspine_amd.runtime import worker as Wk

    bs, T, V = 5, 16, 4099
    logits, info, q_ids, q, cand = _seam_case(12, bs, T, V)
    wk = Wk.VerifyWorker(T, device)
    Wk.set_active_worker(wk)
    with pytest.raises(RuntimeError):
        Wk.accept_dspine_sampled_round(candidates=cand.to(device), next_token_logits=logits.to(device),
                                       sampling_info=W.info_to(info, device))
    wk._dspine_sampler.stage(q_ids[:4].to(device), q[:4].to(device))
    with pytest.raises(RuntimeError):
        Wk.accept_dspine_sampled_round(candidates=cand.to(device), next_token_logits=logits.to(device),
                                       sampling_info=W.info_to(info, device))
    Wk.set_active_worker(None)
