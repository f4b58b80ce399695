"""Pin the CPU oracle before trusting it: published vectors, the reference tests' known answers,
independent float64 references with explicit sorts/loops, and brute force on tiny inputs.
Each check is chosen so that a plausible slip (dropped term, wrong sign, swapped index, wrong
tie rule) fails it."""

import math
import random
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle.verify_oracle as O

# ---------------------------------------------------------------------------------------
# S5 uniforms
# ---------------------------------------------------------------------------------------
MURMUR_VECTORS = [  # MurmurHash3_x86_32 published test vectors (SMHasher / reference ports)
    (b"", 0, 0x00000000), (b"", 1, 0x514E28B7), (b"", 0xFFFFFFFF, 0x81F16F39),
    (b"\0\0\0\0", 0, 0x2362F9DE), (b"aaaa", 0x9747B28C, 0x5A97808A), (b"aaa", 0x9747B28C, 0x283E0130),
    (b"Hello, world!", 0x9747B28C, 0x24884CBA), (b"abc", 0, 0xB3DD93FA), (b"abcd", 0, 0x43ED676A),
    (b"The quick brown fox jumps over the lazy dog", 0x9747B28C, 0x2FA826CD),
    (b"Hello, world!", 1234, 0xFAF6CDB3), (b"The quick brown fox jumps over the lazy dog", 0, 0x2E4FF723),
]


@pytest.mark.parametrize("data,seed,expected", MURMUR_VECTORS)
def test_murmur3_published_vectors(data, seed, expected):
    assert O.murmur3_x86_32(data, seed) == expected


def test_uniforms_are_murmur_of_the_16_byte_message():
    seeds = [0, -1, -(2 ** 63), 2 ** 63 - 1, 2 ** 40 + 7]
    positions = [0, 19, 214, 8192, 131071]
    for stream in range(4):
        u = O.seeded_uniforms(seeds, positions, 15, stream)
        for r, (s, p) in enumerate(zip(seeds, positions)):
            s &= (1 << 64) - 1
            for c in (0, 1, 7, 14):
                msg = b"".join(int(w).to_bytes(4, "little") for w in
                               (s & 0xFFFFFFFF, s >> 32, p & 0xFFFFFFFF, c + (stream << 16)))
                h = O.murmur3_x86_32(msg, 0)
                assert u[r, c] == np.float32((h >> 8) * 2.0 ** -24)


def test_uniform_layout_invariants():
    # tests/test_random.py:25-53: reordering / compaction / other requests do not change draws;
    # streams, positions and both seed halves matter; values in [0, 1)
    seeds = np.array([0, -1, -(2 ** 63), 2 ** 63 - 1, 2 ** 40 + 7])
    pos = np.array([0, 19, 214, 8192, 131071])
    ref = O.seeded_uniforms(seeds, pos, 15, O.ACCEPT)
    order = [4, 1, 3]
    assert np.array_equal(ref[order], O.seeded_uniforms(seeds[order], pos[order], 15, O.ACCEPT))
    assert ((ref >= 0) & (ref < 1)).all()
    v = [O.seeded_uniforms([7], [99], 15, s) for s in range(4)]
    assert all(not np.array_equal(v[i], v[j]) for i in range(4) for j in range(i))
    assert not np.array_equal(v[0], O.seeded_uniforms([7 + 2 ** 32], [99], 15, 0))
    assert not np.array_equal(v[0], O.seeded_uniforms([7], [100], 15, 0))


# ---------------------------------------------------------------------------------------
# S1 target distribution
# ---------------------------------------------------------------------------------------
def _info(bs, temperature, top_k=None, top_p=None, min_p=None):
    # tests/ref_utils.py:150-162 stand-in: a filter left None is off
    from types import SimpleNamespace
    return SimpleNamespace(
        temperatures=torch.full((bs, 1), float(temperature)),
        top_ks=torch.full((bs,), top_k or O.TOP_K_ALL, dtype=torch.int32),
        top_ps=torch.full((bs,), top_p or 1.0), min_ps=torch.full((bs,), min_p or 0.0),
        need_top_k_sampling=top_k is not None, need_top_p_sampling=top_p is not None,
        need_min_p_sampling=min_p is not None, is_all_greedy=False)


def test_target_probs_hand_computed():
    # tests/test_sampling.py:38-59 with unfiltered p = [.4, .3, .2, .1]
    logits = torch.log(torch.tensor([[4.0, 3.0, 2.0, 1.0]]))
    got = O.build_target_probs(logits, _info(1, 1.0, top_k=2, top_p=0.5), 1, 1, "flashinfer")[0, 0]
    torch.testing.assert_close(got.double(), torch.tensor([4 / 7, 3 / 7, 0, 0]).double(), rtol=0, atol=1e-6)
    got = O.build_target_probs(logits, _info(1, 1.0, top_k=3, top_p=0.8, min_p=0.6), 1, 1, "flashinfer")[0, 0]
    torch.testing.assert_close(got.double(), torch.tensor([4 / 7, 3 / 7, 0, 0]).double(), rtol=0, atol=1e-6)
    got = O.build_target_probs(logits, _info(1, 1.0, top_p=0.75), 1, 1, "pytorch")[0, 0]
    torch.testing.assert_close(got.double(), torch.tensor([4 / 9, 3 / 9, 2 / 9, 0]).double(), rtol=0, atol=1e-6)
    # pytorch backend, top_k=2 and top_p=.5 jointly: support {0, 1}
    got = O.build_target_probs(logits, _info(1, 1.0, top_k=2, top_p=0.5), 1, 1, "pytorch")[0, 0]
    torch.testing.assert_close(got.double(), torch.tensor([4 / 7, 3 / 7, 0, 0]).double(), rtol=0, atol=1e-6)


def _independent_row(logits_row, temperature, top_k, top_p, min_p):
    """float64, explicit Python sort by (-p, id) and explicit mass-ahead loop: the definition of
    the joint top-k / top-p / min-p support (tests/ref_utils.py:79-108)."""
    x = [float(v) for v in logits_row]
    m = max(v / temperature for v in x)
    e = [math.exp(v / temperature - m) for v in x]
    z = sum(e)
    p = [v / z for v in e]
    order = sorted(range(len(p)), key=lambda i: (-p[i], i))
    keep = [False] * len(p)
    ahead = 0.0
    for rank, i in enumerate(order):
        keep[i] = rank < top_k and ahead <= top_p and p[i] >= min_p * p[order[0]]
        ahead += p[i]
    w = [p[i] if keep[i] else 0.0 for i in range(len(p))]
    s = sum(w)
    return torch.tensor([v / s for v in w], dtype=torch.float64)


@pytest.mark.parametrize("temperature,top_k,top_p,min_p", [
    (0.8, None, None, 0.2), (0.6, 20, 0.95, None), (1.0, 7, None, None), (1.2, None, 0.6, None),
    (0.9, 30, 0.9, 0.05)])
def test_target_probs_match_independent_reference(temperature, top_k, top_p, min_p):
    bs, T, V = 3, 4, 200
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(bs * T, V, generator=g) * 3
    info = _info(bs, temperature, top_k, top_p, min_p)
    got = O.build_target_probs(logits, info, T, bs, "pytorch").view(bs * T, V)
    for r in range(bs * T):
        ref = _independent_row(logits[r], temperature, top_k or O.TOP_K_ALL, top_p or 1.0, min_p or 0.0)
        assert torch.equal(got[r] > 0, ref > 0), r
        torch.testing.assert_close(got[r].double(), ref, rtol=1e-5, atol=1e-7)


def test_ties_rank_lower_ids_first():
    # equal probabilities straddling top_k keep the lower ids (stable sort)
    logits = torch.tensor([[1.0, 3.0, 2.0, 3.0, 3.0, 0.0]])
    got = O.build_target_probs(logits, _info(1, 1.0, top_k=2), 1, 1, "pytorch")[0, 0]
    assert (got > 0).tolist() == [False, True, False, True, False, False]


def test_mixed_greedy_rows_are_one_hot_at_first_argmax():
    # tests/test_dynamic_sampling.py:306-331: all-equal greedy rows pick id 0
    info = _info(3, 0.7, top_k=10, top_p=0.8)
    info.is_any_greedy = True
    info.top_ks[[0, 2]] = 1
    logits = torch.randn(3 * 2, 11)
    logits[0:2] = 0
    logits[4:6] = 0
    p = O.build_target_probs(logits, info, 2, 3, "pytorch")
    onehot = torch.zeros(2, 11)
    onehot[:, 0] = 1
    assert torch.equal(p[0], onehot) and torch.equal(p[2], onehot)
    assert bool((p[1] > 0).sum(-1).ge(1).all())


def test_unfiltered_rows_are_not_renormalised():
    # runtime/worker.py:477-478: no filter flag -> the softmax itself
    logits = torch.randn(2, 50)
    p = O.build_target_probs(logits, _info(2, 0.7), 1, 2, "pytorch")
    assert torch.equal(p.view(2, 50), torch.softmax(logits / 0.7, -1))


# ---------------------------------------------------------------------------------------
# S9 adjustments
# ---------------------------------------------------------------------------------------
def test_adjustments_known_answer():
    # tests/test_compact_integration.py:37-46
    from types import SimpleNamespace
    owner = torch.tensor([0, 1, 1])
    info = SimpleNamespace(acc_scaling_penalties=torch.tensor([[2.0, 2.0], [.5, .5]]),
                           logit_bias=torch.tensor([[.5, -.5], [1.0, -1.0]]))
    x = torch.tensor([[2.0, -2.0], [-3.0, 3.0], [4.0, -4.0]])
    O.adjust_logits(x, info, owner)
    assert torch.equal(x, torch.tensor([[1.5, -4.5], [-.5, 5.0], [9.0, -3.0]]))


def test_adjustments_alias_and_noop():
    from types import SimpleNamespace
    # tests/test_logit_adjustments.py:105-115: the additive name wins, never both
    info = SimpleNamespace(acc_linear_penalties=torch.tensor([[1.0, -1.0]]),
                           acc_additive_penalties=torch.tensor([[.5, -.5]]))
    x = torch.tensor([[2.0, -2.0]])
    O.adjust_logits(x, info, torch.tensor([0]))
    assert torch.equal(x, torch.tensor([[2.5, -2.5]]))
    # :118-129: no adjustments leave every bit untouched
    x = torch.tensor([[float("nan"), -0.0, 0.0, -3.0, float("inf")]])
    before = x.view(torch.int32).clone()
    O.adjust_logits(x, SimpleNamespace(), torch.tensor([0]))
    assert torch.equal(x.view(torch.int32), before)


def test_history_penalties_closed_form():
    hist = torch.tensor([[3, 1, 3, -1], [0, 2, -1, -1]], dtype=torch.int32)
    add, scl = O.penalties_from_history(hist, torch.tensor([0.5, 1.0]), torch.tensor([1.25, 2.0]), 5)
    assert add.tolist() == [[0, -0.5, 0, -0.5, 0], [-1.0, 0, -1.0, 0, 0]]
    assert scl.tolist() == [[1, 1.25, 1, 1.25, 1], [2.0, 1, 2.0, 1, 1]]
    from types import SimpleNamespace
    x = torch.tensor([[1.0, 2.0, 3.0, -4.0, 5.0], [-1.0, 2.0, -2.0, 0.0, 3.0]]).bfloat16()
    O.adjust_logits(x, SimpleNamespace(acc_additive_penalties=add, acc_scaling_penalties=scl),
                    torch.tensor([0, 1]))
    # history tokens: (x - pres) then x<0 ? x*r : x/r, rounded to bf16 after each step
    expected = torch.tensor([[1.0, 1.5 / 1.25, 3.0, -4.5 * 1.25, 5.0],
                             [-2.0 * 2.0, 2.0, -3.0 * 2.0, 0.0, 3.0]]).bfloat16()
    assert torch.equal(x, expected)


# ---------------------------------------------------------------------------------------
# S3 chain rejection
# ---------------------------------------------------------------------------------------
def _pure_python_reference(p, candidates, qids, qvals, caps, u, uf, prefix):
    """tests/test_sparse_accept_compact.py:22-53, restated: dense CPU rejection with float64
    sums, written independently of the oracle's vectorised form."""
    answer, offset = [], 0
    for b, length in enumerate(caps):
        a = 0
        while a < length - 1:
            token = candidates[b][a + 1]
            q = sum(v for k, v in zip(qids[b][a], qvals[b][a]) if k == token)
            if q > 0 and q <= 1 and float(np.float32(np.float32(u[b][a]) * np.float32(q))) < p[offset + a][token]:
                a += 1
            else:
                break
        row = p[offset + a]
        weights = list(row)
        if a != length - 1:
            q = dict(zip(qids[b][a], qvals[b][a]))
            weights = [max(v - q.get(k, 0), 0) for k, v in enumerate(row)]
            if sum(weights) <= 0:
                weights = list(row)
        threshold = uf[b] * sum(weights)
        cumulative, bonus = 0, len(row) - 1
        for k, value in enumerate(weights):
            cumulative += value
            if cumulative > threshold:
                bonus = k
                break
        T = len(candidates[b])
        emitted = candidates[b][1:a + 1] + [bonus] + [0] * (T - 1 - a)
        answer.append((a, a + 1, bonus, emitted, prefix[b] + a + 1))
        offset += length
    return answer


@pytest.mark.parametrize("bs", [1, 9, 32])
def test_chain_accept_matches_pure_python(bs):
    rng = torch.Generator().manual_seed(713)
    vocab, T, K = 257, 16, 16
    caps = (torch.arange(bs) % T + 1).tolist()
    caps[0] = T
    rows = sum(caps)
    p = torch.zeros(rows, vocab)
    support = torch.tensor([0, 2, 3, 7, 11, 13, 15])
    p[:, support] = torch.softmax(torch.randn(rows, len(support), generator=rng), -1)
    qids = torch.arange(16).expand(bs, T - 1, K).contiguous()
    qvals = torch.softmax(torch.randn(bs, T - 1, K, generator=rng), -1)
    cand = torch.zeros(bs, T, dtype=torch.int64)
    cand[:, 1:] = torch.multinomial(qvals.reshape(-1, K), 1, generator=rng).view(bs, T - 1)
    u = torch.full((bs, T - 1), .371)
    uf = torch.linspace(.071, .917, bs)
    prefix = torch.arange(bs) + 8191
    cand[0, 1:] = 0
    u[0] = 0  # all accepted
    offsets = np.concatenate(([0], np.cumsum(caps)))[:-1]
    if bs > 1:  # zero residual with u = 1 must resample p
        lo, hi = int(offsets[1]), int(offsets[1]) + caps[1]
        same = torch.softmax(torch.arange(16, dtype=torch.float32), 0)
        p[lo:hi] = 0
        p[lo:hi, :16] = same
        qvals[1] = same
        u[1] = 1
    pn = p.numpy()
    expected = _pure_python_reference(pn.tolist(), cand.tolist(), qids.tolist(), qvals.tolist(), caps,
                                      u.tolist(), uf.tolist(), prefix.tolist())
    got = O.chain_accept(lambda r: pn[r], cand.numpy(), qids.numpy(), qvals.numpy(), caps, u.numpy(),
                         uf.numpy(), prefix.numpy(), row_offsets=offsets)
    for b, (a, c, bonus, emitted, ns) in enumerate(expected):
        assert (int(got[0][b]), int(got[1][b]), int(got[2][b]), got[3][b].tolist(), int(got[4][b])) == \
            (a, c, bonus, emitted, ns), b


def test_chain_accept_is_lossless_monte_carlo():
    """Committed tokens at every reached position follow the target row (chi-square)."""
    from scipy.stats import chisquare

    rng = np.random.default_rng(0)
    V, T, K, trials = 12, 4, 4, 20000
    target = rng.dirichlet(np.ones(V) * 0.7, size=T).astype(np.float32)
    target[:, 5] = 0
    target /= target.sum(1, keepdims=True)
    target = target.astype(np.float32)
    qids = np.array([[0, 3, 5, 9], [1, 2, 3, 4], [0, 6, 7, 11]])
    qv = rng.dirichlet(np.ones(K), size=T - 1).astype(np.float32)
    lanes = np.stack([rng.choice(K, size=trials, p=qv[i] / qv[i].sum()) for i in range(T - 1)], 1)
    drafts = qids[np.arange(T - 1)[None, :], lanes]
    cand = np.concatenate([np.zeros((trials, 1), np.int64), drafts], 1)
    u = rng.random((trials, T - 1), dtype=np.float32)
    uf = rng.random(trials, dtype=np.float32)
    out = O.chain_accept(lambda r: target[r % T], cand, np.broadcast_to(qids, (trials, T - 1, K)),
                         np.broadcast_to(qv, (trials, T - 1, K)), np.full(trials, T), u, uf,
                         np.zeros(trials), row_offsets=np.arange(trials) * T)
    acc, output = out[0], out[3]
    for pos in range(T):
        toks = output[acc >= pos, pos]
        counts = np.bincount(toks, minlength=V)
        assert counts[target[pos] == 0].sum() == 0
        live = target[pos] > 0
        exp = target[pos][live] / target[pos][live].sum() * toks.size
        assert chisquare(counts[live], exp).pvalue > 1e-4, pos


# ---------------------------------------------------------------------------------------
# S4, S6, S8, S10, S11, a19
# ---------------------------------------------------------------------------------------
def test_greedy_accept_brute_force():
    rng = random.Random(3)
    for _ in range(200):
        T = rng.randint(1, 6)
        bs = rng.randint(1, 4)
        top1 = [[rng.randint(0, 3) for _ in range(T)] for _ in range(bs)]
        cand = [[rng.randint(0, 3) for _ in range(T)] for _ in range(bs)]
        caps = [rng.randint(1, T) for _ in range(bs)]
        got = O.greedy_accept(np.array(top1).reshape(-1), np.array(cand), caps, [5] * bs)
        for b in range(bs):
            a = next((i for i in range(caps[b] - 1) if cand[b][i + 1] != top1[b][i]), caps[b] - 1)
            out = [top1[b][a] if i == a else (cand[b][i + 1] if i < T - 1 else 0) for i in range(T)]
            assert int(got[0][b]) == a and int(got[2][b]) == top1[b][a] and got[3][b].tolist() == out
            assert int(got[4][b]) == 5 + a + 1


@pytest.mark.parametrize("k", [16, 128])
def test_topk_known_answer(k):
    # tests/test_topk_compat.py:70-84
    scores = torch.arange(257).remainder(7).float().repeat(2, 1)
    scores[1, 254:] = -torch.inf
    expected = torch.tensor([sorted(range(257), key=lambda i: (-row[i], i))[:k] for row in scores.tolist()])
    v, ids = O.topk(scores, k)
    assert torch.equal(ids, expected) and torch.equal(v, scores.gather(-1, expected))


def test_topk_merge_rule():
    # tests/test_tp_head.py:49-53: [[9, 8, 8]] on ids [0,1,2] and [4,5,6] -> [0, 4, 1, 2]
    values = torch.tensor([[9.0, 8.0, 8.0, 9.0, 8.0, 8.0]])
    ids = torch.tensor([[0, 1, 2, 4, 5, 6]])
    v, pos = O.topk(values, 4)
    assert ids.gather(-1, pos).tolist() == [[0, 4, 1, 2]] and v.tolist() == [[9, 9, 8, 8]]


def test_compress_invariants():
    p = torch.zeros(3, 40)
    p[0, [3, 7, 9]] = torch.tensor([.2, .3, .5])
    p[1, :] = 1 / 40
    p[2, 5] = -0.1
    ids, vals, lens, ovf = O.compress(p, 8)
    assert ids[0, :3].tolist() == [3, 7, 9] and lens.tolist() == [3, 8, 0] and ovf.tolist() == [0, 1, 1]
    assert ids[0, 3:].tolist() == [-1] * 5 and bool((ids[1, 1:] > ids[1, :-1]).all())


def test_window_index_and_kv_slots():
    lens = [1, 3, 16, 2]
    assert O.window_index(lens, 16).tolist() == [b * 16 + d for b, n in enumerate(lens) for d in range(n)]
    pt = np.arange(4 * 30).reshape(4, 30)
    slots = O.kv_slots(pt, [0, 5, 10, 28], [0, 2, 15, 1], 16)
    assert slots[1].tolist()[:4] == [35, 36, 37, -1] and slots[3].tolist()[:3] == [118, 119, -1]


def test_padding_rows_are_one_point():
    # tests/test_release.py:45-67
    padded = O.logits_padding(torch.empty(2, 3), (4, 3))
    assert torch.equal(padded.softmax(-1), torch.tensor([[1.0, 0.0, 0.0]]).expand(4, 3))


def test_sample_chain_ties_to_lower_lane():
    # tests/test_cuda.py:213-232
    T, k = 3, 8
    table = np.zeros((T - 1, k, k), np.float32)
    table[:, :, 2] = 5.0
    table[:, :, 6] = 5.0
    cand = np.arange(k)[None].repeat(T - 1, 0) + 100
    tok, q = O.sample_chain(table, [1.0], [1], [1.0], [0.0], [0], np.zeros(T - 1), cand, cand[:, 0], T)
    assert tok.tolist() == [102, 102] and q[:, 2].tolist() == [1.0, 1.0]


def test_sample_chain_brute_force_distribution():
    """The sampled lane follows q exactly: u sweeps [0, 1) and each lane's share equals q."""
    k, T = 6, 2
    table = np.random.default_rng(1).normal(size=(1, k, k)).astype(np.float32) * 2
    cand = np.arange(k)[None] + 10
    n = 4000
    us = (np.arange(n) + 0.5) / n
    counts = np.zeros(k)
    q_ref = None
    for uval in us:
        tok, q = O.sample_chain(table, [1.0], [4], [0.9], [0.0], [0], np.array([uval]), cand, cand[:, 0], T)
        counts[int(tok[0]) - 10] += 1
        q_ref = q[0]
    np.testing.assert_allclose(counts / n, q_ref, atol=2.0 / n)


def test_exact_softmax_is_rounded_float64():
    # the exact form equals float64 softmax of the float32 values x / T, rounded once; on a
    # flat row it sums to 1 within float32 rounding while torch's float32 softmax does not
    x = torch.zeros(2, 151936)
    x[:, ::7919] = 0.5
    x[1] = torch.randn(151936, generator=torch.Generator().manual_seed(0)) * 3
    T = torch.tensor([1.0, 0.7])
    ex = O.softmax_temp(x, T, exact=True)
    xd = (x / T.view(-1, 1)).double()
    ref = torch.softmax(xd, -1).float()
    assert torch.equal(ex, ref)
    assert abs(ex[0].double().sum().item() - 1.0) < 1e-6
    # closed form on the flat row: p(0) = 1 / (V - 20 + 20 e^0.5)
    p0 = 1.0 / (151936 - 20 + 20 * np.exp(0.5))
    assert abs(ex[0, 1].item() / p0 - 1) < 1e-7


# ---------------------------------------------------------------------------------------
# packed P (sampling/sparse/accept.py:179-204,239-304), RAW rows, sparse joint target (S7),
# draft-chain confidence
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("bs", [1, 9, 32])
@pytest.mark.parametrize("kind", ["compact", "pure_packed", "overflow"])
def test_packed_chain_matches_pure_python(bs, kind):
    """tests/test_sparse_accept_compact.py:56-105: packed rows (support 7, stored in reverse id
    order) give exactly the dense pure-Python reference's outputs."""
    rng = torch.Generator().manual_seed(713)
    vocab, T, K = 257, 16, 16
    caps = (torch.arange(bs) % T + 1).tolist()
    caps[0] = T
    rows = sum(caps)
    p = torch.zeros(rows, vocab)
    support = torch.tensor([0, 2, 3, 7, 11, 13, 15])
    p[:, support] = torch.softmax(torch.randn(rows, len(support), generator=rng), -1)
    qids = torch.arange(16).expand(bs, T - 1, K).contiguous()
    qvals = torch.softmax(torch.randn(bs, T - 1, K, generator=rng), -1)
    cand = torch.zeros(bs, T, dtype=torch.int64)
    cand[:, 1:] = torch.multinomial(qvals.reshape(-1, K), 1, generator=rng).view(bs, T - 1)
    u = torch.full((bs, T - 1), .371)
    uf = torch.linspace(.071, .917, bs)
    prefix = torch.arange(bs) + 8191
    cand[0, 1:] = 0
    u[0] = 0
    offsets = np.concatenate(([0], np.cumsum(caps)))[:-1]
    if bs > 1:
        lo, hi = int(offsets[1]), int(offsets[1]) + caps[1]
        same = torch.softmax(torch.arange(16, dtype=torch.float32), 0)
        p[lo:hi] = 0
        p[lo:hi, :16] = same
        qvals[1] = same
        u[1] = 1
    if kind == "overflow":
        p[::11] = torch.softmax(torch.randn((len(p[::11]), vocab), generator=rng), -1)
    ids, vals, lens, ovf = O.compress(p, 32)
    lane = torch.arange(32)[None, :]
    perm = (lens[:, None].long() - 1 - lane).clamp_min(0)
    packed = (ids.gather(1, perm).where(lane < lens[:, None], -1), vals.gather(1, perm).where(lane < lens[:, None], 0),
              lens, ovf)
    pn = p.numpy()
    expected = _pure_python_reference(pn.tolist(), cand.tolist(), qids.tolist(), qvals.tolist(), caps,
                                      u.tolist(), uf.tolist(), prefix.tolist())
    prob_row = None if kind == "pure_packed" else (lambda r: pn[r])
    got = O.chain_accept(prob_row, cand.numpy(), qids.numpy(), qvals.numpy(), caps, u.numpy(), uf.numpy(),
                         prefix.numpy(), row_offsets=offsets, packed=packed, vocab=vocab)
    for b, (a, c, bonus, emitted, ns) in enumerate(expected):
        assert (int(got[0][b]), int(got[1][b]), int(got[2][b]), got[3][b].tolist(), int(got[4][b])) == \
            (a, c, bonus, emitted, ns), b


def test_packed_bonus_sums_repeated_q_lanes():
    """Packed residual subtracts the clamped q summed over the lanes with an id
    (accept.py:186-193); lanes outside [0, 1] count as 0."""
    packed = (np.array([[7, 3, 9]]), np.array([[0.2, 0.5, 0.3]], np.float32), np.array([3]), np.array([0]))
    qids = np.array([3, 3, 9, 7])
    qvals = np.array([0.2, 0.25, 1.5, 0.05], np.float32)
    # residual in id order (3, 7, 9): (0.5 - 0.45, 0.2 - 0.05, 0.3 - 0) = (0.05, 0.15, 0.3)
    # cdf (0.05, 0.2, 0.5): coins away from the boundaries
    for coin, want in ((0.0, 3), (0.05, 3), (0.2, 7), (0.3, 7), (0.5, 9), (0.99, 9)):
        assert O.packed_bonus(packed, 0, (qids, qvals), coin, 100)[0] == want, coin
    # zero residual mass falls back to p; all-accepted draws from p directly
    full = (np.array([3, 7, 9]), np.array([1.0, 1.0, 1.0], np.float32))
    assert O.packed_bonus(packed, 0, full, 0.5, 100)[0] == 7  # p in id order: 0.5 | 0.2 | 0.3
    assert O.packed_bonus(packed, 0, None, 0.45, 100)[0] == 3


def test_raw_rows_are_ieee_quotients():
    P = torch.tensor([[3.0, 1.0, 0.5]])
    den = torch.tensor([3.0])
    row = O.raw_prob_row(P, den)(0)
    assert row.dtype == np.float32 and row.tolist() == [1.0, np.float32(1.0) / np.float32(3.0), np.float32(0.5 / 3.0)]


def test_sparse_target_equals_full_vocabulary_joint_filter():
    """On unique scores the top-(cap+1) joint support equals the full-vocabulary flashinfer
    joint filter (tests/ref_utils.py:79-108 restated); packed values are the renormalised p."""
    g = torch.Generator().manual_seed(4)
    rows, V, cap = 16, 3001, 32
    p = torch.softmax(torch.randn(rows, V, generator=g) * 3, -1)
    ks = torch.tensor([1, 5, 20, 32] * 4)
    ps = torch.tensor([1.0, 0.9, 0.5, 0.95] * 4)
    ids, vals, lens, ovf, dense = O.sparse_target(p, ks, ps, cap)
    info = SimpleNamespace(top_ks=ks, top_ps=ps, min_ps=torch.zeros(rows), need_top_k_sampling=True,
                           need_top_p_sampling=True, need_min_p_sampling=False)
    full = O.filter_target_probs(p.clone(), info, 1, rows, "flashinfer").view(rows, V)
    assert int(ovf.sum()) == 0 and torch.equal(dense, p)
    for r in range(rows):
        support = torch.nonzero(full[r] > 0).view(-1)
        n = int(lens[r])
        assert torch.equal(ids[r, :n].long(), support) and bool((ids[r, n:] == -1).all())
        torch.testing.assert_close(vals[r, :n], full[r, support], rtol=2e-6, atol=0)


def test_sparse_target_overflow_rows_are_densified():
    """A tie group at the k-th place larger than the capacity overflows; the dense row keeps
    every p >= p[k-1], renormalised (sparse/target.py:60-66,174-177)."""
    p = torch.zeros(1, 100)
    p[0, 10:50] = 0.02
    p[0, 60] = 0.2
    ids, vals, lens, ovf, dense = O.sparse_target(p, torch.tensor([4]), torch.tensor([1.0]), 8)
    assert int(ovf[0]) == 1 and int(lens[0]) == 8
    assert ids[0].tolist() == list(range(10, 18))
    expect = torch.zeros(100)
    expect[10:50] = 0.02 / 1.0
    expect[60] = 0.2
    torch.testing.assert_close(dense[0], expect / expect.sum(), rtol=1e-6, atol=0)


def test_sparse_target_ties_known_answers():
    """The reference's CPU branch (sampling/sparse/target.py:158-165) by hand: every p tied with
    the k-th is kept, and the nucleus tests the mass of the strictly larger p (p = [.3, .2, .2,
    .2, .1], k = 2)."""
    p = torch.tensor([[0.3, 0.2, 0.2, 0.2, 0.1]] * 4)
    ks = torch.tensor([2, 2, 2, 2])
    ps = torch.tensor([1.0, 0.4, 0.3, 0.31])
    ids, vals, lens, ovf, dense = O.sparse_target(p, ks, ps, 8)
    assert lens.tolist() == [4, 4, 1, 4] and ovf.tolist() == [0, 0, 0, 0]
    for r in (0, 1, 3):  # the three ties of the 2nd value are kept: 0.3 < top_p, or top_p = 1
        assert ids[r, :4].tolist() == [0, 1, 2, 3]
        torch.testing.assert_close(vals[r, :4], torch.tensor([0.3, 0.2, 0.2, 0.2]) / 0.9, rtol=1e-6, atol=0)
    assert ids[2, :1].tolist() == [0] and float(vals[2, 0]) == 1.0  # mass 0.3 ahead of the ties: not < 0.3


def test_sparse_target_brute_force_definition():
    """Rows with many ties: the support is, by definition, every p > 0 with fewer than k values
    strictly larger and (top_p >= 1 or their mass < top_p); packed ids ascending with p / sum,
    overflow when more than the capacity are kept (then the dense row holds them)."""
    g = torch.Generator().manual_seed(11)
    rows, V, cap = 40, 60, 8
    levels = torch.randint(0, 6, (rows, V), generator=g).float()
    p = torch.softmax(levels * 0.7, -1)
    ks = torch.randint(1, 8, (rows,), generator=g)
    ps = torch.tensor([1.0, 0.9, 0.5, 0.3, 0.05])[torch.randint(0, 5, (rows,), generator=g)]
    ids, vals, lens, ovf, dense = O.sparse_target(p, ks, ps, cap)
    n_ovf = 0
    for r in range(rows):
        row = p[r].double()
        keep = []
        for j in range(V):
            larger = row > row[j]
            if row[j] > 0 and int(larger.sum()) < int(ks[r]) and (
                    float(ps[r]) >= 1 or float(row[larger].sum()) < float(ps[r])):
                keep.append(j)
        total = float(row[keep].sum())
        if len(keep) > cap:
            n_ovf += 1
            assert int(ovf[r]) == 1
            want = torch.zeros(V, dtype=torch.float64)
            want[keep] = row[keep] / total
            torch.testing.assert_close(dense[r].double(), want, rtol=2e-6, atol=0)
        else:
            assert int(ovf[r]) == 0 and int(lens[r]) == len(keep)
            assert ids[r, :len(keep)].tolist() == keep
            torch.testing.assert_close(vals[r, :len(keep)].double(), row[keep] / total, rtol=2e-6, atol=0)
    assert 0 < n_ovf < rows


def test_sample_chain_confidence_known_answers():
    """tests/test_sampled_confidence.py:169-196: confidence is max p before filtering, also when
    the filter leaves q one-hot; greedy requests leave it untouched."""
    p = np.array([[0.85, 0.14, 0.009, 0.001], [0.99, 0.008, 0.001, 0.001]], np.float32)
    k, width, temperature = 4, 2, 0.7
    table = np.repeat((np.log(p) * temperature)[:, None, :], k, 1).astype(np.float32)
    conf = np.full(2, -1.0, np.float32)
    tok, q = O.sample_chain(table, [1 / temperature] * 2, [5, 5], [0.8, 0.8], [0.05, 0.05], [0, 0],
                            np.array([0.2, 0.8]), np.arange(k)[None].repeat(2, 0), np.zeros(2, np.int64), width,
                            confidence=conf)
    np.testing.assert_allclose(q.max(-1), 1.0)
    np.testing.assert_allclose(conf, p.max(-1), rtol=1e-5)
    conf2 = np.full(2, -1.0, np.float32)
    O.sample_chain(table, [1 / temperature] * 2, [5, 5], [0.8, 0.8], [0.05, 0.05], [0, 1], np.array([0.2, 0.8]),
                   np.arange(k)[None].repeat(2, 0), np.zeros(2, np.int64), width, confidence=conf2)
    assert conf2[1] == -1.0 and conf2[0] == conf[0]


# ------------------------------------------------------------------------------------------
# SPS planner (verification/sps.py:35-99)
# ------------------------------------------------------------------------------------------
def _order_lens(survival, bs, gamma, budget):
    """The reference's brute-force rule (tests/test_sps.py:369-384): positions ordered by
    (-survival, depth, request), the first budget - bs taken, lengths 1 + taken per request."""
    order = sorted(((b, d) for b in range(bs) for d in range(gamma)),
                   key=lambda pair: (-float(survival[pair]), pair[1], pair[0]))
    selected = set(order[:budget - bs])
    return [1 + sum((b, d) in selected for d in range(gamma)) for b in range(bs)], selected


@pytest.mark.parametrize("bs", [1, 3, 9, 17, 65])
def test_allocation_matches_global_survival_order(bs):
    """tests/test_sps.py:360-384: equal confidences tie across rows and depths; the selection
    is the global (-survival, depth, request) order and never takes a descendant without its
    ancestors."""
    generator = torch.Generator().manual_seed(714)
    raw = torch.rand((bs, 15), generator=generator)
    raw[::2] = 1
    table = torch.linspace(0.1, 1.0, 16).expand(15, 16)
    conditional = table[torch.arange(15), (raw * 16).long().clamp(0, 15)]
    survival = conditional.cumprod(-1)
    for budget in (bs, bs * 7 + (bs > 1), bs * 16):
        lens = O.allocate_verify_lens(raw, table, torch.arange(15), budget)
        expected, selected = _order_lens(survival, bs, 15, budget)
        assert lens.tolist() == expected and int(lens.sum()) == budget
        assert all((b, d) in selected for b, n in enumerate(expected) for d in range(n - 1))


def test_allocation_fp32_extreme_survival():
    """tests/test_sps.py:387-417: survival values at the float32 extremes (1 - 2^-24, tiny,
    1e-30) keep ancestor order at every budget, lengths only grow with the budget."""
    bs, gamma = 4, 15
    conditional = torch.tensor([
        [1.0] * gamma,
        [1.0, 1.0 - 2**-24, 1.0 - 2**-23] * 5,
        [1e-30, 1.0, 1e-30] + [1.0] * 12,
        [1.0, torch.finfo(torch.float32).tiny, 1.0, 1e-10] + [1.0] * 11,
    ], dtype=torch.float32)
    table = conditional.T.contiguous()
    raw = torch.tensor([0.125, 0.375, 0.625, 0.875])[:, None].expand(bs, gamma)
    survival = conditional.cumprod(-1).cummin(-1).values
    previous = [1] * bs
    for budget in range(bs, bs * (gamma + 1) + 1):
        lens = O.allocate_verify_lens(raw, table, torch.arange(gamma), budget).tolist()
        expected, selected = _order_lens(survival, bs, gamma, budget)
        assert lens == expected and sum(lens) == budget
        assert all(1 <= n <= gamma + 1 and n >= old for n, old in zip(lens, previous))
        previous = lens


def test_allocation_bucketize_boundaries():
    """Bins from float64 boundaries (tests/test_sps.py:420-448's logit grid): each confidence's
    bin is the count of boundaries strictly below it in float64 (np.searchsorted, left), and the
    lengths follow the brute-force order of the looked-up survival."""
    logits = torch.linspace(-13.815509557963773, 13.815509557963773, 1024, dtype=torch.float64)
    boundaries = ((logits[1:] + logits[:-1]) / 2).sigmoid()
    table = (0.216 * logits + 0.3).sigmoid().float().repeat(15, 1)
    g = torch.Generator().manual_seed(3)
    raw = torch.rand((5, 15), generator=g)
    raw[0] = 1.0
    raw[1, :3] = 0.0
    raw[2, 4] = float(boundaries[500])  # a confidence equal to a boundary (rounded to float32)
    bins = np.searchsorted(boundaries.numpy(), raw.double().numpy(), side="left")
    conditional = table[torch.arange(15), torch.as_tensor(bins)]
    survival = conditional.double().cumprod(-1).float().cummin(-1).values
    for budget in (5, 17, 40, 80):
        lens = O.allocate_verify_lens(raw, table, torch.arange(15), budget, boundaries)
        assert lens.tolist() == _order_lens(survival, 5, 15, budget)[0]


def test_allocation_rejects_budget_outside_block():
    with pytest.raises(ValueError, match="SPS budget"):
        O.allocate_verify_lens(torch.rand(3, 15), torch.rand(15, 4), torch.arange(15), 2)
    with pytest.raises(ValueError, match="SPS budget"):
        O.allocate_verify_lens(torch.rand(3, 15), torch.rand(15, 4), torch.arange(15), 49)


def test_sps_layout_closed_form():
    qo, idx = O.sps_layout([1, 3, 2], 16)
    assert qo.tolist() == [0, 1, 4, 6]
    assert idx.tolist() == [0, 16, 17, 18, 32, 33]


# ------------------------------------------------------------------------------------------
# commit of an accepted round (closed form; parity with SGLang's _commit_accept unpinned)
# ------------------------------------------------------------------------------------------
def test_commit_accept_known_answer():
    """Two requests in pool rows 3 and 0, T = 4: request 0 (prefix 10) accepts 1 of its 4
    positions (commits 2), request 1 (prefix 5, verify length 3) accepts 2 (commits 3)."""
    table = np.full((4, 16), -9, np.int32)
    seq = np.zeros(4, np.int64)
    ocl = np.arange(100, 108, dtype=np.int64)  # window slots b*4 + i
    freed = O.commit_accept([1, 2], [10, 5], [3, 0], table, 4, out_cache_loc=ocl, verify_lens=[4, 3], seq_lens=seq)
    assert table[3, 10:12].tolist() == [100, 101] and (table[3, 12:] == -9).all()
    assert table[0, 5:8].tolist() == [104, 105, 106] and table[0, 8] == -9
    assert seq.tolist() == [8, 0, 0, 12]
    assert freed.tolist() == [102, 103]  # request 1 committed all three verified positions


def test_commit_accept_invariants():
    """Committed + freed slots are exactly the verified window slots; slots already in the
    table are read from it when no window slots are given."""
    rng = np.random.default_rng(3)
    bs, T = 9, 6
    acc = rng.integers(0, T, bs)
    lens = rng.integers(1, T + 1, bs)
    prefix = rng.integers(0, 20, bs)
    rows = rng.permutation(12)[:bs]
    ocl = rng.permutation(1000)[: bs * T].astype(np.int64)
    table = np.full((12, 40), -1, np.int32)
    freed = O.commit_accept(acc, prefix, rows, table, T, out_cache_loc=ocl, verify_lens=lens)
    committed = [int(table[rows[b], prefix[b] + i]) for b in range(bs)
                 for i in range(min(acc[b] + 1, lens[b]))]
    verified = [int(ocl[b * T + i]) for b in range(bs) for i in range(lens[b])]
    assert sorted(committed + freed.tolist()) == sorted(verified)
    # the same round with the slots already in the table
    table2 = np.full((12, 40), -1, np.int32)
    for b in range(bs):
        table2[rows[b], prefix[b]: prefix[b] + T] = ocl[b * T: b * T + T]
    freed2 = O.commit_accept(acc, prefix, rows, table2, T, verify_lens=lens)
    assert freed2.tolist() == freed.tolist()


# ------------------------------------------------------------------------------------------
# draft-side sampling table of the redone last write (kernels/dspine.py:505-613)
# ------------------------------------------------------------------------------------------
def _rs_inputs(seed, bs=2, T=4, H=32, R=16, C=8, V=50, k=4, residual=False):
    g = torch.Generator().manual_seed(seed)
    m, n = bs * T, bs * (T - 1)
    d = dict(raw=torch.randn(m, H, generator=g), rms=torch.rand(m, generator=g) + 0.5,
             query=torch.randn(m, 3 * R, generator=g), codebook=torch.randn(V, C, generator=g) / math.sqrt(C),
             pg=torch.randn(R, C, generator=g) / math.sqrt(C), pv=torch.randn(R, C, generator=g) / math.sqrt(C),
             gb=torch.randn(R, generator=g) * 0.1, w_last=torch.randn(H, R, generator=g) / math.sqrt(R),
             norm_w=1 + 0.1 * torch.randn(H, generator=g), head=torch.randn(V, H, generator=g) / math.sqrt(H))
    d["cand"] = torch.stack([torch.randperm(V, generator=g)[:k].sort().values for _ in range(n)])
    d["anchors"] = torch.randint(0, V, (bs,), generator=g)
    if residual:
        d["res_emb"] = torch.randn(V, 8, generator=g)
        d["res_proj"] = torch.randn(R, 8, generator=g) / math.sqrt(8)
    return d


def _rs_call(d, T, eps=1e-6):
    return O.rs_table(d["raw"], d["rms"], d["query"], d["anchors"], d["cand"], d["codebook"], d["pg"], d["pv"],
                      d["gb"], d["w_last"], d["norm_w"], d["head"], eps, T, res_emb=d.get("res_emb"),
                      res_proj=d.get("res_proj"))


@pytest.mark.parametrize("residual", [False, True])
def test_rs_table_matches_explicit_loops(residual):
    """The explicit per-row, per-sender float64 loops of tests/ref_utils.py:52-76 (senders: the
    anchor on a request's first block row, the previous row's candidates after), with the
    terminal residual added to the value when given."""
    T, eps = 4, 1e-6
    d = _rs_inputs(7, T=T, residual=residual)
    got = _rs_call(d, T, eps)
    m, h = d["raw"].shape
    n, k = d["cand"].shape
    C = d["codebook"].shape[1]
    R = d["pg"].shape[0]
    for b in range(m // T):
        for i in range(T - 1):
            row, nn = b * T + 1 + i, b * (T - 1) + i
            senders = [int(d["anchors"][b])] * k if i == 0 else d["cand"][nn - 1].tolist()
            x = d["raw"][row].double()
            for j, s in enumerate(senders):
                e = math.sqrt(C) * d["codebook"][s].double()
                gate = torch.sigmoid(d["query"][row, :R].double() + d["pg"].double() @ e + d["gb"].double())
                value = d["pv"].double() @ e
                if residual:
                    value = value + d["res_proj"].double() @ d["res_emb"][s].double()
                xr = x + d["rms"][row].double() * (d["w_last"].double() @ (gate * value))
                normalized = xr / torch.sqrt(xr.square().mean() + eps) * d["norm_w"].double()
                want = d["head"][d["cand"][nn]].double() @ normalized
                torch.testing.assert_close(got[nn, j], want, rtol=1e-12, atol=1e-12)


def test_rs_table_closed_forms():
    """A request's first block row has one sender (the anchor) for every lane: all K table rows
    agree; with write_w = 0 the refinement is the identity and T[n, j, c] is the normalised state
    row dotted with the candidate's head row, whatever the sender."""
    T = 5
    d = _rs_inputs(11, T=T)
    got = _rs_call(d, T)
    for b in range(2):
        first = got[b * (T - 1)]
        assert torch.equal(first, first[:1].expand_as(first))
    d["w_last"] = torch.zeros_like(d["w_last"])
    got = _rs_call(d, T)
    for nn in range(got.shape[0]):
        x = d["raw"][nn // (T - 1) * T + 1 + nn % (T - 1)].double()
        xn = x / torch.sqrt(x.square().mean() + 1e-6) * d["norm_w"].double()
        want = d["head"][d["cand"][nn]].double() @ xn
        for j in range(got.shape[1]):
            torch.testing.assert_close(got[nn, j], want, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------------------------------
# Factorized q table (sampling/factorized/kernels.py:179-300, cancellation.py:82-147)
# ------------------------------------------------------------------------------------------
def _factor_inputs(seed, bs=3, T=5, H=64, R=8, C=16, V=64, k=16, f32=False):
    g = torch.Generator().manual_seed(seed)
    dt = torch.float32 if f32 else torch.bfloat16
    rand = lambda *shape: torch.randn(*shape, generator=g) * 0.1  # noqa: E731
    m, n = bs * T, bs * (T - 1)
    return dict(raw=rand(m, H).to(dt), rms=(torch.rand(m, generator=g) + 0.5).float(), query=rand(m, R).to(dt),
                anchors=torch.randint(0, V, (bs,), generator=g),
                cand=torch.stack([torch.randperm(V, generator=g)[:k] for _ in range(n)]),
                codebook=rand(V, C).bfloat16(), pred=rand(R, C), prev=rand(R, C), bias=rand(R), W=rand(H, R),
                norm=1.0 + rand(H), head=rand(V, H).bfloat16())


def test_factor_table_equals_direct_table():
    """The factorized float64 table equals the direct formula of rs_table (pinned by the
    explicit loops of tests/ref_utils.py:52-76) to float64 rounding."""
    d = _factor_inputs(1)
    T = 5
    cache = O.factor_cache(d["codebook"], d["pred"], d["prev"], d["bias"], d["W"], d["norm"], d["head"])
    out, base, safe, out64 = O.factor_table(d["raw"], d["rms"], d["query"], d["anchors"], d["cand"], cache, 1e-6, T)
    direct = O.rs_table(d["raw"], d["rms"], d["query"], d["anchors"], d["cand"], d["codebook"], d["pred"], d["prev"],
                        d["bias"], d["W"], d["norm"], d["head"], 1e-6, T)
    assert bool(safe.all())
    torch.testing.assert_close(out64, direct, rtol=1e-9, atol=1e-12)


def test_factor_table_cancellation_takes_the_direct_form():
    """State rows that cancel a lane's write (x = -a W m in float32) fail the 2^-24 test; those
    entries take the direct form, which still equals the direct table."""
    d = _factor_inputs(2, f32=True)
    T = 5
    cache = O.factor_cache(d["codebook"], d["pred"], d["prev"], d["bias"], d["W"], d["norm"], d["head"])
    # cancel lane 3 of block rows 1 and 6: raw[state row] = -rms * (W m)
    for i, j in ((1, 3), (6, 3)):
        src = i // (T - 1) * T + i % (T - 1) + 1
        sid = int(d["anchors"][i // (T - 1)]) if i % (T - 1) == 0 else int(d["cand"][i - 1, j])
        gate = d["query"][src].double() + cache["G"][sid] + cache["bias"]
        m = torch.sigmoid(gate) * cache["V"][sid]
        d["raw"][src] = (-d["rms"][src].double() * (cache["W"] @ m)).float()
    out, base, safe, out64 = O.factor_table(d["raw"], d["rms"], d["query"], d["anchors"], d["cand"], cache, 1e-6, T)
    assert not bool(safe[1, 3]) and not bool(safe[6, 3]) and int((~safe).sum()) == 2
    direct = O.rs_table(d["raw"], d["rms"], d["query"], d["anchors"], d["cand"], d["codebook"], d["pred"], d["prev"],
                        d["bias"], d["W"], d["norm"], d["head"], 1e-6, T)
    torch.testing.assert_close(out64, direct, rtol=1e-9, atol=1e-12)
