"""CPU restatement of the reference's draft-verification semantics (TEST INFRASTRUCTURE).

Only tests, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use this
module, and only as the checker.  Every function cites the reference file:line it restates
(paths relative to the reference repository root, package ``sglang_dspine``).

Numerics follow the reference's own torch CPU path:
  * softmax with temperature is ``torch.softmax(logits.float() / T)`` (the reference's CPU
    branch, ``sampling/sparse/target.py:133``);
  * the pytorch sampling-backend filter uses ``sort`` + ``cumsum`` exactly as
    ``runtime/worker.py:52-67`` (CPU ``cumsum`` accumulates fp32 in double), with the sort made
    stable so that equal probabilities rank lower ids first (the tie rule of
    ``layers/fp8/coarse.py:20-25`` and ``sampling/tp_head.py:9-14``);
  * chain rejection follows the Triton kernels ``sampling/rejection.py:36-98`` and
    ``sampling/sparse/accept.py:239-307``: the accept test ``u*q < p`` in fp32, the residual and
    its CDF in float64 summed sequentially in vocabulary-id order, as the reference's own
    pure-Python reference does (``tests/test_sparse_accept_compact.py:22-53``).

``PINNED`` lists, per function, what independent check pins it (see tests/test_oracle_*.py).
"""

from __future__ import annotations

import math
from types import SimpleNamespace

import numpy as np
import torch

MASK32 = 0xFFFFFFFF
DRAFT, ACCEPT, BONUS, PREFILL = range(4)  # sampling/random.py:18
TOP_K_ALL = 1 << 30  # "no top-k" in SGLang's sampling params (tests/ref_utils.py:155)

PINNED = {
    "murmur3_x86_32": "published MurmurHash3_x86_32 vectors (SMHasher)",
    "seeded_uniforms": "equals murmur3_x86_32 of the 16-byte message; layout invariants of "
    "tests/test_random.py:25-65",
    "adjust_logits": "known answer tests/test_compact_integration.py:37-46, alias rule "
    "tests/test_logit_adjustments.py:105-115, bit-preserving no-op :118-129",
    "penalties_from_history": "dense==sparse identity and closed form (parity vs SGLang's "
    "penalizer accumulation unpinned)",
    "build_target_probs": "hand-computed tests/test_sampling.py:38-59, float64 independent "
    "reference (explicit sort) on random rows, greedy ties tests/test_dynamic_sampling.py:306-331",
    "chain_accept": "pure-Python dense rejection of tests/test_sparse_accept_compact.py:22-53 "
    "with its special cases, plus Monte-Carlo losslessness (chi-square)",
    "greedy_accept": "closed form; brute force on tiny inputs",
    "topk": "tests/test_topk_compat.py:70-84 known answer, tests/test_tp_head.py:49-53",
    "compress": "invariants of tests/test_p_distribution_reference.py:156-175",
    "window_index": "closed form tests/test_sps.py:446-448",
    "allocate_verify_lens": "the reference's brute-force order (-survival, depth, request) of "
    "tests/test_sps.py:360-384 and its fp32 extreme rows :387-417; bucketize boundaries of :420-448",
    "sps_layout": "closed form (exclusive prefix; tests/test_sps.py:446-448)",
    "rs_table": "the reference's explicit-loop float64 restatement (tests/ref_utils.py:52-76, retold "
    "as scalar loops in the pin); anchor rows identical across senders; write_w = 0 closed form",
    "commit_accept": "hand-computed known answer and invariants (committed + freed = verified "
    "slots); parity with SGLang's _commit_accept unpinned (SGLang is not in the reference)",
    "logits_padding": "tests/test_release.py:45-67",
    "sample_chain": "ties-to-lower-lane known answer tests/test_cuda.py:213-232, brute force; "
    "confidence known answers tests/test_sampled_confidence.py:124-196",
    "packed_bonus": "packed == dense identity on the same P and coins "
    "(tests/test_sparse_accept_compact.py:58-105, whose pure-Python reference :22-53 is the spec)",
    "sparse_target": "equals the full-vocabulary joint filter (flashinfer restatement) on unique "
    "scores; hand-computed ties at the k-th place and the strict nucleus of sampling/sparse/target.py:"
    "158-165; a brute-force restatement of the support's definition on rows of many ties; closed-form "
    "overflow densification",
    "factor_table": "equals the direct float64 table of rs_table (pinned by tests/ref_utils.py:52-76) "
    "within float64 rounding on the reference's shapes, the cancellation rows included; the direct "
    "form is the one taken where the factors cancel",
    "sparse_route": "the eligibility rules of sampling/target.py:53-54 and sampling/sparse/target.py:"
    "106-116, each turned off alone",
}


# ---------------------------------------------------------------------------------------
# S5. Seeded uniforms (sampling/random.py:22-43)
# ---------------------------------------------------------------------------------------

def fmix32(h: int) -> int:
    h ^= h >> 16
    h = (h * 0x85EBCA6B) & MASK32
    h ^= h >> 13
    h = (h * 0xC2B2AE35) & MASK32
    h ^= h >> 16
    return h


def murmur3_x86_32(data: bytes, seed: int = 0) -> int:
    """MurmurHash3_x86_32 (Appleby, public domain), restated from the published algorithm."""
    c1, c2 = 0xCC9E2D51, 0x1B873593
    h = seed & MASK32
    n = len(data)
    nblocks = n // 4
    for i in range(nblocks):
        k = int.from_bytes(data[4 * i: 4 * i + 4], "little")
        k = (k * c1) & MASK32
        k = ((k << 15) | (k >> 17)) & MASK32
        k = (k * c2) & MASK32
        h ^= k
        h = ((h << 13) | (h >> 19)) & MASK32
        h = (h * 5 + 0xE6546B64) & MASK32
    tail = data[4 * nblocks:]
    k = 0
    if len(tail) >= 3:
        k ^= tail[2] << 16
    if len(tail) >= 2:
        k ^= tail[1] << 8
    if len(tail) >= 1:
        k ^= tail[0]
        k = (k * c1) & MASK32
        k = ((k << 15) | (k >> 17)) & MASK32
        k = (k * c2) & MASK32
        h ^= k
    h ^= n
    return fmix32(h)


def seeded_uniforms(seeds, positions, width: int, stream: int) -> np.ndarray:
    """random.py:22-43: for request r and column c, the 32-bit murmur3 of the four words
    (seed & 0xFFFFFFFF, seed >> 32 & 0xFFFFFFFF, position & 0xFFFFFFFF, c + (stream << 16))
    with initial hash 0, finalised with the byte length 16; u = (h >> 8) * 2**-24 (float32)."""
    s = np.asarray(seeds, dtype=np.int64).reshape(-1).astype(np.uint64)
    pos = np.asarray(positions, dtype=np.int64).reshape(-1).astype(np.uint64)
    m = np.uint64(MASK32)
    cols = np.arange(width, dtype=np.uint64) + np.uint64(stream << 16)
    blocks = (
        np.broadcast_to((s & m)[:, None], (s.size, width)),
        np.broadcast_to(((s >> np.uint64(32)) & m)[:, None], (s.size, width)),
        np.broadcast_to((pos & m)[:, None], (s.size, width)),
        np.broadcast_to(cols[None, :], (s.size, width)),
    )
    h = np.zeros((s.size, width), dtype=np.uint64)
    for blk in blocks:
        k = (blk * np.uint64(0xCC9E2D51)) & m
        k = ((k << np.uint64(15)) | (k >> np.uint64(17))) & m
        h ^= (k * np.uint64(0x1B873593)) & m
        h = ((h << np.uint64(13)) | (h >> np.uint64(19))) & m
        h = (h * np.uint64(5) + np.uint64(0xE6546B64)) & m
    h ^= np.uint64(16)
    h ^= h >> np.uint64(16)
    h = (h * np.uint64(0x85EBCA6B)) & m
    h ^= h >> np.uint64(13)
    h = (h * np.uint64(0xC2B2AE35)) & m
    h ^= h >> np.uint64(16)
    return ((h >> np.uint64(8)).astype(np.float32) * np.float32(2.0 ** -24)).astype(np.float32)


def verification_uniforms(seeds, positions, width: int):
    """random.py:107-118 (seeded branch): ACCEPT draws [bs, width-1] and BONUS draws [bs]."""
    u = seeded_uniforms(seeds, positions, width - 1, ACCEPT)
    uf = seeded_uniforms(seeds, positions, 1, BONUS).reshape(-1)
    return u, uf


# ---------------------------------------------------------------------------------------
# S9. Logit adjustments (sampling/compact.py:14-79)
# ---------------------------------------------------------------------------------------

def adjust_logits(logits: torch.Tensor, info, row_to_request=None) -> None:
    """In place, in the reference's order: additive (alias acc_linear_penalties, never both),
    multiplicative ``x<0 ? x*s : x/s``, grammar mask (a boolean ``vocab_mask`` [bs, V], True =
    allowed), then logit_bias.  Full blocks are [B, T, V] (row_to_request None) and packed rows
    are [rows, V] with ``row_to_request``.  Each step rounds to the logits dtype, as the
    in-place torch ops of the reference do."""
    if info is None:
        return

    def mapped(value):
        return (value.index_select(0, row_to_request) if row_to_request is not None
                else value[:, None, :])

    def scale(value):
        pen = mapped(value)
        logits.copy_(torch.where(logits < 0, logits * pen, logits / pen))

    linear = getattr(info, "acc_additive_penalties", None)
    if linear is None:
        linear = getattr(info, "acc_linear_penalties", None)
    if linear is not None:
        logits.add_(mapped(linear))
    scaling = getattr(info, "acc_scaling_penalties", None)
    if scaling is not None:
        scale(scaling)
    mask = getattr(info, "vocab_mask", None)
    if mask is not None:
        m = mask.index_select(0, row_to_request) if row_to_request is not None else mask[:, None, :]
        logits.masked_fill_(~m.expand_as(logits), float("-inf"))
    bias = getattr(info, "logit_bias", None)
    if bias is not None:
        logits.add_(mapped(bias))


def penalties_from_history(hist_ids, presence, repetition, vocab: int):
    """Dense additive/scaling buffers of a presence + repetition penalty over each request's
    token history (ids < 0 are padding): additive[b, t] = -presence[b] and scaling[b, t] =
    repetition[b] for every t in the history of b, 0 and 1 elsewhere."""
    hist = torch.as_tensor(hist_ids).long()
    bs = hist.shape[0]
    present = torch.zeros((bs, vocab), dtype=torch.bool)
    valid = hist >= 0
    rows = torch.arange(bs)[:, None].expand_as(hist)
    present[rows[valid], hist[valid]] = True
    pres = torch.as_tensor(presence, dtype=torch.float32).view(bs, 1)
    rep = torch.as_tensor(repetition, dtype=torch.float32).view(bs, 1)
    additive = torch.where(present, -pres, torch.zeros((), dtype=torch.float32))
    scaling = torch.where(present, rep, torch.ones((), dtype=torch.float32))
    return additive, scaling


# ---------------------------------------------------------------------------------------
# S1 / S2. Target distribution (runtime/worker.py:440-508, :52-67)
# ---------------------------------------------------------------------------------------

def softmax_temp(logits: torch.Tensor, temperatures_rows: torch.Tensor, exact: bool = False) -> torch.Tensor:
    """sampling/sparse/target.py:133 (CPU branch): softmax(logits.float() / T) per row.

    ``exact``: the softmax of the same float32 values x / T evaluated in float64 and rounded
    once to float32.  CPU torch's float32 softmax accumulates its normaliser in float32; on
    flat rows of ~10^5 near-equal values that sum is off by up to ~1e-4 relative (every p
    carries the error), which moves a top-p cut inside a large tie group by a few ties.  The
    exact form is what such rows are pinned against."""
    x = logits.float() / temperatures_rows.float().view(-1, 1)
    if not exact:
        return torch.softmax(x, dim=-1)
    xd = x.double()
    e = torch.exp(xd - xd.max(dim=-1, keepdim=True).values)
    return (e / e.sum(dim=-1, keepdim=True)).float()


def torch_backend_filtered_probs(probs, top_ks, top_ps, min_ps, need_min_p):
    """runtime/worker.py:52-67 with a stable sort (lower id first among equal p)."""
    probs_sort, probs_idx = probs.sort(dim=-1, descending=True, stable=True)
    probs_sum = torch.cumsum(probs_sort, dim=-1)
    probs_sort[torch.arange(0, probs.shape[-1]).view(1, -1) >= top_ks.view(-1, 1)] = 0.0
    probs_sort[probs_sum - probs_sort > top_ps.view(-1, 1)] = 0.0
    if need_min_p:
        thr = probs_sort[:, 0] * min_ps
        probs_sort[probs_sort < thr.view(-1, 1)] = 0.0
    return probs_sort, probs_idx


def _rank_keep(p: torch.Tensor, k: torch.Tensor):
    order = torch.argsort(p, dim=-1, descending=True, stable=True)
    rank = torch.empty_like(order)
    rank.scatter_(-1, order, torch.arange(p.shape[-1]).expand_as(order).contiguous())
    return rank < k.view(-1, 1), order


def _mass_ahead(w: torch.Tensor, order: torch.Tensor) -> torch.Tensor:
    ws = w.gather(-1, order).double()
    ahead = torch.cumsum(ws, -1) - ws
    out = torch.empty_like(ahead)
    out.scatter_(-1, order, ahead)
    return out


def filter_target_probs(probs, info, t, bs, sampling_backend, normalize=True):
    """runtime/worker.py:473-508.  "pytorch" is restated exactly; "flashinfer" (whose
    renorm primitives are not vendored) follows the float64 definition of
    tests/ref_utils.py:79-108 with lower ids first among ties."""
    need_k = bool(getattr(info, "need_top_k_sampling", False))
    need_p = bool(getattr(info, "need_top_p_sampling", False))
    need_min_p = bool(getattr(info, "need_min_p_sampling", False))
    if not (need_k or need_p or need_min_p):
        return probs.view(bs, t, -1)
    top_ks = torch.repeat_interleave(info.top_ks.view(-1), t)
    top_ps = torch.repeat_interleave(info.top_ps.view(-1).float(), t)
    min_ps = torch.repeat_interleave(info.min_ps.view(-1).float(), t)
    if sampling_backend == "pytorch":
        weights, token_ids = torch_backend_filtered_probs(probs, top_ks, top_ps, min_ps, need_min_p)
        probs = torch.zeros_like(probs).scatter_(-1, token_ids, weights)
    elif sampling_backend == "flashinfer":
        in_k, order = _rank_keep(probs, top_ks)
        if need_min_p:
            w = torch.where(in_k, probs, torch.zeros_like(probs))
            w = w / w.sum(-1, keepdim=True)
            w = torch.where(_mass_ahead(w, order) <= top_ps.view(-1, 1).double(), w,
                            torch.zeros_like(w))
            w = w / w.sum(-1, keepdim=True)
            keep = w >= w.amax(-1, keepdim=True) * min_ps.view(-1, 1)
            probs = probs.masked_fill(~(keep & (w > 0)), 0.0)
        else:
            keep = torch.ones_like(probs, dtype=torch.bool)
            if need_k:
                keep &= in_k
            if need_p:
                keep &= _mass_ahead(probs, order) <= top_ps.view(-1, 1).double()
            probs = probs.masked_fill(~keep, 0.0)
    else:
        raise ValueError(f"unsupported sampling backend {sampling_backend!r}")
    if normalize:
        probs = probs / probs.sum(dim=-1, keepdim=True)
    return probs.view(bs, t, -1)


def build_target_probs(logits, info, block_size, bs, sampling_backend="pytorch", exact_softmax=False):
    """runtime/worker.py:440-470: softmax(logits/T) per request, backend filter, then rows of
    greedy requests (top_k <= 1) become one-hot at argmax(logits) (first maximal id)."""
    t = int(block_size)
    temps = torch.repeat_interleave(info.temperatures.view(-1).float(), t)
    probs = softmax_temp(logits, temps, exact=exact_softmax)
    filtered = filter_target_probs(probs, info, t, bs, sampling_backend)
    if getattr(info, "is_any_greedy", False):
        flat = filtered.reshape(bs * t, -1)
        greedy = torch.repeat_interleave(info.top_ks.view(-1) <= 1, t)
        tokens = logits.argmax(dim=-1, keepdim=True)
        selected = flat.gather(-1, tokens).masked_fill(greedy[:, None], 1.0)
        flat.masked_fill_(greedy[:, None], 0.0)
        flat.scatter_(-1, tokens, selected)
    return filtered


def row_info(info, request_of_row):
    """Per-row copy of the sampling parameters (TargetDistribution.dense,
    sampling/target.py:20-25)."""
    idx = torch.as_tensor(request_of_row).long()
    out = SimpleNamespace(**vars(info))
    for name in ("temperatures", "top_ks", "top_ps", "min_ps"):
        setattr(out, name, getattr(info, name).view(-1)[idx].clone())
    return out


# ---------------------------------------------------------------------------------------
# S3. Chain rejection, residual resample and compaction
#     (sampling/rejection.py:36-98, sampling/sparse/accept.py:239-307)
# ---------------------------------------------------------------------------------------

def _clamp01(v: float) -> float:
    return v if (v >= 0.0 and v <= 1.0) else 0.0


def chain_accept(prob_row, candidates, q_ids, q_values, verify_lens, uniforms, uniform_final,
                 prefix_lens, row_offsets=None, dense_q=None, packed=None, vocab=None):
    """Chain rejection for every request.

    prob_row(r) returns target row r as a float32 numpy vector; rows are ``b*T + s`` or
    ``row_offsets[b] + s``.  The draft q of draft s (1-based) is row s-1 of request b: sparse
    ``(q_ids, q_values)`` [bs, T-1, K] (q at a token = sum of its lanes; residual uses the last
    lane with that id, clamped to [0, 1]) or a dense ``dense_q(b, s) -> float32 [V]``.
    Accept iff q > 0, q <= 1 and float32(u*q) < p.  The residual max(p - q, 0) (or p when every
    draft was accepted or the residual has no mass) is summed in float64 in id order; bonus =
    first id with cdf > u_final*mass, default V-1.

    ``packed`` = (ids, values, lengths, overflow) [rows, cap] is packed P
    (sampling/sparse/accept.py:239-304): a row whose overflow flag is 0 (every row when
    ``prob_row`` is None, then ``vocab`` gives V) takes p at a token as the sum of its entries
    with that id, and draws its bonus by ``packed_bonus``.

    Returns (accept, commit, bonus, output [bs, T], new_seq, margins) where margins[b] holds
    the smallest relative decision margin of request b (accept tests and the bonus draw)."""
    cand = np.asarray(candidates, dtype=np.int64)
    bs, T = cand.shape
    caps = np.asarray(verify_lens, dtype=np.int64).reshape(-1)
    u = np.asarray(uniforms, dtype=np.float32).reshape(bs, -1)
    uf = np.asarray(uniform_final, dtype=np.float32).reshape(-1)
    prefix = np.asarray(prefix_lens, dtype=np.int64).reshape(-1)
    offs = None if row_offsets is None else np.asarray(row_offsets, dtype=np.int64).reshape(-1)
    qi = None if q_ids is None else np.asarray(q_ids, dtype=np.int64)
    qv = None if q_values is None else np.asarray(q_values, dtype=np.float32)
    accept = np.zeros(bs, np.int32)
    commit = np.zeros(bs, np.int32)
    bonus_out = np.zeros(bs, np.int64)
    output = np.zeros((bs, T), np.int64)
    new_seq = np.zeros(bs, np.int32)
    margins = np.full(bs, np.inf)

    def is_packed(r):
        return packed is not None and (prob_row is None or int(np.asarray(packed[3])[r]) == 0)

    for b in range(bs):
        cap = int(caps[b])
        base = int(offs[b]) if offs is not None else b * T
        a = 0
        margin = math.inf
        while a < cap - 1:
            token = int(cand[b, a + 1])
            if is_packed(base + a):
                p = packed_p_at(packed, base + a, token)
                V = int(vocab) if prob_row is None else prob_row(base + a).shape[0]
            else:
                row = prob_row(base + a)
                V = row.shape[0]
                p = np.float32(row[token]) if 0 <= token < V else np.float32(0.0)
            if dense_q is not None:
                qrow = dense_q(b, a)
                q = np.float32(qrow[token]) if 0 <= token < V else np.float32(0.0)
            else:
                q = np.float32(0.0)
                for lane in range(qi.shape[-1]):
                    if qi[b, a, lane] == token:
                        q = np.float32(q + qv[b, a, lane])
            coin = np.float32(u[b, a])
            prod = np.float32(coin * q)
            ok = bool(q > 0.0) and bool(q <= 1.0) and bool(prod < p)
            if q > 0.0 and q <= 1.0:
                margin = min(margin, abs(float(prod) - float(p)) / max(float(p), float(prod), 1e-38))
            if ok:
                a += 1
            else:
                break
        all_acc = a == cap - 1
        if is_packed(base + a):
            V = int(vocab) if prob_row is None else prob_row(base + a).shape[0]
            qrow = None if (all_acc or qi is None) else (qi[b, a], qv[b, a])
            bonus, m = packed_bonus(packed, base + a, qrow, float(uf[b]), V)
            margin = min(margin, m)
            accept[b], commit[b], bonus_out[b] = a, a + 1, bonus
            for i in range(T):
                output[b, i] = cand[b, i + 1] if i < a else (bonus if i == a else 0)
            new_seq[b] = prefix[b] + a + 1
            margins[b] = margin
            continue
        prow = prob_row(base + a).astype(np.float64)
        V = prow.shape[0]
        w = prow
        if not all_acc:
            w = prow.copy()
            if dense_q is not None:
                qd = np.asarray(dense_q(b, a), dtype=np.float32).astype(np.float64)
                qd = np.where((qd >= 0.0) & (qd <= 1.0), qd, 0.0)
                w = np.maximum(prow - qd, 0.0)
            else:
                last = {}
                for lane in range(qi.shape[-1]):
                    tid = int(qi[b, a, lane])
                    if 0 <= tid < V:
                        last[tid] = _clamp01(float(qv[b, a, lane]))
                for tid, qval in last.items():
                    w[tid] = max(prow[tid] - qval, 0.0)
            if np.cumsum(w)[-1] <= 0.0:
                w = prow
        cdf = np.cumsum(w)
        mass = float(cdf[-1])
        thr = float(uf[b]) * mass
        hit = np.flatnonzero(cdf > thr)
        bonus = int(hit[0]) if hit.size else V - 1
        if mass > 0 and hit.size:
            lo = float(cdf[bonus - 1]) if bonus > 0 else 0.0
            margin = min(margin, (float(cdf[bonus]) - thr) / mass, (thr - lo) / mass)
        accept[b], commit[b], bonus_out[b] = a, a + 1, bonus
        for i in range(T):
            output[b, i] = cand[b, i + 1] if i < a else (bonus if i == a else 0)
        new_seq[b] = prefix[b] + a + 1
        margins[b] = margin
    return accept, commit, bonus_out, output, new_seq, margins


def packed_p_at(packed, row: int, token: int) -> np.float32:
    """p of a packed row at a token: the float32 sum of its entries with that id
    (sampling/sparse/accept.py:270-274)."""
    ids, vals, lens = (np.asarray(x) for x in packed[:3])
    p = np.float32(0.0)
    for i in range(int(lens[row])):
        if int(ids[row, i]) == token:
            p = np.float32(p + np.float32(vals[row, i]))
    return p


def packed_bonus(packed, row: int, q, coin: float, V: int):
    """sampling/sparse/accept.py:179-204: the packed entries in ascending id order; the
    residual subtracts, at each id, the clamped q summed over the draft lanes with that id (q
    None: every draft accepted, the residual is p); zero residual mass falls back to p; bonus =
    first id with cdf > coin*mass (float64, id order), default V-1.  Returns (bonus, margin)."""
    ids, vals, lens = (np.asarray(x) for x in packed[:3])
    n = int(lens[row])
    entries = sorted(int(ids[row, i]) for i in range(n))
    p = [float(packed_p_at(packed, row, t)) for t in entries]
    w = list(p)
    if q is not None:
        qids, qvals = q
        at = []
        for t in entries:
            acc = 0.0
            for lane in range(len(qids)):
                if int(qids[lane]) == t:
                    acc += _clamp01(float(qvals[lane]))
            at.append(acc)
        w = [max(pv - av, 0.0) for pv, av in zip(p, at)]
        if sum(w) <= 0.0:
            w = list(p)
    cdf = np.cumsum(np.asarray(w, dtype=np.float64)) if w else np.zeros(0)
    mass = float(cdf[-1]) if cdf.size else 0.0
    thr = coin * mass
    for i, t in enumerate(entries):
        if cdf[i] > thr and t < V:
            lo = float(cdf[i - 1]) if i > 0 else 0.0
            m = min((float(cdf[i]) - thr) / mass, (thr - lo) / mass) if mass > 0 else math.inf
            return t, m
    return V - 1, math.inf


def raw_prob_row(dense_p, denominator):
    """RAW target rows (sampling/sparse/accept.py:119-128,153-160,259-268): p / denominator[row]
    in IEEE float32."""
    P = torch.as_tensor(dense_p, dtype=torch.float32)
    den = torch.as_tensor(denominator, dtype=torch.float32).view(-1)
    return lambda r: (P[r] / den[r]).numpy()


# ---------------------------------------------------------------------------------------
# S4. Greedy accept (verification/caps.py:46-59, verification/ragged.py:64-76)
# ---------------------------------------------------------------------------------------

def greedy_accept(top1, candidates, caps, prefix_lens):
    """a = first i < cap-1 with cand[b, i+1] != top1[b*T+i] (else cap-1); bonus = top1[b*T+a];
    output keeps the proposed tokens after a (not zeroed); row T-1 has proposal 0."""
    cand = np.asarray(candidates, dtype=np.int64)
    bs, T = cand.shape
    top = np.asarray(top1, dtype=np.int64).reshape(bs, T)
    caps = np.asarray(caps, dtype=np.int64).reshape(-1)
    prefix = np.asarray(prefix_lens, dtype=np.int64).reshape(-1)
    accept = np.zeros(bs, np.int32)
    bonus = np.zeros(bs, np.int64)
    output = np.zeros((bs, T), np.int64)
    for b in range(bs):
        cap = int(caps[b])
        a = cap - 1
        for i in range(cap - 1):
            if cand[b, i + 1] != top[b, i]:
                a = i
                break
        bonus[b] = top[b, a]
        for i in range(T):
            proposed = cand[b, i + 1] if i < T - 1 else 0
            output[b, i] = bonus[b] if i == a else proposed
        accept[b] = a
    return accept, accept + 1, bonus, output, (prefix + accept + 1).astype(np.int32)


def argmax_rows(logits: torch.Tensor) -> np.ndarray:
    """First maximal id per row (torch CPU argmax semantics)."""
    return logits.argmax(dim=-1).numpy().astype(np.int64)


# ---------------------------------------------------------------------------------------
# S6 / S8 / S10 / S11
# ---------------------------------------------------------------------------------------

def topk(scores: torch.Tensor, k: int):
    """layers/fp8/coarse.py:20-25, sampling/tp_head.py:9-14: the first k entries of a stable
    descending sort (lower id wins ties), as (values, ids)."""
    ids = torch.argsort(scores, dim=-1, descending=True, stable=True)[..., :k].contiguous()
    return scores.gather(-1, ids), ids


def compress(p: torch.Tensor, capacity: int):
    """sampling/sparse/accept.py:7-78: ids with p > 0 in id order, up to capacity; length =
    min(n, capacity); overflow = n > capacity or any negative/NaN/inf; padding id -1, value 0."""
    rows, vocab = p.shape
    ids = torch.full((rows, capacity), -1, dtype=torch.int32)
    vals = torch.zeros((rows, capacity), dtype=torch.float32)
    lengths = torch.zeros(rows, dtype=torch.int32)
    overflow = torch.zeros(rows, dtype=torch.int32)
    for r in range(rows):
        x = p[r].float()
        nz = torch.nonzero(x > 0).view(-1)
        n = int(nz.numel())
        m = min(n, capacity)
        ids[r, :m] = nz[:m].int()
        vals[r, :m] = x[nz[:m]]
        lengths[r] = m
        bad = bool(((x < 0) | torch.isnan(x) | torch.isinf(x)).any())
        overflow[r] = int(n > capacity or bad)
    return ids, vals, lengths, overflow


def logits_padding(value: torch.Tensor, shape):
    """sampling/padding.py:4-12: rows become the one-point distribution [0, -inf, ...]."""
    padded = value.new_full(shape, float("-inf"))
    padded[..., 0] = 0.0
    return padded


def window_index(lens, T: int) -> np.ndarray:
    """verification/sps.py:27-32 and :94-98: [b*T + d for each b, for d < lens[b]]."""
    return np.array([b * T + d for b, n in enumerate(np.asarray(lens).tolist()) for d in range(n)],
                    dtype=np.int64)


def allocate_verify_lens(raw, probabilities, depth, budget, boundaries=None) -> torch.Tensor:
    """verification/sps.py:35-58 on CPU torch: bins by ``bucketize`` against the float64
    boundaries (else ``(raw * bins).to(int64).clamp(0, bins-1)``), conditional =
    ``probabilities[depth, bins]``, survival = ``cumprod`` (CPU: float64 accumulation, each
    prefix rounded to float32) then ``cummin``; the first ``budget - bs`` positions of a stable
    descending argsort of the position-major survival; lengths = 1 + positions per request."""
    raw = torch.as_tensor(raw, dtype=torch.float32)
    bs, gamma = raw.shape
    if not bs <= budget <= bs * (gamma + 1):
        raise ValueError("SPS budget must include every root and fit the draft block")
    probabilities = torch.as_tensor(probabilities, dtype=torch.float32)
    n_bins = probabilities.shape[-1]
    if boundaries is not None:
        bins = torch.bucketize(raw.contiguous(), torch.as_tensor(boundaries, dtype=torch.float64))
    else:
        bins = (raw * n_bins).to(torch.int64).clamp_(0, n_bins - 1)
    conditional = probabilities[torch.as_tensor(depth, dtype=torch.int64), bins]
    survival = conditional.cumprod(dim=-1).cummin(dim=-1).values
    survival = survival.transpose(0, 1).contiguous().view(-1)
    selected = torch.argsort(survival, descending=True, stable=True)[: budget - bs]
    lens = torch.ones((bs,), dtype=torch.int32)
    lens.scatter_add_(0, selected.remainder(bs), torch.ones_like(selected, dtype=torch.int32))
    return lens


def sps_layout(lens, T: int):
    """The ragged layout of verify lengths: (qo_indptr int32 [bs + 1] = exclusive prefix,
    window index int64 = [b*T + d for d < lens[b]]) (verification/sps.py:86-98)."""
    lens = np.asarray(lens, dtype=np.int64).reshape(-1)
    qo = np.zeros(lens.size + 1, dtype=np.int32)
    qo[1:] = np.cumsum(lens)
    return qo, window_index(lens, T)


def commit_accept(accept, prefix_lens, req_pool_indices, req_to_token, T: int, out_cache_loc=None,
                  verify_lens=None, slot_offsets=None, seq_lens=None):
    """The commit after a verified round (SGLang's _commit_accept, which the reference's
    tests/test_tp_accept.py:106-180 drive; SGLang is not part of the reference, so this is the
    closed form -- parity with SGLang unpinned): request b verified n_b positions prefix_b + i
    and commits c_b = accept_b + 1 of them.  With window slots, req_to_token[row_b, prefix_b + i]
    = slot for i < c_b; seq_lens[row_b] = prefix_b + c_b; the slots of positions c_b .. n_b - 1
    in (b, i) order are freed.  Mutates req_to_token / seq_lens (numpy) in place; returns the
    freed slots (int64)."""
    acc = np.asarray(accept, dtype=np.int64).reshape(-1)
    bs = acc.size
    prefix = np.asarray(prefix_lens, dtype=np.int64).reshape(-1)
    rows = np.asarray(req_pool_indices, dtype=np.int64).reshape(-1)
    lens = np.full(bs, T) if verify_lens is None else np.asarray(verify_lens, dtype=np.int64).reshape(-1)
    freed = []
    for b in range(bs):
        n = int(min(max(lens[b], 1), T))
        c = int(min(max(acc[b] + 1, 1), n))
        base = int(slot_offsets[b]) if slot_offsets is not None else b * T
        for i in range(n):
            pos = int(prefix[b]) + i
            in_table = 0 <= pos < req_to_token.shape[1]
            if out_cache_loc is not None:
                slot = int(out_cache_loc[base + i])
                if i < c and in_table:
                    req_to_token[rows[b], pos] = slot
            else:
                slot = int(req_to_token[rows[b], pos]) if in_table else -1
            if i >= c:
                freed.append(slot)
        if seq_lens is not None:
            seq_lens[rows[b]] = int(prefix[b]) + c
    return np.asarray(freed, dtype=np.int64)


def kv_slots(page_table, prefix_lens, accept, T: int) -> np.ndarray:
    """Committed KV slots (page size 1): page_table[b, prefix_b + i] for i <= a_b, -1 after
    (verify writes KV for prefix..prefix+T-1, verification/caps.py:255-257; NewSeq =
    prefix + a + 1)."""
    pt = np.asarray(page_table, dtype=np.int64)
    prefix = np.asarray(prefix_lens, dtype=np.int64).reshape(-1)
    acc = np.asarray(accept, dtype=np.int64).reshape(-1)
    out = np.full((acc.size, T), -1, dtype=np.int32)
    for b in range(acc.size):
        for i in range(int(acc[b]) + 1):
            pos = int(prefix[b]) + i
            out[b, i] = pt[b, pos] if 0 <= pos < pt.shape[1] else -1
    return out


# ---------------------------------------------------------------------------------------
# S7. Sparse joint target (sampling/sparse/target.py:95-178, CPU form :156-178)
# ---------------------------------------------------------------------------------------

def sparse_target(p: torch.Tensor, top_ks_rows, top_ps_rows, capacity: int):
    """From softmax rows p [rows, V] float32: the top-(capacity+1) prefix (lower id first among
    equal p); keep p > 0, p >= p[k-1] and the nucleus (mass of strictly larger prefix p <
    top_p, or top_p >= 1); pack ids ascending with p / sum(kept) into [rows, capacity] (-1 / 0
    padding); lengths = min(count, capacity); overflow = count > capacity.  Overflow rows of the
    returned dense copy are p * (p >= p[k-1]) / sum; other rows are p unchanged.
    Returns (ids, values, lengths, overflow, dense)."""
    rows, vocab = p.shape
    width = min(capacity + 1, vocab)
    order = torch.argsort(p, dim=-1, descending=True, stable=True)[:, :width]
    top = p.gather(1, order)
    ks = torch.as_tensor(top_ks_rows).long().view(-1).clamp(1, width)
    tps = torch.as_tensor(top_ps_rows, dtype=torch.float32).view(-1)
    threshold = top.gather(1, (ks - 1)[:, None])
    higher = (top[:, None, :] * (top[:, None, :] > top[:, :, None])).sum(-1)
    keep = (top > 0) & (top >= threshold) & ((higher < tps[:, None]) | (tps[:, None] >= 1))
    count = keep.sum(-1)
    kept = top.masked_fill(~keep, 0)
    kept = kept / kept.sum(-1, keepdim=True)
    key = order.masked_fill(~keep, 2147483647)
    sorted_ids, perm = key.sort(-1)
    kept = kept.gather(1, perm)
    ids = torch.full((rows, capacity), -1, dtype=torch.int32)
    vals = torch.zeros((rows, capacity), dtype=torch.float32)
    n = min(width, capacity)
    ids[:, :n] = sorted_ids[:, :n].masked_fill(sorted_ids[:, :n] == 2147483647, -1).int()
    vals[:, :n] = kept[:, :n]
    overflow = (count > capacity).int()
    dense = p.clone()
    for r in range(rows):
        if overflow[r]:
            dense[r] = dense[r].masked_fill(dense[r] < threshold[r], 0)
            dense[r] /= dense[r].sum()
    return ids, vals, count.clamp_max(capacity).int(), overflow, dense


# ---------------------------------------------------------------------------------------
# a19. Draft-side K-lane chain (kernels/dspine.py:616-674)
# ---------------------------------------------------------------------------------------

def sample_chain(table, inv_temp, top_k, top_p, min_p, greedy, u, cand, greedy_tok, block_size,
                 confidence=None):
    """Per request, walk T-1 rows of the [K, K] table: p = softmax(table[row, sender] * inv_t);
    rank/mass-ahead with lower lanes first among ties; keep rank < top_k, mass-ahead <= top_p,
    p >= min_p * max p; q = w / sum w; choice = #(cdf <= u * cdf[K-1]) clamped to the last kept
    lane.  Greedy requests emit greedy_tok with a one-hot q.  The sender of the next row is the
    sampled lane.  fp32 arithmetic, sums in lane order.  ``confidence`` (float32 [>= n], kernels/
    dspine.py:645-648) receives max p of each row of a non-greedy request (before filtering);
    rows of greedy requests are left as they are."""
    table = np.asarray(table, dtype=np.float32)
    n, K, _ = table.shape
    tm1 = int(block_size) - 1
    out_tok = np.zeros(n, np.int64)
    out_q = np.zeros((n, K), np.float32)
    cand = np.asarray(cand, dtype=np.int64)
    for b in range(n // tm1):
        sender = 0
        for i in range(tm1):
            r = b * tm1 + i
            scores = (table[r, sender] * np.float32(inv_temp[b])).astype(np.float32)
            mx = scores.max()
            mass = np.exp((scores - mx).astype(np.float32)).astype(np.float32)
            tot = np.float32(0.0)
            for c in range(K):
                tot = np.float32(tot + mass[c])
            p = (mass / tot).astype(np.float32)
            pmax = p.max()
            if confidence is not None and not int(greedy[b]):
                confidence[r] = pmax
            keep = np.zeros(K, bool)
            for c in range(K):
                ahead = [d for d in range(K) if p[d] > p[c] or (p[d] == p[c] and d < c)]
                before = np.float32(0.0)
                for d in sorted(ahead, key=lambda d: (-p[d], d)):
                    before = np.float32(before + p[d])
                keep[c] = (len(ahead) < int(top_k[b]) and before <= np.float32(top_p[b])
                           and p[c] >= np.float32(np.float32(min_p[b]) * pmax))
            w = np.where(keep, p, np.float32(0.0)).astype(np.float32)
            ws = np.float32(0.0)
            for c in range(K):
                ws = np.float32(ws + w[c])
            q = (w / ws).astype(np.float32)
            cdf = np.zeros(K, np.float32)
            acc = np.float32(0.0)
            for c in range(K):
                acc = np.float32(acc + q[c])
                cdf[c] = acc
            threshold = np.float32(np.float32(u[r]) * cdf[K - 1])
            choice = int((cdf <= threshold).sum())
            last = max([c for c in range(K) if keep[c]], default=0)
            choice = min(choice, last)
            if int(greedy[b]):
                out_tok[r] = greedy_tok[r]
                out_q[r] = (cand[r] == greedy_tok[r]).astype(np.float32)
            else:
                out_tok[r] = cand[r, choice]
                out_q[r] = q
            sender = choice
    return out_tok, out_q


# ---------------------------------------------------------------------------------------
# The full verify step (S9 -> S1 -> S3 -> S11)
# ---------------------------------------------------------------------------------------

def rs_table(raw, rms, query, anchors, cand, codebook, pg, pv, gb, w_last, norm_w, head, eps, T,
             res_emb=None, res_proj=None, candidate_head=None) -> torch.Tensor:
    """float64 [n, K, K] table of the redone last write (kernels/dspine.py:505-613, the float64
    reference tests/ref_utils.py:52-76, vectorised): for block row n of request b (state row
    b*T + 1 + i), sender lane j (the anchor on i == 0, else candidate j of row n-1) and candidate
    c: e = sqrt(C) codebook[s]; msg = sigmoid(q + pg e + gb) * (pv e [+ res_proj res_emb[s]]);
    ref = x + rms * (w_last msg); T[n, j, c] = head[c] . (ref / sqrt(mean(ref^2) + eps) * norm_w)."""
    d = torch.float64
    m, h = raw.shape
    n, k = cand.shape
    r = pg.shape[0]
    bs = m // T
    rows = torch.tensor([b * T + 1 + i for b in range(bs) for i in range(T - 1)])
    prev = torch.cat((torch.as_tensor(anchors).view(bs, 1, 1).expand(bs, 1, k),
                      torch.as_tensor(cand).view(bs, T - 1, k)[:, :-1, :]), 1).reshape(n, k)
    e = math.sqrt(codebook.shape[1]) * codebook.to(d)[prev]                      # [n, K, C]
    gate = torch.sigmoid(query[rows, :r].to(d)[:, None, :] + e @ pg.to(d).T + gb.to(d))
    value = e @ pv.to(d).T
    if res_emb is not None:
        value = value + res_emb.to(d)[prev] @ res_proj.to(d).T
    ref = raw.to(d)[rows][:, None, :] + rms.to(d)[rows][:, None, None] * ((gate * value) @ w_last.to(d).T)
    normalized = ref / torch.sqrt(ref.square().mean(-1, keepdim=True) + eps) * norm_w.to(d)
    hd = (head.to(d)[torch.as_tensor(cand)] if candidate_head is None else candidate_head.to(d))  # [n, K, H]
    return torch.einsum("njh,nch->njc", normalized, hd)


def factor_cache(codebook, pred, prev, bias, W, norm, head, res_emb=None, res_proj=None) -> dict:
    """sampling/factorized/weights.py:34-80 in float64: W, norm, bias, Gram = W^T W, and per
    vocabulary row G = e pred^T, V = e prev^T (+ res_emb res_proj^T), TG = (head * norm) W with
    e = sqrt(C) codebook."""
    c = codebook.shape[1]
    wd, pd, vd, nd, bd = (z.double() for z in (W, pred, prev, norm, bias))
    e = math.sqrt(c) * codebook.double()
    value = e @ vd.T
    if res_emb is not None:
        value = value + res_emb.double() @ res_proj.double().T
    return {"W": wd, "norm": nd, "bias": bd, "Gram": wd.T @ wd, "head": head, "G": e @ pd.T, "V": value,
            "TG": head.double() * nd @ wd}


def factor_table(raw, rms, query, anchors, cand, cache, eps, T, candidate_head=None):
    """sampling/factorized/kernels.py:15-300 with cancellation.py:82-147, float64 on the CPU.
    Returns (out float32 [n, K, K], base float64 [n, K], safe bool [n, K], out64 float64)."""
    d = torch.float64
    n, k = cand.shape
    h, r = raw.shape[1], query.shape[1]
    bs = anchors.numel()
    rows = torch.tensor([i // (T - 1) * T + i % (T - 1) + 1 for i in range(n)])
    x = raw[rows].to(d)
    a = rms[rows].to(d)
    first = (x * x).sum(-1)
    cand = torch.as_tensor(cand)
    # the sender of (i, j): the anchor on a request's first block row, else candidate j of row i-1
    sid = torch.cat((torch.as_tensor(anchors).view(bs, 1, 1).expand(bs, 1, k),
                     cand.view(bs, T - 1, k)[:, :-1, :]), 1).reshape(n, k)
    gate = query[rows].to(d)[:, None, :] + cache["G"][sid] + cache["bias"]
    message = 1.0 / (1.0 + torch.exp(-gate)) * cache["V"][sid]                    # [n, K, R]
    tg = cache["TG"][cand]                                                       # [n, K, R]
    heads = cache["head"][cand].to(d) if candidate_head is None else candidate_head.reshape(n, k, h).to(d)
    base = (x[:, None, :] * heads * cache["norm"]).sum(-1)                       # [n, K]
    product = torch.einsum("njr,ncr->njc", message, tg)
    xw = x @ cache["W"]
    mg = message @ cache["Gram"]
    cross = (xw[:, None, :] * message).sum(-1)
    quadratic = (mg * message).sum(-1)
    second = 2.0 * a[:, None] * cross
    third = a[:, None] * a[:, None] * quadratic
    dd = first[:, None] + second + third
    magnitude = first[:, None].abs() + second.abs() + third.abs()
    safe = (torch.isfinite(dd) & torch.isfinite(magnitude) & (dd >= 0)
            & ((magnitude == 0) | (dd > 2.0 ** (-24) * magnitude)))
    out64 = (base[:, None, :] + a[:, None, None] * product) / torch.sqrt(dd / h + eps)[..., None]
    for ni, ji in (~safe).nonzero().tolist():
        y = x[ni] + a[ni] * (cache["W"] @ message[ni, ji])
        z = y / torch.sqrt(y.square().mean() + eps) * cache["norm"]
        out64[ni, ji] = heads[ni] @ z
    return out64.float(), base, safe, out64


def make_info(temperatures, top_ks, top_ps, min_ps=None, *, need_top_k=None, need_top_p=None,
              need_min_p=None, is_any_greedy=None):
    """A duck-typed SamplingBatchInfo holding the fields the verify path reads."""
    t = torch.as_tensor(temperatures, dtype=torch.float32).view(-1, 1)
    k = torch.as_tensor(top_ks, dtype=torch.int32).view(-1)
    p = torch.as_tensor(top_ps, dtype=torch.float32).view(-1)
    mp = torch.zeros_like(p) if min_ps is None else torch.as_tensor(min_ps, dtype=torch.float32).view(-1)
    greedy = bool((k <= 1).any())
    return SimpleNamespace(
        temperatures=t, top_ks=k, top_ps=p, min_ps=mp,
        need_top_k_sampling=bool((k < TOP_K_ALL).any() & ~greedy) if need_top_k is None else need_top_k,
        need_top_p_sampling=bool((p < 1.0).any()) if need_top_p is None else need_top_p,
        need_min_p_sampling=bool((mp > 0).any()) if need_min_p is None else need_min_p,
        is_any_greedy=greedy if is_any_greedy is None else is_any_greedy,
        is_all_greedy=bool((k <= 1).all()),
        max_top_k=int(k.max()),
    )


def request_of_rows(bs, T, verify_lens=None, row_offsets=None, rows=None):
    if row_offsets is None:
        return np.repeat(np.arange(bs), T)
    offs = np.asarray(row_offsets, dtype=np.int64).reshape(-1)
    total = int(rows) if rows is not None else int(offs[-1] + np.asarray(verify_lens)[-1])
    return np.searchsorted(offs, np.arange(total), side="right") - 1


SPARSE_CAPACITY = 32  # packed capacity of the sparse joint target (sampling/target.py:84-87)


def sparse_route(info, sampling_backend, vocab, q_width, capacity=SPARSE_CAPACITY) -> bool:
    """Whether TargetDistribution.sample_prefix verifies against the sparse joint target:
    its sparse-q path needs K = 16 q lanes (sampling/target.py:53-54) and build_sparse_target
    takes only flashinfer batches without min-p or greedy rows whose host-known max top-k lies in
    [1, capacity] and within the vocabulary (sampling/sparse/target.py:106-116)."""
    max_k = getattr(info, "max_top_k", None)
    return (int(q_width) == 16 and sampling_backend == "flashinfer"
            and not getattr(info, "need_min_p_sampling", False)
            and not getattr(info, "is_any_greedy", False)
            and isinstance(max_k, int) and 1 <= max_k <= capacity and 1 <= vocab and max_k <= vocab)


def verify_step(logits, info, *, candidates, q_ids, q_values, verify_lens, uniforms,
                uniform_final, prefix_lens, hist_ids=None, presence=None, repetition=None,
                page_table=None, row_offsets=None, sampling_backend="pytorch", requests=None,
                exact_softmax=False, sparse_joint=False):
    """The fused verify step on the CPU: history penalties -> target P per verified row ->
    sparse-q chain rejection -> compaction + KV slots.  ``logits`` is [rows, V] (bf16/fp32) in
    the dense ``b*T+s`` layout or ragged with ``row_offsets``.  ``requests`` (optional) limits
    the work to a subset of requests (outputs of the others are left zero).

    ``sparse_joint``: the route TargetDistribution.sample_prefix takes for batches that
    build_sparse_target accepts (``sparse_route``; sampling/target.py:58-121): the softmax rows'
    sparse joint target (``sparse_target``, capacity 32) as packed P, its overflow rows dense,
    then accept_sparse on them (packed rows: lanes summed at an id, sampling/sparse/accept.py:
    179-204; dense rows: the last lane).  Otherwise the backend filter of
    build_dspine_target_probs (runtime/worker.py:440-508).

    Returns a dict with accept/commit/bonus/output/new_seq/kv_slots/margins and ``probs``
    (dict row -> float32 target row) for the verified rows that were built."""
    cand = np.asarray(candidates)
    bs, T = cand.shape
    V = logits.shape[-1]
    caps = np.asarray(verify_lens, dtype=np.int64).reshape(-1)
    offs = None if row_offsets is None else np.asarray(row_offsets, dtype=np.int64).reshape(-1)
    reqs = list(range(bs)) if requests is None else list(requests)
    base = [int(offs[b]) if offs is not None else b * T for b in range(bs)]
    rows, owners = [], []
    for b in reqs:
        for s in range(int(caps[b])):
            rows.append(base[b] + s)
            owners.append(b)
    x = logits[torch.as_tensor(rows, dtype=torch.long)].clone()
    owner_t = torch.as_tensor(owners, dtype=torch.long)
    if hist_ids is not None:
        add, scl = penalties_from_history(hist_ids, presence, repetition, V)
        adjust_logits(x, SimpleNamespace(acc_additive_penalties=add, acc_scaling_penalties=scl),
                      owner_t)
    rinfo = row_info(info, owner_t)
    packed = None
    if sparse_joint:
        p = softmax_temp(x, rinfo.temperatures.view(-1), exact=exact_softmax)
        ids, vals, lens, ovf, dense = sparse_target(p, rinfo.top_ks, rinfo.top_ps, SPARSE_CAPACITY)
        P = dense
        # packed P indexed by the logits row, as accept_sparse reads it
        total = int(logits.shape[0])
        g_ids = np.full((total, SPARSE_CAPACITY), -1, np.int32)
        g_vals = np.zeros((total, SPARSE_CAPACITY), np.float32)
        g_lens = np.zeros(total, np.int32)
        g_ovf = np.zeros(total, np.int32)
        idx = np.asarray(rows, dtype=np.int64)
        g_ids[idx], g_vals[idx] = ids.numpy(), vals.numpy()
        g_lens[idx], g_ovf[idx] = lens.numpy(), ovf.numpy()
        packed = (g_ids, g_vals, g_lens, g_ovf)
    else:
        P = build_target_probs(x, rinfo, 1, len(rows), sampling_backend,
                               exact_softmax=exact_softmax).reshape(len(rows), V)
    probs = {r: P[i].numpy() for i, r in enumerate(rows)}
    sub = np.asarray(reqs, dtype=np.int64)
    qi = None if q_ids is None else np.asarray(q_ids)[sub]
    qv = None if q_values is None else np.asarray(q_values)[sub]
    # rows of the subset keep their global index: pass each request's first row explicitly
    sub_base = np.array([base[b] for b in reqs], dtype=np.int64)
    acc = chain_accept(lambda r: probs[r], cand[sub], qi, qv, caps[sub],
                       np.asarray(uniforms)[sub], np.asarray(uniform_final)[sub],
                       np.asarray(prefix_lens)[sub], row_offsets=sub_base, packed=packed)
    accept = np.zeros(bs, np.int32)
    commit = np.zeros(bs, np.int32)
    bonus = np.zeros(bs, np.int64)
    output = np.zeros((bs, T), np.int64)
    new_seq = np.zeros(bs, np.int32)
    margins = np.full(bs, np.inf)
    for j, b in enumerate(reqs):
        accept[b], commit[b], bonus[b] = acc[0][j], acc[1][j], acc[2][j]
        output[b], new_seq[b], margins[b] = acc[3][j], acc[4][j], acc[5][j]
    slots = None
    if page_table is not None:
        slots = np.full((bs, T), -1, np.int32)
        ks = kv_slots(np.asarray(page_table)[sub], np.asarray(prefix_lens)[sub], acc[0], T)
        for j, b in enumerate(reqs):
            slots[b] = ks[j]
    return dict(accept=accept, commit=commit, bonus=bonus, output=output, new_seq=new_seq,
                kv_slots=slots, margins=margins, probs=probs, adjusted=dict(zip(rows, x)), packed=packed)
