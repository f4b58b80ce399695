"""Seeded synthetic verification workloads (no datasets or checkpoints are involved).

Five shapes, each generated on the CPU from fixed seeds so that the device path and any CPU
checker see identical logits, drafts and coins:

* ``greedy_round``     1 x 17 rows x 151936 fp32, temperature 0: drafts are the target argmax
                       with one seeded mismatch.
* ``topk_rows``        [64*17, 151936] bf16 N(0, 2^2) with 32 planted peaks at +8..+14 and ~1%
                       exact duplicates (ties straddling the k-th place).
* ``rejection_round``  32 x 17 x 151936 fp32, T=1, top-k 20, top-p 0.95; draft logits = target +
                       N(0, sigma^2); q is the draft's filtered softmax, drafts sampled from q.
* ``serving_round``    64 x 17 x 151936 bf16; per-request temperature {0, 0.6, 1.0}, top-k {off,
                       20}, top-p {1.0, 0.95}; presence/repetition penalties over a 512-token
                       history; sparse q [64, 16, 16]; int32 page table.
* ``ragged_round``     32 requests x verify lengths U{4..16} x 262144 bf16, heavy-tailed logits
                       (2 * Student-t, nu=3), T=1, top-p 0.9, compact rows with row offsets.

Uniforms come from NumPy's Philox generator, as float32.
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import torch

TOP_K_ALL = 1 << 30


def sampling_info(temperatures, top_ks, top_ps, min_ps=None):
    """A duck-typed SGLang SamplingBatchInfo: temperature 0 means greedy (top_k 1, T 1), top_k 0
    means no top-k (2^30), and the batch flags follow SGLang's definitions."""
    t = torch.as_tensor(temperatures, dtype=torch.float32).view(-1).clone()
    k = torch.as_tensor(top_ks, dtype=torch.int64).view(-1).clone()
    greedy = t <= 0
    k = torch.where(k <= 0, torch.full_like(k, TOP_K_ALL), k)
    k = torch.where(greedy, torch.ones_like(k), k).to(torch.int32)
    t = torch.where(greedy, torch.ones_like(t), t)
    p = torch.as_tensor(top_ps, dtype=torch.float32).view(-1).clone()
    mp = torch.zeros_like(p) if min_ps is None else torch.as_tensor(min_ps, dtype=torch.float32).view(-1)
    return SimpleNamespace(
        temperatures=t.view(-1, 1), top_ks=k, top_ps=p, min_ps=mp,
        need_top_k_sampling=bool(((k > 1) & (k < TOP_K_ALL)).any()),
        need_top_p_sampling=bool((p < 1.0).any()),
        need_min_p_sampling=bool((mp > 0).any()),
        is_any_greedy=bool((k <= 1).any()),
        is_all_greedy=bool((k <= 1).all()),
        max_top_k=int(k.max()),
    )


def info_to(info, device):
    out = SimpleNamespace(**vars(info))
    for name in ("temperatures", "top_ks", "top_ps", "min_ps"):
        setattr(out, name, getattr(info, name).to(device))
    return out


def to_device(batch: dict, device) -> dict:
    out = {}
    for key, v in batch.items():
        if isinstance(v, torch.Tensor):
            out[key] = v.to(device)
        elif key == "info":
            out[key] = info_to(v, device)
        else:
            out[key] = v
    return out


def philox_uniforms(seed: int, *shape) -> torch.Tensor:
    rng = np.random.Generator(np.random.Philox(seed))
    return torch.from_numpy(rng.random(shape, dtype=np.float32))


def _filtered_q(draft_logits: torch.Tensor, temperature: float, top_k: int, top_p: float):
    """q over the top-k draft tokens: temperature softmax, keep ranks whose preceding mass
    <= top_p, renormalise.  Returns (ids sorted ascending [n, k], q [n, k])."""
    p = torch.softmax(draft_logits.float() / temperature, -1)
    vals, ids = torch.topk(p, top_k, dim=-1)
    ahead = torch.cumsum(vals.double(), -1) - vals.double()
    vals = torch.where(ahead <= top_p, vals, torch.zeros_like(vals))
    vals = vals / vals.sum(-1, keepdim=True)
    order = ids.argsort(-1)
    return ids.gather(-1, order), vals.gather(-1, order).float()


def _sample_lanes(q: torch.Tensor, gen: torch.Generator) -> torch.Tensor:
    return torch.multinomial(q, 1, generator=gen).view(-1)


def greedy_round(V=151936, T=17, seed=1, sigma=3.0):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, V, generator=g) * sigma
    top1 = logits.argmax(-1)
    cand = torch.zeros(1, T, dtype=torch.int64)
    cand[0, 1:] = top1[: T - 1]
    pos = int(torch.randint(0, T - 1, (1,), generator=g))
    repl = int(torch.randint(0, V, (1,), generator=g))
    if repl == int(top1[pos]):
        repl = (repl + 1) % V
    cand[0, pos + 1] = repl
    return dict(logits=logits, candidates=cand, prefix_lens=torch.tensor([1000], dtype=torch.int32),
                mismatch=pos)


def topk_rows(rows=64 * 17, V=151936, seed=2, sigma=2.0, peaks=32, dup_frac=0.01, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, V, generator=g) * sigma
    idx = torch.stack([torch.randperm(V, generator=g)[:peaks] for _ in range(rows)])
    x.scatter_(1, idx, 8.0 + 6.0 * torch.rand(rows, peaks, generator=g))
    x = x.to(dtype)
    ndup = int(V * dup_frac)
    src = torch.randint(0, V, (rows, ndup), generator=g)
    # a quarter of the copies duplicate planted peaks so ties straddle the k-th place
    src[:, : ndup // 4] = idx[:, torch.randint(0, peaks, (ndup // 4,), generator=g)]
    dst = torch.randint(0, V, (rows, ndup), generator=g)
    x.scatter_(1, dst, x.gather(1, src))
    return dict(logits=x)


def rejection_round(bs=32, T=17, V=151936, sigma_draft=0.5, seed=3, top_k=20, top_p=0.95):
    g = torch.Generator().manual_seed(seed)
    target = torch.randn(bs * T, V, generator=g) * 2.5
    draft = target.view(bs, T, V)[:, : T - 1] + torch.randn(bs, T - 1, V, generator=g) * sigma_draft
    q_ids, q = _filtered_q(draft.reshape(-1, V), 1.0, top_k, top_p)
    lanes = _sample_lanes(q, g)
    drafts = q_ids.gather(1, lanes[:, None]).view(bs, T - 1)
    cand = torch.cat((torch.zeros(bs, 1, dtype=torch.int64), drafts), 1)
    u = philox_uniforms(seed, bs, T)
    return dict(
        logits=target, info=sampling_info([1.0] * bs, [top_k] * bs, [top_p] * bs),
        candidates=cand, q_ids=q_ids.view(bs, T - 1, top_k), q_values=q.view(bs, T - 1, top_k),
        uniforms=u[:, : T - 1].contiguous(), uniform_final=u[:, T - 1].contiguous(),
        prefix_lens=torch.full((bs,), 512, dtype=torch.int32),
    )


def serving_round(bs=64, T=17, V=151936, seed=4, K=16, hist_len=512, dtype=torch.bfloat16, sigma=2.5,
                  presence=0.5, repetition=1.1, peak=None):
    """``peak``: one planted logit per row at U[peak - 1, peak + 1] (a likely next token that the
    draft's noisy top-K also ranks first), which raises the drafts' acceptance."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(bs * T, V, generator=g) * sigma
    if peak is not None:
        at = torch.randint(0, V, (bs * T,), generator=g)
        x[torch.arange(bs * T), at] = peak - 1.0 + 2.0 * torch.rand(bs * T, generator=g)
    logits = x.to(dtype)
    temps = torch.tensor([0.0, 0.6, 1.0])[torch.randint(0, 3, (bs,), generator=g)]
    ks = torch.tensor([0, 20])[torch.randint(0, 2, (bs,), generator=g)]
    ps = torch.tensor([1.0, 0.95])[torch.randint(0, 2, (bs,), generator=g)]
    info = sampling_info(temps, ks, ps)
    hist = torch.randint(0, V, (bs, hist_len), generator=g, dtype=torch.int64).to(torch.int32)
    pres = torch.full((bs,), presence)
    rep = torch.full((bs,), repetition)
    # draft q: top-K of noisy target rows, softmax over those lanes; drafts sampled from q
    noisy = logits.view(bs, T, V)[:, : T - 1].float() + torch.randn(bs, T - 1, V, generator=g)
    vals, ids = torch.topk(noisy.reshape(-1, V), K, dim=-1)
    order = ids.argsort(-1)
    q_ids = ids.gather(-1, order)
    q = torch.softmax(vals.gather(-1, order), -1)
    lanes = _sample_lanes(q, g)
    drafts = q_ids.gather(1, lanes[:, None]).view(bs, T - 1)
    cand = torch.cat((torch.randint(0, V, (bs, 1), generator=g), drafts), 1)
    u = philox_uniforms(seed, bs, T)
    prefix = torch.randint(64, 4096, (bs,), generator=g, dtype=torch.int64).to(torch.int32)
    L = 4096 + T + 64
    page = torch.stack([torch.randperm(1 << 20, generator=g)[:L] for _ in range(bs)]).to(torch.int32)
    return dict(
        logits=logits, info=info, candidates=cand, q_ids=q_ids.view(bs, T - 1, K),
        q_values=q.view(bs, T - 1, K).float(), uniforms=u[:, : T - 1].contiguous(),
        uniform_final=u[:, T - 1].contiguous(), prefix_lens=prefix, hist_ids=hist,
        presence=pres, repetition=rep, page_table=page,
    )


def sparse_round(bs=24, T=16, V=151936, seed=6, K=16, hist_len=64, dtype=torch.bfloat16, sigma=2.5,
                 coarse_every=4):
    """A batch that the reference verifies against its sparse joint target (flashinfer backend,
    no min-p, no greedy rows, top-k <= 32): temperature {0.6, 1.0}, top-k {8, 20, 32}, top-p
    {1.0, 0.95, 0.6}, bf16 logits N(0, sigma^2) -- at top-k 20 most rows tie at the k-th value
    -- and every ``coarse_every``-th request with integer-valued logits N(0, 1) rounded, whose
    rows hold hundreds of ties at the k-th value (more than 32 kept: dense rows).  Presence /
    repetition penalties over a short history; sparse q [bs, T-1, K] from noisy target rows."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(bs * T, V, generator=g) * sigma
    for b in range(0, bs, max(1, coarse_every)):
        x[b * T:(b + 1) * T] = torch.round(torch.randn(T, V, generator=g))
    logits = x.to(dtype)
    temps = torch.tensor([0.6, 1.0])[torch.randint(0, 2, (bs,), generator=g)]
    ks = torch.tensor([8, 20, 32])[torch.randint(0, 3, (bs,), generator=g)]
    ps = torch.tensor([1.0, 0.95, 0.6])[torch.randint(0, 3, (bs,), generator=g)]
    info = sampling_info(temps, ks, ps)
    hist = torch.randint(0, V, (bs, hist_len), generator=g, dtype=torch.int64).to(torch.int32)
    noisy = logits.view(bs, T, V)[:, : T - 1].float() + 0.5 * torch.randn(bs, T - 1, V, generator=g)
    vals, ids = torch.topk(noisy.reshape(-1, V), K, dim=-1)
    order = ids.argsort(-1)
    q_ids = ids.gather(-1, order)
    q = torch.softmax(vals.gather(-1, order), -1)
    lanes = _sample_lanes(q, g)
    drafts = q_ids.gather(1, lanes[:, None]).view(bs, T - 1)
    cand = torch.cat((torch.randint(0, V, (bs, 1), generator=g), drafts), 1)
    u = philox_uniforms(seed, bs, T)
    return dict(
        logits=logits, info=info, candidates=cand, q_ids=q_ids.view(bs, T - 1, K),
        q_values=q.view(bs, T - 1, K).float(), uniforms=u[:, : T - 1].contiguous(),
        uniform_final=u[:, T - 1].contiguous(), prefix_lens=torch.full((bs,), 300, dtype=torch.int32),
        hist_ids=hist, presence=torch.full((bs,), 0.5), repetition=torch.full((bs,), 1.1),
    )


def ragged_round(bs=32, T=17, V=262144, seed=5, K=16, top_p=0.9, lo=4, hi=16):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (bs,), generator=g, dtype=torch.int64)
    rows = int(lens.sum())
    offsets = torch.cat((torch.zeros(1, dtype=torch.int64), lens.cumsum(0)))[:-1]
    tdist = torch.distributions.StudentT(3.0)
    torch.manual_seed(seed)
    logits = (2.0 * tdist.sample((rows, V))).to(torch.bfloat16)
    info = sampling_info([1.0] * bs, [0] * bs, [top_p] * bs)
    q_ids = torch.zeros(bs, T - 1, K, dtype=torch.int64)
    q = torch.zeros(bs, T - 1, K)
    for b in range(bs):
        r0, n = int(offsets[b]), int(lens[b])
        rowsel = logits[r0: r0 + n].float()
        noisy = rowsel[torch.clamp(torch.arange(T - 1), max=n - 1)] + torch.randn(T - 1, V, generator=g)
        vals, ids = torch.topk(noisy, K, dim=-1)
        order = ids.argsort(-1)
        q_ids[b] = ids.gather(-1, order)
        q[b] = torch.softmax(vals.gather(-1, order), -1)
    lanes = _sample_lanes(q.view(-1, K), g)
    drafts = q_ids.view(-1, K).gather(1, lanes[:, None]).view(bs, T - 1)
    cand = torch.cat((torch.zeros(bs, 1, dtype=torch.int64), drafts), 1)
    u = philox_uniforms(seed, bs, T)
    return dict(
        logits=logits, info=info, candidates=cand, q_ids=q_ids, q_values=q.float(),
        uniforms=u[:, : T - 1].contiguous(), uniform_final=u[:, T - 1].contiguous(),
        prefix_lens=torch.full((bs,), 2048, dtype=torch.int32), verify_lens=lens.to(torch.int32),
        row_offsets=offsets,
    )
