"""Shared parity bookkeeping of the GPU tests.

Integer outputs of the HIP path must equal the oracle's.  A decision of the reference (an
accept test ``u*q < p``, a top-p test, a bonus CDF step) can only come out differently when
the two sides' probabilities differ by more than the decision's own relative margin, so a
request may differ only when the oracle reports a margin below MARGIN for it.

MARGIN is derived from the measured probability error: the dense target P of the HIP path is
within ~1.5e-6 relative of the float64 softmax on the serving rows (asserted below half of
MARGIN by ``test_target_p_error_bounds_margin``), so the comparisons use the oracle with its
exact softmax (float64, rounded once) and MARGIN = 4e-6, about 2.5 times that error.

The oracle's literal path -- CPU torch's float32 softmax, the reference's own CPU branch
(sampling/sparse/target.py:133) -- is itself up to ~3e-5 off on 151936-wide rows (asserted below
LITERAL_MARGIN by the same test) and can move a top-p cut inside a bf16 tie group.  Comparisons
with it record their differences; a request may differ from it only where it is decided as the
exact oracle decides it or where the literal margin is below LITERAL_MARGIN.

Every comparison records (requests compared, requests whose oracle margin is below the bound,
the differing requests with their margins); ``conftest.py`` prints the table at the end of the
run.
"""

from __future__ import annotations

import numpy as np

MARGIN = 4e-6
LITERAL_MARGIN = 1e-4

RECORDS: list[tuple[str, int, int, list]] = []


def _fmt(differing) -> str:
    return "[" + ", ".join(f"{b} (margin {m:.2g})" for b, m in differing) + "]"


def record(tag: str, compared: int, near: int, differing: list) -> None:
    """differing: (request, oracle margin) pairs."""
    RECORDS.append((tag, int(compared), int(near), list(differing)))
    print(f"[parity] {tag}: compared {compared}, near-margin {near}, differing {len(differing)} {_fmt(differing)}",
          flush=True)


def _same(gpu, ref, b, names, extra) -> bool:
    same = all(np.array_equal(np.asarray(gpu[n][b]), np.asarray(ref[n][b])) for n in names)
    for n in extra:
        if same and ref.get(n) is not None and gpu.get(n) is not None:
            same = np.array_equal(gpu[n][b], ref[n][b])
    return same


def compare_requests(gpu: dict, ref: dict, requests, tag: str, names=("accept", "bonus", "output", "new_seq"),
                     extra=("kv_slots",)) -> list:
    """gpu / ref: dicts of numpy arrays indexed by request; ref from the oracle with its exact
    softmax.  Asserts that every differing request has an oracle margin below MARGIN, records
    the counts and returns the differing requests."""
    differing, near = [], 0
    requests = list(requests)
    for b in requests:
        m = float(ref["margins"][b])
        near += m < MARGIN
        if not _same(gpu, ref, b, names, extra):
            assert m < MARGIN, (tag, b, {k: gpu[k][b] for k in names}, {k: ref[k][b] for k in names}, m)
            differing.append((b, m))
    record(tag, len(requests), near, differing)
    return [b for b, _ in differing]


def compare_literal(gpu: dict, literal: dict, exact: dict, requests, tag: str,
                    names=("accept", "bonus", "output", "new_seq")) -> list:
    """The same outputs against the oracle's literal float32 softmax: a request may differ from it
    only where the exact oracle decides it as the HIP path does (the literal softmax's own error
    moved the decision) or where the literal margin is below LITERAL_MARGIN.  Records the counts
    (near: literal margin below LITERAL_MARGIN) and returns the differing requests."""
    differing, near = [], 0
    requests = list(requests)
    for b in requests:
        m = float(literal["margins"][b])
        near += m < LITERAL_MARGIN
        if not _same(gpu, literal, b, names, ()):
            assert m < LITERAL_MARGIN or _same(gpu, exact, b, names, ()), (tag, b, m)
            differing.append((b, m))
    record(tag + " (literal fp32 softmax)", len(requests), near, differing)
    return [b for b, _ in differing]
