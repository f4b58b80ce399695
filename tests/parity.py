"""Shared parity bookkeeping of the GPU tests.

Integer outputs of the HIP path must equal the oracle's.  A decision of the reference (an
accept test ``u*q < p``, a top-p test, a bonus CDF step) can only come out differently when
the two sides' probabilities differ by more than the decision's own relative margin, so a
request may differ only when the oracle reports a margin below MARGIN for it.

MARGIN is derived from the measured probability error: the dense target P of the HIP path is
within ~1.5e-6 relative of the float64 softmax on the serving rows (asserted below a quarter of
MARGIN by ``test_target_p_error_bounds_margin``), so the comparisons use the oracle with its
exact softmax (float64, rounded once).  CPU torch's float32 softmax is up to ~3e-5 off on those
151936-wide rows, too far from either to carry a bit-exact claim at this MARGIN.

Every comparison records (requests compared, requests whose oracle margin is below MARGIN,
requests that differ); ``conftest.py`` prints the table at the end of the run.
"""

from __future__ import annotations

import numpy as np

MARGIN = 2e-5

RECORDS: list[tuple[str, int, int, list]] = []


def record(tag: str, compared: int, near: int, differing: list) -> None:
    RECORDS.append((tag, int(compared), int(near), list(differing)))
    print(f"[parity] {tag}: compared {compared}, near-margin {near}, differing {len(differing)} {differing}",
          flush=True)


def compare_requests(gpu: dict, ref: dict, requests, tag: str, names=("accept", "bonus", "output", "new_seq"),
                     extra=("kv_slots",)) -> list:
    """gpu / ref: dicts of numpy arrays indexed by request.  Asserts that every differing
    request has an oracle margin below MARGIN, records the counts and returns the differing
    requests."""
    differing, near = [], 0
    requests = list(requests)
    for b in requests:
        m = float(ref["margins"][b])
        near += m < MARGIN
        same = all(np.array_equal(np.asarray(gpu[n][b]), np.asarray(ref[n][b])) for n in names)
        for n in extra:
            if same and ref.get(n) is not None and gpu.get(n) is not None:
                same = np.array_equal(gpu[n][b], ref[n][b])
        if not same:
            assert m < MARGIN, (tag, b, {k: gpu[k][b] for k in names}, {k: ref[k][b] for k in names}, m)
            differing.append(b)
    record(tag, len(requests), near, differing)
    return differing
