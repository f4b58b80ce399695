"""CPU oracle for the DSpine draft-verification path (TEST INFRASTRUCTURE ONLY).

This package restates, on the CPU with torch/numpy, the semantics of the reference's
verification path so that the HIP kernels can be checked against it.  It is the checker,
never the thing measured or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product package ``dspine_amd``
must never import anything from here, and it fails loudly when its HIP library is missing.

Pinning status of each function is recorded in ``verify_oracle.PINNED``.
"""

from oracle.verify_oracle import *  # noqa: F401,F403
