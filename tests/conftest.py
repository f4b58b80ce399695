import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


def pytest_terminal_summary(terminalreporter):
    """The near-margin table of every parity comparison of the run (tests/parity.py)."""
    import parity

    if not parity.RECORDS:
        return
    tr = terminalreporter
    tr.section(f"parity vs oracle (near-margin: oracle margin < {parity.MARGIN:g}; literal fp32 softmax rows: "
               f"< {parity.LITERAL_MARGIN:g})")
    total = [0, 0, 0]
    for tag, compared, near, differing in parity.RECORDS:
        tr.write_line(f"{tag}: compared {compared}, near-margin {near}, differing {len(differing)} "
                      f"{parity._fmt(differing)}")
        total[0] += compared
        total[1] += near
        total[2] += len(differing)
    tr.write_line(f"TOTAL: compared {total[0]}, near-margin {total[1]}, differing {total[2]}")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("GPU required")
    from dspine_amd import _lib

    _lib.load()  # the product path must load the native library, never fall back
    return torch.device("cuda:0")
