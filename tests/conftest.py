import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "pocket-engine_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def pytest_terminal_summary(terminalreporter):
    """Prints the figures of every oracle comparison of the run
    (tests/_util.close), so the parity evidence is in the log."""
    try:
        from _util import ATOL, EXPLAIN_LOG, PARITY_LOG, RTOL
    except ImportError:
        return
    if not PARITY_LOG:
        return
    tr = terminalreporter
    tr.write_sep("-", f"attention parity (bound |d| <= {ATOL} + {RTOL} |want|; rel over |want| > {ATOL})")
    for test, what, n, mabs, mrel, mulp, neither in PARITY_LOG:
        tr.write_line(f"{test} {what}: n={n} max_abs={mabs:.3e} max_rel={mrel:.3e} max_ulp={mulp:.0f} "
                      f"beyond_both_alone={neither}")
    tr.write_line(f"{len(PARITY_LOG)} comparisons, {sum(r[2] for r in PARITY_LOG)} elements; worst max_abs "
                  f"{max(r[3] for r in PARITY_LOG):.3e}, worst max_rel {max(r[4] for r in PARITY_LOG):.3e}, worst "
                  f"{max(r[5] for r in PARITY_LOG):.0f} ulp, {sum(r[6] for r in PARITY_LOG)} elements beyond both "
                  f"bounds alone")
    for test, line in EXPLAIN_LOG:
        tr.write_line(f"{test} {line}")
