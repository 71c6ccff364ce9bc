import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "wam-egale_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def pytest_terminal_summary(terminalreporter):
    """Parity margins of the session: each assert_close with its max-abs and
    the share of the bound it uses (printed on success too)."""
    try:
        from oracle.metrics import RECORD
    except Exception:
        return
    if not RECORD:
        return
    tr = terminalreporter
    tr.write_sep("-", f"parity margins ({len(RECORD)} comparisons)")
    for what, got, bound, cos, cos_bound in RECORD:
        share = got / bound if bound > 0 else float("nan")
        tr.write_line(f"{what[:60]:<60} max_abs {got:.4g} / {bound:g} ({share:6.1%})  "
                      f"cos {cos:.7f} (>= {cos_bound})")
