import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


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
    return torch.device("cuda", 0)


def pytest_terminal_summary(terminalreporter):
    """Achieved parity errors of this session (tests/parity.py)."""
    try:
        import parity
    except ImportError:
        return
    recs = parity.RECORDS
    if not recs:
        return
    terminalreporter.write_sep("-", f"parity errors ({len(recs)} checks)")
    worst = {}
    for r in recs:
        w = worst.setdefault(r["test"], dict(r))
        w["max_abs"] = max(w["max_abs"], r["max_abs"])
        w["max_rel"] = max(w["max_rel"], r["max_rel"])
    for t, r in worst.items():
        terminalreporter.write_line(f"{r['max_abs']:.3e} abs {r['max_rel']:.3e} rel  {t}")
    path = os.environ.get("TITAN_PARITY_LOG")
    if path:
        import json
        with open(path, "w") as f:
            for r in recs:
                f.write(json.dumps(r) + "\n")
