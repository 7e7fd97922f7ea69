import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: longer CPU test")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter):
    """The parity margins the tests recorded (checks.margin): the worst error
    per configuration against its bound."""
    try:
        from checks import MARGINS
    except ImportError:
        return
    if not MARGINS:
        return
    tr = terminalreporter
    tr.section("parity margins (worst per config)")
    for (config, measure), (err, bound) in sorted(MARGINS.items()):
        frac = err / bound if bound else float("nan")
        tr.write_line(f"{config:<58} {measure:<34} {err:.3e}  bound {bound:g}  ({100 * frac:5.1f}% of bound)")
