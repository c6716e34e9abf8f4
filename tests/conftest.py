import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "ssd-llm_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (runs the HIP kernels through the C ABI)")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if any(item.get_closest_marker("gpu") for item in items) and not _gpu_available():
        skip = pytest.mark.skip(reason="no GPU visible to torch")
        for item in items:
            if item.get_closest_marker("gpu"):
                item.add_marker(skip)


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Prints how many outputs each tolerance check took against the exact sum
    instead of the reference's serial fp32 value (helpers.assert_close_attributed)."""
    try:
        from helpers import SUBSTITUTIONS
    except ImportError:
        return
    if not SUBSTITUTIONS:
        return
    tr = terminalreporter
    tr.section("exact-sum substitutions (outputs outside tolerance of the fp32 reference, where the "
               "reference's own chain is more than half a tolerance from the exact sum)")
    total = sum(s[2] for s in SUBSTITUTIONS)
    outputs = sum(s[3] for s in SUBSTITUTIONS)
    worst = max(s[4] for s in SUBSTITUTIONS)
    for test, what, n, m, w in SUBSTITUTIONS:
        if n:
            tr.write_line(f"{n:6d} of {m:9d}  worst |gpu-exact|/tol {w:.3f}  {test} [{what}]")
    tr.write_line(f"total: {total} of {outputs} outputs in {len(SUBSTITUTIONS)} checks "
                  f"({sum(1 for s in SUBSTITUTIONS if s[2])} checks used any); worst substituted "
                  f"|gpu - exact| / tol(exact): {worst:.3f}")
