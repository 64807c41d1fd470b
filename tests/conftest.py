"""Shared fixtures.  GPU tests are marked `gpu` and run on an MI355X; the
rest run on the CPU (oracle, host logic, library loading)."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.build()
    return O


@pytest.fixture(scope="session")
def talos():
    import talos_amd
    talos_amd.lib()  # fails loudly if the library was not built
    return talos_amd


def record_parity(case: str, worst: float, tol: float, **extra) -> None:
    """Append one parity margin (worst max-abs difference against the
    oracle, and the bar it was held to) to the JSON-lines file named by
    TALOS_PARITY_LOG, when that is set."""
    import json
    path = os.environ.get("TALOS_PARITY_LOG")
    if not path:
        return
    rec = {"case": case, "worst_max_abs": float(worst), "tol": float(tol), **extra}
    with open(path, "a") as f:
        f.write(json.dumps(rec) + "\n")
