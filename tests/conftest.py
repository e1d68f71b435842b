"""Shared test configuration: the `gpu` marker, import paths, seeded inputs."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # noqa: BLE001
        return False


@pytest.fixture
def dev():
    if not gpu_available():
        pytest.skip("no GPU in this environment")
    import torch
    return torch.device("cuda", 0)


# figures a GPU test measures (step times, ratios), printed in the run's
# terminal summary so that they survive a quiet (-q) run's output
_METRICS: dict = {}


@pytest.fixture
def metrics():
    return _METRICS


def pytest_terminal_summary(terminalreporter):
    if _METRICS:
        terminalreporter.write_sep("-", "t2t measured figures")
        for k in sorted(_METRICS):
            terminalreporter.write_line(f"{k} = {_METRICS[k]}")
