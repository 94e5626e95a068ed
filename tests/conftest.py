import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    return torch.device("cuda:0")


@pytest.fixture(scope="session", autouse=True)
def _oracle_threads():
    """The oracle's OpenMP loops use the host cores (at most 16, the GPU
    box's CPU share) so full-size parity checks stay quick."""
    from oracle import oracle
    oracle.set_threads(min(16, os.cpu_count() or 1))
    yield


@pytest.fixture
def tune():
    """set(name, value) for the library's plan / cache-mode overrides
    (TFMA_SetTuningOverride); every override set is restored at teardown."""
    import tensorflow_musa_extension_amd as tfma
    touched = set()

    def set_(name, value):
        touched.add(name)
        tfma.raw_ops.set_tuning_override(name, value)

    yield set_
    for name in touched:
        tfma.raw_ops.set_tuning_override(name, None)
