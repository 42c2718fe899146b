"""Shared fixtures.  GPU tests are marked ``gpu`` and need a built extension."""

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from rnn_with_grm_amd import cuda_ops

    assert cuda_ops.load_grm_cuda_extension(), cuda_ops.extension_load_error()
    return torch.device("cuda:0")
