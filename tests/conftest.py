import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "selective-attention-study_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm GPU) and the built HIP library")


def gpu_ready() -> bool:
    import torch

    from selective_attention import kernels

    return torch.cuda.is_available() and kernels.HAS_HIP


@pytest.fixture
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a GPU")
    from selective_attention import kernels

    if not kernels.HAS_HIP:
        pytest.fail("libsa_hip.so did not load on a GPU box")
    return torch.device("cuda:0")
