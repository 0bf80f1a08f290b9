import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "tests")):   # the package, and test modules sharing helpers
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


@pytest.fixture(scope="session")
def torch_cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a visible GPU")
    return torch


@pytest.fixture(scope="session")
def hip_ctx(torch_cuda):
    from air_amd import capi

    stream = torch_cuda.cuda.current_stream(torch_cuda.device("cuda:0")).cuda_stream
    ctx = capi.Context(0, stream)
    yield ctx
    ctx.close()
