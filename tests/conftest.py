"""Test configuration: import paths, the `gpu` marker, shared helpers."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "dllm-qwen38_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no ROCm device is visible")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _kernel_status_clean(request):
    """After every GPU test: no bounded wait inside a kernel gave up (a set status bit means some
    launch of the test produced invalid outputs, whatever the test compared)."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    import torch

    if not torch.cuda.is_available():
        return
    from dllm_qwen38_amd import gdn

    st = gdn.kernel_status(reset=True)
    assert st == 0, f"a bounded wait inside a HIP kernel gave up during this test (status bits {st:#x})"
