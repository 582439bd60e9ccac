import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "veystrix-core_amd")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a visible GPU")
    from veymoe import _lib

    if not _lib.lib().vm_available():
        pytest.fail(f"libveymoe cannot use this device: {_lib.last_error()}")
    print(f"[gpu] {torch.cuda.get_device_name(0)}", flush=True)
    return torch.device("cuda:0")
