import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libsimp_hip.so)")


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with libsimp_hip.so bound to torch's current stream."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import simplang_amd as sa
    torch.cuda.set_device(0)
    sa.set_stream(torch.cuda.current_stream())
    return torch.device("cuda:0")
