import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libpe_attn.so")


def gpu_ready() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("a GPU test was selected but no GPU is visible")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _seed_global_rng(request):
    """Seed torch's global generator from the test's own id, so a test that draws from it (rather
    than from a seeded generator) gets the same inputs alone, in its file or in the whole suite."""
    import zlib

    import torch
    torch.manual_seed(zlib.crc32(request.node.nodeid.encode()))
