import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "needle-rs_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def golden_dir():
    return os.path.join(ROOT, "tests", "golden")


@pytest.fixture(scope="session")
def ctx():
    """nd_ctx on cuda:0 (torch's current stream)."""
    import needle_amd as nd
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = nd.Ctx(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def dev(a):
    import torch
    return torch.from_numpy(__import__("numpy").ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()
