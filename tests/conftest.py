import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "rapid-h3_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through librh3)")


@pytest.fixture(scope="session")
def dev():
    """cuda:0 for GPU tests. Skips only when no GPU is visible; with a GPU, a missing librh3 fails."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from rapid_h3 import _native
    _native.lib()
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def golden():
    def load(name):
        with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as f:
            return {k: f[k] for k in f.files}
    return load


def to_dev(a, device, dtype=None):
    """numpy (bf16 bits as uint16, e4m3 bits as uint8 when dtype says so) -> device tensor."""
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(device).view(torch.bfloat16)
    if dtype == "fp8":
        return torch.from_numpy(a).to(device).view(torch.float8_e4m3fn)
    return torch.from_numpy(a).to(device)


def to_np(t):
    """device tensor -> numpy (bf16 as uint16 bits, fp8 as uint8 bits)."""
    import torch
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()
