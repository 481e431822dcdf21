import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import w4_oracle

    w4_oracle.lib()  # builds libw4oracle.so with gcc on first use if it is missing
    return w4_oracle


@pytest.fixture(scope="session")
def kernels():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from nanoserve_amd import Kernels

    return Kernels()


def to_dev(a: np.ndarray, dtype):
    """numpy bit patterns -> GPU torch tensor of `dtype` with the same bytes."""
    import torch

    a = np.ascontiguousarray(a)
    view = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32}.get(a.dtype, a.dtype)
    t = torch.from_numpy(a.view(view).copy())
    return t.view(dtype).cuda()


def to_host_bits(t) -> np.ndarray:
    """GPU bf16 / int32 tensor -> numpy uint16 / uint32 bit patterns."""
    import torch

    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.int32:
        return t.numpy().view(np.uint32)
    raise TypeError(t.dtype)
