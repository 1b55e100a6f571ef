"""Shared test helpers. `-m gpu` tests need an MI355X; everything else runs on the CPU."""
import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950) and the built libpqint8.so")


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw uint16 bit patterns of a bf16/fp16 tensor (on any device)."""
    assert t.dtype in (torch.bfloat16, torch.float16)
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def dcode(dt: torch.dtype) -> int:
    return 0 if dt == torch.bfloat16 else 1


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    O.lib()
    return O


@pytest.fixture(scope="session")
def cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import pyraquant_amd._lib as L

    L.load()   # fail loudly if the HIP library is missing
    return torch.device("cuda:0")


# Tolerance of the floating-point outputs (the build's parity bar): against the oracle's fp32 result r computed
# from the same int8 codes, max relative error max|y - r| / max|r| <= 1e-2 and mean relative error
# sum|y - r| / sum|r| <= 5e-3. (An element-wise ratio is undefined where r crosses zero.)
MAX_REL, MEAN_REL = 1e-2, 5e-3


def rel_errors(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    return float(err.max() / np.abs(ref).max()), float(err.sum() / np.abs(ref).sum())
