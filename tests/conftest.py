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
# sum|y - r| / sum|r| <= 5e-3.
MAX_REL, MEAN_REL = 1e-2, 5e-3


def rel_errors(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    return float(err.max() / np.abs(ref).max()), float(err.sum() / np.abs(ref).sum())


# Element-wise bar, beside the normwise one: every output element y of a low-rank layer satisfies
#   |y - r| <= 1e-2 |r| + 2^-7 (|t| @ |L2|) + 2^-16 max|r|
# * 1e-2 |r|: the element's own relative tolerance (the 16-bit output rounding is 2^-9 |r| for bf16);
# * 2^-7 (|t| @ |L2|): t = x @ L1 is rounded to 16 bits by both sides from fp32 sums taken in different orders
#   (the reference's library GEMM fixes none), so a t element may land one 16-bit step (<= 2^-7 |t|) apart; the
#   low-rank product carries that into the row's outputs through |L2|;
# * 2^-16 max|r|: fp32 accumulation-order noise of the epilogue's low-rank product.
# Without a low-rank branch the outputs are compared bit for bit instead.
ELEM_REL, T_STEP, ACC_FLOOR = 1e-2, 2.0 ** -7, 2.0 ** -16


def elem_violation(got, ref, t=None, l2=None, extra=None):
    """Largest ratio |y - r| / bound over the elements (<= 1 passes). t [M, R] and l2 [R, N] as float arrays (the
    oracle's low-rank operands), or None without a low-rank branch; `extra`, an array added to the bound for a
    rounding the result carries beyond one layer's (a sum of two rounded layer outputs)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    bound = ELEM_REL * np.abs(ref) + ACC_FLOOR * np.abs(ref).max()
    if t is not None:
        bound = bound + T_STEP * (np.abs(np.asarray(t, np.float64)) @ np.abs(np.asarray(l2, np.float64)))
    if extra is not None:
        bound = bound + np.asarray(extra, np.float64)
    return float((np.abs(got - ref) / bound).max())
