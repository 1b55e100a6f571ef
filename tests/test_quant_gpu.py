"""GPU parity of the per-token quantizer (pq_quant_rows) against the CPU oracle: bit-exact int8 codes and
fp32 scales (deploy/int8_exec.py:508-509 semantics), incl. the routed row gather, row-slice views, the
per-element kernel, all-zero rows, exact ties and the full c1 / c2a shapes."""
import numpy as np
import pytest
import torch

from conftest import bits, dcode

pytestmark = pytest.mark.gpu


def _check(oracle, x, row_idx=None, q=None, s=None):
    from pyraquant_amd import int8_exec as E

    if q is None:
        q, s = E.quant_rows(x, row_idx)
    torch.cuda.synchronize()
    xb = bits(x.cpu() if x.stride(1) == 1 else x.contiguous())
    ri = None if row_idx is None else row_idx.cpu().numpy()
    qo, so = oracle.quant_rows(xb, dcode(x.dtype), ri)
    qg, sg = q.cpu().numpy(), s.cpu().numpy()
    assert qg.shape == qo.shape and sg.shape == so.shape
    mism = int((qg != qo).sum())
    assert mism == 0, f"{mism} code mismatches of {qo.size}"
    assert np.array_equal(sg.view(np.uint32), so.view(np.uint32)), "scales differ"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K", [(1, 3072), (7, 1280), (64, 640), (300, 3072), (33, 12288), (17, 15360),
                                 (5, 2048), (9, 2560), (3, 8), (2, 16384)])
def test_quant_rows_shapes(oracle, cuda, dtype, M, K):
    from pyraquant_amd.workloads import make_x

    x = make_x(M, K, dtype, seed=M * 7 + K).to(cuda)
    _check(oracle, x)


@pytest.mark.parametrize("K", [1, 5, 100, 1000, 3000])
def test_quant_rows_scalar_kernel(oracle, cuda, K):
    """K % 8 != 0 takes the per-element kernel."""
    from pyraquant_amd.workloads import make_x

    x = make_x(37, K, torch.bfloat16, seed=K).to(cuda)
    _check(oracle, x)


def test_quant_rows_unaligned_view(oracle, cuda):
    """A row-slice view (ldx > K, odd column offset) runs without a copy on the per-element kernel and a
    16-byte aligned view on the vector kernel."""
    from pyraquant_amd.workloads import make_x

    base = make_x(100, 3072 + 15360, torch.bfloat16, seed=5).to(cuda)
    _check(oracle, base[:, 3072:])          # aligned offset (3072 * 2 bytes), ldx = 18432
    _check(oracle, base[:, 1:3073])         # unaligned offset -> per-element kernel


def test_quant_rows_edge_values(oracle, cuda):
    """All-zero rows (scale 1e-8/127), tiny rows, exact ties (x = (k + 1/2) s), +-0, subnormals, a row
    whose absmax is negative, and huge magnitudes."""
    K = 512
    x = torch.zeros(8, K)
    x[1, :] = 1e-12                                   # below the 1e-8 clamp
    # row 2: exact half-integer multiples of the scale: a = 127 -> s = 1, x = k + 0.5
    x[2, 0] = 127.0
    x[2, 1:255] = torch.arange(-127, 127).float() + 0.5
    x[3, 0] = -127.0                                  # negative absmax
    x[3, 1:] = torch.linspace(-127, 127, K - 1)
    x[4, :] = torch.randn(K) * 1e-39                  # subnormal fp32 -> bf16 subnormals
    x[5, :] = torch.randn(K) * 1e30
    x[6, ::2] = -0.0
    x[6, 1] = 3.0
    x[7, :] = torch.randn(K)
    xb = x.to(torch.bfloat16).to(cuda)
    _check(oracle, xb)
    # ties at a non-unit scale: a = 254 -> s = 2, x = 2k + 1 are exact ties in x / s
    y = torch.zeros(2, K)
    y[0, 0] = 254.0
    y[0, 1:128] = torch.arange(-127, 0).float() * 2 + 1
    y[1, 0] = 63.5
    y[1, 1:200] = torch.arange(1, 200).float() * 0.25
    _check(oracle, y.to(torch.bfloat16).to(cuda))
    _check(oracle, y.to(torch.float16).to(cuda))


def test_quant_rows_gather(oracle, cuda):
    """Routed gather fused into the quantizer: output row m quantizes x[row_idx[m]]; duplicates allowed."""
    from pyraquant_amd.workloads import make_x

    x = make_x(1000, 3072, torch.bfloat16, seed=11).to(cuda)
    g = torch.Generator().manual_seed(3)
    idx = torch.randint(0, 1000, (513,), generator=g, dtype=torch.int32)
    idx[:4] = torch.tensor([999, 0, 0, 5], dtype=torch.int32)
    _check(oracle, x, idx.to(cuda))


def test_quant_rows_empty(cuda):
    from pyraquant_amd import int8_exec as E

    x = torch.empty(0, 3072, dtype=torch.bfloat16, device=cuda)
    q, s = E.quant_rows(x)
    assert q.shape == (0, 3072) and s.shape == (0,)


@pytest.mark.parametrize("cfg", ["c1", "c2a"])
def test_quant_rows_full_size(oracle, cuda, cfg):
    """Full c1 / c2a shapes, bit-exact against the oracle."""
    from pyraquant_amd.workloads import CONFIGS, make_x

    c = CONFIGS[cfg]
    x = make_x(c.M, c.K, c.dtype).to(cuda)
    _check(oracle, x)


def test_quant_rows_routed_c4(oracle, cuda):
    """Config 4: gather of the 33,316 routed rows of the 65,536-row canvas."""
    from pyraquant_amd.workloads import make_x, routed_rows

    x = make_x(65536, 3072, torch.bfloat16).to(cuda)
    idx = routed_rows(cuda)
    assert idx.numel() == 33316
    _check(oracle, x, idx)


@pytest.mark.parametrize("fixture", ["quant_bf16.npz", "quant_f16.npz"])
def test_quant_rows_golden_fixture(cuda, fixture):
    """The HIP quantizer reproduces the committed golden vectors (torch CPU, deploy/int8_exec.py:508-509)."""
    import os

    from pyraquant_amd import int8_exec as E

    f = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", fixture), allow_pickle=False)
    dt = torch.bfloat16 if int(f["dtype"]) == 0 else torch.float16
    x = torch.from_numpy(f["x_bits"].view(np.int16)).view(dt).to(cuda)
    q, s = E.quant_rows(x)
    assert np.array_equal(q.cpu().numpy(), f["q"])
    assert np.array_equal(s.cpu().numpy().view(np.uint32), f["s"].view(np.uint32))


def test_linear_golden_fixture(cuda):
    """Golden layer (tests/golden/linear_lr.npz): codes, int32 accumulator and no-low-rank fp32 epilogue
    bit-exact, low-rank output within the tolerance of the float64 value."""
    import os

    from conftest import MAX_REL, MEAN_REL, rel_errors
    from pyraquant_amd import int8_exec as E

    f = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "linear_lr.npz"), allow_pickle=False)
    x = torch.from_numpy(f["x_bits"].view(np.int16)).view(torch.bfloat16).to(cuda)
    wq = torch.from_numpy(f["w_q"]).to(cuda)
    ws = torch.from_numpy(f["w_s"]).to(cuda)
    b = torch.from_numpy(f["bias"]).to(cuda)
    l1 = torch.from_numpy(f["l1_bits"].view(np.int16)).view(torch.bfloat16)
    l2 = torch.from_numpy(f["l2_bits"].view(np.int16)).view(torch.bfloat16)
    q, s = E.quant_rows(x)
    assert np.array_equal(q.cpu().numpy(), f["q"])
    acc = E.int8_gemm_i32(q, wq)
    assert np.array_equal(acc.cpu().numpy(), f["acc"])
    y = E.int8_gemm_fused(q, s, wq, ws, b, torch.bfloat16)
    ref = torch.from_numpy(f["y_nolr"]).to(torch.bfloat16)
    assert torch.equal(y.cpu(), ref)
    t = E.lowrank_down(x, l1.t().contiguous().to(cuda))
    ylr = E.int8_gemm_lr(q, s, wq, ws, b, t, l2.to(cuda), torch.bfloat16)
    mx, mean = rel_errors(ylr.float().cpu().numpy(), f["y_lr_f64"])
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
