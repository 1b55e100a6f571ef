"""GPU parity of the fused INT8 GEMM (pq_int8_gemm / pq_int8_gemm_i32) against the CPU oracle.

* int32 accumulators: bit-exact (pq_int8_gemm_i32) on ragged M / N / K.
* per-channel dequant (+bias), no low rank: bit-exact 16-bit output -- the kernel's fp32 epilogue runs in the
  reference's operation order (deploy/int8_exec.py:176-178), so nothing but the rounding of identical fp32
  values is involved.
* group-32 (no low rank): bit-exact (sequential fma over groups in both).
* low rank: max rel <= 1e-2, mean rel <= 5e-3 against the oracle's fp32 result (the MFMA's internal fp32
  summation order of t @ L2 is not the oracle's sequential order).
* routed scatter: written rows bit-exact, untouched rows keep the canvas bits.
* full c1 shape: checksum identity sum_n acc[m, n] == a[m] . (sum_n w[n]) in int64 for every row, and
  sampled rows bit-exact against the oracle.
"""
import numpy as np
import pytest
import torch

from conftest import MAX_REL, MEAN_REL, bits, dcode, rel_errors

pytestmark = pytest.mark.gpu



def _codes(M, N, K, seed, dev):
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    return a.to(dev), w.to(dev)


@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (7, 640, 640), (255, 256, 128), (257, 768, 1280),
                                   (1000, 320, 3072), (64, 12288, 64), (513, 1280, 2560)])
def test_gemm_i32_exact(oracle, cuda, M, N, K):
    from pyraquant_amd import int8_exec as E

    a, w = _codes(M, N, K, M + N + K, cuda)
    c = E.int8_gemm_i32(a, w)
    ref = oracle.gemm_i32(a.cpu().numpy(), w.cpu().numpy())
    assert np.array_equal(c.cpu().numpy(), ref)


def test_gemm_i32_extremes(oracle, cuda):
    """All +-127 / -127 codes at K = 12288: |acc| = 127^2 * 12288 = 198,193,152 (no overflow, exact)."""
    from pyraquant_amd import int8_exec as E

    M, N, K = 64, 128, 12288
    a = torch.full((M, K), 127, dtype=torch.int8)
    a[1::2] = -127
    w = torch.full((N, K), -127, dtype=torch.int8)
    w[::3] = 127
    c = E.int8_gemm_i32(a.to(cuda), w.to(cuda))
    ref = oracle.gemm_i32(a.numpy(), w.numpy())
    assert np.array_equal(c.cpu().numpy(), ref)
    assert abs(int(ref.max())) == 127 * 127 * K


def _scales(M, N, seed):
    g = torch.Generator().manual_seed(seed)
    s_row = torch.rand(M, generator=g) * 0.05 + 1e-3
    s_w = torch.rand(N, generator=g) * 2e-4 + 1e-5
    bias = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16).float()
    return s_row, s_w, bias


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("with_bias", [True, False])
@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (300, 640, 640), (1024, 768, 3072), (77, 3072, 128)])
def test_gemm_channel_exact(oracle, cuda, out_dtype, with_bias, M, N, K):
    from pyraquant_amd import int8_exec as E

    a, w = _codes(M, N, K, 3 * M + N, cuda)
    s_row, s_w, bias = _scales(M, N, M)
    b = bias if with_bias else None
    y = E.int8_gemm_fused(a, s_row.to(cuda), w, s_w.to(cuda), None if b is None else b.to(cuda), out_dtype)
    acc = oracle.gemm_i32(a.cpu().numpy(), w.cpu().numpy())
    yo = oracle.epilogue_f32(acc, s_row.numpy(), s_w.numpy(), None if b is None else b.numpy())
    ref = oracle.from_f32(yo, dcode(out_dtype))
    got = bits(y)
    mism = int((got != ref).sum())
    assert mism == 0, f"{mism} of {ref.size} outputs differ"


@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (200, 1280, 1280), (513, 640, 2048), (64, 5120, 1280)])
def test_gemm_group32_exact(oracle, cuda, M, N, K):
    from pyraquant_amd import int8_exec as E

    a, w = _codes(M, N, K, 5 * M + K, cuda)
    G = K // 32
    g = torch.Generator().manual_seed(9)
    s_row = torch.rand(M, generator=g) * 0.05 + 1e-3
    s_w = torch.rand(N, G, generator=g) * 2e-4 + 1e-5       # [N, G], the reference's qdq layout
    bias = (torch.randn(N, generator=g) * 0.01).float()
    y = E._gemm(a, s_row.to(cuda), w, s_w.t().contiguous().to(cuda), 32, bias.to(cuda), None, None, torch.float16)
    part = oracle.gemm_group_i32(a.cpu().numpy(), w.cpu().numpy(), 32)
    yo = oracle.epilogue_f32(part, s_row.numpy(), s_w.numpy(), bias.numpy())
    ref = oracle.from_f32(yo, 1)
    got = bits(y)
    mism = int((got != ref).sum())
    assert mism == 0, f"{mism} of {ref.size} outputs differ"


@pytest.mark.parametrize("R", [16, 32, 64])
@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (333, 768, 1024), (1024, 3072, 3072)])
def test_gemm_lowrank_tolerance(oracle, cuda, R, M, N, K):
    from pyraquant_amd import int8_exec as E

    a, w = _codes(M, N, K, 7 * M + R, cuda)
    s_row, s_w, bias = _scales(M, N, R)
    g = torch.Generator().manual_seed(R)
    t = (torch.randn(M, R, generator=g) * 0.5).to(torch.bfloat16)
    l2 = (torch.randn(R, N, generator=g) * 0.02).to(torch.bfloat16)
    y = E.int8_gemm_lr(a, s_row.to(cuda), w, s_w.to(cuda), bias.to(cuda), t.to(cuda), l2.to(cuda), torch.bfloat16)
    acc = oracle.gemm_i32(a.cpu().numpy(), w.cpu().numpy())
    yo = oracle.epilogue_f32(acc, s_row.numpy(), s_w.numpy(), bias.numpy(), bits(t), bits(l2), 0)
    got = oracle.to_f32(bits(y), 0)
    mx, mean = rel_errors(got, yo)
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)


def test_gemm_scatter(oracle, cuda):
    """Routed scatter: row m lands in canvas row out_row_idx[m]; all other canvas rows keep their bits."""
    from pyraquant_amd import int8_exec as E

    M, N, K, C = 300, 640, 640, 1000
    a, w = _codes(M, N, K, 21, cuda)
    s_row, s_w, bias = _scales(M, N, 4)
    g = torch.Generator().manual_seed(5)
    rows = torch.randperm(C, generator=g)[:M].to(torch.int32)
    canvas = torch.randn(C, N, generator=g).to(torch.bfloat16)
    before = bits(canvas)
    out = canvas.to(cuda)
    E.int8_gemm_fused(a, s_row.to(cuda), w, s_w.to(cuda), bias.to(cuda), torch.bfloat16, out=out,
                      out_row_idx=rows.to(cuda))
    acc = oracle.gemm_i32(a.cpu().numpy(), w.cpu().numpy())
    ref = oracle.from_f32(oracle.epilogue_f32(acc, s_row.numpy(), s_w.numpy(), bias.numpy()), 0)
    got = bits(out)
    r = rows.numpy()
    assert np.array_equal(got[r], ref)
    untouched = np.setdiff1d(np.arange(C), r)
    assert np.array_equal(got[untouched], before[untouched])


def test_dequant_epilogue_exact(oracle, cuda):
    from pyraquant_amd import int8_exec as E

    M, N = 129, 768
    g = torch.Generator().manual_seed(8)
    acc = torch.randint(-2**27, 2**27, (M, N), generator=g, dtype=torch.int32)
    s_row, s_w, bias = _scales(M, N, 8)
    y = E.dequant_epilogue(acc.to(cuda), s_row.to(cuda), s_w.to(cuda), bias.to(cuda), torch.bfloat16)
    ref = oracle.from_f32(oracle.epilogue_f32(acc.numpy(), s_row.numpy(), s_w.numpy(), bias.numpy()), 0)
    assert np.array_equal(bits(y), ref)


def test_gemm_full_c1_checksum(oracle, cuda):
    """c1 shape (M=65536, K=3072, N=12288): int64 row checksums of the int32 accumulator equal
    a @ colsum(w) exactly, and 64 sampled rows match the oracle bit for bit."""
    from pyraquant_amd import int8_exec as E

    M, N, K = 65536, 12288, 3072
    a, w = _codes(M, N, K, 42, cuda)
    c = E.int8_gemm_i32(a, w)
    rowsum = c.to(torch.int64).sum(dim=1)
    colsum_w = w.to(torch.int64).sum(dim=0)                       # [K]
    expect = (a.to(torch.int64) * colsum_w[None, :]).sum(dim=1)
    assert torch.equal(rowsum, expect)
    colsum_c = c.to(torch.int64).sum(dim=0)
    colsum_a = a.to(torch.int64).sum(dim=0)
    expect_c = (w.to(torch.int64) * colsum_a[None, :]).sum(dim=1)
    assert torch.equal(colsum_c, expect_c)
    g = torch.Generator().manual_seed(1)
    sample = torch.randperm(M, generator=g)[:64].sort().values
    ref = oracle.gemm_i32(a[sample.to(cuda)].cpu().numpy(), w.cpu().numpy())
    assert np.array_equal(c[sample.to(cuda)].cpu().numpy(), ref)


def test_gemm_rejects_bad_shapes(cuda):
    from pyraquant_amd import int8_exec as E

    a, w = _codes(16, 64, 96, 1, cuda)        # K % 64 != 0
    with pytest.raises(AssertionError):
        E.int8_gemm_i32(a, w)
    a, w = _codes(16, 96, 64, 1, cuda)        # N % 64 != 0
    with pytest.raises(AssertionError):
        E.int8_gemm_fused(a, torch.ones(16, device=cuda), w, torch.ones(96, device=cuda), None, torch.bfloat16)
