"""GPU parity of pq_quant_rows_lowrank, the quantizer and the rank-32 low-rank down-projection from one pass over x
(deploy/int8_exec.py:390-391):
* packed codes and scales bit-identical to pq_quant_rows_packed on the same rows (which the quantizer tests pin
  against the oracle);
* t within bf16 rounding of the float64 product and within the build's tolerance of the oracle's fp32 result;
* K = 4096 .. 12288 in steps of 2048 (c2a's 12288) and 15360 (FLUX's single-block proj_out) run the wide kernel,
  which holds rows in registers (two per wave, one at 15360, in batches of 16 or 8 rows): the same bar;
* other shapes (K outside both lists, R != 32) run the two kernels: the same bar, and exactly what the two separate
  entry points give;
* the fragment-order copy of l1t (pq_pack_lowrank_l1t) matches its documented index formula, and the one-pass kernel
  gives the same bits from it as from l1t.
"""
import numpy as np
import pytest
import torch

from conftest import MAX_REL, MEAN_REL, bits, dcode, rel_errors

pytestmark = pytest.mark.gpu


def _l1(K, R, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(K, R, generator=g) * 0.02).to(dtype)


def _check_t(oracle, t, x_rows, l1, dtype):
    ref64 = x_rows.double() @ l1.double()
    got = t.cpu().double()
    err = (got - ref64).abs() / ref64.abs().clamp_min(1e-3 * ref64.abs().max())
    assert float(err.max()) <= 1.5e-2, float(err.max())
    ref_bits = oracle.lowrank_down(bits(x_rows.contiguous()), dcode(dtype), bits(l1))
    mx, mean = rel_errors(oracle.to_f32(bits(t), dcode(dtype)), oracle.to_f32(ref_bits, dcode(dtype)))
    assert mx <= MAX_REL * 2 and mean <= MEAN_REL, (mx, mean)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K", [(1, 3072), (16, 3072), (17, 3072), (1000, 1280), (4099, 3072), (300, 2048),
                                 (65, 2560), (33, 1024), (20000, 3072),
                                 (1, 12288), (7, 12288), (1001, 12288), (37, 4096), (100, 5120), (50, 6144),
                                 (23, 15360), (9000, 12288), (4111, 8192), (17, 10240),
                                 (1, 15360), (8, 15360), (9, 15360), (16, 15360), (4352, 15360), (5003, 15360)])
def test_quant_rows_lowrank_fused(oracle, cuda, dtype, M, K):
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_x

    x = make_x(M, K, dtype, seed=M + K).to(cuda)
    l1 = _l1(K, 32, dtype, K)
    qp, s, t = E.quant_rows_lowrank(x, l1.t().contiguous().to(cuda))
    qr, sr = E.quant_rows_packed(x)
    assert torch.equal(qp, qr)                                   # padding rows to 16 included
    assert torch.equal(s.view(torch.int32), sr.view(torch.int32))
    if M <= 4099:
        _check_t(oracle, t, x.cpu(), l1, dtype)
    else:   # large M: t against the separate low-rank kernel (same fp32 accumulation up to order)
        t2 = E.lowrank_down(x, l1.t().contiguous().to(cuda))
        mx, mean = rel_errors(t.float().cpu().numpy(), t2.float().cpu().numpy())
        assert mx <= 1e-2 and mean <= 1e-3, (mx, mean)


def test_quant_rows_lowrank_gather_view(oracle, cuda):
    """Routed gather (duplicates, first and last row) through a row-slice view of a wider activation."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_x

    rows, K, M = 3000, 3072, 1234
    base = make_x(rows, K + 128, seed=7).to(cuda)
    x = base[:, 128:]                                            # ldx = K + 128
    g = torch.Generator().manual_seed(3)
    idx = torch.randint(0, rows, (M,), generator=g, dtype=torch.int32)
    idx[:4] = torch.tensor([rows - 1, 0, 0, 5], dtype=torch.int32)
    l1 = _l1(K, 32, torch.bfloat16, 11)
    qp, s, t = E.quant_rows_lowrank(x, l1.t().contiguous().to(cuda), idx.to(cuda))
    qr, sr = E.quant_rows_packed(x, idx.to(cuda))
    assert torch.equal(qp, qr)
    assert torch.equal(s, sr)
    _check_t(oracle, t, x.cpu()[idx.long()], l1, torch.bfloat16)


@pytest.mark.parametrize("M,K,R", [(100, 5120, 32), (70, 640, 32), (300, 3072, 64), (40, 12288, 64),
                                   (50, 14336, 32)])
def test_quant_rows_lowrank_fallback(cuda, M, K, R):
    """Shapes outside the fused kernels' sets run the two kernels: identical to calling them one after the other."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_x

    x = make_x(M, K, seed=K).to(cuda)
    l1t = _l1(K, R, torch.bfloat16, R).t().contiguous().to(cuda)
    qp, s, t = E.quant_rows_lowrank(x, l1t)
    qr, sr = E.quant_rows_packed(x)
    assert torch.equal(qp, qr) and torch.equal(s, sr)
    assert torch.equal(t, E.lowrank_down(x, l1t))


@pytest.mark.parametrize("K", [12288, 15360])
def test_quant_rows_lowrank_wide_gather_view(oracle, cuda, K):
    """K = 12288 and 15360 (the wide kernel, two and one rows per wave) through a gather with duplicates and a
    row-slice view (ldx = K + 512): codes and scales bit-identical to the packed quantizer's, t within bf16 rounding
    of the float64 product."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_x

    rows, M = 600, 333
    base = make_x(rows, K + 512, seed=9).to(cuda)
    x = base[:, 512:]
    g = torch.Generator().manual_seed(4)
    idx = torch.randint(0, rows, (M,), generator=g, dtype=torch.int32)
    idx[:3] = torch.tensor([rows - 1, 0, 0], dtype=torch.int32)
    l1 = _l1(K, 32, torch.bfloat16, 13)
    qp, s, t = E.quant_rows_lowrank(x, l1.t().contiguous().to(cuda), idx.to(cuda))
    qr, sr = E.quant_rows_packed(x, idx.to(cuda))
    assert torch.equal(qp, qr)
    assert torch.equal(s, sr)
    _check_t(oracle, t, x.cpu()[idx.long()], l1, torch.bfloat16)


@pytest.mark.parametrize("K,N,M", [(3072, 12288, 2000), (15360, 3072, 333)])
def test_int8linear_uses_fused_pass(oracle, cuda, K, N, M):
    """Int8Linear.forward takes the fused pass, at the c1 shape (reduced M) and at FLUX's unsplit single-block
    proj_out (K = 15360, the wide kernel at one row per wave): output within the tolerance of the oracle from the same
    codes, and equal to the GEMM fed with the fused t."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    q = E.Int8Linear(make_linear(K, N, 32, True), device=cuda)
    x = make_x(M, K).to(cuda)
    y = q(x)
    qp, sx, t = E.quant_rows_lowrank(x, q.lr_At)
    ref = E.int8_gemm_packed(qp, sx, q.weight_packed, q.w_scale, q.bias, M, N, K, torch.bfloat16, t=t,
                             l2t=q.lr_Bt)
    assert torch.equal(y, ref)
    o = oracle.linear(bits(x), 0, q.weight_int8.cpu().numpy(), q.w_scale.cpu().numpy(), q.bias.cpu().numpy(), 0,
                      bits(q.lr_A), bits(q.lr_B))
    mx, mean = rel_errors(oracle.to_f32(bits(y), 0), o["y"])
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)


def _fragment_order_np(l1t: np.ndarray) -> np.ndarray:
    """The fragment order pq_pack_lowrank_l1t documents, from its index formula (numpy, uint16 bits): piece
    p = ((w * 2 + h) * NS + i) * 64 + l of 8 values holds l1t[16 h + l % 16][w K / W + 64 (i // 2) + 16 (l // 16)
    + 8 (i % 2) + (0..7)], W = 16 / 8 / 4 waves for K / 256 divisible by 4 / 2 / neither, NS = K / (32 W)."""
    R, K = l1t.shape
    nc = K // 256
    W = 16 if nc % 4 == 0 else (8 if nc % 2 == 0 else 4)
    NS = K // (32 * W)
    out = np.empty((4 * K, 8), dtype=l1t.dtype)
    for p in range(4 * K):
        l, rest = p % 64, p // 64
        i, wh = rest % NS, rest // NS
        h, w = wh % 2, wh // 2
        col = w * (K // W) + 64 * (i // 2) + 16 * (l // 16) + 8 * (i % 2)
        out[p] = l1t[16 * h + l % 16, col:col + 8]
    return out.reshape(R, K)


@pytest.mark.parametrize("K", [1024, 1280, 2048, 2560, 3072])
def test_pack_lowrank_l1t_order(cuda, K):
    """pq_pack_lowrank_l1t against its documented index formula, bit for bit; a permutation (every value once)."""
    from pyraquant_amd import int8_exec as E

    l1t = _l1(K, 32, torch.bfloat16, 7 + K).t().contiguous()
    got = E.pack_lowrank_l1t(l1t.to(cuda))
    ref = _fragment_order_np(bits(l1t).reshape(32, K))
    assert np.array_equal(bits(got).reshape(32, K), ref)
    assert np.array_equal(np.sort(ref.ravel()), np.sort(bits(l1t).ravel()))
    assert E.pack_lowrank_l1t(torch.zeros(64, K, dtype=torch.bfloat16, device=cuda)) is None


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K", [(1, 3072), (17, 1280), (4096, 3072), (1000, 1024), (300, 2048), (65, 2560),
                                 (20000, 3072)])
def test_quant_rows_lowrank_fragment_order_identical(cuda, dtype, M, K):
    """Codes, scales and t are bit-identical whether the one-pass kernel reads l1t or its fragment-order copy,
    plain and through a routed gather."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_x

    x = make_x(M, K, dtype, seed=3 * M + K, device=cuda)
    l1t = _l1(K, 32, dtype, K + 1).t().contiguous().to(cuda)
    l1f = E.pack_lowrank_l1t(l1t)
    assert l1f is not None
    idx = torch.randint(0, M, (max(1, M // 3),), generator=torch.Generator().manual_seed(M), dtype=torch.int32)
    for idx in (None, idx.to(cuda)):
        a = E.quant_rows_lowrank(x, l1t, idx)
        b = E.quant_rows_lowrank(x, l1t, idx, l1f)
        for u, v in zip(a, b):   # codes (int8), scales (fp32 bits), t (16-bit bits)
            as_int = {1: torch.int8, 2: torch.int16, 4: torch.int32}[u.element_size()]
            assert torch.equal(u.view(as_int), v.view(as_int))


def test_int8linear_keeps_fragment_order_through_casts(cuda):
    """Int8Linear packs lr_At_frag at conversion where the order exists (K = 3072, rank 32) and not otherwise
    (K = 4096); a module-wide cast carries it with lr_At, and the forward's output is the same with or without it."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    q = E.Int8Linear(make_linear(3072, 640, 32, True, seed=5), device=cuda)
    assert q.lr_At_frag is not None and "lr_At_frag" not in q.state_dict()
    assert E.Int8Linear(make_linear(4096, 640, 32, True, seed=5), device=cuda).lr_At_frag is None
    x = make_x(333, 3072, torch.bfloat16, seed=9, device=cuda)
    y = q(x)
    frag = q.lr_At_frag
    q.lr_At_frag = None
    y_plain = q(x)
    q.lr_At_frag = frag
    assert torch.equal(y.view(torch.int16), y_plain.view(torch.int16))
    q.half()
    assert q.lr_At_frag.dtype == torch.float16 and q._lr_frag() is not None
    xh = x.half()
    yh = q(xh)
    q.lr_At_frag = None
    assert torch.equal(yh.view(torch.int16), q(xh).view(torch.int16))


def test_int8linear_fragment_order_follows_lr_At(cuda):
    """lr_At_frag is derived from lr_At: after load_state_dict (an in-place copy into lr_At) or an in-place edit of
    lr_At the module repacks it, so the one-pass kernel never reads a stale copy. Checked against a module built from
    the loaded weights and against the row-major path after the edit."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    q1 = E.Int8Linear(make_linear(3072, 640, 32, True, seed=5), device=cuda)
    q2 = E.Int8Linear(make_linear(3072, 640, 32, True, seed=6), device=cuda)
    x = make_x(333, 3072, torch.bfloat16, seed=9, device=cuda)
    y2 = q2(x)
    q1.load_state_dict(q2.state_dict())
    assert torch.equal(q1(x).view(torch.int16), y2.view(torch.int16))
    with torch.no_grad():
        q1.lr_At.mul_(2)
    y_frag = q1(x)                   # repacked from the edited lr_At
    q1.lr_At_frag = None             # the row-major path, same lr_At
    y_plain = q1(x)
    assert torch.equal(y_frag.view(torch.int16), y_plain.view(torch.int16))
    assert not torch.equal(y_frag.view(torch.int16), y2.view(torch.int16))
