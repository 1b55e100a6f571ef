"""GPU parity of the packed K64 layer path (pq_pack_k64, pq_quant_rows_packed, pq_int8_gemm_packed): the packed
bytes equal the oracle's restatement of the layout (oracle.pack_k64), the packed quantizer equals the row-major
quantizer packed, the packed GEMM's int32 accumulator is exact, and its fused output equals the row-major GEMM's
bit for bit (same arithmetic, only the operand layout differs)."""
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


@pytest.mark.parametrize("R,K", [(1, 64), (16, 64), (37, 192), (300, 640), (1000, 3072), (64, 12288)])
def test_pack_k64_matches_oracle(oracle, cuda, R, K):
    from pyraquant_amd import int8_exec as E

    a, _ = _codes(R, 1, K, R + K, cuda)
    p = E.pack_k64(a)
    assert np.array_equal(p.cpu().numpy(), oracle.pack_k64(a.cpu().numpy()))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K", [(1, 3072), (15, 640), (17, 1280), (300, 3072), (33, 12288)])
def test_quant_rows_packed(oracle, cuda, dtype, M, K):
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_x

    x = make_x(M, K, dtype, seed=3 * M + K).to(cuda)
    qp, s = E.quant_rows_packed(x)
    qo, so = oracle.quant_rows(bits(x), dcode(dtype))
    assert np.array_equal(qp.cpu().numpy(), oracle.pack_k64(qo))        # padding rows are zero too
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))


def test_quant_rows_packed_gather_and_view(oracle, cuda):
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_x

    base = make_x(500, 3072 + 12288, torch.bfloat16, seed=4).to(cuda)
    x = base[:, 3072:]                                           # row-slice view, ldx = 15360
    idx = torch.tensor([499, 0, 7, 7, 250, 31, 100], dtype=torch.int32)
    qp, s = E.quant_rows_packed(x, idx.to(cuda))
    qo, so = oracle.quant_rows(bits(x.contiguous()), 0, idx.numpy())
    assert np.array_equal(qp.cpu().numpy(), oracle.pack_k64(qo))
    assert np.array_equal(s.cpu().numpy(), so)


@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (7, 640, 640), (255, 256, 192), (257, 768, 1280),
                                   (1000, 320, 3072), (513, 1280, 2560), (4096, 3072, 3072)])
def test_gemm_packed_i32_exact(oracle, cuda, M, N, K):
    from pyraquant_amd import int8_exec as E

    a, w = _codes(M, N, K, M * 3 + N + K, cuda)
    c = E.int8_gemm_packed(E.pack_k64(a), None, E.pack_k64(w), None, None, M, N, K, torch.int32)
    assert np.array_equal(c.cpu().numpy(), oracle.gemm_i32(a.cpu().numpy(), w.cpu().numpy()))


@pytest.mark.parametrize("lr", [0, 16, 32, 64])
@pytest.mark.parametrize("M,N,K", [(333, 640, 1280), (1024, 3072, 3072), (77, 9216, 192)])
def test_gemm_packed_equals_rowmajor(cuda, lr, M, N, K):
    """Same fp32 epilogue on the same accumulators: bit-identical to the row-major kernel, with bias, low rank
    and both output dtypes."""
    from pyraquant_amd import int8_exec as E

    a, w = _codes(M, N, K, 5 * M + lr, cuda)
    g = torch.Generator().manual_seed(lr + 1)
    s_row = (torch.rand(M, generator=g) * 0.05 + 1e-3).to(cuda)
    s_w = (torch.rand(N, generator=g) * 2e-4 + 1e-5).to(cuda)
    bias = (torch.randn(N, generator=g) * 0.01).to(cuda)
    for dt in (torch.bfloat16, torch.float16):
        t = l2t = None
        if lr:
            t = (torch.randn(M, lr, generator=g) * 0.5).to(dt).to(cuda)
            l2t = (torch.randn(N, lr, generator=g) * 0.02).to(dt).to(cuda)
        ref = E._gemm(a, s_row, w, s_w, 0, bias, t, l2t, dt)
        got = E.int8_gemm_packed(E.pack_k64(a), s_row, E.pack_k64(w), s_w, bias, M, N, K, dt, t=t, l2t=l2t)
        assert torch.equal(got, ref), (dt, lr)


def test_gemm_packed_scatter(oracle, cuda):
    """Routed scatter on the packed path: gathered rows land in their canvas rows, other rows keep their bits."""
    from pyraquant_amd import int8_exec as E

    M, N, K, C = 300, 640, 640, 1000
    a, w = _codes(M, N, K, 21, cuda)
    g = torch.Generator().manual_seed(5)
    s_row = torch.rand(M, generator=g) * 0.05 + 1e-3
    s_w = torch.rand(N, generator=g) * 2e-4 + 1e-5
    bias = (torch.randn(N, generator=g) * 0.01).float()
    rows = torch.randperm(C, generator=g)[:M].to(torch.int32)
    canvas = torch.randn(C, N, generator=g).to(torch.bfloat16)
    before = bits(canvas)
    out = canvas.to(cuda)
    E.int8_gemm_packed(E.pack_k64(a), s_row.to(cuda), E.pack_k64(w), s_w.to(cuda), bias.to(cuda), M, N, K,
                       torch.bfloat16, out=out, out_row_idx=rows.to(cuda))
    acc = oracle.gemm_i32(a.cpu().numpy(), w.cpu().numpy())
    ref = oracle.from_f32(oracle.epilogue_f32(acc, s_row.numpy(), s_w.numpy(), bias.numpy()), 0)
    got = bits(out)
    r = rows.numpy()
    assert np.array_equal(got[r], ref)
    keep = np.setdiff1d(np.arange(C), r)
    assert np.array_equal(got[keep], before[keep])


def test_gemm_packed_full_c1_checksum(oracle, cuda):
    """c1 shape on the packed path: int64 row and column checksums of the int32 accumulator are exact, and 64
    sampled rows match the oracle bit for bit."""
    from pyraquant_amd import int8_exec as E

    M, N, K = 65536, 12288, 3072
    a, w = _codes(M, N, K, 42, cuda)
    c = E.int8_gemm_packed(E.pack_k64(a), None, E.pack_k64(w), None, None, M, N, K, torch.int32)
    rowsum = c.to(torch.int64).sum(dim=1)
    expect = (a.to(torch.int64) * w.to(torch.int64).sum(dim=0)[None, :]).sum(dim=1)
    assert torch.equal(rowsum, expect)
    colsum = c.to(torch.int64).sum(dim=0)
    expect_c = (w.to(torch.int64) * a.to(torch.int64).sum(dim=0)[None, :]).sum(dim=1)
    assert torch.equal(colsum, expect_c)
    g = torch.Generator().manual_seed(1)
    sample = torch.randperm(M, generator=g)[:64].sort().values.to(cuda)
    assert np.array_equal(c[sample].cpu().numpy(), oracle.gemm_i32(a[sample].cpu().numpy(), w.cpu().numpy()))


@pytest.mark.parametrize("cfg,M", [("c0", 4096), ("c1", 777)])
def test_int8linear_packed_path(oracle, cuda, cfg, M):
    """Int8Linear.forward runs on the packed path for per-channel layers; output within the tolerance of the
    oracle and equal to the row-major GEMM on the same codes."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import CONFIGS, make_linear, make_x

    c = CONFIGS[cfg]
    q = E.Int8Linear(make_linear(c.K, c.N, c.lowrank, c.bias), device=cuda)
    assert q.weight_packed is not None
    x = make_x(M, c.K).to(cuda)
    y = q(x)
    o = oracle.linear(bits(x), 0, q.weight_int8.cpu().numpy(), q.w_scale.cpu().numpy(), q.bias.cpu().numpy(), 0,
                      bits(q.lr_A), bits(q.lr_B))
    mx, mean = rel_errors(oracle.to_f32(bits(y), 0), o["y"])
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
    xq, sx = E.quant_rows(x)
    _, _, t = E.quant_rows_lowrank(x, q.lr_At, None, q._lr_frag())   # the low-rank rows the forward computed
    ref = E._gemm(xq, sx, q.weight_int8, q.w_scale, 0, q.bias, t, q.lr_Bt, torch.bfloat16)
    assert torch.equal(y, ref)


@pytest.mark.parametrize("M,N,K", [(8191, 6464, 1280), (16400, 4160, 192), (16400, 4160, 64), (16400, 4160, 256),
                                   (16400, 4160, 320)])
def test_gemm_big_tile_path_ragged(oracle, cuda, M, N, K):
    """Shapes with >= 1024 tiles of 256 x 128 take the 256 x 256 block of 8 waves (the ping-pong main loop, whose
    prologue issues 4 stages: K = 64 - 320 put the end of K inside, at and just past it); ragged M and N (tail tiles
    on both edges) stay exact there, row-major and packed, and the fused outputs agree bit for bit."""
    from pyraquant_amd import int8_exec as E

    a, w = _codes(M, N, K, M + N, cuda)
    c = E.int8_gemm_i32(a, w)
    cp = E.int8_gemm_packed(E.pack_k64(a), None, E.pack_k64(w), None, None, M, N, K, torch.int32)
    assert torch.equal(c, cp)
    g = torch.Generator().manual_seed(1)
    sample = torch.cat([torch.arange(M - 40, M), torch.randperm(M - 40, generator=g)[:24]]).sort().values.to(cuda)
    assert np.array_equal(c[sample].cpu().numpy(), oracle.gemm_i32(a[sample].cpu().numpy(), w.cpu().numpy()))
    s_row = (torch.rand(M, generator=g) * 0.05 + 1e-3).to(cuda)
    s_w = (torch.rand(N, generator=g) * 2e-4 + 1e-5).to(cuda)
    bias = (torch.randn(N, generator=g) * 0.01).to(cuda)
    t = (torch.randn(M, 32, generator=g) * 0.5).to(torch.bfloat16).to(cuda)
    l2t = (torch.randn(N, 32, generator=g) * 0.02).to(torch.bfloat16).to(cuda)
    ref = E._gemm(a, s_row, w, s_w, 0, bias, t, l2t, torch.bfloat16)
    got = E.int8_gemm_packed(E.pack_k64(a), s_row, E.pack_k64(w), s_w, bias, M, N, K, torch.bfloat16, t=t, l2t=l2t)
    assert torch.equal(got, ref)
    acc = c[sample].cpu().numpy()
    yo = oracle.epilogue_f32(acc, s_row[sample].cpu().numpy(), s_w.cpu().numpy(), bias.cpu().numpy(),
                             bits(t[sample]), bits(l2t.t().contiguous()), 0)
    mx, mean = rel_errors(oracle.to_f32(bits(got[sample]), 0), yo)
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)


@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (200, 1280, 1280), (513, 640, 2048), (64, 5120, 1280),
                                   (300, 640, 5120), (4107, 320, 192)])
def test_gemm_packed_group32_exact(oracle, cuda, M, N, K):
    """Group-32 on the packed path: per-group int32 partials fma'd in group order, bit-exact against the oracle
    and equal to the row-major kernel's output."""
    from pyraquant_amd import int8_exec as E

    a, w = _codes(M, N, K, 11 * M + K, cuda)
    G = K // 32
    g = torch.Generator().manual_seed(M + N)
    s_row = torch.rand(M, generator=g) * 0.05 + 1e-3
    s_w = torch.rand(N, G, generator=g) * 2e-4 + 1e-5       # [N, G], the reference's qdq layout
    bias = (torch.randn(N, generator=g) * 0.01).float()
    s_gn = s_w.t().contiguous().to(cuda)
    y = E.int8_gemm_packed(E.pack_k64(a), s_row.to(cuda), E.pack_k64(w), s_gn, bias.to(cuda), M, N, K,
                           torch.float16, group=32)
    part = oracle.gemm_group_i32(a.cpu().numpy(), w.cpu().numpy(), 32)
    ref = oracle.from_f32(oracle.epilogue_f32(part, s_row.numpy(), s_w.numpy(), bias.numpy()), 1)
    mism = int((bits(y) != ref).sum())
    assert mism == 0, f"{mism} of {ref.size} outputs differ"
    y_rm = E._gemm(a, s_row.to(cuda), w, s_gn, 32, bias.to(cuda), None, None, torch.float16)
    assert torch.equal(y, y_rm)


@pytest.mark.parametrize("lr", [16, 32, 64])
def test_gemm_packed_group32_lowrank_scatter(oracle, cuda, lr):
    """Group-32 with a low-rank branch and a routed scatter: within the tolerance of the oracle, equal to the
    row-major kernel, untouched canvas rows keep their bits."""
    from pyraquant_amd import int8_exec as E

    M, N, K, C = 500, 1280, 1280, 2000
    a, w = _codes(M, N, K, lr, cuda)
    g = torch.Generator().manual_seed(lr)
    s_row = torch.rand(M, generator=g) * 0.05 + 1e-3
    s_w = torch.rand(N, K // 32, generator=g) * 2e-4 + 1e-5
    t = (torch.randn(M, lr, generator=g) * 0.5).to(torch.float16)
    l2t = (torch.randn(N, lr, generator=g) * 0.02).to(torch.float16)
    rows = torch.randperm(C, generator=g)[:M].to(torch.int32)
    canvas = torch.randn(C, N, generator=g).to(torch.float16)
    before = bits(canvas)
    s_gn = s_w.t().contiguous().to(cuda)
    out = canvas.to(cuda)
    E.int8_gemm_packed(E.pack_k64(a), s_row.to(cuda), E.pack_k64(w), s_gn, None, M, N, K, torch.float16,
                       t=t.to(cuda), l2t=l2t.to(cuda), out=out, out_row_idx=rows.to(cuda), group=32)
    out_rm = canvas.to(cuda)
    E._gemm(a, s_row.to(cuda), w, s_gn, 32, None, t.to(cuda), l2t.to(cuda), torch.float16, out_rm, rows.to(cuda))
    assert torch.equal(out, out_rm)
    got = bits(out)
    r = rows.numpy()
    keep = np.setdiff1d(np.arange(C), r)
    assert np.array_equal(got[keep], before[keep])
    part = oracle.gemm_group_i32(a.cpu().numpy(), w.cpu().numpy(), 32)
    yo = oracle.epilogue_f32(part, s_row.numpy(), s_w.numpy(), None, bits(t), bits(l2t.t().contiguous()), 1)
    mx, mean = rel_errors(oracle.to_f32(got[r], 1), yo)
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)


@pytest.mark.parametrize("M,N,K,lr", [(4352, 3072, 3072, 32), (4100, 3008, 1280, 0), (3000, 3072, 12288, 32),
                                      (4096, 4096, 512, 0), (4096, 3072, 64, 0), (4100, 3008, 128, 32)])
def test_gemm_one_round_big_tiles(oracle, cuda, M, N, K, lr):
    """Problems whose 256 x 256 blocks all fit in one round on the chip (at most one per CU) while their 128 x 128
    blocks would need more than one round take the 256 x 256 block (M = 4352 is FLUX's 1K token count; 4096 x 4096
    is exactly one block per CU; the others are ragged in M and N, long in K, or a single 64-wide K stage against
    the ring's five). The int32 accumulators are exact against the oracle on sampled rows, the
    last ragged ones included, row-major and packed. The fused output is bit-identical to the same product computed
    in 256-row slices, whose few blocks run the 128 x 64 kernel with the same per-element epilogue arithmetic."""
    from pyraquant_amd import int8_exec as E

    a, w = _codes(M, N, K, M + N + lr, cuda)
    ap, wp = E.pack_k64(a), E.pack_k64(w)
    c = E.int8_gemm_i32(a, w)
    assert torch.equal(c, E.int8_gemm_packed(ap, None, wp, None, None, M, N, K, torch.int32))
    g = torch.Generator().manual_seed(lr + 5)
    sample = torch.cat([torch.arange(M - 40, M), torch.randperm(M - 40, generator=g)[:24]]).sort().values.to(cuda)
    assert np.array_equal(c[sample].cpu().numpy(), oracle.gemm_i32(a[sample].cpu().numpy(), w.cpu().numpy()))
    s_row = (torch.rand(M, generator=g) * 0.05 + 1e-3).to(cuda)
    s_w = (torch.rand(N, generator=g) * 2e-4 + 1e-5).to(cuda)
    bias = (torch.randn(N, generator=g) * 0.01).to(cuda)
    t = l2t = None
    if lr:
        t = (torch.randn(M, lr, generator=g) * 0.5).to(torch.bfloat16).to(cuda)
        l2t = (torch.randn(N, lr, generator=g) * 0.02).to(torch.bfloat16).to(cuda)
    got = E.int8_gemm_packed(ap, s_row, wp, s_w, bias, M, N, K, torch.bfloat16, t=t, l2t=l2t)
    ref = torch.empty_like(got)
    for r0 in range(0, M, 256):     # rows r0 .. r0 + 255 of a packed operand are its bytes [r0 K, (r0 + 256) K)
        r1 = min(r0 + 256, M)
        E.int8_gemm_packed(ap[r0 * K:], s_row[r0:], wp, s_w, bias, r1 - r0, N, K, torch.bfloat16,
                           t=None if t is None else t[r0:r1], l2t=l2t, out=ref[r0:r1])
    assert torch.equal(got, ref)
    assert torch.equal(E._gemm(a, s_row, w, s_w, 0, bias, t, l2t, torch.bfloat16), got)


@pytest.mark.parametrize("M,N,K,lr", [(4352, 12288, 3072, 0), (4352, 12288, 3072, 32), (2100, 9216, 1280, 0)])
def test_gemm_big_tile_rowmajor_equals_packed_repeated(cuda, M, N, K, lr):
    """256 x 256 blocks on row-major operands (the reference self-test's int8_gemm_fused shape) give the packed path's
    bits on every call. The last ring stages carry the epilogue operands; each stage must issue its full DMA count
    for the ring's vmcnt waits, so a stage that issues fewer leaves the previous stage's last tiles racing."""
    from pyraquant_amd import int8_exec as E

    a, w = _codes(M, N, K, M + lr, cuda)
    g = torch.Generator().manual_seed(lr + 3)
    s_row = (torch.rand(M, generator=g) * 0.05 + 1e-3).to(cuda)
    s_w = (torch.rand(N, generator=g) * 2e-4 + 1e-5).to(cuda)
    bias = (torch.randn(N, generator=g) * 0.01).to(cuda)
    t = l2t = None
    if lr:
        t = (torch.randn(M, lr, generator=g) * 0.5).to(torch.bfloat16).to(cuda)
        l2t = (torch.randn(N, lr, generator=g) * 0.02).to(torch.bfloat16).to(cuda)
    ref = E.int8_gemm_packed(E.pack_k64(a), s_row, E.pack_k64(w), s_w, bias, M, N, K, torch.bfloat16, t=t, l2t=l2t)
    for _ in range(4):
        y = E._gemm(a, s_row, w, s_w, 0, bias, t, l2t, torch.bfloat16)
        assert torch.equal(y, ref)


@pytest.mark.parametrize("R,dt", [(16, torch.bfloat16), (32, torch.float16), (64, torch.bfloat16)])
def test_gemm_big_tile_lowrank_ranks(oracle, cuda, R, dt):
    """Ranks 16, 32 (fp16) and 64 on the 256 x 256 block: ranks 16 and 32 ride the ring's epilogue stages, rank 64's
    rows do not fit them and take the register epilogue. All stay within the tolerance of the oracle on sampled rows
    (ragged last rows included), and the row-major and packed paths agree bit for bit."""
    from pyraquant_amd import int8_exec as E

    M, N, K = 4352 + 37, 12288, 1024
    code = dcode(dt)
    a, w = _codes(M, N, K, 5 * R, cuda)
    g = torch.Generator().manual_seed(R)
    s_row = (torch.rand(M, generator=g) * 0.05 + 1e-3).to(cuda)
    s_w = (torch.rand(N, generator=g) * 2e-4 + 1e-5).to(cuda)
    bias = (torch.randn(N, generator=g) * 0.01).to(cuda)
    t = (torch.randn(M, R, generator=g) * 0.5).to(dt).to(cuda)
    l2t = (torch.randn(N, R, generator=g) * 0.02).to(dt).to(cuda)
    got = E.int8_gemm_packed(E.pack_k64(a), s_row, E.pack_k64(w), s_w, bias, M, N, K, dt, t=t, l2t=l2t)
    ref = E._gemm(a, s_row, w, s_w, 0, bias, t, l2t, dt)
    assert torch.equal(got, ref)
    sample = torch.cat([torch.arange(M - 40, M), torch.randperm(M - 40, generator=g)[:24]]).sort().values.to(cuda)
    acc = oracle.gemm_i32(a[sample].cpu().numpy(), w.cpu().numpy())
    yo = oracle.epilogue_f32(acc, s_row[sample].cpu().numpy(), s_w.cpu().numpy(), bias.cpu().numpy(),
                             bits(t[sample]), bits(l2t.t().contiguous()), code)
    mx, mean = rel_errors(oracle.to_f32(bits(got[sample]), code), yo)
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)


@pytest.mark.parametrize("packed", [False, True])
def test_gemm_deep_k_tiles(oracle, cuda, packed):
    """Long K (>= 8192) on >= 1024 tiles runs 256 x 256 blocks of 8 waves: exact int32 accumulator (int64 row and
    column checksums, sampled rows against the oracle) and a fused rank-32 output equal to the other layout's."""
    from pyraquant_amd import int8_exec as E

    M, N, K = 16384, 3072, 12288
    a, w = _codes(M, N, K, 77, cuda)
    if packed:
        c = E.int8_gemm_packed(E.pack_k64(a), None, E.pack_k64(w), None, None, M, N, K, torch.int32)
    else:
        c = E.int8_gemm_i32(a, w)
    rowsum = c.to(torch.int64).sum(dim=1)
    assert torch.equal(rowsum, (a.to(torch.int64) * w.to(torch.int64).sum(dim=0)[None, :]).sum(dim=1))
    colsum = c.to(torch.int64).sum(dim=0)
    assert torch.equal(colsum, (w.to(torch.int64) * a.to(torch.int64).sum(dim=0)[None, :]).sum(dim=1))
    g = torch.Generator().manual_seed(2)
    sample = torch.cat([torch.arange(M - 16, M), torch.randperm(M - 16, generator=g)[:16]]).sort().values.to(cuda)
    assert np.array_equal(c[sample].cpu().numpy(), oracle.gemm_i32(a[sample].cpu().numpy(), w.cpu().numpy()))
    del c
    s_row = (torch.rand(M, generator=g) * 0.05 + 1e-3).to(cuda)
    s_w = (torch.rand(N, generator=g) * 2e-4 + 1e-5).to(cuda)
    bias = (torch.randn(N, generator=g) * 0.01).to(cuda)
    t = (torch.randn(M, 32, generator=g) * 0.5).to(torch.bfloat16).to(cuda)
    l2t = (torch.randn(N, 32, generator=g) * 0.02).to(torch.bfloat16).to(cuda)
    yp = E.int8_gemm_packed(E.pack_k64(a), s_row, E.pack_k64(w), s_w, bias, M, N, K, torch.bfloat16, t=t, l2t=l2t)
    yr = E._gemm(a, s_row, w, s_w, 0, bias, t, l2t, torch.bfloat16)
    assert torch.equal(yp, yr)
