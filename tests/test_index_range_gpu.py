"""Gather and scatter indices outside their tensors (pq_quant_rows, pq_quant_rows_packed, pq_quant_rows_lowrank,
pq_lowrank_down, pq_int8_gemm, pq_int8_gemm_packed): a gathered source row outside [0, x_rows) quantizes as a row of
zeros (codes 0, scale fl(1e-8) / 127, t = 0), a scattered row outside [0, c_rows) is not written, and every in-range
row is what the same call gives with only in-range indices. Each out-of-range index here still points inside a larger
parent allocation (x and the canvas are views into the middle of one), so a missing check would show up as a wrong
value, never as an access past the allocation."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

PAD = 8
ZERO_SCALE = np.float32(np.float32(1e-8) / np.float32(127.0))


def _view_in_parent(rows, cols, dtype, seed, dev):
    from pyraquant_amd.workloads import make_x

    parent = make_x(rows + 2 * PAD, cols, dtype, seed=seed, device=dev)
    return parent, parent[PAD:PAD + rows]


def _bits_equal(a, b):
    as_int = {1: torch.int8, 2: torch.int16, 4: torch.int32}[a.element_size()]
    return torch.equal(a.view(as_int), b.view(as_int))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K", [100, 200, 1280, 3072, 4096])
def test_gather_out_of_range_reads_zero_rows(cuda, dtype, K):
    """K = 100: the per-element quantizer; 200: the vector quantizer and the register low-rank kernel; 1280 and 3072:
    the one-pass fused kernel (with and without the fragment-order L1^T); 4096: the wide-row fused kernel."""
    from pyraquant_amd import int8_exec as E

    rows = 40
    _, x = _view_in_parent(rows, K, dtype, seed=K, dev=cuda)
    idx_list = [3, -1, rows, 0, rows + 5, rows - 1, -PAD, 7, 11, rows + PAD - 1]
    live = [0 <= i < rows for i in idx_list]
    print(f"[index_range] gather K={K} {dtype}", flush=True)
    idx = torch.tensor(idx_list, dtype=torch.int32, device=cuda)
    ref_idx = torch.tensor([i if ok else 0 for i, ok in zip(idx_list, live)], dtype=torch.int32, device=cuda)
    dead = torch.tensor([not ok for ok in live], device=cuda)

    def check_rows(q, s, q_ref, s_ref):
        assert _bits_equal(q[~dead], q_ref[~dead]) and _bits_equal(s[~dead], s_ref[~dead])
        assert not q[dead].any()
        assert np.all(s[dead].cpu().numpy().view(np.uint32) == ZERO_SCALE.view(np.uint32))

    q, s = E.quant_rows(x, idx)
    check_rows(q, s, *E.quant_rows(x, ref_idx))
    if K % 64 == 0:
        qp, sp = E.quant_rows_packed(x, idx)
        assert torch.equal(qp, E.pack_k64(q)) and _bits_equal(sp, s)
    if K % 8 == 0:
        l1t = (torch.randn(32, K, generator=torch.Generator().manual_seed(K)) * 0.02).to(dtype).to(cuda)
        t = E.lowrank_down(x, l1t, idx)
        t_ref = E.lowrank_down(x, l1t, ref_idx)
        assert _bits_equal(t[~dead], t_ref[~dead]) and not t[dead].any()
        if K % 64 == 0:
            for frag in (None, E.pack_lowrank_l1t(l1t)):
                qf, sf, tf = E.quant_rows_lowrank(x, l1t, idx, frag)
                qr, sr, tr = E.quant_rows_lowrank(x, l1t, ref_idx, frag)
                assert torch.equal(qf, qp) and _bits_equal(sf, sp)
                assert _bits_equal(tf[~dead], tr[~dead]) and not tf[dead].any()


@pytest.mark.parametrize("M,N,K,group,rank,accumulate", [
    (300, 640, 1280, 0, 32, False),      # 128 x 64 blocks
    (300, 640, 1280, 0, 32, True),       # the accumulating epilogue (reads the destination row first)
    (300, 1280, 1280, 32, 0, False),     # group-32
    (12000, 3072, 1024, 0, 32, False),   # 256 x 256 blocks
    (12000, 3072, 1024, 0, 0, True),
])
def test_scatter_out_of_range_rows_not_written(cuda, M, N, K, group, rank, accumulate):
    """Int8Linear.forward scattering into a canvas view: rows named outside the canvas are skipped, rows named inside
    it get the layer's output (added to the row with accumulate=True, as torch's 16-bit add rounds it), every other
    row of the canvas and of its parent keeps its bits."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    dtype = torch.float16 if group else torch.bfloat16
    q = E.Int8Linear(make_linear(K, N, rank, True, seed=M + N, dtype=dtype), device=cuda, group_size=group)
    x = make_x(M, K, dtype, seed=M, device=cuda)
    rows_c = M + 64
    parent, canvas = _view_in_parent(rows_c, N, dtype, seed=N, dev=cuda)
    g = torch.Generator().manual_seed(M + K)
    ori_list = torch.randperm(rows_c, generator=g)[:M].tolist()
    bad = {1: -1, 5: rows_c, M // 2: rows_c + PAD - 1, M - 1: -PAD}
    for m, v in bad.items():
        ori_list[m] = v
    ori = torch.tensor(ori_list, dtype=torch.int32, device=cuda)
    print(f"[index_range] scatter M={M} N={N} K={K} group={group} rank={rank} acc={accumulate}", flush=True)
    y = q(x)                                               # the dense result of the same layer
    before = parent.clone()
    q(x, out=canvas, out_row_idx=ori, accumulate=accumulate)
    torch.cuda.synchronize()
    good = [m for m in range(M) if m not in bad]
    dst = torch.tensor([ori_list[m] for m in good], device=cuda) + PAD
    src = torch.tensor(good, device=cuda)
    expect = before.clone()
    expect[dst] = before[dst] + y[src] if accumulate else y[src]
    assert _bits_equal(parent, expect)
    if not group and not rank:   # the row-major GEMM entry, same rule
        xq, sx = E.quant_rows(x)
        canvas.copy_(before[PAD:PAD + rows_c])
        E.int8_gemm_fused(xq, sx, q.weight_int8, q.w_scale, q.bias, dtype, out=canvas, out_row_idx=ori)
        torch.cuda.synchronize()
        expect = before.clone()
        expect[dst] = E.int8_gemm_fused(xq, sx, q.weight_int8, q.w_scale, q.bias, dtype)[src]
        assert _bits_equal(parent, expect)
