"""Full-size parity: Int8Linear.forward at every benchmark configuration's real shape (c0, c1, c2a, c2b, c3 in bf16 as
the configuration states it and in fp16, c4), checked against the CPU oracle on sampled rows (deploy/int8_exec.py:382-393
for the layer, :303-309 for the epilogue order).

Each unrouted case runs the whole layer on the GPU twice: through the module (Int8Linear.forward, whose common call is
one pq_int8_linear per layer), and through pq_int8_linear directly with a workspace the test holds. The two outputs
must be bit-identical, and the int8 codes and row scales are read back from that workspace: the packed buffer and
the scales the layer's first kernel staged for its GEMM. The test then takes 64 seeded random rows plus the last 40
rows (the last, possibly ragged, tiles) and computes those rows on the CPU with the oracle from the module's own int8
weights:
* int8 codes and row scales bit-exact;
* without a low-rank branch (c3), the 16-bit outputs bit-exact;
* with one, the normwise bar (max 1e-2, mean 5e-3) and the element-wise bar of conftest.elem_violation.
The routed case (c4) runs on the full 65536-row canvas through the general path (the gathering quantizer, then the
scattering GEMM): the routed rows land where the gather list says, every other row of the canvas is left as it was;
its codes come from a second call of the gathering quantizer. A last case runs c1 at batch 2 (131584 rows), whose
output rows lie past 2 GiB of byte offset.
"""
import ctypes

import numpy as np
import pytest
import torch

from conftest import MAX_REL, MEAN_REL, bits, dcode, elem_violation, rel_errors

pytestmark = pytest.mark.gpu


def _sample_rows(M: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    rows = torch.cat([torch.randperm(M - 40, generator=g)[:64], torch.arange(M - 40, M)])
    return rows.sort().values


def _packed_rows(qp: torch.Tensor, rows: torch.Tensor, K: int) -> np.ndarray:
    """Rows of a packed K64 code buffer, back in row-major order (the layout's definition: block (rb, kt) at
    (rb * KT + kt) * 1024, row r' = r % 16 at 64 r', 16-byte chunk c at slot c ^ swz(r'))."""
    from oracle import oracle as O

    KT = K // 64
    blocks = qp.view(-1, KT, 16, 4, 16)[(rows // 16).to(qp.device)].cpu().numpy()   # [n, KT, 16, 4, 16]
    rr = (rows % 16).numpy()
    n = rows.numel()
    sel = blocks[np.arange(n), :, rr]                                                 # [n, KT, 4, 16]
    slot = np.arange(4)[None, :] ^ O.k64_swz(rr)[:, None]                             # chunk c sits at slot[c]
    out = np.take_along_axis(sel, slot[:, None, :, None], axis=2)
    return out.reshape(n, K)


def _first_stage(E, q, x2, row_idx=None):
    """The codes, scales (and t) of the routed layer's first kernel, through the entry point its general path uses."""
    if q.lr_At is not None:
        return E.quant_rows_lowrank(x2, q.lr_At, row_idx, q._lr_frag())
    xq, sx = E.quant_rows_packed(x2, row_idx)
    return xq, sx, None


def _layer_call(q, x):
    """The layer through pq_int8_linear with a workspace held here (filled with 0xA5 first, so nothing is read from a
    clean buffer): (y, packed codes, row scales) with the codes and scales read from that workspace. Its layout for M
    rows and K inputs: the packed codes at byte 0 (ceil(M / 16) * 16 * K bytes), the fp32 row scales from the next
    256-byte boundary."""
    from pyraquant_amd import _lib

    L = _lib.load()
    M, K = x.shape
    N = q.out_features
    R = 0 if q.lr_At is None else q.lr_At.shape[0]
    Re = 0 if q.lr_Bt is None else q.lr_Bt.shape[1]
    ws = torch.full((L.pq_int8_linear_workspace_size(M, K, R),), 0xA5, dtype=torch.uint8, device=x.device)
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    frag = q._lr_frag() if R else None
    _lib.check(L.pq_int8_linear(p(x), _lib.dtype_code(x.dtype), M, K, x.stride(0), p(q.weight_packed), p(q._scale_k()),
                                q.group_size, p(q.bias), p(q.lr_At), p(frag), R, p(q.lr_Bt), Re, p(y), N, N, p(ws),
                                ws.numel(), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "pq_int8_linear")
    qb = (M + 15) // 16 * 16 * K
    so = (qb + 255) // 256 * 256
    return y, ws[:qb].view(torch.int8), ws[so:so + 4 * M].view(torch.float32)


def _check_rows(oracle, q, x_rows_bits, dt, y_rows, codes, scales):
    """Oracle of the sampled rows from the module's own buffers; codes / scales exact, outputs to the bar."""
    lr = q.lr_A is not None
    o = oracle.linear(x_rows_bits, dt, q.weight_int8.cpu().numpy(), q.w_scale.cpu().numpy(),
                      None if q.bias is None else q.bias.cpu().numpy(), q.group_size,
                      bits(q.lr_A) if lr else None, bits(q.lr_B) if lr else None)
    assert np.array_equal(codes, o["q"]), "int8 codes differ from the oracle"
    assert np.array_equal(scales.view(np.uint32), o["s"].view(np.uint32)), "row scales differ from the oracle"
    got = bits(y_rows)
    if not lr:
        assert np.array_equal(got, o["out"]), "outputs without a low-rank branch must be bit-exact"
        return
    y = oracle.to_f32(got, dt)
    mx, mean = rel_errors(y, o["y"])
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
    v = elem_violation(y, o["y"], oracle.to_f32(o["t"], dt), oracle.to_f32(bits(q.lr_B), dt))
    assert v <= 1.0, v


@pytest.mark.parametrize("cfg", ["c0", "c1", "c2a", "c2b", "c3_1280", "c3_5120", "c3_1280_f16", "c3_5120_f16"])
def test_layer_full_size(oracle, cuda, cfg):
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import CONFIGS, make_linear, make_x

    c = CONFIGS[cfg]
    print(f"[fullsize] {cfg} M={c.M} K={c.K} N={c.N} rank={c.lowrank} group={c.group} dtype={c.dtype}", flush=True)
    q = E.Int8Linear(make_linear(c.K, c.N, c.lowrank, c.bias, dtype=c.dtype), device=cuda, group_size=c.group)
    x = make_x(c.M, c.K, c.dtype, seed=7, device=cuda)
    y = q(x)
    assert y.shape == (c.M, c.N) and y.dtype == c.dtype
    y2, xq, sx = _layer_call(q, x)
    assert torch.equal(y2, y), "pq_int8_linear and Int8Linear.forward differ"
    del y2
    rows = _sample_rows(c.M, seed=c.M + c.N)
    rd = rows.to(cuda)
    _check_rows(oracle, q, bits(x[rd]), dcode(c.dtype), y[rd], _packed_rows(xq, rows, c.K), sx[rd].cpu().numpy())


def test_routed_full_canvas(oracle, cuda):
    """c4: config 4's 33,316 routed rows gathered from the 65536-token x and scattered into the 65536-row canvas."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import CONFIGS, make_linear, make_x, routed_rows

    c = CONFIGS["c4"]
    q = E.Int8Linear(make_linear(c.K, c.N, c.lowrank, c.bias), device=cuda)
    x = make_x(c.M, c.K, seed=8, device=cuda)
    ri = routed_rows(cuda)
    M = ri.numel()
    print(f"[fullsize] c4 routed M={M} of {c.M}", flush=True)
    canvas = make_x(c.M, c.N, seed=9, outlier_frac=0.0, device=cuda)
    before = canvas.clone()
    q(x, row_idx=ri, out=canvas, out_row_idx=ri)
    xq, sx, _ = _first_stage(E, q, x, ri)
    m = _sample_rows(M, seed=4)                      # positions in the routed list (the last 40: the ragged tile)
    src = ri.cpu()[m].long()
    _check_rows(oracle, q, bits(x[src.to(cuda)]), dcode(c.dtype), canvas[src.to(cuda)], _packed_rows(xq, m, c.K),
                sx[m.to(cuda)].cpu().numpy())
    keep = torch.ones(c.M, dtype=torch.bool, device=cuda)
    keep[ri.long()] = False
    assert torch.equal(canvas[keep], before[keep]), "rows outside the gather list must keep the cached canvas"


def test_layer_output_beyond_2gib(oracle, cuda):
    """FLUX's 4K stage at batch 2 (M = 131584 tokens, the c1 layer): the 3.2 GB bf16 output and the 404 MB of codes
    put rows past 2 GiB of byte offset (output rows from 87382 on), so every row address must be a 64-bit
    product. 64 sampled rows past that point, the last 40 included, against the oracle."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import CONFIGS, make_linear, make_x

    c = CONFIGS["c1"]
    M = 2 * (c.M + 256)
    print(f"[fullsize] c1 at batch 2: M={M} K={c.K} N={c.N}", flush=True)
    q = E.Int8Linear(make_linear(c.K, c.N, c.lowrank, c.bias, dtype=c.dtype), device=cuda)
    x = make_x(M, c.K, c.dtype, seed=11, device=cuda)
    y = q(x)
    assert y.shape == (M, c.N)
    first = (1 << 31) // (c.N * 2) + 1                      # the first output row wholly past 2 GiB
    g = torch.Generator().manual_seed(12)
    rows = torch.cat([first + torch.randperm(M - 40 - first, generator=g)[:24], torch.arange(M - 40, M)])
    rows = rows.sort().values
    y2, xq, sx = _layer_call(q, x)
    assert torch.equal(y2, y), "pq_int8_linear and Int8Linear.forward differ"
    del y2
    rd = rows.to(cuda)
    _check_rows(oracle, q, bits(x[rd]), dcode(c.dtype), y[rd], _packed_rows(xq, rows, c.K), sx[rd].cpu().numpy())
