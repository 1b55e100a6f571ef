"""GPU parity of the Int8Linear module path (quantizer + low-rank down + fused GEMM) against the CPU oracle,
the routed executor (gather + scatter), the SDXL group-32 module and the reference's own self-test
(deploy/int8_exec.py:495-536)."""
import numpy as np
import pytest
import torch

from conftest import MAX_REL, MEAN_REL, bits, dcode, rel_errors

pytestmark = pytest.mark.gpu



def _oracle_module(oracle, q, x, row_idx=None, out_dtype=None):
    """Oracle of Int8Linear.forward from the module's own int8 weights / scales / low-rank buffers."""
    dt = dcode(x.dtype)
    l1 = None if q.lr_A is None else bits(q.lr_A)
    l2 = None if q.lr_B is None else bits(q.lr_B)
    return oracle.linear(bits(x), dt, q.weight_int8.cpu().numpy(), q.w_scale.cpu().numpy(),
                         None if q.bias is None else q.bias.cpu().numpy(), q.group_size, l1, l2,
                         None if row_idx is None else row_idx.cpu().numpy(), out_dtype)


def test_weight_rtn_matches_oracle(oracle, cuda):
    """Per-channel and group-32 weight RTN on the GPU give the oracle's codes and scales bit for bit."""
    from pyraquant_amd.int8_exec import quantize_weight
    from pyraquant_amd.workloads import make_weights

    w = make_weights(1280, 640, 0, False)["w"]
    for group in (0, 32):
        q, s = quantize_weight(w.to(cuda), group)
        qo, so = oracle.quant_weight(w.numpy(), group)
        assert np.array_equal(q.cpu().numpy(), qo)
        assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("M,K,R", [(1, 3072, 32), (333, 3072, 32), (4096, 3072, 32), (100, 1280, 64),
                                   (64, 12288, 32), (7, 15360, 96), (70, 1024, 128)])
def test_lowrank_down(oracle, cuda, M, K, R):
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_x

    x = make_x(M, K, seed=K + M)
    g = torch.Generator().manual_seed(R)
    l1 = (torch.randn(K, R, generator=g) * 0.02).to(torch.bfloat16)
    t = E.lowrank_down(x.to(cuda), l1.t().contiguous().to(cuda))
    ref_bits = oracle.lowrank_down(bits(x), 0, bits(l1))
    # fp64 reference of the same product: the 16-bit result is within bf16 rounding of it
    ref64 = x.double() @ l1.double()
    got = t.cpu().double()
    err = (got - ref64).abs() / ref64.abs().clamp_min(1e-3 * ref64.abs().max())
    assert float(err.max()) <= 1.5e-2, float(err.max())
    mx, mean = rel_errors(oracle.to_f32(bits(t), 0), oracle.to_f32(ref_bits, 0))
    assert mx <= MAX_REL * 2 and mean <= MEAN_REL, (mx, mean)


@pytest.mark.parametrize("cfg,M", [("c0", 4096), ("c1", 1000), ("c2a", 500), ("c2b", 700)])
def test_int8linear_flux(oracle, cuda, cfg, M):
    """Int8Linear with the rank-32 branch: codes / scales bit-exact, output within 1e-2 max / 5e-3 mean
    relative of the oracle's fp32 result computed from the same codes."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import CONFIGS, make_linear, make_x

    c = CONFIGS[cfg]
    lin = make_linear(c.K, c.N, c.lowrank, c.bias)
    q = E.Int8Linear(lin, device=cuda)
    x = make_x(M, c.K, c.dtype).to(cuda)
    y = q(x)
    assert y.dtype == x.dtype and y.shape == (M, c.N)
    o = _oracle_module(oracle, q, x)
    xq, sx = E.quant_rows(x)
    assert np.array_equal(xq.cpu().numpy(), o["q"])
    assert np.array_equal(sx.cpu().numpy().view(np.uint32), o["s"].view(np.uint32))
    mx, mean = rel_errors(oracle.to_f32(bits(y), 0), o["y"])
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)


@pytest.mark.parametrize("K,R", [(1280, 8), (1280, 16), (640, 16), (3072, 48), (640, 96), (1280, 128), (640, 160)])
def test_int8linear_any_rank(oracle, cuda, K, R):
    """The reference's Int8Linear takes a low-rank branch of any rank (deploy/int8_exec.py:371-407). Ranks the
    kernels do not take as they are run zero-padded, and above 64 with the up-projection after the GEMM (the
    reference's unfused order). The output is within tolerance of the oracle, the direct path equals the general
    path, and a routed call (gather + scatter into a canvas) matches the oracle's gathered rows."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    lin = make_linear(K, 640, R, True, seed=R)
    q = E.Int8Linear(lin, device=cuda)
    assert q.lr_A.shape == (K, R) and q.lr_B.shape == (R, 640)   # the reference's buffers keep their rank
    x = make_x(300, K, torch.bfloat16, seed=R).to(cuda)
    y = q(x)
    o = _oracle_module(oracle, q, x)
    mx, mean = rel_errors(oracle.to_f32(bits(y), 0), o["y"])
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
    E.DIRECT_CALLS = False
    try:
        y2 = q(x)
    finally:
        E.DIRECT_CALLS = True
    assert torch.equal(y, y2)

    g = torch.Generator().manual_seed(R)
    ri = torch.randperm(300, generator=g)[:77].to(torch.int32)
    ori = torch.randperm(500, generator=g)[:77].to(torch.int32)
    canvas = torch.randn(500, 640, generator=g).to(torch.bfloat16).to(cuda)
    before = canvas.clone()
    q(x, row_idx=ri.to(cuda), out=canvas, out_row_idx=ori.to(cuda))
    o = _oracle_module(oracle, q, x, row_idx=ri)
    rows = ori.long()
    mx, mean = rel_errors(oracle.to_f32(bits(canvas[rows.to(cuda)]), 0), o["y"])
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
    keep = torch.ones(500, dtype=torch.bool)
    keep[rows] = False
    assert torch.equal(canvas[keep.to(cuda)], before[keep.to(cuda)])


def test_int8linear_fp32_lowrank(oracle, cuda):
    """A 32-bit low-rank branch (rank 48): t from torch's fp32 product, zero-padded to the epilogue's rank 64,
    rounded to the activation type with lr_B. Within tolerance of the oracle run on the 16-bit-rounded factors."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    lin = make_linear(1280, 640, 0, True, seed=5)
    g = torch.Generator().manual_seed(5)
    A, B = torch.randn(1280, 48, generator=g) * 0.02, torch.randn(48, 640, generator=g) * 0.02
    q = E.Int8Linear(lin, device=cuda, lowrank=(A, B))
    assert q.lr_At is None and q.lr_Bt.shape == (640, 64)
    x = make_x(200, 1280, torch.bfloat16, seed=5).to(cuda)
    y = q(x)
    o = oracle.linear(bits(x), 0, q.weight_int8.cpu().numpy(), q.w_scale.cpu().numpy(), q.bias.cpu().numpy(), 0,
                      bits(A.to(torch.bfloat16)), bits(B.to(torch.bfloat16)))
    mx, mean = rel_errors(oracle.to_f32(bits(y), 0), o["y"])
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)


def test_int8linear_3d_and_views(cuda):
    """Leading dims are flattened and restored; a 3-D input gives the same result as its 2-D view
    (deploy/int8_exec.py:530-531); a row-slice input needs no copy."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    lin = make_linear(3072, 3072, 32, True)
    q = E.Int8Linear(lin, device=cuda)
    x = make_x(2048, 3072).to(cuda)
    assert torch.equal(q(x.reshape(8, 256, 3072)).reshape(2048, -1), q(x))
    big = make_x(64, 3072 + 12288).to(cuda)
    assert torch.equal(q(big[:, :3072]), q(big[:, :3072].contiguous()))


@pytest.mark.parametrize("N", [1280, 5120])
def test_sdxl_group32_module(oracle, cuda, N):
    """Config 3 at reduced M: group-32 weights, fp16 activations, no low rank; bit-exact against the oracle."""
    from pyraquant_amd import sdxl
    from pyraquant_amd.workloads import make_linear, make_x

    lin = make_linear(1280, N, 0, True)
    q = sdxl.SdxlInt8Linear(lin, device=cuda, group_size=32)
    assert q.w_scale.shape == (N, 40)
    x = make_x(2048, 1280, torch.float16).to(cuda)
    y = q(x)
    o = _oracle_module(oracle, q, x)
    assert np.array_equal(bits(y), o["out"])


def test_sdxl_narrow_n(oracle, cuda):
    """N = 640 (not a multiple of 256) runs on the same kernel (deploy/run_sdxl_latency.py:104-140)."""
    from pyraquant_amd import sdxl
    from pyraquant_amd.workloads import make_linear, make_x

    for K, N in sdxl.SDXL_TOKEN_SHAPES[:4]:
        lin = make_linear(K, N, 0, True)
        q = sdxl.SdxlInt8Linear(lin, device=cuda)
        x = make_x(154, K, torch.float16, seed=K).to(cuda)
        o = _oracle_module(oracle, q, x)
        assert np.array_equal(bits(q(x)), o["out"])


def test_routed_linear_small(oracle, cuda):
    """Gather + scatter at a reduced canvas: every routed row equals the oracle on the gathered rows, every
    other canvas row keeps the cached input bits."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.routing import routed_row_index
    from pyraquant_amd.workloads import make_linear, make_x

    H = W = 64
    sel = torch.zeros(4, 4, dtype=torch.bool)
    sel[0, 1] = sel[1, 1] = sel[1, 2] = sel[3, 3] = True
    rows = routed_row_index(sel, leaf_tokens=16, halo_tokens=2, token_hw=(H, W)).to(cuda)
    lin = make_linear(3072, 768, 32, True)
    q = E.Int8Linear(lin, device=cuda)
    x = make_x(H * W, 3072).to(cuda)
    cache = make_x(H * W, 768, seed=99).to(cuda)
    canvas = cache.clone()
    q(x, row_idx=rows, out=canvas, out_row_idx=rows)
    o = _oracle_module(oracle, q, x, rows)
    r = rows.cpu().numpy()
    got = oracle.to_f32(bits(canvas)[r], 0)
    mx, mean = rel_errors(got, o["y"])
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
    keep = np.setdiff1d(np.arange(H * W), r)
    assert np.array_equal(bits(canvas)[keep], bits(cache)[keep])


def test_routed_linear_c4_full(oracle, cuda):
    """Config 4 at full size: 33,316 gathered rows of the 65,536-row canvas. Routed output rows equal the
    dense Int8Linear output rows bit for bit (row-local math), untouched rows keep the cache, and the codes
    of the gather equal the oracle's."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x, routed_rows

    lin = make_linear(3072, 12288, 32, True)
    q = E.Int8Linear(lin, device=cuda)
    x = make_x(65536, 3072).to(cuda)
    rows = routed_rows(cuda)
    cache = torch.full((65536, 12288), 7.0, dtype=torch.bfloat16, device=cuda)
    canvas = cache.clone()
    q(x, row_idx=rows, out=canvas, out_row_idx=rows)
    dense = q(x)
    ri = rows.long()
    assert torch.equal(canvas[ri], dense[ri])
    mask = torch.ones(65536, dtype=torch.bool, device=cuda)
    mask[ri] = False
    assert bool((canvas[mask] == 7.0).all())
    xq, _ = E.quant_rows(x, rows)
    qo, _ = oracle.quant_rows(bits(x), 0, rows.cpu().numpy())
    assert np.array_equal(xq.cpu().numpy(), qo)


def test_reference_selftest(cuda):
    """The reference's own GPU self-test assertions (deploy/int8_exec.py:533-536) on the HIP kernels."""
    from pyraquant_amd import int8_exec as E

    rep = E.selftest_and_bench(Ms=(), iters=1)["selftest"]
    # The self-test's reference codes come from torch's GPU ops, whose `amax / 127` by a scalar is a reciprocal
    # multiply (1-ulp scale differences); its bar is a mismatch fraction <= 1e-4 (deploy/int8_exec.py:533).
    # Bit-exactness against the IEEE semantics is checked against the CPU oracle in test_quant_gpu.py.
    assert rep["act_quant_mismatch_frac"] <= 1e-4
    assert rep["3d_input_ok"]


def test_backend_api():
    from pyraquant_amd import int8_exec as E

    assert E.set_backend("triton") == "hip" and E.get_backend() == "hip"
    with pytest.raises(ValueError):
        E.set_backend("cublas")
    E.set_backend(E.DEFAULT_BACKEND)


@pytest.mark.parametrize("M,K,R,gather", [(4096, 3072, 32, False), (1000, 3072, 64, False), (777, 1280, 32, True),
                                          (129, 12288, 32, True), (64, 520, 32, False)])
def test_lowrank_down_dma_and_fallback(oracle, cuda, M, K, R, gather):
    """K % 64 == 0 and R <= 64 run the LDS-DMA kernel (also with a gather list holding duplicates and through a
    row-slice view); K = 520 runs the per-fragment kernel. Both within bf16 rounding of the float64 product."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_x

    rows = M + 37 if gather else M
    base = make_x(rows, K + 64, seed=K + R).to(cuda)
    x = base[:, 64:]                                            # row-slice view: ldx = K + 64
    g = torch.Generator().manual_seed(R + K)
    l1 = (torch.randn(K, R, generator=g) * 0.02).to(torch.bfloat16)
    idx = None
    if gather:
        idx = torch.randint(0, rows, (M,), generator=g, dtype=torch.int32)
        idx[:3] = torch.tensor([rows - 1, 0, 0], dtype=torch.int32)
    t = E.lowrank_down(x, l1.t().contiguous().to(cuda), None if idx is None else idx.to(cuda))
    xs = x.cpu()[idx.long()] if gather else x.cpu()
    ref64 = xs.double() @ l1.double()
    got = t.cpu().double()
    err = (got - ref64).abs() / ref64.abs().clamp_min(1e-3 * ref64.abs().max())
    assert float(err.max()) <= 1.5e-2, float(err.max())
    ref_bits = oracle.lowrank_down(bits(x.contiguous()), 0, bits(l1), None if idx is None else idx.numpy())
    mx, mean = rel_errors(oracle.to_f32(bits(t), 0), oracle.to_f32(ref_bits, 0))
    assert mx <= MAX_REL * 2 and mean <= MEAN_REL, (mx, mean)


@pytest.mark.parametrize("K,N,R,group,dtype,M", [(3072, 3072, 32, 0, torch.bfloat16, 2048),
                                                 (640, 640, 0, 0, torch.float16, 2048),
                                                 (1280, 1280, 0, 32, torch.float16, 154),
                                                 (3072, 12288, 32, 0, torch.bfloat16, 17),
                                                 (2560, 640, 32, 0, torch.float16, 1)])
def test_int8linear_direct_path_matches_general(cuda, K, N, R, group, dtype, M):
    """Int8Linear.forward's direct path (one workspace, raw pointers) returns the same bits as the general
    wrappers, for 2-D and 3-D inputs."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    lin = make_linear(K, N, R, True, dtype=dtype)
    q = E.Int8Linear(lin, device=cuda, group_size=group)
    x = make_x(M, K, dtype, seed=K + M).to(cuda)
    y_direct = q(x)
    y3 = q(x.reshape(1, M, K))
    E.DIRECT_CALLS = False
    try:
        y_general = q(x)
    finally:
        E.DIRECT_CALLS = True
    assert torch.equal(y_direct, y_general)
    assert torch.equal(y3.reshape(M, N), y_general)


def test_direct_path_follows_buffer_changes(cuda):
    """The direct path keeps the module's raw pointers per input dtype. Every way a buffer can change under it
    (edited in place, replaced, removed, added to a layer built without it, lr_At repacked, a module-wide cast)
    still gives the general path's bits on the next call."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    def both(q, x):
        y = q(x)
        E.DIRECT_CALLS = False
        try:
            y_general = q(x)
        finally:
            E.DIRECT_CALLS = True
        assert torch.equal(y, y_general)
        return y

    q = E.Int8Linear(make_linear(1280, 640, 32, True), device=cuda)
    x = make_x(300, 1280, seed=3).to(cuda)
    y0 = both(q, x)
    assert "_direct_plans" in q.__dict__                      # the direct path ran and kept its plan
    q.w_scale.mul_(2.0)                                         # in place: same pointer, new values
    y1 = both(q, x)
    assert not torch.equal(y1, y0)
    q.w_scale = q.w_scale * 0.5                                 # a new tensor in the buffer's place
    assert torch.equal(both(q, x), y0)
    q.bias = None                                               # the buffer removed
    y2 = both(q, x)
    assert not torch.equal(y2, y0)
    q.lr_At.mul_(0.0)                                           # in place: lr_At's fragment copy is repacked
    y3 = both(q, x)
    assert not torch.equal(y3, y2)
    q.half()                                                    # a cast: 16-bit operands, fp32 scales kept
    both(q, x.half())

    p = E.Int8Linear(make_linear(640, 640, 0, False), device=cuda)
    xb = make_x(64, 640, seed=4).to(cuda)
    z0 = both(p, xb)
    p.bias = torch.full((640,), 0.25, device=cuda)              # added to a layer built without one
    assert not torch.equal(both(p, xb), z0)


def test_int8linear_graph_replay(cuda):
    """A chain of Int8Linear forwards captured in a HIP graph (torch.cuda.graph) replays to the eager bits, replay
    after replay, with eager work and synchronisation between replays: the kernels allocate and clear nothing
    themselves, so a captured layer is launch-overhead free."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    a = E.Int8Linear(make_linear(1280, 5120, 32, True, dtype=torch.float16), device=cuda)
    b = E.Int8Linear(make_linear(5120, 1280, 0, True, dtype=torch.float16), device=cuda, group_size=32)
    x = make_x(2048, 1280, torch.float16).to(cuda)
    static_x = x.clone()
    ref = b(a(x))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            b(a(static_x))
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_y = b(a(static_x))
    for i in range(4):
        noise = make_x(2048, 1280, torch.float16, seed=100 + i).to(cuda)
        eager_other = b(a(noise))             # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_y, ref), i
        assert torch.equal(eager_other, b(a(noise))), i
    static_x.copy_(make_x(2048, 1280, torch.float16, seed=7).to(cuda))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(static_y, b(a(static_x)))


class _FluxLike(torch.nn.Module):
    """Module names as in FLUX's transformer: embedders, adaLN norms and proj_out stay bf16, token Linears convert."""

    def __init__(self):
        super().__init__()
        L = lambda k, n: torch.nn.Linear(k, n, dtype=torch.bfloat16)   # noqa: E731
        self.x_embedder = L(64, 128)
        self.proj_out = L(128, 64)
        self.transformer_blocks = torch.nn.ModuleList([torch.nn.Module()])
        blk = self.transformer_blocks[0]
        blk.attn = torch.nn.Module()
        blk.attn.to_q = L(128, 128)
        blk.norm1 = torch.nn.Module()
        blk.norm1.linear = L(128, 768)
        blk.ff = torch.nn.Module()
        blk.ff.proj = L(128, 512)


def test_module_conversion_and_warmup(cuda):
    """convert_linears_to_int8 with the reference's default whitelist (deploy/int8_exec.py:415-445): the token
    Linears become Int8Linear, whose outputs equal a directly built Int8Linear's; embedders, adaLN and proj_out stay
    bf16; the statistics dict carries the reference's keys. warm_kernels runs every FLUX shape. The SDXL twins
    (deploy/run_sdxl_latency.py:159-298) convert with their fp16 whitelist, per channel and group-32, and the
    direct-launch helpers give the general wrappers' bits."""
    import copy

    from pyraquant_amd import int8_exec as E
    from pyraquant_amd import sdxl

    m = _FluxLike().to(cuda)
    ref_q = copy.deepcopy(m.transformer_blocks[0].attn.to_q)
    rep = E.convert_linears_to_int8(m, device=cuda)
    assert set(rep) == {"n_int8_linear", "n_bf16_linear_kept", "params_int8", "params_bf16_linear_kept",
                        "bf16_kept_names", "int8_weight_gib", "bf16_equiv_gib"}
    assert rep["n_int8_linear"] == 2 and rep["n_bf16_linear_kept"] == 3
    assert sorted(rep["bf16_kept_names"]) == ["proj_out", "transformer_blocks.0.norm1.linear", "x_embedder"]
    assert rep["params_int8"] == 128 * 128 + 128 * 512
    blk = m.transformer_blocks[0]
    assert isinstance(blk.attn.to_q, E.Int8Linear) and isinstance(blk.ff.proj, E.Int8Linear)
    assert type(blk.norm1.linear) is torch.nn.Linear and type(m.x_embedder) is torch.nn.Linear
    x = torch.randn(50, 128, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(cuda)
    with torch.no_grad():
        assert torch.equal(blk.attn.to_q(x), E.Int8Linear(ref_q, device=cuda)(x))
    E.warm_kernels(device=cuda)

    u = torch.nn.Module()
    u.time_embedding = torch.nn.Module()
    u.time_embedding.linear_1 = torch.nn.Linear(320, 1280, dtype=torch.float16)
    u.down = torch.nn.Module()
    u.down.to_q = torch.nn.Linear(640, 640, dtype=torch.float16)
    u.down.ff = torch.nn.Linear(640, 2560, dtype=torch.float16)
    u = u.to(cuda)
    u32 = copy.deepcopy(u)
    rep = sdxl.convert_unet_linears_to_int8(u, device=cuda)
    assert rep["n_int8_linear"] == 2 and rep["fp16_kept_names"] == ["time_embedding.linear_1"]
    assert rep["shapes_KxN"] == {"640x2560": 1, "640x640": 1}
    rep32 = sdxl.convert_unet_linears_to_int8(u32, device=cuda, group_size=32)
    assert isinstance(u32.down.ff, sdxl.SdxlInt8Linear) and u32.down.ff.group_size == 32 and rep32["n_int8_linear"] == 2
    xs = torch.randn(154, 640, generator=torch.Generator().manual_seed(3)).to(torch.float16).to(cuda)
    with torch.no_grad():
        y, y32 = u.down.ff(xs), u32.down.ff(xs)
    assert y.shape == y32.shape == (154, 2560) and torch.isfinite(y32.float()).all()
    rel = float((y32.float() - y.float()).norm() / y.float().norm())
    assert rel < 2e-2, rel                    # group-32 and per-channel RTN of the same weights
    sdxl.warm_sdxl_kernels(device=cuda)
    xq, sx = sdxl.fast_quant_rows(xs)
    xq2, sx2 = E.quant_rows(xs)
    assert torch.equal(xq, xq2) and torch.equal(sx, sx2)
    q = u.down.to_q
    assert torch.equal(sdxl.fast_gemm_fused(xq, sx, q.weight_int8, q.w_scale, q.bias, torch.float16),
                       E.int8_gemm_fused(xq, sx, q.weight_int8, q.w_scale, q.bias, torch.float16))


def test_int8linear_module_cast(oracle, cuda):
    """A module-wide cast (.to(torch.bfloat16), .half()) keeps the fp32 scale and bias buffers fp32, so the kernels,
    which read them through raw pointers, never see 16-bit scales: the bf16 outputs are unchanged bit for bit, and an
    fp16 call after .half() equals a module built in fp16 from the same weights (codes / scales exact against the
    oracle, outputs within tolerance)."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    for group in (0, 32):
        lin = make_linear(1280, 640, 0 if group else 32, True)
        q = E.Int8Linear(lin, device=cuda, group_size=group)
        x = make_x(200, 1280, seed=group + 1).to(cuda)
        y = q(x)
        q.to(torch.bfloat16)
        for name in ("w_scale", "bias") + (("w_scale_gn",) if group else ()):
            assert getattr(q, name).dtype == torch.float32, name
        assert torch.equal(q(x), y)
        q.half()
        assert q.w_scale.dtype == torch.float32 and q.bias.dtype == torch.float32
        xh = x.half()
        yh = q(xh)
        E.DIRECT_CALLS = False
        try:
            assert torch.equal(q(xh), yh)          # the general path gives the same bits
        finally:
            E.DIRECT_CALLS = True
        o = _oracle_module(oracle, q, xh)
        if group:
            assert np.array_equal(bits(yh), o["out"])
        else:
            mx, mean = rel_errors(oracle.to_f32(bits(yh), 1), o["y"])
            assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)


def test_int8linear_under_inference_mode(cuda):
    """Int8Linear built and run inside torch.inference_mode(): inference tensors carry no version counter, so the
    fragment-order copy of lr_At is keyed on its storage, dtype and device there. A rank-32 layer (whose quantizer
    reads that copy) built and called under inference_mode gives the bits of the same layer built outside it, and
    so does a module conversion under inference_mode."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    lin = make_linear(3072, 1024, 32, True, seed=21)
    x = make_x(300, 3072, seed=22).to(cuda)
    ref = E.Int8Linear(lin, device=cuda)(x)
    with torch.inference_mode():
        q = E.Int8Linear(lin, device=cuda)
        assert q.lr_At.is_inference() and q.lr_At_frag is not None
        y = q(x)
        assert torch.equal(q(x), y)                  # the cached fragment copy is reused
        model = torch.nn.Sequential(make_linear(3072, 1024, 32, True, seed=21)).to(cuda)
        E.convert_linears_to_int8(model, device=cuda)
        y2 = model(x)
    assert torch.equal(y, ref)
    assert torch.equal(y2, ref)
