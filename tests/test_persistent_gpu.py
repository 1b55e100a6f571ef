"""The persistent 256 x 256 GEMM (one workgroup per CU looping over tiles). With a scheduling buffer (the caller's:
the GEMM entries' `sched`, which the Python layer keeps per stream, or the slice of pq_int8_linear's workspace that
its quantizer kernel zeroes) the workgroups claim tiles from per-XCD counters and the last one out zeroes them
again; without one (a stream under graph capture in the Python layer) the tiles follow a fixed per-workgroup share.
Every schedule must produce every tile exactly as the one-tile-per-workgroup kernels do:
* consecutive launches on one stream, each into a NaN-filled output (a counter left non-zero by a launch would make
  the next one skip tiles);
* two streams running large GEMMs at the same time (each stream has its own buffer);
* a captured graph replayed between eager launches (the graph keeps the fixed share);
* the single-call layer with a freshly allocated workspace whose bytes hold garbage, eagerly and replayed from a
  graph (its quantizer kernel zeroes the counters each time);
* the allocation-free layer call against the workspace call at a size that runs persistent blocks.
The reference is the same product computed in 256-row slices, whose few blocks run one tile per workgroup with the
same per-element epilogue arithmetic, so the results agree bit for bit."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

# 256 x 256 blocks: 16 x 32 = 512 tiles, more than the 256 CUs (persistent); 128 x 256 blocks: 1024 (large tiles)
M, N, K = 4096, 8192, 512
# ragged: 17 x 31 = 527 tiles (527 % 8 = 7: the XCD lists differ in length by one), the last tile column 0.75 wide
RAGGED = (4352, 7936, 384)


def _problem(cuda, seed, lr, shape=(M, N, K)):
    M, N, K = shape
    from pyraquant_amd import int8_exec as E

    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s_row = (torch.rand(M, generator=g) * 0.05 + 1e-3).to(cuda)
    s_w = (torch.rand(N, generator=g) * 2e-4 + 1e-5).to(cuda)
    bias = (torch.randn(N, generator=g) * 0.01).to(cuda)
    t = l2t = None
    if lr:
        t = (torch.randn(M, lr, generator=g) * 0.5).to(torch.bfloat16).to(cuda)
        l2t = (torch.randn(N, lr, generator=g) * 0.02).to(torch.bfloat16).to(cuda)
    return dict(ap=E.pack_k64(a.to(cuda)), wp=E.pack_k64(w.to(cuda)), s_row=s_row, s_w=s_w, bias=bias, t=t, l2t=l2t,
                shape=(M, N, K))


def _run(P, out):
    from pyraquant_amd import int8_exec as E

    M, N, K = P["shape"]
    return E.int8_gemm_packed(P["ap"], P["s_row"], P["wp"], P["s_w"], P["bias"], M, N, K, torch.bfloat16,
                              t=P["t"], l2t=P["l2t"], out=out)


def _sliced(P):
    """The reference: 256 rows at a time (rows r0 .. r0 + 255 of the flat packed operand are its bytes
    [r0 K, (r0 + 256) K), r0 a multiple of 16)."""
    from pyraquant_amd import int8_exec as E

    M, N, K = P["shape"]
    out = torch.empty((M, N), dtype=torch.bfloat16, device=P["ap"].device)
    for r0 in range(0, M, 256):
        t = None if P["t"] is None else P["t"][r0:r0 + 256]
        E.int8_gemm_packed(P["ap"][r0 * K:(r0 + 256) * K], P["s_row"][r0:], P["wp"], P["s_w"], P["bias"], 256, N, K,
                           torch.bfloat16, t=t, l2t=P["l2t"], out=out[r0:r0 + 256])
    return out


@pytest.mark.parametrize("lr,shape", [(0, (M, N, K)), (32, (M, N, K)), (32, RAGGED)])
def test_consecutive_launches_write_every_tile(cuda, lr, shape):
    P = _problem(cuda, 11 + lr, lr, shape)
    ref = _sliced(P)
    out = torch.empty(shape[:2], dtype=torch.bfloat16, device=cuda)
    for i in range(5):
        out.fill_(float("nan"))
        _run(P, out)
        torch.cuda.synchronize()
        print(f"[persistent] lr={lr} shape={shape} launch {i}", flush=True)
        assert not torch.isnan(out).any(), f"launch {i}: tiles left unwritten"
        assert torch.equal(out, ref), f"launch {i}"


def test_two_streams_at_once(cuda):
    Pa, Pb = _problem(cuda, 21, 32), _problem(cuda, 22, 0)
    ref_a, ref_b = _sliced(Pa), _sliced(Pb)
    outs_a = [torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=cuda) for _ in range(3)]
    outs_b = [torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=cuda) for _ in range(3)]
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for i in range(3):               # enqueued back to back on both streams, no synchronisation in between
        with torch.cuda.stream(s1):
            _run(Pa, outs_a[i])
        with torch.cuda.stream(s2):
            _run(Pb, outs_b[i])
    torch.cuda.synchronize()
    for i in range(3):
        print(f"[persistent] two streams, launch {i}", flush=True)
        assert torch.equal(outs_a[i], ref_a), f"stream 1, launch {i}"
        assert torch.equal(outs_b[i], ref_b), f"stream 2, launch {i}"


def test_graph_replay_between_eager_launches(cuda):
    P = _problem(cuda, 31, 32)
    ref = _sliced(P)
    out_g = torch.empty((M, N), dtype=torch.bfloat16, device=cuda)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):    # warm-up off the capturing stream, as torch requires
        _run(P, out_g)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _run(P, out_g)
    out_e = torch.empty_like(out_g)
    for i in range(3):
        out_g.fill_(float("nan"))
        out_e.fill_(float("nan"))
        g.replay()
        _run(P, out_e)               # an eager launch (per-stream buffer) right behind the replay
        torch.cuda.synchronize()
        print(f"[persistent] graph replay {i}", flush=True)
        assert torch.equal(out_g, ref), f"replay {i}"
        assert torch.equal(out_e, ref), f"eager launch {i}"


def test_noalloc_layer_at_a_persistent_size(cuda):
    """pq_int8_linear_noalloc (fixed shares, nothing allocated) against pq_int8_linear (scheduling buffer) on a
    rank-32 layer large enough for persistent blocks."""
    from pyraquant_amd import _lib
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    L = _lib.load()
    q = E.Int8Linear(make_linear(3072, 8192, 32, True, seed=5, dtype=torch.bfloat16), device=cuda)
    x = make_x(4096, 3072, torch.bfloat16, seed=6, device=cuda)
    Mx, Nq = x.shape[0], q.out_features
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    args = [p(x), _lib.dtype_code(x.dtype), Mx, 3072, x.stride(0), p(q.weight_packed), p(q._scale_k()), 0, p(q.bias),
            p(q.lr_At), p(q._lr_frag()), 32, p(q.lr_Bt), q.lr_Bt.shape[1]]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws = torch.empty(L.pq_int8_linear_workspace_size(Mx, 3072, 32), dtype=torch.uint8, device=cuda)
    y_ws = torch.full((Mx, Nq), float("nan"), dtype=x.dtype, device=cuda)
    y_na = torch.full((Mx, Nq), float("nan"), dtype=x.dtype, device=cuda)
    for i in range(2):
        _lib.check(L.pq_int8_linear(*args, ctypes.c_void_p(y_ws.data_ptr()), Nq, Nq, ctypes.c_void_p(ws.data_ptr()),
                                    ws.numel(), stream), "pq_int8_linear")
        _lib.check(L.pq_int8_linear_noalloc(*args, ctypes.c_void_p(y_na.data_ptr()), Nq, Nq, stream),
                   "pq_int8_linear_noalloc")
        torch.cuda.synchronize()
        print(f"[persistent] noalloc layer, call {i}", flush=True)
        assert not torch.isnan(y_na).any() and not torch.isnan(y_ws).any()
        assert torch.equal(y_na, y_ws), f"call {i}"
        y_ws.fill_(float("nan"))
        y_na.fill_(float("nan"))


def test_layer_call_fresh_workspace_and_graph(cuda):
    """pq_int8_linear on a workspace fresh from torch.empty, filled with garbage first (a scheduling buffer left as
    found would start the claims past the end and leave tiles unwritten): eager calls into NaN-filled outputs, then a
    captured call replayed three times with an eager call on another workspace between the replays. Every output
    equals the layer computed in 256-row slices."""
    from pyraquant_amd import _lib
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    L = _lib.load()
    Mx, Kx, Nx = 4096, 3072, 8192            # 16 x 32 = 512 blocks of 256 x 256: persistent
    q = E.Int8Linear(make_linear(Kx, Nx, 32, True, seed=15, dtype=torch.bfloat16), device=cuda)
    x = make_x(Mx, Kx, torch.bfloat16, seed=16, device=cuda)
    ref = torch.cat([q(x[r0:r0 + 256]) for r0 in range(0, Mx, 256)])
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    size = L.pq_int8_linear_workspace_size(Mx, Kx, 32)

    def call(ws, y):
        args = [p(x), _lib.dtype_code(x.dtype), Mx, Kx, x.stride(0), p(q.weight_packed), p(q._scale_k()), 0, p(q.bias),
                p(q.lr_At), p(q._lr_frag()), 32, p(q.lr_Bt), q.lr_Bt.shape[1], p(y), Nx, Nx, p(ws), ws.numel(),
                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)]
        _lib.check(L.pq_int8_linear(*args), "pq_int8_linear")

    for i, fill in enumerate((0xFF, 0x5A, 0x01)):
        ws = torch.empty(size, dtype=torch.uint8, device=cuda)
        ws.fill_(fill)
        y = torch.full((Mx, Nx), float("nan"), dtype=x.dtype, device=cuda)
        call(ws, y)
        torch.cuda.synchronize()
        print(f"[persistent] layer call, fresh workspace filled with {fill:#x}", flush=True)
        assert torch.equal(y, ref), f"eager call {i}"
    ws_g = torch.full((size,), 0x77, dtype=torch.uint8, device=cuda)
    ws_e = torch.empty(size, dtype=torch.uint8, device=cuda)
    y_g = torch.empty((Mx, Nx), dtype=x.dtype, device=cuda)
    y_e = torch.empty_like(y_g)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(ws_g, y_g)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(ws_g, y_g)
    for i in range(3):
        y_g.fill_(float("nan"))
        y_e.fill_(float("nan"))
        ws_e.fill_(0xC3)
        g.replay()
        call(ws_e, y_e)
        torch.cuda.synchronize()
        print(f"[persistent] layer call, graph replay {i}", flush=True)
        assert torch.equal(y_g, ref), f"replay {i}"
        assert torch.equal(y_e, ref), f"eager call beside replay {i}"
