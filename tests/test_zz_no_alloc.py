"""pq_int8_linear_noalloc (the allocation-free layer call) against pq_int8_linear (the same layer over a caller
workspace), through the C ABI: bit-identical outputs on consecutive calls, a smaller input after a larger one and two
different layers interleaved (the device array keeps the previous call's contents, which must not matter), and the
refusal of a layer whose staging exceeds the array, before any work."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _layer(cuda, K, N, R, group, dtype, seed):
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear

    return E.Int8Linear(make_linear(K, N, R, True, seed=seed, dtype=dtype), device=cuda, group_size=group)


def _args(q, x):
    from pyraquant_amd import _lib

    R = 0 if q.lr_At is None else q.lr_At.shape[0]
    Re = 0 if q.lr_Bt is None else q.lr_Bt.shape[1]
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    return [p(x), _lib.dtype_code(x.dtype), x.shape[0], x.shape[1], x.stride(0), p(q.weight_packed), p(q._scale_k()),
            q.group_size, p(q.bias), p(q.lr_At), p(q._lr_frag()), R, p(q.lr_Bt), Re]


def _run_both(L, q, x):
    from pyraquant_amd import _lib

    M, N = x.shape[0], q.out_features
    R = 0 if q.lr_At is None else q.lr_At.shape[0]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws = torch.empty(L.pq_int8_linear_workspace_size(M, q.in_features, R), dtype=torch.uint8, device=x.device)
    y_ws = torch.full((M, N), float("nan"), dtype=x.dtype, device=x.device)
    y_na = torch.full((M, N), float("nan"), dtype=x.dtype, device=x.device)
    _lib.check(L.pq_int8_linear(*_args(q, x), ctypes.c_void_p(y_ws.data_ptr()), N, N, ctypes.c_void_p(ws.data_ptr()),
                                ws.numel(), stream), "pq_int8_linear")
    _lib.check(L.pq_int8_linear_noalloc(*_args(q, x), ctypes.c_void_p(y_na.data_ptr()), N, N, stream),
               "pq_int8_linear_noalloc")
    return y_ws, y_na


def test_noalloc_matches_workspace_entry(cuda):
    from pyraquant_amd import _lib
    from pyraquant_amd.workloads import make_x

    L = _lib.load()
    assert L.pq_int8_linear_noalloc_max_bytes() == 64 << 20
    lr = _layer(cuda, 3072, 3072, 32, 0, torch.bfloat16, seed=1)          # FLUX 1K attention projection, rank 32
    g32 = _layer(cuda, 1280, 5120, 0, 32, torch.float16, seed=2)          # SDXL group-32 MLP up
    cases = [(lr, 4096, torch.bfloat16), (g32, 2048, torch.float16), (lr, 1000, torch.bfloat16),
             (g32, 77, torch.float16)]
    for i, (q, M, dt) in enumerate(cases):
        x = make_x(M, q.in_features, dt, seed=10 + i, device=cuda)
        y_ws, y_na = _run_both(L, q, x)
        torch.cuda.synchronize()
        print(f"[no_alloc] case {i}: M={M} K={q.in_features} N={q.out_features} group={q.group_size}", flush=True)
        assert not torch.isnan(y_na).any(), "every output written"
        assert torch.equal(y_na, y_ws), f"case {i}: allocation-free output differs from the workspace entry's"
        assert torch.equal(y_na, q(x)), f"case {i}: differs from Int8Linear.forward"


def test_noalloc_refuses_oversized_layer(cuda):
    """FLUX's 4K-stage layer (M = 65536, K = 3072, rank 32) needs 201 MB of staging: refused with PQ_ESHAPE and a
    message naming the limit; the output is left untouched."""
    from pyraquant_amd import _lib

    L = _lib.load()
    q = _layer(cuda, 3072, 3072, 32, 0, torch.bfloat16, seed=3)
    x = torch.zeros(65536, 3072, dtype=torch.bfloat16, device=cuda)
    y = torch.full((65536, 3072), 7.0, dtype=torch.bfloat16, device=cuda)
    st = L.pq_int8_linear_noalloc(*_args(q, x), ctypes.c_void_p(y.data_ptr()), 3072, 3072,
                                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == _lib.PQ_ESHAPE
    assert b"scratch" in L.pq_last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
