"""INT8 deployment executor for MI355X (gfx950): the `Int8Linear` module API of PyraQuant's
``deploy/int8_exec.py``, backed by hand-written HIP kernels in ``libpqint8.so``.

Drop-in surface (same names, argument meaning and error types as deploy/int8_exec.py):
  BACKENDS / DEFAULT_BACKEND / BACKEND / set_backend / get_backend           (:58-74)
  quant_rows(x2) -> (int8 [M,K], fp32 [M])                                   (:216-230)
  dequant_epilogue(acc, s_row, s_col, bias, out_dtype)                       (:233-243)
  int8_linear_2d(x2, w_int8, w_scale, bias, backend=None)                    (:246-261)
  int8_gemm_fused(xq, s_row, w_int8, w_scale, bias, out_dtype)               (:202-212)
  int8_gemm_lr(xq, s_row, w_i8, w_scale, bias, t, lb, out_dtype)             (:327-336)
  LOWRANK_A_ATTR / LOWRANK_B_ATTR, Int8Linear(lin, device=None, lowrank=None) (:341-411)
  is_bf16_whitelisted, convert_linears_to_int8, warm_kernels                 (:415-474)
  FLUX_TOKEN_SHAPES, _bench, selftest_and_bench, CLI                         (:478-588)
Additions for the MI355X build: the routed row gather (``row_idx``) and scatter (``out_row_idx``),
group-32 weight scales (``group_size=32``), the HIP low-rank down-projection ``lowrank_down``, the
int32 accumulator entry ``int8_gemm_i32``, and the packed K64 layer path (``pack_k64``, ``quant_rows_packed``,
``int8_gemm_packed``) that Int8Linear.forward runs on.

There is one backend, "hip" (the reference's fused "triton" path; the name "triton" is accepted as an alias
so existing ``--int8-backend triton`` flags keep working). The reference's "cublas" path (an int32 round
trip through torch._int_mm) is not provided: set_backend("cublas") raises ValueError.

Every kernel runs on the caller's current stream; nothing synchronises. CPU tensors raise AssertionError
(as the reference's ``assert x2.is_cuda``); a missing library raises at the first call.
"""
from __future__ import annotations

import time
from typing import Callable, Dict, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib

# --------------------------------------------------------------------------- backend selection
BACKENDS = ("hip",)
DEFAULT_BACKEND = "hip"
BACKEND = DEFAULT_BACKEND
_BACKEND_ALIASES = {"hip": "hip", "triton": "hip"}


def set_backend(name: str) -> str:
    """Select the INT8 GEMM backend (deploy/int8_exec.py:64-70). Only the fused HIP path exists."""
    global BACKEND
    if name not in _BACKEND_ALIASES:
        raise ValueError(f"unknown INT8 backend {name!r} (expected one of {BACKENDS}; 'triton' is an alias of 'hip')")
    BACKEND = _BACKEND_ALIASES[name]
    return BACKEND


def get_backend() -> str:
    return BACKEND


# --------------------------------------------------------------------------- kernel wrappers
def _check_cuda(*ts):
    for t in ts:
        if t is not None:
            assert t.is_cuda, "the INT8 executor runs on the GPU only (got a CPU tensor)"


def _row_index(idx: Optional[torch.Tensor], device) -> Optional[torch.Tensor]:
    if idx is None:
        return None
    assert idx.dtype == torch.int32 and idx.dim() == 1 and idx.is_contiguous(), "row index must be contiguous int32 [M]"
    assert idx.device == device, "row index must be on the input's device"
    return idx


def quant_rows(x2: torch.Tensor, row_idx: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """x2 [rows, K] bf16/fp16 -> (int8 [M, K], fp32 scale [M]), per-row symmetric absmax
    (deploy/int8_exec.py:216-230). Row-slice views pass without a copy (the kernel takes the row stride).
    ``row_idx`` (int32 [M]): fused routed gather, output row m quantizes x2[row_idx[m]]; an entry outside
    [0, rows) quantizes a row of zeros (codes 0, scale fl(1e-8)/127) where torch's indexing would raise."""
    assert x2.dim() == 2 and x2.is_cuda
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    rows, K = x2.shape
    ri = _row_index(row_idx, x2.device)
    M = rows if ri is None else ri.shape[0]
    q = torch.empty((M, K), dtype=torch.int8, device=x2.device)
    s = torch.empty((M,), dtype=torch.float32, device=x2.device)
    L = _lib.load()
    _lib.check(L.pq_quant_rows(_lib.ptr(x2), _lib.dtype_code(x2.dtype), M, K, x2.stride(0), rows, _lib.ptr(ri),
                               _lib.ptr(q), _lib.ptr(s), _lib.stream_of(x2.device)), "quant_rows")
    return q, s


def lowrank_down(x2: torch.Tensor, lr_At: torch.Tensor, row_idx: Optional[torch.Tensor] = None) -> torch.Tensor:
    """t = x2[rows] @ lr_A on the GPU (deploy/int8_exec.py:390), fp32 accumulation, 16-bit result.
    ``lr_At`` is lr_A transposed, [R, K] contiguous, same dtype as x2."""
    assert x2.dim() == 2 and x2.is_cuda and lr_At.is_cuda
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    assert lr_At.dtype == x2.dtype, "x2 and lr_A must share a dtype (cast x2 first, as the reference does)"
    assert lr_At.is_contiguous() and lr_At.shape[1] == x2.shape[1], "lr_At must be [R, K] contiguous"
    rows, K = x2.shape
    R = lr_At.shape[0]
    ri = _row_index(row_idx, x2.device)
    M = rows if ri is None else ri.shape[0]
    t = torch.empty((M, R), dtype=x2.dtype, device=x2.device)
    L = _lib.load()
    _lib.check(L.pq_lowrank_down(_lib.ptr(x2), _lib.dtype_code(x2.dtype), M, K, x2.stride(0), rows, _lib.ptr(ri),
                                 _lib.ptr(lr_At), R, _lib.ptr(t), R, _lib.stream_of(x2.device)), "lowrank_down")
    return t


def dequant_epilogue(acc: torch.Tensor, s_row: torch.Tensor, s_col: torch.Tensor,
                     bias: Optional[torch.Tensor], out_dtype: torch.dtype) -> torch.Tensor:
    """int32 [M,N] * s_row[M] * s_col[N] (+bias[N]) -> bf16/fp16 (deploy/int8_exec.py:233-243)."""
    assert acc.dtype == torch.int32 and acc.is_contiguous()
    _check_cuda(acc, s_row, s_col, bias)
    M, N = acc.shape
    s_row, s_col = s_row.float().contiguous(), s_col.float().contiguous()
    assert s_row.numel() >= M and s_col.numel() >= N, (s_row.numel(), s_col.numel(), M, N)
    out = torch.empty((M, N), dtype=out_dtype, device=acc.device)
    L = _lib.load()
    _lib.check(L.pq_dequant_epilogue(_lib.ptr(acc), _lib.ptr(s_row), _lib.ptr(s_col),
                                     _lib.ptr(None if bias is None else bias.float().contiguous()), _lib.ptr(out), N,
                                     _lib.dtype_code(out_dtype), M, N, _lib.stream_of(acc.device)), "dequant_epilogue")
    return out


# Scheduling buffers of the GEMM's persistent blocks (pq_int8_gemm's `sched`): 9 int32 counters per (device, stream),
# zeroed once by torch and left zeroed by every launch, so the launches ordered on one stream share it. A stream
# being captured into a graph gets none (the graph's launches take fixed shares), so a replay never shares a buffer
# with eager launches on that stream.
_SCHED: Dict[Tuple[int, int], torch.Tensor] = {}


def _sched_buffer(dev: torch.device) -> Optional[torch.Tensor]:
    if torch.cuda.is_current_stream_capturing():
        return None
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (idx, _raw_stream(dev))
    buf = _SCHED.get(key)
    if buf is None:
        buf = torch.zeros(16, dtype=torch.int32, device=torch.device("cuda", idx))
        _SCHED[key] = buf
    return buf


def _gemm(xq: torch.Tensor, s_row: torch.Tensor, w_int8: torch.Tensor, w_scale_k: torch.Tensor, group: int,
          bias: Optional[torch.Tensor], t: Optional[torch.Tensor], l2t: Optional[torch.Tensor],
          out_dtype: torch.dtype, out: Optional[torch.Tensor] = None,
          out_row_idx: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Core launcher of pq_int8_gemm. w_scale_k is in the kernel layout ([N] or [K/32, N])."""
    assert xq.dim() == 2 and xq.dtype == torch.int8 and w_int8.dtype == torch.int8
    _check_cuda(xq, s_row, w_int8, w_scale_k, bias, t, l2t, out, out_row_idx)
    M, K = xq.shape
    N = w_int8.shape[0]
    assert w_int8.shape[1] == K, (tuple(xq.shape), tuple(w_int8.shape))
    assert xq.stride(1) == 1 and w_int8.stride(1) == 1
    assert s_row.dtype == torch.float32 and s_row.is_contiguous() and s_row.numel() >= M
    assert w_scale_k.dtype == torch.float32 and w_scale_k.is_contiguous()
    assert w_scale_k.numel() == (N * K // 32 if group else N), (tuple(w_scale_k.shape), N, K, group)
    if bias is not None:
        assert bias.dtype == torch.float32 and bias.is_contiguous() and bias.numel() == N
    ori = _row_index(out_row_idx, xq.device)
    if ori is not None:
        assert ori.shape[0] == M and out is not None, "a scatter needs the destination canvas (out=)"
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=xq.device)
    assert out.dtype == out_dtype and out.dim() == 2 and out.shape[1] == N and out.stride(1) == 1
    if ori is None:
        assert out.shape[0] >= M
    lr_code, R, ldt = 0, 0, 0
    if t is not None:
        assert l2t is not None and t.dtype == l2t.dtype and t.stride(1) == 1 and l2t.is_contiguous()
        assert t.dim() == 2 and t.shape[0] >= M, (tuple(t.shape), M)
        R = t.shape[1]
        assert l2t.shape == (N, R), (tuple(l2t.shape), (N, R))
        lr_code, ldt = _lib.dtype_code(t.dtype), t.stride(0)
    L = _lib.load()
    _lib.check(L.pq_int8_gemm(_lib.ptr(xq), xq.stride(0), _lib.ptr(w_int8), w_int8.stride(0), _lib.ptr(s_row),
                              _lib.ptr(w_scale_k), group, _lib.ptr(bias), _lib.ptr(t), ldt, _lib.ptr(l2t), R, lr_code,
                              _lib.ptr(out), out.stride(0), _lib.dtype_code(out_dtype), _lib.ptr(ori), out.shape[0],
                              M, N, K, _lib.ptr(_sched_buffer(xq.device)), _lib.stream_of(xq.device)), "int8_gemm")
    return out


def int8_gemm_fused(xq: torch.Tensor, s_row: torch.Tensor, w_int8: torch.Tensor, w_scale: torch.Tensor,
                    bias: Optional[torch.Tensor], out_dtype: torch.dtype, *, out: Optional[torch.Tensor] = None,
                    out_row_idx: Optional[torch.Tensor] = None) -> torch.Tensor:
    """C = (xq @ w_int8^T) * s_row * w_scale (+bias) -> out_dtype in one kernel (deploy/int8_exec.py:202-212).
    Requires K % 64 == 0 and N % 64 == 0 (the reference asserts N % 256 == 0; N = 640 of SDXL also runs here).
    ``out``/``out_row_idx``: write row m into out[out_row_idx[m]] (routed scatter; other rows untouched, and a row
    whose index lies outside [0, out.shape[0]) is not written)."""
    assert xq.shape[1] % 64 == 0 and w_int8.shape[0] % 64 == 0, (xq.shape[1], w_int8.shape[0])
    return _gemm(xq, s_row, w_int8, w_scale, 0, bias, None, None, out_dtype, out, out_row_idx)


def int8_gemm_lr(xq, s_row, w_i8, w_scale, bias, t, lb, out_dtype, *, lb_t: Optional[torch.Tensor] = None,
                 out: Optional[torch.Tensor] = None, out_row_idx: Optional[torch.Tensor] = None):
    """int8_gemm_fused + the low-rank up-projection t @ lb in the epilogue (deploy/int8_exec.py:327-336);
    order: acc*scales, + t@lb, + bias. ``lb`` is lr_B [R, N]; pass ``lb_t`` = lb^T [N, R] contiguous to
    skip the transpose (Int8Linear keeps it as a buffer)."""
    if lb_t is None:
        lb_t = lb.t().contiguous()
    assert xq.shape[1] % 64 == 0 and w_i8.shape[0] % 64 == 0, (xq.shape[1], w_i8.shape[0])
    return _gemm(xq, s_row, w_i8, w_scale, 0, bias, t, lb_t, out_dtype, out, out_row_idx)


def int8_gemm_i32(xq: torch.Tensor, w_int8: torch.Tensor) -> torch.Tensor:
    """Exact int32 accumulator xq @ w_int8^T with the same MFMA kernel body (torch._int_mm's role,
    deploy/int8_exec.py:259)."""
    assert xq.dim() == 2 and xq.dtype == torch.int8 and w_int8.dtype == torch.int8
    _check_cuda(xq, w_int8)
    M, K = xq.shape
    N = w_int8.shape[0]
    c = torch.empty((M, N), dtype=torch.int32, device=xq.device)
    L = _lib.load()
    _lib.check(L.pq_int8_gemm_i32(_lib.ptr(xq), xq.stride(0), _lib.ptr(w_int8), w_int8.stride(0), _lib.ptr(c), N,
                                  M, N, K, _lib.stream_of(xq.device)), "int8_gemm_i32")
    return c


# --------------------------------------------------------------------------- packed K64 layer path
# Int8Linear.forward's direct path (one workspace allocation, raw pointers); False routes every call through the
# general wrappers (same kernels, same bits).
DIRECT_CALLS = True
_DIRECT_DTYPES = {torch.bfloat16: _lib.PQ_BF16, torch.float16: _lib.PQ_F16}


def _raw_stream(dev: torch.device) -> int:
    """The current HIP stream of `dev` as an integer handle."""
    return torch._C._cuda_getCurrentRawStream(dev.index if dev.index is not None else torch.cuda.current_device())


def packed_rows(rows: int) -> int:
    """Rows of a packed K64 buffer holding `rows` rows (a multiple of 16)."""
    return (rows + 15) // 16 * 16


def pack_k64(w_int8: torch.Tensor) -> torch.Tensor:
    """Row-major int8 [R, K] -> packed K64 layout (flat int8 tensor of packed_rows(R) * K bytes), pq_pack_k64.
    Int8Linear packs its weights once at conversion."""
    assert w_int8.dim() == 2 and w_int8.dtype == torch.int8 and w_int8.is_cuda and w_int8.stride(1) == 1
    R, K = w_int8.shape
    assert K % 64 == 0, K
    out = torch.empty((packed_rows(R) * K,), dtype=torch.int8, device=w_int8.device)
    L = _lib.load()
    _lib.check(L.pq_pack_k64(_lib.ptr(w_int8), R, K, w_int8.stride(0), _lib.ptr(out), _lib.stream_of(w_int8.device)),
               "pack_k64")
    return out


def quant_rows_packed(x2: torch.Tensor, row_idx: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """quant_rows with the codes written in the packed K64 layout (flat int8 [packed_rows(M) * K]) for
    int8_gemm_packed; scales and the gather's range rule as quant_rows. K % 64 == 0."""
    assert x2.dim() == 2 and x2.is_cuda
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    rows, K = x2.shape
    ri = _row_index(row_idx, x2.device)
    M = rows if ri is None else ri.shape[0]
    q = torch.empty((packed_rows(M) * K,), dtype=torch.int8, device=x2.device)
    s = torch.empty((M,), dtype=torch.float32, device=x2.device)
    L = _lib.load()
    _lib.check(L.pq_quant_rows_packed(_lib.ptr(x2), _lib.dtype_code(x2.dtype), M, K, x2.stride(0), rows,
                                      _lib.ptr(ri), _lib.ptr(q), _lib.ptr(s), _lib.stream_of(x2.device)),
               "quant_rows_packed")
    return q, s


def lowrank_l1t_packable(R: int, K: int) -> bool:
    """Whether pq_pack_lowrank_l1t defines a fragment order for lr_At [R, K] (the one-pass quantizer's shapes)."""
    return R == 32 and K % 256 == 0 and K // 256 in (4, 5, 8, 10, 12)


def pack_lowrank_l1t(lr_At: torch.Tensor) -> Optional[torch.Tensor]:
    """lr_At [R, K] in the one-pass quantizer's fragment order (pq_pack_lowrank_l1t), a tensor of the same shape and
    dtype whose memory the kernel reads as contiguous 1 KB register loads; None where no such order exists. Int8Linear
    packs it once at conversion, beside lr_At."""
    assert lr_At.dim() == 2 and lr_At.is_cuda and lr_At.is_contiguous()
    R, K = lr_At.shape
    if not lowrank_l1t_packable(R, K) or lr_At.dtype not in (torch.bfloat16, torch.float16):
        return None
    out = torch.empty_like(lr_At)
    L = _lib.load()
    _lib.check(L.pq_pack_lowrank_l1t(_lib.ptr(lr_At), _lib.dtype_code(lr_At.dtype), R, K, _lib.ptr(out),
                                     _lib.stream_of(lr_At.device)), "pack_lowrank_l1t")
    return out


def quant_rows_lowrank(x2: torch.Tensor, lr_At: torch.Tensor, row_idx: Optional[torch.Tensor] = None,
                       lr_At_frag: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """quant_rows_packed(x2, row_idx) and lowrank_down(x2, lr_At, row_idx) from one pass over x2
    (pq_quant_rows_lowrank; deploy/int8_exec.py:390-391). Returns (packed codes, scales, t). ``lr_At_frag``: lr_At in
    fragment order (pack_lowrank_l1t) or None; the results are the same either way."""
    assert x2.dim() == 2 and x2.is_cuda and lr_At.is_cuda
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    assert lr_At.dtype == x2.dtype, "x2 and lr_A must share a dtype (cast x2 first, as the reference does)"
    rows, K = x2.shape
    assert K % 64 == 0, K
    assert lr_At.is_contiguous() and lr_At.shape[1] == K, "lr_At must be [R, K] contiguous"
    R = lr_At.shape[0]
    if lr_At_frag is not None:
        assert lr_At_frag.shape == lr_At.shape and lr_At_frag.dtype == lr_At.dtype and lr_At_frag.is_contiguous()
        assert lr_At_frag.device == lr_At.device
    ri = _row_index(row_idx, x2.device)
    M = rows if ri is None else ri.shape[0]
    q = torch.empty((packed_rows(M) * K,), dtype=torch.int8, device=x2.device)
    s = torch.empty((M,), dtype=torch.float32, device=x2.device)
    t = torch.empty((M, R), dtype=x2.dtype, device=x2.device)
    L = _lib.load()
    _lib.check(L.pq_quant_rows_lowrank(_lib.ptr(x2), _lib.dtype_code(x2.dtype), M, K, x2.stride(0), rows, _lib.ptr(ri),
                                       _lib.ptr(lr_At), _lib.ptr(lr_At_frag), R, _lib.ptr(q), _lib.ptr(s),
                                       _lib.ptr(t), R, _lib.stream_of(x2.device)), "quant_rows_lowrank")
    return q, s, t


def int8_gemm_packed(xq_p: torch.Tensor, s_row: torch.Tensor, w_p: torch.Tensor, w_scale: torch.Tensor,
                     bias: Optional[torch.Tensor], M: int, N: int, K: int, out_dtype: torch.dtype, *,
                     t: Optional[torch.Tensor] = None, l2t: Optional[torch.Tensor] = None,
                     out: Optional[torch.Tensor] = None, out_row_idx: Optional[torch.Tensor] = None,
                     group: int = 0, accumulate: bool = False) -> torch.Tensor:
    """The fused GEMM over packed K64 operands (pq_int8_gemm_packed): xq_p from quant_rows_packed, w_p from
    pack_k64. group 0: w_scale [N]; group 32: w_scale [K/32, N] (group-major). out_dtype torch.int32 returns the
    raw accumulator. accumulate=True (per-channel weights, 16-bit out): out += result in the epilogue, each element
    rounded as torch's 16-bit add rounds it."""
    assert xq_p.dtype == torch.int8 and w_p.dtype == torch.int8
    _check_cuda(xq_p, s_row, w_p, w_scale, bias, t, l2t, out, out_row_idx)
    assert xq_p.numel() >= packed_rows(M) * K and w_p.numel() >= packed_rows(N) * K
    ori = _row_index(out_row_idx, xq_p.device)
    L = _lib.load()
    if out_dtype == torch.int32:
        c = torch.empty((M, N), dtype=torch.int32, device=xq_p.device)
        _lib.check(L.pq_int8_gemm_packed(_lib.ptr(xq_p), _lib.ptr(w_p), None, None, 0, None, None, 0, None, 0, 0,
                                         _lib.ptr(c), N, _lib.PQ_I32, None, 0, M, N, K, None,
                                         _lib.stream_of(xq_p.device)),
                   "int8_gemm_packed")
        return c
    assert s_row.dtype == torch.float32 and s_row.is_contiguous() and s_row.numel() >= M
    assert group in (0, 32), group
    assert w_scale.dtype == torch.float32 and w_scale.is_contiguous()
    assert w_scale.numel() == (N * K // 32 if group else N), (tuple(w_scale.shape), N, K, group)
    if bias is not None:
        assert bias.dtype == torch.float32 and bias.is_contiguous() and bias.numel() == N
    if ori is not None:
        assert ori.shape[0] == M and out is not None, "a scatter needs the destination canvas (out=)"
    assert out is not None or not accumulate, "accumulate=True adds into out="
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=xq_p.device)
    assert out.dtype == out_dtype and out.dim() == 2 and out.shape[1] == N and out.stride(1) == 1
    if ori is None:
        assert out.shape[0] >= M
    lr_code, R, ldt = 0, 0, 0
    if t is not None:
        assert l2t is not None and t.dtype == l2t.dtype and t.stride(1) == 1 and l2t.is_contiguous()
        assert t.dim() == 2 and t.shape[0] >= M, (tuple(t.shape), M)
        R = t.shape[1]
        assert l2t.shape == (N, R), (tuple(l2t.shape), (N, R))
        lr_code, ldt = _lib.dtype_code(t.dtype), t.stride(0)
    out_code = _lib.dtype_code(out_dtype) | (_lib.PQ_ACCUMULATE if accumulate else 0)
    _lib.check(L.pq_int8_gemm_packed(_lib.ptr(xq_p), _lib.ptr(w_p), _lib.ptr(s_row), _lib.ptr(w_scale), group,
                                     _lib.ptr(bias), _lib.ptr(t), ldt, _lib.ptr(l2t), R, lr_code, _lib.ptr(out),
                                     out.stride(0), out_code, _lib.ptr(ori), out.shape[0], M, N, K,
                                     _lib.ptr(_sched_buffer(xq_p.device)), _lib.stream_of(xq_p.device)),
               "int8_gemm_packed")
    return out


def int8_linear_2d(x2: torch.Tensor, w_int8: torch.Tensor, w_scale: torch.Tensor,
                   bias: Optional[torch.Tensor], backend: Optional[str] = None) -> torch.Tensor:
    """x2 [M,K] bf16/fp16 -> [M,N] in x2's dtype: quantizer + fused GEMM (deploy/int8_exec.py:246-261)."""
    if backend is not None:
        if backend not in _BACKEND_ALIASES:
            raise ValueError(f"unknown INT8 backend {backend!r}")
    xq, sx = quant_rows(x2)
    return int8_gemm_fused(xq, sx, w_int8, w_scale, bias, x2.dtype)


# --------------------------------------------------------------------------- weight quantization
def quantize_weight(w: torch.Tensor, group_size: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """Weight RTN on the GPU (pq_quant_weight), fp32 math with IEEE divisions.
    group_size 0: per output channel, s [N] (deploy/int8_exec.py:355-357).
    group_size g: qdq_weight(w, 8, g) codes and scales, s [N, K/g] (pyraquant/quantizers_weight.py:96-109)."""
    assert w.dim() == 2 and w.is_cuda, "weight quantization runs on the GPU (move the Linear to the device first)"
    wf = w.detach().float()
    if wf.stride(1) != 1:
        wf = wf.contiguous()
    N, K = wf.shape
    if group_size:
        assert K % group_size == 0, (K, group_size)
    q = torch.empty((N, K), dtype=torch.int8, device=w.device)
    s = torch.empty((N, K // group_size) if group_size else (N,), dtype=torch.float32, device=w.device)
    L = _lib.load()
    _lib.check(L.pq_quant_weight(_lib.ptr(wf), N, K, wf.stride(0), group_size, _lib.ptr(q), _lib.ptr(s),
                                 _lib.stream_of(w.device)), "quant_weight")
    return q, s


# Attribute names under which a weight loader may attach a 16-bit low-rank branch to an nn.Linear
# before conversion (A: [in_features, r], B: [r, out_features]) -- deploy/int8_exec.py:341-342.
LOWRANK_A_ATTR = "_lowrank_A"
LOWRANK_B_ATTR = "_lowrank_B"

# Ranks the kernels take: the down-projection writes t in multiples of 32 columns (up to 128), the GEMM epilogue
# holds 16, 32 or 64 of them. Other ranks run zero-padded (zero columns of lr_A / rows of lr_B add exact zeros);
# above 64 the up-projection runs after the GEMM as an in-place addmm, the reference's unfused order
# (deploy/int8_exec.py:394-407).
_LR_DOWN_MAX = 128
_LR_EPILOGUE_RANKS = (16, 32, 64)


def _lowrank_widths(R: int) -> Tuple[int, int]:
    """(columns of t the down-projection computes, rank the GEMM epilogue takes; 0 = after the GEMM)."""
    r_down = (R + 31) // 32 * 32
    r_epi = next((r for r in _LR_EPILOGUE_RANKS if r >= R), 0)
    return (r_down if r_down <= _LR_DOWN_MAX else 0), r_epi


class Int8Linear(nn.Module):
    """INT8 stand-in for nn.Linear (deploy/int8_exec.py:345-411): int8 weights (buffers) + per-token dynamic
    int8 activations through the HIP kernels.

    Buffers as in the reference: ``weight_int8`` [N, K], ``w_scale`` ([N]; [N, K/32] with group_size=32),
    ``bias`` (fp32) and ``lr_A`` [K, R] / ``lr_B`` [R, N]. Kernel-layout copies: ``lr_At`` [R, K], ``lr_Bt``
    [N, R], ``lr_At_frag`` (lr_At in the one-pass quantizer's fragment order where one exists, else None; not saved
    in the state dict) and, for group_size=32, ``w_scale_gn`` [K/32, N]."""

    def __init__(self, lin: nn.Linear, device: Optional[torch.device] = None,
                 lowrank: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, group_size: int = 0):
        super().__init__()
        w = lin.weight.detach()
        if device is not None:
            w = w.to(device, non_blocking=False)
        q, s = quantize_weight(w, group_size)
        self.group_size = int(group_size)
        self.register_buffer("weight_int8", q)
        self.register_buffer("w_scale", s)
        N, K = q.shape
        # layers whose shape the packed GEMM takes (per-channel and group-32) run on the packed K64 path
        if K % 64 == 0 and N % 64 == 0:
            self.register_buffer("weight_packed", pack_k64(q))
        else:
            self.weight_packed = None
        if group_size:
            self.register_buffer("w_scale_gn", s.t().contiguous())
        else:
            self.w_scale_gn = None
        if lin.bias is not None:
            b = lin.bias.detach().float()
            self.register_buffer("bias", (b.to(device) if device is not None else b).contiguous())
        else:
            self.bias = None
        self.in_features = int(lin.in_features)
        self.out_features = int(lin.out_features)
        if lowrank is not None:
            A, B = lowrank
        else:
            A = getattr(lin, LOWRANK_A_ATTR, None)
            B = getattr(lin, LOWRANK_B_ATTR, None)
        if A is not None and B is not None:
            A = A.to(device) if device is not None else A
            B = B.to(device) if device is not None else B
            assert A.dim() == 2 and B.dim() == 2 and A.shape[1] == B.shape[0], (tuple(A.shape), tuple(B.shape))
            assert A.shape[0] == K and B.shape[1] == N, (tuple(A.shape), tuple(B.shape), K, N)
            self.register_buffer("lr_A", A.contiguous())
            self.register_buffer("lr_B", B.contiguous())
            R = A.shape[1]
            r_down, r_epi = _lowrank_widths(R)
            # kernel copies: lr_At [r_down, K] and lr_Bt [N, r_epi], zero-padded past rank R
            At = None
            if r_down and A.dtype in (torch.bfloat16, torch.float16):
                At = A.new_zeros((r_down, K))
                At[:R] = A.t()
            self.register_buffer("lr_At", At)
            self.register_buffer("lr_At_frag", None, persistent=False)
            self._lr_frag_key = None
            self._lr_frag()
            Bt = B.new_zeros((N, r_epi)) if r_epi else None
            if Bt is not None:
                Bt[:, :R] = B.t()
            self.register_buffer("lr_Bt", Bt)
        else:
            self.lr_A = None
            self.lr_B = None
            self.lr_At = None
            self.lr_At_frag = None
            self._lr_frag_key = None
            self.lr_Bt = None
        del w

    # Buffers the kernels read as fp32 whatever the model's dtype: a module-wide cast (.to(torch.bfloat16), .half())
    # moves them with the module but leaves their dtype, so the kernels never see 16-bit scales or bias. (The
    # reference's buffers follow the cast and its Triton kernels load any float type, deploy/int8_exec.py:356-362;
    # keeping fp32 keeps its pre-cast precision.)
    _FP32_BUFFERS = ("w_scale", "w_scale_gn", "bias")

    def _apply(self, fn, recurse=True):
        self.__dict__.pop("_direct_plans", None)   # (they hold the old buffers)
        keep = {n: self._buffers[n] for n in self._FP32_BUFFERS if self._buffers.get(n) is not None}
        super()._apply(fn, recurse)
        for n, old in keep.items():
            new = self._buffers[n]
            if new is not None and new.dtype != torch.float32:
                self._buffers[n] = old.to(new.device)
        return self

    def _lr_frag(self) -> Optional[torch.Tensor]:
        """lr_At in fragment order, repacked whenever lr_At is not the tensor it was packed from: a module-wide cast
        or move, load_state_dict (which copies into lr_At in place) or any other in-place update (torch's version
        counter). Tensors made under torch.inference_mode() carry no version counter: for them the key is the
        storage, dtype and device alone, so an in-place edit of an inference-mode lr_At needs the module rebuilt.
        None where no fragment order exists for lr_At's shape."""
        At = self.lr_At
        if At is None:
            return None
        key = (At.data_ptr(), None if At.is_inference() else At._version, At.dtype, At.device)
        if key != self._lr_frag_key:
            self.lr_At_frag = pack_lowrank_l1t(At) if At.is_cuda and At.is_contiguous() else None
            self._lr_frag_key = key
        return self.lr_At_frag

    def _scale_k(self) -> torch.Tensor:
        return self.w_scale_gn if self.group_size else self.w_scale

    def _lr_bt(self, dtype: torch.dtype) -> Optional[torch.Tensor]:
        """lr_B^T [N, R] in the output dtype (the fused epilogue takes t and lr_B in the output's 16-bit type)."""
        if self.lr_Bt is None:
            return None
        if self.lr_Bt.dtype != dtype:
            return self.lr_Bt.to(dtype)
        return self.lr_Bt

    # The tensors the direct call reads through raw pointers, looked up as nn.Module resolves attributes (instance
    # dict first, then the registered buffers) without its __getattr__: a replaced, moved or re-registered one
    # changes this tuple's identities and rebuilds the call's plan.
    _DIRECT_SOURCES = ("weight_packed", "w_scale", "w_scale_gn", "bias", "lr_A", "lr_At", "lr_Bt")

    def _direct_sources(self) -> tuple:
        d, b = self.__dict__, self._buffers
        return tuple(d[n] if n in d else b.get(n) for n in self._DIRECT_SOURCES) + (self._lr_frag(), self.group_size)

    def _direct_plan(self, dt: torch.dtype, src: tuple):
        """The part of the direct call that depends on the module alone, for input dtype dt: (source ids, the
        sources themselves (kept alive, so their ids stay theirs), device, dtype code, R, the static C arguments),
        or None where the direct path does not apply to this module and dtype."""
        code = _DIRECT_DTYPES.get(dt)
        wp, w_scale, w_scale_gn, bias, lr_A, lr_At, lr_Bt, frag, group = src
        if code is None or wp is None:
            return None
        if lr_A is not None and (lr_At is None or lr_Bt is None):
            return None
        R = 0 if lr_At is None else lr_At.shape[0]          # columns of t
        Re = 0 if lr_Bt is None else lr_Bt.shape[1]         # rank of the epilogue
        if R and (lr_At.dtype != dt or lr_Bt.dtype != dt):
            return None
        # the GEMM reads these as fp32 through raw pointers: anything else goes to the general path, which asserts
        sk = w_scale_gn if group else w_scale
        dev = wp.device
        if sk is None or sk.dtype != torch.float32 or sk.device != dev or not sk.is_contiguous():
            return None
        if bias is not None and (bias.dtype != torch.float32 or bias.device != dev):
            return None
        args = (wp.data_ptr(), sk.data_ptr(), group, None if bias is None else bias.data_ptr(),
                lr_At.data_ptr() if R else None, frag.data_ptr() if R and frag is not None else None,
                R, lr_Bt.data_ptr() if R else None, Re)
        return tuple(map(id, src)), src, dev, code, R, args

    def _forward_direct(self, x: torch.Tensor) -> Optional[torch.Tensor]:
        """The common layer call (no routing arguments, packed weights) with the host work cut to one C call,
        pq_int8_linear: codes, scales and t share one workspace allocation, operands go as raw pointers, the stream
        is the raw current stream. What depends on the module alone (the checks of its buffers and their pointers)
        is kept per input dtype and checked by identity on every call. Same kernels and arguments as the general
        path, so the same bits; returns None when a precondition of this path does not hold."""
        dt = x.dtype
        src = self._direct_sources()
        plans = self.__dict__.setdefault("_direct_plans", {})
        plan = plans.get(dt)
        if plan is None or plan[0] != tuple(map(id, src)):
            plan = self._direct_plan(dt, src)
            if plan is None:
                return None
            plans[dt] = plan
        _, _, dev, code, R, args = plan
        K, N = self.in_features, self.out_features
        if x.shape[-1] != K or x.device != dev:
            return None
        x2 = x if x.dim() == 2 else x.reshape(-1, K)
        ldx = x2.stride(0)
        xp = x2.data_ptr()
        if x2.stride(1) != 1 or ldx % 8 or xp % 16:
            return None
        M = x2.shape[0]
        L = _lib.load()
        ws = torch.empty(L.pq_int8_linear_workspace_size(M, K, R), dtype=torch.uint8, device=dev)
        out = torch.empty((M, N), dtype=dt, device=dev)
        st = L.pq_int8_linear(xp, code, M, K, ldx, *args, out.data_ptr(), N, N, ws.data_ptr(), ws.numel(),
                              _raw_stream(dev))
        if st:
            _lib.check(st, "int8_linear")
        return out if x.dim() == 2 else out.reshape(*x.shape[:-1], N)

    def forward(self, x: torch.Tensor, row_idx: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None, out_row_idx: Optional[torch.Tensor] = None,
                accumulate: bool = False) -> torch.Tensor:
        """y = Linear(x) through quantizer (+ low-rank down) + fused GEMM (deploy/int8_exec.py:382-408).
        Routed use: ``row_idx`` gathers rows of x (2-D x only), ``out``/``out_row_idx`` scatter into a canvas. Indices
        belong in range (rows of x, rows of out). On the kernel paths one that is not never reaches memory past the
        tensor: a gathered row outside x reads as zeros and a scattered row outside out is not written. The torch
        fallbacks (low-rank branches above rank 64) index with torch's own ops, which stop the process on it.
        ``accumulate=True`` adds the result into ``out`` (2-D, [rows, N]) instead of overwriting it, each element
        rounded as torch's 16-bit ``out + y`` rounds it: a Linear split along its input sums its halves this way."""
        if accumulate:
            assert out is not None, "accumulate=True adds into out="
        if row_idx is None and out is None and out_row_idx is None and self.weight_packed is not None and DIRECT_CALLS:
            y = self._forward_direct(x)
            if y is not None:
                return y
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if x2.stride(1) != 1:
            x2 = x2.contiguous()
        t = xq = sx = None
        fused = self.weight_packed is not None and self.lr_At is not None and x2.dtype == self.lr_A.dtype
        if fused:
            # quantizer and low-rank down-projection from one pass over x (deploy/int8_exec.py:390-391)
            xq, sx, t = quant_rows_lowrank(x2, self.lr_At, row_idx, self._lr_frag())
        elif self.lr_A is not None:
            xl = x2 if x2.dtype == self.lr_A.dtype else x2.to(self.lr_A.dtype)
            if self.lr_At is not None:
                t = lowrank_down(xl, self.lr_At, row_idx)
            else:   # a rank beyond the down-projection kernel's, or a 32-bit lr_A: torch's product, as the reference
                t = (xl if row_idx is None else xl.index_select(0, row_idx.long())) @ self.lr_A
                if self.lr_Bt is not None and t.shape[1] < self.lr_Bt.shape[1]:
                    t = F.pad(t, (0, self.lr_Bt.shape[1] - t.shape[1]))   # zero columns, as the padded lr_At gives
            if t.dtype != x2.dtype:
                t = t.to(x2.dtype)
        t_epi = None if t is None or self.lr_Bt is None else t[:, :self.lr_Bt.shape[1]]
        if t is not None and t_epi is None:
            return self._forward_lr_after(x2, shape, xq, sx, t, row_idx, out, out_row_idx, accumulate)
        if self.weight_packed is not None and (not accumulate or not self.group_size):
            if xq is None:
                xq, sx = quant_rows_packed(x2, row_idx)
            y = int8_gemm_packed(xq, sx, self.weight_packed, self._scale_k(), self.bias, sx.shape[0],
                                 self.out_features, self.in_features, x2.dtype, t=t_epi, l2t=self._lr_bt(x2.dtype),
                                 out=out, out_row_idx=out_row_idx, group=self.group_size, accumulate=accumulate)
        else:
            if xq is None:
                xq, sx = quant_rows_packed(x2, row_idx) if self.weight_packed is not None else quant_rows(x2, row_idx)
            if self.weight_packed is not None:   # group-32 weights accumulating: the GEMM's own output, then the add
                y = int8_gemm_packed(xq, sx, self.weight_packed, self._scale_k(), self.bias, sx.shape[0],
                                     self.out_features, self.in_features, x2.dtype, t=t_epi,
                                     l2t=self._lr_bt(x2.dtype), group=self.group_size)
            else:
                y = _gemm(xq, sx, self.weight_int8, self._scale_k(), self.group_size, self.bias, t_epi,
                          self._lr_bt(x2.dtype), x2.dtype, None if accumulate else out,
                          None if accumulate else out_row_idx)
            if accumulate:
                return _add_into(out, y, out_row_idx)
        if out is not None or row_idx is not None:
            return y
        return y.reshape(*shape[:-1], self.out_features)

    def _forward_lr_after(self, x2, shape, xq, sx, t, row_idx, out, out_row_idx, accumulate=False):
        """Ranks above the epilogue's: the GEMM without the low-rank term, then y += t @ lr_B in place
        (deploy/int8_exec.py:394-407), then the scatter into (or the add to) the canvas if one is given."""
        if xq is None:
            xq, sx = quant_rows_packed(x2, row_idx) if self.weight_packed is not None else quant_rows(x2, row_idx)
        M = sx.shape[0]
        if self.weight_packed is not None:
            y = int8_gemm_packed(xq, sx, self.weight_packed, self._scale_k(), self.bias, M, self.out_features,
                                 self.in_features, x2.dtype, group=self.group_size)
        else:
            y = _gemm(xq, sx, self.weight_int8, self._scale_k(), self.group_size, self.bias, None, None, x2.dtype)
        y.addmm_(t[:, :self.lr_A.shape[1]], self.lr_B.to(y.dtype))
        if accumulate:
            return _add_into(out, y, out_row_idx)
        if out is not None:
            if out_row_idx is not None:
                out.index_copy_(0, out_row_idx.long(), y)
            else:
                out[:M].copy_(y)
            return out
        if row_idx is not None:
            return y
        return y.reshape(*shape[:-1], self.out_features)

    def extra_repr(self) -> str:
        g = f"group-{self.group_size}" if self.group_size else "per-channel"
        lr = f", low-rank r={self.lr_A.shape[1]}" if self.lr_A is not None else ""
        return f"in={self.in_features}, out={self.out_features}, int8 {g} W / per-token A{lr} (HIP gfx950)"


def _add_into(out: torch.Tensor, y: torch.Tensor, out_row_idx: Optional[torch.Tensor]) -> torch.Tensor:
    """out[rows] += y with torch's 16-bit add (the accumulate mode where the GEMM's epilogue cannot do it)."""
    if out_row_idx is None:
        out[: y.shape[0]].add_(y)
    else:
        idx = out_row_idx.long()
        out.index_copy_(0, idx, out.index_select(0, idx).add_(y))
    return out


# --------------------------------------------------------------------------- model conversion
def is_bf16_whitelisted(name: str) -> bool:
    """SVDQuant-style whitelist + adaLN modulation projections, kept in bf16 (deploy/int8_exec.py:415-421)."""
    top = name.split(".")[0]
    if top in ("x_embedder", "context_embedder", "proj_out", "time_text_embed", "norm_out"):
        return True
    parts = name.split(".")
    return len(parts) >= 2 and parts[-1] == "linear" and parts[-2].startswith("norm")


def convert_linears_to_int8(model: nn.Module, device: Optional[str] = "cuda",
                            whitelist: Callable[[str], bool] = is_bf16_whitelisted) -> Dict[str, object]:
    """Replace the token-level nn.Linear layers by Int8Linear in place (deploy/int8_exec.py:424-445); returns the
    same statistics dict. A low-rank branch attached under LOWRANK_A_ATTR / LOWRANK_B_ATTR is carried over."""
    dev = torch.device(device) if device is not None else None
    n_int8, n_keep, p_int8, p_keep, kept = 0, 0, 0, 0, []
    targets = [(n, m) for n, m in model.named_modules() if isinstance(m, nn.Linear)]
    for name, lin in targets:
        if whitelist(name):
            n_keep += 1
            p_keep += lin.weight.numel()
            kept.append(name)
            continue
        parent_name, _, attr = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, attr, Int8Linear(lin, device=dev))
        n_int8 += 1
        p_int8 += lin.weight.numel()
        del lin
    if dev is not None and dev.type == "cuda":
        torch.cuda.synchronize()
    return {"n_int8_linear": n_int8, "n_bf16_linear_kept": n_keep, "params_int8": p_int8,
            "params_bf16_linear_kept": p_keep, "bf16_kept_names": kept, "int8_weight_gib": p_int8 / 2**30,
            "bf16_equiv_gib": p_int8 * 2 / 2**30}


# --------------------------------------------------------------------------- warm-up / self-test / micro-benchmark
FLUX_TOKEN_SHAPES = {   # (K, N): count -- FLUX.1-schnell token-level Linears (deploy/int8_exec.py:478-483)
    (3072, 3072): 19 * 8 + 38 * 3,
    (3072, 12288): 19 * 2 + 38,
    (12288, 3072): 19 * 2,
    (15360, 3072): 38,
}


def warm_kernels(Ms=(4352, 16640, 65792), device="cuda", lowrank_R=32, warm_lowrank: bool = True):
    """Signature of deploy/int8_exec.py:448-474. The HIP kernels are compiled ahead of time, so there is no JIT
    or autotune to pre-pay; this runs every (K, N) shape once at a small M to load the code objects and
    surface any launch error before a timed region. ``Ms`` is accepted for compatibility."""
    t0 = time.perf_counter()
    for (K, N) in FLUX_TOKEN_SHAPES:
        w = torch.randint(-127, 127, (N, K), device=device, dtype=torch.int8)
        s = torch.rand(N, device=device)
        b = torch.rand(N, device=device)
        x = torch.randn(64, K, device=device, dtype=torch.bfloat16)
        int8_linear_2d(x, w, s, b)
        int8_linear_2d(x[:8], w, s, b)
        if warm_lowrank:
            lbt = torch.randn(N, lowrank_R, device=device, dtype=torch.bfloat16)
            lat = torch.randn(lowrank_R, K, device=device, dtype=torch.bfloat16)
            xq, sx = quant_rows(x)
            t = lowrank_down(x, lat)
            _gemm(xq, sx, w, s, 0, b, t, lbt, torch.bfloat16)
            _gemm(xq, sx, w, s, 0, None, t, lbt, torch.bfloat16)
    torch.cuda.synchronize()
    print(f"[int8_exec] kernels warmed (backend={BACKEND}, gemm+lowrank r={lowrank_R}) in "
          f"{time.perf_counter() - t0:.1f}s", flush=True)


def _bench(fn, iters=20, warm=3):
    """Mean ms per call after ``warm`` calls, synced around the loop (deploy/int8_exec.py:486-492)."""
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t) / iters * 1e3


def selftest_and_bench(Ms=(4352, 16640, 33744, 65792), iters=10):
    """The reference's GPU self-test and per-shape micro-benchmark (deploy/int8_exec.py:495-571), run on the HIP
    kernels. Same inputs, same report keys, same assertions."""
    dev = "cuda"
    torch.manual_seed(0)
    lin = nn.Linear(3072, 12288, bias=True).to(dev, torch.bfloat16)
    x = (torch.randn(4352, 3072, device=dev) * 2).to(torch.bfloat16)
    x[:, 5] *= 30.0
    ref_bf16 = F.linear(x, lin.weight, lin.bias).float()
    q = Int8Linear(lin, device=torch.device(dev))
    y = q(x).float()
    xq, sx = quant_rows(x)
    ref_int8 = (xq.float() @ q.weight_int8.float().t()) * sx[:, None] * q.w_scale[None, :] + q.bias[None, :]
    xf = x.float()
    sc = xf.abs().amax(1, keepdim=True).clamp_min(1e-8) / 127
    xq_ref = torch.round(xf / sc).clamp(-127, 127).to(torch.int8)
    ref_int8_bf16 = ref_int8.to(torch.bfloat16).float()
    x_plain = torch.randn(4352, 3072, device=dev).to(torch.bfloat16)
    y_plain = q(x_plain).float()
    ref_plain = F.linear(x_plain, lin.weight, lin.bias).float()
    rep = {
        "act_quant_mismatch_elems": int((xq != xq_ref).sum().item()),
        "act_scale_max_rel_err": float(((sx - sc[:, 0]).abs() / sc[:, 0]).max().item()),
        "fused_vs_unfused_int8_max_abs": float((y - ref_int8_bf16).abs().max().item()),
        "fused_vs_unfused_int8_rel": float(((y - ref_int8_bf16).norm() / ref_int8_bf16.norm()).item()),
        "int8_vs_bf16_rel_outlier30x": float(((y - ref_bf16).norm() / ref_bf16.norm()).item()),
        "int8_vs_bf16_rel_plain": float(((y_plain - ref_plain).norm() / ref_plain.norm()).item()),
    }
    xs = x[:8]
    ys = q(xs).float()
    qs, ss = quant_rows(xs)
    rs = ((qs.float() @ q.weight_int8.float().t()) * ss[:, None] * q.w_scale[None, :] + q.bias[None, :]).to(torch.bfloat16).float()
    rep["smallM_fused_vs_unfused_rel"] = float(((ys - rs).norm() / rs.norm()).item())
    yt = int8_gemm_fused(xq, sx, q.weight_int8, q.w_scale, q.bias, torch.bfloat16).float()
    rep["hip_gemm_vs_module_max_abs"] = float((yt - y).abs().max().item())
    rep["hip_gemm_vs_unfused_rel"] = float(((yt - ref_int8_bf16).norm() / ref_int8_bf16.norm()).item())
    yts = int8_gemm_fused(qs, ss, q.weight_int8, q.w_scale, q.bias, torch.bfloat16).float()
    rep["hip_smallM_vs_unfused_rel"] = float(((yts - rs).norm() / rs.norm()).item())
    x3 = x[:2048].reshape(8, 256, 3072)
    rep["3d_input_ok"] = bool(torch.equal(q(x3).reshape(2048, -1), q(x[:2048])))
    print("[int8_exec] selftest:", rep, flush=True)
    rep["act_quant_mismatch_frac"] = rep["act_quant_mismatch_elems"] / x.numel()
    assert rep["act_quant_mismatch_frac"] <= 1e-4, rep
    assert rep["fused_vs_unfused_int8_rel"] < 1e-3 and rep["int8_vs_bf16_rel_plain"] < 2e-2, rep
    assert rep["hip_gemm_vs_unfused_rel"] < 1e-3 and rep["hip_smallM_vs_unfused_rel"] < 1e-3, rep
    del lin, q, x, ref_bf16, ref_int8, y, x_plain, y_plain, ref_plain
    torch.cuda.empty_cache()
    out = {"selftest": rep, "gpu": torch.cuda.get_device_name(), "per_M": {}}
    for M in Ms:
        tot = {"bf16_ms": 0.0, "int8_fused_ms": 0.0, "quant_ms": 0.0, "gemm_fused_ms": 0.0}
        per_shape = {}
        for (K, N), cnt in FLUX_TOKEN_SHAPES.items():
            lin = nn.Linear(K, N, bias=True).to(dev, torch.bfloat16)
            x = torch.randn(M, K, device=dev, dtype=torch.bfloat16)
            q = Int8Linear(lin, device=torch.device(dev))
            b = _bench(lambda: F.linear(x, lin.weight, lin.bias), iters)
            f = _bench(lambda: q(x), iters)
            xq, sx = quant_rows(x)
            qq = _bench(lambda: quant_rows(x), iters)
            tg = _bench(lambda: int8_gemm_fused(xq, sx, q.weight_int8, q.w_scale, q.bias, torch.bfloat16), iters)
            per_shape[f"{K}x{N}"] = {"count": cnt, "bf16_ms": round(b, 3), "int8_fused_ms": round(f, 3),
                                     "quant_ms": round(qq, 3), "gemm_fused_ms": round(tg, 3),
                                     "speedup": round(b / f, 3)}
            tot["bf16_ms"] += b * cnt
            tot["int8_fused_ms"] += f * cnt
            tot["quant_ms"] += qq * cnt
            tot["gemm_fused_ms"] += tg * cnt
            del lin, x, q, xq, sx
            torch.cuda.empty_cache()
        tot = {k: round(v, 2) for k, v in tot.items()}
        tot["speedup_fused_vs_bf16"] = round(tot["bf16_ms"] / tot["int8_fused_ms"], 3)
        tot["per_shape"] = per_shape
        out["per_M"][str(M)] = tot
        print(f"[int8_exec] M={M}: bf16 {tot['bf16_ms']} ms | int8 {tot['int8_fused_ms']} ms "
              f"(quant {tot['quant_ms']}, gemm {tot['gemm_fused_ms']}) -> x{tot['speedup_fused_vs_bf16']}", flush=True)
    return out


if __name__ == "__main__":
    import argparse
    import json

    ap = argparse.ArgumentParser(description="INT8 kernel self-test and micro-benchmark on the FLUX token-level "
                                             "Linear shapes (needs an MI355X).")
    ap.add_argument("out", nargs="?", default=None, help="optional JSON path for the results")
    ap.add_argument("--int8-backend", choices=tuple(_BACKEND_ALIASES), default=DEFAULT_BACKEND)
    args = ap.parse_args()
    set_backend(args.int8_backend)
    res = selftest_and_bench()
    res["int8_backend"] = BACKEND
    if args.out:
        with open(args.out, "w") as fh:
            json.dump(res, fh, indent=1)
        print(f"[int8_exec] saved {args.out}")
