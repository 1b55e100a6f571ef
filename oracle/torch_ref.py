"""The reference's torch CPU quantize + int-matmul path, restated -- TEST AND CPU-BASELINE INFRASTRUCTURE ONLY.

Used only as bench.py's ``cpu_baseline`` leg (kind "port") and as an independent cross-check of the C oracle in
tests/. Never imported by the product package.

  quantizer   deploy/int8_exec.py:508-509   sc = |x|.amax(1).clamp_min(1e-8) / 127 ; round(x / sc).clamp(+-127)
  int32 GEMM  deploy/int8_exec.py:259       torch._int_mm(xq, w_int8.t())
  dequant     deploy/int8_exec.py:119-123   acc * (s_row * s_col) + bias
  low rank    deploy/int8_exec.py:390, 403-407   t = x @ A ; y.addmm_(t, B)
"""
from __future__ import annotations

from typing import Optional

import torch


def quant_rows(x: torch.Tensor):
    xf = x.float()
    sc = xf.abs().amax(1, keepdim=True).clamp_min(1e-8) / 127
    q = torch.round(xf / sc).clamp(-127, 127).to(torch.int8)
    return q, sc[:, 0]


def quant_weight(w: torch.Tensor):
    wf = w.float()
    s = wf.abs().amax(dim=1).clamp_min(1e-8) / 127.0
    q = torch.round(wf / s[:, None]).clamp_(-127, 127).to(torch.int8)
    return q, s


def int8_linear(x: torch.Tensor, w_int8: torch.Tensor, w_scale: torch.Tensor, bias: Optional[torch.Tensor],
                lr_A: Optional[torch.Tensor] = None, lr_B: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One Int8Linear forward on the CPU through the reference's torch ops (deploy/int8_exec.py:246-261 with
    the cublas-backend structure, which is what torch offers on a CPU, + the unfused low-rank branch)."""
    xq, sx = quant_rows(x)
    M = xq.shape[0]
    if M < 17:                                   # torch._int_mm needs M > 16 (deploy/int8_exec.py:54-55, 256-258)
        xq = torch.nn.functional.pad(xq, (0, 0, 0, 32 - M))
    acc = torch._int_mm(xq, w_int8.t())[:M]
    y = acc.float() * (sx[:, None] * w_scale[None, :])
    if bias is not None:
        y = y + bias[None, :]
    y = y.to(x.dtype)
    if lr_A is not None:
        t = x.to(lr_A.dtype) @ lr_A
        y.addmm_(t, lr_B)
    return y


def fold_one(W: torch.Tensor, smooth=None, shift=None, bias=None):
    """deploy/run_flux_latency.py:219-239 on the CPU: W [N, K] 16-bit, smooth / shift fp32 scalar or [K], bias 16-bit
    or None. Returns (folded W in W's dtype, new bias or None), op for op as the reference writes it."""
    dt = W.dtype
    Wf = W.float()
    if smooth is not None:
        s = smooth.float()
        Wf = Wf / s.reshape(()) if s.numel() == 1 else Wf / s.reshape(1, -1)
    b = bias
    if shift is not None:
        sh = shift.float()
        add = Wf.sum(dim=1) * sh.reshape(()) if sh.numel() == 1 else Wf @ sh.reshape(-1)
        b = add.to(dt) if bias is None else bias.clone().add_(add.to(bias.dtype))
    return Wf.to(dt), b
