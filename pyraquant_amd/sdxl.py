"""SDXL flavour of the INT8 executor (deploy/run_sdxl_latency.py:104-298) on the HIP kernels.

The reference needs a second Triton autotune set for N % 256 != 0 (N = 640) and a direct-launch cache
("FAST_LAUNCH") to bring the per-call Python overhead from 75/100 us down to 8/11 us
(deploy/run_sdxl_latency.py:143-195). Here both are native: the HIP GEMM takes any N % 64 == 0 and every
call is one ctypes call into the C ABI, with no JIT or autotune dispatch. ``FAST_LAUNCH`` is kept as a flag
for driver compatibility; it changes nothing.

Group-32 W8A8 (config 3): ``SdxlInt8Linear(lin, group_size=32)`` keeps one fp32 scale per 32 consecutive K
elements per output channel (pyraquant/quantizers_weight.py:96-109) and applies it inside the MFMA K loop.
"""
from __future__ import annotations

import time
from collections import defaultdict

import torch
import torch.nn as nn

from . import int8_exec

FAST_LAUNCH = True


def sdxl_int8_linear_2d(x2, w_int8, w_scale, bias):
    """x2 [M,K] fp16/bf16 -> [M,N] (deploy/run_sdxl_latency.py:198-211): quantizer + fused GEMM."""
    xq, sx = int8_exec.quant_rows(x2)
    return int8_exec.int8_gemm_fused(xq, sx, w_int8, w_scale, bias, x2.dtype)


def fast_quant_rows(x2):
    """deploy/run_sdxl_latency.py:159-170; the HIP quantizer is already a direct launch."""
    return int8_exec.quant_rows(x2)


def fast_gemm_fused(xq, s_row, w_int8, w_scale, bias, out_dtype):
    """deploy/run_sdxl_latency.py:173-195; the HIP GEMM is already a direct launch."""
    return int8_exec.int8_gemm_fused(xq, s_row, w_int8, w_scale, bias, out_dtype)


class SdxlInt8Linear(int8_exec.Int8Linear):
    """SDXL Int8Linear (deploy/run_sdxl_latency.py:214-224); ``group_size=32`` selects group-32 weight scales."""

    def forward(self, x, row_idx=None, out=None, out_row_idx=None):
        return super().forward(x, row_idx=row_idx, out=out, out_row_idx=out_row_idx)


def is_fp16_whitelisted_sdxl(name: str) -> bool:
    """Tiny per-image Linears stay fp16 (deploy/run_sdxl_latency.py:227-229)."""
    return ("time_embedding" in name) or ("add_embedding" in name) or name.endswith("time_emb_proj")


def convert_unet_linears_to_int8(unet: nn.Module, device="cuda", group_size: int = 0):
    """deploy/run_sdxl_latency.py:232-249; ``group_size=32`` converts to group-32 weight scales."""
    dev = torch.device(device)
    n_int8, n_keep, p_int8, p_keep, kept = 0, 0, 0, 0, []
    shapes = defaultdict(int)
    for name, lin in [(n, m) for n, m in unet.named_modules() if isinstance(m, nn.Linear)]:
        if is_fp16_whitelisted_sdxl(name):
            n_keep += 1
            p_keep += lin.weight.numel()
            kept.append(name)
            continue
        parent_name, _, attr = name.rpartition(".")
        parent = unet.get_submodule(parent_name) if parent_name else unet
        setattr(parent, attr, SdxlInt8Linear(lin, device=dev, group_size=group_size))
        shapes[f"{lin.in_features}x{lin.out_features}"] += 1
        n_int8 += 1
        p_int8 += lin.weight.numel()
        del lin
    if dev.type == "cuda":
        torch.cuda.synchronize()
    return {"n_int8_linear": n_int8, "n_fp16_linear_kept": n_keep, "params_int8": p_int8,
            "params_fp16_linear_kept": p_keep, "fp16_kept_names": kept, "int8_weight_gib": p_int8 / 2**30,
            "fp16_equiv_gib": p_int8 * 2 / 2**30, "shapes_KxN": dict(sorted(shapes.items()))}


SDXL_TOKEN_SHAPES = [(640, 640), (2048, 640), (640, 5120), (2560, 640), (1280, 1280), (2048, 1280), (1280, 10240),
                     (5120, 1280)]   # (K, N) -- deploy/run_sdxl_latency.py:280


def warm_sdxl_kernels(Ms=(2048, 8192, 65536, 154, 8202, 32778), device="cuda"):
    """deploy/run_sdxl_latency.py:283-298: runs every SDXL (K, N) once at small M (no JIT to pre-pay)."""
    t0 = time.perf_counter()
    for (K, N) in SDXL_TOKEN_SHAPES:
        w = torch.randint(-127, 127, (N, K), device=device, dtype=torch.int8)
        s = torch.rand(N, device=device)
        b = torch.rand(N, device=device)
        x = torch.randn(154, K, device=device, dtype=torch.float16)
        sdxl_int8_linear_2d(x, w, s, b)
        sdxl_int8_linear_2d(x, w, s, None)
    torch.cuda.synchronize()
    print(f"[sdxl-int8] kernels warmed (backend={int8_exec.BACKEND}) in {time.perf_counter() - t0:.1f}s", flush=True)
