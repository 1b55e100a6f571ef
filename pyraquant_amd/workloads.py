"""Synthetic workloads of the five benchmark configurations (seed 42), generated on the CPU with torch's
generator so every process (tests, bench, smoke) sees identical inputs.

  c0  M=4096,  K=3072,  N=3072   FLUX 1K attention projection, rank-32 low-rank, bias
  c1  M=65536, K=3072,  N=12288  FLUX 4K MLP up (the headline shape), rank-32 low-rank, bias
  c2a M=65536, K=12288, N=3072   FLUX 4K MLP down, rank-32 low-rank, bias
  c2b M=65536, K=3072,  N=9216   FLUX 4K fused QKV, rank-32 low-rank (one shared L1), bias
  c3  M=16384, K=1280,  N in {1280, 5120}  SDXL W8A8 group-32, no low-rank
  c4  c1 routed: rows gathered by the union of 2-token-halo-dilated active 16x16-token leaves

Distributions: x ~ N(0,1) in the activation dtype with round(0.005 K) seeded K-channels scaled x20
(outliers); W ~ N(0, 0.02) fp32; L1, L2 ~ N(0, 0.02) bf16; bias ~ N(0, 0.01) bf16, stored fp32.

Activation dtype: bf16 everywhere, as the benchmark configurations state it (c3 included: "Activations are bf16").
The fp16 twins c3_1280_f16 / c3_5120_f16 run the same layers in the dtype SDXL's UNet runs in
(deploy/run_sdxl_latency.py keeps the UNet in fp16); they are extra cases, not the stated configuration.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch


@dataclass(frozen=True)
class Config:
    name: str
    M: int
    K: int
    N: int
    lowrank: int = 32
    group: int = 0
    bias: bool = True
    routed: bool = False
    dtype: torch.dtype = torch.bfloat16


CONFIGS = {
    "c0": Config("c0", 4096, 3072, 3072),
    "c1": Config("c1", 65536, 3072, 12288),
    "c2a": Config("c2a", 65536, 12288, 3072),
    "c2b": Config("c2b", 65536, 3072, 9216),
    "c3_1280": Config("c3_1280", 16384, 1280, 1280, lowrank=0, group=32),
    "c3_5120": Config("c3_5120", 16384, 1280, 5120, lowrank=0, group=32),
    "c3_1280_f16": Config("c3_1280_f16", 16384, 1280, 1280, lowrank=0, group=32, dtype=torch.float16),
    "c3_5120_f16": Config("c3_5120_f16", 16384, 1280, 5120, lowrank=0, group=32, dtype=torch.float16),
    "c4": Config("c4", 65536, 3072, 12288, routed=True),
}


def make_x(M: int, K: int, dtype=torch.bfloat16, seed: int = 42, outlier_frac: float = 0.005,
           outlier_scale: float = 20.0, device: Optional[torch.device] = None) -> torch.Tensor:
    """Activations of the configs. With `device`, the same distribution is drawn by that device's generator (fast
    at full sizes; a different random stream from the CPU one)."""
    g = torch.Generator(device=device if device is not None else "cpu").manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=device)
    n_out = int(round(outlier_frac * K))
    if n_out:
        cols = torch.randperm(K, generator=g, device=device)[:n_out]
        x[:, cols] *= outlier_scale
    return x.to(dtype)


def make_weights(K: int, N: int, lowrank: int = 32, bias: bool = True, seed: int = 43,
                 lr_dtype=torch.bfloat16) -> dict:
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    out = {"w": w}
    if lowrank:
        out["L1"] = (torch.randn(K, lowrank, generator=g) * 0.02).to(lr_dtype)
        out["L2"] = (torch.randn(lowrank, N, generator=g) * 0.02).to(lr_dtype)
    if bias:
        out["bias"] = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16).float()
    return out


def make_linear(K: int, N: int, lowrank: int = 32, bias: bool = True, seed: int = 43,
                dtype=torch.bfloat16) -> torch.nn.Linear:
    """An nn.Linear carrying the synthetic weights (fp32 master weight) and, if lowrank, the low-rank
    branch attached under the reference's attribute names (deploy/int8_exec.py:341-342)."""
    from .int8_exec import LOWRANK_A_ATTR, LOWRANK_B_ATTR

    ws = make_weights(K, N, lowrank, bias, seed)
    lin = torch.nn.Linear(K, N, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(ws["w"])
        if bias:
            lin.bias.copy_(ws["bias"])
    if lowrank:
        setattr(lin, LOWRANK_A_ATTR, ws["L1"])
        setattr(lin, LOWRANK_B_ATTR, ws["L2"])
    return lin


def routed_rows(device: Optional[torch.device] = None) -> torch.Tensor:
    from .routing import routed_row_index

    return routed_row_index(device=device)
