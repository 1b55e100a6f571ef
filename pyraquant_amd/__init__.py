"""pyraquant_amd -- PyraQuant's INT8 deployment hot path (Int8Linear executor) for AMD MI355X (gfx950).

Modules:
  int8_exec  the reference's deploy/int8_exec.py API on hand-written HIP kernels (libpqint8.so)
  sdxl       the SDXL executor surface (deploy/run_sdxl_latency.py:104-298), incl. group-32 weights
  routing    routed-executor row geometry (gather / scatter lists, flux/routing.py)
  build      hipcc build of libpqint8.so
"""
from . import int8_exec, routing, sdxl  # noqa: F401
from .int8_exec import (  # noqa: F401
    BACKENDS, DEFAULT_BACKEND, FLUX_TOKEN_SHAPES, LOWRANK_A_ATTR, LOWRANK_B_ATTR, Int8Linear,
    convert_linears_to_int8, dequant_epilogue, get_backend, int8_gemm_fused, int8_gemm_i32, int8_gemm_lr,
    int8_gemm_packed, int8_linear_2d, is_bf16_whitelisted, lowrank_down, lowrank_l1t_packable, pack_k64,
    pack_lowrank_l1t, quant_rows, quant_rows_lowrank, quant_rows_packed, quantize_weight, set_backend, warm_kernels,
)

__all__ = [n for n in dir() if not n.startswith("_")]
