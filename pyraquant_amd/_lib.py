"""ctypes binding of libpqint8.so (include/pyraquant_amd.h).

The library must be built (``python -m pyraquant_amd.build``); there is no fallback: every entry point of
the package raises if the HIP library is missing. Status codes map to the exception types the reference
raises for the same conditions (deploy/int8_exec.py:67-68, 206, 221, 235): AssertionError for shapes,
strides and alignment, ValueError for dtypes, RuntimeError for HIP launch failures.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads torch's HIP runtime first, so the library binds to the same one)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpqint8.so")

PQ_OK, PQ_EINVAL, PQ_ESHAPE, PQ_EALIGN, PQ_EDTYPE, PQ_ELAUNCH = 0, -1, -2, -3, -4, -5
PQ_BF16, PQ_F16, PQ_I32 = 0, 1, 2
PQ_ACCUMULATE = 0x100   # OR'ed into pq_int8_gemm_packed's out_dtype
ABI_VERSION = 3

# every entry point declared in include/pyraquant_amd.h
EXPORTS = (
    "pq_abi_version",
    "pq_last_error",
    "pq_quant_rows",
    "pq_quant_weight",
    "pq_lowrank_down",
    "pq_int8_gemm",
    "pq_int8_gemm_i32",
    "pq_int8_gemm_packed",
    "pq_pack_k64",
    "pq_quant_rows_packed",
    "pq_quant_rows_lowrank",
    "pq_pack_lowrank_l1t",
    "pq_dequant_epilogue",
    "pq_route_union_rows",
    "pq_route_patches",
    "pq_gather_rows",
    "pq_fuse_patches",
    "pq_fold_weight",
    "pq_int8_linear_workspace_size",
    "pq_int8_linear",
    "pq_int8_linear_noalloc",
    "pq_int8_linear_noalloc_max_bytes",
)

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

_SIGNATURES = {
    "pq_abi_version": ([], ctypes.c_int),
    "pq_last_error": ([], ctypes.c_char_p),
    "pq_quant_rows": ([_p, _i32, _i64, _i64, _i64, _i64, _p, _p, _p, _p], ctypes.c_int),
    "pq_quant_weight": ([_p, _i64, _i64, _i64, _i64, _p, _p, _p], ctypes.c_int),
    "pq_lowrank_down": ([_p, _i32, _i64, _i64, _i64, _i64, _p, _p, _i64, _p, _i64, _p], ctypes.c_int),
    "pq_int8_gemm": ([_p, _i64, _p, _i64, _p, _p, _i64, _p, _p, _i64, _p, _i64, _i32, _p, _i64, _i32, _p, _i64,
                      _i64, _i64, _i64, _p, _p], ctypes.c_int),
    "pq_int8_gemm_i32": ([_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _p], ctypes.c_int),
    "pq_int8_gemm_packed": ([_p, _p, _p, _p, _i64, _p, _p, _i64, _p, _i64, _i32, _p, _i64, _i32, _p, _i64, _i64, _i64,
                             _i64, _p, _p],
                            ctypes.c_int),
    "pq_pack_k64": ([_p, _i64, _i64, _i64, _p, _p], ctypes.c_int),
    "pq_quant_rows_packed": ([_p, _i32, _i64, _i64, _i64, _i64, _p, _p, _p, _p], ctypes.c_int),
    "pq_quant_rows_lowrank": ([_p, _i32, _i64, _i64, _i64, _i64, _p, _p, _p, _i64, _p, _p, _p, _i64, _p], ctypes.c_int),
    "pq_pack_lowrank_l1t": ([_p, _i32, _i64, _i64, _p, _p], ctypes.c_int),
    "pq_dequant_epilogue": ([_p, _p, _p, _p, _p, _i64, _i32, _i64, _i64, _p], ctypes.c_int),
    "pq_route_union_rows": ([_p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p], ctypes.c_int),
    "pq_route_patches": ([_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _i64, _p], ctypes.c_int),
    "pq_gather_rows": ([_p, _i64, _p, _p, _i64, _i64, _p, _i64, _p], ctypes.c_int),
    "pq_fuse_patches": ([_p, _i64, _p, _i64, _p, _p, _p, _i64, ctypes.c_float, _i64, _i64, _i64, _i32, _p, _i64, _p],
                        ctypes.c_int),
    "pq_fold_weight": ([_p, _i32, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _p, _i64, _p, _p], ctypes.c_int),
    "pq_int8_linear_workspace_size": ([_i64, _i64, _i64], _i64),
    "pq_int8_linear": ([_p, _i32, _i64, _i64, _i64, _p, _p, _i64, _p, _p, _p, _i64, _p, _i64, _p, _i64, _i64, _p, _i64,
                        _p], ctypes.c_int),
    "pq_int8_linear_noalloc": ([_p, _i32, _i64, _i64, _i64, _p, _p, _i64, _p, _p, _p, _i64, _p, _i64, _p, _i64, _i64,
                                _p], ctypes.c_int),
    "pq_int8_linear_noalloc_max_bytes": ([], _i64),
}

_lib = None


class LibraryMissing(RuntimeError):
    pass


def load():
    """Load libpqint8.so once (raises LibraryMissing if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(
                f"{LIB_PATH} is not built; run `python -m pyraquant_amd.build` (hipcc, gfx950). "
                "The INT8 executor has no CPU fallback.")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        v = L.pq_abi_version()
        if v != ABI_VERSION:
            raise LibraryMissing(f"libpqint8.so ABI version {v} != expected {ABI_VERSION}; rebuild it")
        _lib = L
    return _lib


def check(status: int, what: str) -> None:
    if status == PQ_OK:
        return
    msg = f"{what}: {load().pq_last_error().decode(errors='replace')}"
    if status in (PQ_EINVAL, PQ_ESHAPE, PQ_EALIGN):
        raise AssertionError(msg)
    if status == PQ_EDTYPE:
        raise ValueError(msg)
    raise RuntimeError(msg)


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return PQ_BF16
    if dt == torch.float16:
        return PQ_F16
    raise ValueError(f"unsupported 16-bit float dtype {dt} (expected bfloat16 or float16)")


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
