"""CPU oracle of PyraQuant's INT8 deployment hot path -- TEST INFRASTRUCTURE ONLY.

This module is the checker for the HIP library ``pyraquant_amd``; it is never part of it. Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it. The
product path never calls it and has no CPU fallback.

It wraps ``oracle/libpqoracle.so`` (built from ``oracle/pq_oracle.c`` by ``oracle/Makefile``), a plain C
restatement of the reference's arithmetic. Each function names the reference lines it restates
(paths relative to the PyraQuant repository). Arrays are numpy; 16-bit floats travel as their raw
``uint16`` bit patterns with a dtype code (``BF16`` / ``F16``).

Each function is pinned by checks that do not restate it (``tests/test_oracle_cpu.py``): golden fixtures computed
by torch's CPU operators on the reference's torch lines (``tests/golden/``), ``torch._int_mm``, exact-rational and
float64 arithmetic, closed-form special cases and invariants. ``lowrank_down`` is pinned only to a tolerance.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Tuple

import numpy as np

BF16 = 0
F16 = 1

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libpqoracle.so")
_lib = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int


def build() -> str:
    """Compile libpqoracle.so with the committed Makefile (gcc, no GPU)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE, "-B", "libpqoracle.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.pqo_quant_rows.argtypes = [_p, _int, _i64, _i64, _i64, _p, _p, _p]
        L.pqo_quant_weight.argtypes = [_p, _i64, _i64, _i64, _p, _p]
        L.pqo_gemm_i32.argtypes = [_p, _i64, _p, _i64, _p, _i64, _i64, _i64]
        L.pqo_gemm_group_i32.argtypes = [_p, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64]
        L.pqo_lowrank_down.argtypes = [_p, _int, _i64, _i64, _i64, _p, _p, _i64, _p]
        L.pqo_epilogue_f32.argtypes = [_p, _i64, _i64, _p, _p, _p, _p, _p, _i64, _int, _p, _i64, _i64]
        L.pqo_route_rows_union.argtypes = [_p, _i64, _i64, _i64, _i64, _p]
        L.pqo_route_rows_union.restype = _i64
        L.pqo_to_f32.argtypes = [_p, _int, _i64, _p]
        L.pqo_from_f32.argtypes = [_p, _int, _i64, _p]
        _lib = L
    return _lib


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------------------------------- 16-bit floats
def to_f32(bits: np.ndarray, dtype: int) -> np.ndarray:
    """Exact widening of bf16 / fp16 bit patterns to fp32."""
    b = _c(bits, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().pqo_to_f32(_ptr(b), dtype, b.size, _ptr(out))
    return out


def from_f32(x: np.ndarray, dtype: int) -> np.ndarray:
    """fp32 -> bf16 / fp16 bit patterns, round to nearest even (torch's .to(bfloat16/float16))."""
    f = _c(x, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().pqo_from_f32(_ptr(f), dtype, f.size, _ptr(out))
    return out


# ---------------------------------------------------------------------------------------- A. quantizer
def quant_rows(x_bits: np.ndarray, dtype: int, row_idx: Optional[np.ndarray] = None) -> Tuple[np.ndarray, np.ndarray]:
    """Per-token absmax int8 quantizer, deploy/int8_exec.py:508-509 (kernel :78-101).

    x_bits: [rows, K] 16-bit patterns (row-major). row_idx: optional int32 [M] gather list.
    Returns (q int8 [M, K], s fp32 [M])."""
    x = _c(x_bits, np.uint16)
    rows, K = x.shape
    ri = None if row_idx is None else _c(row_idx, np.int32)
    M = rows if ri is None else ri.shape[0]
    if ri is not None and M and (ri.min() < 0 or ri.max() >= rows):
        raise IndexError("row_idx out of range")
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    lib().pqo_quant_rows(_ptr(x), dtype, M, K, K, _ptr(ri), _ptr(q), _ptr(s))
    return q, s


# ---------------------------------------------------------------------------------------- B / G. weights
def quant_weight(w: np.ndarray, group: int = 0) -> Tuple[np.ndarray, np.ndarray]:
    """Weight RTN. group=0: per output channel, deploy/int8_exec.py:355-357 -> s [N].
    group=g: qdq_weight(w, 8, g) codes/scales, pyraquant/quantizers_weight.py:96-109 -> s [N, K/g]."""
    wf = _c(w, np.float32)
    N, K = wf.shape
    if group and K % group:
        raise ValueError("K must be a multiple of the group size")
    q = np.empty((N, K), np.int8)
    s = np.empty((N,) if not group else (N, K // group), np.float32)
    lib().pqo_quant_weight(_ptr(wf), N, K, group, _ptr(q), _ptr(s))
    return q, s


# ---------------------------------------------------------------------------------------- C. int32 GEMM
def gemm_i32(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """acc[m, n] = sum_k a[m, k] w[n, k], exact int32 (deploy/int8_exec.py:259, torch._int_mm)."""
    a = _c(a, np.int8)
    w = _c(w, np.int8)
    M, K = a.shape
    N = w.shape[0]
    c = np.empty((M, N), np.int32)
    lib().pqo_gemm_i32(_ptr(a), K, _ptr(w), K, _ptr(c), M, N, K)
    return c


def gemm_group_i32(a: np.ndarray, w: np.ndarray, group: int = 32) -> np.ndarray:
    """Per-group partial accumulators part[m, n, j] = sum over K group j (exact int32)."""
    a = _c(a, np.int8)
    w = _c(w, np.int8)
    M, K = a.shape
    N = w.shape[0]
    part = np.empty((M, N, K // group), np.int32)
    lib().pqo_gemm_group_i32(_ptr(a), K, _ptr(w), K, group, _ptr(part), M, N, K)
    return part


# ---------------------------------------------------------------------------------------- E. low rank
def lowrank_down(x_bits: np.ndarray, dtype: int, l1_bits: np.ndarray, row_idx: Optional[np.ndarray] = None) -> np.ndarray:
    """t = (x @ L1) rounded to the 16-bit type, fp32 accumulation (deploy/int8_exec.py:390). L1: [K, R]."""
    x = _c(x_bits, np.uint16)
    l1 = _c(l1_bits, np.uint16)
    rows, K = x.shape
    R = l1.shape[1]
    ri = None if row_idx is None else _c(row_idx, np.int32)
    M = rows if ri is None else ri.shape[0]
    t = np.empty((M, R), np.uint16)
    lib().pqo_lowrank_down(_ptr(x), dtype, M, K, K, _ptr(ri), _ptr(l1), R, _ptr(t))
    return t


# ---------------------------------------------------------------------------------------- C / D / G epilogue
def epilogue_f32(acc: np.ndarray, s_row: np.ndarray, s_w: np.ndarray, bias: Optional[np.ndarray] = None,
                 t_bits: Optional[np.ndarray] = None, l2_bits: Optional[np.ndarray] = None,
                 lr_dtype: int = BF16) -> np.ndarray:
    """fp32 epilogue before the 16-bit rounding (deploy/int8_exec.py:176-178, :303-309).

    acc: int32 [M, N] (per-channel, s_w [N]) or int32 [M, N, G] group partials (s_w [N, G]).
    t_bits [M, R] / l2_bits [R, N]: the low-rank operands in lr_dtype."""
    acc = _c(acc, np.int32)
    M, N = acc.shape[:2]
    group = 0 if acc.ndim == 2 else 1
    G = 1 if acc.ndim == 2 else acc.shape[2]
    sr = _c(s_row, np.float32)
    sw = _c(s_w, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    t = None if t_bits is None else _c(t_bits, np.uint16)
    l2 = None if l2_bits is None else _c(l2_bits, np.uint16)
    R = 0 if t is None else t.shape[1]
    y = np.empty((M, N), np.float32)
    lib().pqo_epilogue_f32(_ptr(acc), group, G, _ptr(sr), _ptr(sw), _ptr(b), _ptr(t), _ptr(l2), R, lr_dtype, _ptr(y), M, N)
    return y


def linear(x_bits: np.ndarray, dtype: int, w_q: np.ndarray, w_s: np.ndarray, bias: Optional[np.ndarray] = None,
           group: int = 0, l1_bits: Optional[np.ndarray] = None, l2_bits: Optional[np.ndarray] = None,
           row_idx: Optional[np.ndarray] = None, out_dtype: Optional[int] = None) -> dict:
    """The whole Int8Linear forward (deploy/int8_exec.py:382-393) on the CPU: codes, accumulators, t, fp32
    result and the rounded output bits. Returns a dict of every intermediate."""
    q, s = quant_rows(x_bits, dtype, row_idx)
    acc = gemm_i32(q, w_q) if not group else gemm_group_i32(q, w_q, group)
    t = None
    if l1_bits is not None:
        t = lowrank_down(x_bits, dtype, l1_bits, row_idx)
    y = epilogue_f32(acc, s, w_s, bias, t, l2_bits, dtype)
    od = dtype if out_dtype is None else out_dtype
    return {"q": q, "s": s, "acc": acc, "t": t, "y": y, "out": from_f32(y, od)}


# ---------------------------------------------------------------------------------------- I. routing
def route_rows_union(mask: np.ndarray, leaf: int = 16, halo: int = 2) -> np.ndarray:
    """Sorted unique token rows of the union of halo-dilated active leaves (brute force on a canvas;
    dilation and clamping as flux/routing.py:235-244)."""
    m = _c(mask, np.uint8)
    gh, gw = m.shape
    n = lib().pqo_route_rows_union(_ptr(m), gh, gw, leaf, halo, None)
    rows = np.empty((n,), np.int32)
    lib().pqo_route_rows_union(_ptr(m), gh, gw, leaf, halo, _ptr(rows))
    return rows


# ---------------------------------------------------------------------------------------- packed K64 layout
def k64_swz(r: np.ndarray) -> np.ndarray:
    """Slot permutation of the packed K64 layout (include/pyraquant_amd.h): bit 0 = bit 2 of r, bit 1 = bit 1 xor
    bit 3 of r."""
    r = np.asarray(r)
    return ((r >> 2) & 1) | ((((r >> 1) ^ (r >> 3)) & 1) << 1)


def pack_k64(x: np.ndarray) -> np.ndarray:
    """Row-major int8 [R, K] -> packed K64 bytes (ceil(R / 16) * 16 * K), restated from the layout's definition:
    block (rb, kt) at (rb * KT + kt) * 1024, row r' = r % 16 at 64 r', chunk c at slot c ^ swz(r'); padding rows 0.
    Layout of this build (no reference counterpart); used to check pq_pack_k64 / pq_quant_rows_packed."""
    x = _c(x, np.int8)
    R, K = x.shape
    if K % 64:
        raise ValueError("K must be a multiple of 64")
    RB, KT = (R + 15) // 16, K // 64
    xp = np.zeros((RB * 16, K), np.int8)
    xp[:R] = x
    # [RB, 16, KT, 4, 16] -> blocks [RB, KT, 16 rows, 4 slots, 16 bytes]
    v = xp.reshape(RB, 16, KT, 4, 16).transpose(0, 2, 1, 3, 4)
    out = np.empty_like(v)
    rows = np.arange(16)
    for c in range(4):
        slot = c ^ k64_swz(rows)                       # [16]
        out[:, :, rows, slot, :] = v[:, :, rows, c, :]
    return out.reshape(-1)


def unpack_k64(p: np.ndarray, R: int, K: int) -> np.ndarray:
    """Inverse of pack_k64 (the first R rows)."""
    RB, KT = (R + 15) // 16, K // 64
    v = _c(p, np.int8).reshape(RB, KT, 16, 4, 16)
    out = np.empty_like(v)
    rows = np.arange(16)
    for c in range(4):
        out[:, :, rows, c, :] = v[:, :, rows, c ^ k64_swz(rows), :]
    return out.transpose(0, 2, 1, 3, 4).reshape(RB * 16, K)[:R]
