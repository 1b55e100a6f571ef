"""CPU oracle of the routed executor's geometry and feathered fusion -- TEST INFRASTRUCTURE ONLY.

Checker for pyraquant_amd's routing kernels (pq_route_union_rows, pq_route_patches, pq_gather_rows,
pq_fuse_patches); never imported by the product package. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may use it.

Restated from the reference (paths relative to the PyraQuant repository):
  route_boxes            flux/run_flux.py:340-355    row-wise runs of selected leaves, latent coordinates
  token_box              flux/routing.py:202-232     latent box -> packed-token box (2x2 packing phase)
  expand_box             flux/routing.py:235-244     halo dilation clamped to the grid
  patch_geometry         flux/routing.py:253-315     repeated cores dropped, grouped by shape (ascending), row-major
  smooth_ramp            flux/routing.py:21-31
  halo_feather_mask      flux/routing.py:34-75
  fuse_patch_predictions flux/routing.py:328-379     torch CPU ops in the background's dtype, op for op

How they are pinned (tests/test_oracle_cpu.py): the golden config-4 record (tests/golden/route_c4.json) and the C
brute-force union (oracle.route_rows_union); hand-counted masks; the ramp against the float64 closed form
0.5 - 0.5 cos(pi u) and its end points; the fusion against closed forms (no patch -> background, a lone core ->
the patch prediction, fusion_beta 0 -> background, equal weights -> the mean) and against a float64 blend within
16-bit rounding.
"""
from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np
import torch

Box = Tuple[int, int, int, int]   # (y0, y1, x0, x1), half-open


def route_boxes(sel, leaf_latent: int) -> List[Box]:
    """Row-wise runs of selected leaves as latent boxes (flux/run_flux.py:340-355)."""
    sm = np.asarray(sel.cpu().numpy() if torch.is_tensor(sel) else sel) > 0.5
    boxes: List[Box] = []
    for i in range(sm.shape[0]):
        j = 0
        while j < sm.shape[1]:
            if sm[i, j]:
                j0 = j
                while j < sm.shape[1] and sm[i, j]:
                    j += 1
                boxes.append((i * leaf_latent, (i + 1) * leaf_latent, j0 * leaf_latent, j * leaf_latent))
            else:
                j += 1
    return boxes


def token_box(box: Box, packing_offset_latent: int = 0) -> Box:
    """Latent box -> packed-token box (flux/routing.py:202-232), with the reference's validation."""
    values = tuple(int(v) for v in box)
    if any(v < 0 for v in values):
        raise ValueError(f"Negative route coordinate: {values}")
    if any(v % 2 for v in values):
        raise ValueError(f"Route coordinates must align to FLUX 2x2 packing: {values}")
    off = int(packing_offset_latent)
    if off not in (0, 1):
        raise ValueError(f"Packing offset must be 0 or 1, got {off}")
    y0, y1, x0, x1 = values
    if y1 <= y0 or x1 <= x0:
        raise ValueError(f"Empty route box: {values}")
    return ((y0 + off) // 2, (y1 + off + 1) // 2, (x0 + off) // 2, (x1 + off + 1) // 2)


def expand_box(box: Box, halo: int, token_hw: Tuple[int, int]) -> Box:
    """Halo dilation clamped to the grid (flux/routing.py:235-244)."""
    y0, y1, x0, x1 = (int(v) for v in box)
    h, w = int(token_hw[0]), int(token_hw[1])
    halo = max(0, int(halo))
    return (max(0, y0 - halo), min(h, y1 + halo), max(0, x0 - halo), min(w, x1 + halo))


def patch_geometry(boxes: Sequence[Box], halo: int, token_hw: Tuple[int, int], packing_offset_latent: int = 0):
    """Patches in build_patch_buckets order (flux/routing.py:253-315).

    Returns (patches, rows): patches is a list of dicts {core, halo, inner, box_index, bucket} in extraction order;
    rows the int32 token rows of every patch, row-major inside a patch, patches in order."""
    h, w = int(token_hw[0]), int(token_hw[1])
    by_shape = {}
    seen = set()
    for bi, rb in enumerate(boxes):
        core = token_box(tuple(rb), packing_offset_latent)
        if core in seen:
            continue
        seen.add(core)
        y0, y1, x0, x1 = core
        if not (0 <= y0 < y1 <= h and 0 <= x0 < x1 <= w):
            raise ValueError(f"Route box {core} lies outside token grid {token_hw}")
        outer = expand_box(core, halo, token_hw)
        oy0, oy1, ox0, ox1 = outer
        inner = (y0 - oy0, y1 - oy0, x0 - ox0, x1 - ox0)
        by_shape.setdefault((oy1 - oy0, ox1 - ox0), []).append({"core": core, "halo": outer, "inner": inner,
                                                                "box_index": bi})
    patches, parts = [], []
    for bucket, shp in enumerate(sorted(by_shape)):
        for p in by_shape[shp]:
            p["bucket"] = bucket
            patches.append(p)
            oy0, oy1, ox0, ox1 = p["halo"]
            ys, xs = np.meshgrid(np.arange(oy0, oy1), np.arange(ox0, ox1), indexing="ij")
            parts.append((ys * w + xs).reshape(-1))
    rows = np.concatenate(parts).astype(np.int32) if parts else np.zeros((0,), np.int32)
    return patches, rows


def smooth_ramp(values: torch.Tensor, mode: str = "cosine", power: float = 1.0) -> torch.Tensor:
    """flux/routing.py:21-31."""
    out = values.clamp(0.0, 1.0)
    if mode in {"cosine", "hann", "raised_cosine"}:
        out = 0.5 - 0.5 * torch.cos(torch.pi * out)
    elif mode in {"smoothstep", "cubic"}:
        out = out * out * (3.0 - 2.0 * out)
    elif mode not in {"linear", "lin"}:
        raise ValueError(f"Unsupported feather ramp mode: {mode}")
    if float(power) != 1.0:
        out = out.pow(max(float(power), 1e-6))
    return out.clamp(0.0, 1.0)


def halo_feather_mask(patch_hw, inner, dtype, mode: str = "cosine", power: float = 1.0) -> torch.Tensor:
    """flux/routing.py:34-75 with min_alpha = 0 (the value fuse_patch_predictions passes, :356-364)."""
    height, width = int(patch_hw[0]), int(patch_hw[1])
    iy0, iy1, ix0, ix1 = [int(v) for v in inner]
    iy0, iy1 = max(0, min(iy0, height)), max(iy0, min(iy1, height))
    ix0, ix1 = max(0, min(ix0, width)), max(ix0, min(ix1, width))
    yw = torch.ones(height, dtype=torch.float32)
    xw = torch.ones(width, dtype=torch.float32)
    if iy0 > 0:
        yw[:iy0] = smooth_ramp(torch.linspace(0.0, 1.0, iy0), mode, power)
    if iy1 < height:
        yw[iy1:] = smooth_ramp(torch.linspace(1.0, 0.0, height - iy1), mode, power)
    if ix0 > 0:
        xw[:ix0] = smooth_ramp(torch.linspace(0.0, 1.0, ix0), mode, power)
    if ix1 < width:
        xw[ix1:] = smooth_ramp(torch.linspace(1.0, 0.0, width - ix1), mode, power)
    mask = torch.minimum(yw[:, None], xw[None, :]).clamp(0.0, 1.0)
    return mask.clamp(0.0, 1.0).to(dtype)


def fuse_patch_predictions(background: torch.Tensor, patches, patch_out: torch.Tensor, fusion_beta: float = 1.0,
                           mode: str = "cosine", power: float = 1.0) -> torch.Tensor:
    """flux/routing.py:328-379 on the CPU, op for op in the background's dtype.

    background [H, W, C]; patches from patch_geometry; patch_out [rows, C] in the order of patch_geometry's rows.
    Returns [H, W, C]."""
    if not 0.0 <= float(fusion_beta) <= 1.0:
        raise ValueError(f"fusion_beta must be in [0,1], got {fusion_beta}")
    bg = background[None]
    _, H, W, C = bg.shape
    local = torch.zeros_like(bg)
    bacc = torch.zeros((1, H, W, 1), dtype=bg.dtype)
    off = 0
    for p in patches:
        y0, y1, x0, x1 = p["halo"]
        ph, pw = y1 - y0, x1 - x0
        out = patch_out[off:off + ph * pw].reshape(1, ph, pw, C)
        off += ph * pw
        beta = halo_feather_mask((ph, pw), p["inner"], bg.dtype, mode, power)
        beta = (float(fusion_beta) * beta).clamp(0.0, 1.0)[None, :, :, None]
        local[:, y0:y1, x0:x1, :] += beta * out
        bacc[:, y0:y1, x0:x1, :] += beta
    bmap = bacc.clamp(0.0, 1.0)
    comb = torch.where(bacc > 0.0, local / bacc.clamp_min(1e-8), torch.zeros_like(local))
    return ((1.0 - bmap) * bg + bmap * comb)[0]
