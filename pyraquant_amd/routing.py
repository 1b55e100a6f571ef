"""Routed-executor row geometry (config 4): which token rows the routed INT8 Linear gathers and scatters.

The reference routes selected leaves of the FLUX 4K token grid through the transformer
(flux/run_flux.py:340-358 builds row-run boxes of selected leaves; flux/routing.py:202-315 maps them to
packed-token boxes, dilates them by the halo and extracts patches). A token-level Linear sees only those rows,
so its gather list is the set of rows the patches cover. Two orders are provided:

* ``mode="union"`` (the Linear-level gather used for config 4): the sorted, unique rows of the union of all
  halo-dilated active leaves. Overlapping halos are computed once. 16x16-token leaves, Bernoulli(0.35) from
  torch.Generator().manual_seed(42), 2-token halo on the 256x256 grid give M = 33,316 rows.
* ``mode="patches"``: the rows in the order build_patch_buckets (flux/routing.py:253-315) extracts them --
  boxes from row runs of selected leaves, deduplicated cores, grouped by patch shape (shapes ascending),
  row-major inside each patch. Overlapping halos appear once per patch.

Row id of token (y, x) is y * W + x (packed-token order, flux/routing.py:288 reshape of the [H, W] grid).
This is host-side index construction (a few thousand boxes at most); the GPU consumes the int32 lists.
"""
from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np
import torch

Box = Tuple[int, int, int, int]   # (y0, y1, x0, x1), half-open


def leaf_mask(n_leaf: int = 16, p: float = 0.35, seed: int = 42) -> torch.Tensor:
    """Seeded Bernoulli(p) active-leaf map [n_leaf, n_leaf] (torch.Generator().manual_seed(seed))."""
    g = torch.Generator().manual_seed(seed)
    return torch.rand(n_leaf, n_leaf, generator=g) < p


def route_boxes_from_leaves(sel, leaf: int) -> List[Box]:
    """Row-wise runs of selected leaves as boxes (flux/run_flux.py:340-355), in units of ``leaf``."""
    sm = np.asarray(sel.cpu().numpy() if torch.is_tensor(sel) else sel) > 0.5
    boxes: List[Box] = []
    for i in range(sm.shape[0]):
        j = 0
        while j < sm.shape[1]:
            if sm[i, j]:
                j0 = j
                while j < sm.shape[1] and sm[i, j]:
                    j += 1
                boxes.append((i * leaf, (i + 1) * leaf, j0 * leaf, j * leaf))
            else:
                j += 1
    return boxes


def unpacked_box_to_token_box(box: Box, packing_offset_latent: int = 0) -> Box:
    """VAE-latent box -> packed-token box (flux/routing.py:202-232), 2x2 packing."""
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


def expand_box(box: Box, halo_tokens: int, token_hw: Tuple[int, int]) -> Box:
    """Dilate by the halo and clamp to the grid (flux/routing.py:235-244)."""
    y0, y1, x0, x1 = (int(v) for v in box)
    h, w = int(token_hw[0]), int(token_hw[1])
    halo = max(0, int(halo_tokens))
    return (max(0, y0 - halo), min(h, y1 + halo), max(0, x0 - halo), min(w, x1 + halo))


def patch_rows(route_boxes_latent: Sequence[Box], halo_tokens: int, token_hw: Tuple[int, int],
               packing_offset_latent: int = 0) -> np.ndarray:
    """Token rows in build_patch_buckets order (flux/routing.py:253-315)."""
    h, w = int(token_hw[0]), int(token_hw[1])
    by_shape = {}
    seen = set()
    for rb in route_boxes_latent:
        core = unpacked_box_to_token_box(tuple(rb), packing_offset_latent)
        if core in seen:
            continue
        seen.add(core)
        y0, y1, x0, x1 = core
        if not (0 <= y0 < y1 <= h and 0 <= x0 < x1 <= w):
            raise ValueError(f"Route box {core} lies outside token grid {token_hw}")
        oy0, oy1, ox0, ox1 = expand_box(core, halo_tokens, token_hw)
        ys, xs = np.meshgrid(np.arange(oy0, oy1), np.arange(ox0, ox1), indexing="ij")
        by_shape.setdefault((oy1 - oy0, ox1 - ox0), []).append((ys * w + xs).reshape(-1))
    parts = [r for shp in sorted(by_shape) for r in by_shape[shp]]
    return np.concatenate(parts).astype(np.int32) if parts else np.zeros((0,), np.int32)


def union_rows(sel, leaf_tokens: int, halo_tokens: int, token_hw: Tuple[int, int]) -> np.ndarray:
    """Sorted unique rows of the union of halo-dilated active leaves (box arithmetic per grid row)."""
    sm = np.asarray(sel.cpu().numpy() if torch.is_tensor(sel) else sel) > 0.5
    h, w = int(token_hw[0]), int(token_hw[1])
    covered = np.zeros((h, w), dtype=bool)
    for i, j in zip(*np.nonzero(sm)):
        y0, y1, x0, x1 = expand_box((i * leaf_tokens, (i + 1) * leaf_tokens, j * leaf_tokens, (j + 1) * leaf_tokens),
                                    halo_tokens, token_hw)
        covered[y0:y1, x0:x1] = True
    return np.flatnonzero(covered.reshape(-1)).astype(np.int32)


def routed_row_index(sel=None, *, leaf_tokens: int = 16, halo_tokens: int = 2, token_hw=(256, 256),
                     mode: str = "union", device=None) -> torch.Tensor:
    """int32 gather/scatter list for the routed INT8 Linear (config 4 defaults)."""
    if sel is None:
        sel = leaf_mask(token_hw[0] // leaf_tokens)
    if mode == "union":
        rows = union_rows(sel, leaf_tokens, halo_tokens, token_hw)
    elif mode == "patches":
        boxes_tok = route_boxes_from_leaves(sel, leaf_tokens)
        boxes_lat = [tuple(2 * v for v in b) for b in boxes_tok]   # token -> latent (2x2 packing)
        rows = patch_rows(boxes_lat, halo_tokens, token_hw)
    else:
        raise ValueError(f"unknown mode {mode!r} (union | patches)")
    t = torch.from_numpy(rows)
    return t.to(device) if device is not None else t
