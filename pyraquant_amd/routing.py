"""Routed-executor geometry and feathered fusion on the device (config 4 and the routed FLUX executor).

The reference routes the selected leaves of the FLUX 4K token grid through the transformer: it copies the leaf
mask to the host (flux/run_flux.py:343), builds row-run boxes (:340-355), maps them to packed-token cores, dilates
them by the halo and extracts one patch per core, grouped by shape (flux/routing.py:202-315), and after the
transformer blends the patch predictions into the background (flux/routing.py:328-379), one torch op per patch.
Here every step is one HIP kernel of libpqint8.so on a device-resident mask:

* ``union_rows`` / ``routed_row_index(mode="union")``: the Linear-level gather list of config 4 -- the sorted,
  unique rows of the union of the halo-dilated active leaves (pq_route_union_rows). 16 x 16-token leaves,
  Bernoulli(0.35) from torch.Generator().manual_seed(42) and a 2-token halo on the 256 x 256 grid give
  M = 33,316 rows.
* ``route_patches`` / ``routed_row_index(mode="patches")``: the patch table and the rows in build_patch_buckets
  order (pq_route_patches); ``build_patch_buckets`` extracts hidden states and ids with one gather each
  (pq_gather_rows) and hands out per-shape views.
* ``fuse_patch_predictions``: the continuous-beta feathered blend (pq_fuse_patches), 16-bit rounding per torch op
  as the reference computes it.

Row id of token (y, x) is y * W + x (packed-token order, flux/routing.py:105-115). Counts stay on the device;
only the calls that hand the host a Python object (exact-length row lists, PatchBucket shapes) read them.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import _lib

Box = Tuple[int, int, int, int]   # (y0, y1, x0, x1), half-open
TABLE_STRIDE = 12                 # int32 per patch in the device table (include/pyraquant_amd.h)
MAX_BOXES = 2048


def leaf_mask(n_leaf: int = 16, p: float = 0.35, seed: int = 42) -> torch.Tensor:
    """Config 4's seeded Bernoulli(p) active-leaf map [n_leaf, n_leaf] (torch.Generator().manual_seed(seed))."""
    g = torch.Generator().manual_seed(seed)
    return torch.rand(n_leaf, n_leaf, generator=g) < p


def _device(device) -> torch.device:
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    if dev.type != "cuda":
        raise AssertionError(f"routing kernels run on the GPU; got device {dev}")
    return dev


def _mask_device(sel):
    return sel.device if torch.is_tensor(sel) and sel.is_cuda else None


def _mask_u8(sel, device) -> torch.Tensor:
    """Leaf mask as a contiguous uint8 device tensor (selected = value > 0.5, flux/run_flux.py:343)."""
    _lib.load()
    t = sel if torch.is_tensor(sel) else torch.as_tensor(sel)
    if t.ndim != 2:
        raise AssertionError(f"leaf mask must be 2-D, got shape {tuple(t.shape)}")
    if t.dtype == torch.uint8 and t.device == device and t.is_contiguous():
        return t
    t = t.to(device)
    t = (t > 0.5) if t.is_floating_point() else (t != 0)
    return t.to(torch.uint8).contiguous()


# --------------------------------------------------------------------------------------------- union (config 4)
def union_rows(sel, leaf_tokens: int = 16, halo_tokens: int = 2, token_hw: Optional[Tuple[int, int]] = None,
               device=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Rows of the union of the halo-dilated active leaves: (rows [H * W] int32, count [1] int32), both on the
    device; rows[:count] is sorted and unique. token_hw defaults to the leaf grid times leaf_tokens."""
    dev = _device(device if device is not None else _mask_device(sel))
    m = _mask_u8(sel, dev)
    Lh, Lw = m.shape
    H, W = token_hw if token_hw is not None else (Lh * leaf_tokens, Lw * leaf_tokens)
    rows = torch.empty(int(H) * int(W), dtype=torch.int32, device=dev)
    count = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.check(_lib.load().pq_route_union_rows(_lib.ptr(m), Lh, Lw, int(leaf_tokens), int(halo_tokens), int(H), int(W),
                                               _lib.ptr(rows), _lib.ptr(count), _lib.stream_of(dev)),
               "route_union_rows")
    return rows, count


# ------------------------------------------------------------------------------------------------- patches
@dataclass(frozen=True)
class PatchGeometry:
    """Geometry of one selected leaf run in packed-token coordinates (flux/routing.py:78-84)."""
    core_box: Box
    halo_box: Box
    inner_box_in_patch: Box


@dataclass
class PatchBucket:
    """Same-shaped patches that share one transformer call (flux/routing.py:87-94)."""
    patch_hw: Tuple[int, int]
    hidden_states: torch.Tensor
    img_ids: torch.Tensor
    geometries: List[PatchGeometry]


@dataclass
class RouteTable:
    """Device outputs of pq_route_patches: table [capacity, 12] int32, counts [4] int32, rows [max_rows] int32."""
    table: torch.Tensor
    counts: torch.Tensor
    rows: torch.Tensor
    token_hw: Tuple[int, int]
    halo: int

    def host(self) -> Dict[str, object]:
        """Read the counts and table (one device -> host copy): {patches, rows, buckets, entries}."""
        c = self.counts.cpu().tolist()
        if c[3] & 1:
            raise RuntimeError(f"route_patches: {c[1]} rows exceed the {self.rows.numel()}-row buffer")
        n = c[0]
        return {"patches": n, "rows": c[1], "buckets": c[2], "entries": self.table[:n].cpu().tolist()}


def max_patch_rows(Lh: int, Lw: int, leaf_latent: int, halo: int, token_hw: Tuple[int, int]) -> int:
    """Upper bound on the patch rows of any Lh x Lw mask: every run box, at most ceil(Lw / 2) per leaf row, covers
    at most (leaf + 1 + 2 halo) x min(W, Lw (leaf + 1) + 2 halo) tokens (leaf = leaf_latent / 2 tokens)."""
    lt = leaf_latent // 2 + 1
    return Lh * ((Lw + 1) // 2) * (lt + 2 * halo) * min(int(token_hw[1]), Lw * lt + 2 * halo)


def route_patches(sel, *, leaf_latent: int = 64, halo_tokens: int = 8, token_hw: Optional[Tuple[int, int]] = None,
                  packing_offset_latent: int = 0, max_rows: Optional[int] = None, device=None) -> RouteTable:
    """Patch geometry of the routed executor on the device (flux/run_flux.py:340-355, flux/routing.py:202-315).
    Defaults follow the reference's 4K stage: 64-latent leaves (32 tokens); token_hw defaults to the leaf grid."""
    dev = _device(device if device is not None else _mask_device(sel))
    m = _mask_u8(sel, dev)
    Lh, Lw = m.shape
    if token_hw is None:
        token_hw = (Lh * leaf_latent // 2, Lw * leaf_latent // 2)
    H, W = int(token_hw[0]), int(token_hw[1])
    cap = Lh * ((Lw + 1) // 2)
    if cap > MAX_BOXES:
        raise AssertionError(f"route_patches: a {Lh}x{Lw} mask can hold {cap} row-run boxes (at most {MAX_BOXES})")
    if max_rows is None:
        max_rows = max_patch_rows(Lh, Lw, leaf_latent, halo_tokens, (H, W))
    table = torch.empty(cap, TABLE_STRIDE, dtype=torch.int32, device=dev)
    counts = torch.empty(4, dtype=torch.int32, device=dev)
    rows = torch.empty(max(int(max_rows), 1), dtype=torch.int32, device=dev)
    _lib.check(_lib.load().pq_route_patches(_lib.ptr(m), Lh, Lw, int(leaf_latent), int(halo_tokens), H, W,
                                            int(packing_offset_latent), _lib.ptr(table), _lib.ptr(counts),
                                            _lib.ptr(rows), int(max_rows), _lib.stream_of(dev)), "route_patches")
    return RouteTable(table, counts, rows, (H, W), int(halo_tokens))


def routed_row_index(sel=None, *, leaf_tokens: int = 16, halo_tokens: int = 2, token_hw=(256, 256),
                     mode: str = "union", device=None) -> torch.Tensor:
    """Exact-length int32 gather/scatter list on the device (config 4 defaults). mode "union": sorted unique rows
    of the union of the dilated leaves; "patches": the rows in build_patch_buckets order (halo overlaps repeated).
    Reads the row count back to the host."""
    if sel is None:
        sel = leaf_mask(int(token_hw[0]) // leaf_tokens)
    if mode == "union":
        rows, count = union_rows(sel, leaf_tokens, halo_tokens, token_hw, device)
        return rows[: int(count.item())]
    if mode == "patches":
        rt = route_patches(sel, leaf_latent=2 * leaf_tokens, halo_tokens=halo_tokens, token_hw=token_hw,
                           device=device)
        info = rt.host()
        return rt.rows[: info["rows"]]
    raise ValueError(f"unknown mode {mode!r} (union | patches)")


def gather_rows(src: torch.Tensor, rows: torch.Tensor, count: torch.Tensor, n_max: Optional[int] = None,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[r] = src[rows[r]] for r < min(count, n_max) on the device (pq_gather_rows); src is [n, ...] with
    contiguous rows whose byte size is a multiple of 4. Rows past the count are left as they are."""
    if not src.is_cuda:
        raise AssertionError("gather_rows: src must be a CUDA tensor")
    n_max = rows.numel() if n_max is None else int(n_max)
    s2 = src.reshape(src.shape[0], -1)
    if s2.stride(1) != 1:
        raise AssertionError("gather_rows: rows of src must be contiguous")
    if out is None:
        out = torch.empty((n_max,) + tuple(src.shape[1:]), dtype=src.dtype, device=src.device)
    o2 = out.reshape(out.shape[0], -1)
    rb = s2.shape[1] * s2.element_size()
    _lib.check(_lib.load().pq_gather_rows(_lib.ptr(s2), s2.stride(0) * s2.element_size(), _lib.ptr(rows),
                                          _lib.ptr(count), n_max, rb, _lib.ptr(o2), o2.stride(0) * o2.element_size(),
                                          _lib.stream_of(src.device)), "gather_rows")
    return out


def _geometry(entry) -> PatchGeometry:
    oy0, oy1, ox0, ox1, cy0, cy1, cx0, cx1 = entry[:8]
    return PatchGeometry((cy0, cy1, cx0, cx1), (oy0, oy1, ox0, ox1), (cy0 - oy0, cy1 - oy0, cx0 - ox0, cx1 - ox0))


def build_patch_buckets(hidden_states: torch.Tensor, img_ids: torch.Tensor, *, route: RouteTable) -> List[PatchBucket]:
    """Extract the selected patches with their ids (flux/routing.py:253-315) from a device route table: one gather
    of hidden_states [1, H * W, C] and one of img_ids [H * W, 3] in extraction order; each bucket is a view."""
    if int(hidden_states.shape[0]) != 1:
        raise ValueError("The routed executor supports one generated image per run")
    H, W = route.token_hw
    if int(hidden_states.shape[1]) != H * W or int(img_ids.shape[0]) != H * W:
        raise ValueError(f"token count {hidden_states.shape[1]} / ids {img_ids.shape[0]} != grid {H}x{W}")
    info = route.host()
    n = info["rows"]
    hs = gather_rows(hidden_states[0], route.rows, route.counts[1:2], n)
    ids = gather_rows(img_ids.contiguous(), route.rows, route.counts[1:2], n)
    buckets: List[PatchBucket] = []
    entries = info["entries"]
    i = 0
    while i < len(entries):
        b = entries[i][10]
        j = i
        while j < len(entries) and entries[j][10] == b:
            j += 1
        ph, pw = entries[i][1] - entries[i][0], entries[i][3] - entries[i][2]
        r0, r1 = entries[i][8], entries[i][8] + (j - i) * ph * pw
        buckets.append(PatchBucket((ph, pw), hs[r0:r1].view(j - i, ph * pw, hs.shape[-1]),
                                   ids[r0:r1].view(j - i, ph * pw, ids.shape[-1]),
                                   [_geometry(e) for e in entries[i:j]]))
        i = j
    return buckets


_RAMPS: Dict[tuple, torch.Tensor] = {}


def feather_ramps(halo: int, mode: str = "cosine", power: float = 1.0, device=None) -> torch.Tensor:
    """Ramp table of pq_fuse_patches: for every length m = 1 .. halo the rising ramp r(linspace(0, 1, m)) and the
    falling ramp r(linspace(1, 0, m)), interleaved, r = the reference's _smooth_ramp (flux/routing.py:21-31).
    A constant per (halo, mode, power), evaluated once with torch's fp32 operators and kept on the device."""
    dev = _device(device)
    key = (int(halo), mode, float(power), str(dev))
    t = _RAMPS.get(key)
    if t is None:
        vals = [0.0, 0.0]    # halo 0: never read
        if halo > 0:
            vals = []
            for m in range(1, int(halo) + 1):
                up = _smooth_ramp(torch.linspace(0.0, 1.0, m), mode, power)
                dn = _smooth_ramp(torch.linspace(1.0, 0.0, m), mode, power)
                vals.extend(torch.stack([up, dn], 1).reshape(-1).tolist())
        t = torch.tensor(vals, dtype=torch.float32).to(dev)
        _RAMPS[key] = t
    return t


def _smooth_ramp(values: torch.Tensor, mode: str, power: float) -> torch.Tensor:
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


def fuse_patches(background: torch.Tensor, patch_out: torch.Tensor, route: RouteTable, *, fusion_beta: float = 1.0,
                 feather_mode: str = "cosine", feather_power: float = 1.0,
                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """pq_fuse_patches: background [H * W, C] or [1, H, W, C], patch_out [rows, C] in route.rows order. Returns the
    fused prediction in background's shape."""
    if not 0.0 <= float(fusion_beta) <= 1.0:
        raise ValueError(f"fusion_beta must be in [0,1], got {fusion_beta}")
    H, W = route.token_hw
    C = int(background.shape[-1])
    bg = background.reshape(H * W, C)
    po = patch_out.reshape(-1, C)
    if bg.stride(1) != 1 or po.stride(1) != 1:
        raise AssertionError("fuse_patches: channel dimension must be contiguous")
    if out is None:
        out = torch.empty_like(background)
    o2 = out.reshape(H * W, C)
    ramp = feather_ramps(route.halo, feather_mode, feather_power, background.device)
    if po.numel() == 0:   # no patch rows: the kernel reads no prediction; hand it a valid pointer all the same
        po = bg
    _lib.check(_lib.load().pq_fuse_patches(_lib.ptr(bg), bg.stride(0), _lib.ptr(po), po.stride(0),
                                           _lib.ptr(route.table), _lib.ptr(route.counts), _lib.ptr(ramp),
                                           int(route.halo), float(fusion_beta), H, W, C, _lib.dtype_code(background.dtype),
                                           _lib.ptr(o2), o2.stride(0), _lib.stream_of(background.device)),
               "fuse_patches")
    return out


def fuse_patch_predictions(background: torch.Tensor, bucket_outputs: Sequence, *, route: RouteTable,
                           fusion_beta: float, feather_mode: str = "cosine",
                           feather_power: float = 1.0) -> torch.Tensor:
    """Mirror of flux/routing.py:328-379 on the device: background [1, H, W, C]; bucket_outputs the
    (bucket, output [k, h * w, C]) pairs of build_patch_buckets' buckets, in order (chunks of a bucket in order)."""
    if int(background.shape[0]) != 1:
        raise ValueError("Only batch-one full-image fusion is supported")
    C = int(background.shape[-1])
    parts = []
    for bucket, output in bucket_outputs:
        if output.ndim != 3:
            raise ValueError(f"Expected bucket output K,N,C, got {tuple(output.shape)}")
        if int(output.shape[0]) != len(bucket.geometries):
            raise ValueError("Bucket output batch does not match geometry count")
        ph, pw = bucket.patch_hw
        if int(output.shape[1]) != ph * pw or int(output.shape[2]) != C:
            raise ValueError("Bucket output shape does not match patch geometry/background channels")
        parts.append(output.reshape(-1, C))
    if not parts:
        po = background.reshape(-1, C)[:0]
    else:
        po = torch.cat(parts) if len(parts) > 1 else parts[0]
    if int(po.shape[0]) != int(route.counts[1].item()):
        raise ValueError("bucket outputs do not cover the route table's rows")
    return fuse_patches(background, po, route, fusion_beta=fusion_beta, feather_mode=feather_mode,
                        feather_power=feather_power)
