"""GPU parity of the routed-executor geometry and fusion kernels against the CPU oracle (oracle/routing_ref.py,
oracle.route_rows_union):
* pq_route_union_rows: the config-4 list bit for bit (count, sha256 of the golden record), random masks, halo 0,
  halo wider than a leaf, empty and full masks;
* pq_route_patches: table (halo / core boxes, row offsets, source box, bucket) and rows in build_patch_buckets order
  (flux/routing.py:253-315), packing offset 1, empty mask, a too-small rows buffer reported, not overrun;
* pq_gather_rows: hidden states and ids in extraction order, equal to torch indexing;
* pq_fuse_patches: bit-identical to the op-by-op torch CPU restatement of fuse_patch_predictions
  (flux/routing.py:328-379), bf16 and fp16, fusion_beta 1 and 0.5, halo 0 and 1, no patch at all.
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from conftest import bits

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _c4_mask():
    rec = json.load(open(os.path.join(GOLD, "route_c4.json")))
    return rec, np.array([[c == "1" for c in r] for r in rec["mask_rows"]])


def test_route_union_c4(oracle, cuda):
    from pyraquant_amd import routing

    rec, mask = _c4_mask()
    rows = routing.routed_row_index(torch.from_numpy(mask), device=cuda)
    got = rows.cpu().numpy()
    assert got.size == rec["union_rows"] == 33316
    assert hashlib.sha256(got.astype("<i4").tobytes()).hexdigest() == rec["sha256_int32_le"]
    assert np.array_equal(got, oracle.route_rows_union(mask.astype(np.uint8), 16, 2))


@pytest.mark.parametrize("n,leaf,halo,p,seed", [(16, 16, 2, 0.35, 1), (8, 32, 8, 0.5, 2), (5, 12, 0, 0.4, 3),
                                                (6, 8, 11, 0.3, 4), (16, 16, 2, 0.0, 5), (16, 16, 2, 1.0, 6),
                                                (3, 40, 1, 0.6, 7)])
def test_route_union_random(oracle, cuda, n, leaf, halo, p, seed):
    from pyraquant_amd import routing

    g = torch.Generator().manual_seed(seed)
    mask = (torch.rand(n, n, generator=g) < p).numpy()
    rows, count = routing.union_rows(torch.from_numpy(mask).to(cuda), leaf, halo)
    ref = oracle.route_rows_union(mask.astype(np.uint8), leaf, halo)
    c = int(count.item())
    assert c == ref.size
    assert np.array_equal(rows[:c].cpu().numpy(), ref)


def _table_ref(RR, mask, leaf_latent, halo, hw, off=0):
    patches, rows = RR.patch_geometry(RR.route_boxes(mask, leaf_latent), halo, hw, off)
    tab, o = [], 0
    for p in patches:
        oy0, oy1, ox0, ox1 = p["halo"]
        tab.append(list(p["halo"]) + list(p["core"]) + [o, p["box_index"], p["bucket"], 0])
        o += (oy1 - oy0) * (ox1 - ox0)
    return tab, rows


@pytest.mark.parametrize("n,leaf_latent,halo,hw,off,p,seed", [
    (16, 32, 2, (256, 256), 0, None, 0),        # config 4's mask
    (8, 64, 8, (256, 256), 0, 0.4, 11),         # the reference's 4K stage: 64-latent leaves, halo 8
    (8, 64, 8, (257, 257), 1, 0.5, 12),         # packing phase 1: cores cover the straddling tokens
    (12, 10, 3, (60, 60), 0, 0.6, 13),
    (8, 64, 0, (256, 256), 0, 0.7, 14),
    (8, 64, 8, (256, 256), 0, 0.0, 15),         # nothing selected
    (32, 16, 4, (256, 256), 0, 0.5, 16),        # many boxes
])
def test_route_patches(cuda, n, leaf_latent, halo, hw, off, p, seed):
    from oracle import routing_ref as RR
    from pyraquant_amd import routing

    if p is None:
        mask = _c4_mask()[1]
    else:
        g = torch.Generator().manual_seed(seed)
        mask = (torch.rand(n, n, generator=g) < p).numpy()
    rt = routing.route_patches(torch.from_numpy(mask).to(cuda), leaf_latent=leaf_latent, halo_tokens=halo,
                               token_hw=hw, packing_offset_latent=off)
    info = rt.host()
    tab, rows = _table_ref(RR, mask, leaf_latent, halo, hw, off)
    assert info["patches"] == len(tab) and info["rows"] == rows.size
    assert info["buckets"] == (max(t[10] for t in tab) + 1 if tab else 0)
    assert info["entries"] == tab
    assert np.array_equal(rt.rows[: rows.size].cpu().numpy(), rows)


def test_route_patches_small_buffer(cuda):
    """A rows buffer smaller than the patches' rows is flagged (RuntimeError on read) and never overrun."""
    from pyraquant_amd import routing

    mask = _c4_mask()[1]
    rt = routing.route_patches(torch.from_numpy(mask).to(cuda), leaf_latent=32, halo_tokens=2, token_hw=(256, 256),
                               max_rows=1000)
    guard = torch.full((4096,), -7, dtype=torch.int32, device=cuda)
    rt2 = routing.RouteTable(rt.table, rt.counts, guard[:1000], rt.token_hw, rt.halo)
    with pytest.raises(RuntimeError):
        rt2.host()
    # same call again into the head of a guarded buffer: nothing past max_rows is written
    from pyraquant_amd import _lib

    m = torch.from_numpy(mask).to(cuda).to(torch.uint8)
    _lib.check(_lib.load().pq_route_patches(_lib.ptr(m), 16, 16, 32, 2, 256, 256, 0, _lib.ptr(rt.table),
                                            _lib.ptr(rt.counts), _lib.ptr(guard), 1000,
                                            _lib.stream_of(cuda)), "route_patches")
    assert bool((guard[1000:] == -7).all())


def test_build_patch_buckets_gather(cuda):
    """hidden_states / img_ids extracted by one gather each equal torch indexing with the oracle's rows; bucket
    shapes and geometries follow the table."""
    from oracle import routing_ref as RR
    from pyraquant_amd import routing

    g = torch.Generator().manual_seed(21)
    mask = (torch.rand(8, 8, generator=g) < 0.4).numpy()
    H = W = 256
    hs = torch.randn(1, H * W, 64, generator=g).to(torch.bfloat16).to(cuda)
    ids = torch.randn(H * W, 3, generator=g).to(cuda)
    rt = routing.route_patches(torch.from_numpy(mask).to(cuda), leaf_latent=64, halo_tokens=8, token_hw=(H, W))
    buckets = routing.build_patch_buckets(hs, ids, route=rt)
    patches, rows = RR.patch_geometry(RR.route_boxes(mask, 64), 8, (H, W))
    ri = torch.from_numpy(rows).long().to(cuda)
    got_hs = torch.cat([b.hidden_states.reshape(-1, 64) for b in buckets])
    got_ids = torch.cat([b.img_ids.reshape(-1, 3) for b in buckets])
    assert torch.equal(got_hs, hs[0, ri])
    assert torch.equal(got_ids, ids[ri])
    geoms = [gm for b in buckets for gm in b.geometries]
    assert [gm.halo_box for gm in geoms] == [p["halo"] for p in patches]
    assert [gm.inner_box_in_patch for gm in geoms] == [p["inner"] for p in patches]
    shapes = [b.patch_hw for b in buckets]
    assert shapes == sorted(set(shapes))


@pytest.mark.parametrize("dtype,beta,halo,leaf_latent,n,hw,C,seed", [
    (torch.bfloat16, 1.0, 2, 32, 16, (256, 256), 64, 31),     # config 4's geometry, FLUX packed channels
    (torch.bfloat16, 1.0, 8, 64, 8, (256, 256), 64, 32),      # the reference's 4K stage
    (torch.float16, 0.5, 8, 64, 8, (256, 256), 64, 33),
    (torch.bfloat16, 0.75, 1, 16, 6, (48, 48), 16, 34),       # 1-token halo: falling ramp of length 1 is 1
    (torch.bfloat16, 1.0, 0, 16, 6, (48, 48), 8, 35),         # no halo
    (torch.bfloat16, 1.0, 5, 12, 10, (60, 60), 24, 36),       # halo wider than a leaf: many overlaps
])
def test_fuse_patches(cuda, dtype, beta, halo, leaf_latent, n, hw, C, seed):
    from oracle import routing_ref as RR
    from pyraquant_amd import routing

    g = torch.Generator().manual_seed(seed)
    mask = (torch.rand(n, n, generator=g) < 0.45).numpy()
    H, W = hw
    bg = torch.randn(H, W, C, generator=g).to(dtype)
    patches, rows = RR.patch_geometry(RR.route_boxes(mask, leaf_latent), halo, hw)
    po = (torch.randn(rows.size, C, generator=g) * 2).to(dtype)
    ref = RR.fuse_patch_predictions(bg, patches, po, fusion_beta=beta)
    rt = routing.route_patches(torch.from_numpy(mask).to(cuda), leaf_latent=leaf_latent, halo_tokens=halo,
                               token_hw=hw)
    out = routing.fuse_patches(bg.to(cuda), po.to(cuda), rt, fusion_beta=beta)
    assert np.array_equal(bits(out), bits(ref))


def test_fuse_patch_predictions_api(cuda):
    """The reference-shaped entry (background [1, H, W, C], per-bucket outputs from build_patch_buckets) gives the
    oracle's result; no selected leaf leaves the background (up to -0 -> +0, as torch computes it)."""
    from oracle import routing_ref as RR
    from pyraquant_amd import routing

    g = torch.Generator().manual_seed(41)
    mask = (torch.rand(8, 8, generator=g) < 0.4).numpy()
    H = W = 256
    C = 64
    bg = torch.randn(1, H, W, C, generator=g).to(torch.bfloat16)
    hs = torch.randn(1, H * W, C, generator=g).to(torch.bfloat16).to(cuda)
    ids = torch.zeros(H * W, 3, device=cuda)
    rt = routing.route_patches(torch.from_numpy(mask).to(cuda), leaf_latent=64, halo_tokens=8, token_hw=(H, W))
    buckets = routing.build_patch_buckets(hs, ids, route=rt)
    outs = [(b, torch.tanh(b.hidden_states.float()).to(torch.bfloat16)) for b in buckets]   # a stand-in prediction
    fused = routing.fuse_patch_predictions(bg.to(cuda), outs, route=rt, fusion_beta=1.0)
    patches, rows = RR.patch_geometry(RR.route_boxes(mask, 64), 8, (H, W))
    po = torch.cat([o.reshape(-1, C).cpu() for _, o in outs])
    ref = RR.fuse_patch_predictions(bg[0], patches, po)
    assert np.array_equal(bits(fused[0]), bits(ref))
    empty = torch.zeros(8, 8, dtype=torch.bool)
    rt0 = routing.route_patches(empty.to(cuda), leaf_latent=64, halo_tokens=8, token_hw=(H, W))
    f0 = routing.fuse_patch_predictions(bg.to(cuda), [], route=rt0, fusion_beta=1.0)
    assert np.array_equal(bits(f0), bits(RR.fuse_patch_predictions(bg[0], [], po[:0])[None]))
