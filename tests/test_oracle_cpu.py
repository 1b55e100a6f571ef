"""CPU tests of the oracle (oracle/pq_oracle.c via oracle/oracle.py): each oracle function is pinned by a check
that does not restate its own formula -- the committed golden fixtures (computed by torch's CPU operators on the
reference's torch lines, tests/golden/make_golden.py), torch's own integer matmul, float64 / exact-rational
arithmetic, closed-form special cases and invariants -- chosen so that a plausible mistake (a reciprocal instead of
a division, round-half-up, a dropped clamp, a transposed operand, a wrong operation order) fails at least one.
A planted-mistake section runs deliberately wrong variants through the same checks to show that they fail."""
import hashlib
import json
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

from conftest import bits

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


# ------------------------------------------------------------------------------------------- 16-bit conversions
def test_f16_conversions_match_torch(oracle):
    g = torch.Generator().manual_seed(0)
    x = torch.cat([torch.randn(4000, generator=g) * s for s in (1e-6, 1e-3, 1.0, 1e3, 6e4)])
    x = torch.cat([x, torch.tensor([0.0, -0.0, float("inf"), -float("inf"), 65504.0, 65520.0, 1e-8, 2.0 ** -24,
                                    2.0 ** -25, 3 * 2.0 ** -26, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11])])
    for dt, code in ((torch.bfloat16, 0), (torch.float16, 1)):
        ref = bits(x.to(dt))
        got = oracle.from_f32(x.numpy(), code)
        assert np.array_equal(got, ref), dt
        back = oracle.to_f32(ref, code)
        assert np.array_equal(back.view(np.uint32), x.to(dt).float().numpy().view(np.uint32)), dt


# ------------------------------------------------------------------------------------------- A. quantizer
@pytest.mark.parametrize("fixture", ["quant_bf16.npz", "quant_f16.npz"])
def test_quant_rows_golden(oracle, fixture):
    """Oracle codes and scales equal the torch-computed golden vectors bit for bit."""
    f = _load(fixture)
    q, s = oracle.quant_rows(f["x_bits"], int(f["dtype"]))
    assert np.array_equal(q, f["q"])
    assert np.array_equal(s.view(np.uint32), f["s"].view(np.uint32))


def _f32_round(fr: Fraction) -> float:
    """Round a rational to the nearest binary32 value, ties to even (subnormals included)."""
    if fr == 0:
        return 0.0
    sign = -1 if fr < 0 else 1
    fr = abs(fr)
    e = fr.numerator.bit_length() - fr.denominator.bit_length()
    if Fraction(2) ** e > fr:
        e -= 1
    e = max(e, -126)                                     # below 2^-126 the quantum stays 2^-149
    q = round(fr * Fraction(2) ** (23 - e))              # Fraction.__round__: half to even
    return sign * float(Fraction(q) * Fraction(2) ** (e - 23))


def _exact_code(x: float, s: float) -> int:
    """clamp(round_half_even(fl32(x / s)), -127, 127) with the fp32 division done in exact rationals."""
    return max(-127, min(127, round(Fraction(_f32_round(Fraction(x) / Fraction(s))))))


def test_quant_rows_bruteforce_rational(oracle):
    """Tiny rows against exact rational arithmetic: s = fl32(a / 127), q = rne(fl32(x / s)), clamped."""
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(6, 24, generator=g) * torch.tensor([1e-3, 0.1, 1.0, 3.0, 50.0, 1e4])[:, None]).to(torch.bfloat16)
    xb = bits(x)
    q, s = oracle.quant_rows(xb, 0)
    xf = x.float().numpy()
    for m in range(x.shape[0]):
        a = max(float(np.abs(xf[m]).max()), float(np.float32(1e-8)))
        s_exact = np.float32(_f32_round(Fraction(a) / 127))
        assert s[m] == s_exact
        for k in range(x.shape[1]):
            assert q[m, k] == _exact_code(float(xf[m, k]), float(s_exact)), (m, k)


def test_quant_rows_invariants(oracle):
    """|q| <= 127; each non-zero row reaches 127 in magnitude at its absmax; sign symmetry; an all-zero row has
    s = fl32(1e-8) / 127 and q = 0; scaling a row by 2^k scales s by 2^k and keeps q."""
    from pyraquant_amd.workloads import make_x

    x = make_x(64, 640, torch.bfloat16, seed=5)
    x[3] = 0
    q, s = oracle.quant_rows(bits(x), 0)
    assert np.abs(q.astype(np.int32)).max() <= 127
    nz = np.arange(64) != 3
    assert (np.abs(q[nz].astype(np.int32)).max(axis=1) == 127).all()
    assert (q[3] == 0).all() and s[3] == np.float32(np.float32(1e-8) / np.float32(127))
    qn, sn = oracle.quant_rows(bits(-x), 0)
    assert np.array_equal(qn, -q) and np.array_equal(sn, s)
    q4, s4 = oracle.quant_rows(bits(x * 4), 0)
    assert np.array_equal(q4[nz], q[nz]) and np.array_equal(s4[nz], s[nz] * 4)


def test_quant_rows_ties_round_to_even(oracle):
    """Absmax 127 gives s = 1, so x = k + 1/2 are exact ties: rint goes to the even neighbour."""
    x = torch.zeros(1, 256)
    x[0, 0] = 127.0
    x[0, 1:255] = torch.arange(-127, 127).float() + 0.5
    q, s = oracle.quant_rows(bits(x.to(torch.bfloat16)), 0)
    assert s[0] == 1.0
    v = x[0, 1:255].numpy()
    expect = np.where(np.floor(v) % 2 == 0, np.floor(v), np.ceil(v))
    assert np.array_equal(q[0, 1:255].astype(np.float32), np.clip(expect, -127, 127))


def test_quant_rows_matches_torch_restatement(oracle):
    """Against oracle/torch_ref.py (torch CPU, deploy/int8_exec.py:508-509) on the outlier workload, both dtypes,
    and with a gather list."""
    from oracle import torch_ref
    from pyraquant_amd.workloads import make_x

    for dt, code in ((torch.bfloat16, 0), (torch.float16, 1)):
        x = make_x(512, 3072, dt, seed=9)
        qt, st = torch_ref.quant_rows(x)
        qo, so = oracle.quant_rows(bits(x), code)
        assert np.array_equal(qo, qt.numpy()) and np.array_equal(so.view(np.uint32), st.numpy().view(np.uint32))
    idx = np.array([511, 0, 7, 7, 300], np.int32)
    qg, sg = oracle.quant_rows(bits(x), 1, idx)
    qf, sf = oracle.quant_rows(bits(x), 1)
    assert np.array_equal(qg, qf[idx]) and np.array_equal(sg, sf[idx])


def test_quant_rows_division_not_reciprocal(oracle):
    """The codes come from x / s, not x * (1 / s): on the bf16 grid the two differ for some elements, and the
    oracle agrees with the division (exact rationals) wherever they do."""
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(256, 1024, generator=g) * 3).to(torch.bfloat16)
    q, s = oracle.quant_rows(bits(x), 0)
    xf = x.float().numpy()
    recip = np.clip(np.rint(xf * (np.float32(1) / s[:, None])), -127, 127)
    differ = np.argwhere(recip != q)
    assert len(differ) > 0, "workload does not separate division from reciprocal"
    for m, k in differ[:50]:
        assert q[m, k] == _exact_code(float(xf[m, k]), float(s[m]))


# ------------------------------------------------------------------------------------------- B / G. weights
def test_quant_weight_golden(oracle):
    f = _load("weight_rtn.npz")
    q, s = oracle.quant_weight(f["w"], 0)
    assert np.array_equal(q, f["q_ch"]) and np.array_equal(s.view(np.uint32), f["s_ch"].view(np.uint32))
    qg, sg = oracle.quant_weight(f["w"], 32)
    assert np.array_equal(qg, f["q_g32"]) and np.array_equal(sg.view(np.uint32), f["s_g32"].view(np.uint32))


def test_quant_weight_group_invariants(oracle):
    """qdq_weight group semantics (pyraquant/quantizers_weight.py:890-933): the group absmax element maps to
    +-127 exactly; at most 255 levels per group; changing one group leaves the other groups' codes and scales
    unchanged; group = K equals per-channel."""
    g = torch.Generator().manual_seed(4)
    w = (torch.randn(16, 256, generator=g) * 0.02).numpy()
    q, s = oracle.quant_weight(w, 32)
    wg = w.reshape(16, 8, 32)
    am = np.abs(wg).argmax(axis=2)
    qg = q.reshape(16, 8, 32)
    for n in range(16):
        for j in range(8):
            assert abs(int(qg[n, j, am[n, j]])) == 127
            assert len(np.unique(qg[n, j])) <= 255
    w2 = w.copy()
    w2[:, 32:64] *= 7.0
    q2, s2 = oracle.quant_weight(w2, 32)
    keep = np.r_[0:32, 64:256]
    assert np.array_equal(q2[:, keep], q[:, keep])
    assert np.array_equal(np.delete(s2, 1, axis=1), np.delete(s, 1, axis=1))
    qk, sk = oracle.quant_weight(w, 256)
    qc, sc = oracle.quant_weight(w, 0)
    assert np.array_equal(qk, qc) and np.array_equal(sk[:, 0], sc)


def test_quant_weight_matches_torch_restatement(oracle):
    from oracle import torch_ref

    g = torch.Generator().manual_seed(6)
    w = torch.randn(300, 640, generator=g) * 0.02
    qt, st = torch_ref.quant_weight(w)
    qo, so = oracle.quant_weight(w.numpy(), 0)
    assert np.array_equal(qo, qt.numpy()) and np.array_equal(so.view(np.uint32), st.numpy().view(np.uint32))


# ------------------------------------------------------------------------------------------- C. int32 GEMM
def test_gemm_i32_golden_and_int_mm(oracle):
    f = _load("linear_lr.npz")
    acc = oracle.gemm_i32(f["q"], f["w_q"])
    assert np.array_equal(acc, f["acc"])
    g = torch.Generator().manual_seed(2)
    a = torch.randint(-127, 128, (67, 320), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (96, 320), generator=g, dtype=torch.int8)
    assert np.array_equal(oracle.gemm_i32(a.numpy(), w.numpy()), torch._int_mm(a, w.t()).numpy())
    assert np.array_equal(oracle.gemm_i32(a.numpy(), w.numpy()),
                          a.numpy().astype(np.int64) @ w.numpy().astype(np.int64).T)


def test_gemm_group_partials_sum_to_acc(oracle):
    g = torch.Generator().manual_seed(5)
    a = torch.randint(-127, 128, (9, 128), generator=g, dtype=torch.int8).numpy()
    w = torch.randint(-127, 128, (16, 128), generator=g, dtype=torch.int8).numpy()
    part = oracle.gemm_group_i32(a, w, 32)
    assert part.shape == (9, 16, 4)
    assert np.array_equal(part.sum(axis=2), oracle.gemm_i32(a, w))
    assert np.array_equal(part[:, :, 1], oracle.gemm_i32(a[:, 32:64].copy(), w[:, 32:64].copy()))


# ------------------------------------------------------------------------------------------- C / D epilogue
def test_epilogue_per_channel_golden(oracle):
    """Bit-exact against torch's acc.float() * (s_row * s_col) + bias (deploy/int8_exec.py:506)."""
    f = _load("linear_lr.npz")
    y = oracle.epilogue_f32(f["acc"], f["s"], f["w_s"], f["bias"])
    assert np.array_equal(y.view(np.uint32), f["y_nolr"].view(np.uint32))


def test_epilogue_operation_order(oracle):
    """acc * (s_row * s_col) and (acc * s_row) * s_col differ in the last bit for some elements; the oracle
    follows torch's (reference) grouping on all of them."""
    g = torch.Generator().manual_seed(8)
    acc = torch.randint(-2 ** 24, 2 ** 24, (64, 96), generator=g, dtype=torch.int32)
    sr = torch.rand(64, generator=g) * 0.01 + 1e-4
    sc = torch.rand(96, generator=g) * 1e-3 + 1e-5
    ref = acc.float() * (sr[:, None] * sc[None, :])
    alt = (acc.float() * sr[:, None]) * sc[None, :]
    assert not torch.equal(ref, alt)
    y = oracle.epilogue_f32(acc.numpy(), sr.numpy(), sc.numpy())
    assert np.array_equal(y.view(np.uint32), ref.numpy().view(np.uint32))


def test_epilogue_lowrank_vs_float64(oracle):
    """With the low-rank branch: within fp32 rounding of the float64 value of the same expression."""
    f = _load("linear_lr.npz")
    y = oracle.epilogue_f32(f["acc"], f["s"], f["w_s"], f["bias"], f["t_bits"], f["l2_bits"], 0)
    ref = f["y_lr_f64"]
    err = np.abs(y.astype(np.float64) - ref)
    assert err.max() <= 1e-5 * np.abs(ref).max()
    # the branch is really added: removing it moves the result by far more than the tolerance
    y0 = oracle.epilogue_f32(f["acc"], f["s"], f["w_s"], f["bias"])
    assert np.abs(y0.astype(np.float64) - ref).max() > 100 * err.max()


def test_epilogue_group_equal_scales_reduces_to_channel(oracle):
    """With every group scale of a row equal to the channel scale, the group-32 epilogue equals the per-channel
    epilogue within fp32 rounding (closed form), and a transposed group-scale layout does not."""
    g = torch.Generator().manual_seed(12)
    a = torch.randint(-127, 128, (20, 256), generator=g, dtype=torch.int8).numpy()
    w = torch.randint(-127, 128, (32, 256), generator=g, dtype=torch.int8).numpy()
    sr = (torch.rand(20, generator=g) * 0.01 + 1e-3).numpy()
    sc = (torch.rand(32, generator=g) * 1e-3 + 1e-5).numpy()
    part = oracle.gemm_group_i32(a, w, 32)
    yg = oracle.epilogue_f32(part, sr, np.repeat(sc[:, None], 8, axis=1))
    yc = oracle.epilogue_f32(oracle.gemm_i32(a, w), sr, sc)
    assert np.allclose(yg, yc, rtol=1e-5, atol=1e-6 * np.abs(yc).max())
    sg = (torch.rand(32, 8, generator=g) * 1e-3 + 1e-5).numpy()
    y1 = oracle.epilogue_f32(part, sr, sg)
    ref64 = (part.astype(np.float64) * sg[None, :, :].astype(np.float64)).sum(axis=2) * sr[:, None]
    assert np.abs(y1 - ref64).max() <= 1e-5 * np.abs(ref64).max()


# ------------------------------------------------------------------------------------------- E. low-rank down
def test_lowrank_down_golden_and_float64(oracle):
    f = _load("linear_lr.npz")
    t = oracle.lowrank_down(f["x_bits"], 0, f["l1_bits"])
    tf = oracle.to_f32(t, 0)
    ref = oracle.to_f32(f["t_bits"], 0)                       # torch CPU bf16 matmul
    x64 = oracle.to_f32(f["x_bits"], 0).astype(np.float64)
    l64 = oracle.to_f32(f["l1_bits"], 0).astype(np.float64)
    exact = x64 @ l64
    # both are within one bf16 rounding (+ fp32 accumulation) of the exact product
    tol = 2 ** -7 * np.abs(exact) + 1e-6 * np.abs(exact).max()
    assert (np.abs(tf - exact) <= tol).all()
    assert (np.abs(ref - exact) <= tol).all()


# ------------------------------------------------------------------------------------------- whole layer
def test_linear_golden_codes_and_output(oracle):
    f = _load("linear_lr.npz")
    o = oracle.linear(f["x_bits"], 0, f["w_q"], f["w_s"], f["bias"], 0, f["l1_bits"], f["l2_bits"])
    assert np.array_equal(o["q"], f["q"]) and np.array_equal(o["acc"], f["acc"])
    err = np.abs(o["y"].astype(np.float64) - f["y_lr_f64"])
    assert err.max() <= 1e-2 * np.abs(f["y_lr_f64"]).max()


# ------------------------------------------------------------------------------------------- I. routing
def _c4_mask():
    rec = json.load(open(os.path.join(GOLD, "route_c4.json")))
    return rec, np.array([[c == "1" for c in r] for r in rec["mask_rows"]])


def test_route_rows_c4_golden(oracle):
    """Config-4 row set: the C brute force, the union of the restated patch geometry (flux/routing.py:253-315) and
    the golden record agree (count, hash); the leaf map is the seeded Bernoulli(0.35) of the record."""
    from oracle import routing_ref as RR
    from pyraquant_amd import routing

    rec, mask = _c4_mask()
    sel = routing.leaf_mask()
    assert int(sel.sum()) == rec["active_leaves"] == 103
    assert np.array_equal(sel.numpy(), mask)
    rows_c = oracle.route_rows_union(mask.astype(np.uint8), 16, 2)
    _, prow = RR.patch_geometry(RR.route_boxes(mask, 32), 2, (256, 256))
    assert np.array_equal(rows_c, np.unique(prow))
    assert rows_c.size == rec["union_rows"] == 33316
    assert hashlib.sha256(rows_c.astype("<i4").tobytes()).hexdigest() == rec["sha256_int32_le"]
    assert np.all(np.diff(rows_c) > 0)
    core = oracle.route_rows_union(mask.astype(np.uint8), 16, 0)
    assert core.size == rec["core_rows"] == 26368 == 103 * 256


def test_route_rows_small_cases(oracle):
    """Hand-countable cases: one interior leaf with halo 2 covers 20 x 20 rows; a corner leaf is clamped to
    18 x 18; two adjacent leaves share their halo overlap once."""
    m = np.zeros((4, 4), np.uint8)
    m[1, 1] = 1
    assert oracle.route_rows_union(m, 16, 2).size == 20 * 20
    m[:] = 0
    m[0, 0] = 1
    assert oracle.route_rows_union(m, 16, 2).size == 18 * 18
    m[:] = 0
    m[1, 1] = m[1, 2] = 1
    assert oracle.route_rows_union(m, 16, 2).size == 20 * 36


def test_route_boxes_and_patch_order():
    """Row-run boxes (flux/run_flux.py:340-355) of a hand mask, and the extraction order of flux/routing.py:253-315:
    shapes ascending, box order inside a shape, rows row-major, halo overlaps repeated."""
    from oracle import routing_ref as RR

    m = np.array([[0, 1, 1, 0, 1],
                  [1, 1, 1, 1, 1],
                  [0, 0, 0, 0, 1]], bool)
    boxes = RR.route_boxes(m, 8)
    assert boxes == [(0, 8, 8, 24), (0, 8, 32, 40), (8, 16, 0, 40), (16, 24, 32, 40)]
    patches, rows = RR.patch_geometry(boxes, 1, (12, 20))
    # token cores (latent / 2): (0,4,4,12) (0,4,16,20) (4,8,0,20) (8,12,16,20); halo 1 clamped to the 12 x 20
    # grid gives shapes 5x10, 5x5, 6x20, 5x5: buckets (5,5) (5,5) (5,10) (6,20)
    shapes = [(p["halo"][1] - p["halo"][0], p["halo"][3] - p["halo"][2]) for p in patches]
    assert shapes == sorted(shapes)
    assert [p["box_index"] for p in patches] == [1, 3, 0, 2]
    assert patches[0]["halo"] == (0, 5, 15, 20) and patches[0]["inner"] == (0, 4, 1, 5)
    assert [p["bucket"] for p in patches] == [0, 0, 1, 2]
    assert rows.size == sum(h * w for h, w in shapes)
    assert list(rows[:5]) == [15, 16, 17, 18, 19]          # first patch, first row, row-major
    # the c4 mask: the patch rows cover the union exactly, with overlaps repeated
    _, mask = _c4_mask()
    _, prow = RR.patch_geometry(RR.route_boxes(mask, 32), 2, (256, 256))
    assert prow.size > np.unique(prow).size


def test_unpacked_box_errors():
    """Validation of flux/routing.py:202-232: negative, odd and empty boxes raise ValueError; offset 1 covers both
    straddling tokens."""
    from oracle import routing_ref as RR

    assert RR.token_box((0, 4, 2, 8)) == (0, 2, 1, 4)
    assert RR.token_box((0, 4, 2, 8), 1) == (0, 3, 1, 5)
    for bad in ((-2, 4, 0, 4), (1, 4, 0, 4), (4, 4, 0, 4)):
        with pytest.raises(ValueError):
            RR.token_box(bad)


def test_feather_ramp_closed_form():
    """The cosine ramp is 0.5 - 0.5 cos(pi u) on linspace points (float64 closed form within fp32 rounding), starts
    at 0, ends at 1, and the falling ramp mirrors the rising one except at length 1; the mask is 1 over the core and min of the two
    edge ramps in a halo corner."""
    import torch

    from oracle import routing_ref as RR

    for m in range(1, 9):
        up = RR.smooth_ramp(torch.linspace(0.0, 1.0, m)).double().numpy()
        dn = RR.smooth_ramp(torch.linspace(1.0, 0.0, m)).double().numpy()
        u = np.linspace(0.0, 1.0, m)
        assert np.allclose(up, 0.5 - 0.5 * np.cos(np.pi * u), atol=3e-7)
        if m == 1:   # linspace(0, 1, 1) = [0] but linspace(1, 0, 1) = [1]: a 1-token falling halo keeps weight 1
            assert up[0] == 0.0 and dn[0] == 1.0
            continue
        assert np.allclose(dn, up[::-1], atol=3e-7)
        assert up[0] == 0.0 and up[-1] == 1.0
    mask = RR.halo_feather_mask((8, 10), (3, 6, 2, 8), torch.float32).numpy()
    assert np.all(mask[3:6, 2:8] == 1.0)
    yr = RR.smooth_ramp(torch.linspace(0.0, 1.0, 3)).numpy()
    xr = RR.smooth_ramp(torch.linspace(0.0, 1.0, 2)).numpy()
    assert mask[1, 1] == min(yr[1], xr[1]) and mask[0, 5] == 0.0 and mask[4, 0] == 0.0


def _fusion_case(seed, H=24, W=28, C=16, dtype=None, halo=3):
    import torch

    from oracle import routing_ref as RR

    dtype = dtype or torch.bfloat16
    g = torch.Generator().manual_seed(seed)
    m = (torch.rand(3, 3, generator=g) < 0.5).numpy()
    m[1, 1] = True
    patches, rows = RR.patch_geometry(RR.route_boxes(m, 16), halo, (H, W))
    bg = torch.randn(H, W, C, generator=g).to(dtype)
    po = torch.randn(rows.size, C, generator=g).to(dtype)
    return RR, patches, rows, bg, po


def test_fusion_closed_forms():
    """fuse_patch_predictions: no patch -> background bits; fusion_beta 0 -> background; a token inside exactly one
    core -> that patch's prediction bits; two equal full weights -> their mean within one rounding."""
    import torch

    RR, patches, rows, bg, po = _fusion_case(1)
    H, W, C = bg.shape
    assert torch.equal(RR.fuse_patch_predictions(bg, [], po[:0]), bg)
    assert torch.equal(RR.fuse_patch_predictions(bg, patches, po, fusion_beta=0.0), bg)
    out = RR.fuse_patch_predictions(bg, patches, po)
    cover = np.zeros((H, W), int)
    for p in patches:
        y0, y1, x0, x1 = p["halo"]
        cover[y0:y1, x0:x1] += 1
    off = 0
    for p in patches:
        y0, y1, x0, x1 = p["halo"]
        cy0, cy1, cx0, cx1 = p["core"]
        pw = x1 - x0
        for y in range(cy0, cy1):
            for x in range(cx0, cx1):
                if cover[y, x] == 1:
                    assert torch.equal(out[y, x], po[off + (y - y0) * pw + (x - x0)])
        off += (y1 - y0) * pw
    assert torch.equal(out[cover == 0], bg[torch.from_numpy(cover == 0)])
    # two identical patches over the same core: the blend of a prediction with itself is that prediction
    two = [patches[0], patches[0]]
    n0 = (patches[0]["halo"][1] - patches[0]["halo"][0]) * (patches[0]["halo"][3] - patches[0]["halo"][2])
    o2 = RR.fuse_patch_predictions(bg, two, torch.cat([po[:n0], po[:n0]]))
    y0, y1, x0, x1 = patches[0]["core"]
    ref = out if cover[y0:y1, x0:x1].max() == 1 else None
    if ref is not None:
        assert torch.equal(o2[y0:y1, x0:x1], ref[y0:y1, x0:x1])


def test_fusion_against_float64_blend():
    """The op-by-op 16-bit fusion stays within a few 16-bit roundings of the float64 blend
    (1 - b) bg + b (sum beta_i out_i / sum beta_i), b = min(sum beta_i, 1), for bf16 and fp16."""
    import torch

    for dt, tol in ((torch.bfloat16, 4 * 2.0 ** -8), (torch.float16, 4 * 2.0 ** -11)):
        RR, patches, rows, bg, po = _fusion_case(7, dtype=dt)
        H, W, C = bg.shape
        out = RR.fuse_patch_predictions(bg, patches, po).double()
        num = torch.zeros(H, W, C, dtype=torch.float64)
        den = torch.zeros(H, W, 1, dtype=torch.float64)
        off = 0
        for p in patches:
            y0, y1, x0, x1 = p["halo"]
            ph, pw = y1 - y0, x1 - x0
            beta = RR.halo_feather_mask((ph, pw), p["inner"], torch.float64)[:, :, None]
            num[y0:y1, x0:x1] += beta * po[off:off + ph * pw].double().reshape(ph, pw, C)
            den[y0:y1, x0:x1] += beta
            off += ph * pw
        b = den.clamp(0, 1)
        ref = (1 - b) * bg.double() + b * torch.where(den > 0, num / den.clamp_min(1e-30), torch.zeros_like(num))
        scale = ref.abs().clamp_min(1.0)
        assert float(((out - ref).abs() / scale).max()) <= tol


# ------------------------------------------------------------------------------------------- weight fold
def test_fold_one_closed_forms():
    """The smoothing / shift fold (deploy/run_flux_latency.py:219-239): no smooth and no shift is the identity;
    a power-of-two smooth halves every normal weight exactly; a per-channel smooth of equal values equals the
    scalar form; the shift term is within 16-bit rounding of the float64 dot product (per-channel and scalar);
    a planted multiply-instead-of-divide fails."""
    import torch

    from oracle import torch_ref as T

    g = torch.Generator().manual_seed(3)
    for dt in (torch.bfloat16, torch.float16):
        W = (torch.randn(64, 96, generator=g) * 0.05).to(dt)
        b = (torch.randn(64, generator=g) * 0.01).to(dt)
        w0, b0 = T.fold_one(W, None, None, b)
        assert torch.equal(w0, W) and torch.equal(b0, b)
        w2, _ = T.fold_one(W, torch.tensor(2.0), None, b)
        normal = W.float().abs() > (2.0 ** -120 if dt == torch.bfloat16 else 2.0 ** -13)
        assert torch.equal((w2.float() * 2)[normal], W.float()[normal])
        ws, _ = T.fold_one(W, torch.tensor(1.7), None, b)
        wv, _ = T.fold_one(W, torch.full((96,), 1.7), None, b)
        assert torch.equal(ws, wv)
        sm = torch.rand(96, generator=g) + 0.5
        sh = torch.randn(96, generator=g) * 0.1
        wf, bf = T.fold_one(W, sm, sh, b)
        ref = b.double() + (W.double() / sm.double()) @ sh.double()
        ulp = 2.0 ** -8 if dt == torch.bfloat16 else 2.0 ** -11
        assert float(((bf.double() - ref).abs() / ref.abs().clamp_min(1e-3)).max()) <= 3 * ulp
        _, bs = T.fold_one(W, sm, torch.tensor(0.3), None)
        refs = (W.double() / sm.double()).sum(1) * 0.3
        assert float(((bs.double() - refs).abs() / refs.abs().clamp_min(1e-3)).max()) <= 3 * ulp
        wrong = (W.float() * sm.reshape(1, -1)).to(dt)
        assert not torch.equal(wrong, wf)


# ------------------------------------------------------------------------------------------- planted mistakes
def test_planted_mistakes_are_caught(oracle):
    """Wrong variants of the oracle's arithmetic, computed here on the CPU, fail the checks above: round half
    away from zero, a reciprocal multiply, a missing clamp of the scale, and a transposed weight."""
    f = _load("quant_bf16.npz")
    x = oracle.to_f32(f["x_bits"], 0)
    sc = np.maximum(np.abs(x).max(axis=1), np.float32(1e-8)) / np.float32(127)
    sc = sc.astype(np.float32)
    half_up = np.clip(np.sign(x / sc[:, None]) * np.floor(np.abs(x / sc[:, None]) + 0.5), -127, 127)
    assert not np.array_equal(half_up.astype(np.int8), f["q"])
    recip = np.clip(np.rint(x * (np.float32(1) / sc[:, None])), -127, 127)
    assert not np.array_equal(recip.astype(np.int8), f["q"])
    noclamp = np.abs(x).max(axis=1) / np.float32(127)
    assert not np.array_equal(noclamp.astype(np.float32).view(np.uint32), f["s"].view(np.uint32))
    g = torch.Generator().manual_seed(1)
    a = torch.randint(-127, 128, (64, 64), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (64, 64), generator=g, dtype=torch.int8)
    transposed = a.numpy().astype(np.int64) @ w.numpy().astype(np.int64)
    assert not np.array_equal(transposed, torch._int_mm(a, w.t()).numpy())


def test_pack_k64_layout_spot_checks(oracle):
    """The numpy packed-K64 restatement against the layout's definition (include/pyraquant_amd.h), element by element
    on random positions, computed independently: byte (r, k) of X lives at block (r // 16, k // 64), row r % 16, slot
    ((k // 16) % 4) ^ swz(r % 16), byte k % 16; swz taken from its bit formula. Plus the round trip through
    unpack_k64, zero padding rows, and a swizzle check that a plain (unswizzled) layout would fail."""
    rng = np.random.default_rng(5)
    R, K = 37, 192
    x = rng.integers(-128, 128, size=(R, K), dtype=np.int8)
    p = oracle.pack_k64(x)
    KT = K // 64
    assert p.shape == (((R + 15) // 16) * 16 * K,)

    def swz(r):
        b2, b1, b3 = (r >> 2) & 1, (r >> 1) & 1, (r >> 3) & 1
        return b2 | ((b1 ^ b3) << 1)

    assert [swz(r) for r in range(16)] == [int(v) for v in oracle.k64_swz(np.arange(16))]
    for _ in range(2000):
        r, k = int(rng.integers(R)), int(rng.integers(K))
        off = ((r // 16) * KT + k // 64) * 1024 + (r % 16) * 64 + ((((k // 16) % 4) ^ swz(r % 16)) << 4) + k % 16
        assert p[off] == x[r, k], (r, k)
    assert np.array_equal(oracle.unpack_k64(p, R, K), x)
    pad = p.reshape(-1, KT, 16, 64)[-1, :, R % 16:]          # rows 37..47 of the last block
    assert not pad.any()
    # the swizzle is not the identity on every row: an unswizzled copy differs
    plain = np.zeros_like(p).reshape(-1, KT, 16, 64)
    xp = np.zeros((((R + 15) // 16) * 16, K), np.int8)
    xp[:R] = x
    plain[:] = xp.reshape(-1, 16, KT, 64).transpose(0, 2, 1, 3)
    assert not np.array_equal(plain.reshape(-1), p)
