"""Seeded random sweep of Int8Linear through the public API against the CPU oracle.

Each case draws a 16-bit dtype, K, N, M, per-channel or group-32 weights, a low-rank branch (none, or rank 8 to
128: zero-padded in the epilogue up to 64, after the GEMM above), a bias, a padded row stride of x, and optionally
a routed call (gather of M rows of a larger x and a scatter into a larger canvas). For each case:
  * weight codes / scales and activation codes / scales are bit-exact against the oracle
    (pyraquant/quantizers_weight.py:96-109, deploy/int8_exec.py:352-357, :508-509);
  * the layer output is within the build's tolerance of the oracle's fp32 result computed from the same codes
    (deploy/int8_exec.py:382-393; order of the epilogue :303-309), and bit-exact when there is no low-rank term;
  * the direct call path gives the same bits as the general wrappers;
  * rows of a scatter canvas that the call does not name keep their contents.
"""
import numpy as np
import pytest
import torch

from conftest import MAX_REL, MEAN_REL, bits, dcode, rel_errors

pytestmark = pytest.mark.gpu

_KS = (64, 192, 320, 640, 1024, 1280, 1536, 2048, 2560, 3072, 4096, 12288)
N_CASES = 96


def _case(i):
    rng = np.random.default_rng(7000 + i)
    K = int(rng.choice(_KS))
    M = int(rng.integers(1, 600)) if rng.random() < 0.9 else int(rng.integers(600, 2500))
    if K == 12288:
        M = min(M, 300)   # keeps the oracle's CPU GEMM to about a second
    return dict(dtype=(torch.bfloat16, torch.float16)[int(rng.integers(2))], K=K, N=64 * int(rng.integers(1, 17)),
                M=M, group=32 if rng.random() < 0.3 else 0, R=int(rng.choice((0, 0, 8, 16, 32, 32, 48, 64, 96, 128))),
                bias=bool(rng.random() < 0.7), pad=int(rng.choice((0, 0, 8, 136))), routed=bool(rng.random() < 0.35))


def test_sweep_draws_every_option():
    """The seeded cases reach every option the sweep is meant to cover."""
    cases = [_case(i) for i in range(N_CASES)]
    for key, want in (("dtype", {torch.bfloat16, torch.float16}), ("group", {0, 32}), ("routed", {False, True}),
                      ("bias", {False, True})):
        assert {c[key] for c in cases} == want, key
    assert {0, 8, 16, 32, 48, 64, 96, 128} <= {c["R"] for c in cases}
    assert 12288 in {c["K"] for c in cases} and max(c["M"] for c in cases) > 600
    assert {c["pad"] for c in cases} >= {0, 8, 136}
    assert any(c["R"] == 32 and c["K"] in (1024, 1280, 2048, 2560, 3072) for c in cases)   # the fused quantizer


@pytest.mark.parametrize("i", range(N_CASES))
def test_int8linear_random_sweep(oracle, cuda, i):
    from pyraquant_amd import int8_exec as E

    c = _case(i)
    K, N, M, dt, R = c["K"], c["N"], c["M"], c["dtype"], c["R"]
    print(f"[sweep] case {i}: {c}", flush=True)
    g = torch.Generator().manual_seed(100 + i)
    lin = torch.nn.Linear(K, N, bias=c["bias"])
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.02)
        if c["bias"]:
            lin.bias.copy_(torch.randn(N, generator=g) * 0.01)
    lr = None
    if R:
        lr = ((torch.randn(K, R, generator=g) * 0.02).to(dt), (torch.randn(R, N, generator=g) * 0.02).to(dt))
    q = E.Int8Linear(lin, device=cuda, lowrank=lr, group_size=c["group"])

    qo, so = oracle.quant_weight(lin.weight.detach().numpy(), c["group"])
    assert np.array_equal(q.weight_int8.cpu().numpy(), qo)
    assert np.array_equal(q.w_scale.cpu().numpy().view(np.uint32), so.view(np.uint32))

    rows = M + 50 if c["routed"] else M
    xf = torch.randn(rows, K + c["pad"], generator=g)
    xf[:, torch.randperm(K, generator=g)[: max(1, K // 200)]] *= 20.0   # outlier channels, as the workloads have
    x = xf.to(dt).to(cuda)[:, :K]                                      # row stride K + pad
    ri = ori = canvas = before = None
    if c["routed"]:
        ri = torch.randperm(rows, generator=g)[:M].to(torch.int32)
        ori = torch.randperm(M + 30, generator=g)[:M].to(torch.int32)
        canvas = torch.randn(M + 30, N, generator=g).to(dt).to(cuda)
        before = canvas.clone()
        q(x, row_idx=ri.to(cuda), out=canvas, out_row_idx=ori.to(cuda))
        y = canvas[ori.long().to(cuda)]
    else:
        y = q(x)
    assert y.dtype == dt and y.shape == (M, N)

    o = oracle.linear(bits(x.contiguous()), dcode(dt), qo, so, None if q.bias is None else q.bias.cpu().numpy(),
                      c["group"], None if lr is None else bits(lr[0]), None if lr is None else bits(lr[1]),
                      None if ri is None else ri.numpy())
    ri_d = None if ri is None else ri.to(cuda)
    xq, sx = E.quant_rows(x, ri_d)
    assert np.array_equal(xq.cpu().numpy(), o["q"])
    assert np.array_equal(sx.cpu().numpy().view(np.uint32), o["s"].view(np.uint32))
    xqp, sxp = E.quant_rows_packed(x, ri_d)
    assert np.array_equal(xqp.cpu().numpy(), oracle.pack_k64(o["q"]))
    assert torch.equal(sxp, sx)

    mx, mean = rel_errors(oracle.to_f32(bits(y), dcode(dt)), o["y"])
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
    if not R:   # no low-rank sum: the epilogue runs the oracle's fp32 operations in its order, so the bits agree
        assert np.array_equal(bits(y), o["out"])

    if c["routed"]:
        keep = torch.ones(M + 30, dtype=torch.bool)
        keep[ori.long()] = False
        assert torch.equal(canvas[keep.to(cuda)], before[keep.to(cuda)])
    else:
        E.DIRECT_CALLS = False
        try:
            y2 = q(x)
        finally:
            E.DIRECT_CALLS = True
        assert torch.equal(y, y2)


# Large shapes: the 128 x 128 sweep above never reaches the 256 x 256 blocks (one round, or persistent over several),
# so a second seeded family draws M and N large enough for them, with the same options, and checks sampled rows (the
# last 40 included: the ragged tiles) against the oracle.
N_BIG = 16


def _big_case(i):
    rng = np.random.default_rng(9000 + i)
    lo = i % 2 == 0   # even cases about one round of 256 x 256 blocks, odd ones several
    return dict(dtype=(torch.bfloat16, torch.float16)[int(rng.integers(2))],
                K=int(rng.choice((256, 512, 1024, 1280, 3072))),
                N=64 * int(rng.integers(24, 65) if lo else rng.integers(48, 129)),
                M=int(rng.integers(2048, 5001) if lo else rng.integers(6000, 16385)),
                group=32 if rng.random() < 0.25 else 0,
                R=int(rng.choice((0, 16, 32, 32, 64))), bias=bool(rng.random() < 0.7), pad=int(rng.choice((0, 8))),
                routed=bool(rng.random() < 0.35))


def test_big_sweep_reaches_the_large_tiles():
    """The large cases take each of the GEMM's block choices on a 256-CU part (the library's rule): persistent
    256 x 256 blocks (at least 1024 blocks of 256 x 128, more 256 x 256 blocks than CUs), one round of 256 x 256
    blocks (at most one per CU, where 128 x 128 blocks would exceed two per CU), 128 x 128 blocks, and group-32."""
    kinds = []
    for i in range(N_BIG):
        c = _big_case(i)
        M, N = c["M"], c["N"]
        b128, b256, b256x128 = -(-M // 128) * -(-N // 128), -(-M // 256) * -(-N // 256), -(-M // 128) * -(-N // 256)
        if c["group"]:
            kinds.append("group-32")
        elif b256x128 >= 1024:
            kinds.append("persistent" if b256 > 256 else "256")
        elif b256 <= 256 and b128 > 512:
            kinds.append("one round")
        else:
            kinds.append("128")
    for k in ("persistent", "one round", "128", "group-32"):
        assert kinds.count(k) >= (3 if k in ("persistent", "one round") else 1), kinds


@pytest.mark.parametrize("i", range(N_BIG))
def test_int8linear_random_sweep_large(oracle, cuda, i):
    from conftest import elem_violation
    from pyraquant_amd import int8_exec as E

    c = _big_case(i)
    K, N, M, dt, R = c["K"], c["N"], c["M"], c["dtype"], c["R"]
    print(f"[sweep-large] case {i}: {c}", flush=True)
    g = torch.Generator().manual_seed(300 + i)
    lin = torch.nn.Linear(K, N, bias=c["bias"])
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.02)
        if c["bias"]:
            lin.bias.copy_(torch.randn(N, generator=g) * 0.01)
    lr = None
    if R:
        lr = ((torch.randn(K, R, generator=g) * 0.02).to(dt), (torch.randn(R, N, generator=g) * 0.02).to(dt))
    q = E.Int8Linear(lin, device=cuda, lowrank=lr, group_size=c["group"])
    qo, so = oracle.quant_weight(lin.weight.detach().numpy(), c["group"])
    assert np.array_equal(q.weight_int8.cpu().numpy(), qo)
    assert np.array_equal(q.w_scale.cpu().numpy().view(np.uint32), so.view(np.uint32))

    rows = M + 50 if c["routed"] else M
    xf = torch.randn(rows, K + c["pad"], generator=g)
    xf[:, torch.randperm(K, generator=g)[: max(1, K // 200)]] *= 20.0
    x = xf.to(dt).to(cuda)[:, :K]
    sample = torch.cat([torch.randperm(M - 40, generator=g)[:64], torch.arange(M - 40, M)]).sort().values
    if c["routed"]:
        ri = torch.randperm(rows, generator=g)[:M].to(torch.int32)
        ori = torch.randperm(M + 30, generator=g)[:M].to(torch.int32)
        canvas = torch.randn(M + 30, N, generator=g).to(dt).to(cuda)
        before = canvas.clone()
        q(x, row_idx=ri.to(cuda), out=canvas, out_row_idx=ori.to(cuda))
        src, dst = ri[sample].long(), ori[sample].long()
        y_rows = canvas[dst.to(cuda)]
    else:
        y = q(x)
        assert y.dtype == dt and y.shape == (M, N)
        src = sample
        y_rows = y[sample.to(cuda)]
    o = oracle.linear(bits(x[src.to(cuda)].contiguous()), dcode(dt), qo, so,
                      None if q.bias is None else q.bias.cpu().numpy(), c["group"],
                      None if lr is None else bits(lr[0]), None if lr is None else bits(lr[1]))
    got = bits(y_rows)
    if not R:
        assert np.array_equal(got, o["out"]), "outputs without a low-rank branch must be bit-exact"
    else:
        yf = oracle.to_f32(got, dcode(dt))
        mx, mean = rel_errors(yf, o["y"])
        assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
        v = elem_violation(yf, o["y"], oracle.to_f32(o["t"], dcode(dt)), oracle.to_f32(bits(lr[1]), dcode(dt)))
        assert v <= 1.0, v
    if c["routed"]:
        keep = torch.ones(M + 30, dtype=torch.bool)
        keep[ori.long()] = False
        assert torch.equal(canvas[keep.to(cuda)], before[keep.to(cuda)])
