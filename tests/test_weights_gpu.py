"""GPU parity of the weight-side conversion (pq_fold_weight, pyraquant_amd.weights) against the CPU restatement of
the reference's `_fold_one` (oracle/torch_ref.py, deploy/run_flux_latency.py:219-239):
* folded weights bit-identical (the division and the 16-bit rounding are elementwise IEEE);
* the new bias within one 16-bit rounding step of the oracle's (the shift term is an fp32 sum whose order differs
  from torch's matmul), most elements identical;
* scalar and per-channel smooth / shift, no bias, in place, bf16 and fp16, a non-contiguous row stride;
* the package loader on a synthetic package (split module, low-rank factors, a spec for a missing module), and the
  INT8 codes Int8Linear derives from the folded weights equal the oracle's RTN of them.
"""
import json
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _bias_close(got, ref, dt, b_in=None):
    """Within two 16-bit rounding steps of the larger of the new bias and the added shift term (the reference rounds
    the shift term before adding it, so a last-place flip of that term, from the summation order, moves the result by
    an ulp of the term), and mostly identical."""
    ulp = 2.0 ** -8 if dt == torch.bfloat16 else 2.0 ** -11
    r = ref.double()
    add = r - (b_in.double() if b_in is not None else 0.0)
    scale = torch.maximum(r.abs(), add.abs()).clamp_min(1e-3)
    d = (got.double() - r).abs() / scale
    assert float(d.max()) <= 2 * ulp, float(d.max())
    assert float((got == ref).double().mean()) >= 0.9


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N,K,smooth,shift,bias", [(3072, 3072, "vec", "vec", True), (640, 1280, "scalar", "scalar", True),
                                                   (333, 15360, "vec", None, True), (128, 64, None, "vec", False),
                                                   (1000, 640, "vec", "scalar", False), (64, 3072, None, None, True)])
def test_fold_weight_matches_oracle(cuda, dt, N, K, smooth, shift, bias):
    from oracle import torch_ref as T
    from pyraquant_amd import weights

    g = torch.Generator().manual_seed(N + K)
    W = (torch.randn(N, K, generator=g) * 0.03).to(dt)
    b = (torch.randn(N, generator=g) * 0.01).to(dt) if bias else None
    sm = {"vec": torch.rand(K, generator=g) + 0.25, "scalar": torch.tensor(1.37), None: None}[smooth]
    sh = {"vec": torch.randn(K, generator=g) * 0.2, "scalar": torch.tensor(-0.11), None: None}[shift]
    w_ref, b_ref = T.fold_one(W, sm, sh, b)
    w_got, b_got = weights.fold_weight(W.to(cuda), sm, sh, None if b is None else b.to(cuda))
    assert torch.equal(w_got.cpu(), w_ref)
    if sh is None:
        assert (b_got is None) == (b is None)
        if b is not None:
            assert torch.equal(b_got.cpu(), b)
    else:
        _bias_close(b_got.cpu(), b_ref, dt, b)


def test_fold_weight_in_place_and_strided(cuda):
    """out=W folds in place; a column slice (row stride > K) is read through its stride."""
    from oracle import torch_ref as T
    from pyraquant_amd import weights

    g = torch.Generator().manual_seed(5)
    big = (torch.randn(256, 1280 + 64, generator=g) * 0.05).to(torch.bfloat16)
    sm = torch.rand(1280, generator=g) + 0.5
    sh = torch.randn(1280, generator=g)
    Wv = big[:, 64:]
    w_ref, b_ref = T.fold_one(Wv.contiguous(), sm, sh, None)
    Wd = big.to(cuda)[:, 64:]
    w_got, b_got = weights.fold_weight(Wd, sm, sh)
    assert torch.equal(w_got.cpu(), w_ref)
    _bias_close(b_got.cpu(), b_ref, torch.bfloat16)
    Wc = Wv.contiguous().to(cuda)
    weights.fold_weight(Wc, sm, sh, out=Wc)
    assert torch.equal(Wc.cpu(), w_ref)


def test_fold_one_and_lowrank(cuda):
    """fold_one on an nn.Linear with aux-key smoothing / shift: weight and bias folded in place, the low-rank branch
    attached under the reference's attribute names (or folded into the weight with fold_lowrank)."""
    from oracle import torch_ref as T
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd import weights

    g = torch.Generator().manual_seed(9)
    lin = torch.nn.Linear(640, 1280, dtype=torch.bfloat16).to(cuda)
    W0, b0 = lin.weight.data.cpu().clone(), lin.bias.data.cpu().clone()
    aux = {"s": torch.rand(640, generator=g) + 0.5, "h": torch.randn(640, generator=g) * 0.1,
           "A": torch.randn(640, 32, generator=g).to(torch.bfloat16) * 0.02,
           "B": torch.randn(32, 1280, generator=g).to(torch.bfloat16) * 0.02}
    sp = {"smooth": "s", "shift": "h", "lowrank_A": "A", "lowrank_B": "B"}
    weights.fold_one(lin, sp, aux)
    w_ref, b_ref = T.fold_one(W0, aux["s"], aux["h"], b0)
    assert torch.equal(lin.weight.data.cpu(), w_ref)
    _bias_close(lin.bias.data.cpu(), b_ref, torch.bfloat16, b0)
    assert torch.equal(getattr(lin, E.LOWRANK_A_ATTR).cpu(), aux["A"])
    lin2 = torch.nn.Linear(640, 1280, bias=False, dtype=torch.bfloat16).to(cuda)
    W2 = lin2.weight.data.cpu().clone()
    weights.fold_one(lin2, {"smooth": 2.0, "lowrank_A": "A", "lowrank_B": "B"}, aux, fold_lowrank=True)
    w2_ref, _ = T.fold_one(W2, torch.tensor(2.0), None, None)
    exp = (w2_ref.float() + (aux["A"].float() @ aux["B"].float()).t()).to(torch.bfloat16)
    assert torch.allclose(lin2.weight.data.cpu().float(), exp.float(), rtol=0, atol=2e-3)
    assert lin2.bias is None


class _Block(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.to_q = torch.nn.Linear(256, 256, dtype=torch.bfloat16)
        self.proj_out = torch.nn.Linear(512, 256, dtype=torch.bfloat16)


class _Model(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.blocks = torch.nn.ModuleList([_Block(), _Block()])


def test_load_method_weights_package(cuda, tmp_path):
    """A synthetic SVDQuant package through the loader: weights written, proj_out split into two halves with their
    own smoothing, folds equal to the oracle's, live low-rank branches, a spec for a missing module skipped; then
    convert_linears_to_int8 quantizes the folded weights (codes equal to the oracle's RTN)."""
    from safetensors.torch import save_file

    from oracle import oracle as O
    from oracle import torch_ref as T
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd import weights

    g = torch.Generator().manual_seed(11)
    wts, aux, act = {}, {}, {}
    for i in range(2):
        wts[f"blocks.{i}.to_q.weight"] = (torch.randn(256, 256, generator=g) * 0.05).to(torch.bfloat16)
        wts[f"blocks.{i}.to_q.bias"] = (torch.randn(256, generator=g) * 0.01).to(torch.bfloat16)
        aux[f"q{i}.s"] = torch.rand(256, generator=g) + 0.5
        aux[f"q{i}.h"] = torch.randn(256, generator=g) * 0.1
        aux[f"q{i}.A"] = (torch.randn(256, 32, generator=g) * 0.02).to(torch.bfloat16)
        aux[f"q{i}.B"] = (torch.randn(32, 256, generator=g) * 0.02).to(torch.bfloat16)
        act[f"blocks.{i}.to_q"] = {"smooth": f"q{i}.s", "shift": f"q{i}.h", "lowrank_A": f"q{i}.A",
                                   "lowrank_B": f"q{i}.B"}
        for h, k in ((0, 192), (1, 320)):
            wts[f"blocks.{i}.proj_out.linears.{h}.weight"] = (torch.randn(256, k, generator=g) * 0.05).to(torch.bfloat16)
            aux[f"p{i}{h}.s"] = torch.rand(k, generator=g) + 0.5
            act[f"blocks.{i}.proj_out.linears.{h}"] = {"smooth": f"p{i}{h}.s"}
        wts[f"blocks.{i}.proj_out.linears.1.bias"] = (torch.randn(256, generator=g) * 0.01).to(torch.bfloat16)
    act["blocks.9.to_k"] = {"smooth": "q0.s"}
    act["blocks.0.to_q@out"] = {"where": "output"}
    meta = {"method": "svdquant", "w_bits": 4, "a_bits": 4, "group": 64, "lowrank_rank": 32,
            "split_modules": {"blocks.0.proj_out": 192, "blocks.1.proj_out": 192}}
    save_file(wts, str(tmp_path / "weights.safetensors"))
    save_file(aux, str(tmp_path / "aux.safetensors"))
    json.dump(meta, open(tmp_path / "meta.json", "w"))
    json.dump(act, open(tmp_path / "act_spec.json", "w"))

    model = _Model().to(cuda)
    rep = weights.load_method_weights(model, str(tmp_path), verbose=False)
    assert rep["n_split_modules"] == 2 and rep["n_layers_folded"] == 6 and rep["n_specs_skipped"] == 2
    assert rep["n_lowrank_branches_live"] == 2 and rep["n_missing_keys"] == 0
    assert isinstance(model.blocks[0].proj_out, weights.SplitInLinear)
    w_ref, b_ref = T.fold_one(wts["blocks.1.to_q.weight"], aux["q1.s"], aux["q1.h"], wts["blocks.1.to_q.bias"])
    assert torch.equal(model.blocks[1].to_q.weight.data.cpu(), w_ref)
    _bias_close(model.blocks[1].to_q.bias.data.cpu(), b_ref, torch.bfloat16, wts["blocks.1.to_q.bias"])
    wh_ref, _ = T.fold_one(wts["blocks.0.proj_out.linears.1.weight"], aux["p01.s"], None, None)
    assert torch.equal(model.blocks[0].proj_out.linears[1].weight.data.cpu(), wh_ref)

    x = (torch.randn(64, 512, generator=g)).to(torch.bfloat16).to(cuda)
    with torch.no_grad():
        y16 = model.blocks[0].proj_out(x)
    E.convert_linears_to_int8(model, device=cuda, whitelist=lambda n: False)
    assert isinstance(model.blocks[0].proj_out.linears[0], E.Int8Linear)
    q = model.blocks[1].to_q
    qo, so = O.quant_weight(w_ref.float().numpy(), 0)
    assert np.array_equal(q.weight_int8.cpu().numpy(), qo)
    assert q.lr_A is not None
    with torch.no_grad():
        y8 = model.blocks[0].proj_out(x)      # both halves read row-strided views of x
    rel = float((y8.float() - y16.float()).norm() / y16.float().norm())
    assert rel < 2e-2, rel


@pytest.mark.parametrize("M,lowrank", [(300, 0), (300, 32), (2100, 32), (4352, 32), (65792, 32)])
def test_split_linear_accumulates_in_epilogue(oracle, cuda, M, lowrank):
    """The FLUX single-block proj_out split along its input (K = 3072 + 12288 -> N = 3072), both halves Int8Linear:
    the second half adds its result into the first half's output inside its GEMM epilogue (PQ_ACCUMULATE). That is
    bit-identical to torch's y0 + y1 of the two halves' outputs; without a low-rank branch it is bit-identical to the
    oracle's two layers summed with one 16-bit rounding (round(round(y0) + round(y1))), and with one it is within
    the tolerance of the oracle's fp32 sum, on 104 sampled rows (the last 40 included) at every M: 300 runs 128 x 64
    blocks, 2100 128 x 128 blocks, 4352 (FLUX 1K) one round of 256 x 256 blocks and 65792 (FLUX 4K, 4096^2 image +
    256 text tokens) persistent 256 x 256 blocks."""
    from conftest import MAX_REL, MEAN_REL, bits, elem_violation, rel_errors
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd import weights
    from pyraquant_amd.workloads import make_linear, make_x

    K0, K1, N = 3072, 12288, 3072
    lin = make_linear(K0 + K1, N, 0, True, seed=21).to(torch.bfloat16)
    split = weights.SplitInLinear(lin.to(cuda), K0)
    heads = [make_linear(k, N, lowrank, False, seed=30 + h) for h, k in enumerate((K0, K1))]
    for h, half in enumerate(split.linears):
        if lowrank:
            setattr(half, E.LOWRANK_A_ATTR, getattr(heads[h], E.LOWRANK_A_ATTR).to(cuda))
            setattr(half, E.LOWRANK_B_ATTR, getattr(heads[h], E.LOWRANK_B_ATTR).to(cuda))
        split.linears[h] = E.Int8Linear(half, device=cuda)
    x = make_x(M, K0 + K1, seed=M, device=cuda)
    y = split(x)
    q0, q1 = split.linears
    y_sum = q0(x[:, :K0]) + q1(x[:, K0:])
    assert torch.equal(y, y_sum), "the epilogue's accumulate must round as torch's 16-bit add"

    g = torch.Generator().manual_seed(M)
    rows = torch.cat([torch.randperm(M - 40, generator=g)[:64], torch.arange(M - 40, M)]).sort().values.to(cuda)
    xs = x[rows]
    outs = []
    for q, sl in ((q0, slice(0, K0)), (q1, slice(K0, K0 + K1))):
        outs.append(oracle.linear(bits(xs[:, sl].contiguous()), 0, q.weight_int8.cpu().numpy(), q.w_scale.cpu().numpy(),
                                  None if q.bias is None else q.bias.cpu().numpy(), 0,
                                  bits(q.lr_A) if lowrank else None, bits(q.lr_B) if lowrank else None))
    got = bits(y[rows])
    if not lowrank:
        both = oracle.to_f32(outs[0]["out"], 0) + oracle.to_f32(outs[1]["out"], 0)
        assert np.array_equal(got, oracle.from_f32(both, 0))
        return
    ref = outs[0]["y"].astype(np.float64) + outs[1]["y"]
    yf = oracle.to_f32(got, 0)
    mx, mean = rel_errors(yf, ref)
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
    t = np.concatenate([oracle.to_f32(o["t"], 0) for o in outs], axis=1)
    l2 = np.concatenate([oracle.to_f32(bits(q.lr_B), 0) for q in (q0, q1)], axis=0)
    # the sum carries the 16-bit rounding of each half's output (2^-9 of each, bf16) on top of one layer's bar
    halves = 2.0 ** -9 * (np.abs(outs[0]["y"].astype(np.float64)) + np.abs(outs[1]["y"]))
    assert elem_violation(yf, ref, t, l2, extra=halves) <= 1.0


def test_accumulate_scatter_and_group32(cuda):
    """PQ_ACCUMULATE with a routed scatter (canvas[rows] += y, other rows untouched), and Int8Linear's accumulate for
    group-32 weights (the GEMM's output added by torch): both equal canvas + y computed by torch."""
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    for group, dt in ((0, torch.bfloat16), (32, torch.float16)):
        q = E.Int8Linear(make_linear(1280, 640, 0 if group else 32, True, seed=5, dtype=dt), device=cuda,
                         group_size=group)
        x = make_x(500, 1280, dt, seed=6, device=cuda)
        g = torch.Generator().manual_seed(7)
        ri = torch.randperm(500, generator=g)[:123].to(torch.int32).to(cuda)
        ori = torch.randperm(900, generator=g)[:123].to(torch.int32).to(cuda)
        canvas = make_x(900, 640, dt, seed=8, outlier_frac=0.0, device=cuda)
        expect = canvas.clone()
        y = q(x, row_idx=ri)
        expect[ori.long()] = expect[ori.long()] + y
        q(x, row_idx=ri, out=canvas, out_row_idx=ori, accumulate=True)
        assert torch.equal(canvas, expect), group
