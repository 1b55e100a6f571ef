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
