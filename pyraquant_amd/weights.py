"""Weight-side conversion of an SVDQuant package for the INT8 executor (deploy/run_flux_latency.py:203-320).

The reference loads the package (dequantized W4 weights, smoothing / shift vectors, rank-32 low-rank factors) into
the transformer as one effective 16-bit weight per Linear; Int8Linear then derives the INT8 codes from it. This
module keeps that API:

* ``SplitInLinear``: a Linear split along its input (y = L0(x[..., :in0]) + L1(x[..., in0:]),
  pyraquant/external_quant.py:174-192), so each half carries its own smoothing and low rank. Once converted, each
  half is an Int8Linear that reads its slice of x as a row-strided view (no copy).
* ``fold_one``: the smoothing / shift fold of one Linear (deploy/run_flux_latency.py:210-253), the weight pass on
  the GPU (pq_fold_weight), the low-rank branch attached for Int8Linear or folded into the weight.
* ``load_method_weights``: the package loader (deploy/run_flux_latency.py:256-315) built on them.
"""
from __future__ import annotations

import json
import os
from typing import Dict, Optional

import torch
import torch.nn as nn

from . import _lib
from .int8_exec import LOWRANK_A_ATTR, LOWRANK_B_ATTR

LOWRANK_ATTRS = (LOWRANK_A_ATTR, LOWRANK_B_ATTR)


class SplitInLinear(nn.Module):
    """A Linear (in = in0 + in1) split along the input dim: y = L0(x[..., :in0]) + L1(x[..., in0:])
    (pyraquant/external_quant.py:174-192). L1 carries the bias."""

    def __init__(self, lin: nn.Linear, in0: int):
        super().__init__()
        W = lin.weight.data
        b = lin.bias
        l0 = nn.Linear(in0, W.shape[0], bias=False, device=W.device, dtype=W.dtype)
        l1 = nn.Linear(W.shape[1] - in0, W.shape[0], bias=b is not None, device=W.device, dtype=W.dtype)
        l0.weight.data.copy_(W[:, :in0])
        l1.weight.data.copy_(W[:, in0:])
        if b is not None:
            l1.bias.data.copy_(b.data)
        self.linears = nn.ModuleList([l0, l1])
        self.in0 = int(in0)
        self.in_features, self.out_features = W.shape[1], W.shape[0]

    def forward(self, x):
        return self.linears[0](x[..., : self.in0]) + self.linears[1](x[..., self.in0:])


def _vector(v, aux: Dict[str, torch.Tensor], dev) -> torch.Tensor:
    t = aux[v] if isinstance(v, str) else torch.as_tensor(v, dtype=torch.float32)
    return t.float().to(dev).contiguous()


def fold_weight(W: torch.Tensor, smooth: Optional[torch.Tensor] = None, shift: Optional[torch.Tensor] = None,
                bias: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
    """pq_fold_weight: W [N, K] 16-bit CUDA -> (W / smooth rounded to W's type, bias + (W / smooth) @ shift rounded,
    or the bias unchanged without a shift). out=W folds in place. smooth / shift: fp32 scalar or [K]."""
    assert W.is_cuda and W.dim() == 2 and W.stride(1) == 1, "W must be a row-major CUDA matrix"
    N, K = W.shape
    dev = W.device
    sm = None if smooth is None else smooth.float().to(dev).reshape(-1).contiguous()
    sh = None if shift is None else shift.float().to(dev).reshape(-1).contiguous()
    if sm is not None and sm.numel() not in (1, K):
        raise ValueError(f"smooth length {sm.numel()} is neither 1 nor in_features {K}")
    if sh is not None and sh.numel() not in (1, K):
        raise ValueError(f"shift length {sh.numel()} is neither 1 nor in_features {K}")
    if out is None:
        out = torch.empty_like(W)
    b_in = None
    b_out = None
    if sh is not None:
        if bias is not None:
            b_in = bias.to(W.dtype).contiguous()
        b_out = torch.empty(N, dtype=W.dtype, device=dev)
    _lib.check(_lib.load().pq_fold_weight(_lib.ptr(W), _lib.dtype_code(W.dtype), N, K, W.stride(0), _lib.ptr(sm),
                                          0 if sm is None else sm.numel(), _lib.ptr(sh),
                                          0 if sh is None else sh.numel(), _lib.ptr(b_in), _lib.ptr(out), out.stride(0),
                                          _lib.ptr(b_out), _lib.stream_of(dev)), "fold_weight")
    return out, (b_out if b_out is not None else bias)


def fold_one(lin: nn.Linear, sp: dict, aux: Dict[str, torch.Tensor], fold_lowrank: bool = False) -> None:
    """Fold this layer's smoothing / shift into lin.weight and lin.bias in place (deploy/run_flux_latency.py:210-253):
    W_eff = W / smooth, b_eff = b + W_eff @ shift, on the GPU. The low-rank branch (sp['lowrank_A'] [in, r],
    sp['lowrank_B'] [r, out]) is attached under the reference's attribute names for Int8Linear to run live, or with
    fold_lowrank=True added into the weight (the 16-bit path)."""
    W = lin.weight.data
    dt, dev = W.dtype, W.device
    if not W.is_cuda:
        raise AssertionError("fold_one runs on the GPU; move the model to the device first")
    smooth = sp.get("smooth")
    shift = sp.get("shift")
    sm = _vector(smooth, aux, dev) if smooth is not None else None
    sh = _vector(shift, aux, dev) if shift is not None else None
    if sm is not None or sh is not None:
        if dt in (torch.bfloat16, torch.float16):
            _, b = fold_weight(W, sm, sh, None if lin.bias is None else lin.bias.data, out=W)
        else:   # fp32 weights: the reference's own arithmetic, no 16-bit rounding to reproduce
            Wf = W.float() / sm.reshape(1, -1) if sm is not None else W.float()
            b = None
            if sh is not None:
                add = Wf.sum(dim=1) * sh.reshape(()) if sh.numel() == 1 else Wf @ sh.reshape(-1)
                b = add if lin.bias is None else lin.bias.data + add.to(lin.bias.dtype)
            W.copy_(Wf.to(dt))
        if sh is not None:
            if lin.bias is None:
                lin.bias = nn.Parameter(b.to(dt))
            else:
                lin.bias.data.copy_(b.to(lin.bias.dtype))
    a_key, b_key = sp.get("lowrank_A"), sp.get("lowrank_B")
    if a_key is not None and b_key is not None:
        A = aux[a_key].to(dev)
        B = aux[b_key].to(dev)
        if A.shape[0] != lin.weight.shape[1] or B.shape[1] != lin.weight.shape[0]:
            raise ValueError(f"low-rank shapes A{tuple(A.shape)} B{tuple(B.shape)} do not match W{tuple(lin.weight.shape)}")
        if fold_lowrank:
            lin.weight.data.copy_((lin.weight.data.float() + (A.float() @ B.float()).t()).to(dt))
        else:
            setattr(lin, LOWRANK_ATTRS[0], A.to(dt))
            setattr(lin, LOWRANK_ATTRS[1], B.to(dt))


def load_method_weights(model: nn.Module, pkg_dir: str, verbose: bool = True, fold_lowrank: bool = False) -> dict:
    """Put an SVDQuant package (meta.json, weights.safetensors, aux.safetensors, act_spec.json) into the model as one
    effective 16-bit weight per Linear with smoothing / shift folded (deploy/run_flux_latency.py:256-315); the
    caller then converts the Linears to Int8Linear, which derives the INT8 codes from these weights."""
    from safetensors.torch import load_file

    meta = json.load(open(os.path.join(pkg_dir, "meta.json")))
    if meta.get("impl"):
        raise SystemExit(f"package uses a custom implementation impl={meta['impl']}; this loader handles plain "
                         "SVDQuant packages only")
    w = load_file(os.path.join(pkg_dir, "weights.safetensors"))
    aux = load_file(os.path.join(pkg_dir, "aux.safetensors"))
    act = json.load(open(os.path.join(pkg_dir, "act_spec.json")))

    n_split = 0
    for name, in0 in (meta.get("split_modules") or {}).items():
        parent_name, _, child = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        lin = getattr(parent, child)
        if isinstance(lin, nn.Linear):
            setattr(parent, child, SplitInLinear(lin, int(in0)))
            n_split += 1

    mods = dict(model.named_modules())
    n_w, missing = 0, []
    for k, t in w.items():
        if k.endswith(".weight"):
            name, attr = k[:-7], "weight"
        elif k.endswith(".bias"):
            name, attr = k[:-5], "bias"
        else:
            name, attr = k, "weight"
        m = mods.get(name)
        if m is None or getattr(m, attr, None) is None:
            missing.append(k)
            continue
        p = getattr(m, attr)
        if tuple(p.shape) != tuple(t.shape):
            raise ValueError(f"{k}: model shape {tuple(p.shape)} vs package {tuple(t.shape)}")
        p.data.copy_(t.to(p.dtype))
        n_w += attr == "weight"

    n_fold, skipped = 0, []
    for name, sp in act.items():
        base = name.split("@")[0]
        if sp.get("impl") or sp.get("where") == "output":
            skipped.append(name)
            continue
        m = mods.get(base)
        if not isinstance(m, nn.Linear):
            skipped.append(name)
            continue
        fold_one(m, sp, aux, fold_lowrank=fold_lowrank)
        n_fold += 1
    n_lowrank = sum(1 for _, m in model.named_modules() if getattr(m, LOWRANK_ATTRS[0], None) is not None)
    rep = {"method": meta.get("method"), "w_bits": meta.get("w_bits"), "a_bits_simulated_away": meta.get("a_bits"),
           "n_lowrank_branches_live": n_lowrank, "group": meta.get("group"), "lowrank_rank": meta.get("lowrank_rank"),
           "n_weights_written": n_w, "n_layers_folded": n_fold, "n_split_modules": n_split,
           "n_missing_keys": len(missing), "n_specs_skipped": len(skipped),
           "note": "weights = package weights with smooth/shift folded into weight+bias on the GPU; the low-rank "
                   "branch is kept live for Int8Linear (not folded); the INT8 codes are derived from these weights"}
    if verbose:
        print(f"[weight-source] method weights: {meta.get('method')} W{meta.get('w_bits')} group {meta.get('group')} "
              f"low-rank r={meta.get('lowrank_rank')}; wrote {n_w} weights, folded {n_fold} layers ({n_lowrank} live "
              f"low-rank branches), split {n_split} layers, {len(missing)} missing keys, {len(skipped)} specs skipped",
              flush=True)
    return rep
