"""Weight-side conversion of an SVDQuant package for the INT8 executor.

What is kept from the reference, because it is the interface a PyraQuant driver and its packages rely on
(deploy/run_flux_latency.py:203-320, pyraquant/external_quant.py:174-192):
* the package directory: meta.json (``method``, ``w_bits``, ``a_bits``, ``group``, ``lowrank_rank``, ``impl``,
  ``split_modules``), weights.safetensors (``<module>.weight`` / ``<module>.bias``), aux.safetensors and act_spec.json
  (``<module>[@tag]`` -> ``smooth`` / ``shift`` / ``lowrank_A`` / ``lowrank_B`` / ``impl`` / ``where``);
* the report's keys, the low-rank attribute names, the split module's ``linears.0`` / ``linears.1`` children (the
  package's tensor keys address them) and the exception types (SystemExit for a custom-implementation package,
  ValueError for shapes);
* the fold's arithmetic: W_eff = W / smooth rounded to W's type, b_eff = b + round(W_eff @ shift), so the weights the
  INT8 codes are derived from match the reference's bit for bit.

Everything else is this build's: the fold runs on the GPU (pq_fold_weight), and a converted ``SplitInLinear`` sums
its halves inside the second half's GEMM epilogue (PQ_ACCUMULATE) instead of with a separate add.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn as nn

from . import _lib
from .int8_exec import LOWRANK_A_ATTR, LOWRANK_B_ATTR, Int8Linear

LOWRANK_ATTRS = (LOWRANK_A_ATTR, LOWRANK_B_ATTR)


# --------------------------------------------------------------------------- the split-input Linear
class SplitInLinear(nn.Module):
    """A Linear whose input is cut in two at ``in0``: y = L0(x[..., :in0]) + L1(x[..., in0:]), L1 holding the bias
    (the FLUX single-block proj_out, whose attention and MLP halves carry their own smoothing and low rank;
    pyraquant/external_quant.py:174-192). Each half reads its slice of x as a strided view (no copy).

    When both halves are Int8Linear (after convert_linears_to_int8), the first half writes the output and the second
    adds its own result into it in the GEMM's epilogue: one pass over the output, and the same 16-bit roundings as
    the reference's ``L0(x0) + L1(x1)``."""

    def __init__(self, lin: nn.Linear, in0: int):
        super().__init__()
        k_total, n_out = lin.in_features, lin.out_features
        if not 0 < in0 < k_total:
            raise ValueError(f"SplitInLinear: cut at {in0} is outside (0, {k_total})")
        w = lin.weight.detach()
        spans = ((0, int(in0)), (int(in0), k_total))
        parts = []
        for half, (lo, hi) in enumerate(spans):
            with_bias = half == 1 and lin.bias is not None
            part = nn.Linear(hi - lo, n_out, bias=with_bias, device=w.device, dtype=w.dtype)
            with torch.no_grad():
                part.weight.copy_(w[:, lo:hi])
                if with_bias:
                    part.bias.copy_(lin.bias.detach())
            parts.append(part)
        self.linears = nn.ModuleList(parts)
        self.in0 = int(in0)
        self.in_features, self.out_features = k_total, n_out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        head, tail = x[..., : self.in0], x[..., self.in0:]
        first, second = self.linears
        if isinstance(first, Int8Linear) and isinstance(second, Int8Linear):
            y = first(head)
            second(tail.reshape(-1, tail.shape[-1]), out=y.view(-1, self.out_features), accumulate=True)
            return y
        return first(head) + second(tail)


# --------------------------------------------------------------------------- the fold (GPU)
def fold_weight(W: torch.Tensor, smooth: Optional[torch.Tensor] = None, shift: Optional[torch.Tensor] = None,
                bias: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
    """pq_fold_weight: W [N, K] 16-bit CUDA -> (W / smooth rounded to W's type, bias + (W / smooth) @ shift rounded,
    or the bias unchanged without a shift). out=W folds in place. smooth / shift: fp32 scalar or [K]."""
    assert W.is_cuda and W.dim() == 2 and W.stride(1) == 1, "W must be a row-major CUDA matrix"
    N, K = W.shape
    dev = W.device
    sm = None if smooth is None else smooth.float().to(dev).reshape(-1).contiguous()
    sh = None if shift is None else shift.float().to(dev).reshape(-1).contiguous()
    for what, v in (("smooth", sm), ("shift", sh)):
        if v is not None and v.numel() not in (1, K):
            raise ValueError(f"{what} has {v.numel()} entries; a Linear with {K} inputs takes 1 or {K}")
    if out is None:
        out = torch.empty_like(W)
    b_in = b_out = None
    if sh is not None:
        b_in = None if bias is None else bias.to(W.dtype).contiguous()
        b_out = torch.empty(N, dtype=W.dtype, device=dev)
    _lib.check(_lib.load().pq_fold_weight(_lib.ptr(W), _lib.dtype_code(W.dtype), N, K, W.stride(0), _lib.ptr(sm),
                                          0 if sm is None else sm.numel(), _lib.ptr(sh),
                                          0 if sh is None else sh.numel(), _lib.ptr(b_in), _lib.ptr(out), out.stride(0),
                                          _lib.ptr(b_out), _lib.stream_of(dev)), "fold_weight")
    return out, (b_out if b_out is not None else bias)


def _aux_value(ref, aux: Dict[str, torch.Tensor], device) -> Optional[torch.Tensor]:
    """A spec entry is either the name of an aux tensor or an inline number."""
    if ref is None:
        return None
    value = aux[ref] if isinstance(ref, str) else torch.tensor(ref, dtype=torch.float32)
    return value.to(device=device, dtype=torch.float32).contiguous()


def _fold_into_linear(lin: nn.Linear, smooth: Optional[torch.Tensor], shift: Optional[torch.Tensor]) -> None:
    """W <- W / smooth and b <- b + (W / smooth) @ shift on lin, in place."""
    W = lin.weight.data
    old_bias = None if lin.bias is None else lin.bias.data
    if W.dtype in (torch.bfloat16, torch.float16):
        _, new_bias = fold_weight(W, smooth, shift, old_bias, out=W)
    else:
        # 32-bit weights have no 16-bit rounding to reproduce: the same algebra in torch
        scaled = W.float() if smooth is None else W.float() / smooth.reshape(1, -1)
        new_bias = old_bias
        if shift is not None:
            term = scaled.sum(dim=1) * shift.reshape(()) if shift.numel() == 1 else scaled @ shift.reshape(-1)
            new_bias = term if old_bias is None else old_bias + term.to(old_bias.dtype)
        W.copy_(scaled.to(W.dtype))
    if shift is None:
        return
    if lin.bias is None:
        lin.bias = nn.Parameter(new_bias.to(W.dtype))
    else:
        lin.bias.data.copy_(new_bias.to(lin.bias.dtype))


def _place_lowrank(lin: nn.Linear, A: torch.Tensor, B: torch.Tensor, into_weight: bool) -> None:
    """The rank-r branch A [in, r] / B [r, out]: parked on the Linear for Int8Linear to run beside the INT8 GEMM, or
    (the 16-bit path, which has no executor for it) added into the weight."""
    if tuple(A.shape[:1]) != (lin.in_features,) or B.shape[-1] != lin.out_features or A.shape[1] != B.shape[0]:
        raise ValueError(f"low-rank factors {tuple(A.shape)} x {tuple(B.shape)} do not fit a "
                         f"{lin.in_features} -> {lin.out_features} Linear")
    dt = lin.weight.dtype
    if into_weight:
        delta = (A.float() @ B.float()).t()
        lin.weight.data.copy_((lin.weight.data.float() + delta).to(dt))
        return
    setattr(lin, LOWRANK_A_ATTR, A.to(dt))
    setattr(lin, LOWRANK_B_ATTR, B.to(dt))


def fold_one(lin: nn.Linear, sp: dict, aux: Dict[str, torch.Tensor], fold_lowrank: bool = False) -> None:
    """Apply one act_spec entry to its Linear (deploy/run_flux_latency.py:210-253): smoothing and shift folded into
    the weight and bias on the GPU, the low-rank branch attached under LOWRANK_A_ATTR / LOWRANK_B_ATTR (or, with
    fold_lowrank, added into the weight)."""
    dev = lin.weight.device
    if not lin.weight.is_cuda:
        raise AssertionError("fold_one runs on the GPU; move the model to the device first")
    smooth, shift = _aux_value(sp.get("smooth"), aux, dev), _aux_value(sp.get("shift"), aux, dev)
    if smooth is not None or shift is not None:
        _fold_into_linear(lin, smooth, shift)
    a_name, b_name = sp.get("lowrank_A"), sp.get("lowrank_B")
    if a_name is not None and b_name is not None:
        _place_lowrank(lin, aux[a_name].to(dev), aux[b_name].to(dev), fold_lowrank)


# --------------------------------------------------------------------------- the package loader
@dataclass
class _Package:
    """The four files of an SVDQuant package, read once."""
    meta: dict
    tensors: Dict[str, torch.Tensor]
    aux: Dict[str, torch.Tensor]
    specs: Dict[str, dict]

    @classmethod
    def read(cls, pkg_dir: str) -> "_Package":
        from safetensors.torch import load_file

        def js(name):
            with open(os.path.join(pkg_dir, name)) as fh:
                return json.load(fh)

        return cls(js("meta.json"), load_file(os.path.join(pkg_dir, "weights.safetensors")),
                   load_file(os.path.join(pkg_dir, "aux.safetensors")), js("act_spec.json"))


@dataclass
class _Tally:
    splits: int = 0
    weights: int = 0
    folds: int = 0
    missing: List[str] = field(default_factory=list)
    skipped: List[str] = field(default_factory=list)


def _tensor_target(key: str) -> Tuple[str, str]:
    """Package key -> (module path, attribute): "<module>.weight" or "<module>.bias"; any other key is a weight."""
    head, _, tail = key.rpartition(".")
    if tail in ("weight", "bias") and head:
        return head, tail
    return key, "weight"


def _cut_split_modules(model: nn.Module, cuts: Dict[str, int], tally: _Tally) -> None:
    for path, in0 in cuts.items():
        owner_path, _, child = path.rpartition(".")
        owner = model.get_submodule(owner_path) if owner_path else model
        target = getattr(owner, child)
        if isinstance(target, nn.Linear):
            setattr(owner, child, SplitInLinear(target, int(in0)))
            tally.splits += 1


def _write_tensors(modules: Dict[str, nn.Module], tensors: Dict[str, torch.Tensor], tally: _Tally) -> None:
    for key, value in tensors.items():
        path, attr = _tensor_target(key)
        dest = getattr(modules.get(path), attr, None) if path in modules else None
        if dest is None:
            tally.missing.append(key)
            continue
        if dest.shape != value.shape:
            raise ValueError(f"package tensor {key} is {tuple(value.shape)}, the model's is {tuple(dest.shape)}")
        dest.data.copy_(value.to(dest.dtype))
        tally.weights += attr == "weight"


def _apply_specs(modules: Dict[str, nn.Module], pkg: _Package, fold_lowrank: bool, tally: _Tally) -> None:
    for name, spec in pkg.specs.items():
        target = modules.get(name.partition("@")[0])
        # custom-implementation specs and output-side quantizers have nothing to fold into a weight
        if spec.get("impl") or spec.get("where") == "output" or not isinstance(target, nn.Linear):
            tally.skipped.append(name)
            continue
        fold_one(target, spec, pkg.aux, fold_lowrank=fold_lowrank)
        tally.folds += 1


def load_method_weights(model: nn.Module, pkg_dir: str, verbose: bool = True, fold_lowrank: bool = False) -> dict:
    """Load an SVDQuant package into `model` as one effective 16-bit weight per Linear (the package's dequantized
    weights with smoothing / shift folded in, low-rank branches parked for Int8Linear), for convert_linears_to_int8 to
    derive the INT8 codes from (deploy/run_flux_latency.py:256-315). Returns the report dict the reference's drivers
    read."""
    pkg = _Package.read(pkg_dir)
    if pkg.meta.get("impl"):
        raise SystemExit(f"load_method_weights: {pkg_dir} declares its own implementation ({pkg.meta['impl']!r}); "
                         "only plain SVDQuant packages can be loaded as folded 16-bit weights")
    tally = _Tally()
    _cut_split_modules(model, pkg.meta.get("split_modules") or {}, tally)   # first: later keys name the halves
    modules = dict(model.named_modules())
    _write_tensors(modules, pkg.tensors, tally)
    _apply_specs(modules, pkg, fold_lowrank, tally)
    live = sum(getattr(m, LOWRANK_A_ATTR, None) is not None for m in model.modules())
    meta = pkg.meta
    report = {
        "method": meta.get("method"), "w_bits": meta.get("w_bits"), "a_bits_simulated_away": meta.get("a_bits"),
        "n_lowrank_branches_live": live, "group": meta.get("group"), "lowrank_rank": meta.get("lowrank_rank"),
        "n_weights_written": tally.weights, "n_layers_folded": tally.folds, "n_split_modules": tally.splits,
        "n_missing_keys": len(tally.missing), "n_specs_skipped": len(tally.skipped),
        "note": "package weights with smooth/shift folded into weight and bias on the GPU; low-rank branches kept "
                "live for Int8Linear; the INT8 codes are derived from these weights",
    }
    if verbose:
        print(f"[weights] {pkg_dir}: {meta.get('method')} W{meta.get('w_bits')} g{meta.get('group')} "
              f"r{meta.get('lowrank_rank')} | tensors {tally.weights} | folds {tally.folds} "
              f"(low-rank live {live}) | splits {tally.splits} | missing {len(tally.missing)} | "
              f"skipped {len(tally.skipped)}", flush=True)
    return report
