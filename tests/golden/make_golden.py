#!/usr/bin/env python3
"""Writes the golden fixtures of this directory from torch CPU restatements of the reference's own formulas.

The reference (PyraQuant) ships no golden vectors for its INT8 executor, so these fixtures are computed
here, independently of the C oracle (oracle/pq_oracle.c), by torch's own CPU operators following the
reference's torch lines:

  quant_*.npz      per-token quantizer      deploy/int8_exec.py:508-509
                   sc = |x|.amax(1).clamp_min(1e-8) / 127 ; q = round(x / sc).clamp(-127, 127)
  weight_rtn.npz   per-channel weight RTN    deploy/int8_exec.py:355-357
                   group-32 weight RTN       pyraquant/quantizers_weight.py:96-109 (qdq_weight(w, 8, 32))
  linear_lr.npz    int32 accumulator         deploy/int8_exec.py:259 (torch._int_mm(xq, w_int8.t()))
                   fp32 dequant (+bias)      deploy/int8_exec.py:506 / :119-123
                   low-rank down             deploy/int8_exec.py:390 (t = x @ lr_A, bf16)
  route_c4.json    config-4 routed row set   (16x16-token leaves, Bernoulli(0.35), seed 42, 2-token halo,
                                              union of the dilated leaves on the 256x256 token grid)

Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _quant_torch(x):
    xf = x.float()
    sc = xf.abs().amax(1, keepdim=True).clamp_min(1e-8) / 127
    q = torch.round(xf / sc).clamp(-127, 127).to(torch.int8)
    return q, sc[:, 0]


def _special_rows(K):
    """Rows that exercise the edges of the quantizer."""
    rows = torch.zeros(8, K)
    rows[1, :] = 1e-12                                       # below the 1e-8 clamp
    rows[2, 0] = 127.0                                       # scale 1: x = k + 0.5 are exact ties
    n = min(K - 1, 254)
    rows[2, 1:1 + n] = torch.arange(-127, -127 + n).float() + 0.5
    rows[3, 0] = -254.0                                      # negative absmax, scale 2: odd x are ties
    m = min(K - 1, 127)
    rows[3, 1:1 + m] = torch.arange(-127, -127 + m).float() * 2 + 1
    g = torch.Generator().manual_seed(7)
    rows[4, :] = torch.randn(K, generator=g) * 1e-39         # subnormals
    rows[5, :] = torch.randn(K, generator=g) * 1e30          # huge magnitudes
    rows[6, ::2] = -0.0
    rows[6, 1] = 3.0
    rows[7, :] = torch.randn(K, generator=g)
    return rows


def quant_fixture(dtype, name, M=24, K=1024, seed=101):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    cols = torch.randperm(K, generator=g)[: max(1, round(0.005 * K))]
    x[:, cols] *= 20.0
    x = torch.cat([x, _special_rows(K)]).to(dtype)
    q, s = _quant_torch(x)
    np.savez_compressed(os.path.join(HERE, name), x_bits=_bits(x), dtype=np.int32(0 if dtype == torch.bfloat16 else 1),
                        q=q.numpy(), s=s.numpy())


def weight_fixture(N=64, K=256, seed=102):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    w[3, :] = 0.0                                            # all-zero channel -> clamp
    w[5, 40] = 0.5                                           # one large element in group 1
    s = w.abs().amax(dim=1).clamp_min(1e-8) / 127.0
    q = torch.round(w / s[:, None]).clamp(-127, 127).to(torch.int8)
    wg = w.reshape(N, K // 32, 32)
    sg = wg.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8) / 127.0
    qg = torch.round(wg / sg).clamp(-127, 127).to(torch.int8).reshape(N, K)
    np.savez_compressed(os.path.join(HERE, "weight_rtn.npz"), w=w.numpy(), q_ch=q.numpy(), s_ch=s.numpy(),
                        q_g32=qg.numpy(), s_g32=sg.reshape(N, K // 32).numpy())


def linear_fixture(M=40, K=512, N=256, R=32, seed=103):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[:3]] *= 20.0
    x = x.to(torch.bfloat16)
    w = torch.randn(N, K, generator=g) * 0.02
    l1 = (torch.randn(K, R, generator=g) * 0.02).to(torch.bfloat16)
    l2 = (torch.randn(R, N, generator=g) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16).float()
    ws = w.abs().amax(dim=1).clamp_min(1e-8) / 127.0
    wq = torch.round(w / ws[:, None]).clamp(-127, 127).to(torch.int8)
    xq, sx = _quant_torch(x)
    acc = torch._int_mm(xq, wq.t())                          # M > 16 as torch._int_mm requires
    y = acc.float() * (sx[:, None] * ws[None, :]) + bias[None, :]
    t = x @ l1
    y_lr64 = (acc.double() * (sx[:, None].double() * ws[None, :].double()) + t.double() @ l2.double()
              + bias[None, :].double())
    np.savez_compressed(os.path.join(HERE, "linear_lr.npz"), x_bits=_bits(x), w_q=wq.numpy(), w_s=ws.numpy(),
                        bias=bias.numpy(), l1_bits=_bits(l1), l2_bits=_bits(l2), q=xq.numpy(), s=sx.numpy(),
                        acc=acc.numpy(), y_nolr=y.numpy(), t_bits=_bits(t), y_lr_f64=y_lr64.numpy())


def route_fixture():
    gen = torch.Generator().manual_seed(42)
    sel = (torch.rand(16, 16, generator=gen) < 0.35).numpy()
    covered = np.zeros((256, 256), bool)
    core = np.zeros((256, 256), bool)
    for i, j in zip(*np.nonzero(sel)):
        core[i * 16:(i + 1) * 16, j * 16:(j + 1) * 16] = True
        covered[max(0, i * 16 - 2):min(256, (i + 1) * 16 + 2), max(0, j * 16 - 2):min(256, (j + 1) * 16 + 2)] = True
    rows = np.flatnonzero(covered.reshape(-1)).astype(np.int32)
    rec = {"active_leaves": int(sel.sum()), "core_rows": int(core.sum()), "union_rows": int(rows.size),
           "first_rows": rows[:8].tolist(), "last_rows": rows[-8:].tolist(),
           "sha256_int32_le": hashlib.sha256(rows.astype("<i4").tobytes()).hexdigest(),
           "mask_rows": ["".join("1" if v else "0" for v in r) for r in sel]}
    with open(os.path.join(HERE, "route_c4.json"), "w") as fh:
        json.dump(rec, fh, indent=1)


if __name__ == "__main__":
    quant_fixture(torch.bfloat16, "quant_bf16.npz")
    quant_fixture(torch.float16, "quant_f16.npz", M=16, K=640, seed=104)
    weight_fixture()
    linear_fixture()
    route_fixture()
    print("fixtures written to", HERE)
