#!/usr/bin/env python3
"""Benchmark of the INT8 deployment hot path on one MI355X: one Int8Linear forward per step at the FLUX 4K MLP
up-projection (config c1: M=65536 tokens, K=3072, N=12288, rank-32 low-rank branch, bias, bf16 in/out).

A step is the whole layer on inputs already resident in HBM, as Int8Linear.forward runs it: per-token quantizer
writing packed K64 codes and the low-rank down-projection (t = x @ L1) in one pass over x, fused INT8 GEMM over
packed operands
+ dequant + low-rank up + bias epilogue (group-32 layers: per-group rescale in the GEMM's main loop). `value` = 2*M*N*K / step time (INT8 TOPS
of the whole layer). `roofline` prices the dominant kernel (the fused GEMM) against the dense INT8 MFMA peak
(5.0 POP/s) from HIP events recorded around every GEMM launch of the timed steps, on the stream it runs on.
`cpu_baseline` times the reference's torch CPU quantize + int-matmul path (restated in oracle/torch_ref.py) on
a bounded row sample of the same layer.

    python bench.py [--steps K] [--warmup W] [--config c1|c0|c2a|c2b|c3_1280|c3_5120|c3_1280_f16|c3_5120_f16|c4]
                    [--no-cpu] [--no-side] [--blaslt | --gemm-data | --copy-probe BYTES]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0      # dense INT8 MFMA, MI355X (TOP/s)
METRIC = "INT8 TOPS & % MFMA peak per Int8Linear at FLUX 4K shapes; µs/layer"


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c1")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-rows", type=int, default=16384, help="row sample of the CPU baseline")
    ap.add_argument("--cpu-iters", type=int, default=5)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run device-to-device copies of BYTES (3 to calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE "
                         "against a plain copy kernel of known size, then 10 timed: its read + write rate) and exit")
    ap.add_argument("--no-side", action="store_true",
                    help="skip the side measurements (routing kernels, SDXL small-M launches, weight fold), e.g. for "
                         "profiler runs that should hold the layer's kernels only")
    ap.add_argument("--gemm-data", action="store_true",
                    help="only time the layer's fused GEMM at the config's shape on the workload's own int8 codes and on "
                         "synthetic operand bytes (uniform random, constant, zero), interleaved, and print one JSON line")
    ap.add_argument("--blaslt", action="store_true",
                    help="only compare the int32-output GEMM with hipBLASLt's (torch._int_mm) on the config's "
                         "operands, like for like, and print one JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the INT8 executor "
              "has no multi-GPU path. Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import CONFIGS, make_linear, make_x, routed_rows

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    if args.copy_probe:
        # 3 device-to-device copies of BYTES (the PMC calibration), then 10 more timed by HIP events: the read + write
        # rate of a plain copy kernel, the practical roofline of a pass that reads and writes HBM at once
        src = torch.ones(args.copy_probe // 4, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            dst.copy_(src)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / 10 * 1e3
        nb = src.numel() * 4
        print(json.dumps({"copy_probe_bytes": nb, "copy_us": round(us, 1),
                          "read_plus_write_GBps": round(2 * nb / us / 1e3, 1),
                          "frac_hbm": round(2 * nb / us / 1e3 / HBM_PEAK_GBS, 4)}), flush=True)
        return 0
    cfg = CONFIGS[args.config]
    if args.blaslt:
        print(json.dumps(blaslt_compare(dev, cfg)), flush=True)
        return 0
    if args.gemm_data:
        print(json.dumps(gemm_data(dev, cfg)), flush=True)
        return 0
    lin = make_linear(cfg.K, cfg.N, cfg.lowrank, cfg.bias, dtype=cfg.dtype)
    q = E.Int8Linear(lin, device=dev, group_size=cfg.group)
    x = make_x(cfg.M, cfg.K, cfg.dtype).to(dev)
    rows = routed_rows(dev) if cfg.routed else None
    M = cfg.M if rows is None else int(rows.numel())
    canvas = torch.zeros(cfg.M, cfg.N, dtype=cfg.dtype, device=dev) if rows is not None else None
    out = canvas if canvas is not None else torch.empty(M, cfg.N, dtype=cfg.dtype, device=dev)

    ev = {k: [] for k in ("down", "quant", "gemm")}

    def step(record: bool):
        def mark():
            if not record:
                return None
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            return e

        e0 = mark()
        fused = q.weight_packed is not None and q.lr_At is not None
        if fused:   # quantizer + low-rank down-projection in one pass over x, as Int8Linear.forward runs it
            e1 = e0
            xq, sx, t = E.quant_rows_lowrank(x, q.lr_At, rows, q._lr_frag())
            e2 = mark()
        else:
            t = E.lowrank_down(x, q.lr_At, rows) if q.lr_At is not None else None
            e1 = mark()
        if fused:
            E.int8_gemm_packed(xq, sx, q.weight_packed, q._scale_k(), q.bias, M, cfg.N, cfg.K, cfg.dtype, t=t,
                               l2t=q.lr_Bt, out=out, out_row_idx=rows, group=q.group_size)
        elif q.weight_packed is not None:
            xq, sx = E.quant_rows_packed(x, rows)
            e2 = mark()
            E.int8_gemm_packed(xq, sx, q.weight_packed, q._scale_k(), q.bias, M, cfg.N, cfg.K, cfg.dtype, t=t,
                               l2t=q.lr_Bt, out=out, out_row_idx=rows, group=q.group_size)
        else:
            xq, sx = E.quant_rows(x, rows)
            e2 = mark()
            E._gemm(xq, sx, q.weight_int8, q._scale_k(), q.group_size, q.bias, t, q.lr_Bt, cfg.dtype, out, rows)
        e3 = mark()
        if record:
            if t is not None and not fused:
                ev["down"].append((e0, e1))
            ev["quant"].append((e1, e2))
            ev["gemm"].append((e2, e3))

    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    def avg_ms(k):
        v = [a.elapsed_time(b) for a, b in ev[k]]
        return sum(v) / len(v) if v else 0.0

    ms_step = elapsed / args.steps * 1e3
    ops = 2.0 * M * cfg.N * cfg.K
    value = ops / (ms_step * 1e-3) / 1e12
    gemm_ms = avg_ms("gemm")
    gemm_tops = ops / (gemm_ms * 1e-3) / 1e12
    quant_ms = avg_ms("quant")
    fused = q.weight_packed is not None and q.lr_At is not None
    # quantizer bytes: bf16 read + int8 codes + fp32 scale (+ index read); the fused pass also writes t
    quant_bytes = 3.0 * M * cfg.K + 4.0 * M + (4.0 * M if rows is not None else 0.0)
    if fused:
        quant_bytes += 2.0 * M * cfg.lowrank
    quant_gbs = quant_bytes / (quant_ms * 1e-3) / 1e9
    down_ms = avg_ms("down")

    # The per-token quantizer alone (north-star target: >= 70 % of HBM), timed outside the steps with HIP events:
    # the packed quantizer, as Int8Linear runs it on layers without the fused low-rank pass.
    qe0, qe1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(3):
        E.quant_rows_packed(x, rows)
    qe0.record()
    for _ in range(10):
        E.quant_rows_packed(x, rows)
    qe1.record()
    torch.cuda.synchronize()
    qa_ms = qe0.elapsed_time(qe1) / 10
    qa_bytes = 3.0 * M * cfg.K + 4.0 * M + (4.0 * M if rows is not None else 0.0)
    qa_gbs = qa_bytes / (qa_ms * 1e-3) / 1e9

    # The low-rank down-projection alone (t = x[rows] @ L1 by the LDS-DMA kernel), the path of layers the fused
    # quantizer pass does not take (other ranks, other K): x read once, L1^T, t written.
    lowrank_alone = None
    if q.lr_At is not None and x.dtype == q.lr_At.dtype:
        for _ in range(3):
            E.lowrank_down(x, q.lr_At, rows)
        qe0.record()
        for _ in range(10):
            E.lowrank_down(x, q.lr_At, rows)
        qe1.record()
        torch.cuda.synchronize()
        la_ms = qe0.elapsed_time(qe1) / 10
        rd = q.lr_At.shape[0]
        la_bytes = 2.0 * M * cfg.K + 2.0 * rd * cfg.K + 2.0 * M * rd + (4.0 * M if rows is not None else 0.0)
        lowrank_alone = {"kernel": "lowrank_down", "us": round(la_ms * 1e3, 1),
                         "GBps": round(la_bytes / (la_ms * 1e-3) / 1e9, 1),
                         "frac_hbm": round(la_bytes / (la_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         "bytes": "2 M K + 2 R K + 2 M R"}

    # HBM bytes per GEMM launch measured by rocprofv3 (FETCH_SIZE + WRITE_SIZE, copy-calibrated) for this config
    traffic, traffic_src = None, None
    prof = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"int8_gemm_{cfg.name}_traffic.json")
    if os.path.exists(prof):
        with open(prof) as fh:
            traffic = json.load(fh).get("traffic_bytes")
        traffic_src = os.path.relpath(prof, os.path.dirname(os.path.abspath(__file__)))

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(cfg, lin, args.cpu_rows, args.cpu_iters)
    side = not args.no_side
    routing = route_bench(dev, not args.no_cpu) if cfg.routed and side else None
    launch = launch_bench(dev) if cfg.group and side else None
    fold = fold_bench(dev, cfg) if cfg.name == "c1" and side else None
    mix = flux_linear_mix(dev) if cfg.name == "c1" and side else None

    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": f"{cfg.name}: one Int8Linear forward, M={M}, K={cfg.K}, N={cfg.N}, "
                        f"{'rank-%d low-rank, ' % cfg.lowrank if cfg.lowrank else ''}"
                        f"{'group-32 weights, ' if cfg.group else 'per-channel weights, '}"
                        f"{'bias, ' if cfg.bias else ''}{str(cfg.dtype).replace('torch.', '')} in/out"
                        f"{', routed gather/scatter into a 65536-row canvas' if rows is not None else ''}",
            "M": M, "K": cfg.K, "N": cfg.N,
            "us_per_layer": round(ms_step * 1e3, 1),
            "pct_int8_peak_layer": round(100.0 * value / INT8_PEAK_TOPS, 2),
            "kernels_us": ({"quant_rows_lowrank": round(quant_ms * 1e3, 1)} if fused else
                           ({"lowrank_down": round(down_ms * 1e3, 1)} if q.lr_At is not None else {}) |
                           {"quant_rows": round(quant_ms * 1e3, 1)}) | {"int8_gemm": round(gemm_ms * 1e3, 1)},
            ("quant_lowrank_GBps" if fused else "quant_rows_GBps"): round(quant_gbs, 1),
            ("quant_lowrank_frac_hbm" if fused else "quant_rows_frac_hbm"): round(quant_gbs / HBM_PEAK_GBS, 4),
            "quantizer_alone": {"kernel": "quant_rows_packed", "us": round(qa_ms * 1e3, 1),
                                "GBps": round(qa_gbs, 1), "frac_hbm": round(qa_gbs / HBM_PEAK_GBS, 4),
                                "bytes": f"3 M K + 4 M{' + 4 M (gather list)' if rows is not None else ''}"},
        } | ({"lowrank_down_alone": lowrank_alone} if lowrank_alone else {})
          | ({"routing": routing} if routing is not None else {}) | ({"small_m_launch": launch} if launch else {}) | ({"weight_fold": fold} if fold else {}) | ({"flux_linear_mix": mix} if mix else {}),
        "roofline": {
            "bound": "mfma",
            "achieved": round(gemm_tops, 2),
            "peak": INT8_PEAK_TOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_tops / INT8_PEAK_TOPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "kernel": "int8_gemm (fused dequant + low-rank + bias epilogue)",
            "work_per_launch": f"2*M*N*K = {ops:.4e} int8 ops",
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)
    return 0


def blaslt_compare(dev, cfg):
    """The same int8 operands through hipBLASLt (torch._int_mm: int32 [M, N] out, no epilogue) and through this build's
    GEMM with int32 output (packed and row-major operands), and the fused bf16 layer GEMM for reference. Each: 2
    warm-up calls, then 10 calls interleaved round-robin across the variants, each timed by its own HIP event pair on
    the launch stream; medians reported."""
    import torch

    from pyraquant_amd import int8_exec as E

    g = torch.Generator(device=dev).manual_seed(3)
    xq = torch.randint(-127, 128, (cfg.M, cfg.K), generator=g, device=dev, dtype=torch.int8)
    wq = torch.randint(-127, 128, (cfg.N, cfg.K), generator=g, device=dev, dtype=torch.int8)
    sx = torch.rand(cfg.M, generator=g, device=dev) * 0.02 + 0.001
    sw = torch.rand(cfg.N, generator=g, device=dev) * 0.001 + 1e-4
    bias = torch.randn(cfg.N, generator=g, device=dev) * 0.01
    xp, wp = E.pack_k64(xq), E.pack_k64(wq)
    out = torch.empty(cfg.M, cfg.N, dtype=torch.bfloat16, device=dev)
    wt = wq.t()
    variants = {
        "hipblaslt_int_mm_i32": lambda: torch._int_mm(xq, wt),
        "pq_int8_gemm_packed_i32": lambda: E.int8_gemm_packed(xp, None, wp, None, None, cfg.M, cfg.N, cfg.K, torch.int32),
        "pq_int8_gemm_i32_rowmajor": lambda: E.int8_gemm_i32(xq, wq),
        "pq_int8_gemm_packed_bf16_fused": lambda: E.int8_gemm_packed(xp, sx, wp, sw, bias, cfg.M, cfg.N, cfg.K,
                                                                     torch.bfloat16, out=out),
    }
    ref = torch._int_mm(xq, wt)
    same = {k: bool(torch.equal(f(), ref)) for k, f in variants.items() if k.endswith("i32") or "i32_" in k}
    times = {k: [] for k in variants}
    for f in variants.values():
        f()
        f()
    torch.cuda.synchronize()
    for _ in range(10):
        for k, f in variants.items():
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            f()
            e1.record()
            torch.cuda.synchronize()
            times[k].append(e0.elapsed_time(e1) * 1e3)
    ops = 2.0 * cfg.M * cfg.N * cfg.K
    res = {}
    for k, v in times.items():
        us = sorted(v)[len(v) // 2]
        res[k] = {"us": round(us, 1), "TOPS": round(ops / us / 1e6, 1), "frac_int8_peak": round(ops / us / 1e6 / INT8_PEAK_TOPS, 4)}
    return {"blaslt_compare": res, "int32_equal_to_int_mm": same, "config": cfg.name, "M": cfg.M, "K": cfg.K, "N": cfg.N}


def gemm_data(dev, cfg):
    """The layer's fused GEMM (packed operands, dequant + low-rank + bias epilogue, bf16 out) at the config's shape on
    four operand sets with the same scales, bias, t and lr_B: the workload's own codes (the config's x quantized by
    the layer's quantizer, its weights by the layer's RTN), uniform random codes in [-127, 127], a constant 90, and
    zeros. The MFMA's power draw, and so the clock it runs at, depends on the operand bits; the time on constant or
    zero operands is the same kernel with that dependence taken out. 2 warm-up calls each, then 10 rounds interleaved
    over the sets, each call timed by its own HIP event pair on the launch stream; medians."""
    import torch

    from pyraquant_amd import int8_exec as E
    from pyraquant_amd.workloads import make_linear, make_x

    q = E.Int8Linear(make_linear(cfg.K, cfg.N, cfg.lowrank, cfg.bias, dtype=cfg.dtype), device=dev,
                     group_size=cfg.group)
    x = make_x(cfg.M, cfg.K, cfg.dtype).to(dev)
    if q.lr_At is not None:
        xp, sx, t = E.quant_rows_lowrank(x, q.lr_At, None, q._lr_frag())
    else:
        (xp, sx), t = E.quant_rows_packed(x), None
    del x
    wp = q.weight_packed
    g = torch.Generator(device=dev).manual_seed(5)
    sets = {"workload": (xp, wp)}
    for name, fill in (("random", None), ("constant", 90), ("zero", 0)):
        if fill is None:
            a = torch.randint(-127, 128, (cfg.M, cfg.K), generator=g, device=dev, dtype=torch.int8)
            w = torch.randint(-127, 128, (cfg.N, cfg.K), generator=g, device=dev, dtype=torch.int8)
        else:
            a = torch.full((cfg.M, cfg.K), fill, device=dev, dtype=torch.int8)
            w = torch.full((cfg.N, cfg.K), fill, device=dev, dtype=torch.int8)
        sets[name] = (E.pack_k64(a), E.pack_k64(w))
        del a, w
    out = torch.empty(cfg.M, cfg.N, dtype=cfg.dtype, device=dev)

    def call(ap, wq):
        E.int8_gemm_packed(ap, sx, wq, q._scale_k(), q.bias, cfg.M, cfg.N, cfg.K, cfg.dtype, t=t, l2t=q.lr_Bt, out=out,
                           group=q.group_size)

    for ap, wq in sets.values():
        call(ap, wq)
        call(ap, wq)
    torch.cuda.synchronize()
    times = {k: [] for k in sets}
    stream = torch.cuda.current_stream(dev)
    for _ in range(10):
        for k, (ap, wq) in sets.items():
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            call(ap, wq)
            e1.record(stream)
            torch.cuda.synchronize()
            times[k].append(e0.elapsed_time(e1) * 1e3)
    ops = 2.0 * cfg.M * cfg.N * cfg.K
    res = {}
    for k, v in times.items():
        us = sorted(v)[len(v) // 2]
        res[k] = {"us": round(us, 1), "TOPS": round(ops / us / 1e6, 1),
                  "frac_int8_peak": round(ops / us / 1e6 / INT8_PEAK_TOPS, 4)}
    return {"gemm_data": res, "order": list(sets), "config": cfg.name, "M": cfg.M, "K": cfg.K, "N": cfg.N}


def fold_bench(dev, cfg):
    """The SVDQuant smoothing / shift fold of this layer's weight ([N, K] bf16, per-channel smooth and shift, bias) on
    the GPU (pq_fold_weight), beside the reference's own torch-op sequence for it (deploy/run_flux_latency.py:219-239)
    on the same GPU; 20 calls each after 3, queued behind a GPU sleep."""
    import torch

    from pyraquant_amd import weights

    g = torch.Generator().manual_seed(1)
    W = (torch.randn(cfg.N, cfg.K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    sm = (torch.rand(cfg.K, generator=g) + 0.5).to(dev)
    sh = (torch.randn(cfg.K, generator=g) * 0.1).to(dev)
    b = (torch.randn(cfg.N, generator=g) * 0.01).to(torch.bfloat16).to(dev)
    out = torch.empty_like(W)

    def torch_ops():
        Wf = W.float() / sm.reshape(1, -1)
        add = Wf @ sh.reshape(-1)
        b2 = b.clone().add_(add.to(b.dtype))
        out.copy_(Wf.to(W.dtype))
        return b2

    def timed(fn, n=20):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(50_000_000)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n * 1e3

    us = timed(lambda: weights.fold_weight(W, sm, sh, b, out=out))
    us_torch = timed(torch_ops)
    nbytes = 4.0 * cfg.N * cfg.K
    return {"shape": [cfg.N, cfg.K], "us": round(us, 1), "GBps": round(nbytes / us / 1e3, 1),
            "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "bytes": "2 N K read + 2 N K written",
            "reference_torch_ops_us": round(us_torch, 1)}


def launch_bench(dev):
    """SDXL's 1K stage (M = 2048 tokens) over its token-level (K, N) shapes, group-32 fp16 Int8Linear: per-layer GPU
    time (50 calls queued behind a GPU sleep), host time per eager call (200 calls, no synchronisation inside), and
    the per-layer time of a HIP graph of 10 captured calls replayed (deploy/run_sdxl_latency.py:144-147 quotes the
    reference's per-call launch overhead at this M)."""
    import torch

    from pyraquant_amd import sdxl
    from pyraquant_amd.workloads import make_linear, make_x

    M = 2048
    rows = []
    for K, N in sdxl.SDXL_TOKEN_SHAPES:
        q = sdxl.SdxlInt8Linear(make_linear(K, N, 0, True, dtype=torch.float16), device=dev, group_size=32)
        x = make_x(M, K, torch.float16, seed=K + N).to(dev)
        for _ in range(5):
            y = q(x)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(50_000_000)
        e0.record()
        for _ in range(50):
            y = q(x)
        e1.record()
        torch.cuda.synchronize()
        gpu = e0.elapsed_time(e1) / 50 * 1e3
        t0 = time.perf_counter()
        for _ in range(200):
            y = q(x)
        host = (time.perf_counter() - t0) / 200 * 1e6
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            y = q(x)
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ys = [q(x) for _ in range(10)]
        g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(20):
            g.replay()
        torch.cuda.synchronize()
        graph = (time.perf_counter() - t0) / 200 * 1e6
        rows.append({"K": K, "N": N, "gpu_us": round(gpu, 1), "host_us_per_eager_call": round(host, 1),
                     "graph_us_per_call": round(graph, 1), "graph_equals_eager": bool(torch.equal(ys[-1], y))})
    return {"M": M, "dtype": "fp16 in/out, group-32 weights, bias", "layers": rows}


def route_bench(dev, with_cpu: bool):
    """The routed executor's geometry and fusion kernels on config 4's mask (16 x 16-token leaves, 2-token halo,
    256 x 256 tokens; patches of 32-latent leaves) with FLUX's 64 packed latent channels, bf16: each kernel's
    average time over 20 calls after 3, HBM bytes per launch and the fraction of 8 TB/s. With with_cpu, the
    fusion of the oracle's torch CPU restatement (the reference's op sequence, flux/routing.py:328-379) is timed
    beside it."""
    import torch

    from pyraquant_amd import routing as RT

    H = W = 256
    C = 64
    sel = RT.leaf_mask().to(dev).to(torch.uint8)
    g = torch.Generator().manual_seed(5)
    hs = torch.randn(1, H * W, C, generator=g).to(torch.bfloat16).to(dev)
    bg = torch.randn(H * W, C, generator=g).to(torch.bfloat16).to(dev)

    def timed(fn, n=20):
        # The calls are queued behind a GPU sleep long enough to cover their host-side launch cost, so the event
        # pair brackets GPU execution only (these kernels run for microseconds, less than a Python call).
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(20_000_000)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n * 1e3

    us_union = timed(lambda: RT.union_rows(sel, 16, 2, (H, W), dev))
    rt = RT.route_patches(sel, leaf_latent=32, halo_tokens=2, token_hw=(H, W))
    us_patch = timed(lambda: RT.route_patches(sel, leaf_latent=32, halo_tokens=2, token_hw=(H, W)))
    info = rt.host()
    n = info["rows"]
    dst = torch.empty(n, C, dtype=torch.bfloat16, device=dev)
    us_gather = timed(lambda: RT.gather_rows(hs[0], rt.rows, rt.counts[1:2], n, out=dst))
    po = (torch.randn(n, C, generator=g) * 2).to(torch.bfloat16).to(dev)
    out = torch.empty_like(bg)
    us_fuse = timed(lambda: RT.fuse_patches(bg, po, rt, fusion_beta=1.0, out=out))
    gather_bytes = n * (2 * C * 2 + 4)
    fuse_bytes = 2 * H * W * C * 2 + n * C * 2
    res = {
        "mask": "config 4: 103 of 256 leaves, 16 x 16 tokens, halo 2, 256 x 256 tokens, 64 channels bf16",
        "patches": info["patches"], "patch_rows": n, "buckets": info["buckets"],
        "union_rows_us": round(us_union, 1), "route_patches_us": round(us_patch, 1),
        "gather_us": round(us_gather, 1), "gather_GBps": round(gather_bytes / us_gather / 1e3, 1),
        "fuse_us": round(us_fuse, 1), "fuse_GBps": round(fuse_bytes / us_fuse / 1e3, 1),
        "fuse_frac_hbm": round(fuse_bytes / us_fuse / 1e3 / HBM_PEAK_GBS, 4),
        "fuse_bytes": "2 H W C (background) + 2 H W C (out) + 2 rows C (patch predictions), x 2 bytes",
    }
    if with_cpu:
        from oracle import routing_ref as RR

        patches, _ = RR.patch_geometry(RR.route_boxes(sel.cpu(), 32), 2, (H, W))
        bgc, poc = bg.cpu().view(H, W, C), po.cpu()
        RR.fuse_patch_predictions(bgc, patches, poc)
        t0 = time.perf_counter()
        RR.fuse_patch_predictions(bgc, patches, poc)
        res["cpu_fuse_ms"] = round((time.perf_counter() - t0) * 1e3, 2)
        res["cpu_fuse_threads"] = torch.get_num_threads()
    return res


def _cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo, what lscpu prints as "Model name")."""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(cfg, lin, rows: int, iters: int):
    """The reference's torch CPU path (oracle/torch_ref.py) on the first `rows` rows of the same layer: median of
    `iters` timed calls after one warm-up, all host threads torch may use."""
    import torch

    from oracle import torch_ref
    from pyraquant_amd.workloads import make_x

    torch.set_num_threads(min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
    rows = min(rows, cfg.M)
    x = make_x(cfg.M, cfg.K, cfg.dtype)[:rows].contiguous()
    wq, ws = torch_ref.quant_weight(lin.weight.detach())
    b = lin.bias.detach().float() if lin.bias is not None else None
    from pyraquant_amd.int8_exec import LOWRANK_A_ATTR, LOWRANK_B_ATTR

    A = getattr(lin, LOWRANK_A_ATTR, None)
    B = getattr(lin, LOWRANK_B_ATTR, None)
    torch_ref.int8_linear(x, wq, ws, b, A, B)        # warm-up
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        torch_ref.int8_linear(x, wq, ws, b, A, B)
        times.append(time.perf_counter() - t0)
    dt = sorted(times)[len(times) // 2]
    ops = 2.0 * rows * cfg.N * cfg.K
    return {"value": round(ops / dt / 1e12, 4), "unit": "TOPS", "cores": torch.get_num_threads(), "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": f"{rows} of {cfg.M} rows of {cfg.name} (K={cfg.K}, N={cfg.N}), torch CPU quantize + "
                      f"_int_mm + dequant + low-rank, median of {iters} after 1 warm-up; "
                      f"{dt * 1e3:.1f} ms per sample (all: {', '.join(f'{t * 1e3:.0f}' for t in times)} ms)"}


def flux_linear_mix(dev):
    """The reference's own per-image micro-benchmark (deploy/int8_exec.py:539-571, run here by
    int8_exec.selftest_and_bench): for each token count M the four FLUX token-level Linear shapes, bf16 F.linear
    against Int8Linear, summed with the per-image layer counts of FLUX_TOKEN_SHAPES (418 layers)."""
    import contextlib

    from pyraquant_amd import int8_exec as E

    with contextlib.redirect_stdout(sys.stderr):   # its progress lines; stdout carries the one JSON line
        res = E.selftest_and_bench(Ms=(4352, 16640, 33744, 65792), iters=10)
    out = {}
    for M, r in res["per_M"].items():
        out[M] = {k: r[k] for k in ("bf16_ms", "int8_fused_ms", "quant_ms", "gemm_fused_ms", "speedup_fused_vs_bf16")}
        out[M]["per_shape_int8_ms"] = {k: v["int8_fused_ms"] for k, v in r["per_shape"].items()}
    return {"per_M": out, "selftest": res["selftest"],
            "note": "ms per image for the 418 token-level Linears (per-shape mean x layer count); bf16 = torch F.linear "
                    "(hipBLASLt), int8 = Int8Linear.forward without low rank, as the reference's benchmark"}


if __name__ == "__main__":
    sys.exit(main())
