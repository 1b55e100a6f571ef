"""Build libpqint8.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python -m pyraquant_amd.build          # compiles every csrc/*.hip, links pyraquant_amd/libpqint8.so

Flags: gfx950 only; -ffp-contract=off so the fp32 epilogue follows source order (multiply, then add, as
the reference's epilogue is written); correctly rounded fp32 division (the quantizer's codes depend on
it); packed-fp32 instruction selection disabled.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_PATH = os.path.join(HERE, "libpqint8.so")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build libpqint8.so")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build(verbose: bool = False) -> str:
    """Compile every csrc/*.hip for gfx950 and link libpqint8.so (always recompiles)."""
    hipcc = _hipcc()
    srcs = sources()
    with tempfile.TemporaryDirectory(prefix="pq_build_") as tmp:
        def compile_one(src):
            obj = os.path.join(tmp, os.path.basename(src) + ".o")
            cmd = [hipcc, *HIP_FLAGS, "-c", src, "-o", obj]
            r = subprocess.run(cmd, capture_output=True, text=True)
            msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "not a recognized feature" not in l)
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src}:\n{msg}")
            if verbose and msg.strip():
                print(msg, file=sys.stderr)
            return obj

        with ThreadPoolExecutor(max_workers=min(4, len(srcs))) as ex:
            objs = list(ex.map(compile_one, srcs))
        out_tmp = LIB_PATH + ".tmp"
        cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out_tmp, *objs]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
        os.replace(out_tmp, LIB_PATH)
    build_probe()
    return LIB_PATH


PROBE_SRC = os.path.join(CSRC, "probe", "mfma_ceiling.hip")
PROBE_PATH = os.path.join(HERE, "libpqprobe.so")


def build_probe() -> str:
    """The register-only MFMA throughput probe (`bench.py --mfma-ceiling`), a library of its own: it measures the
    chip, it is not part of the executor's ABI."""
    cmd = [_hipcc(), *HIP_FLAGS, "-shared", PROBE_SRC, "-o", PROBE_PATH + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {PROBE_SRC}:\n{r.stdout}{r.stderr}")
    os.replace(PROBE_PATH + ".tmp", PROBE_PATH)
    return PROBE_PATH


if __name__ == "__main__":
    print(build(verbose=True))
