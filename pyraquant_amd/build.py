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


RESOURCES_PATH = os.path.join(HERE, "kernel_resources.tsv")
_RESOURCE_KEYS = {"VGPRs": "vgprs", "AGPRs": "agprs", "VGPRs Spill": "vgpr_spill", "SGPRs Spill": "sgpr_spill",
                  "ScratchSize [bytes/lane]": "scratch", "Occupancy [waves/SIMD]": "occupancy",
                  "LDS Size [bytes/block]": "lds"}


def _parse_resources(text: str) -> list:
    """The compiler's per-kernel resource remarks (-Rpass-analysis=kernel-resource-usage) as dicts."""
    rows, cur = [], None
    for line in text.splitlines():
        if "remark:" not in line or "kernel-resource-usage" not in line:
            continue
        body = line.split("remark:", 1)[1].rsplit("[-Rpass-analysis", 1)[0].strip()
        if body.startswith("Function Name:"):
            cur = {"name": body.split(":", 1)[1].strip()}
            rows.append(cur)
        elif cur is not None and ":" in body:
            key, val = body.rsplit(":", 1)
            if key.strip() in _RESOURCE_KEYS:
                cur[_RESOURCE_KEYS[key.strip()]] = val.strip()
    return rows


def _write_resources(rows: list) -> None:
    """kernel_resources.tsv beside the library: one line per kernel (demangled where c++filt exists), read by the
    CPU test that keeps the hot kernels free of register spills."""
    names = [r["name"] for r in rows]
    filt = shutil.which("c++filt")
    if filt and names:
        out = subprocess.run([filt], input="\n".join(names), capture_output=True, text=True).stdout.splitlines()
        if len(out) == len(names):
            names = out
    cols = ("vgprs", "agprs", "vgpr_spill", "sgpr_spill", "scratch", "occupancy", "lds")
    with open(RESOURCES_PATH + ".tmp", "w") as f:
        f.write("kernel\t" + "\t".join(cols) + "\n")
        for name, r in sorted(zip(names, rows)):
            f.write(name.replace("\t", " ") + "\t" + "\t".join(r.get(c, "") for c in cols) + "\n")
    os.replace(RESOURCES_PATH + ".tmp", RESOURCES_PATH)


def build(verbose: bool = False) -> str:
    """Compile every csrc/*.hip for gfx950 and link libpqint8.so (always recompiles); record each kernel's registers
    and spills in kernel_resources.tsv."""
    hipcc = _hipcc()
    srcs = sources()
    resources = []
    with tempfile.TemporaryDirectory(prefix="pq_build_") as tmp:
        def compile_one(src):
            obj = os.path.join(tmp, os.path.basename(src) + ".o")
            cmd = [hipcc, *HIP_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", src, "-o", obj]
            r = subprocess.run(cmd, capture_output=True, text=True)
            text = r.stdout + r.stderr
            msg = "\n".join(l for l in text.splitlines()
                            if "not a recognized feature" not in l and "kernel-resource-usage" not in l
                            and not l.startswith(" ") and l.strip())
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src}:\n{msg}")
            if verbose and msg.strip():
                print(msg, file=sys.stderr)
            return obj, _parse_resources(text)

        with ThreadPoolExecutor(max_workers=min(4, len(srcs))) as ex:
            done = list(ex.map(compile_one, srcs))
        objs = [o for o, _ in done]
        for _, rows in done:
            resources.extend(rows)
        _write_resources(resources)
        out_tmp = LIB_PATH + ".tmp"
        cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out_tmp, *objs]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
        os.replace(out_tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
