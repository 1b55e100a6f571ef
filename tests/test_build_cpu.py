"""The build's per-kernel resource record (pyraquant_amd/kernel_resources.tsv, written by build() from the compiler's
resource-usage remarks): no kernel of libpqint8.so spills registers to scratch. A spill's reload waits with
vmcnt(0), which in the persistent, prefetching kernels also waits for the next batch's loads, so one spilled
register can serialise a pipeline without any test noticing a wrong value. Scalar registers the compiler parks in
vector-register lanes (v_writelane / v_readlane: the persistent 256 x 256 GEMM keeps its per-launch scalars there
across the tile loop) touch no memory and are allowed as long as the kernel uses no scratch at all."""
import csv
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PATH = os.path.join(ROOT, "pyraquant_amd", "kernel_resources.tsv")


def _rows():
    if not os.path.exists(PATH):
        pytest.skip("kernel_resources.tsv is written by build(); run it first")
    with open(PATH) as f:
        return list(csv.DictReader(f, delimiter="\t"))


def test_resource_record_covers_the_hot_kernels():
    names = " ".join(r["kernel"] for r in _rows())
    for k in ("gemm_dma_kernel", "quant_rows_vec_kernel", "quant_lowrank_kernel", "quant_lowrank_wide_kernel",
              "lowrank_down_dma_kernel", "pack_lowrank_l1t_kernel", "fuse_patches_kernel"):
        assert k in names, k


def test_no_kernel_spills_registers():
    bad = [(r["kernel"][:120], r["vgpr_spill"], r["sgpr_spill"], r["scratch"]) for r in _rows()
           if int(r["vgpr_spill"] or 0) or int(r["scratch"] or 0)]
    assert not bad, bad


def test_scalar_spills_stay_in_vector_lanes():
    # a scalar spill with no scratch is held in VGPR lanes; only the persistent GEMM blocks have any
    rows = [r for r in _rows() if int(r["sgpr_spill"] or 0)]
    assert all(int(r["scratch"] or 0) == 0 for r in rows)
    assert all("gemm_dma_kernel<4, 2, 4, 5, 1," in r["kernel"] for r in rows), [r["kernel"][:80] for r in rows]
