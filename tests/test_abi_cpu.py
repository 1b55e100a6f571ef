"""CPU checks of the C ABI (no GPU needed): libpqint8.so loads, exports every entry point that
include/pyraquant_amd.h declares, reports its ABI version, and rejects invalid arguments with the documented
status codes before touching the GPU; the Python layer maps those codes to the reference's exception types."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pyraquant_amd.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pq_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    import pyraquant_amd._lib as L

    return L.load()


def test_header_declares_expected_symbols():
    names = _declared()
    assert "pq_quant_rows" in names and "pq_int8_gemm" in names and "pq_quant_weight" in names
    import pyraquant_amd._lib as L

    assert names == sorted(L.EXPORTS), (names, sorted(L.EXPORTS))


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), f"libpqint8.so does not export {name}"


def test_abi_version(lib):
    import pyraquant_amd._lib as L

    assert lib.pq_abi_version() == L.ABI_VERSION


def test_invalid_arguments_rejected_without_gpu(lib):
    """Argument validation runs on the host before any HIP call."""
    import pyraquant_amd._lib as L

    nul = None
    # quantizer: null pointers, bad shapes, bad dtype
    assert lib.pq_quant_rows(nul, 0, 4, 64, 64, 4, nul, nul, nul, nul) == L.PQ_EINVAL
    assert lib.pq_quant_rows(nul, 0, -1, 64, 64, 4, nul, nul, nul, nul) == L.PQ_ESHAPE
    assert lib.pq_quant_rows(ctypes.c_void_p(16), 0, 4, 64, 32, 4, nul, ctypes.c_void_p(16), ctypes.c_void_p(16),
                             nul) == L.PQ_ESHAPE          # ldx < K
    assert lib.pq_quant_rows(ctypes.c_void_p(16), 7, 4, 64, 64, 4, nul, ctypes.c_void_p(16), ctypes.c_void_p(16),
                             nul) == L.PQ_EDTYPE
    assert lib.pq_quant_rows(nul, 0, 0, 64, 64, 0, nul, nul, nul, nul) == L.PQ_OK      # empty: nothing to do
    # x_rows: at least one row, and every row of an ungathered x
    assert lib.pq_quant_rows(ctypes.c_void_p(16), 0, 4, 64, 64, 3, nul, ctypes.c_void_p(16), ctypes.c_void_p(16),
                             nul) == L.PQ_ESHAPE
    assert b"x_rows" in lib.pq_last_error()
    assert lib.pq_quant_rows_packed(ctypes.c_void_p(16), 0, 4, 64, 64, 0, ctypes.c_void_p(16), ctypes.c_void_p(16),
                                    ctypes.c_void_p(16), nul) == L.PQ_ESHAPE
    assert b"dtype" in lib.pq_last_error() or lib.pq_last_error() is not None
    # GEMM: K % 64, N % 64, alignment, group, rank
    p16 = ctypes.c_void_p(256)
    args = dict(a=p16, lda=128, w=p16, ldw=128, s_row=p16, s_w=p16, group=0, bias=nul, t=nul, ldt=0, l2t=nul, R=0,
                lr=0, c=p16, ldc=128, od=0, ori=nul, c_rows=0, M=8, N=128, K=128, sched=nul, st=nul)

    def gemm(**kw):
        a = dict(args, **kw)
        return lib.pq_int8_gemm(a["a"], a["lda"], a["w"], a["ldw"], a["s_row"], a["s_w"], a["group"], a["bias"],
                                a["t"], a["ldt"], a["l2t"], a["R"], a["lr"], a["c"], a["ldc"], a["od"], a["ori"],
                                a["c_rows"], a["M"], a["N"], a["K"], a["sched"], a["st"])

    assert gemm(K=96, lda=96, ldw=96) == L.PQ_ESHAPE
    assert gemm(N=96) == L.PQ_ESHAPE
    assert gemm(a=ctypes.c_void_p(8)) == L.PQ_EALIGN
    assert gemm(group=16) == L.PQ_ESHAPE
    assert gemm(group=32, N=1 << 17, K=1 << 16, lda=1 << 16, ldw=1 << 16, ldc=1 << 17) == L.PQ_ESHAPE   # s_w > 1 GB
    assert b"group-32 scales" in lib.pq_last_error()
    assert gemm(ldc=1 << 31) == L.PQ_ESHAPE             # row offsets are 32 x 32-bit products
    assert gemm(t=p16, l2t=p16, R=24, ldt=24) == L.PQ_ESHAPE
    assert gemm(t=p16, l2t=nul, R=32, ldt=32) == L.PQ_EINVAL
    assert gemm(t=p16, l2t=p16, R=32, ldt=(1 << 22) + 8) == L.PQ_ESHAPE   # t rows at 32-bit buffer offsets
    assert lib.pq_int8_gemm_packed(p16, p16, p16, p16, 0, nul, p16, (1 << 22) + 8, p16, 32, 0, p16, 128, 0, nul, 0,
                                   8, 128, 128, nul, nul) == L.PQ_ESHAPE
    # the scheduling buffer holds int32 counters
    assert gemm(sched=ctypes.c_void_p(258)) == L.PQ_EALIGN
    assert lib.pq_int8_gemm_packed(p16, p16, p16, p16, 0, nul, nul, 0, nul, 0, 0, p16, 128, 0, nul, 0,
                                   8, 128, 128, ctypes.c_void_p(258), nul) == L.PQ_EALIGN
    assert b"sched" in lib.pq_last_error()
    # a scatter needs the canvas's row count
    assert gemm(ori=p16, c_rows=0) == L.PQ_ESHAPE
    assert b"c_rows" in lib.pq_last_error()
    assert lib.pq_int8_gemm_packed(p16, p16, p16, p16, 0, nul, nul, 0, nul, 0, 0, p16, 128, 0, p16, 0,
                                   8, 128, 128, nul, nul) == L.PQ_ESHAPE
    assert gemm(od=5) == L.PQ_EDTYPE or gemm(od=5) == L.PQ_ELAUNCH
    assert gemm(M=0) == L.PQ_OK
    assert lib.pq_int8_gemm_i32(p16, 128, p16, 128, nul, 128, 8, 128, 128, nul) == L.PQ_EINVAL
    assert lib.pq_quant_weight(nul, 4, 64, 64, 0, nul, nul, nul) == L.PQ_EINVAL
    assert lib.pq_quant_weight(p16, 4, 64, 64, 48, p16, p16, nul) == L.PQ_ESHAPE
    assert lib.pq_lowrank_down(p16, 0, 8, 128, 128, 8, nul, p16, 24, p16, 32, nul) == L.PQ_ESHAPE
    assert lib.pq_lowrank_down(p16, 0, 8, 128, 128, 4, nul, p16, 32, p16, 32, nul) == L.PQ_ESHAPE   # x_rows < M
    # grids beyond the 32-bit work-item count of one dispatch are refused before any launch
    assert lib.pq_quant_rows(p16, 0, (1 << 26) + 64, 64, 64, (1 << 26) + 64, nul, p16, p16, nul) == L.PQ_ESHAPE
    assert b"32-bit dispatch" in lib.pq_last_error()
    assert lib.pq_pack_k64(p16, 1 << 31, 64 * 1024, 64 * 1024, p16, nul) == L.PQ_ESHAPE
    assert lib.pq_int8_gemm_i32(p16, 64, p16, 64, p16, 1 << 16, 1 << 30, 1 << 16, 64, nul) == L.PQ_ESHAPE
    assert b"32-bit dispatch" in lib.pq_last_error()
    assert lib.pq_dequant_epilogue(nul, nul, nul, nul, nul, 128, 0, 8, 128, nul) == L.PQ_EINVAL
    # routing geometry and fusion
    assert lib.pq_route_union_rows(nul, 16, 16, 16, 2, 256, 256, p16, p16, nul) == L.PQ_EINVAL
    assert lib.pq_route_union_rows(p16, 16, 16, 16, 2, 200, 256, p16, p16, nul) == L.PQ_ESHAPE   # leaves past H
    assert lib.pq_route_union_rows(p16, 16, 16, 16, -1, 256, 256, p16, p16, nul) == L.PQ_ESHAPE
    assert lib.pq_route_patches(p16, 8, 8, 63, 8, 256, 256, 0, p16, p16, p16, 100, nul) == L.PQ_EINVAL  # odd leaf
    assert lib.pq_route_patches(p16, 8, 8, 64, 8, 256, 256, 2, p16, p16, p16, 100, nul) == L.PQ_EINVAL  # offset
    assert lib.pq_route_patches(p16, 8, 8, 64, 8, 255, 256, 0, p16, p16, p16, 100, nul) == L.PQ_ESHAPE
    assert lib.pq_route_patches(p16, 64, 128, 4, 1, 256, 256, 0, p16, p16, p16, 100, nul) == L.PQ_ESHAPE  # boxes
    assert lib.pq_gather_rows(p16, 12, p16, p16, 10, 6, p16, 12, nul) == L.PQ_EALIGN
    assert lib.pq_gather_rows(p16, 12, p16, p16, 0, 12, p16, 12, nul) == L.PQ_OK
    fuse = lambda C, beta, dt, ldb, halo=2: lib.pq_fuse_patches(p16, ldb, p16, C, p16, p16, p16, halo, beta, 16, 16,
                                                                C, dt, p16, C, nul)
    assert fuse(12, 1.0, 0, 12) == L.PQ_ESHAPE           # C % 8
    assert fuse(16, 1.5, 0, 16) == L.PQ_EINVAL           # fusion_beta outside [0, 1]
    assert fuse(16, 1.0, 0, 20) == L.PQ_EALIGN
    assert fuse(16, 1.0, 2, 16) == L.PQ_EDTYPE
    assert fuse(16, 1.0, 0, 16, halo=65) == L.PQ_EINVAL
    assert lib.pq_route_union_rows(p16, 4, 65, 4, 1, 256, 260, p16, p16, nul) == L.PQ_ESHAPE   # > 64 leaf columns


def test_status_codes_map_to_reference_exceptions(lib):
    """AssertionError for shapes / alignment (deploy/int8_exec.py:206, 221, 235), ValueError for dtypes
    (:67-68), RuntimeError for launch failures."""
    import pyraquant_amd._lib as L

    with pytest.raises(AssertionError):
        L.check(L.PQ_ESHAPE, "x")
    with pytest.raises(AssertionError):
        L.check(L.PQ_EALIGN, "x")
    with pytest.raises(ValueError):
        L.check(L.PQ_EDTYPE, "x")
    with pytest.raises(RuntimeError):
        L.check(L.PQ_ELAUNCH, "x")
    L.check(L.PQ_OK, "x")


def test_python_api_surface():
    """The reference's module-level names exist (deploy/int8_exec.py:58-74, 202-474; run_sdxl_latency.py:104-298)
    and fail loudly on CPU tensors instead of falling back."""
    import torch

    from pyraquant_amd import int8_exec as E
    from pyraquant_amd import sdxl

    for n in ("BACKENDS", "DEFAULT_BACKEND", "set_backend", "get_backend", "quant_rows", "dequant_epilogue",
              "int8_linear_2d", "int8_gemm_fused", "int8_gemm_lr", "LOWRANK_A_ATTR", "LOWRANK_B_ATTR", "Int8Linear",
              "is_bf16_whitelisted", "convert_linears_to_int8", "warm_kernels", "FLUX_TOKEN_SHAPES", "_bench",
              "selftest_and_bench"):
        assert hasattr(E, n), n
    for n in ("SdxlInt8Linear", "sdxl_int8_linear_2d", "convert_unet_linears_to_int8", "warm_sdxl_kernels",
              "SDXL_TOKEN_SHAPES", "fast_quant_rows", "fast_gemm_fused", "is_fp16_whitelisted_sdxl"):
        assert hasattr(sdxl, n), n
    assert E.LOWRANK_A_ATTR == "_lowrank_A" and E.LOWRANK_B_ATTR == "_lowrank_B"
    with pytest.raises(AssertionError):
        E.quant_rows(torch.zeros(4, 64, dtype=torch.bfloat16))
    with pytest.raises(AssertionError):
        E.Int8Linear(torch.nn.Linear(64, 64))
    assert E.set_backend("triton") == "hip"
    with pytest.raises(ValueError):
        E.set_backend("cublas")


def test_whitelists():
    """bf16 whitelist of deploy/int8_exec.py:415-421 and the SDXL fp16 whitelist of run_sdxl_latency.py:227-229."""
    from pyraquant_amd.int8_exec import is_bf16_whitelisted
    from pyraquant_amd.sdxl import is_fp16_whitelisted_sdxl

    for n in ("x_embedder", "context_embedder.linear", "proj_out", "time_text_embed.timestep_embedder.linear_1",
              "norm_out.linear", "transformer_blocks.0.norm1.linear", "single_transformer_blocks.3.norm.linear"):
        assert is_bf16_whitelisted(n), n
    for n in ("transformer_blocks.0.attn.to_q", "single_transformer_blocks.3.proj_mlp", "transformer_blocks.0.ff.net.2",
              "single_transformer_blocks.0.proj_out"):
        assert not is_bf16_whitelisted(n), n
    assert is_fp16_whitelisted_sdxl("time_embedding.linear_1") and is_fp16_whitelisted_sdxl("down.0.time_emb_proj")
    assert not is_fp16_whitelisted_sdxl("down_blocks.1.attentions.0.proj_in")


def test_lowrank_widths():
    """Rank -> (columns of t the down-projection computes, rank the GEMM epilogue takes; 0 = after the GEMM)."""
    from pyraquant_amd.int8_exec import _lowrank_widths

    expect = {1: (32, 16), 16: (32, 16), 17: (32, 32), 32: (32, 32), 33: (64, 64), 48: (64, 64), 64: (64, 64),
              65: (96, 0), 96: (96, 0), 128: (128, 0), 129: (0, 0), 200: (0, 0)}
    for r, w in expect.items():
        assert _lowrank_widths(r) == w, (r, _lowrank_widths(r), w)


def test_pack_lowrank_l1t_rejects_without_gpu(lib):
    """pq_pack_lowrank_l1t refuses shapes without a fragment order, bad dtypes and null or misaligned pointers before
    any HIP call; pq_quant_rows_lowrank refuses a misaligned l1f the same way. lowrank_l1t_packable states the same
    shape rule on the host."""
    import pyraquant_amd._lib as L
    from pyraquant_amd.int8_exec import lowrank_l1t_packable

    p16, nul = ctypes.c_void_p(256), None
    assert lib.pq_pack_lowrank_l1t(nul, 0, 32, 3072, p16, nul) == L.PQ_EINVAL
    assert lib.pq_pack_lowrank_l1t(p16, 2, 32, 3072, p16, nul) == L.PQ_EDTYPE
    for R, K in ((64, 3072), (16, 3072), (32, 4096), (32, 3136), (32, 768), (32, 12288)):
        assert not lowrank_l1t_packable(R, K)
        assert lib.pq_pack_lowrank_l1t(p16, 0, R, K, p16, nul) == L.PQ_ESHAPE, (R, K)
    assert b"fragment order" in lib.pq_last_error()
    assert lib.pq_pack_lowrank_l1t(p16, 1, 32, 1280, ctypes.c_void_p(264), nul) == L.PQ_EINVAL
    assert [K for K in range(256, 16384, 256) if lowrank_l1t_packable(32, K)] == [1024, 1280, 2048, 2560, 3072]
    assert lib.pq_quant_rows_lowrank(p16, 0, 16, 3072, 3072, 16, nul, p16, ctypes.c_void_p(264), 32, p16, p16, p16, 32,
                                     nul) == L.PQ_EINVAL
    assert b"l1f" in lib.pq_last_error()
