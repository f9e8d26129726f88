"""The C-ABI boundary without a GPU: libqmm.so loads, exports every entry point include/qmm.h declares with the
argument count the ctypes binding uses, and its host-side validation turns bad arguments into the documented
negative status before anything reaches the device (the reference's generators assert the same preconditions at
generation time, S/gen_llm.py:4573, S/gen_moe.py:121). No compute call is made here.
"""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qmm.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^(?:int|int64_t|const char \*)\s*(qmm_\w+)\(([^)]*)\);", text, flags=re.M):
        args = [a.strip() for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        out[m.group(1)] = len(args)
    return out


def header_enum(name):
    text = open(HEADER).read()
    body = re.search(r"enum %s \{(.*?)\};" % name, text, flags=re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    return {k.strip(): int(v) for k, v in re.findall(r"(\w+)\s*=\s*(-?\d+)", body)}


@pytest.fixture(scope="module")
def lib():
    from qmm import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from qmm import build
        build.build()
    return _lib.load()


def test_binding_covers_the_header():
    from qmm import _lib
    decl = header_functions()
    assert len(decl) >= 15
    assert set(decl) == set(_lib.SIGNATURES), set(decl) ^ set(_lib.SIGNATURES)
    for name, n in decl.items():
        assert len(_lib.SIGNATURES[name]) == n, name


def test_library_exports_every_declared_symbol(lib):
    for name in header_functions():
        assert hasattr(lib, name), name


def test_enums_match_python_tables():
    from qmm import formats
    fmt = header_enum("qmm_format")
    assert {k.lower()[4:]: v for k, v in fmt.items()} == formats.CODE
    dt = header_enum("qmm_dtype")
    assert {k.lower()[4:]: v for k, v in dt.items()} == formats.DTYPE
    st = header_enum("qmm_status")
    assert st["QMM_OK"] == 0 and all(v < 0 for k, v in st.items() if k != "QMM_OK")


def test_host_only_entry_points(lib):
    assert lib.qmm_version() >= 100
    assert lib.qmm_row_bytes(1, 4096) == 2304
    assert lib.qmm_row_bytes(0, 2816) == 1584
    assert lib.qmm_row_bytes(2, 2880) == 1530
    assert lib.qmm_row_bytes(3, 2880) == 1440
    assert lib.qmm_row_bytes(4, 2880) == 1440          # MFMA-tiled planes: the split nibble plane's bytes
    assert lib.qmm_row_bytes(5, 4096) == 2304          # tiled Q4_K: the GGUF row's bytes
    assert lib.qmm_row_bytes(6, 768) == 630            # Q6_K: 210 bytes per 256 values
    assert lib.qmm_mxfp4t_scale_bytes(64, 2880) == 2 * 12 * 256   # 45 chunks -> 12 groups of four
    assert lib.qmm_mxfp4t_scale_bytes(48, 2880) == 0 and lib.qmm_mxfp4t_scale_bytes(64, 2848) == 0
    assert lib.qmm_row_bytes(1, 100) == 0
    assert lib.qmm_row_bytes(7, 256) == 0
    assert lib.qmm_strerror(-2) == b"invalid shape"


def test_argument_validation_without_a_device(lib):
    """Each call fails host-side validation, so nothing is launched (the pointers are never dereferenced)."""
    st = header_enum("qmm_status")
    fake = ctypes.c_void_p(0x1000)      # a non-null, 4 KiB-aligned address that is never touched
    odd = ctypes.c_void_p(0x1002)
    n = None
    # qmm_mv: unsupported format, null x, K not a multiple of the block, bad dtype, misaligned Q4_K weights
    assert lib.qmm_mv(9, 256, 4, 1, 0, fake, 0, fake, n, fake, n) == st["QMM_ERR_FORMAT"]
    assert lib.qmm_mv(1, 256, 4, 1, 0, n, 0, fake, n, fake, n) == st["QMM_ERR_NULL"]
    assert lib.qmm_mv(1, 100, 4, 1, 0, fake, 0, fake, n, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_mv(1, 256, 4, 1, 0, fake, 1, fake, n, fake, n) == st["QMM_ERR_DTYPE"]
    assert lib.qmm_mv(1, 256, 4, 1, 0, fake, 0, odd, n, fake, n) == st["QMM_ERR_ALIGN"]
    assert lib.qmm_mv(0, 32, 4, 1, 0, fake, 0, fake, n, fake, n) == st["QMM_ERR_SHAPE"]     # Q4_0 needs K % 64
    assert lib.qmm_mv(3, 64, 4, 1, 0, fake, 0, fake, n, fake, n) == st["QMM_ERR_NULL"]      # split planes need ws
    # dequant
    assert lib.qmm_dequant(1, n, n, 4, 256, fake, n) == st["QMM_ERR_NULL"]
    assert lib.qmm_dequant(1, fake, n, 0, 256, fake, n) == st["QMM_ERR_SHAPE"]
    # top-k: E, KU and gating ranges
    assert lib.qmm_moe_topk(fake, 4, 300, 4, 1, 1, ctypes.c_float(1), n, fake, fake, n) == st["QMM_ERR_RANGE"]
    assert lib.qmm_moe_topk(fake, 4, 32, 9, 1, 1, ctypes.c_float(1), n, fake, fake, n) == st["QMM_ERR_RANGE"]
    assert lib.qmm_moe_topk(fake, 4, 32, 4, 4, 1, ctypes.c_float(1), n, fake, fake, n) == st["QMM_ERR_RANGE"]
    assert lib.qmm_moe_topk(fake, 4, 32, 4, 1, 1, ctypes.c_float(1), fake, fake, fake, n) == st["QMM_ERR_RANGE"]
    # top-k + operand: bf16 rows only, f16 / MXFP8 operands, rows up to 4096 values (MXFP8: whole 32-blocks)
    f1 = ctypes.c_float(1)
    assert lib.qmm_moe_topk_operand(fake, 4, 32, 4, 1, 1, f1, n, fake, fake, 2048, fake, 0, 1, fake, fake,
                                    n) == st["QMM_ERR_DTYPE"]
    assert lib.qmm_moe_topk_operand(fake, 4, 32, 4, 1, 1, f1, n, fake, fake, 2048, fake, 2, 2, fake, fake,
                                    n) == st["QMM_ERR_DTYPE"]
    assert lib.qmm_moe_topk_operand(fake, 4, 32, 4, 1, 1, f1, n, fake, fake, 8192, fake, 2, 1, fake, fake,
                                    n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_moe_topk_operand(fake, 4, 32, 4, 1, 1, f1, n, fake, fake, 2056, fake, 2, 3, fake, fake,
                                    n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_moe_topk_operand(fake, 4, 32, 4, 1, 1, f1, n, fake, fake, 2048, fake, 2, 1, fake, n,
                                    n) == st["QMM_ERR_NULL"]
    # bucket: too few tiles for the worst case T*KU/64 + E
    assert lib.qmm_moe_bucket(256, 4, 32, 47, n, fake, fake, fake, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_moe_bucket(256, 4, 300, 500, n, fake, fake, fake, fake, n) == st["QMM_ERR_RANGE"]
    # combine and expert matvecs
    assert lib.qmm_moe_combine(4, 2, 8, 4, fake, n, fake, 0, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_moe_expert_mv(1, 2, 0, 0, 256, 8, 4, 2, 4, fake, fake, 0, fake, fake, n, n, fake, n) \
        == st["QMM_ERR_RANGE"]
    assert lib.qmm_moe_expert_mv(3, 0, 0, 0, 64, 8, 4, 2, 4, fake, fake, 0, fake, fake, n, n, fake, n) \
        == st["QMM_ERR_FORMAT"]
    # listed-rows row scale: no list, K not a multiple of 8
    assert lib.qmm_row_scale_f16_rows(4, n, 256, fake, 0, fake, fake, n) == st["QMM_ERR_NULL"]
    assert lib.qmm_row_scale_f16_rows(4, fake, 100, fake, 0, fake, fake, n) == st["QMM_ERR_SHAPE"]
    # routing + gate/up matvecs: E past 256, the gating-1 bias, a tiled layout, K, dtype
    assert lib.qmm_moe_topk_expert_mv(fake, 1, 300, 4, 1, 1, f1, n, fake, fake, 1, 0, 0, 256, 8, fake, 2, fake, n, fake,
                                      n, n, n, fake, n) == st["QMM_ERR_RANGE"]
    assert lib.qmm_moe_topk_expert_mv(fake, 1, 32, 4, 1, 1, f1, fake, fake, fake, 1, 0, 0, 256, 8, fake, 2, fake, n,
                                      fake, n, n, n, fake, n) == st["QMM_ERR_RANGE"]
    assert lib.qmm_moe_topk_expert_mv(fake, 1, 32, 4, 1, 1, f1, n, fake, fake, 5, 0, 0, 256, 8, fake, 2, fake, n, fake,
                                      n, n, n, fake, n) == st["QMM_ERR_FORMAT"]
    assert lib.qmm_moe_topk_expert_mv(fake, 1, 32, 4, 1, 1, f1, n, fake, fake, 1, 0, 0, 100, 8, fake, 2, fake, n, fake,
                                      n, n, n, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_moe_topk_expert_mv(fake, 1, 32, 4, 1, 1, f1, n, fake, fake, 1, 0, 0, 256, 8, fake, 1, fake, n, fake,
                                      n, n, n, fake, n) == st["QMM_ERR_DTYPE"]
    # fused down matvecs + combine: tiled Q4_K, MXFP4 tiles of whole 32-row blocks and 64-value chunks with their
    # scale groups, KU above 8, null weights, split planes without scales, K, dtype
    assert lib.qmm_moe_expert_mv_combine(5, 256, 32, 4, 2, 1, fake, fake, fake, 0, fake, fake, n, 0, n, fake, n) \
        == st["QMM_ERR_FORMAT"]
    assert lib.qmm_moe_expert_mv_combine(4, 256, 8, 4, 2, 1, fake, fake, fake, 0, fake, fake, n, 0, n, fake, n) \
        == st["QMM_ERR_SHAPE"]
    assert lib.qmm_moe_expert_mv_combine(4, 96, 32, 4, 2, 1, fake, fake, fake, 0, fake, fake, n, 0, n, fake, n) \
        == st["QMM_ERR_SHAPE"]
    assert lib.qmm_moe_expert_mv_combine(4, 256, 32, 4, 2, 1, fake, fake, fake, 0, fake, n, n, 0, n, fake, n) \
        == st["QMM_ERR_NULL"]
    # decode expert matvecs on tiled MXFP4 planes: mode, whole row blocks / chunks, scale planes, unfused up, assignments
    assert lib.qmm_moe_expert_mv_tiled(2, 1, 0, 256, 32, 4, 2, 2, fake, fake, 0, fake, fake, n, n, n, n, fake,
                                       n) == st["QMM_ERR_RANGE"]
    assert lib.qmm_moe_expert_mv_tiled(0, 1, 0, 256, 48, 4, 2, 2, fake, fake, 0, fake, fake, n, n, n, n, fake,
                                       n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_moe_expert_mv_tiled(0, 1, 0, 160, 32, 4, 2, 2, fake, fake, 0, fake, fake, n, n, n, n, fake,
                                       n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_moe_expert_mv_tiled(1, 0, 0, 256, 32, 4, 2, 2, fake, fake, 0, fake, n, n, n, n, n, fake,
                                       n) == st["QMM_ERR_NULL"]
    assert lib.qmm_moe_expert_mv_tiled(0, 0, 0, 256, 32, 4, 2, 2, fake, fake, 0, fake, fake, n, n, n, n, fake,
                                       n) == st["QMM_ERR_NULL"]
    assert lib.qmm_moe_expert_mv_tiled(0, 1, 0, 256, 32, 4, 2, 3, fake, fake, 0, fake, fake, n, n, n, n, fake,
                                       n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_moe_expert_mv_tiled(0, 1, 0, 256, 32, 4, 2, 2, fake, fake, 1, fake, fake, n, n, n, n, fake,
                                       n) == st["QMM_ERR_DTYPE"]
    assert lib.qmm_moe_expert_mv_combine(1, 256, 8, 4, 9, 1, fake, fake, fake, 0, fake, n, n, 0, n, fake, n) \
        == st["QMM_ERR_RANGE"]
    assert lib.qmm_moe_expert_mv_combine(1, 256, 8, 4, 2, 1, fake, n, fake, 0, fake, n, n, 0, n, fake, n) \
        == st["QMM_ERR_NULL"]
    assert lib.qmm_moe_expert_mv_combine(3, 64, 8, 4, 2, 1, fake, fake, fake, 0, fake, n, n, 0, n, fake, n) \
        == st["QMM_ERR_NULL"]
    assert lib.qmm_moe_expert_mv_combine(1, 100, 8, 4, 2, 1, fake, fake, fake, 0, fake, n, n, 0, n, fake, n) \
        == st["QMM_ERR_SHAPE"]
    assert lib.qmm_moe_expert_mv_combine(1, 256, 8, 4, 2, 70000, fake, fake, fake, 0, fake, n, n, 0, n, fake, n) \
        == st["QMM_ERR_SHAPE"]
    assert lib.qmm_moe_expert_mv_combine(1, 256, 8, 4, 2, 1, fake, fake, fake, 1, fake, n, n, 0, n, fake, n) \
        == st["QMM_ERR_DTYPE"]
    # quantizer / repack shapes
    assert lib.qmm_quant_mxfp8(4, 48, fake, 0, n, fake, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_repack_mxfp4(fake, 4, 48, fake, fake, n) == st["QMM_ERR_SHAPE"]
    # MFMA-tiled planes: whole 32-row blocks and 64-value chunks; no GEMV or decode matvec reads them
    assert lib.qmm_tile_mxfp4(fake, fake, 48, 64, fake, fake, n) == st["QMM_ERR_SHAPE"]
    # tiled Q4_K: whole 16-row blocks and super-blocks (the GEMV: 512-value slices, at most 4 a wave of at most 8
    # waves); the grouped GEMMs read it up to K = 4096
    assert lib.qmm_tile_q4k(fake, 24, 512, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_tile_q4k(fake, 16, 640, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_tile_q4k(fake, 16, 512, n, n) == st["QMM_ERR_NULL"]
    assert lib.qmm_mv_q8(5, 4096, 24, 1, 0, fake, 2, fake, fake, n) == st["QMM_ERR_SHAPE"]     # n % 16
    assert lib.qmm_mv_q8(5, 768, 16, 1, 0, fake, 2, fake, fake, n) == st["QMM_ERR_SHAPE"]      # K % 512
    assert lib.qmm_mv_q8(5, 512 * 37, 16, 1, 0, fake, 2, fake, fake, n) == st["QMM_ERR_SHAPE"]  # 37 slices
    assert lib.qmm_dequant(5, fake, n, 16, 640, fake, n) == st["QMM_ERR_SHAPE"]
    # the prefill GEMM on tiled Q4_K: whole 16-row blocks and 512-value units; no QMM_GATE_UP pair with a tiled gate
    assert lib.qmm_gemm(5, 0, 64, 4096, 24, fake, 1, n, fake, n, fake, 0, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_gemm(5, 0, 64, 768, 32, fake, 1, n, fake, n, fake, 0, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_gemm(5 | (7 << 8), 2, 64, 4096, 32, fake, 1, n, fake, fake, fake, 0, n) == st["QMM_ERR_FORMAT"]
    # tiled Q4_0: whole 16-row blocks and 512-value units only
    assert lib.qmm_tile_q40(fake, 24, 512, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_tile_q40(fake, 16, 768, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_tile_q40(fake, 16, 512, n, n) == st["QMM_ERR_NULL"]
    assert lib.qmm_mv_q8(7, 4096, 24, 1, 0, fake, 2, fake, fake, n) == st["QMM_ERR_SHAPE"]     # n % 16
    assert lib.qmm_mv_q8(7, 768, 16, 1, 0, fake, 2, fake, fake, n) == st["QMM_ERR_SHAPE"]      # K % 512
    assert lib.qmm_dequant(7, fake, n, 16, 768, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_row_bytes(7, 4096) == 4096 // 32 * 18 and lib.qmm_row_bytes(7, 768) == 0
    # the tiled Q4_0 f32-activation matvec: 16-row blocks, K % 512, x f32 / bf16
    assert lib.qmm_mv(7, 4096, 24, 1, 0, fake, 0, fake, n, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_mv(7, 4000, 16, 1, 0, fake, 0, fake, n, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_mv(7, 4096, 16, 1, 0, fake, 4, fake, n, fake, n) == st["QMM_ERR_DTYPE"]
    assert lib.qmm_mv(7, 4096, 16, 1, 0, fake, 0, n, n, fake, n) == st["QMM_ERR_NULL"]
    assert lib.qmm_tile_mxfp4(fake, fake, 32, 96, fake, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_tile_mxfp4(fake, n, 32, 64, fake, fake, n) == st["QMM_ERR_NULL"]
    assert lib.qmm_dequant(4, fake, fake, 48, 64, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_mv(4, 64, 4, 1, 0, fake, 0, fake, fake, fake, n) == st["QMM_ERR_FORMAT"]
    # grouped GEMMs, the reference's launch order (max_rows, k, n, xrows, ...) after the name fields (fmt, mode,
    # fused, act, E, KU)
    assert lib.qmm_moe_grouped(4, 0, 1, 0, 4, 2, 256, 128, 48, 8, fake, fake, fake, 3, fake, fake, fake, n, n,
                               n, n, fake, n) == st["QMM_ERR_SHAPE"]          # n % 32 != 0
    assert lib.qmm_moe_grouped(4, 0, 1, 0, 4, 2, 256, 128, 64, 8, fake, fake, fake, 3, fake, fake, fake, n, n,
                               odd, n, fake, n) == st["QMM_ERR_ALIGN"]         # biases are f32
    assert lib.qmm_moe_grouped(4, 0, 1, 0, 4, 2, 250, 128, 64, 8, fake, fake, fake, 3, fake, fake, fake, n, n,
                               n, n, fake, n) == st["QMM_ERR_SHAPE"]          # max_rows: whole 64-row tiles
    assert lib.qmm_moe_grouped(0, 1, 0, 0, 4, 2, 256, 128, 64, 256, fake, fake, fake, 1, fake, fake, n, n, n,
                               n, n, fake, n) == st["QMM_ERR_SHAPE"]          # Q4_0 experts: K % 256
    assert lib.qmm_moe_grouped(0, 1, 0, 0, 4, 2, 256, 256, 64, 128, fake, fake, fake, 1, fake, fake, n, n, n,
                               n, n, fake, n) == st["QMM_ERR_SHAPE"]          # down: xrows >= max_rows
    # the gate/up GEMM with MXFP8 output: MXFP4 weights only, whole 32-column blocks, both outputs
    assert lib.qmm_moe_grouped_mxfp8(1, 1, 0, 4, 2, 256, 256, 64, 8, fake, fake, fake, fake, fake, n, n, n, n, n,
                                     fake, fake, n) == st["QMM_ERR_FORMAT"]
    assert lib.qmm_moe_grouped_mxfp8(4, 1, 0, 4, 2, 256, 128, 48, 8, fake, fake, fake, fake, fake, fake, n, n, n, n,
                                     fake, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_moe_grouped_mxfp8(4, 1, 0, 4, 2, 256, 128, 64, 8, fake, fake, fake, fake, fake, fake, n, n, n, n,
                                     fake, n, n) == st["QMM_ERR_NULL"]
    # the MXFP4 dense GEMM: split / tiled planes only, K % 64, the weights' scale planes, whole 32-row tiled blocks
    assert lib.qmm_gemm_mxfp4(2, 0, 64, 256, 64, fake, fake, fake, fake, n, n, fake, 0, n) == st["QMM_ERR_FORMAT"]
    assert lib.qmm_gemm_mxfp4(3, 0, 64, 96, 64, fake, fake, fake, fake, n, n, fake, 0, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_gemm_mxfp4(3, 0, 64, 256, 64, fake, fake, fake, n, n, n, fake, 0, n) == st["QMM_ERR_NULL"]
    assert lib.qmm_gemm_mxfp4(3, 2, 64, 256, 64, fake, fake, fake, fake, fake, n, fake, 0, n) == st["QMM_ERR_NULL"]
    assert lib.qmm_gemm_mxfp4(4, 0, 64, 256, 48, fake, fake, fake, fake, n, n, fake, 0, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_gemm_mxfp4(3, 0, 64, 256, 64, fake, fake, fake, fake, n, n, fake, 1, n) == st["QMM_ERR_DTYPE"]
    # int8 two-matrix matvecs and expert matvecs
    assert lib.qmm_mv_swiglu_q8(2, 256, 16, 1, 0, fake, 4, fake, fake, fake, n) == st["QMM_ERR_FORMAT"]
    assert lib.qmm_mv_swiglu_q8(1, 256, 16, 1, 0, fake, 2, fake, fake, fake, n) == st["QMM_ERR_DTYPE"]  # GGUF: Q8 x
    assert lib.qmm_mv_swiglu_q8(5, 4096, 16, 1, 0, fake, 2, fake, n, fake, n) == st["QMM_ERR_NULL"]
    assert lib.qmm_mv_swiglu_q8(5, 4096, 24, 1, 0, fake, 2, fake, fake, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_mv_pair_q8(5, 4096, 16, 1, 0, fake, 2, fake, fake, fake, n, n) == st["QMM_ERR_NULL"]  # y2
    assert lib.qmm_mv_pair_q8(1, 256, 16, 1, 0, fake, 4, fake, odd, fake, fake, n) == st["QMM_ERR_ALIGN"]
    assert lib.qmm_moe_expert_mv_q8(2, 0, 0, 0, 256, 16, 4, 2, 4, fake, fake, fake, fake, n, n, fake, n) \
        == st["QMM_ERR_FORMAT"]
    assert lib.qmm_moe_expert_mv_q8(1, 0, 0, 0, 256, 16, 4, 2, 3, fake, fake, fake, fake, n, n, fake, n) \
        == st["QMM_ERR_SHAPE"]                                                 # gu: whole tokens of KU
    assert lib.qmm_moe_expert_mv_q8(1, 0, 0, 0, 256, 16, 4, 2, 4, fake, fake, fake, n, n, n, fake, n) \
        == st["QMM_ERR_NULL"]                                                  # gu, not fused: the up tensor
    assert lib.qmm_moe_expert_mv_q8(0, 1, 0, 0, 96, 16, 4, 2, 4, fake, fake, fake, n, n, n, fake, n) \
        == st["QMM_ERR_SHAPE"]                                                 # Q4_0: K % 64
    # the opt-in int8 matvecs of MXFP4 split planes: modes 0..2, the scale planes, planar Q8_1 input, K % 64
    mq = lib.qmm_mv_mxfp4s_q8
    assert mq(3, 256, 16, 1, 0, fake, 4, fake, fake, n, n, fake, n, n) == st["QMM_ERR_RANGE"]
    assert mq(0, 256, 16, 1, 0, fake, 4, fake, n, n, n, fake, n, n) == st["QMM_ERR_NULL"]      # ws
    assert mq(1, 256, 16, 1, 0, fake, 4, fake, fake, fake, n, fake, n, n) == st["QMM_ERR_NULL"]  # ws2
    assert mq(2, 256, 16, 1, 0, fake, 4, fake, fake, fake, fake, fake, n, n) == st["QMM_ERR_NULL"]   # y2
    assert mq(0, 256, 16, 1, 0, fake, 0, fake, fake, n, n, fake, n, n) == st["QMM_ERR_DTYPE"]
    assert mq(0, 96, 16, 1, 0, fake, 4, fake, fake, n, n, fake, n, n) == st["QMM_ERR_SHAPE"]
    assert mq(0, 256, 16, 1, 0, fake, 4, odd, fake, n, n, fake, n, n) == st["QMM_ERR_ALIGN"]
    me = lib.qmm_moe_expert_mv_mxfp4s_q8
    assert me(2, 0, 0, 256, 16, 4, 2, 4, fake, fake, fake, fake, n, n, n, n, fake, n) == st["QMM_ERR_RANGE"]
    assert me(0, 1, 0, 256, 16, 4, 2, 4, fake, fake, fake, n, n, n, n, n, fake, n) == st["QMM_ERR_NULL"]   # ws
    assert me(0, 0, 0, 256, 16, 4, 2, 4, fake, fake, fake, fake, fake, n, n, n, fake, n) == st["QMM_ERR_NULL"]
    assert me(1, 0, 0, 96, 16, 4, 2, 4, fake, fake, fake, fake, n, n, n, n, fake, n) == st["QMM_ERR_SHAPE"]
    assert me(0, 1, 0, 256, 16, 4, 2, 3, fake, fake, fake, fake, n, n, n, n, fake, n) == st["QMM_ERR_SHAPE"]
    # the prefill GEMM on Q4_0: K % 256
    assert lib.qmm_gemm(0, 0, 64, 128, 64, fake, 1, n, fake, n, fake, 0, n) == st["QMM_ERR_SHAPE"]
    # decode swiglu matvec: GGUF-layout weights only, both matrices; the GEMM's swiglu mode needs the up matrix
    assert lib.qmm_mv_swiglu(3, 256, 4, 1, 0, fake, 0, fake, fake, fake, n) == st["QMM_ERR_FORMAT"]
    assert lib.qmm_mv_swiglu(1, 256, 4, 1, 0, fake, 0, fake, n, fake, n) == st["QMM_ERR_NULL"]
    assert lib.qmm_mv_swiglu(1, 100, 4, 1, 0, fake, 0, fake, fake, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_mv_swiglu(1, 256, 4, 1, 0, fake, 0, fake, odd, fake, n) == st["QMM_ERR_ALIGN"]
    assert lib.qmm_gemm(1, 2, 64, 256, 64, fake, 1, n, fake, n, fake, 0, n) == st["QMM_ERR_NULL"]
    assert lib.qmm_row_scale_f16_live(64, n, 256, fake, 0, fake, fake, n) == st["QMM_ERR_NULL"]
    # Q6_K: K % 256, a 4-byte aligned tensor
    assert lib.qmm_mv(6, 320, 4, 1, 0, fake, 0, fake, n, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_mv(6, 256, 4, 1, 0, fake, 0, odd, n, fake, n) == st["QMM_ERR_ALIGN"]
    assert lib.qmm_mv_q8(6, 256, 4, 1, 0, fake, 4, odd, fake, n) == st["QMM_ERR_ALIGN"]
    assert lib.qmm_dequant(6, fake, n, 4, 320, fake, n) == st["QMM_ERR_SHAPE"]
    assert lib.qmm_gemm(6, 0, 64, 256, 64, fake, 1, n, odd, n, fake, 0, n) == st["QMM_ERR_ALIGN"]
    assert lib.qmm_gemm(2, 0, 64, 256, 64, fake, 1, n, fake, n, fake, 0, n) == st["QMM_ERR_FORMAT"]   # MXFP4: own entry
    # router / shared gate / wscale / gated combine
    assert lib.qmm_moe_route(4, 2882, 32, 4, 3, 0, ctypes.c_float(1), fake, 0, fake, 0, n, n, fake, fake, fake,
                             n) == st["QMM_ERR_SHAPE"]                        # H % 4
    assert lib.qmm_moe_route(4, 2880, 32, 4, 1, 0, ctypes.c_float(1), fake, 0, fake, 0, fake, n, fake, fake, fake,
                             n) == st["QMM_ERR_RANGE"]                        # gating 1 takes no bias
    assert lib.qmm_moe_route(4, 2880, 32, 4, 3, 0, ctypes.c_float(1), fake, 0, fake, 3, n, n, fake, fake, fake,
                             n) == st["QMM_ERR_DTYPE"]
    assert lib.qmm_moe_shared_gate(4, 2048, fake, 0, n, 0, fake, n) == st["QMM_ERR_NULL"]
    assert lib.qmm_moe_wscale(4, 9, 32, fake, fake, fake, n) == st["QMM_ERR_RANGE"]
    assert lib.qmm_moe_combine_gated(4, 16, 8, 4, fake, n, fake, n, fake, n) == st["QMM_ERR_NULL"]
    # an unfused gate/up without its up matrix, on every kernel path: the tiled layout and GGUF Q4_K with few rows an
    # expert (the narrow kernel), GGUF Q4_K with many (the 64-row tile), and the whole chain
    for fmt, max_rows in ((5, 256), (1, 256), (1, 64 * 40)):
        assert lib.qmm_moe_grouped(fmt, 0, 0, 0, 4, 2, max_rows, 2048, 768, 64, fake, fake, fake, 1, fake, fake, n,
                                   n, n, n, n, fake, n) == st["QMM_ERR_NULL"], (fmt, max_rows)
    assert lib.qmm_moe_grouped_mxfp8(4, 0, 0, 4, 2, 256, 128, 64, 8, fake, fake, fake, fake, fake, fake, n, n, n, n,
                                     fake, fake, n) == st["QMM_ERR_NULL"]
    for T in (4, 64):   # decode and prefill chains
        assert lib.qmm_moe_routed(1, -1, 0, 0, 1, 1, f1, 0, 128, 8, T, 2048, 768, fake, 2, fake, n, 0, n, n, fake, n,
                                  n, n, fake, n, n, n, n, n, 0, fake, fake, 1 << 30, n) == st["QMM_ERR_NULL"], T
    # the prefill GEMM's weight rows are addressed by 32-bit buffer offsets: 2 GiB of weights at most
    assert lib.qmm_gemm(1, 0, 64, 1 << 20, 1 << 14, fake, 1, n, fake, n, fake, 0, n) == st["QMM_ERR_SHAPE"]


def test_gate_up_format_pairs(lib):
    """QMM_GATE_UP(gate, up) as the header defines it, the Python code for "gate+up", and the entry points' checks:
    a pair is the format of a gate/up call only (swiglu GEMM, gate/up expert matvecs and grouped GEMM, two tensors,
    f32 / bf16 decode activations in the chain)."""
    from qmm.formats import CODE
    text = open(HEADER).read()
    assert "#define QMM_GATE_UP(gate, up) ((gate) | (((up) + 1) << 8))" in text
    assert CODE["q4_k+q6_k"] == 1 | (7 << 8) and CODE["q6_k+q4_k"] == 6 | (2 << 8)
    st = header_enum("qmm_status")
    fake, n, f1 = ctypes.c_void_p(0x1000), None, ctypes.c_float(1)
    pair = CODE["q4_k+q6_k"]
    # the GEMM: swiglu only; formats of the f16 MFMA kernels only
    assert lib.qmm_gemm(pair, 0, 64, 256, 64, fake, 1, n, fake, n, fake, 0, n) == st["QMM_ERR_FORMAT"]
    assert lib.qmm_gemm(CODE["q4_k+mxfp4"], 2, 64, 256, 64, fake, 1, n, fake, fake, fake, 0, n) == st["QMM_ERR_FORMAT"]
    assert lib.qmm_gemm(pair, 2, 64, 256, 64, fake, 1, n, fake, n, fake, 0, n) == st["QMM_ERR_NULL"]
    # the grouped GEMM: gate/up of two tensors
    assert lib.qmm_moe_grouped(pair, 1, 0, 0, 4, 2, 256, 256, 64, 256, fake, fake, fake, 1, fake, fake, n, n, n,
                               n, n, fake, n) == st["QMM_ERR_FORMAT"]
    assert lib.qmm_moe_grouped(pair, 0, 1, 0, 4, 2, 256, 256, 64, 8, fake, fake, fake, 1, fake, fake, n, fake, n,
                               n, n, fake, n) == st["QMM_ERR_FORMAT"]
    # the expert matvecs: gate/up of two tensors; the fused routing launch and the down + combine take one format
    assert lib.qmm_moe_expert_mv(pair, 1, 0, 0, 256, 8, 4, 2, 4, fake, fake, 0, fake, fake, n, n, fake, n) \
        == st["QMM_ERR_FORMAT"]
    assert lib.qmm_moe_expert_mv(pair, 0, 1, 0, 256, 8, 4, 2, 4, fake, fake, 0, fake, fake, n, n, fake, n) \
        == st["QMM_ERR_FORMAT"]
    assert lib.qmm_moe_expert_mv(pair, 0, 0, 0, 256, 8, 4, 2, 4, fake, fake, 0, fake, n, n, n, fake, n) \
        == st["QMM_ERR_NULL"]
    assert lib.qmm_moe_topk_expert_mv(fake, 1, 32, 4, 1, 1, f1, n, fake, fake, pair, 0, 0, 256, 8, fake, 2, fake, n,
                                      fake, n, n, n, fake, n) == st["QMM_ERR_FORMAT"]
    assert lib.qmm_mv_swiglu(CODE["q4_k+mxfp4s"], 256, 4, 1, 0, fake, 0, fake, fake, fake, n) == st["QMM_ERR_FORMAT"]
    # the chain: f32 / bf16 decode activations, two tensors; the workspace of a pair is its gate format's
    size = lib.qmm_moe_routed_workspace_size
    assert size(pair, 0, 128, 8, 4, 2048, 768, 0) == size(1, 0, 128, 8, 4, 2048, 768, 0) > 0
    assert size(pair, 1, 128, 8, 4, 2048, 768, 0) == -1
    assert lib.qmm_moe_routed(pair, -1, 1, 0, 1, 1, f1, 0, 128, 8, 4, 2048, 768, fake, 2, fake, n, 0, n, n, fake, n,
                              fake, n, fake, n, n, n, n, n, 0, fake, fake, 1 << 30, n) == st["QMM_ERR_FORMAT"]


def test_static_chain_scratch_bounds(lib):
    """qmm_moe_routed_static's 16 MiB array holds the decode chain of an H + FE <= 8192, top-8 model on given logits
    at up to 63 tokens on f32 / bf16 activations and up to 48 on the Q8_1 path (the bounds its header states), and
    the bound is tight where the header says the Q8_1 buffers take the rest."""
    lim = 16 << 20
    size = lib.qmm_moe_routed_workspace_size
    for H in range(256, 8192, 256):
        assert 0 < size(1, 0, 256, 8, 63, H, 8192 - H, 0) <= lim, H
        assert 0 < size(1, 1, 256, 8, 48, H, 8192 - H, 0) <= lim, H
    assert size(1, 1, 128, 8, 55, 4096, 4096, 0) > lim
    assert size(1, 0, 128, 8, 64, 4096, 4096, 0) > lim   # 64 tokens: the prefill chain


def test_python_surface_refuses_host_tensors():
    torch = pytest.importorskip("torch")
    from qmm import ops
    with pytest.raises(ValueError):
        ops.mv("q4_k", torch.zeros(144, dtype=torch.uint8), torch.zeros((1, 256)), 1, 256)


def test_decode_int8_defaults_follow_the_reference():
    """The decode matvecs take int8 activations by default for the reference's ICODES formats (Q4_K, Q6_K; Q4_0 and
    MXFP4 split planes only with their Q4_0_Q8=1 / MXFP4S_Q8=1 switches, S/formats.py:20-30), the tiled layouts with
    their format, the tiled Q4_0 always."""
    import importlib
    import os
    from qmm import formats
    assert formats.decode_q8("q4_k") and formats.decode_q8("q6_k") and formats.decode_q8("q4_kt")
    assert formats.decode_q8("q4_0t")
    for fmt, switch in (("q4_0", "Q4_0_Q8"), ("mxfp4s", "MXFP4S_Q8")):   # the reference's opt-in switches
        old = os.environ.pop(switch, None)
        try:
            assert not importlib.reload(formats).decode_q8(fmt)
            os.environ[switch] = "1"
            assert importlib.reload(formats).decode_q8(fmt)
            os.environ[switch] = "off"
            assert not importlib.reload(formats).decode_q8(fmt)
        finally:
            os.environ.pop(switch, None)
            if old is not None:
                os.environ[switch] = old
            importlib.reload(formats)
    assert not formats.decode_q8("mxfp4")
