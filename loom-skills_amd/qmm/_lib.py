"""ctypes binding of libqmm.so (include/qmm.h). Loading fails loudly when the library is missing: there is no
fallback implementation."""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("QMM_LIB", os.path.join(HERE, "libqmm.so"))   # QMM_LIB: another build of the library

c_i64, c_int, c_float, c_vp = ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_void_p

# name -> argument types (every entry returns int status unless listed in RESTYPE)
SIGNATURES = {
    "qmm_version": [],
    "qmm_strerror": [c_int],
    "qmm_row_bytes": [c_int, c_i64],
    "qmm_dequant": [c_int, c_vp, c_vp, c_i64, c_i64, c_vp, c_vp],
    "qmm_mv": [c_int, c_i64, c_i64, c_i64, c_int, c_vp, c_int, c_vp, c_vp, c_vp, c_vp],
    "qmm_mv_swiglu": [c_int, c_i64, c_i64, c_i64, c_int, c_vp, c_int, c_vp, c_vp, c_vp, c_vp],
    "qmm_quant_q8": [c_i64, c_i64, c_vp, c_int, c_vp, c_vp],
    "qmm_mv_q8": [c_int, c_i64, c_i64, c_i64, c_int, c_vp, c_int, c_vp, c_vp, c_vp],
    "qmm_gemm": [c_int, c_int, c_i64, c_i64, c_i64, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_int, c_vp],
    "qmm_moe_topk": [c_vp, c_i64, c_int, c_int, c_int, c_int, c_float, c_vp, c_vp, c_vp, c_vp],
    "qmm_moe_topk_operand": [c_vp, c_i64, c_int, c_int, c_int, c_int, c_float, c_vp, c_vp, c_vp, c_i64, c_vp, c_int,
                             c_int, c_vp, c_vp, c_vp],
    "qmm_moe_bucket": [c_i64, c_int, c_int, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp],
    "qmm_moe_expert_mv": [c_int, c_int, c_int, c_int, c_i64, c_i64, c_int, c_int, c_i64, c_vp, c_vp, c_int, c_vp,
                          c_vp, c_vp, c_vp, c_vp, c_vp],
    "qmm_moe_expert_mv_split": [c_int, c_int, c_int, c_i64, c_i64, c_int, c_int, c_i64, c_vp, c_vp, c_int, c_vp,
                                c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp],
    "qmm_moe_expert_mv_tiled": [c_int, c_int, c_int, c_i64, c_i64, c_int, c_int, c_i64, c_vp, c_vp, c_int, c_vp,
                                c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp],
    "qmm_moe_grouped": [c_int, c_int, c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_int,
                        c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp],
    "qmm_moe_grouped_mxfp8": [c_int, c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp,
                              c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp],
    "qmm_gemm_mxfp4": [c_int, c_int, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_vp],
    "qmm_mv_swiglu_q8": [c_int, c_i64, c_i64, c_i64, c_int, c_vp, c_int, c_vp, c_vp, c_vp, c_vp],
    "qmm_mv_pair_q8": [c_int, c_i64, c_i64, c_i64, c_int, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp],
    "qmm_mv_mxfp4s_q8": [c_int, c_i64, c_i64, c_i64, c_int, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp],
    "qmm_moe_expert_mv_mxfp4s_q8": [c_int, c_int, c_int, c_i64, c_i64, c_int, c_int, c_i64, c_vp, c_vp, c_vp, c_vp,
                                    c_vp, c_vp, c_vp, c_vp, c_vp, c_vp],
    "qmm_moe_expert_mv_q8": [c_int, c_int, c_int, c_int, c_i64, c_i64, c_int, c_int, c_i64, c_vp, c_vp, c_vp, c_vp,
                             c_vp, c_vp, c_vp, c_vp],
    "qmm_moe_route": [c_i64, c_i64, c_int, c_int, c_int, c_int, c_float, c_vp, c_int, c_vp, c_int, c_vp, c_vp, c_vp,
                      c_vp, c_vp, c_vp],
    "qmm_moe_shared_gate": [c_i64, c_i64, c_vp, c_int, c_vp, c_int, c_vp, c_vp],
    "qmm_moe_wscale": [c_i64, c_int, c_int, c_vp, c_vp, c_vp, c_vp],
    "qmm_moe_combine_gated": [c_i64, c_i64, c_i64, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp],
    "qmm_row_scale_f16": [c_i64, c_i64, c_vp, c_int, c_vp, c_vp, c_vp, c_vp],
    "qmm_row_scale_f16_rows": [c_i64, c_vp, c_i64, c_vp, c_int, c_vp, c_vp, c_vp],
    "qmm_row_scale_f16_live": [c_i64, c_vp, c_i64, c_vp, c_int, c_vp, c_vp, c_vp],
    "qmm_quant_mxfp8": [c_i64, c_i64, c_vp, c_int, c_vp, c_vp, c_vp, c_vp],
    "qmm_repack_mxfp4": [c_vp, c_i64, c_i64, c_vp, c_vp, c_vp],
    "qmm_tile_mxfp4": [c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp],
    "qmm_tile_q4k": [c_vp, c_i64, c_i64, c_vp, c_vp],
    "qmm_tile_q40": [c_vp, c_i64, c_i64, c_vp, c_vp],
    "qmm_mxfp4t_scale_bytes": [c_i64, c_i64],
    "qmm_moe_combine": [c_i64, c_i64, c_i64, c_int, c_vp, c_vp, c_vp, c_int, c_vp, c_vp],
    "qmm_moe_topk_expert_mv": [c_vp, c_i64, c_int, c_int, c_int, c_int, c_float, c_vp, c_vp, c_vp, c_int, c_int, c_int,
                               c_i64, c_i64, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp],
    "qmm_moe_expert_mv_combine": [c_int, c_i64, c_i64, c_int, c_int, c_i64, c_vp, c_vp, c_vp, c_int, c_vp, c_vp, c_vp,
                                  c_int, c_vp, c_vp, c_vp],
    "qmm_moe_routed": [c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_i64, c_i64, c_i64,
                       c_vp, c_int, c_vp, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                       c_vp, c_vp, c_int, c_vp, c_vp, c_i64, c_vp],
    "qmm_moe_routed_workspace_size": [c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64, c_int],
    "qmm_moe_routed_static": [c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_i64, c_i64,
                              c_i64, c_vp, c_int, c_vp, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                              c_vp, c_vp, c_vp, c_vp, c_int, c_vp, c_vp],
}
RESTYPE = {"qmm_strerror": ctypes.c_char_p, "qmm_row_bytes": c_i64, "qmm_mxfp4t_scale_bytes": c_i64,
           "qmm_moe_routed_workspace_size": c_i64}


class QmmError(RuntimeError):
    def __init__(self, name, status, text):
        super().__init__(f"{name} failed: {text} ({status})")
        self.status = status


_LIB = None


def load(path=LIB_PATH):
    """The loaded library (cached). Raises OSError when libqmm.so has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(path):
            raise OSError(f"{path} is missing: build it with `python loom-skills_amd/qmm/build.py`")
        lib = ctypes.CDLL(path)
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = RESTYPE.get(name, c_int)
        _LIB = lib
    return _LIB


def call(name, *args):
    """Calls an entry point and raises QmmError on a nonzero status."""
    lib = load()
    st = getattr(lib, name)(*args)
    if st != 0:
        raise QmmError(name, st, lib.qmm_strerror(st).decode())
    return st
