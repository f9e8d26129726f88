"""Weight formats of the quantized matmul path: bytes per block, values per block and the C-ABI format codes.

Mirrors the reference's format table (skills/loom-port-llm/starter/formats.py:5-19, FMT / SB / SPLIT / SCALE_DIV)
for the formats this library decodes. The integer codes are this library's own (include/qmm.h, enum qmm_format).
"""
import os

# mxfp4t: MXFP4 in MFMA-tiled planes (this library's load-time layout for the grouped GEMM, qmm_tile_mxfp4)
# q4_kt / q4_0t: Q4_K / Q4_0 in the lane-ordered tiled layout of the int8-activation decode GEMV (qmm_tile_q4k /
# qmm_tile_q40; a q4_0t "block" is one row's 512 values of a tile unit)
FMT = {"q4_0": 18, "q4_k": 144, "mxfp4": 17, "mxfp4s": 16, "mxfp4t": 16, "q4_kt": 144, "q6_k": 210,
       "q4_0t": 288}   # bytes per block
SB = {"q4_0": 32, "q4_k": 256, "mxfp4": 32, "mxfp4s": 32, "mxfp4t": 32, "q4_kt": 256, "q6_k": 256,
      "q4_0t": 512}    # values per block
SPLIT = frozenset({"mxfp4s", "mxfp4t"})                         # weight plane + scale plane (two operands)
SCALE_DIV = {"mxfp4s": 16}                                      # nibble-plane bytes per scale-plane byte

class _Codes(dict):
    """enum qmm_format; a key "gate+up" (the reference's GATE+UP notation for gate and up matrices in two formats,
    S/gen_moe.py:535-552) gives QMM_GATE_UP(gate, up) = gate | (up + 1) << 8."""

    def __missing__(self, key):
        if isinstance(key, str) and key.count("+") == 1:
            g, u = key.split("+")
            return self[g] | ((self[u] + 1) << 8)
        raise KeyError(key)


CODE = _Codes({"q4_0": 0, "q4_k": 1, "mxfp4": 2, "mxfp4s": 3, "mxfp4t": 4, "q4_kt": 5, "q6_k": 6,
               "q4_0t": 7})   # enum qmm_format


def gate_format(fmt):
    """The gate matrix's format of a "gate+up" pair (the format itself otherwise)."""
    return fmt.split("+")[0]
DTYPE = {"f32": 0, "f16": 1, "bf16": 2, "mxfp8": 3, "q8": 4}    # enum qmm_dtype
MX_BLOCK = 32                                                   # values per E8M0 scale of an MXFP8 operand
GEMM_MODE = {"store": 0, "acc": 1, "swiglu": 2}                 # enum qmm_gemm_mode
ACT = {"silu": 0, "swiglu_oai": 1}                              # enum qmm_act
GATING = {"softmax": 1, "sigmoid": 2, "softmax_weight": 3}      # llama.cpp expert_gating_func values


def row_bytes(fmt, k):
    """Bytes of one row of K values (S/gen_llm.py:182-183); for mxfp4s the nibble plane's bytes."""
    if k % SB[fmt]:
        raise ValueError(f"{fmt}: K={k} is not a multiple of {SB[fmt]}")
    return k // SB[fmt] * FMT[fmt]


def scale_row_bytes(fmt, k):
    """Bytes of one row of a split format's scale plane: K/32 E8M0 bytes (mxfp4s), or the tiled plane's share of a
    32-row block, 8 bytes per started group of four 64-value chunks (mxfp4t)."""
    if fmt == "mxfp4t":
        return (k // 64 + 3) // 4 * 8
    return row_bytes(fmt, k) // SCALE_DIV[fmt] if fmt in SPLIT else 0


def _opt_in(name):
    return os.environ.get(name, "0").strip().lower() not in ("", "0", "false", "no", "off")


# The formats whose decode takes int8 (Q8_1) activations by default: the reference's formats.ICODES (S/formats.py:20-30)
# restricted to the formats here. Q4_K and Q6_K always; Q4_0 only with Q4_0_Q8=1 and MXFP4 split planes only with
# MXFP4S_Q8=1, the reference's own opt-in switches (llama.cpp's vec_dot_q4_0_q8_1 arithmetic; @g_mxfp4s_icodes); the
# tiled layouts follow their format, except that the tiled Q4_0 layout has no other decode kernel than the int8 one.
ICODES = frozenset({"q4_k", "q6_k"} | ({"q4_0"} if _opt_in("Q4_0_Q8") else set())
                   | ({"mxfp4s"} if _opt_in("MXFP4S_Q8") else set()))


def decode_q8(fmt):
    """Whether the decode matvecs of weight format `fmt` take int8 activations by default (see ICODES)."""
    return fmt in ICODES or fmt == "q4_kt" or fmt == "q4_0t"
