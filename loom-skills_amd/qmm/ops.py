"""Op surface of the quantized matmul path: torch device tensors in, HIP kernels of libqmm.so underneath.

The functions mirror the reference's kernel families (paths relative to the reference root,
S/ = skills/loom-port-llm/starter/):

    mv                g_mv_{fmt}_k{K}[_t{TG}][_r{R}]          S/gen_llm.py:1159-1378, launch args :1187-1197
    mv_q8             g_mv_{fmt}_k{K}[_t{TG}]_q8[_r{R}]       S/gen_llm.py:1288-1301 (int8 activations)
    mv_swiglu_q8      g_mv_{fmt}_k{K}_swiglu[_t{TG}]_q8       S/gen_llm.py:1159-1197
    mv_pair_q8        g_mv_{fmt}_k{K}_pair[_t{TG}]_q8         S/gen_llm.py:1166-1176
    gemm              g_gemm_{fmt}_{store|acc|swiglu}[_m*]    S/gen_gemm.py:535-703, launch args :549-556
    gemm_mxfp4        g_gemm_mxfp4s_{store|swiglu}_f8_m256    S/gen_mxfp4s.py:50-101
    moe_topk          g_moe_route / g_moe_route_tr            S/gen_moe.py:116-500
    moe_route         the same with the router matvec         S/gen_moe.py:116-500 (+ _live, :474-500)
    moe_shared_gate   g_moe_shared_gate                       S/gen_moe.py:780-823
    moe_wscale        g_moe_wscale                            S/gen_moe.py:1010-1045
    moe_bucket        g_moe_bucket                            S/gen_moe.py:829-955
    moe_expert_mv     g_moe_gu_* / g_moe_dn_*                 S/gen_moe.py:535-727
    moe_expert_mv_q8  g_moe_gu_*_q8_* / g_moe_dn_*_q8_*       S/gen_moe.py:535-727 (MOE_Q8, S/gen_llm.py:5290-5303)
    moe_topk_expert_mv     g_moe_route + g_moe_gu_* in one       S/gen_moe.py:116-727 (the decode chain's first two)
    moe_expert_mv_combine  g_moe_dn_* + g_moe_combine in one    S/gen_moe.py:535-762 (the decode chain's last two)
    moe_grouped       g_moe_ggu_* / g_moe_gdn_*               S/gen_moe.py:1126-1228
    moe_combine       g_moe_combine[_sorted] [shared_gated]   S/gen_moe.py:730-779, :1231-1280
    moe_prefill       the prefill chain of moe_routed          S/gen_llm.py:5324-5385 (t >= 64)
    moe_decode        the decode chain of moe_routed           S/gen_llm.py:5324-5385 (t < 64)
    moe_chain         moe_routed in one library call            qmm_moe_routed, S/gen_llm.py:5324-5432
    moe_layer         shared experts + routed experts          moe_layer, S/gen_llm.py:5306-5321
    row_scale_f16     g_row_scale_f16[_tiles]                 S/gen_llm.py:1843-1915, S/gen_moe.py:503-527
    dequant           the @g_<fmt>_values helpers (bit-exact f32 values)

plus the gfx950-specific producers ``quant_mxfp8`` (A operand of the scaled MFMA), ``repack_mxfp4`` (GGUF
MXFP4 blocks to split planes) and ``tile_mxfp4`` (split planes to the MFMA-tiled planes the grouped GEMM streams
fastest), the last two one-time weight preparations.

Every function validates its arguments on the host (the C ABI returns a status that becomes ``QmmError``) and
launches asynchronously on torch's current stream. Weights are uint8 tensors holding the raw GGUF block bytes.
"""
import weakref

import torch

from . import _lib
from .formats import ACT, CODE, DTYPE, GEMM_MODE, ICODES, MX_BLOCK, SPLIT, decode_q8, gate_format, row_bytes

TILE = 64


def _dt(t):
    if t.dtype == torch.float32:
        return DTYPE["f32"]
    if t.dtype == torch.bfloat16:
        return DTYPE["bf16"]
    if t.dtype == torch.float16:
        return DTYPE["f16"]
    raise TypeError(f"unsupported activation dtype {t.dtype}")


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _dev(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("qmm ops take device tensors")
        if t is not None and not t.is_contiguous():
            raise ValueError("qmm ops take contiguous tensors")


def _out(y, shape, dtype, dev, accumulate=False):
    """The output tensor: a new one, or y checked against the shape and dtype the kernel writes (the C ABI cannot see
    sizes, so a wrong y would be written out of bounds). Accumulating needs the caller's y."""
    if y is None:
        if accumulate:
            raise ValueError("accumulating into y needs y")
        return torch.empty(shape, dtype=dtype, device=dev)
    if tuple(y.shape) != tuple(shape) or y.dtype != dtype:
        raise ValueError(f"y is {tuple(y.shape)} {y.dtype}, the kernel writes {tuple(shape)} {dtype}")
    return y


def _cols(x, k, what="x"):
    if x.shape[-1] != k:
        raise ValueError(f"{what} has {x.shape[-1]} columns, K is {k}")


def dequant(fmt, w, rows, k, ws=None, out=None):
    """f32 [rows, k] values of the weight bytes, bit-exact to the reference's value helpers."""
    _dev(w, ws)
    out = torch.empty((rows, k), dtype=torch.float32, device=w.device) if out is None else out
    _lib.call("qmm_dequant", CODE[fmt], _ptr(w), _ptr(ws), rows, k, _ptr(out), _stream())
    return out


def mv(fmt, w, x, n, k, y=None, accumulate=False, ws=None):
    """y[t, r] (+)= sum_k x[t, k] W[r, k]; x f32 or bf16 [tokens, k]; returns y f32 [tokens, n]."""
    _dev(w, x, y, ws)
    tokens = x.shape[0]
    _cols(x, k)
    y = _out(y, (tokens, n), torch.float32, x.device, accumulate)
    _lib.call("qmm_mv", CODE[fmt], k, n, tokens, int(bool(accumulate)), _ptr(x), _dt(x), _ptr(w), _ptr(ws),
              _ptr(y), _stream())
    return y


def mv_swiglu(fmt, w, w2, x, n, k, y=None, accumulate=False):
    """y[t, r] (+)= silu(x W^T) * (x W2^T) (g_mv_{fmt}_k{K}_swiglu); x f32 or bf16 [tokens, k]; y f32 [tokens, n]."""
    _dev(w, w2, x, y)
    tokens = x.shape[0]
    _cols(x, k)
    y = _out(y, (tokens, n), torch.float32, x.device, accumulate)
    _lib.call("qmm_mv_swiglu", CODE[fmt], k, n, tokens, int(bool(accumulate)), _ptr(x), _dt(x), _ptr(w), _ptr(w2),
              _ptr(y), _stream())
    return y


def q8_bytes(rows, k):
    """Bytes of the planar Q8_1 buffer of `rows` rows of k values: codes, then an f32 pair per 32 values."""
    return rows * k + rows * (k // 32) * 8


def quant_q8(x, xq=None):
    """Planar Q8_1 (g_quant_q8, S/gen_llm.py:684-749) of f32 / bf16 rows x [rows, k]: a uint8 tensor of
    q8_bytes(rows, k) bytes (int8 codes [rows, k], then f32 (f16-rounded d, code sum) per 32 values)."""
    _dev(x, xq)
    rows, k = x.shape
    xq = torch.empty(q8_bytes(rows, k), dtype=torch.uint8, device=x.device) if xq is None else xq
    _lib.call("qmm_quant_q8", rows, k, _ptr(x), _dt(x), _ptr(xq), _stream())
    return xq


def mv_q8(fmt, w, x, n, k, tokens=None, y=None, accumulate=False, ws=None):
    """The int8-activation decode matvec (g_mv_{fmt}_k{K}[_t{TG}]_q8, S/gen_llm.py:1288-1301): x is the planar Q8_1
    buffer of `tokens` rows (uint8, from quant_q8), or f32 / bf16 rows [tokens, k], which the Q4_K K = 4096 / 8192
    and (up to two tokens) tiled-layout q4_kt / q4_0t kernels quantize themselves and any other call quantizes through
    quant_q8 first (identical results). mxfp4s (the reference's opt-in MXFP4S_Q8): w the nibble plane, ws the E8M0
    plane."""
    _dev(w, ws, x, y)
    x, xd, tokens = _q8_input(fmt, x, k, tokens, staged_tokens=2)
    y = _out(y, (tokens, n), torch.float32, w.device, accumulate)
    if fmt == "mxfp4s":
        _split_q8(0, k, n, tokens, accumulate, x, xd, w, ws, None, None, y, None)
        return y
    _lib.call("qmm_mv_q8", CODE[fmt], k, n, tokens, int(bool(accumulate)), _ptr(x), xd, _ptr(w), _ptr(y), _stream())
    return y


def _split_q8(mode, k, n, tokens, accumulate, x, xd, w, ws, w2, ws2, y, y2):
    """qmm_mv_mxfp4s_q8: the int8 matvecs of MXFP4 split planes (mode 0 plain, 1 swiglu, 2 pair)."""
    if ws is None or (mode and ws2 is None):
        raise ValueError("mxfp4s weights need their E8M0 scale planes (ws / ws2)")
    _lib.call("qmm_mv_mxfp4s_q8", mode, k, n, tokens, int(bool(accumulate)), _ptr(x), xd, _ptr(w), _ptr(ws), _ptr(w2),
              _ptr(ws2), _ptr(y), _ptr(y2), _stream())


TILED_Q8 = ("q4_kt", "q4_0t")   # the tiled layouts of the int8 matvec, which quantize f32 / bf16 rows themselves


def _q8_input(fmt, x, k, tokens, staged_tokens):
    """(x, its dtype code, tokens) for an int8 matvec: a planar Q8_1 buffer as it is (uint8, `tokens` rows), or f32 /
    bf16 rows, which the Q4_K K = 4096 / 8192 and (up to `staged_tokens` tokens) tiled-layout kernels quantize
    themselves and every other call quantizes through quant_q8 first (identical results)."""
    if x.dtype == torch.uint8:
        if tokens is None:
            raise ValueError("a planar Q8_1 buffer needs its token count")
        if x.numel() < q8_bytes(tokens, k):
            raise ValueError(f"the planar Q8_1 buffer holds {x.numel()} bytes, {tokens} rows of K {k} need "
                             f"{q8_bytes(tokens, k)}")
        return x, DTYPE["q8"], tokens
    tokens = x.shape[0]
    _cols(x, k)
    # the kernels that quantize f32 / bf16 rows themselves do so in every workgroup; from three tokens on a separate
    # quant_q8 pass is cheaper for the tiled layout (same bits either way)
    if (fmt == "q4_k" and k in (4096, 8192) and staged_tokens >= 2) or (fmt in TILED_Q8 and tokens <= staged_tokens):
        return x, _dt(x), tokens
    return quant_q8(x), DTYPE["q8"], tokens


def mv_swiglu_q8(fmt, w, w2, x, n, k, tokens=None, y=None, accumulate=False, ws=None, ws2=None):
    """The int8 swiglu matvec y (+)= silu(x W^T) (x W2^T) (g_mv_{fmt}_k{K}_swiglu[_t{TG}]_q8): gate W and up W2
    [n, k]; x a planar Q8_1 buffer (with tokens) or f32 / bf16 rows (quantized as quant_q8 does). fmt q4_kt / q4_0t
    (tiled layouts), GGUF q4_k / q4_0 / q6_k, or mxfp4s with ws / ws2 the scale planes. Returns y f32 [tokens, n]."""
    _dev(w, w2, ws, ws2, x, y)
    x, xd, tokens = _q8_input(fmt, x, k, tokens, staged_tokens=2 if fmt in TILED_Q8 else 0)
    y = _out(y, (tokens, n), torch.float32, w.device, accumulate)
    if fmt == "mxfp4s":
        _split_q8(1, k, n, tokens, accumulate, x, xd, w, ws, w2, ws2, y, None)
        return y
    _lib.call("qmm_mv_swiglu_q8", CODE[fmt], k, n, tokens, int(bool(accumulate)), _ptr(x), xd, _ptr(w), _ptr(w2),
              _ptr(y), _stream())
    return y


def mv_pair_q8(fmt, w, w2, x, n, k, tokens=None, y=None, y2=None, accumulate=False, ws=None, ws2=None):
    """Two int8 matvecs of one input in one launch (g_mv_{fmt}_k{K}_pair[_t{TG}]_q8): y (+)= x W^T, y2 (+)= x W2^T,
    each equal bit for bit to the one-matrix kernel's of the same layout (mxfp4s: ws / ws2 the scale planes).
    Returns (y, y2) f32 [tokens, n]."""
    _dev(w, w2, ws, ws2, x, y, y2)
    x, xd, tokens = _q8_input(fmt, x, k, tokens, staged_tokens=2 if fmt in TILED_Q8 else 0)
    y = _out(y, (tokens, n), torch.float32, w.device, accumulate)
    y2 = _out(y2, (tokens, n), torch.float32, w.device, accumulate)
    if fmt == "mxfp4s":
        _split_q8(2, k, n, tokens, accumulate, x, xd, w, ws, w2, ws2, y, y2)
        return y, y2
    _lib.call("qmm_mv_pair_q8", CODE[fmt], k, n, tokens, int(bool(accumulate)), _ptr(x), xd, _ptr(w), _ptr(w2),
              _ptr(y), _ptr(y2), _stream())
    return y, y2


def gemm(fmt, mode, x, w, n, k, w2=None, scales=None, out_dtype=torch.float32, y=None, ws=None, ws2=None):
    """Y = (X16 W^T) inv (store), Y += ... (acc) or Y = silu(X16 W^T inv) (X16 W2^T inv) (swiglu, w2 the up matrix).
    GGUF q4_k / q6_k / q4_0: x is the row-scaled f16 operand with its scales (the reference's g_row_scale_f16
    output), or bf16 / f32 rows, which are row-scaled here first (qmm_row_scale_f16). With scales, 64-row tiles whose
    rows all have scale 0 (padding rows of row_scale_f16(x, info=...)) are skipped and their y rows are not written.
    mxfp4s / mxfp4t (ws / ws2 the weights' scale planes): see gemm_mxfp4; x is E4M3 codes with their E8M0 scales, or
    bf16 / f32 rows, quantized to MXFP8 here first."""
    if fmt in SPLIT or fmt == "mxfp4t":
        return gemm_mxfp4(fmt, mode, x, w, ws, n, k, w2=w2, ws2=ws2, x_scales=scales, out_dtype=out_dtype, y=y)
    _dev(x, w, w2, scales, y)
    if mode == "swiglu" and w2 is None:
        raise ValueError("swiglu needs the up matrix w2")
    rows = x.shape[0]
    _cols(x, k)
    if x.dtype != torch.float16:
        if scales is not None:
            raise ValueError("scales come with an f16 operand; pass bf16 / f32 rows without them")
        x, scales = row_scale_f16(x)
    elif scales is not None and tuple(scales.shape) != (rows, 2):
        raise ValueError(f"scales are {tuple(scales.shape)}, the operand has {rows} rows")
    y = _out(y, (rows, n), out_dtype if y is None else y.dtype, x.device, mode == "acc")
    _lib.call("qmm_gemm", CODE[fmt], GEMM_MODE[mode], rows, k, n, _ptr(x), _dt(x), _ptr(scales), _ptr(w), _ptr(w2),
              _ptr(y), _dt(y), _stream())
    return y


def gemm_mxfp4(fmt, mode, x, w, ws, n, k, w2=None, ws2=None, x_scales=None, out_dtype=torch.float32, y=None):
    """The MXFP4 prefill GEMM on the scaled MFMA (g_gemm_mxfp4s_{store|swiglu}_f8_m256): store Y = X8 W^T, acc
    Y += X8 W^T, swiglu Y = silu(X8 W^T) (X8 W2^T). x: E4M3 codes u8 [rows, k] with x_scales u8 [rows, k/32]
    (quant_mxfp8), or f32 / bf16 rows quantized here first. w / ws: split planes (mxfp4s) or MFMA-tiled planes
    (mxfp4t) of [n, k]. y: [rows, n] f32 or bf16."""
    _dev(x, w, ws, w2, ws2, x_scales, y)
    if mode == "swiglu" and (w2 is None or ws2 is None):
        raise ValueError("swiglu needs the up matrix w2 and its scales ws2")
    rows = x.shape[0]
    _cols(x, k)
    if x.dtype != torch.uint8:
        if x_scales is not None:
            raise ValueError("x_scales come with E4M3 codes; pass bf16 / f32 rows without them")
        x, x_scales = quant_mxfp8(x)
    elif x_scales is None or tuple(x_scales.shape) != (rows, k // MX_BLOCK):
        raise ValueError("E4M3 codes need their E8M0 scales [rows, k/32]")
    y = _out(y, (rows, n), out_dtype if y is None else y.dtype, x.device, mode == "acc")
    _lib.call("qmm_gemm_mxfp4", CODE[fmt], GEMM_MODE[mode], rows, k, n, _ptr(x), _ptr(x_scales), _ptr(w), _ptr(ws),
              _ptr(w2), _ptr(ws2), _ptr(y), _dt(y), _stream())
    return y


def moe_topk(logits, KU, gating, norm, scale=1.0, bias=None):
    """(ids i32 [T, KU], wts f32 [T, KU]) from router logits f32 [T, E]."""
    _dev(logits, bias)
    T, E = logits.shape
    ids = torch.empty((T, KU), dtype=torch.int32, device=logits.device)
    wts = torch.empty((T, KU), dtype=torch.float32, device=logits.device)
    _lib.call("qmm_moe_topk", _ptr(logits), T, E, KU, gating, int(bool(norm)), float(scale), _ptr(bias), _ptr(ids),
              _ptr(wts), _stream())
    return ids, wts


def moe_topk_operand(logits, KU, gating, norm, x, op, scale=1.0, bias=None):
    """moe_topk together with the grouped gate/up GEMM's activation operand of the bf16 token rows x [T, H] in one
    launch (qmm_moe_topk_operand): op "f16" -> (ids, wts, x16, scales) with x16, scales as row_scale_f16(x);
    "mxfp8" -> (ids, wts, codes, scales) as quant_mxfp8(x). H <= 4096."""
    _dev(logits, x, bias)
    T, E = logits.shape
    H = x.shape[1]
    dev = logits.device
    ids = torch.empty((T, KU), dtype=torch.int32, device=dev)
    wts = torch.empty((T, KU), dtype=torch.float32, device=dev)
    if op == "f16":
        xo = torch.empty((T, H), dtype=torch.float16, device=dev)
        xs = torch.empty((T, 2), dtype=torch.float32, device=dev)
    else:
        xo = torch.empty((T, H), dtype=torch.uint8, device=dev)
        xs = torch.empty((T, H // MX_BLOCK), dtype=torch.uint8, device=dev)
    _lib.call("qmm_moe_topk_operand", _ptr(logits), T, E, KU, gating, int(bool(norm)), float(scale), _ptr(bias),
              _ptr(ids), _ptr(wts), H, _ptr(x), _dt(x), DTYPE["f16" if op == "f16" else "mxfp8"], _ptr(xo), _ptr(xs),
              _stream())
    return ids, wts, xo, xs


def moe_route(x, w_router, KU, gating, norm, scale=1.0, bias=None, info=None, logits=None):
    """(ids, wts, logits f32 [T, E]) from the hidden rows x f32 / bf16 [T, H] and the router weight f32 / bf16
    [E, H]: logits = x W^T, then moe_topk. With info (i32 [T, 4]) padding tokens (info[t, 2] == 0) get no ids."""
    _dev(x, w_router, bias, info, logits)
    T, H = x.shape
    E = w_router.shape[0]
    logits = torch.empty((T, E), dtype=torch.float32, device=x.device) if logits is None else logits
    ids = torch.empty((T, KU), dtype=torch.int32, device=x.device)
    wts = torch.empty((T, KU), dtype=torch.float32, device=x.device)
    _lib.call("qmm_moe_route", T, H, E, KU, gating, int(bool(norm)), float(scale), _ptr(x), _dt(x), _ptr(w_router),
              _dt(w_router), _ptr(bias), _ptr(info), _ptr(logits), _ptr(ids), _ptr(wts), _stream())
    return ids, wts, logits


def moe_shared_gate(x, w):
    """sg f32 [T] = sigmoid(x[t] . w) (the Qwen-MoE shared-expert gate ffn_gate_inp_shexp, w f32 / bf16 [H])."""
    _dev(x, w)
    T, H = x.shape
    sg = torch.empty(T, dtype=torch.float32, device=x.device)
    _lib.call("qmm_moe_shared_gate", T, H, _ptr(x), _dt(x), _ptr(w), _dt(w), _ptr(sg), _stream())
    return sg


def moe_wscale(ids, wts, scale):
    """wts[t, k] *= scale[clamp(ids[t, k], 0, E - 1)] in place (ffn_down_exps.scale folded into the weights)."""
    _dev(ids, wts, scale)
    T, KU = ids.shape
    _lib.call("qmm_moe_wscale", T, KU, scale.shape[0], _ptr(ids), _ptr(scale), _ptr(wts), _stream())
    return wts


def max_tiles(tokens, KU, E):
    """Worst-case bucketed tiles: T*KU/64 + E (S/gen_llm.py:5407-5411)."""
    return tokens * KU // TILE + E


def moe_bucket(ids, E, n_tiles=None, info=None):
    """(tile_info i32 [max_tiles, 2], rowmap i32 [max_tiles*64], pos i32 [T*KU]) of the assignments."""
    _dev(ids, info)
    T, KU = ids.shape
    n_tiles = max_tiles(T, KU, E) if n_tiles is None else n_tiles
    dev = ids.device
    tile_info = torch.empty((n_tiles, 2), dtype=torch.int32, device=dev)
    rowmap = torch.empty(n_tiles * TILE, dtype=torch.int32, device=dev)
    pos = torch.empty(T * KU, dtype=torch.int32, device=dev)
    _lib.call("qmm_moe_bucket", T, KU, E, n_tiles, _ptr(info), _ptr(ids), _ptr(tile_info), _ptr(rowmap), _ptr(pos),
              _stream())
    return tile_info, rowmap, pos


def moe_expert_mv(fmt, mode, ids, x, w, n, k, E, KU, w2=None, ws=None, ws2=None, fused=False, act="silu",
                  bias=None, bias2=None, y=None):
    """Decode expert matvecs: mode 'gu' act[a] = act(Wg[e] x[a/KU], Wu[e] x[a/KU]) or 'dn' ys[a] = Wd[e] x[a].
    MXFP4 as split planes (mxfp4s) or as the grouped GEMM's MFMA-tiled planes (mxfp4t: one weight copy for decode and
    prefill); ws / ws2 the scale planes."""
    _dev(ids, x, w, w2, ws, ws2, bias, bias2, y)
    A = ids.numel()
    _cols(x, k)
    y = _out(y, (A, n), torch.float32, x.device)
    m = {"gu": 0, "dn": 1}[mode]
    if fmt in SPLIT:
        _lib.call("qmm_moe_expert_mv_split" if fmt == "mxfp4s" else "qmm_moe_expert_mv_tiled", m, int(fused), ACT[act], k, n, E, KU, A, _ptr(ids), _ptr(x), _dt(x),
                  _ptr(w), _ptr(ws), _ptr(w2), _ptr(ws2), _ptr(bias), _ptr(bias2), _ptr(y), _stream())
    else:
        _lib.call("qmm_moe_expert_mv", CODE[fmt], m, int(fused), ACT[act], k, n, E, KU, A, _ptr(ids), _ptr(x), _dt(x),
                  _ptr(w), _ptr(w2), _ptr(bias), _ptr(bias2), _ptr(y), _stream())
    return y


def moe_expert_mv_q8(fmt, mode, ids, x, w, n, k, E, KU, w2=None, fused=False, act="silu", bias=None, bias2=None,
                     y=None, x_rows=None, ws=None, ws2=None):
    """Decode expert matvecs on Q8_1 activations (g_moe_gu_{fmt}[_fused]_q8_k{H}_r{R} / g_moe_dn_{fmt}_q8_k{FE}_r{R}):
    x is the planar Q8_1 buffer of x_rows rows (gu: the tokens, dn: the assignments), or f32 / bf16 rows quantized
    here first (quant_q8). fmt q4_k / q4_0 / q6_k, or mxfp4s (the reference's opt-in MXFP4S_Q8) with ws / ws2 the
    scale planes. Returns y f32 [assignments, n]."""
    _dev(ids, x, w, w2, ws, ws2, bias, bias2, y)
    A = ids.numel()
    rows = A // KU if mode == "gu" else A
    if x.dtype != torch.uint8:
        _cols(x, k)
        if x.shape[0] != rows:
            raise ValueError(f"x has {x.shape[0]} rows, the {mode} matvec reads {rows}")
        x = quant_q8(x)
    elif x.numel() < q8_bytes(rows, k):
        raise ValueError(f"the planar Q8_1 buffer holds {x.numel()} bytes, {rows} rows of K {k} need "
                         f"{q8_bytes(rows, k)}")
    y = _out(y, (A, n), torch.float32, x.device)
    if fmt == "mxfp4s":
        if ws is None or (mode == "gu" and not fused and ws2 is None):
            raise ValueError("mxfp4s experts need their E8M0 scale planes (ws / ws2)")
        _lib.call("qmm_moe_expert_mv_mxfp4s_q8", {"gu": 0, "dn": 1}[mode], int(fused), ACT[act], k, n, E, KU, A,
                  _ptr(ids), _ptr(x), _ptr(w), _ptr(ws), _ptr(w2), _ptr(ws2), _ptr(bias), _ptr(bias2), _ptr(y),
                  _stream())
        return y
    _lib.call("qmm_moe_expert_mv_q8", CODE[fmt], {"gu": 0, "dn": 1}[mode], int(fused), ACT[act], k, n, E, KU, A,
              _ptr(ids), _ptr(x), _ptr(w), _ptr(w2), _ptr(bias), _ptr(bias2), _ptr(y), _stream())
    return y


def moe_grouped(fmt, mode, tile_info, rowmap, x, w, n, k, E, KU, w2=None, ws=None, ws2=None, x_scales=None,
                fused=False, act="silu", y=None, bias=None, bias2=None):
    """Grouped expert GEMM over bucketed 64-row tiles (include/qmm.h, qmm_moe_grouped).
    q4_k / q6_k / q4_0: x f16 row-scaled rows with x_scales f32 [rows, 2] (row_scale_f16); mxfp4s / mxfp4t: x E4M3
    codes uint8 [rows, k] with x_scales uint8 [rows, k/32] (quant_mxfp8). y: f32 [max_tiles * 64, n]. bias / bias2:
    per-expert output biases f32 [E, n] (gu: gate and up; dn: bias)."""
    _dev(tile_info, rowmap, x, w, w2, ws, ws2, x_scales, y, bias, bias2)
    _cols(x, k)
    max_rows = tile_info.shape[0] * TILE
    y = _out(y, (max_rows, n), torch.float32, x.device)
    xd = DTYPE["mxfp8"] if x.dtype == torch.uint8 else _dt(x)
    _lib.call("qmm_moe_grouped", CODE[fmt], {"gu": 0, "dn": 1}[mode], int(fused), ACT[act], E, KU, max_rows, k, n,
              x.shape[0], _ptr(tile_info), _ptr(rowmap), _ptr(x), xd, _ptr(x_scales), _ptr(w), _ptr(ws), _ptr(w2),
              _ptr(ws2), _ptr(bias), _ptr(bias2), _ptr(y), _stream())
    return y


def moe_grouped_mxfp8(fmt, tile_info, rowmap, x, w, n, k, E, KU, w2=None, ws=None, ws2=None, x_scales=None,
                      fused=False, act="silu", codes=None, scales=None, bias=None, bias2=None):
    """The MXFP4 gate/up grouped GEMM with its activation quantized to MXFP8 in the epilogue: (codes u8
    [max_tiles*64, n], scales u8 [max_tiles*64, n/32]) == quant_mxfp8(moe_grouped(fmt, "gu", ...), tile_info) bit
    for bit. x: E4M3 codes with x_scales (quant_mxfp8)."""
    _dev(tile_info, rowmap, x, w, w2, ws, ws2, x_scales, codes, scales, bias, bias2)
    _cols(x, k)
    rows = tile_info.shape[0] * TILE
    codes = _out(codes, (rows, n), torch.uint8, x.device)
    scales = _out(scales, (rows, n // MX_BLOCK), torch.uint8, x.device)
    _lib.call("qmm_moe_grouped_mxfp8", CODE[fmt], int(fused), ACT[act], E, KU, rows, k, n, x.shape[0],
              _ptr(tile_info), _ptr(rowmap), _ptr(x), _ptr(x_scales), _ptr(w), _ptr(ws), _ptr(w2), _ptr(ws2),
              _ptr(bias), _ptr(bias2), _ptr(codes), _ptr(scales), _stream())
    return codes, scales


def moe_combine(ys, wts, pos=None, y=None, accumulate=False, sg=None):
    """y[t] (+)= sum_k w[t, k] ys[row(t, k)], row = pos[t*KU + k] (sorted rows) or t*KU + k. With sg (f32 [T], the
    shared-expert gate) y holds the shared experts' output and becomes sg[t] y[t] + sum_k ..."""
    _dev(ys, wts, pos, y, sg)
    T, KU = wts.shape
    H = ys.shape[1]
    if sg is not None:
        if y is None:
            raise ValueError("the gated combine scales the shared experts' output already in y")
        _lib.call("qmm_moe_combine_gated", T, ys.shape[0], H, KU, _ptr(ys), _ptr(pos), _ptr(wts), _ptr(sg), _ptr(y),
                  _stream())
        return y
    y = torch.empty((T, H), dtype=torch.float32, device=ys.device) if y is None else y
    _lib.call("qmm_moe_combine", T, ys.shape[0], H, KU, _ptr(ys), _ptr(pos), _ptr(wts), int(bool(accumulate)),
              _ptr(y), _stream())
    return y


def moe_topk_expert_mv(fmt, logits, KU, gating, norm, x, w, n, k, E, w2=None, ws=None, ws2=None, fused=False,
                       act="silu", bias=None, bias2=None, scale=1.0, router_bias=None, y=None):
    """The decode chain's routing and gate/up expert matvecs in one launch: (ids, wts, act) equal bit for bit to
    moe_topk(logits, KU, gating, norm, scale, router_bias) then moe_expert_mv(fmt, 'gu', ids, x, w, n, k, E, KU, ...).
    logits f32 [T, E]; x f32 / bf16 [T, k]; act f32 [T*KU, n]."""
    _dev(logits, x, w, w2, ws, ws2, bias, bias2, router_bias, y)
    T, E_ = logits.shape
    if E_ != E:
        raise ValueError(f"logits have {E_} experts, E is {E}")
    _cols(x, k)
    if x.shape[0] != T:
        raise ValueError(f"x has {x.shape[0]} rows, the logits {T}")
    ids = torch.empty((T, KU), dtype=torch.int32, device=x.device)
    wts = torch.empty((T, KU), dtype=torch.float32, device=x.device)
    y = _out(y, (T * KU, n), torch.float32, x.device)
    _lib.call("qmm_moe_topk_expert_mv", _ptr(logits), T, E, KU, gating, int(bool(norm)), float(scale),
              _ptr(router_bias), _ptr(ids), _ptr(wts), CODE[fmt], int(fused), ACT[act], k, n, _ptr(x), _dt(x), _ptr(w),
              _ptr(ws), _ptr(w2), _ptr(ws2), _ptr(bias), _ptr(bias2), _ptr(y), _stream())
    return ids, wts, y


def moe_expert_mv_combine(fmt, ids, wts, x, w, n, k, E, ws=None, bias=None, y=None, accumulate=False, sg=None):
    """The decode chain's down matvecs and combine in one launch: y[t] (+)= sum_j wts[t, j] (Wd[e] x[t*KU + j] +
    bias[e]), e = ids[t, j], equal bit for bit to moe_expert_mv(fmt, 'dn', ...) then moe_combine(...). x f32 / bf16
    [T*KU, k]; ids i32 / wts f32 [T, KU]; with sg (f32 [T]) y holds the shared experts' output and becomes
    sg[t] y[t] + sum_j ... Returns y f32 [T, n]."""
    _dev(ids, wts, x, w, ws, bias, y, sg)
    T, KU = wts.shape
    _cols(x, k)
    if x.shape[0] != T * KU:
        raise ValueError(f"x has {x.shape[0]} rows, the down matvecs read {T * KU}")
    if sg is not None and y is None:
        raise ValueError("the gated combine scales the shared experts' output already in y")
    y = _out(y, (T, n), torch.float32, x.device)
    _lib.call("qmm_moe_expert_mv_combine", CODE[fmt], k, n, E, KU, T, _ptr(ids), _ptr(wts), _ptr(x), _dt(x), _ptr(w),
              _ptr(ws), _ptr(bias), int(bool(accumulate)), _ptr(sg), _ptr(y), _stream())
    return y


def row_scale_f16(x, tile_info=None, x16=None, scales=None, info=None):
    """(x16 f16 [rows, k], scales f32 [rows, 2]) with the per-row power-of-two scale; x f32 or bf16 [rows, k].
    info (i32 [rows, 4], g_row_scale_f16_live): rows with info[row, 2] == 0 are padding, scale 0 and zero values."""
    _dev(x, tile_info, x16, scales, info)
    rows, k = x.shape
    x16 = torch.empty((rows, k), dtype=torch.float16, device=x.device) if x16 is None else x16
    scales = torch.empty((rows, 2), dtype=torch.float32, device=x.device) if scales is None else scales
    if info is not None:
        if tile_info is not None:
            raise ValueError("info (epoch rows) and tile_info (expert tiles) are separate producers")
        _lib.call("qmm_row_scale_f16_live", rows, _ptr(info), k, _ptr(x), _dt(x), _ptr(scales), _ptr(x16), _stream())
    else:
        _lib.call("qmm_row_scale_f16", rows, k, _ptr(x), _dt(x), _ptr(scales), _ptr(x16), _ptr(tile_info), _stream())
    return x16, scales


def row_scale_f16_rows(x, rows, x16=None, scales=None):
    """row_scale_f16 over the listed rows only (rows i32, -1 entries skipped): (x16, scales) of x's shape, the
    listed rows written as row_scale_f16 writes them, the others left as they were."""
    _dev(x, rows, x16, scales)
    n, k = x.shape
    x16 = torch.empty((n, k), dtype=torch.float16, device=x.device) if x16 is None else x16
    scales = torch.empty((n, 2), dtype=torch.float32, device=x.device) if scales is None else scales
    _lib.call("qmm_row_scale_f16_rows", rows.numel(), _ptr(rows), k, _ptr(x), _dt(x), _ptr(scales), _ptr(x16),
              _stream())
    return x16, scales


def quant_mxfp8(x, tile_info=None, codes=None, scales=None):
    """(E4M3 codes u8 [rows, k], E8M0 scales u8 [rows, k/64]) of x f32 / bf16 [rows, k]."""
    _dev(x, tile_info, codes, scales)
    rows, k = x.shape
    codes = torch.empty((rows, k), dtype=torch.uint8, device=x.device) if codes is None else codes
    scales = torch.empty((rows, k // MX_BLOCK), dtype=torch.uint8, device=x.device) if scales is None else scales
    _lib.call("qmm_quant_mxfp8", rows, k, _ptr(x), _dt(x), _ptr(tile_info), _ptr(codes), _ptr(scales), _stream())
    return codes, scales


def repack_mxfp4(w, rows, k):
    """GGUF MXFP4 bytes -> (nibbles u8 [rows, k/2] pairs order, scales u8 [rows, k/32])."""
    _dev(w)
    nib = torch.empty((rows, k // 2), dtype=torch.uint8, device=w.device)
    sc = torch.empty((rows, k // 32), dtype=torch.uint8, device=w.device)
    _lib.call("qmm_repack_mxfp4", _ptr(w), rows, k, _ptr(nib), _ptr(sc), _stream())
    return nib, sc


_SPLIT_PLANES = {}


def split_planes(w, rows, k):
    """The split planes (nibbles, scales) of GGUF MXFP4 weights w [rows, k], made by repack_mxfp4 once per weight
    tensor and kept while that tensor lives: the load-time preparation the reference's mxfp4s tensors get
    (S/formats.py:12-15), which the prefill GEMMs read. A tensor written in place since (its version counter moved)
    or asked for with another shape is repacked again."""
    key, tag = id(w), (w.data_ptr(), w._version, rows, k)
    hit = _SPLIT_PLANES.get(key)
    if hit is not None and hit[0] == tag:
        return hit[1]
    planes = repack_mxfp4(w, rows, k)
    if hit is None:   # the entry goes when the tensor does, before its id can name another object
        weakref.finalize(w, _SPLIT_PLANES.pop, key, None)
    _SPLIT_PLANES[key] = (tag, planes)
    return planes


def tile_q4k(w, rows, k):
    """GGUF Q4_K rows (uint8, rows * k / 256 * 144 bytes) -> the tiled layout (format "q4_kt") the int8-activation
    decode GEMV and the grouped expert GEMMs stream contiguously. rows % 16 == 0, k % 256 == 0 (the GEMV takes
    k % 512 == 0); a byte permutation of the same size. Expert tensors [E, n, k] tile as E * n rows (n % 16 == 0)."""
    _dev(w)
    w_t = torch.empty(rows * row_bytes("q4_k", k), dtype=torch.uint8, device=w.device)
    _lib.call("qmm_tile_q4k", _ptr(w), rows, k, _ptr(w_t), _stream())
    return w_t


def tile_q40(w, rows, k):
    """GGUF Q4_0 rows (uint8, rows * k / 32 * 18 bytes) -> the tiled layout (format "q4_0t") the int8-activation
    decode GEMV streams contiguously, in the units of tile_q4k. rows % 16 == 0, k % 512 == 0; the same size."""
    _dev(w)
    w_t = torch.empty(rows * row_bytes("q4_0", k), dtype=torch.uint8, device=w.device)
    _lib.call("qmm_tile_q40", _ptr(w), rows, k, _ptr(w_t), _stream())
    return w_t


def tile_mxfp4(nib, sc, rows, k):
    """Split planes (nibbles u8 [rows, k/2], scales u8 [rows, k/32]) -> MFMA-tiled planes (nib_t u8 [rows*k/2],
    sc_t u8 [qmm_mxfp4t_scale_bytes]) for the grouped GEMM (format "mxfp4t"). rows % 32 == 0, k % 64 == 0; a
    stack of experts tiles as one matrix when each expert's rows are a multiple of 32."""
    _dev(nib, sc)
    nb = _lib.load().qmm_mxfp4t_scale_bytes(rows, k)
    if nb <= 0:
        raise ValueError(f"mxfp4t needs rows % 32 == 0 and k % 64 == 0 (rows={rows}, k={k})")
    nib_t = torch.empty(rows * k // 2, dtype=torch.uint8, device=nib.device)
    sc_t = torch.empty(nb, dtype=torch.uint8, device=nib.device)
    _lib.call("qmm_tile_mxfp4", _ptr(nib), _ptr(sc), rows, k, _ptr(nib_t), _ptr(sc_t), _stream())
    return nib_t, sc_t


def weight_bytes(fmt, rows, k):
    return rows * row_bytes(fmt, k)


# ------------------------------------------------------------------------------------------------ MoE chains
def _route(x, logits, KU, gating, norm, scale, bias, router, down_scale, info=None):
    """ids, wts (and the logits) of a chain: from given logits (moe_topk) or from the router weight (moe_route),
    then the per-expert down scales folded into the weights (g_moe_wscale)."""
    if (logits is None) == (router is None):
        raise ValueError("give the router logits or the router weight, one of them")
    if logits is None:
        ids, wts, logits = moe_route(x, router, KU, gating, norm, scale=scale, bias=bias, info=info)
    else:
        ids, wts = moe_topk(logits, KU, gating, norm, scale=scale, bias=bias)
    if down_scale is not None:
        moe_wscale(ids, wts, down_scale)
    return ids, wts, logits


def moe_prefill(fmt, x, logits, E, KU, H, FE, gating, norm, w_gate, w_down, w_up=None, ws_gate=None, ws_down=None,
                ws_up=None, fused=False, act="silu", scale=1.0, bias=None, router=None, expert_bias=None,
                down_scale=None, y=None, sg=None, fmt_down=None):
    """The reference's prefill MoE chain (moe_routed with t >= 64, S/gen_llm.py:5324-5385): route, bucket into
    64-row expert tiles, grouped gate/up GEMM with the activation, grouped down GEMM, combine.
    q4_k / q4_kt (tiled, tile_q4k) / q6_k / q4_0: activations row-scaled to f16 (g_row_scale_f16[_tiles]); mxfp4s /
    mxfp4t: quantized to MXFP8.
    x bf16 / f32 [T, H]; logits f32 [T, E], or None with router (the weight f32 / bf16 [E, H]); expert_bias
    (bg [E, FE], bu [E, FE], bd [E, H]) or None; down_scale f32 [E] or None; y: None (y = routed output), or the
    shared experts' output the routed output is added to (scaled first by sg, the shared gate, when given);
    fmt_down: the down tensor's format when it differs (q4_k gate / up with q6_k down, the Q4_K_M expert layout).
    Returns (y f32 [T, H], intermediates dict)."""
    if fmt == "mxfp4":   # GGUF blocks: split planes for the scaled MFMA (repacked once per weight tensor)
        fmt, (w_gate, ws_gate), (w_down, ws_down) = "mxfp4s", split_planes(w_gate, E * FE * (2 if fused else 1), H), \
            split_planes(w_down, E * H, FE)
        if w_up is not None:
            w_up, ws_up = split_planes(w_up, E * FE, H)
    gguf = gate_format(fmt) in ("q4_k", "q4_kt", "q6_k", "q4_0")   # a "gate+up" pair: GGUF gate / up in two formats
    xop = None
    if logits is not None and router is None and x.dtype == torch.bfloat16 and H <= 4096 and \
            (gguf or H % MX_BLOCK == 0):
        # routing and the gate/up operand in one launch (the same bits as the separate calls)
        ids, wts, xop, xos = moe_topk_operand(logits, KU, gating, norm, x, "f16" if gguf else "mxfp8", scale=scale,
                                              bias=bias)
        if down_scale is not None:
            moe_wscale(ids, wts, down_scale)
    else:
        ids, wts, logits = _route(x, logits, KU, gating, norm, scale, bias, router, down_scale)
    bg, bu, bd = expert_bias if expert_bias is not None else (None, None, None)
    tile_info, rowmap, pos = moe_bucket(ids, E)
    if gguf:
        x16, xs = (xop, xos) if xop is not None else row_scale_f16(x)
        a = moe_grouped(fmt, "gu", tile_info, rowmap, x16, w_gate, FE, H, E, KU, w2=w_up, x_scales=xs,
                        fused=fused, act=act, bias=bg, bias2=bu)
        # the down GEMM's operand over the assignments' rows (the rows the tile-wise producer covers)
        a16, as_ = row_scale_f16_rows(a, pos) if FE % 8 == 0 and FE <= 8192 else row_scale_f16(a, tile_info=tile_info)
        ys = moe_grouped(fmt_down or gate_format(fmt), "dn", tile_info, rowmap, a16, w_down, H, FE, E, KU,
                         x_scales=as_, bias=bd)
    elif fmt in ("mxfp4s", "mxfp4t"):
        # the gate/up GEMM writes its activation as MXFP8 directly (the down GEMM's A operand)
        x8, xs = (xop, xos) if xop is not None else quant_mxfp8(x)
        a8, as8 = moe_grouped_mxfp8(fmt, tile_info, rowmap, x8, w_gate, FE, H, E, KU, w2=w_up, ws=ws_gate,
                                    ws2=ws_up, x_scales=xs, fused=fused, act=act, bias=bg, bias2=bu)
        a = None
        ys = moe_grouped(fmt, "dn", tile_info, rowmap, a8, w_down, H, FE, E, KU, ws=ws_down, x_scales=as8, bias=bd)
    else:
        raise ValueError(f"no grouped path for {fmt}")
    y = moe_combine(ys, wts, pos=pos, y=y, accumulate=y is not None, sg=sg)
    mid = {"ids": ids, "wts": wts, "logits": logits, "tile_info": tile_info, "rowmap": rowmap, "pos": pos, "act": a,
           "ys": ys}
    if a is None:
        mid.update(act8=a8, act_scales=as8)
    return y, mid


Q8_FORMATS = ("q4_0", "q4_k", "q6_k", "mxfp4s")   # formats with integer-code expert matvecs (the kernels exist)


def _moe_q8(q8, fmt, fmt_down, expert_bias):
    """Whether a decode chain takes int8 activations: "auto" as the reference decides it (MOE_Q8 on by default,
    moe_iq S/gen_llm.py:5296-5303: both formats in its default int8 set ICODES -- Q4_K, Q6_K; Q4_0 with Q4_0_Q8=1 --
    and no expert biases), else the caller's choice (q8=True for any of Q8_FORMATS)."""
    if q8 == "auto":
        return fmt in ICODES and fmt_down in ICODES and expert_bias is None
    return bool(q8)
# The decode chain routes inside its gate/up matvecs (every workgroup ranks its token's logits itself) where that is
# cheaper than a routing launch: one key slot a lane and few assignments (gpt-oss-20b at one token: 25.0 -> 23.9 us;
# Qwen3-30B-A3B at one token, 128 experts, 24.8 -> 25.5 us, and either at eight tokens +14 to +26 us)
ROUTE_GU_MAX_E, ROUTE_GU_MAX_A = 64, 8


def moe_decode(fmt, x, logits, E, KU, H, FE, gating, norm, w_gate, w_down, w_up=None, ws_gate=None, ws_down=None,
               ws_up=None, fused=False, act="silu", scale=1.0, bias=None, router=None, expert_bias=None,
               down_scale=None, y=None, sg=None, fmt_down=None, q8="auto"):
    """The reference's decode MoE chain (moe_routed with t < 64): route, per-assignment expert matvecs
    (g_moe_gu_* then g_moe_dn_*), combine in assignment order. Arguments as moe_prefill; fmt_down: the down
    tensor's format when it differs (Q4_K_M files: Q4_K gate / up, Q6_K down, S/gen_llm.py:5336-5340).
    q8: the int8-activation chain (the reference's MOE_Q8 default, S/gen_llm.py:5290-5303, :5381-5383): x is
    quantized to Q8_1 once, the gate/up matvecs contract integer codes, their output is quantized again (g_quant_q8)
    for the down matvecs; formats q4_0 / q4_k / q6_k / mxfp4s. "auto" (the default) takes it where the reference
    does: both formats in its int8 set (formats.ICODES) and the experts without biases (gen_llm.moe_iq,
    S/gen_llm.py:5296-5303); False keeps the f32 / bf16 activations (the reference's MOE_Q8=0).
    Returns (y f32 [T, H], intermediates dict)."""
    fd = fmt_down or gate_format(fmt)
    q8 = _moe_q8(q8, fmt, fd, expert_bias)
    if q8 and (fmt not in Q8_FORMATS or fd not in Q8_FORMATS):
        raise ValueError(f"the int8 expert matvecs take {Q8_FORMATS} (gate/up {fmt}, down {fd})")
    bg, bu, bd = expert_bias if expert_bias is not None else (None, None, None)
    if not q8 and logits is not None and router is None and E <= ROUTE_GU_MAX_E and x.shape[0] * KU <= ROUTE_GU_MAX_A \
            and "+" not in fmt:
        # routing and the gate/up matvecs in one launch (equal bit for bit to moe_topk then moe_expert_mv 'gu')
        ids, wts, a = moe_topk_expert_mv(fmt, logits, KU, gating, norm, x, w_gate, FE, H, E, w2=w_up, ws=ws_gate,
                                         ws2=ws_up, fused=fused, act=act, bias=bg, bias2=bu, scale=scale,
                                         router_bias=bias)
        if down_scale is not None:
            moe_wscale(ids, wts, down_scale)
        y = moe_expert_mv_combine(fd, ids, wts, a, w_down, H, FE, E, ws=ws_down, bias=bd, y=y, accumulate=y is not None,
                                  sg=sg)
        return y, {"ids": ids, "wts": wts, "logits": logits, "act": a}
    ids, wts, logits = _route(x, logits, KU, gating, norm, scale, bias, router, down_scale)
    if q8:
        xq = quant_q8(x)
        a = moe_expert_mv_q8(fmt, "gu", ids, xq, w_gate, FE, H, E, KU, w2=w_up, fused=fused, act=act, bias=bg,
                             bias2=bu, ws=ws_gate, ws2=ws_up)
        ys = moe_expert_mv_q8(fd, "dn", ids, quant_q8(a), w_down, H, FE, E, KU, bias=bd, ws=ws_down)
        y = moe_combine(ys, wts, y=y, accumulate=y is not None, sg=sg)
        return y, {"ids": ids, "wts": wts, "logits": logits, "act": a, "ys": ys}
    a = moe_expert_mv(fmt, "gu", ids, x, w_gate, FE, H, E, KU, w2=w_up, ws=ws_gate, ws2=ws_up, fused=fused, act=act,
                      bias=bg, bias2=bu)
    # the down matvecs and the combine in one launch (equal bit for bit to moe_expert_mv 'dn' then moe_combine)
    y = moe_expert_mv_combine(fd, ids, wts, a, w_down, H, FE, E, ws=ws_down, bias=bd, y=y, accumulate=y is not None,
                              sg=sg)
    return y, {"ids": ids, "wts": wts, "logits": logits, "act": a}


# ---------------------------------------------------------------------------------------------------- dispatch
GEMM_MIN_TOKENS = 64   # %gemm: epochs of 64+ tokens take the GEMM / grouped chain (S/gen_llm.py:6107-6126)


# formats with int8-activation decode matvecs (their kernels exist); linear takes them by default for decode_q8(fmt)
LINEAR_Q8_FORMATS = ("q4_0", "q4_k", "q4_kt", "q6_k", "q4_0t", "mxfp4s")


def linear(fmt, x, w, n, k, y=None, mode="store", ws=None, w2=None, ws2=None, q8="auto"):
    """Projection y (+)= x W^T, or swiglu y = silu(x W^T) (x W2^T), with the reference's per-epoch choice (linear,
    S/gen_llm.py:4568-4625): the prefill GEMM for 64+ tokens (GGUF q4_k / q6_k / q4_0 on the f16 MFMA, the activation
    row-scaled to f16 first; MXFP4 on the scaled MFMA, the activation quantized to MXFP8 first -- GGUF mxfp4 blocks
    go through split_planes, repacked once per weight tensor), else the decode GEMV. The decode GEMV takes Q8_1
    activations where the reference does by default (ACT_Q8, iq = ACT_Q8 and fmt in IQ_FMTS and K / 32 <= 1024,
    S/gen_llm.py:514-519, :4590): Q4_K and Q6_K (and the tiled q4_kt), Q4_0 with the reference's Q4_0_Q8=1 switch,
    MXFP4 split planes with MXFP4S_Q8=1, and the tiled q4_0t always (formats.decode_q8); q8=True also takes it for
    q4_0 and mxfp4s; q8=False keeps f32 / bf16 activations (ACT_Q8=0). y is f32."""
    if mode not in ("store", "acc", "swiglu"):
        raise ValueError(f"linear mode {mode}")
    if mode == "swiglu" and w2 is None:
        raise ValueError("swiglu needs the up matrix w2")
    if x.shape[0] >= GEMM_MIN_TOKENS:
        if fmt == "mxfp4":   # GGUF blocks -> split planes (kept per weight tensor after the first call)
            (w, ws), (w2, ws2) = split_planes(w, n, k), (split_planes(w2, n, k) if w2 is not None else (None, None))
            fmt = "mxfp4s"
        if fmt in ("q4_k", "q4_kt", "q6_k", "q4_0", "mxfp4s", "mxfp4t"):
            return gemm(fmt, mode, x, w, n, k, w2=w2, y=y, ws=ws, ws2=ws2)
        raise ValueError(f"no prefill GEMM reads {fmt} weights")
    iq = decode_q8(fmt) if q8 == "auto" else bool(q8) and fmt in LINEAR_Q8_FORMATS
    if iq and k // 32 <= 1024:
        if mode == "swiglu":
            return mv_swiglu_q8(fmt, w, w2, x, n, k, y=y, ws=ws, ws2=ws2)
        return mv_q8(fmt, w, x, n, k, y=y, accumulate=mode == "acc", ws=ws)
    if mode == "swiglu":
        return mv_swiglu(fmt, w, w2, x, n, k, y=y)
    return mv(fmt, w, x, n, k, y=y, accumulate=mode == "acc", ws=ws)


def moe_routed(fmt, x, logits, E, KU, H, FE, gating, norm, **kw):
    """The routed experts of one MoE layer (moe_routed, S/gen_llm.py:5324-5385): the grouped prefill chain for 64+
    tokens, the per-assignment decode chain below (on int8 activations where the reference takes them, q8="auto";
    q8=False keeps f32 / bf16). Returns (y f32 [T, H], intermediates dict)."""
    chain = moe_prefill if x.shape[0] >= GEMM_MIN_TOKENS else moe_decode
    if fmt == "mxfp4s" and "w_gate" in kw and kw.get("ws_gate") is None:
        raise ValueError("mxfp4s weights need their scale planes")
    if chain is moe_prefill:
        kw.pop("q8", None)   # the prefill chain's activations are the GEMMs' (f16 rows, MXFP8)
    return chain(fmt, x, logits, E, KU, H, FE, gating, norm, **kw)


def moe_chain_workspace(fmt, E, KU, T, H, FE, q8=False, router=False):
    """Bytes of the workspace moe_chain (qmm_moe_routed) needs."""
    n = _lib.load().qmm_moe_routed_workspace_size(CODE[fmt], int(bool(q8)), E, KU, T, H, FE, int(bool(router)))
    if n < 0:
        raise ValueError(f"qmm_moe_routed does not run {fmt} at {T} tokens (q8={q8})")
    return n


def moe_chain(fmt, x, logits, E, KU, H, FE, gating, norm, w_gate, w_down, w_up=None, ws_gate=None, ws_down=None,
              ws_up=None, fused=False, act="silu", scale=1.0, bias=None, router=None, expert_bias=None,
              down_scale=None, y=None, sg=None, fmt_down=None, q8="auto", workspace=None):
    """The routed experts of one MoE layer in one library call (qmm_moe_routed, the command sequence of moe_routed,
    S/gen_llm.py:5324-5385): the same kernels as moe_routed's op-by-op chain, the intermediates in one workspace
    (a uint8 device tensor of at least moe_chain_workspace bytes; allocated here when None). Arguments as
    moe_prefill / moe_decode. Returns y f32 [T, H]."""
    _dev(x, logits, w_gate, w_down, w_up, ws_gate, ws_down, ws_up, bias, router, down_scale, y, sg, workspace)
    T = x.shape[0]
    q8 = T < GEMM_MIN_TOKENS and _moe_q8(q8, fmt, fmt_down or fmt, expert_bias)
    _cols(x, H)
    if (logits is None) == (router is None):
        raise ValueError("give the router logits or the router weight, one of them")
    need = moe_chain_workspace(fmt, E, KU, T, H, FE, q8=q8, router=router is not None)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    elif workspace.numel() < need:
        raise ValueError(f"the workspace holds {workspace.numel()} bytes, the chain needs {need}")
    accumulate = y is not None and sg is None
    if sg is not None and y is None:
        raise ValueError("the gated combine scales the shared experts' output already in y")
    y = _out(y, (T, H), torch.float32, x.device)
    bg, bu, bd = expert_bias if expert_bias is not None else (None, None, None)
    _lib.call("qmm_moe_routed", CODE[fmt], CODE[fmt_down] if fmt_down else -1, int(fused), ACT[act], gating,
              int(bool(norm)), float(scale), int(bool(q8)), E, KU, T, H, FE, _ptr(x), _dt(x), _ptr(logits),
              _ptr(router), _dt(router) if router is not None else 0, _ptr(bias), _ptr(down_scale), _ptr(w_gate),
              _ptr(ws_gate), _ptr(w_up), _ptr(ws_up), _ptr(w_down), _ptr(ws_down), _ptr(bg), _ptr(bu), _ptr(bd),
              _ptr(sg), int(accumulate), _ptr(y), _ptr(workspace), workspace.numel(), _stream())
    return y


def moe_layer(fmt, x, logits, E, KU, H, FE, gating, norm, shared=None, **kw):
    """One MoE FFN layer (moe_layer, S/gen_llm.py:5306-5321): the shared experts, a dense swiglu FFN of width FS
    stored into y, then the routed experts added into y; with a shared gate the shared output is scaled per token by
    sigmoid(x . w_gate_inp_shexp) inside the combine. shared: None or a dict with fmt, w_gate, w_up, w_down, FS and
    optionally fmt_down and gate (the f32 / bf16 [H] gate weight). Returns (y f32 [T, H], intermediates dict)."""
    if shared is None:
        return moe_routed(fmt, x, logits, E, KU, H, FE, gating, norm, **kw)
    FS, sf = shared["FS"], shared["fmt"]
    q8 = kw.get("q8", "auto")   # the shared experts' matvecs follow the routed chain's choice of activations
    f = linear(sf, x, shared["w_gate"], FS, H, mode="swiglu", w2=shared["w_up"], q8=q8)
    y = linear(shared.get("fmt_down", sf), f, shared["w_down"], H, FS, q8=q8)
    sg = moe_shared_gate(x, shared["gate"]) if shared.get("gate") is not None else None
    y, mid = moe_routed(fmt, x, logits, E, KU, H, FE, gating, norm, y=y, sg=sg, **kw)
    mid.update(shared_act=f, sg=sg)
    return y, mid
