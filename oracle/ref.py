"""Float64 CPU references of the quantized matmul path (oracle; test infrastructure only).

Restates the numpy references of S/make_kernel_tests.py (paths relative to the reference root, S/ =
skills/loom-port-llm/starter/) and the closed forms of the kernels in S/gen_llm.py and S/gen_moe.py:

* matmuls: float64 brute force on exactly dequantized weights (make_kernel_tests.py:234, :1874, :3197-3221)
* activation quantizers: Q8_1 (make_kernel_tests.py:32-39), row-scale f16 (S/gen_llm.py:1843-1915,
  make_kernel_tests.py:3194-3196), E4M3 rounding (make_kernel_tests.py:2006-2019) and the per-32 MXFP8 quantizer
  the gfx950 scaled MFMA path defines on top of it
* routing: make_kernel_tests.py:3166-3184 (route_ref), S/gen_moe.py:76-252
* bucket / permutation: S/gen_moe.py:829-955 with a canonical (stable) order inside each expert segment
* expert activations: S/gen_moe.py:27-64, make_kernel_tests.py:3208-3213
* combine: S/gen_moe.py:730-762, :1231-1280
"""
import numpy as np

from . import formats

TILE = 64                       # rows per bucketed expert tile (S/gen_moe.py:826)
NORM_FLOOR = 6.103515625e-05    # weight-sum floor of normalized top-k weights (S/gen_moe.py:133)


# ----------------------------------------------------------------------------------------------- number formats
def bf16_round(x):
    """float32 -> nearest bfloat16 (round to nearest even), returned as float32 values."""
    u = np.ascontiguousarray(np.asarray(x, np.float32)).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


def bf16_bits(x):
    """float32 values that are bfloat16 numbers -> their uint16 bit patterns."""
    return (np.ascontiguousarray(np.asarray(x, np.float32)).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_round(x):
    """x -> float64 values of the nearest finite E4M3FN numbers (round to nearest even, saturating at 448);
    restated from make_kernel_tests.py:2006-2012."""
    x = np.asarray(x, np.float64)
    a = np.minimum(np.abs(x), 448.0)
    e = np.maximum(np.floor(np.log2(np.maximum(a, 2.0 ** -20))), -6)
    q = 2.0 ** (e - 3)
    return np.sign(x) * np.minimum(np.rint(a / q) * q, 448.0)


def e4m3_bytes(v):
    """float64 values that are E4M3FN numbers -> their bytes; a negative value that rounds to zero keeps its sign
    (0x80), as the hardware conversion does (make_kernel_tests.py:2013-2019)."""
    v = np.asarray(v, np.float64)
    a = np.abs(v)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -20))).astype(np.int64)
    sub = a < 2.0 ** -6
    ef = np.where(sub, 0, e + 7)
    mant = np.where(sub, np.rint(a / 2.0 ** -9), np.rint((a / 2.0 ** e - 1) * 8)).astype(np.int64)
    b = np.where(a == 0, 0, (ef << 3) | mant) | np.where(np.signbit(v), 0x80, 0)
    return b.astype(np.uint8)


def e4m3_decode(b):
    """E4M3FN bytes -> float64 (sign, 4-bit exponent with bias 7, 3-bit mantissa; exponent 0 is subnormal)."""
    b = np.asarray(b, np.uint8).astype(np.int64)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 15
    m = (b & 7).astype(np.float64)
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7))
    return s * mag


# ----------------------------------------------------------------------------------------- activation quantizers
def q8_1_codes(xs):
    """llama.cpp quantize_q8_1 per 32 values in f32 arithmetic (make_kernel_tests.py:32-39; g_quant_q8,
    S/gen_llm.py:684-749): d = amax/127, q = sign(x/d) floor(|x/d| + 0.5) (0 when d == 0). Returns the int8 codes
    [rows, K], the stored scales f32(f16(d)) and the code sums, both [rows, K/32]."""
    xs = np.asarray(xs, np.float32)
    g = xs.reshape(xs.shape[0], -1, 32)
    d = np.abs(g).max(-1, keepdims=True) / np.float32(127)
    v = np.divide(g, d, out=np.zeros_like(g), where=d > 0)
    q = np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))
    codes = q.astype(np.int8).reshape(xs.shape)
    return codes, d[..., 0].astype(np.float16).astype(np.float32), q.sum(-1, dtype=np.float32)


def q8_1(xs):
    """The Q8_1 activations as the oracle multiplies them: codes times the f16-rounded d (make_kernel_tests.py:32-39)."""
    codes, d16, _ = q8_1_codes(xs)
    g = codes.astype(np.float32).reshape(codes.shape[0], -1, 32)
    return (g * d16[..., None]).reshape(codes.shape)


def q8_planar(xs):
    """The planar Q8_1 buffer of g_quant_q8 (S/gen_llm.py:684-690): int8 codes [rows][K/32][32], then at byte
    rows * K the f32 pairs (f16-rounded d, code sum) [rows][K/32][2]; returned as uint8 bytes."""
    codes, d16, sums = q8_1_codes(xs)
    meta = np.stack([d16, sums], -1).astype(np.float32)
    return np.concatenate([codes.view(np.uint8).reshape(-1), meta.view(np.uint8).reshape(-1)])


def row_scale_exponent(x):
    """e = clamp(exponent(max |x_row|) - 13, 0, 100) per row (S/gen_llm.py:1843-1915)."""
    amax = np.abs(np.asarray(x, np.float64)).max(-1)
    return np.clip(np.frexp(amax)[1] - 1 - 13, 0, 100).astype(np.int64)


def f16_rows(x):
    """g_row_scale_f16 as the oracle sees it: each row scaled by 2^-e into f16 range, rounded to f16, scaled back
    (make_kernel_tests.py:3194-3196)."""
    x = np.asarray(x, np.float64)
    e = row_scale_exponent(x)[..., None].astype(np.float64)
    return (x * 2.0 ** -e).astype(np.float16).astype(np.float64) * 2.0 ** e


MX_BLOCK = 32


def mxfp8_quantize(x, block=MX_BLOCK):
    """MXFP8 (E4M3 elements, one E8M0 scale per `block` values along the last axis, OCP MX: 32), the activation
    operand format of the gfx950 scaled-MFMA path. Shared exponent s = clamp(floor(log2(amax)) - 7, -127, 127) so that every scaled element lies below 256
    and never saturates; elements are E4M3 round-to-nearest-even of x * 2^-s (e4m3_round, restated from
    make_kernel_tests.py:2006-2012). Returns (codes u8 [..., K], scale bytes u8 [..., K/block] = s + 127,
    values f64 [..., K])."""
    x = np.asarray(x, np.float64)
    k = x.shape[-1]
    assert k % block == 0
    g = x.reshape(x.shape[:-1] + (k // block, block))
    amax = np.abs(g).max(-1)
    fl = np.frexp(amax)[1] - 1                    # floor(log2(amax)) for amax > 0
    s = np.where(amax > 0, np.clip(fl - 7, -127, 127), -127).astype(np.int64)
    scaled = g * 2.0 ** (-s[..., None].astype(np.float64))
    q = e4m3_round(scaled)
    codes = e4m3_bytes(q).reshape(x.shape)
    vals = (q * 2.0 ** s[..., None].astype(np.float64)).reshape(x.shape)
    return codes, (s + 127).astype(np.uint8), vals


def mxfp8_values(x):
    return mxfp8_quantize(x)[2]


# ------------------------------------------------------------------------------------------------------ matmuls
def gemv(x, w):
    """y = x W^T in float64 (make_kernel_tests.py:234): x [t, K], W [n, K] exactly dequantized."""
    return np.asarray(x, np.float64) @ np.asarray(w, np.float64).T


def gemm(x, w, inv=None):
    """Y = (X W^T) * inv[row] in float64 (make_kernel_tests.py:1858-1900 'store')."""
    y = np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
    if inv is not None:
        y = y * np.asarray(inv, np.float64)[:, None]
    return y


def rel_l2(actual, expected):
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    return float(np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-300))


# ------------------------------------------------------------------------------------------- expert activations
def silu_mul(g, u):
    """silu(g) * u (S/gen_moe.py:27-32)."""
    g = np.asarray(g, np.float64)
    with np.errstate(over="ignore"):           # e^-g = inf for g < -709: g / inf = -0, the limit
        return g / (1.0 + np.exp(-g)) * np.asarray(u, np.float64)


def swiglu_oai(g, u, alpha=1.702, limit=7.0):
    """ggml_swiglu_oai: x = min(g, limit), y = clamp(u, -limit, limit), x sigmoid(alpha x) (y + 1)
    (S/gen_moe.py:33-46; make_kernel_tests.py:3208-3211)."""
    x = np.minimum(np.asarray(g, np.float64), limit)
    y = np.clip(np.asarray(u, np.float64), -limit, limit)
    with np.errstate(over="ignore"):
        return x / (1.0 + np.exp(-alpha * x)) * (y + 1.0)


ACTIVATIONS = {"silu": silu_mul, "swiglu_oai": swiglu_oai}


# ---------------------------------------------------------------------------------------------------- routing
def router_logits(x, w):
    """logits = x W_router^T in float64 (route_ref, make_kernel_tests.py:3166-3167); W f32 [E, H] (bf16 weights as
    their f32 values)."""
    return np.asarray(x, np.float64) @ np.asarray(w, np.float64).T


def shared_gate(x, w):
    """sg[t] = sigmoid(x[t] . w), the shared-expert gate (make_kernel_tests.py:3252)."""
    d = np.asarray(x, np.float64) @ np.asarray(w, np.float64)
    with np.errstate(over="ignore"):
        return 1.0 / (1.0 + np.exp(-d))


def wscale(ids, wts, scale):
    """wts[t, k] scale[clamp(ids[t, k], 0, E - 1)] (g_moe_wscale; ktest_more.py:99-111)."""
    scale = np.asarray(scale)
    return np.asarray(wts) * scale[np.clip(ids, 0, len(scale) - 1)]


def route(logits, KU, gating, norm, bias=None, scale=1.0):
    """Top-KU experts and weights from router logits (make_kernel_tests.py:3166-3184, with the logits given):
    gating 1 softmax over E then pick; 2 sigmoid (+ selection bias); 3 pick on logit + bias, weights = softmax
    over the picked. Ties go to the lower expert id (stable argsort). Returns (ids i32 [T,KU], wts f64 [T,KU])."""
    logit = np.asarray(logits, np.float64)
    E = logit.shape[-1]
    b = np.zeros(E) if bias is None else np.asarray(bias, np.float64)
    if gating == 3:
        logit = logit + b
        prob = logit
    elif gating == 2:
        prob = 1.0 / (1.0 + np.exp(-logit))
    elif gating == 1:
        ex = np.exp(logit - logit.max(-1, keepdims=True))
        prob = ex / ex.sum(-1, keepdims=True)
    else:
        raise ValueError(gating)
    sel = prob + (b if gating != 3 else 0.0)
    ids = np.argsort(-sel, -1, kind="stable")[:, :KU].astype(np.int32)
    wts = np.take_along_axis(prob, ids.astype(np.int64), -1)
    if gating == 3:
        wts = np.exp(wts - wts.max(-1, keepdims=True))
        wts = wts / wts.sum(-1, keepdims=True)
    if norm:
        wts = wts / np.maximum(wts.sum(-1, keepdims=True), NORM_FLOOR)
    return ids, wts * scale


def route_margin(logits, KU, gating, bias=None):
    """Relative gap between the KU-th and (KU+1)-th selection score per token (make_kernel_tests.py:3181-3184):
    rows with a margin of 0 have a tie at the cut, where only the tie rule decides."""
    logit = np.asarray(logits, np.float64)
    b = np.zeros(logit.shape[-1]) if bias is None else np.asarray(bias, np.float64)
    sel = logit + b if gating == 3 else (1.0 / (1.0 + np.exp(-logit)) + b if gating == 2 else logit)
    ss = np.sort(sel, -1)[:, ::-1]
    if KU >= ss.shape[1]:
        return np.full(ss.shape[0], np.inf)
    return (ss[:, KU - 1] - ss[:, KU]) / np.maximum(np.abs(ss[:, KU - 1]), 1e-30)


# ----------------------------------------------------------------------------------------- bucket / permutation
def max_tiles(tokens, KU, E):
    """Worst-case bucketed tiles: T*KU/64 + E (S/gen_llm.py:5407-5411)."""
    return tokens * KU // TILE + E


def bucket(ids, E, max_tiles_, live=None):
    """Canonical bucket of assignments a = t*KU + k by expert into 64-row tiles (S/gen_moe.py:829-955):
    c_e live assignments per expert, tiles_e = ceil(c_e/64), tiles in expert-id order; inside a segment the
    assignments are in ascending a (the reference's order there is its atomic order). Rows past the used tiles
    are -1 in rowmap (the reference leaves them unwritten). Returns (tile_info i32 [max_tiles,2],
    rowmap i32 [max_tiles*64], pos i32 [T*KU])."""
    ids = np.asarray(ids, np.int64)
    T, KU = ids.shape
    flat = np.clip(ids.reshape(-1), 0, E - 1)       # the reference clamps ids into range (S/gen_moe.py:868-870)
    alive = np.ones(T, bool) if live is None else (np.asarray(live) != 0)
    alive_a = np.repeat(alive, KU)
    counts = np.bincount(flat[alive_a], minlength=E)
    tiles = (counts + TILE - 1) // TILE
    base = np.concatenate([[0], np.cumsum(tiles)[:-1]])
    assert tiles.sum() <= max_tiles_, (tiles.sum(), max_tiles_)
    tile_info = np.tile(np.array([-1, 0], np.int32), (max_tiles_, 1))
    rowmap = np.full(max_tiles_ * TILE, -1, np.int32)
    pos = np.full(T * KU, -1, np.int32)
    cursor = base * TILE
    for e in range(E):
        for j in range(tiles[e]):
            tile_info[base[e] + j] = (e, min(TILE, counts[e] - TILE * j))
    for a in range(T * KU):               # ascending a: the canonical order inside each segment
        if not alive_a[a]:
            continue
        e = flat[a]
        r = cursor[e]
        cursor[e] += 1
        rowmap[r] = a
        pos[a] = r
    return tile_info, rowmap, pos


# ------------------------------------------------------------------------------------------------------ combine
def combine(ys_rows, pos_or_none, wts, y0=None, sg=None):
    """y[t] = (y0[t] or 0) + sum_k w[t,k] ys[row(t,k)], row = pos[t,k] (sorted) or t*KU+k (decode); a row of -1
    contributes 0 (S/gen_moe.py:730-762, :1231-1280). With sg the shared output y0 is scaled first: sg[t] y0[t]
    (shared_gated, S/gen_moe.py:765-779)."""
    wts = np.asarray(wts, np.float64)
    T, KU = wts.shape
    ys = np.asarray(ys_rows, np.float64)
    rows = np.arange(T * KU).reshape(T, KU) if pos_or_none is None else np.asarray(pos_or_none).reshape(T, KU)
    y = np.zeros((T, ys.shape[1])) if y0 is None else np.asarray(y0, np.float64).copy()
    if sg is not None:
        y *= np.asarray(sg, np.float64)[:, None]
    for k in range(KU):
        r = rows[:, k]
        v = np.where((r >= 0)[:, None], ys[np.maximum(r, 0)], 0.0)
        y += wts[:, k][:, None] * v
    return y


# ---------------------------------------------------------------------------------------------------- MoE chain
def moe(x, ids, wts, gate_up, down, act="silu", x_round=None, act_round=None, bias=None):
    """Routed-expert FFN in float64 (make_kernel_tests.py:3197-3221): for each assignment (t, k) with e = ids[t,k]:
    g = Wg[e] xr[t] + bg[e], u = Wu[e] xr[t] + bu[e], a = act(g, u), y[t] += w[t,k] (Wd[e] ar + bd[e]). xr / ar
    are x and a after the activation rounding of the kernel path being checked (identity, f16_rows or
    mxfp8_values). gate_up(e) -> (Wg [FE,H], Wu [FE,H]) and down(e) -> Wd [H,FE] return exactly dequantized expert
    weights; bias: None or (bg [E,FE], bu [E,FE], bd [E,H]), the expert biases (make_kernel_tests.py:3207, :3215).
    Returns (y [T,H], act_rows [T*KU, FE] before rounding)."""
    x = np.asarray(x, np.float64)
    T, KU = ids.shape
    xr = x if x_round is None else x_round(x)
    fn = ACTIVATIONS[act]
    y = acts = None
    for e in np.unique(ids):
        mask = ids == e
        tok, slot = np.nonzero(mask)
        Wg, Wu = gate_up(int(e))
        Wd = down(int(e))
        g = xr[tok] @ np.asarray(Wg, np.float64).T
        u = xr[tok] @ np.asarray(Wu, np.float64).T
        if bias is not None:
            g = g + np.asarray(bias[0][e], np.float64)
            u = u + np.asarray(bias[1][e], np.float64)
        a = fn(g, u)
        if acts is None:
            acts = np.zeros((T * KU, a.shape[1]))
            y = np.zeros((T, Wd.shape[0]))
        acts[tok * KU + slot] = a
        ar = a if act_round is None else act_round(a)
        out = ar @ np.asarray(Wd, np.float64).T
        if bias is not None:
            out = out + np.asarray(bias[2][e], np.float64)
        np.add.at(y, tok, wts[tok, slot][:, None] * out)
    return y, acts
