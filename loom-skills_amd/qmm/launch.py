"""Name-keyed drop-in for the reference's kernel launches: ``launch(name, grid, args)``.

The reference's generators emit ``kernel.launch @name[grid](args)`` (S/ = skills/loom-port-llm/starter/): the kernel
name carries the format, K, variant, token group and rows per workgroup, and the arguments are positional buffers and
indices. ``Launcher.launch`` parses such a name, checks the grid against the arguments, and makes the libqmm call that
computes the same kernel, with the arguments in the reference's order:

    g_mv_{fmt}_k{K}[_swiglu|_pair][_t{TG}][_q8][_r{R}]  [n, tokens]  (n, tokens, accumulate, x, w [, w2|ws], y [, y2])
                                                                      S/gen_llm.py:1187-1197, mv_name :5098-5111
    g_gemm_{fmt}[_{fmt2}]_{store|acc|swiglu}[_m128|_m256] [rows, n]  (rows, k, n, x16, scales, w [, w2|ws], y)
                                                                      S/gen_gemm.py:549-556, S/gen_llm.py:4568-4625
    g_gemm_mxfp4s_{store|swiglu}_f8_m256[_rdna4]        [rows, n]    (rows, k, n, x8, scales, w, ws [, w2, w2s], y)
                                                                      S/gen_mxfp4s.py:50-101
    g_moe_route[_tr][_live]                             [tokens]     (tokens, x, w_router, bias, ids, wts [, info])
                                                                      S/gen_moe.py:170-174, :410
    g_moe_bucket                                        [tokens]     (tokens, max_tiles, info, ids, tile_info, rowmap,
                                                                      pos)  S/gen_moe.py:833-837
    g_moe_{gu|dn}_{fmt}[_{fmt2}][_fused][_q8]_k{K}_r{R} [n, T*KU]    (n, tokens, ids, x, w [, w2] [, biases], y)
                                                                      S/gen_moe.py:535-564
    g_moe_g{gu|dn}_{fmt}[_{fmt2}][_fused]_k{K}          [max_rows, n] (max_rows, k, n, xrows, tile_info, rowmap, x16,
                                                                      scales, w [, w2] [, biases], y)
                                                                      S/gen_moe.py:1147-1148, S/gen_llm.py:5376-5378
    g_moe_combine / g_moe_combine_sorted                [tokens]     (tokens, [rows,] ys, [pos,] wts, [sg,] y)
                                                                      S/gen_moe.py:730-779, :1231-1280
    g_moe_wscale                                        [tokens]     (tokens, ids, wts, scale)  S/gen_moe.py:1010-1045
    g_moe_shared_gate_{ty}                              [tokens]     (tokens, x, w, sg)  S/gen_moe.py:780-823
    g_row_scale_f16 / _live / _tiles                    [rows]       (rows, [info,] k, x, scales, x16 [, tile_info])
                                                                      S/gen_llm.py:1843-1937, S/gen_moe.py:503-527
    g_quant_q8                                          [rows, k]    (rows, k, x, xq)  S/gen_llm.py:684-749

What the reference compiles into a kernel from the model (gen_llm's MOE dict and globals: experts, top-k, gating, the
expert activation, the router / probability biases, whether a layer has shared experts and their gate) is the
``Config`` a launcher is made with. Buffers are torch device tensors; index arguments are ints. Differences a caller
sees: the reference's row-scaled f16 activations (x16 + scales) are the A operand of the GGUF-block GEMMs as there;
the MXFP4 GEMMs take MXFP8 activations (E4M3 codes + one E8M0 scale per 32 values, ``ops.quant_mxfp8``) and the
``g_moe_g{gu|dn}_mxfp4*`` launches convert the reference's x16 rows to it; GGUF MXFP4 (17-byte block) weights given
to a grouped or dense prefill GEMM are repacked to split planes once per weight tensor (``ops.split_planes``).
Kernels whose gate and up matrices differ in format (``g_gemm_{fmt}_{fmt2}_swiglu``, ``g_moe_gu_{fg}_{fu}_*``,
``g_moe_ggu_{fg}_{fu}_*``) call the same entry points with ``QMM_GATE_UP(gate, up)`` as the format.
Unknown names raise ``KeyError``; argument-count and grid mismatches raise ``ValueError``.
"""
import re

import torch

from . import _lib
from . import ops
from .formats import ACT, CODE, DTYPE, GEMM_MODE

_FMT = r"q4_0|q4_k|q6_k|mxfp4s|mxfp4"
_FMT2 = r"q4_0|q4_k|q6_k|mxfp4"   # the up matrix's format of a gate/up kernel whose gate and up formats differ

PATTERNS = [
    ("mv", re.compile(rf"g_mv_(?P<fmt>{_FMT})_k(?P<k>\d+)(?:_(?P<variant>swiglu|pair))?(?:_t(?P<tg>\d+))?"
                      rf"(?P<q8>_q8)?(?:_r(?P<r>\d+))?")),
    ("gemm_f8", re.compile(r"g_gemm_mxfp4s_(?P<mode>store|swiglu)_f8_m256(?:_rdna4)?")),
    ("gemm", re.compile(rf"g_gemm_(?P<fmt>{_FMT})(?:_(?P<fmt2>{_FMT2}))?_(?P<mode>store|acc|swiglu)"
                        rf"(?:_(?P<tile>m128|m256))?")),
    ("route", re.compile(r"g_moe_route(?P<tr>_tr)?(?P<live>_live)?")),
    ("bucket", re.compile(r"g_moe_bucket")),
    ("expert", re.compile(rf"g_moe_(?P<mode>gu|dn)_(?P<fmt>{_FMT})(?:_(?P<fmt2>{_FMT2}))?(?P<fused>_fused)?"
                          rf"(?P<q8>_q8)?_k(?P<k>\d+)_r(?P<r>\d+)")),
    ("grouped", re.compile(rf"g_moe_g(?P<mode>gu|dn)_(?P<fmt>{_FMT})(?:_(?P<fmt2>{_FMT2}))?(?P<fused>_fused)?"
                           rf"_k(?P<k>\d+)")),
    ("combine", re.compile(r"g_moe_combine(?P<sorted>_sorted)?")),
    ("wscale", re.compile(r"g_moe_wscale")),
    ("shared_gate", re.compile(r"g_moe_shared_gate_(?P<ty>f32|bf16|f16)")),
    ("row_scale", re.compile(r"g_row_scale_f16(?P<variant>_live|_tiles)?")),
    ("quant_q8", re.compile(r"g_quant_q8")),
]

# the libqmm entry point each family (and variant) ends in
ENTRY = {
    "mv": "qmm_mv", "mv_swiglu": "qmm_mv_swiglu", "mv_q8": "qmm_mv_q8", "mv_swiglu_q8": "qmm_mv_swiglu_q8",
    "mv_pair_q8": "qmm_mv_pair_q8", "gemm": "qmm_gemm", "gemm_mxfp4": "qmm_gemm_mxfp4", "gemm_f8": "qmm_gemm_mxfp4",
    "route": "qmm_moe_route", "bucket": "qmm_moe_bucket", "expert": "qmm_moe_expert_mv",
    "expert_split": "qmm_moe_expert_mv_split", "expert_q8": "qmm_moe_expert_mv_q8", "grouped": "qmm_moe_grouped",
    "combine": "qmm_moe_combine", "combine_gated": "qmm_moe_combine_gated", "wscale": "qmm_moe_wscale",
    "shared_gate": "qmm_moe_shared_gate", "row_scale": "qmm_row_scale_f16", "row_scale_live": "qmm_row_scale_f16_live",
    "quant_q8": "qmm_quant_q8",
}


def parse(name):
    """(family, fields) of a reference kernel name; KeyError when no family matches. A second format (fmt2, the
    reference's "GATE+UP" kernels: gate and up matrices in different formats) belongs to the gate/up kernels only."""
    for family, pat in PATTERNS:
        m = pat.fullmatch(name)
        if m:
            f = {k: v for k, v in m.groupdict().items() if v is not None}
            if "fmt2" in f and (f.get("mode") not in ("swiglu", "gu") or "fused" in f or "q8" in f):
                raise KeyError(f"{name!r}: a second weight format names the up matrix of a two-tensor gate/up kernel "
                               f"(S/gen_gemm.py:535-547, S/gen_moe.py:535-552, :1126-1141)")
            return family, f
    raise KeyError(f"no libqmm kernel computes {name!r}")


def _fcode(f):
    """The format code of a parsed name: one format, or QMM_GATE_UP(gate, up) for a gate/up pair."""
    return CODE[f"{f['fmt']}+{f['fmt2']}"] if "fmt2" in f else CODE[f["fmt"]]


def entry_point(name, cfg=None):
    """The libqmm entry point a launch of `name` calls (for the name tables of tests and integration code)."""
    family, f = parse(name)
    if family == "mv":
        key = "mv" + ("_" + f["variant"] if "variant" in f else "") + ("_q8" if "q8" in f else "")
        if key == "mv_pair":
            raise KeyError(f"{name!r}: the pair matvecs are int8 only (S/gen_llm.py:1169)")
        return ENTRY[key]
    if family == "gemm":
        return ENTRY["gemm_mxfp4" if f["fmt"].startswith("mxfp4") else "gemm"]
    if family == "expert":
        if "q8" in f:
            return ENTRY["expert_q8"]
        return ENTRY["expert_split" if f["fmt"] == "mxfp4s" else "expert"]
    if family == "combine":
        return ENTRY["combine_gated" if cfg is not None and cfg.shared_gate else "combine"]
    if family == "row_scale":
        return ENTRY["row_scale_live" if f.get("variant") == "_live" else "row_scale"]
    return ENTRY[family]


class Config:
    """What the reference compiles into its kernels from the model (gen_llm.py's MOE dict and globals):
    experts / used (E, top-k), gating (1 softmax, 2 sigmoid, 3 softmax over the picked), norm_weights, scale (the
    router weight scale), act ("silu" or gpt-oss "swiglu_oai"), probs_bias (gating 2 selection bias) or router_bias
    (gating 3 logits bias) -- with neither, the bias slot of g_moe_route carries a placeholder buffer --,
    shared (the layer has shared experts: the combines add into y) and shared_gate (their sigmoid gate: the combines
    take sg). tiled_q4k: the Q4_K weights given to the int8 matvecs are in the tiled layout (ops.tile_q4k, made at
    load)."""

    def __init__(self, experts=None, used=None, gating=1, norm_weights=False, scale=1.0, act="silu",
                 probs_bias=False, router_bias=False, shared=False, shared_gate=False, tiled_q4k=False):
        self.experts, self.used, self.gating, self.norm_weights = experts, used, gating, norm_weights
        self.scale, self.act, self.probs_bias, self.router_bias = scale, act, probs_bias, router_bias
        self.shared, self.shared_gate, self.tiled_q4k = shared, shared_gate, tiled_q4k

    def moe(self):
        if not self.experts or not self.used:
            raise ValueError("a MoE kernel needs Config(experts=..., used=...)")
        return self.experts, self.used


def _p(t):
    return None if t is None else t.data_ptr()


def _s():
    return torch.cuda.current_stream().cuda_stream


def _need(args, counts, name):
    if len(args) not in counts:
        raise ValueError(f"{name}: {len(args)} arguments, the reference launches it with {sorted(counts)}")


def _grid(grid, want, name):
    if [int(g) for g in grid] != [int(w) for w in want]:
        raise ValueError(f"{name}: grid {list(grid)}, the arguments give {list(want)}")


def _dt(t):
    if t.dtype == torch.uint8:
        return DTYPE["q8"]
    return ops._dt(t)


class Launcher:
    """launch(name, grid, args): one reference kernel launch on torch's current stream."""

    def __init__(self, cfg=None):
        self.cfg = cfg or Config()

    # ------------------------------------------------------------------------------------------------- families
    def launch(self, name, grid, args):
        family, f = parse(name)
        getattr(self, "_" + family)(name, f, list(grid), list(args))

    def _mv(self, name, f, grid, a):
        fmt, k = f["fmt"], int(f["k"])
        variant, q8 = f.get("variant"), "q8" in f
        if variant == "pair":
            _need(a, (8,), name)
            n, tokens, acc, x, w, w2, y, y2 = a
        elif variant == "swiglu":
            _need(a, (7,), name)
            n, tokens, acc, x, w, w2, y = a
            y2 = None
        else:
            _need(a, (6, 7), name)   # split planes: (w, ws)
            n, tokens, acc, x, w = a[:5]
            w2, y, y2 = (a[5], a[6], None) if len(a) == 7 else (None, a[5], None)
        _grid(grid, [n, tokens], name)
        if q8:
            kf = "q4_kt" if fmt == "q4_k" and self.cfg.tiled_q4k else fmt
            xd = _dt(x)
            if fmt == "mxfp4s":   # (w, ws): the opt-in int8 matvec of split planes (MXFP4S_Q8, S/formats.py:26-28)
                if variant or w2 is None:
                    raise KeyError(f"{name!r}: split-plane matvecs take (w, ws) and have no swiglu / pair form "
                                   "(S/gen_llm.py:1183-1184)")
                _lib.call("qmm_mv_mxfp4s_q8", 0, k, n, tokens, acc, _p(x), xd, _p(w), _p(w2), None, None, _p(y), None,
                          _s())
            elif variant == "swiglu":
                _lib.call("qmm_mv_swiglu_q8", CODE[kf], k, n, tokens, acc, _p(x), xd, _p(w), _p(w2), _p(y), _s())
            elif variant == "pair":
                _lib.call("qmm_mv_pair_q8", CODE[kf], k, n, tokens, acc, _p(x), xd, _p(w), _p(w2), _p(y), _p(y2), _s())
            else:
                _lib.call("qmm_mv_q8", CODE[kf], k, n, tokens, acc, _p(x), xd, _p(w), _p(y), _s())
        elif variant == "swiglu":
            _lib.call("qmm_mv_swiglu", CODE[fmt], k, n, tokens, acc, _p(x), ops._dt(x), _p(w), _p(w2), _p(y), _s())
        elif variant == "pair":
            raise KeyError(f"{name!r}: the pair matvecs are int8 only (S/gen_llm.py:1169)")
        else:
            _lib.call("qmm_mv", CODE[fmt], k, n, tokens, acc, _p(x), ops._dt(x), _p(w), _p(w2), _p(y), _s())

    def _gemm(self, name, f, grid, a):
        fmt, mode = f["fmt"], f["mode"]
        if fmt == "mxfp4s":   # (w, ws): weight and scale planes; no swiglu on split planes (S/gen_llm.py:4573)
            if mode == "swiglu":
                raise KeyError(f"{name!r}: the reference has no swiglu GEMM on split planes")
            _need(a, (8,), name)
        else:
            _need(a, (8,) if mode == "swiglu" else (7,), name)
        rows, k, n, x16, scales = a[:5]
        _grid(grid, [rows, n], name)
        y = a[-1]
        if fmt.startswith("mxfp4"):
            if fmt == "mxfp4s":
                (w, ws), (w2, ws2) = (a[5], a[6]), (None, None)
            else:   # GGUF blocks -> split planes (once per weight tensor)
                w, ws = ops.split_planes(a[5], n, k)
                w2, ws2 = ops.split_planes(a[6], n, k) if mode == "swiglu" else (None, None)
            x8, xs8 = ops.quant_mxfp8(_rows_f32(x16, scales))
            _lib.call("qmm_gemm_mxfp4", CODE["mxfp4s"], GEMM_MODE[mode], rows, k, n, _p(x8), _p(xs8), _p(w), _p(ws),
                      _p(w2), _p(ws2), _p(y), ops._dt(y), _s())
            return
        w, w2 = (a[5], a[6]) if mode == "swiglu" else (a[5], None)
        _lib.call("qmm_gemm", _fcode(f), GEMM_MODE[mode], rows, k, n, _p(x16), ops._dt(x16), _p(scales), _p(w),
                  _p(w2), _p(y), ops._dt(y), _s())

    def _gemm_f8(self, name, f, grid, a):
        mode = f["mode"]
        _need(a, (10,) if mode == "swiglu" else (8,), name)
        rows, k, n, x8, scales = a[:5]
        _grid(grid, [rows, n], name)
        w, ws = a[5], a[6]
        w2, ws2 = (a[7], a[8]) if mode == "swiglu" else (None, None)
        y = a[-1]
        _lib.call("qmm_gemm_mxfp4", CODE["mxfp4s"], GEMM_MODE[mode], rows, k, n, _p(x8), _p(scales), _p(w), _p(ws),
                  _p(w2), _p(ws2), _p(y), ops._dt(y), _s())

    def _route(self, name, f, grid, a):
        E, KU = self.cfg.moe()
        live = "live" in f
        _need(a, (7,) if live else (6,), name)
        tokens, x, w, bias, ids, wts = a[:6]
        info = a[6] if live else None
        _grid(grid, [tokens], name)
        b = bias if (self.cfg.probs_bias or self.cfg.router_bias) else None   # else a placeholder buffer
        H = x.shape[-1]
        logits = torch.empty((tokens, E), dtype=torch.float32, device=x.device)
        _lib.call("qmm_moe_route", tokens, H, E, KU, self.cfg.gating, int(bool(self.cfg.norm_weights)),
                  float(self.cfg.scale), _p(x), ops._dt(x), _p(w), ops._dt(w), _p(b), _p(info), _p(logits), _p(ids),
                  _p(wts), _s())

    def _bucket(self, name, f, grid, a):
        E, KU = self.cfg.moe()
        _need(a, (7,), name)
        tokens, max_tiles, info, ids, tile_info, rowmap, pos = a
        _grid(grid, [tokens], name)
        _lib.call("qmm_moe_bucket", tokens, KU, E, max_tiles, _p(info), _p(ids), _p(tile_info), _p(rowmap), _p(pos),
                  _s())

    def _expert(self, name, f, grid, a):
        E, KU = self.cfg.moe()
        fmt, mode, k = f["fmt"], f["mode"], int(f["k"])
        fused, q8 = "fused" in f, "q8" in f
        gu = mode == "gu"
        _need(a, ((7, 9) if gu else (6, 7)), name)   # gpt-oss: the expert biases after the weights
        n, ta, ids, x = a[:4]
        _grid(grid, [n, ta], name)
        if gu:
            w, w2 = a[4], a[5]
            bg, bu = (a[6], a[7]) if len(a) == 9 else (None, None)
        else:
            w, w2 = a[4], None
            bg, bu = (a[5] if len(a) == 7 else None), None
        y = a[-1]
        m, act = (0 if gu else 1), ACT[self.cfg.act]
        if fmt == "mxfp4s":
            raise KeyError(f"{name!r}: split-plane expert weights come with their scale planes (ops.moe_expert_mv, "
                           "ops.moe_expert_mv_q8)")
        if q8:
            _lib.call("qmm_moe_expert_mv_q8", CODE[fmt], m, int(fused), act, k, n, E, KU, ta, _p(ids), _p(x), _p(w),
                      _p(None if fused else w2), _p(bg), _p(bu), _p(y), _s())
        else:
            _lib.call("qmm_moe_expert_mv", _fcode(f), m, int(fused), act, k, n, E, KU, ta, _p(ids), _p(x),
                      ops._dt(x), _p(w), _p(None if fused else w2), _p(bg), _p(bu), _p(y), _s())

    def _grouped(self, name, f, grid, a):
        E, KU = self.cfg.moe()
        fmt, mode, k = f["fmt"], f["mode"], int(f["k"])
        fused = "fused" in f
        gu = mode == "gu"
        _need(a, ((11, 13) if gu else (10, 11)), name)
        max_rows, k_arg, n, xrows, tile_info, rowmap, x16, scales = a[:8]
        if int(k_arg) != k:
            raise ValueError(f"{name}: k {k_arg} in the arguments, K {k} in the name")
        _grid(grid, [max_rows, n], name)
        if gu:
            w, w2 = a[8], a[9]
            bg, bu = (a[10], a[11]) if len(a) == 13 else (None, None)
        else:
            w, w2 = a[8], None
            bg, bu = (a[9] if len(a) == 11 else None), None
        y = a[-1]
        m, act = (0 if gu else 1), ACT[self.cfg.act]
        if fmt.startswith("mxfp4"):
            # the reference's x16 rows (power-of-two row scales, exact) become the MXFP8 operand of the scaled MFMA
            rows_needed = xrows
            x8, xs8 = ops.quant_mxfp8(_rows_f32(x16[:rows_needed], scales[:rows_needed]))
            ws = ws2 = None
            if fmt == "mxfp4":   # GGUF blocks -> split planes (once per weight tensor)
                w, ws = ops.split_planes(w, w.numel() // (k // 32 * 17), k)
                if w2 is not None and not fused:
                    w2, ws2 = ops.split_planes(w2, w2.numel() // (k // 32 * 17), k)
            _lib.call("qmm_moe_grouped", CODE["mxfp4s"], m, int(fused), act, E, KU, max_rows, k, n, xrows,
                      _p(tile_info), _p(rowmap), _p(x8), DTYPE["mxfp8"], _p(xs8), _p(w), _p(ws),
                      _p(None if fused else w2), _p(ws2), _p(bg), _p(bu), _p(y), _s())
            return
        _lib.call("qmm_moe_grouped", _fcode(f), m, int(fused), act, E, KU, max_rows, k, n, xrows, _p(tile_info),
                  _p(rowmap), _p(x16), ops._dt(x16), _p(scales), _p(w), None, _p(None if fused else w2), None,
                  _p(bg), _p(bu), _p(y), _s())

    def _combine(self, name, f, grid, a):
        E, KU = self.cfg.moe()
        srt = "sorted" in f
        gated = self.cfg.shared_gate
        _need(a, ((5 if srt else 3) + (1 if gated else 0) + 1,), name)
        if srt:
            tokens, rows, ys, pos, wts = a[:5]
            rest = a[5:]
        else:
            tokens, ys, wts = a[:3]
            rows, pos, rest = tokens * KU, None, a[3:]
        sg, y = (rest[0], rest[1]) if gated else (None, rest[0])
        _grid(grid, [tokens], name)
        H = ys.shape[-1] if ys.dim() > 1 else ys.numel() // rows
        if gated:
            _lib.call("qmm_moe_combine_gated", tokens, rows, H, KU, _p(ys), _p(pos), _p(wts), _p(sg), _p(y), _s())
        else:
            _lib.call("qmm_moe_combine", tokens, rows, H, KU, _p(ys), _p(pos), _p(wts), int(bool(self.cfg.shared)),
                      _p(y), _s())

    def _wscale(self, name, f, grid, a):
        E, KU = self.cfg.moe()
        _need(a, (4,), name)
        tokens, ids, wts, scale = a
        _grid(grid, [tokens], name)
        _lib.call("qmm_moe_wscale", tokens, KU, E, _p(ids), _p(scale), _p(wts), _s())

    def _shared_gate(self, name, f, grid, a):
        _need(a, (4,), name)
        tokens, x, w, sg = a
        _grid(grid, [tokens], name)
        _lib.call("qmm_moe_shared_gate", tokens, x.shape[-1], _p(x), ops._dt(x), _p(w), ops._dt(w), _p(sg), _s())

    def _row_scale(self, name, f, grid, a):
        variant = f.get("variant")
        if variant == "_live":
            _need(a, (6,), name)
            rows, info, k, x, scales, x16 = a
            _grid(grid, [rows], name)
            _lib.call("qmm_row_scale_f16_live", rows, _p(info), k, _p(x), ops._dt(x), _p(scales), _p(x16), _s())
            return
        _need(a, (6,) if variant == "_tiles" else (5,), name)
        rows, k, x, scales, x16 = a[:5]
        tile_info = a[5] if variant == "_tiles" else None
        _grid(grid, [rows], name)
        _lib.call("qmm_row_scale_f16", rows, k, _p(x), ops._dt(x), _p(scales), _p(x16), _p(tile_info), _s())

    def _quant_q8(self, name, f, grid, a):
        _need(a, (4,), name)
        rows, k, x, xq = a
        _grid(grid, [rows, k], name)
        _lib.call("qmm_quant_q8", rows, k, _p(x), ops._dt(x), _p(xq), _s())


def _rows_f32(x16, scales):
    """f32 rows x16 * inv (the reference's row-scaled f16 operand back at its values: inv is a power of two, exact)."""
    return x16.float() * scales[:, 1:2]


_DEFAULT = Launcher()


def launch(name, grid, args, cfg=None):
    """One reference kernel launch (see the module docstring); cfg: the model's compile-time constants (Config)."""
    (Launcher(cfg) if cfg is not None else _DEFAULT).launch(name, grid, args)
