"""GPU parity of the gate/up kernels whose gate and up matrices come in different formats: the reference's "GATE+UP"
kernels of a layer quantized per tensor (a Q4_K_M layer with a Q4_K gate and a Q6_K up, S/gen_llm.py:5335-5336):

    g_gemm_{fmt}_{fmt2}_swiglu          qmm_gemm(QMM_GATE_UP(gate, up), QMM_GEMM_SWIGLU, ...)   S/gen_gemm.py:535-547
    g_moe_ggu_{fg}_{fu}_k{H}            qmm_moe_grouped(QMM_GATE_UP(gate, up), 0, ...)          S/gen_moe.py:1126-1141
    g_moe_gu_{fg}_{fu}_k{H}_r{R}        qmm_moe_expert_mv(QMM_GATE_UP(gate, up), 0, ...)        S/gen_moe.py:535-552
    (and the dense decode swiglu matvec, qmm_mv_swiglu, and the whole routed chain, qmm_moe_routed)

The oracle is the reference's: float64 products of the exactly dequantized weights (each matrix in its own format)
with the activation as the kernel consumes it (the row-scaled f16 rows for the GEMMs, the bf16 rows for the decode
matvecs), silu(g) u (or swiglu_oai) in float64. Bar: rel-L2 <= 1e-3 (fp32 accumulation; the GEMMs stage weights to
f16 as the reference does).
"""
import numpy as np
import pytest

from helpers import assert_close_rel_l2, dev_bf16, dev_f32, dev_u8, host
from oracle import formats as of
from oracle import ref

pytestmark = pytest.mark.gpu

GEN = {"q4_k": "q4_k_weights", "q6_k": "q6_k_weights", "q4_0": "q4_0_weights", "mxfp4": "mxfp4_weights"}


def _weights(rng, fmt, rows, k):
    from qmm import synth
    return getattr(synth, GEN[fmt])(rng, rows, k)


def _x(rng, rows, k):
    from qmm import synth
    xb = synth.to_bf16_bits(rng.standard_normal((rows, k)).astype(np.float32))
    return xb, synth.bf16_bits_to_f32(xb)


@pytest.mark.parametrize("fg,fu,M,N,K,out", [("q4_k", "q6_k", 100, 192, 512, "f32"), ("q6_k", "q4_k", 64, 128, 768, "bf16"),
                                             ("q4_0", "q4_k", 130, 64, 1024, "f32"), ("q4_k", "q4_0", 64, 320, 256, "f32"),
                                             ("q4_k", "q6_k", 512, 1536, 4096, "bf16")])
def test_swiglu_gemm_gate_and_up_in_two_formats(dev, fg, fu, M, N, K, out):
    """g_gemm_{fg}_{fu}_swiglu: silu(X16 Wg^T inv) (X16 Wu^T inv) with Wg in fg and Wu in fu; a bf16 store equals the
    f32 result rounded to nearest even (the plain swiglu GEMM's store)."""
    import torch
    import qmm.ops as ops
    rng = np.random.default_rng(M + N + K + len(fg + fu))
    wg, wu = _weights(rng, fg, N, K), _weights(rng, fu, N, K)
    xb, xv = _x(rng, M, K)
    xr = ref.f16_rows(xv)
    want = ref.silu_mul(ref.gemv(xr, of.dequantize(fg, wg, N, K)), ref.gemv(xr, of.dequantize(fu, wu, N, K)))
    y32 = host(ops.gemm(f"{fg}+{fu}", "swiglu", dev_bf16(xb, dev), dev_u8(wg, dev), N, K, w2=dev_u8(wu, dev)))
    assert_close_rel_l2(y32, want, 1e-3, f"swiglu gemm {fg}+{fu} {M}x{N}x{K}")
    if out == "bf16":   # the bf16 store is the f32 result rounded to nearest even
        y = ops.gemm(f"{fg}+{fu}", "swiglu", dev_bf16(xb, dev), dev_u8(wg, dev), N, K, w2=dev_u8(wu, dev),
                     out_dtype=torch.bfloat16)
        np.testing.assert_array_equal(host(y).view(np.uint32), ref.bf16_round(y32).view(np.uint32))


@pytest.mark.parametrize("fg,fu,act", [("q4_k", "q6_k", "silu"), ("q6_k", "q4_0", "swiglu_oai")])
def test_grouped_gate_up_in_two_formats(dev, fg, fu, act):
    """g_moe_ggu_{fg}_{fu}: the grouped gate/up GEMM over bucketed tiles (8 experts, top-2, 100 tokens, an expert over
    two tiles), every live row against the oracle; dead rows and unused tiles keep a NaN sentinel."""
    import torch
    import qmm.ops as ops
    rng = np.random.default_rng(7 + len(fg + fu))
    E, KU, H, FE, T = 8, 2, 512, 256, 100
    wg, wu = _weights(rng, fg, E * FE, H), _weights(rng, fu, E * FE, H)
    xb, xv = _x(rng, T, H)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[:80, 3] += 6.0
    ids, _ = ops.moe_topk(dev_f32(logits, dev), KU, 1, True)
    ti, rm, _ = ops.moe_bucket(ids, E)
    x16, xs = ops.row_scale_f16(dev_bf16(xb, dev))
    y0 = torch.full((ti.shape[0] * 64, FE), float("nan"), dtype=torch.float32, device=dev)
    y = host(ops.moe_grouped(f"{fg}+{fu}", "gu", ti, rm, x16, dev_u8(wg, dev), FE, H, E, KU, w2=dev_u8(wu, dev),
                             x_scales=xs, act=act, y=y0))
    tih, rmh = host(ti), host(rm)
    assert (tih[:, 0] == 3).sum() == 2
    xr = ref.f16_rows(xv)
    rbg, rbu = of.row_bytes(fg, H), of.row_bytes(fu, H)
    fn = ref.silu_mul if act == "silu" else ref.swiglu_oai
    for t, (e, rows) in enumerate(tih):
        blk = y[64 * t: 64 * t + 64]
        if e < 0:
            assert np.all(np.isnan(blk)), f"unused tile {t} was written"
            continue
        toks = rmh[64 * t: 64 * t + rows] // KU
        G = of.dequantize(fg, wg[e * FE * rbg:(e + 1) * FE * rbg], FE, H)
        U = of.dequantize(fu, wu[e * FE * rbu:(e + 1) * FE * rbu], FE, H)
        want = fn(ref.gemv(xr[toks], G), ref.gemv(xr[toks], U))
        assert_close_rel_l2(blk[:rows], want, 1e-3, f"grouped {fg}+{fu} tile {t}")
        assert np.all(np.isnan(blk[rows:])), f"dead rows of tile {t} were written"


@pytest.mark.parametrize("fg,fu,xdt", [("q4_k", "q6_k", "bf16"), ("q4_0", "mxfp4", "f32"), ("mxfp4", "q4_k", "bf16")])
def test_expert_matvecs_gate_up_in_two_formats(dev, fg, fu, xdt):
    """g_moe_gu_{fg}_{fu}: the decode gate/up expert matvecs (3 tokens, top-2 of 8 experts, expert biases), each
    assignment's row against the oracle; and the dense swiglu matvec of the same pair (one expert, no ids)."""
    import torch
    import qmm.ops as ops
    rng = np.random.default_rng(11 + len(fg + fu))
    E, KU, H, FE, T = 8, 2, 512, 256, 3
    wg, wu = _weights(rng, fg, E * FE, H), _weights(rng, fu, E * FE, H)
    xb, xv = _x(rng, T, H)
    if xdt == "f32":
        xv = rng.standard_normal((T, H)).astype(np.float32)
        xt = dev_f32(xv, dev)
    else:
        xt = dev_bf16(xb, dev)
    ids = rng.integers(0, E, (T, KU)).astype(np.int32)
    bg, bu = (rng.standard_normal((E, FE)) * 0.1).astype(np.float32), (rng.standard_normal((E, FE)) * 0.1).astype(np.float32)
    y = host(ops.moe_expert_mv(f"{fg}+{fu}", "gu", torch.from_numpy(ids).to(dev), xt, dev_u8(wg, dev), FE, H, E, KU,
                               w2=dev_u8(wu, dev), bias=dev_f32(bg, dev), bias2=dev_f32(bu, dev)))
    rbg, rbu = of.row_bytes(fg, H), of.row_bytes(fu, H)
    for a in range(T * KU):
        e, t = ids.reshape(-1)[a], a // KU
        G = of.dequantize(fg, wg[e * FE * rbg:(e + 1) * FE * rbg], FE, H)
        U = of.dequantize(fu, wu[e * FE * rbu:(e + 1) * FE * rbu], FE, H)
        want = ref.silu_mul(ref.gemv(xv[t:t + 1], G) + bg[e], ref.gemv(xv[t:t + 1], U) + bu[e])
        assert_close_rel_l2(y[a:a + 1], want, 1e-3, f"expert mv {fg}+{fu} assignment {a}")
    # the dense swiglu matvec: expert 0's matrices, every token
    ys = host(ops.mv_swiglu(f"{fg}+{fu}", dev_u8(wg[:FE * rbg], dev), dev_u8(wu[:FE * rbu], dev), xt, FE, H))
    want = ref.silu_mul(ref.gemv(xv, of.dequantize(fg, wg[:FE * rbg], FE, H)),
                        ref.gemv(xv, of.dequantize(fu, wu[:FE * rbu], FE, H)))
    assert_close_rel_l2(ys, want, 1e-3, f"swiglu mv {fg}+{fu}")


@pytest.mark.parametrize("T", [64, 4])
def test_routed_chain_gate_up_in_two_formats(dev, T):
    """The routed experts of a Q4_K_M-style layer -- Q4_K gate, Q6_K up, Q6_K down, 16 experts, top-4 -- through the
    op chain (moe_routed: prefill at 64 tokens, decode on bf16 activations at 4) and the one-call chain
    (qmm_moe_routed), equal bit for bit, against the oracle."""
    import qmm.ops as ops
    rng = np.random.default_rng(90 + T)
    E, KU, H, FE = 16, 4, 512, 256
    wg, wu, wd = _weights(rng, "q4_k", E * FE, H), _weights(rng, "q6_k", E * FE, H), _weights(rng, "q6_k", E * H, FE)
    xb, xv = _x(rng, T, H)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    kw = dict(w_gate=dev_u8(wg, dev), w_up=dev_u8(wu, dev), w_down=dev_u8(wd, dev), fmt_down="q6_k")
    y, mid = ops.moe_routed("q4_k+q6_k", dev_bf16(xb, dev), dev_f32(logits, dev), E, KU, H, FE, 1, True, **kw)
    y2 = ops.moe_chain("q4_k+q6_k", dev_bf16(xb, dev), dev_f32(logits, dev), E, KU, H, FE, 1, True, **kw)
    eids, ewts = ref.route(logits, KU, 1, True)
    np.testing.assert_array_equal(host(mid["ids"]), eids)
    rbg, rbu, rbd = of.row_bytes("q4_k", H), of.row_bytes("q6_k", H), of.row_bytes("q6_k", FE)

    def gate_up(e):
        return (of.dequant_q4_k(wg[e * FE * rbg:(e + 1) * FE * rbg], FE, H),
                of.dequant_q6_k(wu[e * FE * rbu:(e + 1) * FE * rbu], FE, H))

    def down(e):
        return of.dequant_q6_k(wd[e * H * rbd:(e + 1) * H * rbd], H, FE)

    rnd = ref.f16_rows if T >= 64 else None
    want, _ = ref.moe(xv, eids, ewts, gate_up, down, x_round=rnd, act_round=rnd)
    assert_close_rel_l2(host(y), want, 1e-3, f"routed q4_k+q6_k T={T}")
    np.testing.assert_array_equal(host(y).view(np.uint32), host(y2).view(np.uint32))


def test_launcher_runs_the_two_format_swiglu_gemm(dev):
    """launch("g_gemm_q4_k_q6_k_swiglu", [rows, n], (rows, k, n, x16, scales, wg, wu, y)) equals ops.gemm on the
    "q4_k+q6_k" pair, bit for bit."""
    import torch
    import qmm.ops as ops
    from qmm import launch
    rng = np.random.default_rng(5)
    M, N, K = 64, 128, 512
    wg, wu = dev_u8(_weights(rng, "q4_k", N, K), dev), dev_u8(_weights(rng, "q6_k", N, K), dev)
    xb, _ = _x(rng, M, K)
    x16, sc = ops.row_scale_f16(dev_bf16(xb, dev))
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    launch.launch("g_gemm_q4_k_q6_k_swiglu", [M, N], [M, K, N, x16, sc, wg, wu, y])
    want = ops.gemm("q4_k+q6_k", "swiglu", x16, wg, N, K, w2=wu, scales=sc)
    np.testing.assert_array_equal(host(y).view(np.uint32), host(want).view(np.uint32))
