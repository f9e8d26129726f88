"""GPU parity of the int8-activation matvecs beyond the one-matrix GEMV: the swiglu and pair matvecs
(g_mv_{fmt}_k{K}_{swiglu|pair}[_t{TG}]_q8, S/gen_llm.py:1159-1197) and the decode expert matvecs of the MOE_Q8 chain
(g_moe_{gu|dn}_{fmt}_q8_k{K}_r{R}, S/gen_moe.py:535-727, S/gen_llm.py:5290-5303).

Oracles, as the reference's (make_kernel_tests.py:246-281, :3197-3214 with q8=True): float64 products of the Q8_1
activations q8_ref(x) (codes times the f16-rounded d) with exactly dequantized weights, silu(g) u for swiglu, and for
the expert chain the gate/up output quantized again before the down matvec; bar rel-L2 <= 1e-3. Exactness properties
(make_kernel_tests.py:264-268): a pair's rows equal the one-matrix kernel's bit for bit, a multi-token call equals
one-token calls bit for bit, and staging f32 / bf16 rows in the kernel equals passing qmm_quant_q8's planar buffer.
"""
import numpy as np
import pytest

from helpers import assert_bits_equal, assert_close_rel_l2, dev_bf16, dev_f32, dev_u8, host
from oracle import formats as of
from oracle import ref

pytestmark = pytest.mark.gpu


def _gate_up(dev, fmt, N, K, seed, tiled=False):
    import qmm.ops as ops
    from qmm import synth
    rng = np.random.default_rng(seed)
    g, u = synth.weights(fmt, rng, N, K), synth.weights(fmt, rng, N, K)
    gt, ut = dev_u8(g, dev), dev_u8(u, dev)
    if tiled:
        gt, ut = ops.tile_q4k(gt, N, K), ops.tile_q4k(ut, N, K)
    return gt, ut, of.dequantize(fmt, g, N, K), of.dequantize(fmt, u, N, K), rng


@pytest.mark.parametrize("M", [1, 4, 8])
def test_swiglu_q8_tiled_qwen3_8b_shape(dev, M):
    """silu(x Wg^T) (x Wu^T) at the Qwen3-8B FFN shape (N = 12288, K = 4096), gate and up in the tiled layout."""
    import qmm.ops as ops
    from qmm import synth
    N, K = 12288, 4096
    gt, ut, Wg, Wu, rng = _gate_up(dev, "q4_k", N, K, seed=80 + M, tiled=True)
    xb = synth.to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    xt = dev_bf16(xb, dev)
    xq = ref.q8_1(synth.bf16_bits_to_f32(xb))
    want = ref.silu_mul(ref.gemv(xq, Wg), ref.gemv(xq, Wu))
    y = host(ops.mv_swiglu_q8("q4_kt", gt, ut, xt, N, K))
    assert_close_rel_l2(y, want, 1e-3, f"swiglu_q8 M={M}")
    # the planar Q8_1 input gives the same bits as rows quantized inside the kernel
    yp = host(ops.mv_swiglu_q8("q4_kt", gt, ut, ops.quant_q8(xt), N, K, tokens=M))
    assert_bits_equal(yp, y, "planar input vs staged rows")
    # every token of a multi-token call equals its one-token call
    for t in range(M):
        assert_bits_equal(host(ops.mv_swiglu_q8("q4_kt", gt, ut, xt[t:t + 1].contiguous(), N, K)), y[t:t + 1],
                          f"token {t} alone")


@pytest.mark.parametrize("M,K", [(1, 4096), (3, 4096), (2, 8192)])
def test_pair_q8_tiled_equals_single_matvecs(dev, M, K):
    """y = x W^T and y2 = x W2^T in one launch are the one-matrix kernel's results bit for bit."""
    import qmm.ops as ops
    from qmm import synth
    N = 1024
    wt, w2t, W, W2, rng = _gate_up(dev, "q4_k", N, K, seed=90 + M + K, tiled=True)
    xt = dev_bf16(synth.to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32)), dev)
    y, y2 = ops.mv_pair_q8("q4_kt", wt, w2t, xt, N, K)
    assert_bits_equal(host(y), host(ops.mv_q8("q4_kt", wt, xt, N, K)), "pair y")
    assert_bits_equal(host(y2), host(ops.mv_q8("q4_kt", w2t, xt, N, K)), "pair y2")
    xq = ref.q8_1(host(xt))
    assert_close_rel_l2(host(y2), ref.gemv(xq, W2), 1e-3, "pair y2 vs oracle")


@pytest.mark.parametrize("fmt", ["q4_k", "q4_0", "q6_k"])
def test_swiglu_and_pair_q8_gguf_layouts(dev, fmt):
    """The GGUF-layout two-matrix matvecs (planar Q8_1 input) against the oracle; pair rows equal the one-matrix
    generic kernel's (K = 2048) bit for bit; accumulate adds into y."""
    import qmm.ops as ops
    from qmm import synth
    N, K, M = 512, 2048, 3
    wt, w2t, W, W2, rng = _gate_up(dev, fmt, N, K, seed=100 + len(fmt))
    x = rng.standard_normal((M, K)).astype(np.float32)
    xt = dev_f32(x, dev)
    xq = ref.q8_1(x)
    g, u = ref.gemv(xq, W), ref.gemv(xq, W2)
    y = host(ops.mv_swiglu_q8(fmt, wt, w2t, xt, N, K))
    assert_close_rel_l2(y, ref.silu_mul(g, u), 1e-3, f"{fmt} swiglu_q8")
    yp, yp2 = ops.mv_pair_q8(fmt, wt, w2t, xt, N, K)
    assert_bits_equal(host(yp), host(ops.mv_q8(fmt, wt, xt, N, K)), f"{fmt} pair y")
    assert_close_rel_l2(host(yp2), u, 1e-3, f"{fmt} pair y2")
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    ya = dev_f32(y0, dev)
    ops.mv_swiglu_q8(fmt, wt, w2t, xt, N, K, y=ya, accumulate=True)
    assert_close_rel_l2(host(ya), ref.silu_mul(g, u) + y0, 1e-3, f"{fmt} swiglu_q8 accumulate")


@pytest.mark.parametrize("T,fmt_down", [(1, None), (4, None), (4, "q6_k"), (16, None)])
def test_moe_decode_q8_chain_qwen3_30b_a3b(dev, T, fmt_down):
    """The int8 decode chain at the Qwen3-30B-A3B shape (128 experts, top-8, H = 2048, FE = 768): the router input
    quantized once, gate/up int8 expert matvecs with SwiGLU, their output quantized, int8 down matvecs (Q4_K, or the
    Q4_K_M files' Q6_K down), combine."""
    import torch
    import qmm.ops as ops
    from qmm import synth
    E, KU, H, FE = 128, 8, 2048, 768
    rng = np.random.default_rng(20261250 + T)
    fd = fmt_down or "q4_k"
    g, u = synth.q4_k_weights(rng, E * FE, H), synth.q4_k_weights(rng, E * FE, H)
    d = synth.weights(fd, rng, E * H, FE)
    xb = synth.to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    logits = rng.standard_normal((T, E)).astype(np.float32)
    y, mid = ops.moe_decode("q4_k", dev_bf16(xb, dev), dev_f32(logits, dev), E, KU, H, FE, 1, True,
                            w_gate=dev_u8(g, dev), w_up=dev_u8(u, dev), w_down=dev_u8(d, dev), fmt_down=fmt_down,
                            q8=True)
    torch.cuda.synchronize()
    eids, ewts = ref.route(logits, KU, 1, True)
    np.testing.assert_array_equal(host(mid["ids"]), eids)
    rb_h, rb_f = of.row_bytes("q4_k", H), of.row_bytes(fd, FE)
    gate_up = lambda e: (of.dequant_q4_k(g[FE * e * rb_h:FE * (e + 1) * rb_h], FE, H),
                         of.dequant_q4_k(u[FE * e * rb_h:FE * (e + 1) * rb_h], FE, H))
    down = lambda e: of.dequantize(fd, d[H * e * rb_f:H * (e + 1) * rb_f], H, FE)
    want, acts = ref.moe(synth.bf16_bits_to_f32(xb), eids, ewts, gate_up, down, act="silu", x_round=ref.q8_1,
                         act_round=ref.q8_1)
    assert_close_rel_l2(host(mid["act"]), acts, 1e-3, f"q8 gate/up T={T}")
    assert_close_rel_l2(host(y), want, 1e-3, f"q8 moe decode T={T} down={fd}")


def test_moe_expert_mv_q8_q4_0_fused_oai_biases(dev):
    """Q4_0 experts with a fused gate_up tensor, swiglu_oai and expert biases (more than the reference's int8 path
    takes, which has no biases): gu and dn against the oracle on the same Q8_1 inputs."""
    import torch
    import qmm.ops as ops
    from qmm import synth
    E, KU, H, FE, T = 8, 2, 512, 256, 3
    rng = np.random.default_rng(61)
    gu = synth.q4_0_weights(rng, E * 2 * FE, H)
    dw = synth.q4_0_weights(rng, E * H, FE)
    bg, bu, bd = (rng.standard_normal((E, n)).astype(np.float32) for n in (FE, FE, H))
    ids = rng.integers(0, E, (T, KU)).astype(np.int32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    it = torch.from_numpy(ids).to(dev)
    a = host(ops.moe_expert_mv_q8("q4_0", "gu", it, dev_f32(x, dev), dev_u8(gu, dev), FE, H, E, KU, fused=True,
                                  act="swiglu_oai", bias=dev_f32(bg, dev), bias2=dev_f32(bu, dev)))
    rb = of.row_bytes("q4_0", H)
    xq = ref.q8_1(x)
    want = np.zeros((T * KU, FE))
    for t in range(T):
        for k in range(KU):
            e = ids[t, k]
            Wg = of.dequant_q4_0(gu[2 * FE * e * rb:(2 * FE * e + FE) * rb], FE, H)
            Wu = of.dequant_q4_0(gu[(2 * FE * e + FE) * rb:2 * FE * (e + 1) * rb], FE, H)
            want[t * KU + k] = ref.swiglu_oai(ref.gemv(xq[t:t + 1], Wg)[0] + bg[e], ref.gemv(xq[t:t + 1], Wu)[0] + bu[e])
    assert_close_rel_l2(a, want, 1e-3, "q4_0 gu q8")
    ys = host(ops.moe_expert_mv_q8("q4_0", "dn", it, dev_f32(a, dev), dev_u8(dw, dev), H, FE, E, KU,
                                   bias=dev_f32(bd, dev)))
    rbf = of.row_bytes("q4_0", FE)
    aq = ref.q8_1(a)
    wd = np.stack([ref.gemv(aq[i:i + 1], of.dequant_q4_0(dw[H * ids.ravel()[i] * rbf:H * (ids.ravel()[i] + 1) * rbf],
                                                          H, FE))[0] + bd[ids.ravel()[i]] for i in range(T * KU)])
    assert_close_rel_l2(ys, wd, 1e-3, "q4_0 dn q8")
