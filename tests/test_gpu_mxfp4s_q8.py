"""GPU parity of the reference's opt-in int8 decode of MXFP4 split planes (MXFP4S_Q8, S/formats.py:26-28): the matvec
g_mv_mxfp4s_k{K}[_t{TG}]_q8 (S/gen_llm.py:1288-1301 with @g_mxfp4s_icodes, S/gen_mxfp4s.py:1113-1160) and the MOE_Q8
expert matvecs of mxfp4s experts (S/gen_moe.py:535-727, S/gen_llm.py:5290-5303).

Oracles, as the reference's (make_kernel_tests.py:246-281, :3197-3214 with q8=True): float64 products of the Q8_1
activations q8_ref(x) with the exactly dequantized split planes (the int8 codes times 2^(e - 128) are those values
exactly: test_oracle_formats), and for the expert chain the gate/up output quantized again before the down matvecs;
bar rel-L2 <= 1e-3. Exactness properties: a multi-token call equals one-token calls bit for bit, f32 rows give the
bits of their planar Q8_1 buffer, a pair's rows equal the one-matrix kernel's bit for bit. Weights: random nibbles
(every E2M1 code, both signs, -0 included) with E8M0 scales 2^-8 .. 1, and the two subnormal scale bytes in a few
blocks.
"""
import numpy as np
import pytest

from helpers import assert_bits_equal, assert_close_rel_l2, dev_bf16, dev_f32, dev_u8, host
from oracle import formats as of
from oracle import ref

pytestmark = pytest.mark.gpu


def _planes(rng, rows, k):
    nib = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
    sc = (127 + rng.integers(-8, 1, (rows, k // 32))).astype(np.uint8)
    sc[0, 0], sc[-1, -1] = 0, 1   # d = 2^-128 and 2^-127 (f32 subnormals)
    return nib, sc


@pytest.mark.parametrize("n,k,m", [(2880, 2880, 1), (4096, 4096, 3), (16, 64, 1), (200, 1472, 5)])
def test_mv_q8_mxfp4s_matches_oracle(dev, n, k, m):
    import qmm.ops as ops
    rng = np.random.default_rng(n + k + m)
    nib, sc = _planes(rng, n, k)
    w, ws = dev_u8(nib, dev), dev_u8(sc, dev)
    x = rng.standard_normal((m, k)).astype(np.float32)
    xt = dev_f32(x, dev)
    xq = ops.quant_q8(xt)
    y = host(ops.mv_q8("mxfp4s", w, xq, n, k, tokens=m, ws=ws))
    assert_close_rel_l2(y, ref.gemv(ref.q8_1(x), of.dequant_mxfp4s(nib, sc, n, k)), 1e-3, f"mxfp4s mv_q8 {n}x{k}")
    assert_bits_equal(host(ops.mv_q8("mxfp4s", w, xt, n, k, ws=ws)), y, "f32 rows vs planar Q8_1")
    for t in range(m):
        assert_bits_equal(host(ops.mv_q8("mxfp4s", w, xt[t:t + 1].contiguous(), n, k, ws=ws))[0], y[t], f"token {t}")
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    ya = dev_f32(y0, dev)
    ops.mv_q8("mxfp4s", w, xq, n, k, tokens=m, y=ya, accumulate=True, ws=ws)
    assert_close_rel_l2(host(ya), y0 + y, 1e-6, "accumulate")


def test_swiglu_and_pair_q8_mxfp4s(dev):
    """The two-matrix forms on split planes: swiglu against the oracle, a pair's rows equal to the one-matrix
    kernel's bit for bit."""
    import qmm.ops as ops
    rng = np.random.default_rng(7)
    n, k, m = 512, 2880, 2
    (g, gs), (u, us) = _planes(rng, n, k), _planes(rng, n, k)
    G, Gs, U, Us = (dev_u8(a, dev) for a in (g, gs, u, us))
    from qmm import synth
    xb = synth.to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    xt = dev_bf16(xb, dev)
    xq = ref.q8_1(synth.bf16_bits_to_f32(xb))
    want = ref.silu_mul(ref.gemv(xq, of.dequant_mxfp4s(g, gs, n, k)), ref.gemv(xq, of.dequant_mxfp4s(u, us, n, k)))
    assert_close_rel_l2(host(ops.mv_swiglu_q8("mxfp4s", G, U, xt, n, k, ws=Gs, ws2=Us)), want, 1e-3, "swiglu")
    y, y2 = ops.mv_pair_q8("mxfp4s", G, U, xt, n, k, ws=Gs, ws2=Us)
    assert_bits_equal(host(y), host(ops.mv_q8("mxfp4s", G, xt, n, k, ws=Gs)), "pair y")
    assert_bits_equal(host(y2), host(ops.mv_q8("mxfp4s", U, xt, n, k, ws=Us)), "pair y2")


@pytest.mark.parametrize("T,fused", [(1, True), (2, False)])
def test_moe_decode_q8_mxfp4s_experts(dev, T, fused):
    """The int8 decode chain on mxfp4s experts at the gpt-oss-20b expert shape (32 experts, top-4, H = FE = 2880;
    without the expert biases the reference's int8 path requires): the router input quantized once, gate/up int8
    expert matvecs (a fused gate_up tensor or two tensors), their output quantized, int8 down matvecs, combine."""
    import torch
    import qmm.ops as ops
    E, KU, H, FE = 32, 4, 2880, 2880
    rng = np.random.default_rng(300 + T)
    if fused:
        gu, gus = _planes(rng, E * 2 * FE, H)
        kw = {"w_gate": dev_u8(gu, dev), "ws_gate": dev_u8(gus, dev)}
        gate_rows = lambda e: (slice(2 * FE * e, 2 * FE * e + FE), slice(2 * FE * e + FE, 2 * FE * (e + 1)))
        gp, gps, up, ups = gu, gus, gu, gus
    else:
        (gp, gps), (up, ups) = _planes(rng, E * FE, H), _planes(rng, E * FE, H)
        kw = {"w_gate": dev_u8(gp, dev), "ws_gate": dev_u8(gps, dev), "w_up": dev_u8(up, dev),
              "ws_up": dev_u8(ups, dev)}
        gate_rows = lambda e: (slice(FE * e, FE * (e + 1)), slice(FE * e, FE * (e + 1)))
    dn, dns = _planes(rng, E * H, FE)
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    y, mid = ops.moe_decode("mxfp4s", dev_f32(x, dev), dev_f32(logits, dev), E, KU, H, FE, 3, False,
                            w_down=dev_u8(dn, dev), ws_down=dev_u8(dns, dev), fused=fused, act="swiglu_oai", q8=True,
                            **kw)
    torch.cuda.synchronize()
    eids, ewts = ref.route(logits, KU, 3, False)
    np.testing.assert_array_equal(host(mid["ids"]), eids)

    def gate_up(e):
        rg, ru = gate_rows(e)
        return (of.dequant_mxfp4s(gp[rg], gps[rg], FE, H), of.dequant_mxfp4s(up[ru], ups[ru], FE, H))

    down = lambda e: of.dequant_mxfp4s(dn[H * e:H * (e + 1)], dns[H * e:H * (e + 1)], H, FE)
    want, acts = ref.moe(x, eids, ewts, gate_up, down, act="swiglu_oai", x_round=ref.q8_1, act_round=ref.q8_1)
    assert_close_rel_l2(host(mid["act"]), acts, 1e-3, f"mxfp4s q8 gate/up T={T}")
    assert_close_rel_l2(host(y), want, 1e-3, f"mxfp4s q8 moe decode T={T}")


def test_mxfp4s_q8_name_through_launch(dev):
    """g_mv_mxfp4s_k2880_q8 with the reference's split-plane arguments (n, tokens, accumulate, x, w, ws, y) equals
    ops.mv_q8 bit for bit; the split planes have no swiglu matvec in the reference, and the launcher says so."""
    import torch
    import qmm.ops as ops
    from qmm import launch
    rng = np.random.default_rng(73)
    n, k, T = 512, 2880, 2
    nib, sc = _planes(rng, n, k)
    w, ws = dev_u8(nib, dev), dev_u8(sc, dev)
    xt = dev_f32(rng.standard_normal((T, k)).astype(np.float32), dev)
    xq = ops.quant_q8(xt)
    y = torch.zeros((T, n), dtype=torch.float32, device=dev)
    L = launch.Launcher(launch.Config())
    L.launch("g_mv_mxfp4s_k2880_t2_q8", [n, T], [n, T, 0, xq, w, ws, y])
    assert_bits_equal(host(y), host(ops.mv_q8("mxfp4s", w, xt, n, k, ws=ws)), "g_mv_mxfp4s_k2880_q8")
    with pytest.raises(KeyError):
        L.launch("g_mv_mxfp4s_k2880_swiglu_q8", [n, T], [n, T, 0, xq, w, w, y])
