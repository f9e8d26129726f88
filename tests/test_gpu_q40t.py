"""GPU parity of Q4_0 in the tiled GEMV layout (qmm_tile_q40, format q4_0t): the int8-activation decode matvecs
g_mv_q4_0_k{K}[_t{TG}]_q8 and their swiglu / pair forms (S/gen_llm.py:1159-1197, :1288-1301; the Q4_0 int8 dot
@g_q4_0_icodes, S/gen_llm.py:536-552) read from the tiled units the Q4_K kernel streams, and the f32 / bf16-activation
matvec g_mv_q4_0_k{K}[_t{TG}] (the reference's default Q4_0 decode; @g_q4_0_values) on the same units.

Bars: the tiled bytes equal the oracle's construction byte for byte and dequantize to the GGUF values bit for bit;
the matvec matches the float64 oracle on the Q8_1 activations and the exactly dequantized weights within rel-L2 1e-3
(make_kernel_tests.py:246-281); a multi-token call equals one-token calls bit for bit; a pair equals two one-matrix
calls bit for bit; f32 / bf16 rows quantized in the kernel equal qmm_quant_q8's planar buffer. Against the GGUF-layout
kernel (the same per-block products summed in another order) the rel-L2 gap is far below the oracle bar. Weights:
random codes with scales of both signs.
"""
import numpy as np
import pytest

from helpers import assert_bits_equal, assert_close_rel_l2, bf16_values, dev_bf16, dev_f32, dev_u8, host
from oracle import formats as of
from oracle import ref

pytestmark = pytest.mark.gpu


def _w(rng, n, k):
    from qmm import synth
    raw = synth.q4_0_weights(rng, n, k).reshape(-1, 18).copy()
    raw[::3, 1] |= 0x80    # a third of the blocks with negative d
    return raw.reshape(-1)


def _x(rng, m, k, dtype, dev):
    from qmm.synth import to_bf16_bits
    x = rng.standard_normal((m, k)).astype(np.float32)
    if dtype == "bf16":
        b = to_bf16_bits(x)
        return dev_bf16(b, dev), bf16_values(b)
    return dev_f32(x, dev), x


def test_tile_q40_bit_exact(dev):
    """qmm_tile_q40 against the oracle's construction from the layout's definition; qmm_dequant of the tiled bytes
    against the GGUF values."""
    import qmm.ops as ops
    rng = np.random.default_rng(71)
    for n, k in ((16, 512), (48, 1536), (32, 4096)):
        w = _w(rng, n, k)
        wt = ops.tile_q40(dev_u8(w, dev), n, k)
        np.testing.assert_array_equal(host(wt), of.q4_0_to_tiled(w, n, k))
        assert_bits_equal(host(ops.dequant("q4_0t", wt, n, k)), of.dequant_q4_0(w, n, k), f"q4_0t dequant {n}x{k}")


@pytest.mark.parametrize("n,k,m,dtype", [
    (16, 512, 1, "bf16"),      # one wave, one unit
    (4096, 4096, 1, "f32"),    # the Q4_0 GEMV workload (4096 x 4096, one token)
    (48, 1536, 3, "f32"),      # three waves
    (64, 8192, 5, "bf16"),     # two units a wave, eight waves
    (32, 16384, 3, "bf16"),    # four units a wave
])
def test_mv_q8_q40t_matches_oracle(dev, n, k, m, dtype):
    import qmm.ops as ops
    rng = np.random.default_rng(n + k + m + 7)
    w = _w(rng, n, k)
    wg = dev_u8(w, dev)
    wt = ops.tile_q40(wg, n, k)
    xt, xv = _x(rng, m, k, dtype, dev)
    y = host(ops.mv_q8("q4_0t", wt, xt, n, k))
    want = ref.gemv(ref.q8_1(xv), of.dequant_q4_0(w, n, k))
    assert_close_rel_l2(y, want, 1e-3, f"q4_0t mv_q8 n={n} k={k} m={m}")
    for t in range(m):
        assert_bits_equal(host(ops.mv_q8("q4_0t", wt, xt[t:t + 1].contiguous(), n, k))[0], y[t], f"token {t}")
    xq = ops.quant_q8(xt)
    assert_bits_equal(host(ops.mv_q8("q4_0t", wt, xq, n, k, tokens=m)), y, "planar Q8_1 input")
    gguf = host(ops.mv_q8("q4_0", wg, xq, n, k, tokens=m))
    assert_close_rel_l2(y, gguf.astype(np.float64), 1e-5, "vs the GGUF-layout kernel")
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    yt = dev_f32(y0, dev)
    ops.mv_q8("q4_0t", wt, xt, n, k, y=yt, accumulate=True)
    assert_close_rel_l2(host(yt), y0 + want, 1e-3, "accumulate")


@pytest.mark.parametrize("m", [1, 4])
def test_swiglu_and_pair_q8_q40t(dev, m):
    """silu(x Wg^T) (x Wu^T) against the oracle; a pair's rows equal the one-matrix kernel's bit for bit."""
    import qmm.ops as ops
    rng = np.random.default_rng(90 + m)
    n, k = 1024, 4096
    g, u = _w(rng, n, k), _w(rng, n, k)
    gt, ut = ops.tile_q40(dev_u8(g, dev), n, k), ops.tile_q40(dev_u8(u, dev), n, k)
    xt, xv = _x(rng, m, k, "bf16", dev)
    xq = ref.q8_1(xv)
    want = ref.silu_mul(ref.gemv(xq, of.dequant_q4_0(g, n, k)), ref.gemv(xq, of.dequant_q4_0(u, n, k)))
    assert_close_rel_l2(host(ops.mv_swiglu_q8("q4_0t", gt, ut, xt, n, k)), want, 1e-3, f"swiglu m={m}")
    y, y2 = ops.mv_pair_q8("q4_0t", gt, ut, xt, n, k)
    assert_bits_equal(host(y), host(ops.mv_q8("q4_0t", gt, xt, n, k)), "pair y")
    assert_bits_equal(host(y2), host(ops.mv_q8("q4_0t", ut, xt, n, k)), "pair y2")


def test_linear_decode_reads_q40t(dev):
    """ops.linear on q4_0t weights takes the int8 matvec (Q8_1 activations, the reference's ACT_Q8 default)."""
    import qmm.ops as ops
    rng = np.random.default_rng(95)
    n, k = 256, 2048
    w = _w(rng, n, k)
    wt = ops.tile_q40(dev_u8(w, dev), n, k)
    xt, xv = _x(rng, 2, k, "f32", dev)
    got = host(ops.linear("q4_0t", xt, wt, n, k))
    assert_close_rel_l2(got, ref.gemv(ref.q8_1(xv), of.dequant_q4_0(w, n, k)), 1e-3, "linear q4_0t")


@pytest.mark.parametrize("n,k,m,dtype", [
    (4096, 4096, 1, "f32"),    # the Q4_0 GEMV workload (4096 x 4096, f32 x)
    (16, 512, 1, "bf16"),      # one wave, one unit
    (48, 1536, 3, "f32"),      # three waves
    (64, 8192, 2, "bf16"),     # two units a wave
    (32, 12288, 2, "f32"),     # three units a wave
])
def test_mv_f32_q40t_matches_oracle(dev, n, k, m, dtype):
    """The f32-activation matvec on the tiled units against the float64 oracle (f32 x, exactly dequantized weights,
    rel-L2 <= 1e-3, make_kernel_tests.py:246-281); a multi-token call equals one-token calls bit for bit; against
    the GGUF-layout f32 kernel (the same products, another summation order) far below the bar; accumulate adds."""
    import qmm.ops as ops
    rng = np.random.default_rng(n + k + m + 17)
    w = _w(rng, n, k)
    wg = dev_u8(w, dev)
    wt = ops.tile_q40(wg, n, k)
    xt, xv = _x(rng, m, k, dtype, dev)
    y = host(ops.mv("q4_0t", wt, xt, n, k))
    assert_close_rel_l2(y, ref.gemv(xv, of.dequant_q4_0(w, n, k)), 1e-3, f"q4_0t mv n={n} k={k} m={m}")
    for t in range(m):
        assert_bits_equal(host(ops.mv("q4_0t", wt, xt[t:t + 1].contiguous(), n, k))[0], y[t], f"token {t}")
    assert_close_rel_l2(y, host(ops.mv("q4_0", wg, xt, n, k)).astype(np.float64), 1e-5, "vs the GGUF-layout kernel")
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    yt = dev_f32(y0, dev)
    ops.mv("q4_0t", wt, xt, n, k, y=yt, accumulate=True)
    assert_close_rel_l2(host(yt), y0 + y, 1e-6, "accumulate")


def test_linear_f32_path_reads_q40t(dev):
    """ops.linear on q4_0t weights with q8=False (the reference's ACT_Q8=0 / default Q4_0 arithmetic) takes the
    f32-activation matvec."""
    import qmm.ops as ops
    rng = np.random.default_rng(96)
    n, k = 256, 2048
    w = _w(rng, n, k)
    wt = ops.tile_q40(dev_u8(w, dev), n, k)
    xt, xv = _x(rng, 2, k, "f32", dev)
    got = host(ops.linear("q4_0t", xt, wt, n, k, q8=False))
    assert_close_rel_l2(got, ref.gemv(xv, of.dequant_q4_0(w, n, k)), 1e-3, "linear q4_0t f32")
