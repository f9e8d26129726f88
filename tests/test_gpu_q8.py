"""GPU parity of the int8-activation decode path (the reference's default, S/gen_llm.py:519): the Q8_1 quantizer
g_quant_q8 (S/gen_llm.py:684-749) and the g_mv_{fmt}_k{K}[_t{TG}]_q8 matvecs (S/gen_llm.py:1288-1301).

The quantizer must reproduce the oracle's planar buffer byte for byte (codes, f16-rounded d, code sums; the oracle is
llama.cpp quantize_q8_1 in f32, make_kernel_tests.py:32-39). The matvec must match the float64 oracle on the Q8_1
activations (codes x f16 d) and the exactly dequantized weights within rel-L2 1e-3 (the reference's q8 tests compare
against the same q8_ref-quantized activations, make_kernel_tests.py:246-281). Bit-exact checks: the Q4_K kernel that
quantizes f32 / bf16 rows itself equals quant_q8 + the planar kernel, and multi-token calls equal one-token calls
(make_kernel_tests.py:264-268). Shapes: the Q4_K GEMV workload (12288 x 4096, M = 1, 4, 8), K = 8192, the generic
kernel (K = 2048, ragged rows) and Q4_0 (the 4096 x 4096 workload and a small shape).
"""
import numpy as np
import pytest

from helpers import assert_bits_equal, assert_close_rel_l2, bf16_values, dev_bf16, dev_f32, dev_u8, host
from oracle import formats as of
from oracle import ref

pytestmark = pytest.mark.gpu


def _ops():
    import qmm.ops as ops
    return ops


def _weights(fmt, rng, n, k):
    from qmm import synth
    return synth.q4_k_weights(rng, n, k) if fmt == "q4_k" else synth.q4_0_weights(rng, n, k)


def _x(rng, m, k, dtype, dev):
    """(device tensor, its f32 values) of m rows of N(0, 1) activations in f32 or bf16."""
    from qmm.synth import to_bf16_bits
    x = rng.standard_normal((m, k)).astype(np.float32)
    if dtype == "bf16":
        b = to_bf16_bits(x)
        return dev_bf16(b, dev), bf16_values(b)
    return dev_f32(x, dev), x


@pytest.mark.parametrize("rows,k,dtype", [(1, 4096, "bf16"), (8, 4096, "f32"), (3, 96, "f32"), (5, 2880, "bf16")])
def test_quant_q8_matches_oracle_bytes(dev, rows, k, dtype):
    """Rows scaled over 2^-6 .. 2^6, a zero group and exact halves (x/d = +-2.5 rounds away from zero)."""
    import torch
    from qmm.synth import to_bf16_bits
    rng = np.random.default_rng(rows + k)
    x = (rng.standard_normal((rows, k)) * np.exp(rng.uniform(-6, 6, (rows, 1)))).astype(np.float32)
    x[0, :32] = 0.0
    x[-1, 32:64] = 0.0
    x[-1, 32], x[-1, 33], x[-1, 34] = 127.0, 2.5, -2.5
    if dtype == "bf16":
        b = to_bf16_bits(x)
        xt, xv = dev_bf16(b, dev), bf16_values(b)
    else:
        xt, xv = dev_f32(x, dev), x
    got = host(_ops().quant_q8(xt))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got, ref.q8_planar(xv))


@pytest.mark.parametrize("fmt,n,k,m,dtype", [
    ("q4_k", 12288, 4096, 1, "bf16"),     # the Q4_K GEMV workload, activations quantized by the kernel
    ("q4_k", 12288, 4096, 4, "bf16"),
    ("q4_k", 12288, 4096, 8, "bf16"),
    ("q4_k", 77, 8192, 3, "f32"),         # two lanes per half row pass; ragged rows
    ("q4_k", 101, 2048, 5, "bf16"),       # the generic kernel (quant_q8 first)
    ("q4_0", 4096, 4096, 1, "f32"),       # the Q4_0 GEMV workload
    ("q4_0", 50, 1024, 3, "bf16"),
])
def test_mv_q8_matches_oracle(dev, fmt, n, k, m, dtype):
    import torch
    rng = np.random.default_rng(n + k + m)
    w = _weights(fmt, rng, n, k)
    xt, xv = _x(rng, m, k, dtype, dev)
    y = host(_ops().mv_q8(fmt, dev_u8(w, dev), xt, n, k))
    torch.cuda.synchronize()
    want = ref.gemv(ref.q8_1(xv), of.dequantize(fmt, w, n, k))
    assert_close_rel_l2(y, want, 1e-3, f"{fmt} mv_q8 n={n} k={k} m={m}")


@pytest.mark.parametrize("k", [4096, 8192])
def test_mv_q8_fused_quantization_equals_planar(dev, k):
    """f32 / bf16 rows quantized inside the Q4_K kernel give the same bits as quant_q8 + the planar kernel."""
    import torch
    ops = _ops()
    rng = np.random.default_rng(k)
    n, m = 96, 3
    w = dev_u8(_weights("q4_k", rng, n, k), dev)
    for dtype in ("bf16", "f32"):
        xt, _ = _x(rng, m, k, dtype, dev)
        fused = host(ops.mv_q8("q4_k", w, xt, n, k))
        planar = host(ops.mv_q8("q4_k", w, ops.quant_q8(xt), n, k, tokens=m))
        assert_bits_equal(fused, planar, f"k={k} {dtype}")
    torch.cuda.synchronize()


@pytest.mark.parametrize("fmt,k", [("q4_k", 4096), ("q4_k", 2048), ("q4_0", 1024)])
def test_mv_q8_multi_token_equals_single_token(dev, fmt, k):
    import torch
    ops = _ops()
    rng = np.random.default_rng(7)
    n, m = 100, 5
    w = dev_u8(_weights(fmt, rng, n, k), dev)
    xt, _ = _x(rng, m, k, "bf16", dev)
    y = host(ops.mv_q8(fmt, w, xt, n, k))
    for t in range(m):
        assert_bits_equal(host(ops.mv_q8(fmt, w, xt[t:t + 1].contiguous(), n, k))[0], y[t], f"{fmt} token {t}")
    torch.cuda.synchronize()


@pytest.mark.parametrize("k", [4096, 2048])
def test_mv_q8_accumulate(dev, k):
    import torch
    rng = np.random.default_rng(9)
    n, m = 64, 2
    w = _weights("q4_k", rng, n, k)
    xt, xv = _x(rng, m, k, "f32", dev)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    yt = dev_f32(y0, dev)
    _ops().mv_q8("q4_k", dev_u8(w, dev), xt, n, k, y=yt, accumulate=True)
    want = y0 + ref.gemv(ref.q8_1(xv), of.dequant_q4_k(w, n, k))
    assert_close_rel_l2(host(yt), want, 1e-3, f"accumulate k={k}")
    torch.cuda.synchronize()


def test_mv_q8_rejects_bad_arguments(dev):
    import torch
    from qmm import _lib
    w = torch.zeros(144 * 16, dtype=torch.uint8, device=dev)
    x = torch.zeros((1, 2048), dtype=torch.bfloat16, device=dev)
    y = torch.zeros((1, 1), dtype=torch.float32, device=dev)
    lib = _lib.load()
    s = torch.cuda.current_stream().cuda_stream
    # f32 / bf16 rows are quantized in-kernel only for Q4_K at K = 4096 / 8192
    assert lib.qmm_mv_q8(1, 2048, 1, 1, 0, x.data_ptr(), 2, w.data_ptr(), y.data_ptr(), s) == -2   # QMM_ERR_SHAPE
    assert lib.qmm_mv_q8(2, 2048, 1, 1, 0, x.data_ptr(), 4, w.data_ptr(), y.data_ptr(), s) == -1   # MXFP4: FORMAT
    assert lib.qmm_mv_q8(1, 300, 1, 1, 0, x.data_ptr(), 4, w.data_ptr(), y.data_ptr(), s) == -2    # K % 256
    assert lib.qmm_quant_q8(1, 40, x.data_ptr(), 2, w.data_ptr(), s) == -2                          # K % 32
    torch.cuda.synchronize()


# ------------------------------------------------------------------------------ Q4_K in the tiled GEMV layout
def test_tile_q4k_bit_exact(dev):
    """qmm_tile_q4k against the oracle's element-by-element construction; qmm_dequant of the tiled bytes against
    the GGUF values."""
    import torch
    ops = _ops()
    rng = np.random.default_rng(61)
    for n, k in ((32, 4096), (48, 1536), (32, 768), (16, 256)):   # 768, 256: a trailing half unit
        w = _weights("q4_k", rng, n, k)
        wt = ops.tile_q4k(dev_u8(w, dev), n, k)
        np.testing.assert_array_equal(host(wt), of.q4_k_to_tiled(w, n, k))
        got = host(ops.dequant("q4_kt", wt, n, k))
        assert_bits_equal(got, of.dequant_q4_k(w, n, k), f"q4_kt dequant {n}x{k}")
    torch.cuda.synchronize()


@pytest.mark.parametrize("m", [1, 2, 3, 8])
def test_mv_q8_tiled_equals_gguf_layout_at_k4096(dev, m):
    """At K = 4096 the tiled-layout GEMV does the GGUF-layout kernel's arithmetic in its order: identical bits, for
    activations quantized in the kernel and for planar Q8_1."""
    import torch
    ops = _ops()
    rng = np.random.default_rng(62 + m)
    n, k = 12288 if m == 1 else 320, 4096
    w = dev_u8(_weights("q4_k", rng, n, k), dev)
    wt = ops.tile_q4k(w, n, k)
    xt, _ = _x(rng, m, k, "bf16", dev)
    assert_bits_equal(host(ops.mv_q8("q4_kt", wt, xt, n, k)), host(ops.mv_q8("q4_k", w, xt, n, k)), f"m={m}")
    xq = ops.quant_q8(xt)
    assert_bits_equal(host(ops.mv_q8("q4_kt", wt, xq, n, k, tokens=m)), host(ops.mv_q8("q4_k", w, xq, n, k, tokens=m)),
                      f"planar m={m}")
    torch.cuda.synchronize()


@pytest.mark.parametrize("n,k,m,dtype", [
    (16, 512, 1, "bf16"),      # one wave, one slice
    (32, 512, 8, "bf16"),      # one wave, eight tokens: more outputs a workgroup (16 x 8) than threads
    (48, 1536, 3, "f32"),      # three waves
    (32, 5120, 2, "bf16"),     # two slices a wave, five waves
    (64, 8192, 5, "bf16"),     # two slices a wave, eight waves
    (16, 12288, 2, "f32"),     # three slices a wave
    (32, 16384, 3, "bf16"),    # four slices a wave (one token a workgroup)
])
def test_mv_q8_tiled_matches_oracle(dev, n, k, m, dtype):
    """Every slices-per-wave configuration against the float64 oracle on Q8_1 activations; a multi-token call
    equals one-token calls bit for bit; accumulate adds to y."""
    import torch
    ops = _ops()
    rng = np.random.default_rng(n + k + m)
    w = _weights("q4_k", rng, n, k)
    wt = ops.tile_q4k(dev_u8(w, dev), n, k)
    xt, xv = _x(rng, m, k, dtype, dev)
    y = host(ops.mv_q8("q4_kt", wt, xt, n, k))
    want = ref.gemv(ref.q8_1(xv), of.dequant_q4_k(w, n, k))
    assert_close_rel_l2(y, want, 1e-3, f"q4_kt mv_q8 n={n} k={k} m={m}")
    for t in range(m):
        assert_bits_equal(host(ops.mv_q8("q4_kt", wt, xt[t:t + 1].contiguous(), n, k))[0], y[t], f"token {t}")
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    yt = dev_f32(y0, dev)
    ops.mv_q8("q4_kt", wt, xt, n, k, y=yt, accumulate=True)
    assert_close_rel_l2(host(yt), y0 + want, 1e-3, "accumulate")
    torch.cuda.synchronize()


@pytest.mark.parametrize("m", [4, 8])
def test_mv_q8_tiled_in_kernel_quantization_equals_planar(dev, m):
    """Four and eight tokens a workgroup through the C ABI with bf16 rows (each workgroup quantizes them) equal
    quant_q8 + the planar kernel bit for bit."""
    import torch
    from qmm import _lib
    ops = _ops()
    rng = np.random.default_rng(70 + m)
    n, k = 64, 4096
    wt = ops.tile_q4k(dev_u8(_weights("q4_k", rng, n, k), dev), n, k)
    xt, _ = _x(rng, m, k, "bf16", dev)
    y = torch.empty((m, n), dtype=torch.float32, device=dev)
    _lib.call("qmm_mv_q8", 5, k, n, m, 0, xt.data_ptr(), 2, wt.data_ptr(), y.data_ptr(),
              torch.cuda.current_stream().cuda_stream)
    planar = host(ops.mv_q8("q4_kt", wt, ops.quant_q8(xt), n, k, tokens=m))
    assert_bits_equal(host(y), planar, f"m={m}")
    torch.cuda.synchronize()
