"""GPU parity of the MXFP4 dense prefill GEMM on the gfx950 scaled MFMA (qmm_gemm_mxfp4; the reference's
g_gemm_mxfp4s_{store|swiglu}_f8_m256, S/gen_mxfp4s.py:50-101, and the MXFP4 helper GEMMs of S/gen_gemm.py:40).

The activation is quantized to MXFP8 (E4M3 with one E8M0 per 32 values, the quantizer qmm_quant_mxfp8 whose bytes the
oracle's mxfp8_quantize reproduces), so the oracle is float64 mxfp8_values(x) W^T with W exactly dequantized
(make_kernel_tests.py:1858-1900 with this path's activation rounding); bar rel-L2 <= 1e-3, a bf16 store equal to the
f32 result rounded to nearest even. Split planes and MFMA-tiled planes give the same bits.
"""
import numpy as np
import pytest

from helpers import assert_close_rel_l2, dev_bf16, dev_f32, dev_u8, host
from oracle import formats as of
from oracle import ref

pytestmark = pytest.mark.gpu


def _weights(dev, rng, N, K):
    import qmm.ops as ops
    from qmm import synth
    raw = synth.mxfp4_weights(rng, N, K)
    nib, sc = ops.repack_mxfp4(dev_u8(raw, dev), N, K)
    nt, st = ops.tile_mxfp4(nib, sc, N, K)
    return raw, (nib, sc), (nt, st), of.dequant_mxfp4(raw, N, K)


@pytest.mark.parametrize("M,N,K", [(512, 2880, 2880), (100, 160, 320), (64, 5760, 2880)])
def test_mxfp4_gemm_store(dev, M, N, K):
    import torch
    import qmm.ops as ops
    from qmm import synth
    rng = np.random.default_rng(M + N + K)
    raw, (nib, sc), (nt, st), W = _weights(dev, rng, N, K)
    xb = synth.to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    xt = dev_bf16(xb, dev)
    want = ref.gemv(ref.mxfp8_values(synth.bf16_bits_to_f32(xb)), W)
    ys = host(ops.gemm("mxfp4s", "store", xt, nib, N, K, ws=sc))
    yt = host(ops.gemm("mxfp4t", "store", xt, nt, N, K, ws=st))
    assert_close_rel_l2(ys, want, 1e-3, f"mxfp4 gemm {M}x{N}x{K}")
    assert np.array_equal(ys.view(np.uint32), yt.view(np.uint32)), "tiled planes differ from split planes"
    y16 = host(ops.gemm("mxfp4t", "store", xt, nt, N, K, ws=st, out_dtype=torch.bfloat16))
    assert np.array_equal(ref.bf16_round(yt).view(np.uint32), y16.view(np.uint32)), "bf16 store is not RNE(f32)"


def test_mxfp4_gemm_acc_swiglu_and_linear(dev):
    """acc adds into y; swiglu = silu(x Wg^T) (x Wu^T); linear() sends 64+ rows of GGUF mxfp4 weights to the GEMM
    (repacking them to split planes) and of split planes straight to it."""
    import qmm.ops as ops
    from qmm import synth
    M, N, K = 96, 256, 640
    rng = np.random.default_rng(11)
    raw, (nib, sc), (nt, st), W = _weights(dev, rng, N, K)
    raw2, (nib2, sc2), (nt2, st2), W2 = _weights(dev, rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    xt = dev_f32(x, dev)
    xq = ref.mxfp8_values(x)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    yt = dev_f32(y0, dev)
    ops.gemm("mxfp4s", "acc", xt, nib, N, K, ws=sc, y=yt)
    assert_close_rel_l2(host(yt), ref.gemv(xq, W) + y0, 1e-3, "mxfp4 acc")
    ysw = host(ops.gemm("mxfp4t", "swiglu", xt, nt, N, K, ws=st, w2=nt2, ws2=st2))
    assert_close_rel_l2(ysw, ref.silu_mul(ref.gemv(xq, W), ref.gemv(xq, W2)), 1e-3, "mxfp4 swiglu")
    yl = host(ops.linear("mxfp4", xt, dev_u8(raw, dev), N, K))
    assert_close_rel_l2(yl, ref.gemv(xq, W), 1e-3, "linear on GGUF mxfp4")
    yl2 = host(ops.linear("mxfp4s", xt, nib, N, K, ws=sc))
    assert np.array_equal(yl.view(np.uint32), yl2.view(np.uint32))


def test_mxfp4_gemm_partial_rows_write_nothing_past_m(dev):
    """Rows M..63 of the last tile and columns of the padded block are not written (a sentinel survives)."""
    import torch
    import qmm.ops as ops
    M, N, K = 70, 96, 128
    rng = np.random.default_rng(3)
    raw, (nib, sc), _, W = _weights(dev, rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    big = torch.full((M + 8, N), 7.25, dtype=torch.float32, device=dev)
    y = big[:M]
    ops.gemm("mxfp4s", "store", dev_f32(x, dev), nib, N, K, ws=sc, y=y)
    b = host(big)
    assert np.all(b[M:] == 7.25), "rows past M were written"
    assert_close_rel_l2(b[:M], ref.gemv(ref.mxfp8_values(x), W), 1e-3, "partial tile")
