"""GPU regression tests for fixed defects and negative controls.

- The MXFP4 split-plane grouped GEMMs stage (64 + 256) x K / 32 scale bytes in dynamic LDS; a launch above the
  default limit raises the kernel's limit once per device, to the largest K the kernel takes, so a call at K = 4096
  followed by one at K = 8192 in the same process both launch (they must equal the MFMA-tiled planes' results, which
  stage no weight scales, bit for bit).
- The E8M0 scale of MXFP4 is 2^(e - 127) for split planes and ggml's 2^(e - 128) times the doubled E2M1 table for GGUF
  blocks (S/gen_llm.py:786-895, S/st_tensors.py:17-33): the device values equal the oracle's bit for bit, and an
  oracle with the bias off by one is caught (every nonzero value differs).
"""
import numpy as np
import pytest

from helpers import assert_bits_equal, dev_u8, host
from oracle import formats as of
from oracle import ref

pytestmark = pytest.mark.gpu


def test_split_grouped_gemms_k4096_then_k8192_in_one_process(dev):
    import torch
    import qmm.ops as ops
    from qmm import synth
    E, KU, T, small = 2, 1, 8, 64
    rng = np.random.default_rng(90)
    ids = torch.from_numpy(np.array([[0], [1]] * (T // 2), np.int32)).to(dev)
    ti, rm, _ = ops.moe_bucket(ids, E)
    live = host(rm) >= 0   # rows without an assignment are not written by the grouped GEMMs
    for K in (4096, 8192):
        x = rng.standard_normal((T, K)).astype(np.float32)
        x8, xs = ops.quant_mxfp8(torch.from_numpy(x).to(dev))
        # gate/up: n = 64 outputs of K = H inputs; down: n = 64 outputs of K = FE inputs (rows sorted in place)
        gu = synth.mxfp4_weights(rng, E * 2 * small, K)
        dn = synth.mxfp4_weights(rng, E * small, K)
        gn, gs = ops.repack_mxfp4(dev_u8(gu, dev), E * 2 * small, K)
        dnn, dns = ops.repack_mxfp4(dev_u8(dn, dev), E * small, K)
        gt, gst = ops.tile_mxfp4(gn, gs, E * 2 * small, K)
        dt, dst = ops.tile_mxfp4(dnn, dns, E * small, K)
        a_s = ops.moe_grouped("mxfp4s", "gu", ti, rm, x8, gn, small, K, E, KU, ws=gs, x_scales=xs, fused=True)
        a_t = ops.moe_grouped("mxfp4t", "gu", ti, rm, x8, gt, small, K, E, KU, ws=gst, x_scales=xs, fused=True)
        assert_bits_equal(host(a_s)[live], host(a_t)[live], f"gu K={K}")
        rows = ti.shape[0] * 64
        xd = rng.standard_normal((rows, K)).astype(np.float32)
        d8, ds8 = ops.quant_mxfp8(torch.from_numpy(xd).to(dev))
        y_s = ops.moe_grouped("mxfp4s", "dn", ti, rm, d8, dnn, small, K, E, KU, ws=dns, x_scales=ds8)
        y_t = ops.moe_grouped("mxfp4t", "dn", ti, rm, d8, dt, small, K, E, KU, ws=dst, x_scales=ds8)
        assert_bits_equal(host(y_s)[live], host(y_t)[live], f"dn K={K}")
        # and the oracle on one expert's rows: the first live tile row of expert 0
        W = of.dequant_mxfp4(gu[:small * of.row_bytes("mxfp4", K)], small, K)
        r0 = int(host(rm)[0])
        g0 = ref.gemv(ref.mxfp8_values(x[r0 // KU:r0 // KU + 1]), W)[0]
        U = of.dequant_mxfp4(gu[small * of.row_bytes("mxfp4", K):2 * small * of.row_bytes("mxfp4", K)], small, K)
        u0 = ref.gemv(ref.mxfp8_values(x[r0 // KU:r0 // KU + 1]), U)[0]
        np.testing.assert_allclose(host(a_s)[0], ref.silu_mul(g0, u0), rtol=2e-3, atol=2e-3 * np.abs(g0).max())


def test_e8m0_bias_negative_control(dev):
    import qmm.ops as ops
    from qmm import synth
    rows, K = 64, 256
    rng = np.random.default_rng(91)
    raw = synth.mxfp4_weights(rng, rows, K, e_lo=-20, e_hi=20)
    got = host(ops.dequant("mxfp4", dev_u8(raw, dev), rows, K))
    assert_bits_equal(got, of.dequant_mxfp4(raw, rows, K), "GGUF MXFP4 values")
    nib, sc = of.mxfp4_to_split(raw, rows, K)
    got_s = host(ops.dequant("mxfp4s", dev_u8(nib, dev), rows, K, ws=dev_u8(sc, dev)))
    want_s = of.dequant_mxfp4s(nib, sc, rows, K)
    assert np.array_equal(np.abs(got_s), np.abs(want_s)), "split-plane values"
    # an oracle with the exponent bias off by one (2^(e - 126) or 2^(e - 128)) differs in every nonzero value
    nz = want_s != 0
    for shift in (1, -1):
        wrong = of.dequant_mxfp4s(nib, (sc.astype(np.int32) + shift).astype(np.uint8), rows, K)
        assert np.all(np.abs(wrong[nz]) != np.abs(got_s[nz])), f"a bias off by {shift} went unnoticed"
