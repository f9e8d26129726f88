"""GPU parity of the Q4_0 prefill GEMM (g_gemm_q4_0_*, the native Q4_0 tiles of S/gen_gemm.py:40-45) and the Q4_0
grouped expert GEMMs (specialize_grouped, S/moe_q4_0.py:41-61) on the f16 MFMA.

The staging itself is checked exhaustively, as the reference's own Q4_0 test does for its half multiply
(tests/test_moe_q4_0.py:24-33): every finite f16 scale (up to 8188, past which d (q - 8) leaves the f16 range) times
every code, read back through the GEMM with identity activation rows, must be the f16 product numpy rounds once,
bit for bit. Matmul outputs follow the reference's GEMM check (make_kernel_tests.py:1858-1900): float64 on exactly
dequantized weights with the f16 row-scaled activation, rel-L2 <= 1e-3; a bf16 store equals the f32 result rounded
to nearest even. The MoE chain is checked against experts_ref (make_kernel_tests.py:3197-3221) at the Qwen3-30B-A3B
shape with Q4_0 experts.
"""
import numpy as np
import pytest

from helpers import assert_close_rel_l2, dev_bf16, dev_f32, dev_u8, host
from oracle import formats as of
from oracle import ref

pytestmark = pytest.mark.gpu


def _q4_0_all_scales():
    """Q4_0 blocks holding every finite f16 scale d with |d| <= 8188 (so d (q - 8) stays finite) once, codes 0..15
    in values 0..15 (low nibbles) and again in values 16..31 (high nibbles); padded with d = 0 to whole rows of
    K = 256 (7168 rows). Returns (raw bytes, rows, expected f16 values as float32 [rows, 256])."""
    bits = np.arange(65536, dtype=np.uint16)
    d = bits.view(np.float16)
    d = d[np.isfinite(d) & (np.abs(d.astype(np.float32)) <= 8188)]
    K = 256
    blocks = -(-d.size // (K // 32)) * (K // 32)
    rows = blocks // (K // 32)
    dd = np.zeros(blocks, np.float16)
    dd[:d.size] = d
    raw = np.zeros((blocks, 18), np.uint8)
    raw[:, :2] = dd.view(np.uint8).reshape(-1, 2)
    j = np.arange(16, dtype=np.uint8)
    raw[:, 2:] = j | (j << 4)
    codes = np.concatenate([np.arange(16), np.arange(16)]).astype(np.float16) - np.float16(8)
    with np.errstate(over="ignore"):
        want = (dd[:, None] * codes[None, :]).astype(np.float16)   # one f16 rounding of the exact product
    # the GEMM's f32 accumulation starts from +0, so a -0 product (code 8 under a negative scale) reads back as +0
    return raw.reshape(-1), rows, want.astype(np.float32).reshape(rows, K) + np.float32(0.0)


def test_q4_0_staging_every_finite_scale(dev):
    import torch
    import qmm.ops as ops
    raw, rows, want = _q4_0_all_scales()
    K = 256
    eye = torch.eye(K, dtype=torch.float16, device=dev)
    y = host(ops.gemm("q4_0", "store", eye, dev_u8(raw, dev), rows, K))   # y[r, c] = W16[c, r]
    got = np.ascontiguousarray(y.T)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{bad.size} staged values differ, first at {bad[:5]}: {got.ravel()[bad[:5]]} vs " \
                          f"{want.ravel()[bad[:5]]}"
    # the negative control: staging with two roundings (f16(d) f16(q) then f16(-8 d)) would not pass
    d = raw.reshape(-1, 18)[:, :2].copy().view(np.float16)[:, 0]
    q = np.arange(16, dtype=np.float16)
    with np.errstate(over="ignore", invalid="ignore"):
        two = ((d[:, None] * q[None, :]).astype(np.float16) + (np.float16(-8) * d)[:, None]).astype(np.float16)
    assert not np.array_equal(two.astype(np.float32), want.reshape(-1, 32)[:, :16])


def _case(dev, M, N, K, seed):
    from qmm import synth
    rng = np.random.default_rng(seed)
    w = synth.q4_0_weights(rng, N, K)
    xb = synth.to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    W = of.dequant_q4_0(w, N, K)
    xv = synth.bf16_bits_to_f32(xb)
    return dev_u8(w, dev), dev_bf16(xb, dev), W, xv


def test_q4_0_gemm_workload_shape(dev):
    """512 x 4096 x 4096 (the Qwen3-8B o_proj shape) with Q4_0 weights: f32 and bf16 stores."""
    import torch
    import qmm.ops as ops
    M, N, K = 512, 4096, 4096
    wt, xt, W, xv = _case(dev, M, N, K, seed=40)
    want = ref.gemv(ref.f16_rows(xv), W)
    y32 = host(ops.gemm("q4_0", "store", xt, wt, N, K))
    y16 = host(ops.gemm("q4_0", "store", xt, wt, N, K, out_dtype=torch.bfloat16))
    assert_close_rel_l2(y32, want, 1e-3, "q4_0 gemm")
    assert np.array_equal(ref.bf16_round(y32).view(np.uint32), y16.view(np.uint32)), "bf16 store is not RNE(f32)"


@pytest.mark.parametrize("M,N,K", [(70, 200, 768), (130, 384, 1280)])
def test_q4_0_gemm_edges_acc_and_swiglu(dev, M, N, K):
    """Partial row / column tiles; acc adds to y; swiglu = silu(x Wg^T) (x Wu^T); linear() sends 64+ rows here."""
    import qmm.ops as ops
    from qmm import synth
    wt, xt, W, xv = _case(dev, M, N, K, seed=M + N)
    x16 = ref.f16_rows(xv)
    rng = np.random.default_rng(7)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    yt = dev_f32(y0, dev)
    ops.gemm("q4_0", "acc", xt, wt, N, K, y=yt)
    assert_close_rel_l2(host(yt), ref.gemv(x16, W) + y0, 1e-3, "q4_0 acc")
    w2 = synth.q4_0_weights(rng, N, K)
    W2 = of.dequant_q4_0(w2, N, K)
    ys = host(ops.gemm("q4_0", "swiglu", xt, wt, N, K, w2=dev_u8(w2, dev)))
    assert_close_rel_l2(ys, ref.silu_mul(ref.gemv(x16, W), ref.gemv(x16, W2)), 1e-3, "q4_0 swiglu")
    yl = host(ops.linear("q4_0", xt, wt, N, K))
    assert_close_rel_l2(yl, ref.gemv(x16, W), 1e-3, "q4_0 linear prefill")


def test_q4_0_moe_qwen3_30b_a3b_shape(dev):
    """The prefill chain with Q4_0 experts at the Qwen3-30B-A3B shape: 128 experts, top-8 (gating 1 + norm),
    H = 2048, FE = 768, T = 64, SwiGLU; grouped gate/up and down GEMMs with the Q4_0 staging."""
    import torch
    import qmm.ops as ops
    from qmm import synth
    E, KU, H, FE, T = 128, 8, 2048, 768, 64
    rng = np.random.default_rng(20261240)
    g, u, d = synth.q4_0_weights(rng, E * FE, H), synth.q4_0_weights(rng, E * FE, H), synth.q4_0_weights(rng, E * H, FE)
    xb = synth.to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    logits = rng.standard_normal((T, E)).astype(np.float32)
    y, mid = ops.moe_prefill("q4_0", dev_bf16(xb, dev), dev_f32(logits, dev), E, KU, H, FE, 1, True,
                             w_gate=dev_u8(g, dev), w_up=dev_u8(u, dev), w_down=dev_u8(d, dev))
    torch.cuda.synchronize()
    eids, ewts = ref.route(logits, KU, 1, True)
    np.testing.assert_array_equal(host(mid["ids"]), eids)
    rb_h, rb_f = of.row_bytes("q4_0", H), of.row_bytes("q4_0", FE)
    gate_up = lambda e: (of.dequant_q4_0(g[FE * e * rb_h:FE * (e + 1) * rb_h], FE, H),
                         of.dequant_q4_0(u[FE * e * rb_h:FE * (e + 1) * rb_h], FE, H))
    down = lambda e: of.dequant_q4_0(d[H * e * rb_f:H * (e + 1) * rb_f], H, FE)
    want, _ = ref.moe(synth.bf16_bits_to_f32(xb), eids, ewts, gate_up, down, act="silu", x_round=ref.f16_rows,
                      act_round=ref.f16_rows)
    assert_close_rel_l2(host(y), want, 1e-3, "q4_0 moe prefill")
