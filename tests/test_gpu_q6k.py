"""GPU parity of the Q6_K format (the ffn_down tensors of the Q4_K_M files: Qwen3-8B ffn_down [4096 x 12288],
Qwen3-30B-A3B ffn_down_exps [128 x 2048 x 768]): bit-exact dequantization (@g_q6_k_values, S/gen_llm.py:320-397),
the decode matvecs on f32 / bf16 activations and on Q8_1 activations (@g_q6_k_icodes, S/gen_llm.py:617-690,
iq_dot :1036-1044), and the decode expert chain with Q4_K gate / up and Q6_K down.

Oracles: the bit-exact decoder oracle.formats.dequant_q6_k (pinned on the CPU against a scalar ggml-order decoder
and known-answer blocks) and float64 products. Matvecs: rel-L2 1e-3; multi-token calls equal one-token calls bit for
bit. K = 768 and 2816 make rows of an odd number of 210-byte super-blocks, so half the blocks start 2 bytes off a
4-byte boundary (the loader's realigned path).
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


def _x(rng, m, k, dtype, dev):
    from qmm.synth import to_bf16_bits
    x = rng.standard_normal((m, k)).astype(np.float32)
    if dtype == "bf16":
        b = to_bf16_bits(x)
        return dev_bf16(b, dev), bf16_values(b)
    return dev_f32(x, dev), x


@pytest.mark.parametrize("rows,k,sigma", [(64, 768, 0.002), (33, 2816, 0.5), (16, 12288, 40.0)])
def test_dequant_q6_k_bit_exact(dev, rows, k, sigma):
    from qmm import synth
    rng = np.random.default_rng(rows + k)
    w = synth.q6_k_weights(rng, rows, k, sigma=sigma)
    got = host(_ops().dequant("q6_k", dev_u8(w, dev), rows, k))
    assert_bits_equal(got, of.dequant_q6_k(w, rows, k), f"q6_k {rows}x{k}")


@pytest.mark.parametrize("n,k,m,dtype", [
    (4096, 12288, 1, "bf16"),     # Qwen3-8B ffn_down at decode
    (4096, 12288, 4, "bf16"),
    (2048, 768, 3, "f32"),        # Qwen3-30B-A3B expert down shape, misaligned blocks
    (37, 2816, 5, "bf16"),        # ragged rows, odd super-block count
    (50, 256, 2, "f32"),
])
def test_mv_q6_k_matches_oracle(dev, n, k, m, dtype):
    import torch
    from qmm import synth
    rng = np.random.default_rng(n + k + m)
    w = synth.q6_k_weights(rng, n, k)
    xt, xv = _x(rng, m, k, dtype, dev)
    y = host(_ops().mv("q6_k", dev_u8(w, dev), xt, n, k))
    torch.cuda.synchronize()
    assert_close_rel_l2(y, ref.gemv(xv, of.dequant_q6_k(w, n, k)), 1e-3, f"q6_k mv {n}x{k} m={m} {dtype}")


@pytest.mark.parametrize("n,k,m", [(4096, 12288, 1), (4096, 12288, 8), (2048, 768, 3), (37, 2816, 5)])
def test_mv_q8_q6_k_matches_oracle(dev, n, k, m):
    import torch
    from qmm import synth
    rng = np.random.default_rng(3 * n + k + m)
    w = synth.q6_k_weights(rng, n, k)
    xt, xv = _x(rng, m, k, "bf16", dev)
    y = host(_ops().mv_q8("q6_k", dev_u8(w, dev), xt, n, k))
    torch.cuda.synchronize()
    want = ref.gemv(ref.q8_1(xv), of.dequant_q6_k(w, n, k))
    assert_close_rel_l2(y, want, 1e-3, f"q6_k mv_q8 {n}x{k} m={m}")


@pytest.mark.parametrize("q8", [False, True])
def test_mv_q6_k_multi_token_equals_single_token(dev, q8):
    import torch
    from qmm import synth
    ops = _ops()
    rng = np.random.default_rng(11 + q8)
    n, k, m = 100, 2816, 5
    w = dev_u8(synth.q6_k_weights(rng, n, k), dev)
    xt, _ = _x(rng, m, k, "bf16", dev)
    f = ops.mv_q8 if q8 else ops.mv
    y = host(f("q6_k", w, xt, n, k))
    for t in range(m):
        assert_bits_equal(host(f("q6_k", w, xt[t:t + 1].contiguous(), n, k))[0], y[t], f"q6_k token {t}")
    torch.cuda.synchronize()


def test_mv_q6_k_accumulate_and_swiglu(dev):
    import torch
    from qmm import synth
    ops = _ops()
    rng = np.random.default_rng(12)
    n, k, m = 96, 1024, 3
    wg, wu = synth.q6_k_weights(rng, n, k), synth.q6_k_weights(rng, n, k)
    xt, xv = _x(rng, m, k, "f32", dev)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    yt = dev_f32(y0, dev)
    ops.mv("q6_k", dev_u8(wg, dev), xt, n, k, y=yt, accumulate=True)
    g = ref.gemv(xv, of.dequant_q6_k(wg, n, k))
    assert_close_rel_l2(host(yt), y0 + g, 1e-3, "q6_k accumulate")
    sw = host(ops.mv_swiglu("q6_k", dev_u8(wg, dev), dev_u8(wu, dev), xt, n, k))
    torch.cuda.synchronize()
    assert_close_rel_l2(sw, ref.silu_mul(g, ref.gemv(xv, of.dequant_q6_k(wu, n, k))), 1e-3, "q6_k swiglu")


@pytest.mark.parametrize("T", [1, 5])
def test_moe_decode_q4_k_gate_up_q6_k_down(dev, T):
    """The Qwen3-30B-A3B Q4_K_M expert layout at decode: 128 experts, top-8, H = 2048, FE = 768, gate / up Q4_K,
    down Q6_K (768 = 3 super-blocks: misaligned blocks in every other row)."""
    import torch
    from qmm import synth
    ops = _ops()
    E, KU, H, FE = 128, 8, 2048, 768
    rng = np.random.default_rng(40 + T)
    wg, wu = synth.q4_k_weights(rng, E * FE, H), synth.q4_k_weights(rng, E * FE, H)
    wd = synth.q6_k_weights(rng, E * H, FE)
    xb = synth.to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    logits = rng.standard_normal((T, E)).astype(np.float32)
    y, mid = ops.moe_decode("q4_k", dev_bf16(xb, dev), dev_f32(logits, dev), E, KU, H, FE, 1, True,
                            w_gate=dev_u8(wg, dev), w_up=dev_u8(wu, dev), w_down=dev_u8(wd, dev), fmt_down="q6_k",
                            q8=False)
    torch.cuda.synchronize()
    eids, ewts = ref.route(logits, KU, 1, True)
    np.testing.assert_array_equal(host(mid["ids"]), eids)
    rbg, rbd = of.row_bytes("q4_k", H), of.row_bytes("q6_k", FE)

    def gate_up(e):
        return (of.dequant_q4_k(wg[e * FE * rbg:(e + 1) * FE * rbg], FE, H),
                of.dequant_q4_k(wu[e * FE * rbg:(e + 1) * FE * rbg], FE, H))

    def down(e):
        return of.dequant_q6_k(wd[e * H * rbd:(e + 1) * H * rbd], H, FE)

    want, _ = ref.moe(bf16_values(xb), eids, ewts, gate_up, down)
    assert_close_rel_l2(host(y), want, 1e-3, f"q4_k/q6_k moe decode T={T}")


@pytest.mark.parametrize("M,N,K,mode,out", [
    (512, 4096, 12288, "store", "bf16"),   # Qwen3-8B ffn_down at a 512-token prefill
    (100, 200, 768, "store", "f32"),       # rows of 3 super-blocks: every other block 2 bytes off
    (64, 128, 2816, "acc", "f32"),
    (70, 96, 512, "swiglu", "f32"),
])
def test_gemm_q6_k(dev, M, N, K, mode, out):
    """g_gemm_q6_k_store (the reference's default GEMM formats, S/gen_gemm.py:2187): weights staged to f16 as
    fma_f16(f16(q), f16(d sc), f16(-32 d sc)) (S/gen_gemm.py:369-444), f16 row-scaled activations, fp32 accumulation.
    Oracle: float64 X16 W^T inv with W exactly dequantized (as the Q4_K GEMM), rel-L2 1e-3."""
    import torch
    from qmm import synth
    ops = _ops()
    rng = np.random.default_rng(M + N + K)
    w = synth.q6_k_weights(rng, N, K)
    xt, xv = _x(rng, M, K, "bf16", dev)
    xr = ref.f16_rows(xv)
    W = of.dequant_q6_k(w, N, K)
    dt = torch.bfloat16 if out == "bf16" else torch.float32
    if mode == "swiglu":
        w2 = synth.q6_k_weights(rng, N, K)
        y = ops.gemm("q6_k", "swiglu", xt, dev_u8(w, dev), N, K, w2=dev_u8(w2, dev))
        want = ref.silu_mul(ref.gemv(xr, W), ref.gemv(xr, of.dequant_q6_k(w2, N, K)))
    elif mode == "acc":
        y0 = rng.standard_normal((M, N)).astype(np.float32)
        y = dev_f32(y0, dev)
        ops.gemm("q6_k", "acc", xt, dev_u8(w, dev), N, K, y=y)
        want = y0 + ref.gemv(xr, W)
    else:
        y = ops.gemm("q6_k", "store", xt, dev_u8(w, dev), N, K, out_dtype=dt)
        want = ref.gemv(xr, W)
    got = host(y)
    torch.cuda.synchronize()
    assert_close_rel_l2(got, want, 1e-3 if out == "f32" else 4e-3, f"q6_k gemm {mode} {M}x{N}x{K}")


def test_moe_prefill_q4_k_gate_up_q6_k_down(dev):
    """The Qwen3-30B-A3B Q4_K_M expert layout at prefill (T = 64 takes the grouped chain): grouped Q4_K gate / up,
    grouped Q6_K down (K = 768, misaligned blocks)."""
    import torch
    from qmm import synth
    ops = _ops()
    E, KU, H, FE, T = 128, 8, 2048, 768, 64
    rng = np.random.default_rng(77)
    wg, wu = synth.q4_k_weights(rng, E * FE, H), synth.q4_k_weights(rng, E * FE, H)
    wd = synth.q6_k_weights(rng, E * H, FE)
    xb = synth.to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    logits = rng.standard_normal((T, E)).astype(np.float32)
    y, mid = ops.moe_prefill("q4_k", dev_bf16(xb, dev), dev_f32(logits, dev), E, KU, H, FE, 1, True,
                             w_gate=dev_u8(wg, dev), w_up=dev_u8(wu, dev), w_down=dev_u8(wd, dev), fmt_down="q6_k")
    torch.cuda.synchronize()
    eids, ewts = ref.route(logits, KU, 1, True)
    np.testing.assert_array_equal(host(mid["ids"]), eids)
    rbg, rbd = of.row_bytes("q4_k", H), of.row_bytes("q6_k", FE)

    def gate_up(e):
        return (of.dequant_q4_k(wg[e * FE * rbg:(e + 1) * FE * rbg], FE, H),
                of.dequant_q4_k(wu[e * FE * rbg:(e + 1) * FE * rbg], FE, H))

    def down(e):
        return of.dequant_q6_k(wd[e * H * rbd:(e + 1) * H * rbd], H, FE)

    want, _ = ref.moe(bf16_values(xb), eids, ewts, gate_up, down, x_round=ref.f16_rows, act_round=ref.f16_rows)
    assert_close_rel_l2(host(y), want, 1e-3, "q4_k/q6_k moe prefill")
