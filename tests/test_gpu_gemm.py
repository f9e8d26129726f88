"""GPU parity of the Q4_K prefill GEMM (g_gemm_q4_k_*, S/gen_gemm.py:535-703) and its row-scale producer
(g_row_scale_f16, S/gen_llm.py:1843-1915).

The oracle is the reference's own GEMM check (make_kernel_tests.py:1858-1900): float64 (X16 W^T) inv with W exactly
dequantized and X16 the row-scaled f16 operand (oracle.ref.f16_rows). Bars: rel-L2 <= 1e-3 for the fp32 accumulation (f32
store); a bf16 store must equal that result rounded to nearest even, bit for bit; the reference's own tolerance
(atol 3e-2 std(y), rtol 1e-2, make_kernel_tests.py:1889) holds for both. Shapes: the Qwen3-8B o_proj
workload (512 x 4096 x 4096) and edge shapes with partial row / column tiles and few super-blocks.
"""
import numpy as np
import pytest

from helpers import assert_close_rel_l2, dev_bf16, dev_f32, dev_u8, host
from oracle import formats as of
from oracle import ref

pytestmark = pytest.mark.gpu


def _case(dev, M, N, K, seed, x_kind="bf16"):
    from qmm import synth
    rng = np.random.default_rng(seed)
    w = synth.q4_k_weights(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if x_kind == "bf16":
        xb = synth.to_bf16_bits(x)
        xv = synth.bf16_bits_to_f32(xb)
        xt = dev_bf16(xb, dev)
    else:                                   # f32 rows with a wide spread of magnitudes: the row scale matters
        x *= np.exp2(rng.integers(-10, 24, (M, 1))).astype(np.float32)
        xv = x
        xt = dev_f32(x, dev)
    W = of.dequant_q4_k(w, N, K)
    want = ref.gemv(ref.f16_rows(xv), W)
    return dev_u8(w, dev), xt, want, xv, w


def _check(y, want, what):
    assert_close_rel_l2(y, want, 1e-3, what)
    np.testing.assert_allclose(y, want, atol=3e-2 * float(np.std(want)), rtol=1e-2)


@pytest.mark.parametrize("M,N,K", [(512, 4096, 4096), (70, 200, 768), (64, 128, 256), (130, 384, 1280),
                                   (64, 128, 8192)])   # K = 8192: the kernel without the staged scale table
def test_gemm_f32_out(dev, M, N, K):
    import qmm.ops as ops
    wt, xt, want, _, _ = _case(dev, M, N, K, seed=M + N + K)
    y = host(ops.gemm("q4_k", "store", xt, wt, N, K))
    _check(y, want, f"gemm {M}x{N}x{K}")


def test_q4_k_staging_one_hot_rows(dev):
    """With one-hot f16 rows (the identity) and no row scale, y[r, c] is the f16-staged weight W16[c, r] exactly
    (fp32 accumulation of a single product). The staging must be the reference's fma_f16(f16(q), f16(d sc),
    f16(-dmin m)) with one rounding (S/gen_gemm.py:499-530), restated here in float64 and rounded once to f16; a
    staging with two roundings (f16(q d sc), then + f16(-dmin m)) differs on this data (the negative control)."""
    import torch
    import qmm.ops as ops
    from qmm import synth
    N, K = 256, 1024
    rng = np.random.default_rng(77)
    w = synth.q4_k_weights(rng, N, K)
    d, dmin, sc, m, q = of.q4_k_fields(w)
    dsc = (d[:, None] * sc.astype(np.float32)).astype(np.float16).astype(np.float64)
    nmn = (-(dmin[:, None] * m.astype(np.float32))).astype(np.float16).astype(np.float64)
    one = (q.astype(np.float64) * dsc[:, :, None] + nmn[:, :, None]).astype(np.float16)
    want = one.astype(np.float32).reshape(N, K).T + np.float32(0.0)   # y[r, c] = W16[c, r]; -0 accumulates to +0
    eye = torch.eye(K, dtype=torch.float16, device=dev)
    got = host(ops.gemm("q4_k", "store", eye, dev_u8(w, dev), N, K))
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{bad.size} staged values differ, first at {bad[:5]}: {got.ravel()[bad[:5]]} vs " \
                          f"{want.ravel()[bad[:5]]}"
    two = ((q.astype(np.float64) * dsc[:, :, None]).astype(np.float16).astype(np.float64)
           + nmn[:, :, None]).astype(np.float16)
    assert not np.array_equal(two, one), "the negative control does not separate one rounding from two"


def test_gemm_bf16_out_workload_shape(dev):
    """The Q4_K prefill workload: bf16 x [512, 4096], W [4096, 4096], bf16 out. The fp32 accumulation meets the
    rel-L2 bar (f32 store); the bf16 store is exactly that result rounded to nearest even, so its distance to the
    oracle is the accumulation error plus bf16's own rounding (about 1.1e-3 rel-L2 on its own)."""
    import torch
    import qmm.ops as ops
    M, N, K = 512, 4096, 4096
    wt, xt, want, _, _ = _case(dev, M, N, K, seed=20261202)
    y32 = host(ops.gemm("q4_k", "store", xt, wt, N, K))
    y16 = host(ops.gemm("q4_k", "store", xt, wt, N, K, out_dtype=torch.bfloat16))
    assert_close_rel_l2(y32, want, 1e-3, "fp32 accumulation")
    assert np.array_equal(ref.bf16_round(y32).view(np.uint32), y16.view(np.uint32)), "bf16 store is not RNE(f32)"
    np.testing.assert_allclose(y16, want, atol=3e-2 * float(np.std(want)), rtol=1e-2)


def test_gemm_row_scaled_f32_rows_and_accumulate(dev):
    """f32 rows spanning 2^-10 .. 2^24 go through the row-scale producer; acc mode adds to y."""
    import qmm.ops as ops
    M, N, K = 96, 256, 1024
    wt, xt, want, _, _ = _case(dev, M, N, K, seed=5, x_kind="f32")
    rng = np.random.default_rng(6)
    y0 = (rng.standard_normal((M, N)) * np.std(want)).astype(np.float32)
    yt = dev_f32(y0, dev)
    ops.gemm("q4_k", "acc", xt, wt, N, K, y=yt)
    _check(host(yt), want + y0, "acc with row scale")


def test_gemm_deterministic_and_negative_control(dev):
    import qmm.ops as ops
    M, N, K = 128, 256, 2048
    wt, xt, want, xv, w = _case(dev, M, N, K, seed=9)
    a = host(ops.gemm("q4_k", "store", xt, wt, N, K))
    b = host(ops.gemm("q4_k", "store", xt, wt, N, K))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    raw = w.reshape(-1, 144).copy()
    raw[:, 16:] = (raw[:, 16:] << 4) | (raw[:, 16:] >> 4)
    wrong = ref.gemv(xv, of.dequant_q4_k(raw.reshape(-1), N, K))
    assert ref.rel_l2(a, wrong) > 0.1 and ref.rel_l2(a, want) <= 1e-3


def test_row_scale_bf16_input(dev):
    import qmm.ops as ops
    from qmm import synth
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 512)) * np.exp2(rng.integers(-4, 30, (64, 1)))).astype(np.float32)
    xb = synth.to_bf16_bits(x)
    x16, sc = ops.row_scale_f16(dev_bf16(xb, dev))
    xv = synth.bf16_bits_to_f32(xb)
    e = ref.row_scale_exponent(xv)
    np.testing.assert_array_equal(host(sc)[:, 1], 2.0 ** e)
    want = (xv.astype(np.float64) * 2.0 ** -e[:, None]).astype(np.float16)
    np.testing.assert_array_equal(host(x16).view(np.uint16), want.view(np.uint16))


def test_gemm_rejects_bad_arguments(dev):
    import torch
    from qmm._lib import QmmError
    import qmm.ops as ops
    w = torch.zeros(144 * 4, dtype=torch.uint8, device=dev)
    with pytest.raises(QmmError):   # GGUF MXFP4 blocks: the scaled-MFMA GEMM reads split / tiled planes only
        ops.gemm("mxfp4", "store", torch.zeros((4, 256), dtype=torch.float16, device=dev), w, 4, 256)
    with pytest.raises(QmmError):
        ops.gemm("q4_k", "store", torch.zeros((4, 128), dtype=torch.float16, device=dev), w, 4, 128)


@pytest.mark.parametrize("M,N,K,out", [(512, 12288, 4096, "f32"), (70, 200, 768, "bf16"), (64, 64, 256, "f32")])
def test_gemm_swiglu(dev, M, N, K, out):
    """g_gemm_q4_k_swiglu (S/gen_gemm.py:10, :688-691): Y = silu(X16 Wg^T inv) (X16 Wu^T inv). Shapes: the Qwen3-8B
    FFN gate/up at a 512-token prefill, and partial row / column tiles. A bf16 store equals the f32 one rounded to
    nearest even, bit for bit."""
    import torch
    import qmm.ops as ops
    from qmm import synth
    rng = np.random.default_rng(M + N + K + 7)
    wg, wu = synth.q4_k_weights(rng, N, K), synth.q4_k_weights(rng, N, K)
    xb = synth.to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    xv = synth.bf16_bits_to_f32(xb)
    xr = ref.f16_rows(xv)
    want = ref.silu_mul(ref.gemv(xr, of.dequant_q4_k(wg, N, K)), ref.gemv(xr, of.dequant_q4_k(wu, N, K)))
    dt = torch.bfloat16 if out == "bf16" else torch.float32
    y = ops.gemm("q4_k", "swiglu", dev_bf16(xb, dev), dev_u8(wg, dev), N, K, w2=dev_u8(wu, dev), out_dtype=dt)
    y32 = host(ops.gemm("q4_k", "swiglu", dev_bf16(xb, dev), dev_u8(wg, dev), N, K, w2=dev_u8(wu, dev)))
    torch.cuda.synchronize()
    assert_close_rel_l2(y32, want, 1e-3, f"swiglu {M}x{N}x{K}")
    if out == "bf16":
        from helpers import assert_bits_equal
        assert_bits_equal(host(y), ref.bf16_round(y32), "bf16 swiglu store")


def test_gemm_skip_padding(dev):
    """GEMM_SKIP_PADDING (S/gen_gemm.py:2188-2220) with g_row_scale_f16_live (S/gen_llm.py:1915-1937): padding rows
    (info[row, 2] == 0) get scale 0 and zero values; a 64-row tile of padding only is not computed and its y rows
    keep what they held; a tile mixing live and padding rows computes every row (padding rows come out 0)."""
    import torch
    import qmm.ops as ops
    from qmm import synth
    rng = np.random.default_rng(23)
    M, N, K = 256, 192, 512
    w = synth.q4_k_weights(rng, N, K)
    xb = synth.to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    xv = synth.bf16_bits_to_f32(xb)
    live = np.ones(M, bool)
    live[64:128] = False               # tile 1: padding only
    live[192 + 40:] = False            # tile 3: 40 live rows, then padding
    info = np.zeros((M, 4), np.int32)
    info[:, 2] = live
    it = torch.from_numpy(info).to(dev)
    x16, sc = ops.row_scale_f16(dev_bf16(xb, dev), info=it)
    x16p, scp = ops.row_scale_f16(dev_bf16(xb, dev))
    assert np.array_equal(host(sc)[~live], np.zeros((int((~live).sum()), 2), np.float32))
    assert np.all(host(x16)[~live] == 0)
    np.testing.assert_array_equal(host(sc)[live], host(scp)[live])
    np.testing.assert_array_equal(host(x16)[live].view(np.uint16), host(x16p)[live].view(np.uint16))
    y = torch.full((M, N), 7.0, dtype=torch.float32, device=dev)
    ops.gemm("q4_k", "store", x16, dev_u8(w, dev), N, K, scales=sc, y=y)
    yh = host(y)
    torch.cuda.synchronize()
    want = ref.gemv(ref.f16_rows(xv), of.dequant_q4_k(w, N, K))
    assert_close_rel_l2(yh[live], want[live], 1e-3, "live rows")
    assert np.all(yh[64:128] == 7.0), "the padding-only tile was written"
    assert np.all(yh[192 + 40:] == 0.0), "padding rows of a live tile are not zero"


# --------------------------------------------------------------------------- one Q4_K weight copy: the tiled layout
@pytest.mark.parametrize("M,N,K,mode,out", [
    (512, 4096, 4096, "store", "bf16"),    # Qwen3-8B o_proj, the workload's shape
    (70, 208, 1536, "acc", "f32"),         # partial row / column tiles, three units a row
    (130, 384, 512, "store", "f32"),       # one unit: waves without super-blocks
    (64, 256, 12288, "store", "f32"),      # K beyond the staged scale table
])
def test_gemm_tiled_layout_equals_gguf(dev, M, N, K, mode, out):
    """The prefill GEMM on the decode GEMV's tiled layout (qmm_tile_q4k) equals the GGUF-layout call bit for bit: a
    model keeps one Q4_K copy for decode and prefill (the reference's single weight view, S/gen_llm.py:5364-5371)."""
    import torch
    import qmm.ops as ops
    wt, xt, want, _, _ = _case(dev, M, N, K, seed=M * 7 + K)
    tiled = ops.tile_q4k(wt, N, K)
    od = torch.bfloat16 if out == "bf16" else torch.float32
    y0 = None if mode == "store" else dev_f32(np.random.default_rng(3).standard_normal((M, N)).astype(np.float32), dev)
    yg = ops.gemm("q4_k", mode, xt, wt, N, K, out_dtype=od, y=None if y0 is None else y0.clone())
    yt = ops.gemm("q4_kt", mode, xt, tiled, N, K, out_dtype=od, y=None if y0 is None else y0.clone())
    torch.cuda.synchronize()
    assert torch.equal(yg.view(torch.int16) if out == "bf16" else yg.view(torch.int32),
                       yt.view(torch.int16) if out == "bf16" else yt.view(torch.int32)), f"{M}x{N}x{K} {mode}"
    if mode == "store" and out == "f32":
        _check(host(yt), want, f"tiled gemm {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(512, 12288, 4096), (70, 208, 1024)])
def test_gemm_swiglu_tiled_layout_equals_gguf(dev, M, N, K):
    """silu(X Wg^T) (X Wu^T) on tiled gate / up weights equals the GGUF-layout call bit for bit."""
    import torch
    import qmm.ops as ops
    from qmm import synth
    wg, xt, _, _, _ = _case(dev, M, N, K, seed=M + 11)
    wu = dev_u8(synth.q4_k_weights(np.random.default_rng(M + 12), N, K), dev)
    yg = ops.gemm("q4_k", "swiglu", xt, wg, N, K, w2=wu)
    yt = ops.gemm("q4_kt", "swiglu", xt, ops.tile_q4k(wg, N, K), N, K, w2=ops.tile_q4k(wu, N, K))
    torch.cuda.synchronize()
    assert torch.equal(yg.view(torch.int32), yt.view(torch.int32)), f"swiglu {M}x{N}x{K}"
