"""GPU parity of the grouped Q4_K expert GEMMs of the narrow kernel (grouped_q4k_narrow.hip), which qmm_moe_grouped
takes for GGUF Q4_K weights when a prefill batch gives the experts at most eight assignments each on average
(Qwen3-30B-A3B at 64 tokens: four), and always for Q4_K in the tiled layout (q4_kt, K % 512 == 0 or a trailing
half unit: the Qwen3-30B-A3B down tensor has K = 768). Every case runs on both layouts.

The oracle is the reference's experts_ref (make_kernel_tests.py:3197-3221) in float64 on exactly dequantized
weights, with the f16 row rounding of the prefill path applied to the hidden rows and the expert activations
(make_kernel_tests.py:3194-3196); the MoE output must match within rel-L2 1e-3. Cases: the workload shape with a
fused gate_up tensor, swiglu_oai and the gpt-oss expert biases (S/gen_moe.py:958-1007); an expert holding all 64
tokens of the batch (four 16-row groups of one tile) and one holding 20 (two groups, the second partly dead); and the
grouped GEMMs alone on sentinel-filled outputs, whose rows without an assignment must stay untouched. Small shapes
cover one and two experts a token, gate/up K of 256 (tiled: a half unit only), 768 and 1280, down K of 256 and 1280,
and a down GEMM of 48 output columns called directly; the tiled layout beyond the narrow kernel's K (5120) goes to
the 64-row tile kernel, whose results equal the GGUF layout's bit for bit.
"""
import numpy as np
import pytest

from helpers import assert_close_rel_l2, dev_bf16, dev_f32, dev_u8, host
from oracle import formats as of
from oracle import ref
from test_gpu_moe import Experts

pytestmark = pytest.mark.gpu

E, KU, H, FE, T = 128, 8, 2048, 768, 64


def _ops():
    import qmm.ops as ops
    return ops


def _inputs(rng, logits=None):
    from qmm import synth
    xb = synth.to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    if logits is None:
        logits = rng.standard_normal((T, E)).astype(np.float32)
    return xb, logits


LAYOUTS = pytest.mark.parametrize("tiled", [False, True], ids=["gguf", "tiled"])


@LAYOUTS
@pytest.mark.parametrize("fused,act,with_bias", [(True, "swiglu_oai", True), (False, "silu", True),
                                                 (True, "silu", False)])
def test_narrow_chain_variants(dev, fused, act, with_bias, tiled):
    from qmm import synth
    rng = np.random.default_rng(20261240 + 2 * fused + with_bias)
    ex = Experts(dev, "q4_k", rng, E, H, FE, fused)
    xb, logits = _inputs(rng)
    x = synth.bf16_bits_to_f32(xb)
    eids, ewts = ref.route(logits, KU, 1, True)
    bias = None
    if with_bias:
        # sized against the values they are added to: a third of the gate / up and routed outputs' rms
        plain, _ = ref.moe(x, eids, ewts, ex.gate_up, ex.down, act=act, x_round=ref.f16_rows, act_round=ref.f16_rows)
        g_rms = np.sqrt(np.mean((ref.f16_rows(x[:8]) @ ex.gate_up(0)[0].T.astype(np.float64)) ** 2))
        y_rms = np.sqrt(np.mean(plain ** 2))
        bias = tuple((rng.standard_normal((E, n)) * sd).astype(np.float32)
                     for n, sd in ((FE, g_rms / 3), (FE, g_rms / 3), (H, y_rms / 3)))
    wfmt, kw = ex.device(split=True, tiled=tiled)
    y, mid = _ops().moe_prefill(wfmt, dev_bf16(xb, dev), dev_f32(logits, dev), E, KU, H, FE, 1, True, fused=fused,
                                act=act, expert_bias=None if bias is None else tuple(dev_f32(b, dev) for b in bias),
                                **kw)
    np.testing.assert_array_equal(host(mid["ids"]), eids)
    want, _ = ref.moe(x, eids, ewts, ex.gate_up, ex.down, act=act, x_round=ref.f16_rows, act_round=ref.f16_rows,
                      bias=bias)
    assert_close_rel_l2(host(y), want, 1e-3, f"narrow chain fused={fused} act={act} bias={with_bias}")
    if with_bias:   # each bias moves the output by more than the tolerance
        zb, zd = np.zeros_like(bias[0]), np.zeros_like(bias[2])
        for b in ((zb, zb, bias[2]), (bias[0], bias[1], zd)):
            part, _ = ref.moe(x, eids, ewts, ex.gate_up, ex.down, act=act, x_round=ref.f16_rows,
                              act_round=ref.f16_rows, bias=b)
            assert ref.rel_l2(part, want) > 5e-3, "biases too small to be seen"


@LAYOUTS
def test_narrow_heavy_experts(dev, tiled):
    """Expert 5 takes every token (a full 64-row tile: four row groups), expert 77 about twenty (two groups, the
    second partly dead); the other experts keep a handful each."""
    from qmm import synth
    rng = np.random.default_rng(20261250)
    ex = Experts(dev, "q4_k", rng, E, H, FE, False)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[:, 5] += 8.0
    logits[:20, 77] += 8.0
    xb, logits = _inputs(rng, logits)
    wfmt, kw = ex.device(split=True, tiled=tiled)
    y, mid = _ops().moe_prefill(wfmt, dev_bf16(xb, dev), dev_f32(logits, dev), E, KU, H, FE, 1, True, **kw)
    ti = host(mid["tile_info"])
    live = ti[ti[:, 0] >= 0]
    r77 = live[live[:, 0] == 77, 1].tolist()
    assert live[live[:, 0] == 5, 1].tolist() == [64] and len(r77) == 1 and 16 < r77[0] < 32
    eids, ewts = ref.route(logits, KU, 1, True)
    np.testing.assert_array_equal(host(mid["ids"]), eids)
    want, _ = ref.moe(synth.bf16_bits_to_f32(xb), eids, ewts, ex.gate_up, ex.down, x_round=ref.f16_rows,
                      act_round=ref.f16_rows)
    assert_close_rel_l2(host(y), want, 1e-3, "narrow chain with heavy experts")


@LAYOUTS
def test_narrow_grouped_gemms_leave_dead_rows(dev, tiled):
    """gu and dn alone on NaN-filled outputs: every live row equals the oracle's, every other row of the sorted
    outputs (dead rows of live tiles, unused tiles) is still NaN."""
    import torch
    from qmm import synth
    ops = _ops()
    rng = np.random.default_rng(20261260)
    ex = Experts(dev, "q4_k", rng, E, H, FE, True)
    xb, logits = _inputs(rng)
    wfmt, kw = ex.device(split=True, tiled=tiled)
    x = dev_bf16(xb, dev)
    ids, _ = ops.moe_topk(dev_f32(logits, dev), KU, 1, True)
    ti, rm, _ = ops.moe_bucket(ids, E)
    rows = ti.shape[0] * 64
    x16, xs = ops.row_scale_f16(x)
    a = torch.full((rows, FE), float("nan"), dtype=torch.float32, device=dev)
    ops.moe_grouped(wfmt, "gu", ti, rm, x16, kw["w_gate"], FE, H, E, KU, x_scales=xs, fused=True, y=a)
    a16, as_ = ops.row_scale_f16(a, tile_info=ti)
    ys = torch.full((rows, H), float("nan"), dtype=torch.float32, device=dev)
    ops.moe_grouped(wfmt, "dn", ti, rm, a16, kw["w_down"], H, FE, E, KU, x_scales=as_, y=ys)
    torch.cuda.synchronize()
    rmh, idh = host(rm), host(ids).reshape(-1)
    live = rmh >= 0
    ah, ysh = host(a), host(ys)
    assert np.all(np.isnan(ah[~live])) and np.all(np.isnan(ysh[~live])), "rows without an assignment were written"
    xr = ref.f16_rows(synth.bf16_bits_to_f32(xb))
    want_a = np.zeros((rows, FE))
    want_y = np.zeros((rows, H))
    for e in np.unique(idh):
        r = np.flatnonzero(live & (idh[np.maximum(rmh, 0)] == e))
        Wg, Wu = ex.gate_up(int(e))
        g, u = xr[rmh[r] // KU] @ Wg.T.astype(np.float64), xr[rmh[r] // KU] @ Wu.T.astype(np.float64)
        want_a[r] = ref.ACTIVATIONS["silu"](g, u)
        want_y[r] = ref.f16_rows(ah[r]) @ ex.down(int(e)).T.astype(np.float64)
    assert_close_rel_l2(ah[live], want_a[live], 1e-3, "gate/up rows")
    assert_close_rel_l2(ysh[live], want_y[live], 1e-3, "down rows")


def test_tiled_many_rows_equal_batches(dev):
    """The tiled layout takes the narrow kernel at every batch size: at 512 tokens (32 assignments an expert, two to
    four 16-row groups a tile, the groups of a tile side by side in the grid) every token's output equals, bit for
    bit, the output of the chain run on a 64-token slice of the same tokens, which the oracle checks above."""
    import torch
    from qmm import synth
    ops = _ops()
    rng = np.random.default_rng(20261270)
    ex = Experts(dev, "q4_k", rng, E, H, FE, False)
    wfmt, kw = ex.device(split=True, tiled=True)
    Tb, lo = 512, 200
    xb = dev_bf16(synth.to_bf16_bits(rng.standard_normal((Tb, H)).astype(np.float32)), dev)
    logits = dev_f32(rng.standard_normal((Tb, E)).astype(np.float32), dev)
    big, mid = ops.moe_prefill(wfmt, xb, logits, E, KU, H, FE, 1, True, **kw)
    small, _ = ops.moe_prefill(wfmt, xb[lo:lo + T].contiguous(), logits[lo:lo + T].contiguous(), E, KU, H, FE, 1,
                               True, **kw)
    torch.cuda.synchronize()
    ti = host(mid["tile_info"])
    assert ti[:, 1].max() > 32, "no tile with three row groups"
    np.testing.assert_array_equal(host(big)[lo:lo + T].view(np.uint32), host(small).view(np.uint32))


@pytest.mark.parametrize("fused", [False, True])
def test_tiled_grouped_gate_up_beyond_narrow_k_equals_gguf(dev, fused):
    """Gate/up of K = 5120 (beyond the narrow kernel's LDS rows) on the tiled layout takes the 64-row tile kernel at
    the tiled addresses, as the GGUF blocks do: the two grouped GEMMs are equal bit for bit, and the tiled chain
    matches the oracle within rel-L2 1e-3."""
    import torch
    from qmm import synth
    ops = _ops()
    E_, KU_, H_, FE_, T_ = 8, 2, 5120, 512, 96
    rng = np.random.default_rng(20261260 + fused)
    ex = Experts(dev, "q4_k", rng, E_, H_, FE_, fused)
    xb = synth.to_bf16_bits(rng.standard_normal((T_, H_)).astype(np.float32))
    logits = rng.standard_normal((T_, E_)).astype(np.float32)
    x, lg = dev_bf16(xb, dev), dev_f32(logits, dev)
    gfmt, gkw = ex.device(split=True, tiled=False)
    tfmt, tkw = ex.device(split=True, tiled=True)
    _, mid = ops.moe_prefill(gfmt, x, lg, E_, KU_, H_, FE_, 1, True, fused=fused, act="silu", **gkw)
    x16, xs = ops.row_scale_f16(x)
    outs = []
    rows = mid["tile_info"].shape[0] * 64
    for fmt, kw in ((gfmt, gkw), (tfmt, tkw)):   # rows without an assignment keep the NaN sentinel in both
        yy = torch.full((rows, FE_), float("nan"), device=dev)
        outs.append(host(ops.moe_grouped(fmt, "gu", mid["tile_info"], mid["rowmap"], x16, kw["w_gate"], FE_, H_, E_,
                                         KU_, w2=kw.get("w_up"), x_scales=xs, fused=fused, act="silu", y=yy)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(outs[1].view(np.uint32), outs[0].view(np.uint32))
    y, _ = ops.moe_prefill(tfmt, x, lg, E_, KU_, H_, FE_, 1, True, fused=fused, act="silu", **tkw)
    eids, ewts = ref.route(logits, KU_, 1, True)
    want, _ = ref.moe(synth.bf16_bits_to_f32(xb), eids, ewts, ex.gate_up, ex.down, act="silu", x_round=ref.f16_rows,
                      act_round=ref.f16_rows)
    assert_close_rel_l2(host(y), want, 1e-3, f"tiled chain, K = 5120, fused={fused}")


@LAYOUTS
@pytest.mark.parametrize("KU_,H_,FE_,fused", [(1, 256, 1280, False), (2, 1280, 256, True), (2, 768, 512, False)])
def test_narrow_small_shapes(dev, tiled, KU_, H_, FE_, fused):
    """The narrow kernels at the shapes the workload does not reach: one and two experts a token (KU = 1, 2), gate/up
    K of 256 (tiled: a half unit only), 768 and 1280 (GGUF: step loops whose K / 128 is not a multiple of four), and
    down K of 256 and 1280; a few rows an expert (16 tokens over 8 experts) keep both layouts on the narrow kernels."""
    from qmm import synth
    E_, T_ = 8, 16
    rng = np.random.default_rng(20261280 + KU_ + H_)
    ex = Experts(dev, "q4_k", rng, E_, H_, FE_, fused)
    xb = synth.to_bf16_bits(rng.standard_normal((T_, H_)).astype(np.float32))
    logits = rng.standard_normal((T_, E_)).astype(np.float32)
    wfmt, kw = ex.device(split=True, tiled=tiled)
    y, mid = _ops().moe_prefill(wfmt, dev_bf16(xb, dev), dev_f32(logits, dev), E_, KU_, H_, FE_, 1, True,
                                fused=fused, act="silu", **kw)
    eids, ewts = ref.route(logits, KU_, 1, True)
    np.testing.assert_array_equal(host(mid["ids"]), eids)
    want, _ = ref.moe(synth.bf16_bits_to_f32(xb), eids, ewts, ex.gate_up, ex.down, act="silu", x_round=ref.f16_rows,
                      act_round=ref.f16_rows)
    assert_close_rel_l2(host(y), want, 1e-3, f"narrow KU={KU_} H={H_} FE={FE_} fused={fused}")


@LAYOUTS
def test_narrow_down_gemm_alone_n48(dev, tiled):
    """A down GEMM called directly with n = 48 output columns (a second 16-column group clamped into the first block's
    columns) on a NaN-filled output: live rows equal the oracle's, dead rows stay NaN."""
    import torch
    from qmm import synth
    ops = _ops()
    E_, KU_, H_, FE_, T_ = 8, 2, 48, 512, 24
    rng = np.random.default_rng(20261290)
    d = synth.q4_k_weights(rng, E_ * H_, FE_)   # the down tensor [E, 48, 512]
    wd = ops.tile_q4k(dev_u8(d, dev), E_ * H_, FE_) if tiled else dev_u8(d, dev)
    ids, _ = ops.moe_topk(dev_f32(rng.standard_normal((T_, E_)).astype(np.float32), dev), KU_, 1, True)
    ti, rm, _ = ops.moe_bucket(ids, E_)
    rows = ti.shape[0] * 64
    a = dev_f32(rng.standard_normal((rows, FE_)).astype(np.float32), dev)
    a16, as_ = ops.row_scale_f16(a, tile_info=ti)
    ys = torch.full((rows, H_), float("nan"), dtype=torch.float32, device=dev)
    ops.moe_grouped("q4_kt" if tiled else "q4_k", "dn", ti, rm, a16, wd, H_, FE_, E_, KU_, x_scales=as_, y=ys)
    torch.cuda.synchronize()
    rmh, idh, ysh, ah = host(rm), host(ids).reshape(-1), host(ys), host(a)
    live = rmh >= 0
    assert np.all(np.isnan(ysh[~live])), "rows without an assignment were written"
    rb = of.row_bytes("q4_k", FE_)
    want = np.zeros((rows, H_))
    for e in np.unique(idh):
        r = np.flatnonzero(live & (idh[np.maximum(rmh, 0)] == e))
        We = of.dequantize("q4_k", d[e * H_ * rb:(e + 1) * H_ * rb], H_, FE_)
        want[r] = ref.f16_rows(ah[r]) @ We.T.astype(np.float64)
    assert_close_rel_l2(ysh[live], want[live], 1e-3, "down rows, n = 48")
