"""GPU parity of the MoE routing / permutation / combine kernels and the activation producers.

ids, tile_info, rowmap and pos must equal the oracle exactly (the canonical permutation); routing weights are
compared with the reference's tolerance (1e-5 abs / 1e-4 rel, make_kernel_tests.py:3333-3338); the MXFP8 codes and
scales, the MXFP4 repack and the row-scale f16 copy are bit-exact.
"""
import numpy as np
import pytest

from helpers import assert_bits_equal, dev_bf16, dev_f32, dev_u8, host
from oracle import formats as of
from oracle import ref

pytestmark = pytest.mark.gpu


def _ops():
    import qmm.ops as ops
    return ops


@pytest.mark.parametrize("T,E,KU,gating,norm", [(64, 128, 8, 1, True), (256, 32, 4, 3, False), (1, 32, 4, 3, False),
                                               (37, 256, 8, 1, True), (9, 8, 2, 2, False), (5, 60, 6, 1, False)])
def test_topk_matches_oracle(dev, T, E, KU, gating, norm):
    rng = np.random.default_rng(T * 1000 + E)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    ids, wts = _ops().moe_topk(dev_f32(logits, dev), KU, gating, norm)
    eids, ewts = ref.route(logits, KU, gating, norm)
    np.testing.assert_array_equal(host(ids), eids)
    np.testing.assert_allclose(host(wts), ewts, atol=1e-5, rtol=1e-4)


def test_topk_ties_go_to_the_lower_id(dev):
    logits = np.zeros((3, 16), np.float32)
    logits[1, [3, 9, 12]] = 1.0
    logits[2] = np.repeat(np.arange(8, dtype=np.float32), 2)[::-1]
    ids, _ = _ops().moe_topk(dev_f32(logits, dev), 4, 1, True)
    eids, _ = ref.route(logits, 4, 1, True)
    np.testing.assert_array_equal(host(ids), eids)
    assert host(ids)[0].tolist() == [0, 1, 2, 3]


@pytest.mark.parametrize("T,E,KU", [(64, 128, 8), (256, 32, 4), (3, 16, 2), (1000, 64, 8), (70, 256, 8), (4096, 32, 4),
                                    (4095, 64, 4), (20000, 256, 8), (2048, 32, 4), (8191, 16, 1), (9300, 256, 1)])
def test_bucket_canonical(dev, T, E, KU):
    """From 8192 assignments on, the bucket runs as count / scan / scatter launches over ranges of 1024 (the last
    with the remainder): 2048 x 4 is the first such case, 8191 x 1 the last one-workgroup case."""
    rng = np.random.default_rng(T + E)
    ids = rng.integers(0, E, (T, KU)).astype(np.int32)
    if T > 3:
        ids[: T // 2, 0] = 5 % E        # a heavy expert with more than 64 rows
    info = np.ones((T, 4), np.int32)
    if T > 10:
        info[T - 3:, 2] = 0             # dead (padding) tokens
    mt = ref.max_tiles(T, KU, E)
    import torch
    ti, rm, pos = _ops().moe_bucket(torch.from_numpy(ids).to(dev), E, mt, info=torch.from_numpy(info).to(dev))
    eti, erm, epos = ref.bucket(ids, E, mt, live=info[:, 2])
    np.testing.assert_array_equal(host(ti), eti)
    np.testing.assert_array_equal(host(rm), erm)
    np.testing.assert_array_equal(host(pos), epos)


@pytest.mark.parametrize("op", ["f16", "mxfp8"])
@pytest.mark.parametrize("T,E,KU,gating,norm,H,bias", [(64, 128, 8, 1, True, 2048, False),
                                                       (256, 32, 4, 3, False, 2880, False),
                                                       (67, 256, 8, 2, True, 4096, True),
                                                       (130, 160, 6, 3, False, 1024, True),
                                                       (5, 60, 6, 1, False, 2048, False)])
def test_topk_operand_equals_separate_calls(dev, op, T, E, KU, gating, norm, H, bias):
    """qmm_moe_topk_operand: ids and weights bit for bit those of moe_topk, the operand bit for bit row_scale_f16 /
    quant_mxfp8 of the same rows (row magnitudes 2^-30 .. 2^30, so row scales and E8M0 exponents over a wide range
    occur; zero rows too); 1 to 4 key slots a lane, rows up to 4096 values."""
    import torch
    from qmm import synth
    ops = _ops()
    if op == "f16" and H % 8 or op == "mxfp8" and H % 32:
        pytest.skip("row length")
    rng = np.random.default_rng(T * 31 + E + H)
    xf = rng.standard_normal((T, H)).astype(np.float32) * np.exp2(rng.integers(-30, 31, (T, 1))).astype(np.float32)
    xf[T // 2] = 0.0
    x = dev_bf16(synth.to_bf16_bits(xf), dev)
    lg = dev_f32(rng.standard_normal((T, E)).astype(np.float32), dev)
    b = dev_f32(rng.standard_normal(E).astype(np.float32) * 0.5, dev) if bias else None
    ids, wts, xo, xs = ops.moe_topk_operand(lg, KU, gating, norm, x, op, scale=1.5, bias=b)
    ids0, wts0 = ops.moe_topk(lg, KU, gating, norm, scale=1.5, bias=b)
    xo0, xs0 = ops.row_scale_f16(x) if op == "f16" else ops.quant_mxfp8(x)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(ids), host(ids0))
    assert_bits_equal(host(wts), host(wts0), "weights")
    np.testing.assert_array_equal(host(xo).view(np.uint8), host(xo0).view(np.uint8))
    np.testing.assert_array_equal(host(xs).view(np.uint8), host(xs0).view(np.uint8))


def test_bucket_dead_range_and_one_expert(dev):
    """Ranges of the many-workgroup bucket whose tokens are all padding (info[t, 2] == 0) and ranges that hold a
    single expert: rows, tiles and pos still equal the oracle's."""
    import torch
    rng = np.random.default_rng(8)
    T, E, KU = 12000, 8, 1
    ids = rng.integers(0, E, (T, KU)).astype(np.int32)
    ids[5600:7900, 0] = 3
    info = np.ones((T, 4), np.int32)
    info[1000:4500, 2] = 0
    mt = ref.max_tiles(T, KU, E)
    ti, rm, pos = _ops().moe_bucket(torch.from_numpy(ids).to(dev), E, mt, info=torch.from_numpy(info).to(dev))
    eti, erm, epos = ref.bucket(ids, E, mt, live=info[:, 2])
    np.testing.assert_array_equal(host(ti), eti)
    np.testing.assert_array_equal(host(rm), erm)
    np.testing.assert_array_equal(host(pos), epos)


def test_bucket_repeat_runs_identical(dev):
    import torch
    rng = np.random.default_rng(4)
    ids = torch.from_numpy(rng.integers(0, 32, (512, 4)).astype(np.int32)).to(dev)
    a = [host(t) for t in _ops().moe_bucket(ids, 32)]
    for _ in range(3):
        b = [host(t) for t in _ops().moe_bucket(ids, 32)]
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize("sorted_rows,acc", [(True, False), (False, True)])
def test_combine(dev, sorted_rows, acc):
    import torch
    rng = np.random.default_rng(12)
    T, KU, H = 33, 4, 2880
    wts = rng.random((T, KU)).astype(np.float32)
    if sorted_rows:
        ids = rng.integers(0, 32, (T, KU)).astype(np.int32)
        mt = ref.max_tiles(T, KU, 32)
        _, _, pos = ref.bucket(ids, 32, mt)
        pos[3] = -1
        ys = rng.standard_normal((mt * 64, H)).astype(np.float32)
        pt = torch.from_numpy(pos).to(dev)
    else:
        pos, pt = None, None
        ys = rng.standard_normal((T * KU, H)).astype(np.float32)
    y0 = rng.standard_normal((T, H)).astype(np.float32)
    yt = dev_f32(y0, dev)
    _ops().moe_combine(dev_f32(ys, dev), dev_f32(wts, dev), pos=pt, y=yt, accumulate=acc)
    e = ref.combine(ys, pos, wts, y0 if acc else None)
    np.testing.assert_allclose(host(yt), e, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("src", ["f32", "bf16"])
def test_quant_mxfp8_bit_exact(dev, src):
    rng = np.random.default_rng(2)
    rows, k = 48, 2880
    x = (rng.standard_normal((rows, k)) * np.exp(rng.uniform(-8, 8, (rows, 1)))).astype(np.float32)
    x[0, :32] = 0.0                      # an all-zero block
    x[1, 5] = -1e-30                     # tiny values around the subnormal range
    if src == "bf16":
        from qmm.synth import to_bf16_bits
        xb = to_bf16_bits(x)
        x = (xb.astype(np.uint32) << 16).view(np.float32)
        xt = dev_bf16(xb, dev)
    else:
        xt = dev_f32(x, dev)
    codes, scales = _ops().quant_mxfp8(xt)
    ec, es, _ = ref.mxfp8_quantize(x)
    np.testing.assert_array_equal(host(scales), es)
    c = host(codes)
    bad = np.flatnonzero(c != ec)
    # -0 and +0 are the same value; compare the decoded values for those, bytes elsewhere
    assert np.all(ref.e4m3_decode(c.reshape(-1)[bad]) == ref.e4m3_decode(ec.reshape(-1)[bad])), bad[:8]


def test_repack_mxfp4_bit_exact(dev):
    from qmm import synth
    rng = np.random.default_rng(6)
    rows, k = 30, 2880
    w = synth.mxfp4_weights(rng, rows, k)
    nib, sc = _ops().repack_mxfp4(dev_u8(w, dev), rows, k)
    en, es = of.mxfp4_to_split(w, rows, k)
    np.testing.assert_array_equal(host(nib), en)
    np.testing.assert_array_equal(host(sc), es)


def test_row_scale_f16(dev):
    rng = np.random.default_rng(10)
    x = (rng.standard_normal((64, 768)) * np.array([1.0] * 32 + [1e6] * 32)[:, None]).astype(np.float32)
    x16, sc = _ops().row_scale_f16(dev_f32(x, dev))
    e = ref.row_scale_exponent(x)
    np.testing.assert_array_equal(host(sc)[:, 1], 2.0 ** e)
    want = (x.astype(np.float64) * 2.0 ** -e[:, None]).astype(np.float16)
    assert_bits_equal(host(x16).astype(np.float32), want.astype(np.float32), "x16")


def test_row_scale_rows_equals_tile_rows(dev):
    """The listed-rows producer writes the bucket's live rows exactly as the tile-wise one does."""
    import torch
    ops = _ops()
    rng = np.random.default_rng(11)
    T, E, KU, k = 64, 128, 8, 768
    ids, _ = ops.moe_topk(dev_f32(rng.standard_normal((T, E)).astype(np.float32), dev), KU, 1, True)
    ti, rm, pos = ops.moe_bucket(ids, E)
    rows = ti.shape[0] * 64
    a = dev_f32((rng.standard_normal((rows, k)) * np.exp2(rng.integers(-20, 20, (rows, 1)))).astype(np.float32), dev)
    want16, wants = ops.row_scale_f16(a, tile_info=ti)
    got16, gots = ops.row_scale_f16_rows(a, pos)
    torch.cuda.synchronize()
    live = host(rm) >= 0
    assert live.sum() == T * KU
    np.testing.assert_array_equal(host(got16.view(torch.int16))[live], host(want16.view(torch.int16))[live])
    np.testing.assert_array_equal(host(gots)[live].view(np.uint32), host(wants)[live].view(np.uint32))
