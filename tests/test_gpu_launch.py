"""The reference's MoE and dense launch sequences driven purely through the name-keyed launcher (qmm.launch), with the
reference's argument lists (S/gen_llm.py:5324-5385 moe_routed, :4568-4625 linear):

  prefill (t >= 64): g_row_scale_f16, g_moe_route_tr_live, g_moe_bucket, g_moe_ggu_{fmt}_k{H},
                     g_row_scale_f16_tiles, g_moe_gdn_{fmt}_k{FE}, g_moe_combine_sorted
  decode (int8):     g_quant_q8, g_moe_route, g_moe_gu_{fmt}_q8_k{H}_r{R}, g_quant_q8, g_moe_dn_{fmt}_q8_k{FE}_r{R},
                     g_moe_combine

at the Qwen3-30B-A3B shape (128 experts, top-8, H = 2048, FE = 768). The launched chain must equal the op surface's
chain (ops.moe_prefill / moe_decode, the same kernels) bit for bit, and the oracle (experts_ref,
make_kernel_tests.py:3197-3221, on the ids and weights the device chose) within rel-L2 1e-3.
"""
import numpy as np
import pytest

from helpers import assert_bits_equal, assert_close_rel_l2, dev_f32, dev_u8, host
from oracle import formats as of
from oracle import ref

pytestmark = pytest.mark.gpu

E, KU, H, FE = 128, 8, 2048, 768


def _layer(dev, seed, T):
    from qmm import synth
    rng = np.random.default_rng(seed)
    g, u, d = (synth.q4_k_weights(rng, E * FE, H), synth.q4_k_weights(rng, E * FE, H),
               synth.q4_k_weights(rng, E * H, FE))
    wr = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    return g, u, d, wr, x


def _oracle(g, u, d, x, ids, wts, rnd):
    rb_h, rb_f = of.row_bytes("q4_k", H), of.row_bytes("q4_k", FE)
    gate_up = lambda e: (of.dequant_q4_k(g[FE * e * rb_h:FE * (e + 1) * rb_h], FE, H),
                         of.dequant_q4_k(u[FE * e * rb_h:FE * (e + 1) * rb_h], FE, H))
    down = lambda e: of.dequant_q4_k(d[H * e * rb_f:H * (e + 1) * rb_f], H, FE)
    return ref.moe(x, ids, wts, gate_up, down, act="silu", x_round=rnd, act_round=rnd)[0]


def test_prefill_chain_through_launch_qwen3_30b_a3b(dev):
    import torch
    import qmm.ops as ops
    from qmm import launch
    T = 64
    g, u, d, wr, x = _layer(dev, 20261260, T)
    L = launch.Launcher(launch.Config(experts=E, used=KU, gating=1, norm_weights=True, act="silu"))
    i32, f32, f16 = torch.int32, torch.float32, torch.float16
    z = lambda shape, dt: torch.zeros(shape, dtype=dt, device=dev)
    h, w_router = dev_f32(x, dev), dev_f32(wr, dev)
    wg, wu, wd = dev_u8(g, dev), dev_u8(u, dev), dev_u8(d, dev)
    max_tiles = T * KU // 64 + E
    max_rows = max_tiles * 64
    info = z((T, 4), i32)
    info[:, 2] = 1   # every token of the epoch is live
    ids, wts, pos = z(T * KU, i32), z(T * KU, f32), z(T * KU, i32)
    tile_info, rowmap = z(2 * max_tiles, i32), z(max_rows, i32)
    h16, s_h = z((T, H), f16), z((T, 2), f32)
    act_sorted, s_rows, act16 = z((max_rows, FE), f32), z((max_rows, 2), f32), z((max_rows, FE), f16)
    ys_sorted, y = z((max_rows, H), f32), z((T, H), f32)
    L.launch("g_row_scale_f16", [T], [T, H, h, s_h, h16])
    L.launch("g_moe_route_tr_live", [T], [T, h, w_router, wts, ids, wts, info])   # no bias: wts fills its slot
    L.launch("g_moe_bucket", [T], [T, max_tiles, info, ids, tile_info, rowmap, pos])
    L.launch("g_moe_ggu_q4_k_k2048", [max_rows, FE],
             [max_rows, H, FE, T, tile_info, rowmap, h16, s_h, wg, wu, act_sorted])
    L.launch("g_row_scale_f16_tiles", [max_rows], [max_rows, FE, act_sorted, s_rows, act16, tile_info])
    L.launch("g_moe_gdn_q4_k_k768", [max_rows, H],
             [max_rows, FE, H, max_rows, tile_info, rowmap, act16, s_rows, wd, ys_sorted])
    L.launch("g_moe_combine_sorted", [T], [T, max_rows, ys_sorted, pos, wts, y])
    torch.cuda.synchronize()
    y_ops, mid = ops.moe_prefill("q4_k", h, None, E, KU, H, FE, 1, True, w_gate=wg, w_up=wu, w_down=wd,
                                 router=w_router)
    assert_bits_equal(host(y), host(y_ops), "launched chain vs op chain")
    ids_h, wts_h = host(ids).reshape(T, KU), host(wts).reshape(T, KU)
    np.testing.assert_array_equal(ids_h, host(mid["ids"]))
    assert_close_rel_l2(host(y), _oracle(g, u, d, x, ids_h, wts_h, ref.f16_rows), 1e-3, "launched prefill chain")


@pytest.mark.parametrize("T", [1, 4])
def test_decode_q8_chain_through_launch_qwen3_30b_a3b(dev, T):
    import torch
    import qmm.ops as ops
    from qmm import launch
    g, u, d, wr, x = _layer(dev, 20261270 + T, T)
    L = launch.Launcher(launch.Config(experts=E, used=KU, gating=1, norm_weights=True, act="silu"))
    i32, f32 = torch.int32, torch.float32
    z = lambda shape, dt: torch.zeros(shape, dtype=dt, device=dev)
    h, w_router = dev_f32(x, dev), dev_f32(wr, dev)
    wg, wu, wd = dev_u8(g, dev), dev_u8(u, dev), dev_u8(d, dev)
    ta = T * KU
    hq = z(ops.q8_bytes(T, H), torch.uint8)
    ids, wts = z(ta, i32), z(ta, f32)
    act, actq, ys, y = z((ta, FE), f32), z(ops.q8_bytes(ta, FE), torch.uint8), z((ta, H), f32), z((T, H), f32)
    L.launch("g_quant_q8", [T, H], [T, H, h, hq])
    L.launch("g_moe_route", [T], [T, h, w_router, wts, ids, wts])
    L.launch("g_moe_gu_q4_k_q8_k2048_r2", [FE, ta], [FE, ta, ids, hq, wg, wu, act])
    L.launch("g_quant_q8", [ta, FE], [ta, FE, act, actq])
    L.launch("g_moe_dn_q4_k_q8_k768_r2", [H, ta], [H, ta, ids, actq, wd, ys])
    L.launch("g_moe_combine", [T], [T, ys, wts, y])
    torch.cuda.synchronize()
    y_ops, mid = ops.moe_decode("q4_k", h, None, E, KU, H, FE, 1, True, w_gate=wg, w_up=wu, w_down=wd,
                                router=w_router, q8=True)
    assert_bits_equal(host(y), host(y_ops), "launched decode chain vs op chain")
    ids_h, wts_h = host(ids).reshape(T, KU), host(wts).reshape(T, KU)
    assert_close_rel_l2(host(y), _oracle(g, u, d, x, ids_h, wts_h, ref.q8_1), 1e-3, "launched decode chain")


def test_dense_names_through_launch(dev):
    """g_mv_q4_k_k4096[_swiglu]_q8 (tiled weights), g_mv_q6_k_k4096 (f32 x) and g_gemm_q4_k_{store,swiglu}_m256:
    the launched kernels equal the op surface's calls bit for bit."""
    import torch
    import qmm.ops as ops
    from qmm import launch, synth
    rng = np.random.default_rng(71)
    N, K, T = 1024, 4096, 2
    wq, wq2 = synth.q4_k_weights(rng, N, K), synth.q4_k_weights(rng, N, K)
    w6 = synth.q6_k_weights(rng, N, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    xt = dev_f32(x, dev)
    wt, wt2 = ops.tile_q4k(dev_u8(wq, dev), N, K), ops.tile_q4k(dev_u8(wq2, dev), N, K)
    L = launch.Launcher(launch.Config(tiled_q4k=True))
    xq = ops.quant_q8(xt)
    y = torch.zeros((T, N), dtype=torch.float32, device=dev)
    L.launch("g_mv_q4_k_k4096_q8_r2", [N, T], [N, T, 0, xq, wt, y])
    assert_bits_equal(host(y), host(ops.mv_q8("q4_kt", wt, xt, N, K)), "g_mv_q4_k_k4096_q8")
    L.launch("g_mv_q4_k_k4096_swiglu_q8_r2", [N, T], [N, T, 0, xq, wt, wt2, y])
    assert_bits_equal(host(y), host(ops.mv_swiglu_q8("q4_kt", wt, wt2, xt, N, K)), "swiglu_q8")
    w6t = dev_u8(w6, dev)
    L.launch("g_mv_q6_k_k4096", [N, T], [N, T, 0, xt, w6t, y])
    assert_bits_equal(host(y), host(ops.mv("q6_k", w6t, xt, N, K)), "g_mv_q6_k_k4096")
    M = 128
    xm = dev_f32(rng.standard_normal((M, K)).astype(np.float32), dev)
    x16, s = ops.row_scale_f16(xm)
    yg = torch.zeros((M, N), dtype=torch.float32, device=dev)
    wg = dev_u8(wq, dev)
    L.launch("g_gemm_q4_k_store_m256", [M, N], [M, K, N, x16, s, wg, yg])
    assert_bits_equal(host(yg), host(ops.gemm("q4_k", "store", x16, wg, N, K, scales=s)), "g_gemm_q4_k_store")
    wg2 = dev_u8(wq2, dev)
    L.launch("g_gemm_q4_k_swiglu_m128", [M, N], [M, K, N, x16, s, wg, wg2, yg])
    assert_bits_equal(host(yg), host(ops.gemm("q4_k", "swiglu", x16, wg, N, K, w2=wg2, scales=s)), "swiglu gemm")
