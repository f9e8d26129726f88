"""GPU parity of the steps either side of the routed experts (S/gen_llm.py:5306-5385 moe_layer / moe_routed): the
router matvec with its top-k (g_moe_route[_tr][_live]), the shared-expert gate (g_moe_shared_gate), the per-expert
down scale (g_moe_wscale), the gated combine (shared_gated), the expert biases of gpt-oss in the grouped GEMMs and
the expert matvecs, and a whole layer with shared experts.

Oracles: route_ref / experts_ref / the chain reference of make_kernel_tests.py:3166-3254 in float64. Router logits
are an fp32 dot product: within rel-L2 1e-5 of float64; the ids are then exactly the top-k the GPU's own logits
give (the same kernel as qmm_moe_topk, bit for bit), and exactly the oracle's on tokens whose k-th and (k+1)-th
scores are clearly apart (the reference's clear_tokens rule, gap > 2e-3). wscale is one f32 product: bit-exact.
Chains: rel-L2 1e-3 with the activation rounding of the path (f16_rows for Q4_K prefill, MXFP8 for MXFP4 prefill).
"""
import numpy as np
import pytest

from helpers import assert_close_rel_l2, dev_bf16, dev_f32, host
from oracle import ref

from test_gpu_moe import Experts, _ops

pytestmark = pytest.mark.gpu


def _act(rng, shape, dtype, dev, scale=1.0):
    """(device tensor, its f32 values) of a random f32 or bf16 array."""
    from qmm import synth
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    if dtype == "bf16":
        b = synth.to_bf16_bits(x)
        return dev_bf16(b, dev), synth.bf16_bits_to_f32(b)
    return dev_f32(x, dev), x


def _clear_rows(rng, n, H, w, KU, gating, bias=None):
    """n f32 rows whose k-th and (k+1)-th router scores differ by more than 0.2 % (make_kernel_tests.py:3185-3192)."""
    x = rng.standard_normal((40 * n, H)).astype(np.float32)
    keep = np.flatnonzero(ref.route_margin(ref.router_logits(x, w), KU, gating, bias) > 2e-3)[:n]
    assert len(keep) == n
    return x[keep]


@pytest.mark.parametrize("T,E,KU,H,gating,norm,has_bias,xdt,wdt", [
    (1, 32, 4, 2880, 3, False, True, "f32", "f32"),       # gpt-oss-20b decode: router bias, softmax of the picked
    (256, 32, 4, 2880, 3, False, True, "bf16", "f32"),    # gpt-oss-20b prefill
    (64, 128, 8, 2048, 1, True, False, "f32", "bf16"),    # Qwen3-30B-A3B: softmax + normalize, bf16 router
    (37, 64, 6, 1024, 2, True, True, "bf16", "bf16"),     # sigmoid with a selection bias; a partial token group
])
def test_moe_route_router_matvec(dev, T, E, KU, H, gating, norm, has_bias, xdt, wdt):
    import torch
    ops = _ops()
    rng = np.random.default_rng(T + E + H)
    x, xv = _act(rng, (T, H), xdt, dev)
    w, wv = _act(rng, (E, H), wdt, dev, scale=H ** -0.5)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if has_bias else None
    bt = dev_f32(bias, dev) if has_bias else None
    ids, wts, logits = ops.moe_route(x, w, KU, gating, norm, bias=bt)
    ids2, wts2 = ops.moe_topk(logits, KU, gating, norm, bias=bt)
    torch.cuda.synchronize()
    want = ref.router_logits(xv, wv)
    lg = host(logits)
    assert_close_rel_l2(lg, want, 1e-5, "router logits")
    np.testing.assert_array_equal(host(ids), host(ids2))
    np.testing.assert_array_equal(host(wts).view(np.uint32), host(wts2).view(np.uint32))
    eids, ewts = ref.route(want, KU, gating, norm, bias)
    clear = ref.route_margin(want, KU, gating, bias) > 2e-3
    assert clear.sum() >= T // 2
    np.testing.assert_array_equal(host(ids)[clear], eids[clear])
    np.testing.assert_allclose(host(wts)[clear], ewts[clear], rtol=1e-4, atol=1e-6)


def test_moe_route_live_skips_padding_tokens(dev):
    """g_moe_route_tr_live: padding tokens of the epoch (info[t, 2] == 0) get no ids or weights; live tokens the
    same as without info."""
    import torch
    ops = _ops()
    rng = np.random.default_rng(7)
    T, E, KU, H = 100, 32, 4, 512
    x, _ = _act(rng, (T, H), "f32", dev)
    w, _ = _act(rng, (E, H), "f32", dev, scale=H ** -0.5)
    info = np.zeros((T, 4), np.int32)
    live = rng.random(T) < 0.6
    live[:8] = False                               # a whole 8-token group of padding
    info[:, 2] = live
    ids, wts, _ = ops.moe_route(x, w, KU, 3, False, info=torch.from_numpy(info).to(dev))
    ids_all, wts_all, _ = ops.moe_route(x, w, KU, 3, False)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(ids)[live], host(ids_all)[live])
    np.testing.assert_array_equal(host(wts)[live], host(wts_all)[live])
    # torch.empty leaves what the allocator held: compare against a sentinel fill instead
    idt = torch.full((T, KU), -7, dtype=torch.int32, device=dev)
    wtt = torch.full((T, KU), 3.5, dtype=torch.float32, device=dev)
    lgt = torch.empty((T, E), dtype=torch.float32, device=dev)
    from qmm import _lib
    _lib.call("qmm_moe_route", T, H, E, KU, 3, 0, 1.0, x.data_ptr(), 0, w.data_ptr(), 0, None,
              torch.from_numpy(info).to(dev).data_ptr(), lgt.data_ptr(), idt.data_ptr(), wtt.data_ptr(),
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.all(host(idt)[~live] == -7) and np.all(host(wtt)[~live] == 3.5)
    np.testing.assert_array_equal(host(idt)[live], host(ids_all)[live])


@pytest.mark.parametrize("T,H,xdt,wdt", [(1, 2048, "f32", "f32"), (64, 2048, "bf16", "bf16"), (13, 1028, "f32", "bf16")])
def test_moe_shared_gate(dev, T, H, xdt, wdt):
    ops = _ops()
    rng = np.random.default_rng(T + H)
    x, xv = _act(rng, (T, H), xdt, dev)
    w, wv = _act(rng, (H,), wdt, dev, scale=2 * H ** -0.5)
    sg = host(ops.moe_shared_gate(x, w))
    np.testing.assert_allclose(sg, ref.shared_gate(xv, wv), rtol=1e-5, atol=1e-7)


def test_moe_wscale_bit_exact(dev):
    """ktest_more.py:99-111: one f32 product per weight; ids out of range are clamped into the experts."""
    import torch
    ops = _ops()
    rng = np.random.default_rng(9)
    T, KU, E = 300, 4, 32
    ids = rng.integers(0, E, (T, KU)).astype(np.int32)
    ids[0, 0], ids[1, 1] = -1, E + 5
    wts = rng.random((T, KU)).astype(np.float32)
    sc = (0.5 + rng.random(E)).astype(np.float32)
    wt = dev_f32(wts, dev)
    ops.moe_wscale(torch.from_numpy(ids).to(dev), wt, dev_f32(sc, dev))
    want = (wts * sc[np.clip(ids, 0, E - 1)]).astype(np.float32)
    np.testing.assert_array_equal(host(wt).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("H,sorted_rows", [(2048, True), (2048, False), (1030, True)])
def test_moe_combine_gated(dev, H, sorted_rows):
    """y = sg y_shared + sum_k w ys (the 16-byte kernel for H % 4 == 0, the scalar one otherwise)."""
    import torch
    ops = _ops()
    rng = np.random.default_rng(H + sorted_rows)
    T, KU = 40, 8
    ys = rng.standard_normal((T * KU + 64, H)).astype(np.float32)
    pos = rng.permutation(T * KU + 64)[:T * KU].astype(np.int32) if sorted_rows else None
    if sorted_rows:
        pos[5] = -1
    wts = rng.random((T, KU)).astype(np.float32)
    y0 = rng.standard_normal((T, H)).astype(np.float32)
    sg = rng.random(T).astype(np.float32)
    yt = dev_f32(y0, dev)
    ops.moe_combine(dev_f32(ys, dev), dev_f32(wts, dev), pos=None if pos is None else torch.from_numpy(pos).to(dev),
                    y=yt, sg=dev_f32(sg, dev))
    want = ref.combine(ys, pos, wts, y0, sg=sg)
    assert_close_rel_l2(host(yt), want, 1e-6, "gated combine")


def _gpt_oss_case(dev, T, prefill, tiled, seed):
    """gpt-oss-20b layer shape with everything the model carries: router weight and bias (gating 3), expert
    biases on gate, up and down, swiglu_oai, fused gate_up, and a per-expert down scale."""
    import torch
    ops = _ops()
    from qmm import synth
    E, KU, H, FE = 32, 4, 2880, 2880
    rng = np.random.default_rng(seed)
    ex = Experts(dev, "mxfp4", rng, E, H, FE, True)
    wr = (rng.standard_normal((E, H)) * H ** -0.5).astype(np.float32)
    rb = (rng.standard_normal(E) * 0.1).astype(np.float32)
    xb = synth.to_bf16_bits(_clear_rows(rng, T, H, wr, KU, 3, rb))   # margins rechecked below on the bf16 rows
    xv = synth.bf16_bits_to_f32(xb)
    bg, bu = (rng.standard_normal((E, FE)) * 0.5).astype(np.float32), (rng.standard_normal((E, FE)) * 0.5).astype(np.float32)
    bd = (rng.standard_normal((E, H)) * 0.5).astype(np.float32)
    dsc = (0.5 + rng.random(E)).astype(np.float32)
    wfmt, kw = ex.device(split=prefill, tiled=tiled)
    chain = ops.moe_prefill if prefill else ops.moe_decode
    y, mid = chain(wfmt, dev_bf16(xb, dev), None, E, KU, H, FE, 3, False, fused=True, act="swiglu_oai",
                   bias=dev_f32(rb, dev), router=dev_f32(wr, dev),
                   expert_bias=(dev_f32(bg, dev), dev_f32(bu, dev), dev_f32(bd, dev)), down_scale=dev_f32(dsc, dev),
                   **kw)
    torch.cuda.synchronize()
    lg = ref.router_logits(xv, wr)
    eids, ewts = ref.route(lg, KU, 3, False, rb)
    clear = ref.route_margin(lg, KU, 3, rb) > 1e-4
    assert clear.mean() > 0.9
    np.testing.assert_array_equal(host(mid["ids"])[clear], eids[clear])
    ids = host(mid["ids"])
    rnd = ref.mxfp8_values if prefill else None
    want, _ = ref.moe(xv, ids, ref.wscale(ids, ref.route(host(mid["logits"]), KU, 3, False, rb)[1], dsc),
                      ex.gate_up, ex.down, act="swiglu_oai", x_round=rnd, act_round=rnd, bias=(bg, bu, bd))
    plain, _ = ref.moe(xv, ids, ref.route(host(mid["logits"]), KU, 3, False, rb)[1], ex.gate_up, ex.down,
                       act="swiglu_oai", x_round=rnd, act_round=rnd)
    assert ref.rel_l2(plain, want) > 0.05, "biases and scales too small to be seen"
    return host(y), want


@pytest.mark.parametrize("T,prefill,tiled", [(256, True, True), (256, True, False), (1, False, False)])
def test_gpt_oss_chain_with_router_biases_and_down_scale(dev, T, prefill, tiled):
    y, want = _gpt_oss_case(dev, T, prefill, tiled, seed=300 + T + tiled)
    assert_close_rel_l2(y, want, 1e-3, f"gpt-oss layer T={T} tiled={tiled}")


def test_q4_k_grouped_expert_biases(dev):
    """Expert biases in the Q4_K grouped GEMMs (gate, up after the row inverse, down on the output)."""
    import torch
    ops = _ops()
    from qmm import synth
    E, KU, H, FE, T = 8, 2, 512, 256, 100
    rng = np.random.default_rng(61)
    ex = Experts(dev, "q4_k", rng, E, H, FE, False)
    xb = synth.to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    logits = rng.standard_normal((T, E)).astype(np.float32)
    x = synth.bf16_bits_to_f32(xb)
    eids, ewts = ref.route(logits, KU, 1, True)
    plain, acts = ref.moe(x, eids, ewts, ex.gate_up, ex.down, act="silu", x_round=ref.f16_rows,
                          act_round=ref.f16_rows)
    gs = float(np.std(ref.f16_rows(x[:8]) @ ex.gate_up(0)[0].T.astype(np.float64)))   # size of a pre-activation
    bg, bu = (rng.standard_normal((E, FE)) * gs).astype(np.float32), (rng.standard_normal((E, FE)) * gs).astype(np.float32)
    bd = (rng.standard_normal((E, H)) * np.std(plain)).astype(np.float32)
    fmt, kw = ex.device(split=True)
    y, mid = ops.moe_prefill(fmt, dev_bf16(xb, dev), dev_f32(logits, dev), E, KU, H, FE, 1, True, act="silu",
                             expert_bias=(dev_f32(bg, dev), dev_f32(bu, dev), dev_f32(bd, dev)), **kw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(mid["ids"]), eids)
    want, _ = ref.moe(x, eids, ewts, ex.gate_up, ex.down, act="silu", x_round=ref.f16_rows, act_round=ref.f16_rows,
                      bias=(bg, bu, bd))
    assert ref.rel_l2(plain, want) > 0.05
    assert_close_rel_l2(host(y), want, 1e-3, "q4_k grouped with biases")


@pytest.mark.parametrize("T", [64, 4])
def test_moe_layer_with_gated_shared_experts(dev, T):
    """A Qwen-MoE-style layer (moe_layer, S/gen_llm.py:5306-5321): the shared experts' swiglu FFN (Q4_K, width FS)
    into y, its gate sigmoid(x . w_shexp_gate), then the routed experts added by the gated combine. T = 64 takes the
    prefill GEMMs (f16 row-scaled operands), T = 4 the decode matvecs."""
    import torch
    ops = _ops()
    from qmm import synth
    E, KU, H, FE, FS = 16, 4, 1024, 256, 512
    rng = np.random.default_rng(70 + T)
    ex = Experts(dev, "q4_k", rng, E, H, FE, False)
    wsg, wsu, wsd = synth.q4_k_weights(rng, FS, H), synth.q4_k_weights(rng, FS, H), synth.q4_k_weights(rng, H, FS)
    gw = (rng.standard_normal(H) * H ** -0.5).astype(np.float32)
    xb = synth.to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    x = synth.bf16_bits_to_f32(xb)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    fmt, kw = ex.device(split=True)
    kw["q8"] = False   # decode on bf16 activations, the float oracle below (int8 decode: test_gpu_q8_matvecs.py)
    from helpers import dev_u8
    shared = dict(fmt="q4_k", w_gate=dev_u8(wsg, dev), w_up=dev_u8(wsu, dev), w_down=dev_u8(wsd, dev), FS=FS,
                  gate=dev_f32(gw, dev))
    y, mid = ops.moe_layer(fmt, dev_bf16(xb, dev), dev_f32(logits, dev), E, KU, H, FE, 1, True, shared=shared, **kw)
    torch.cuda.synchronize()
    from oracle import formats as of
    prefill = T >= ops.GEMM_MIN_TOKENS
    rnd = ref.f16_rows if prefill else (lambda v: np.asarray(v, np.float64))
    xr = rnd(x)
    sh = ref.silu_mul(xr @ of.dequant_q4_k(wsg, FS, H).T.astype(np.float64), xr @ of.dequant_q4_k(wsu, FS, H).T)
    y0 = rnd(sh) @ of.dequant_q4_k(wsd, H, FS).T.astype(np.float64)
    sg = ref.shared_gate(x, gw)
    np.testing.assert_allclose(host(mid["sg"]), sg, rtol=1e-5)
    eids, ewts = ref.route(logits, KU, 1, True)
    np.testing.assert_array_equal(host(mid["ids"]), eids)
    routed, _ = ref.moe(x, eids, ewts, ex.gate_up, ex.down, x_round=rnd if prefill else None,
                        act_round=rnd if prefill else None)
    want = sg[:, None] * y0 + routed
    assert_close_rel_l2(host(y), want, 1e-3, f"moe layer T={T}")
