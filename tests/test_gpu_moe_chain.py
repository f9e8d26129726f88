"""GPU checks of qmm_moe_routed, the routed experts of one MoE layer in one library call (the command sequence of
moe_routed, S/gen_llm.py:5324-5385, with moe_alloc's intermediates in a caller-passed workspace, :5388-5432): it runs
the same kernels as the op-by-op chains (ops.moe_prefill / moe_decode), which are checked against the oracle in
test_gpu_moe.py and test_gpu_q8_matvecs.py, so its output must equal theirs bit for bit. Cases: the Qwen3-30B-A3B
shape (Q4_K; prefill at T = 64, decode at T = 4 with f32 and int8 activations, a Q6_K down tensor), the gpt-oss-20b
shape (MXFP4: tiled planes at T = 256, split or tiled planes at T = 1 and 3, swiglu_oai, expert biases, down scales), routing from
the router weight, a shared-expert gate, and a workspace one byte short.
"""
import numpy as np
import pytest

from helpers import assert_bits_equal, dev_bf16, dev_f32, dev_u8, host

pytestmark = pytest.mark.gpu


def _q4k_layer(dev, rng, E, H, FE, fmt_down="q4_k"):
    from qmm import synth
    g, u = synth.q4_k_weights(rng, E * FE, H), synth.q4_k_weights(rng, E * FE, H)
    d = synth.weights(fmt_down, rng, E * H, FE)
    return dict(w_gate=dev_u8(g, dev), w_up=dev_u8(u, dev), w_down=dev_u8(d, dev))


@pytest.mark.parametrize("T,q8,fmt_down,use_router", [(64, False, None, False), (4, False, None, False),
                                                      (4, True, None, False), (4, True, "q6_k", True),
                                                      (70, False, "q6_k", True)])
def test_chain_equals_op_chain_qwen3_30b_a3b(dev, T, q8, fmt_down, use_router):
    import torch
    import qmm.ops as ops
    from qmm import synth
    E, KU, H, FE = 128, 8, 2048, 768
    rng = np.random.default_rng(20261280 + T)
    kw = _q4k_layer(dev, rng, E, H, FE, fmt_down or "q4_k")
    x = dev_bf16(synth.to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32)), dev)
    if use_router:
        logits, router = None, dev_f32((rng.standard_normal((E, H)) * 0.05).astype(np.float32), dev)
    else:
        logits, router = dev_f32(rng.standard_normal((T, E)).astype(np.float32), dev), None
    y = ops.moe_chain("q4_k", x, logits, E, KU, H, FE, 1, True, fmt_down=fmt_down, q8=q8, router=router, **kw)
    y_ops, _ = ops.moe_routed("q4_k", x, logits, E, KU, H, FE, 1, True, fmt_down=fmt_down, q8=q8, router=router,
                              **kw)
    torch.cuda.synchronize()
    assert_bits_equal(host(y), host(y_ops), f"chain T={T} q8={q8}")


@pytest.mark.parametrize("T,tiled", [(1, False), (1, True), (3, True), (256, True)])
def test_chain_equals_op_chain_gpt_oss_20b(dev, T, tiled):
    """MXFP4 experts (split planes or MFMA-tiled planes for decode, tiled planes for prefill), swiglu_oai, expert
    biases, per-expert down scales, gating 3."""
    import torch
    import qmm.ops as ops
    from qmm import synth
    E, KU, H, FE = 32, 4, 2880, 2880
    rng = np.random.default_rng(20261290 + T)
    gu, dn = synth.mxfp4_weights(rng, E * 2 * FE, H), synth.mxfp4_weights(rng, E * H, FE)
    gn, gs = ops.repack_mxfp4(dev_u8(gu, dev), E * 2 * FE, H)
    dnn, ds = ops.repack_mxfp4(dev_u8(dn, dev), E * H, FE)
    fmt = "mxfp4s"
    if tiled:
        gn, gs = ops.tile_mxfp4(gn, gs, E * 2 * FE, H)
        dnn, ds = ops.tile_mxfp4(dnn, ds, E * H, FE)
        fmt = "mxfp4t"
    eb = tuple(dev_f32(rng.standard_normal((E, n)).astype(np.float32) * 0.1, dev) for n in (FE, FE, H))
    dsc = dev_f32(rng.uniform(0.5, 1.5, E).astype(np.float32), dev)
    x = dev_bf16(synth.to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32)), dev)
    logits = dev_f32(rng.standard_normal((T, E)).astype(np.float32), dev)
    kw = dict(w_gate=gn, ws_gate=gs, w_down=dnn, ws_down=ds, fused=True, act="swiglu_oai", expert_bias=eb,
              down_scale=dsc)
    y = ops.moe_chain(fmt, x, logits, E, KU, H, FE, 3, False, **kw)
    y_ops, _ = ops.moe_routed(fmt, x, logits, E, KU, H, FE, 3, False, **kw)
    torch.cuda.synchronize()
    assert_bits_equal(host(y), host(y_ops), f"gpt-oss chain T={T}")


def test_chain_shared_gate_and_short_workspace(dev):
    import torch
    import qmm.ops as ops
    from qmm import synth
    from qmm._lib import QmmError
    E, KU, H, FE, T = 16, 4, 512, 256, 8
    rng = np.random.default_rng(33)
    kw = _q4k_layer(dev, rng, E, H, FE)
    x = dev_bf16(synth.to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32)), dev)
    logits = dev_f32(rng.standard_normal((T, E)).astype(np.float32), dev)
    shared = rng.standard_normal((T, H)).astype(np.float32)
    sg = dev_f32(rng.uniform(0, 1, T).astype(np.float32), dev)
    y1, y2 = dev_f32(shared, dev), dev_f32(shared, dev)
    ops.moe_chain("q4_k", x, logits, E, KU, H, FE, 1, True, y=y1, sg=sg, **kw)
    ops.moe_routed("q4_k", x, logits, E, KU, H, FE, 1, True, y=y2, sg=sg, **kw)
    torch.cuda.synchronize()
    assert_bits_equal(host(y1), host(y2), "shared-gated chain")
    need = ops.moe_chain_workspace("q4_k", E, KU, T, H, FE)
    short = torch.empty(need - 1, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        ops.moe_chain("q4_k", x, logits, E, KU, H, FE, 1, True, workspace=short, **kw)
    from qmm import _lib
    from qmm.formats import CODE
    st = _lib.load().qmm_moe_routed(CODE["q4_k"], -1, 0, 0, 1, 1, 1.0, 0, E, KU, T, H, FE, x.data_ptr(), 2,
                                    logits.data_ptr(), None, 0, None, None, kw["w_gate"].data_ptr(), None,
                                    kw["w_up"].data_ptr(), None, kw["w_down"].data_ptr(), None, None, None, None,
                                    None, 0, y1.data_ptr(), short.data_ptr(), need - 1, None)
    assert st == -8, st   # QMM_ERR_WORKSPACE, nothing launched
