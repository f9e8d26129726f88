"""qmm_moe_routed_static, the MoE chain for callers that cannot allocate, against qmm_moe_routed with a caller-passed
workspace (the same kernels on the same inputs: equal bit for bit), called through the C ABI twice in a row -- the
second call smaller than the first, so it runs on the scratch the first one left -- and a size beyond the static
scratch refused before anything is launched."""
import numpy as np
import pytest

from helpers import assert_bits_equal, dev_bf16, dev_f32, dev_u8, host

pytestmark = pytest.mark.gpu

E, KU, H, FE = 128, 8, 2048, 768


def _static_fn():
    from qmm import _lib
    return _lib.load().qmm_moe_routed_static


def _args(fmt_code, q8, T, x, logits, kw, y, stream):
    p = lambda t: None if t is None else t.data_ptr()
    return [fmt_code, -1, 0, 0, 1, 1, 1.0, int(q8), E, KU, T, H, FE, p(x), 2, p(logits), None, 0, None, None,
            p(kw["w_gate"]), None, p(kw["w_up"]), None, p(kw["w_down"]), None, None, None, None, None, 0, p(y),
            stream]


def test_static_chain_equals_workspace_chain_twice(dev):
    import torch
    import qmm.ops as ops
    from qmm import synth
    from qmm.formats import CODE
    fn = _static_fn()
    rng = np.random.default_rng(20261300)
    kw = dict(w_gate=dev_u8(synth.q4_k_weights(rng, E * FE, H), dev), w_up=dev_u8(synth.q4_k_weights(rng, E * FE, H), dev),
              w_down=dev_u8(synth.q4_k_weights(rng, E * H, FE), dev))
    stream = torch.cuda.current_stream().cuda_stream
    for T, q8 in ((32, True), (4, False)):   # the second call is smaller and takes the f32 path
        x = dev_bf16(synth.to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32)), dev)
        logits = dev_f32(rng.standard_normal((T, E)).astype(np.float32), dev)
        want = ops.moe_chain("q4_k", x, logits, E, KU, H, FE, 1, True, q8=q8, **kw)
        y = torch.full((T, H), float("nan"), dtype=torch.float32, device=dev)
        st = fn(*_args(CODE["q4_k"], q8, T, x, logits, kw, y, stream))
        assert st == 0, st
        torch.cuda.synchronize()
        assert_bits_equal(host(y), host(want), f"static chain T={T} q8={q8}")


def test_static_chain_refuses_sizes_beyond_its_scratch(dev):
    import torch
    import qmm.ops as ops
    from qmm.formats import CODE
    fn = _static_fn()
    T = 4096   # a prefill whose intermediates need more than the static scratch
    assert ops.moe_chain_workspace("q4_k", E, KU, T, H, FE) > 16 << 20
    x = torch.zeros((T, H), dtype=torch.bfloat16, device=dev)
    logits = torch.zeros((T, E), dtype=torch.float32, device=dev)
    w = torch.zeros(16, dtype=torch.uint8, device=dev)
    y = torch.zeros((T, H), dtype=torch.float32, device=dev)
    st = fn(*_args(CODE["q4_k"], False, T, x, logits, dict(w_gate=w, w_up=w, w_down=w), y, None))
    assert st == -8, st   # QMM_ERR_WORKSPACE, nothing launched
