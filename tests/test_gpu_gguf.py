"""GGUF tensors bound by name (qmm.gguf, the reference's command.parameter) feed the kernels in place: the file's
data region goes to the device once and each tensor is a view of it at its offset. The reference's real Q4_K bytes
(Qwen3-0.6B ffn_gate rows) and synthetic Q6_K / MXFP4 tensors in one file; matvecs on the views against the oracle
(rel-L2 1e-3) and dequantization bit for bit."""
import os

import numpy as np
import pytest

import gguf_writer as gw
from helpers import assert_bits_equal, assert_close_rel_l2, dev_f32, host
from oracle import formats as of
from oracle import ref

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_bound_tensors_feed_the_kernels(dev, tmp_path):
    import torch
    import qmm.ops as ops
    from qmm import gguf, synth
    rng = np.random.default_rng(3)
    q4 = np.load(os.path.join(GOLDEN, "q4k_real_gate_64rows.npy"), allow_pickle=False)
    q6 = synth.q6_k_weights(rng, 48, 768)
    mx = synth.mxfp4_weights(rng, 40, 2880)
    p = str(tmp_path / "w.gguf")
    gw.write(p, [("general.alignment", 4, np.uint32(32).tobytes())],
             [("blk.0.ffn_gate.weight", [1024, 64], 12, q4), ("blk.0.ffn_down.weight", [768, 48], 14, q6),
              ("blk.0.ffn_gate_exps.weight", [2880, 20, 2], 39, mx)])
    g = gguf.GGUFFile(p)
    for name, (fmt, raw) in {"blk.0.ffn_gate.weight": ("q4_k", q4), "blk.0.ffn_down.weight": ("q6_k", q6),
                             "blk.0.ffn_gate_exps.weight": ("mxfp4", mx)}.items():
        t = g[name]
        w = g.view(name, dev)
        assert t.fmt == fmt and w.data_ptr() % 32 == 0 and w.numel() == t.nbytes
        x = rng.standard_normal((3, t.k)).astype(np.float32)
        y = host(ops.mv(fmt, w, dev_f32(x, dev), t.rows, t.k))
        W = of.dequantize(fmt, raw, t.rows, t.k)
        assert_close_rel_l2(y, ref.gemv(x, W), 1e-3, name)
        assert_bits_equal(host(ops.dequant(fmt, w, t.rows, t.k)), W, name)
    torch.cuda.synchronize()
