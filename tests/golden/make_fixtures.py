"""Writes the small fixtures under tests/golden/ from data files the reference's own tests and benchmarks hold.

    python tests/golden/make_fixtures.py [REFERENCE_ROOT]      (default /root/reference)

Nothing of the reference is imported or executed: the .npy files are read with numpy.load (allow_pickle=False) and
the known-answer values are transcribed from the reference's test sources.

* q4k_real_gate_64rows.npy / q4k_real_up_64rows.npy -- the first 64 rows (36,864 bytes each) of the only real
  quantized weights in the reference, Qwen3-0.6B layer 3 ffn_gate / ffn_up as Q4_K [3072 x 1024]
  (.github/devlab/kbench/gemm_r9700/real_gate.npy, real_up.npy; gen_gemm_bench.py:124-125)
* kats.json -- known answers transcribed from the reference's tests:
    mxfp4_split: nibble bytes 0x21, 0x7F with E8M0 128 decode to [1.0, 2.0, -12.0, 12.0]
                 (tests/test_safetensors_source.py:200-206)
    q4_0_required_f16_bits: bit patterns the every-finite-scale Q4_0 proof must contain once rounded to f16
                 (tests/test_moe_q4_0.py:100-103); 32767 never occurs (:104)
    q4_0_scale_count: number of finite f16 scales of that proof (tests/test_moe_q4_0.py:99)
    norm_floor: the weight-sum floor of normalized top-k weights (make_kernel_tests.py:3180; S/gen_moe.py:133)
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROWS = 64
K = 1024
ROW_BYTES = K // 256 * 144


def main(ref_root):
    src = os.path.join(ref_root, ".github/devlab/kbench/gemm_r9700")
    for name in ("real_gate", "real_up"):
        a = np.load(os.path.join(src, name + ".npy"), allow_pickle=False).view(np.uint8).reshape(-1)
        assert a.size == 3072 * ROW_BYTES, a.size
        np.save(os.path.join(HERE, f"q4k_{name}_64rows.npy"), a[:ROWS * ROW_BYTES].copy(), allow_pickle=False)
    kats = {
        "mxfp4_split": {"nibbles": [0x21, 0x7F], "e8m0": 128, "values": [1.0, 2.0, -12.0, 12.0]},
        "q4_0_required_f16_bits": [0x0000, 0x8000, 0x0001, 0x8001, 0x0400, 0x8400, 0x7C00, 0xFC00],
        "q4_0_never_f16_bits": [32767],
        "q4_0_scale_count": 63488,
        "norm_floor": 6.103515625e-05,
        "real_q4k": {"rows": ROWS, "k": K, "source_rows": 3072},
    }
    with open(os.path.join(HERE, "kats.json"), "w") as f:
        json.dump(kats, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
