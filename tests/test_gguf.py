"""The GGUF tensor binding (qmm.gguf) on the CPU: the header parser against the reference's header dumps of three
real files (tests/golden/gguf_headers.json.gz, made by tests/golden/make_gguf_fixtures.py from fleet/*/gguf/*.json.gz:
Qwen3-8B Q4_K_M, Qwen3-Coder-30B-A3B Q4_K_M, gpt-oss-20b), and byte-exact tensor reads of written files.

Each dumped header is rebuilt at its real length (KV values over 4 KiB replaced by values of the same type and byte
length) into a sparse file of the real file size; the parser must then find the dump's data_start and tensor table,
and every tensor's size from the ggml block table must end, padded to the alignment, exactly where the next tensor
begins (a wrong block size or rows x K product breaks the chain).
"""
import gzip
import json
import os

import numpy as np
import pytest

import gguf_writer as gw

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
with gzip.open(os.path.join(GOLDEN, "gguf_headers.json.gz")) as _f:
    HEADERS = json.load(_f)


def _sparse_file(tmp_path, name, model):
    h = gw.header(gw.fixture_kv(model), model["tensors"], model["version"])
    p = tmp_path / f"{name}.gguf"
    with open(p, "wb") as f:
        f.write(h)
        f.truncate(model["size"])
    return str(p)


@pytest.mark.parametrize("name", sorted(HEADERS))
def test_real_headers_parse_to_the_dumped_layout(tmp_path, name):
    from qmm import gguf
    m = HEADERS[name]
    g = gguf.GGUFFile(_sparse_file(tmp_path, name, m))
    assert g.version == m["version"] and g.alignment == m["alignment"] and g.size == m["size"]
    assert g.data_start == m["data_start"]
    assert [(t.name, list(t.dims), t.ggml_type, t.offset) for t in g.tensors.values()] == \
        [(n, d, t, o) for n, d, t, o in m["tensors"]]
    ts = sorted(g.tensors.values(), key=lambda t: t.offset)
    a = g.alignment
    for t, nxt in zip(ts, ts[1:]):
        assert (t.offset + t.nbytes + a - 1) // a * a == nxt.offset, (t, nxt)
    assert g.data_start + ts[-1].offset + ts[-1].nbytes <= g.size
    assert isinstance(g.kv["general.architecture"], str)


def test_the_workload_tensors_and_their_formats(tmp_path):
    """Qwen3-8B Q4_K_M: ffn_gate / ffn_up Q4_K [12288 x 4096], ffn_down Q6_K [4096 x 12288]; gpt-oss-20b: fused-free
    MXFP4 experts [32 x 2880 x 2880] with f32 biases and a router with a bias (gating 3)."""
    from qmm import gguf
    q = gguf.GGUFFile(_sparse_file(tmp_path, "q", HEADERS["qwen3_8b_q4_k_m"]))
    up, down = q["blk.0.ffn_up.weight"], q["blk.0.ffn_down.weight"]
    assert (up.fmt, up.k, up.rows) == ("q4_k", 4096, 12288)
    assert (down.fmt, down.k, down.rows) == ("q6_k", 12288, 4096)
    assert down.nbytes == 4096 * 12288 // 256 * 210
    o = gguf.GGUFFile(_sparse_file(tmp_path, "o", HEADERS["gpt_oss_20b"]))
    L = gguf.moe_layer_tensors(o, 0)
    assert L["gate"].fmt == "mxfp4" and L["down"].fmt == "mxfp4"
    assert L["gate"].dims == (2880, 2880, 32) and L["gate"].rows == 32 * 2880
    assert L["router"].type_name == "f32" and L["router"].dims == (2880, 32)
    assert L["router_bias"].dims == (32,) and L["gate_bias"].dims == (2880, 32) and L["down_bias"].dims == (2880, 32)
    assert o.kv["gpt-oss.expert_count"] == 32 and o.kv["gpt-oss.expert_used_count"] == 4
    c = gguf.GGUFFile(_sparse_file(tmp_path, "c", HEADERS["qwen3_coder_30b_a3b_q4_k_m"]))
    Lc = gguf.moe_layer_tensors(c, 0)
    assert Lc["gate"].dims == (2048, 768, 128) and Lc["down"].dims == (768, 2048, 128)


def test_tensor_bytes_round_trip_and_errors(tmp_path):
    from qmm import gguf, synth
    rng = np.random.default_rng(5)
    q4 = np.load(os.path.join(GOLDEN, "q4k_real_gate_64rows.npy"), allow_pickle=False)
    q6 = synth.q6_k_weights(rng, 16, 768)
    bias = rng.standard_normal(16).astype(np.float32).view(np.uint8)
    kv = [("general.architecture", 8, gw.stand_in(8, 8 + 5)), ("general.alignment", 4, np.uint32(32).tobytes())]
    p = str(tmp_path / "t.gguf")
    gw.write(p, kv, [("a.weight", [1024, 64], 12, q4), ("b.weight", [768, 16], 14, q6), ("b.bias", [16], 0, bias)])
    g = gguf.GGUFFile(p)
    assert np.array_equal(g.raw("a.weight"), q4) and np.array_equal(g.raw("b.weight"), q6)
    assert np.array_equal(g.raw("b.bias").view(np.float32), bias.view(np.float32))
    assert g["b.weight"].fmt == "q6_k" and g["b.bias"].fmt is None
    with open(p, "rb") as f:
        blob = f.read()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + blob[4:])
    with pytest.raises(gguf.GGUFError):
        gguf.GGUFFile(str(bad))
    short = tmp_path / "short.gguf"
    short.write_bytes(blob[:g.data_start + g["b.weight"].offset + 10])
    with pytest.raises(gguf.GGUFError):
        gguf.GGUFFile(str(short))
