"""The name-keyed launcher (qmm.launch) against the kernel names the reference emits for Qwen3-8B, Qwen3-30B-A3B and
gpt-oss-20b, on the CPU (no device: every name must map to an entry point libqmm.so exports, and malformed launches
must fail before any device call).

The names are derived from the three models' real GGUF tensor tables (tests/golden/gguf_headers.json.gz: name, shape,
GGML type of every tensor) with the reference's naming rules, restated here as test infrastructure:
  - mv_name (S/gen_llm.py:5098-5111) with pick_r / iq_r (S/mv_rows.py:19-55): decode matvecs of 1, 4 (and for int8
    activations 8, 16) tokens, `_q8` for the formats with integer codes (K / 32 <= 1024), `_r{R}` when R != 16;
  - the prefill GEMMs g_gemm_{fmt}_{store|acc|swiglu}[_m128|_m256] (S/gen_llm.py:4586-4610);
  - the MoE chain of moe_routed (S/gen_llm.py:5324-5385): R of _moe_rows_per_workgroup (:5274-5288), `_q8` experts
    when moe_iq holds (no expert biases, integer-code formats, :5298-5303), grouped GEMMs g_moe_g{gu|dn}_{fmt}_k{K}.
Only the formats of the quantized-matmul path (Q4_0, Q4_K, Q6_K, MXFP4) are kept; the models' Q8_0 / F16 / F32
tensors go to other kernels.
"""
import gzip
import json
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GGML = {2: "q4_0", 12: "q4_k", 14: "q6_k", 39: "mxfp4"}
IQ_FMTS = ("q4_0", "q4_k", "q6_k")
WG1, WG4, WG_LONG = 4096, 128, 640


def pick_r(n, K, TG):
    """S/mv_rows.py:19-28 (adaptive R, the same R for every token group)."""
    target = WG_LONG if K >= 8192 else WG1
    R = 16
    while R > 1 and n // R < target and n % (R // 2) == 0:
        R //= 2
    return R


def iq_r(n, K, TG, sw=0):
    """S/mv_rows.py:31-55."""
    R = pick_r(n, K, TG)
    if TG >= 8 and n % 16 == 0:
        R = 16
    if sw == 2:
        R = 16
        while R > 4 and n // R < 32 and n % (R // 2) == 0:
            R //= 2
        return R
    waves = (K // 32 + 31) // 32
    lds = waves * 32 * TG * (2 if sw else 1) * 4
    if TG >= 16 and n % 32 == 0 and (sw or K >= 8192) and K // 32 <= 1024 and lds <= 48 * 1024:
        R = 32
    return R


def mv_name(fmt, K, sw, n, TG, iq):
    """S/gen_llm.py:5098-5111."""
    base = f"g_mv_{fmt}_k{K}" + {1: "_swiglu", 2: "_pair"}.get(sw, "") + (f"_t{TG}" if TG > 1 else "")
    if iq:
        R = iq_r(n, K, TG, sw)
        return base + "_q8" + (f"_r{R}" if R != 16 else "")
    R = pick_r(n, K, TG)
    return base + (f"_r{R}" if R != 16 else "")


def moe_r(used, ffn, H):
    """S/gen_llm.py:5274-5288."""
    r = 8
    while r > 2 and used * ffn // r < 3000 and ffn % (r // 2) == 0 and H % (r // 2) == 0:
        r //= 2
    return r


def model_names(model):
    tables = json.load(gzip.open(os.path.join(HERE, "golden", "gguf_headers.json.gz")))
    tensors = {name: (shape, GGML.get(ty)) for name, shape, ty, _ in tables[model]["tensors"]}
    names = set()
    dense = [(n, s, f) for n, (s, f) in tensors.items() if f and n.endswith(".weight") and len(s) == 2
             and not n.startswith("token_embd")]
    for name, (K, n), fmt in dense:
        iq = fmt in IQ_FMTS and K // 32 <= 1024
        sw = 1 if name.endswith("ffn_gate.weight") else 0
        if name.endswith("ffn_up.weight"):
            continue   # the up matrix rides in the gate's swiglu kernels
        for TG in (1, 4) + ((8, 16) if iq else ()):
            names.add(mv_name(fmt, K, sw, n, TG, iq))
            if not iq:
                break
        if not (fmt == "mxfp4"):
            modes = ("swiglu",) if sw else ("store", "acc")
            for mode in modes:
                for tile in ("", "_m128", "_m256"):
                    names.add(f"g_gemm_{fmt}_{mode}{tile}")
    experts = {n: (s, f) for n, (s, f) in tensors.items() if n.endswith("_exps.weight") and f}
    if experts:
        (H, FE, E), fg = next((s, f) for n, (s, f) in experts.items() if "ffn_gate_exps" in n)
        biases = any(n.endswith("_exps.bias") for n in tensors)
        used = 8 if E == 128 else 4
        R = moe_r(used, FE, H)
        fds = {f for n, (s, f) in experts.items() if "ffn_down_exps" in n}
        iq = fg in IQ_FMTS and all(fd in IQ_FMTS for fd in fds) and not biases
        for fd in fds:
            names |= {f"g_moe_ggu_{fg}_k{H}", f"g_moe_gdn_{fd}_k{FE}", f"g_moe_gu_{fg}_k{H}_r{R}",
                      f"g_moe_dn_{fd}_k{FE}_r{R}"}
            if iq:
                names |= {f"g_moe_gu_{fg}_q8_k{H}_r{R}", f"g_moe_dn_{fd}_q8_k{FE}_r{R}"}
        names |= {"g_moe_route", "g_moe_route_tr", "g_moe_route_tr_live", "g_moe_bucket", "g_moe_combine",
                  "g_moe_combine_sorted", "g_row_scale_f16", "g_row_scale_f16_live", "g_row_scale_f16_tiles",
                  "g_quant_q8"}
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    from qmm import _lib
    try:
        return _lib.load()
    except OSError as e:
        pytest.skip(str(e))


@pytest.mark.parametrize("model,expect", [
    ("qwen3_8b_q4_k_m", ["g_mv_q4_k_k4096_swiglu_q8_r2", "g_mv_q6_k_k12288_q8_r4", "g_mv_q4_k_k4096_swiglu_t4_q8_r2",
                         "g_mv_q4_k_k4096_swiglu_t16_q8_r32", "g_gemm_q4_k_swiglu_m256", "g_gemm_q6_k_acc_m128"]),
    ("qwen3_coder_30b_a3b_q4_k_m", ["g_moe_ggu_q4_k_k2048", "g_moe_gdn_q4_k_k768", "g_moe_gu_q4_k_q8_k2048_r2",
                                    "g_moe_dn_q4_k_q8_k768_r2", "g_moe_route_tr_live", "g_moe_combine_sorted"]),
    ("gpt_oss_20b", ["g_moe_ggu_mxfp4_k2880", "g_moe_gdn_mxfp4_k2880", "g_moe_gu_mxfp4_k2880_r2",
                     "g_moe_dn_mxfp4_k2880_r2", "g_mv_q4_k_k4096_q8_r1", "g_gemm_q4_k_acc_m256"]),
])
def test_every_model_kernel_name_maps_to_an_exported_entry_point(lib, model, expect):
    from qmm import launch
    names = model_names(model)
    for e in expect:
        assert e in names, (e, names)
    cfg = launch.Config(experts=32, used=4)
    for name in names:
        ep = launch.entry_point(name, cfg)
        assert hasattr(lib, ep), f"{name} -> {ep}, which libqmm.so does not export"


@pytest.mark.parametrize("name", ["g_mv_q5_k_k4096", "g_mv_iq4_xs_k4096_q8", "g_moe_ggu_iq4_xs_k2048",
                                  "g_attn_prefill_h128", "g_mv_q4_k_k4096_pair", "g_gemm_q4_k_store_m512",
                                  "g_moe_gu_q4_k_k2048", "g_mv_q4_k_kx"])
def test_unknown_names_are_refused(name):
    from qmm import launch
    with pytest.raises(KeyError):
        launch.entry_point(name)


def test_gate_up_kernels_in_two_formats_map_to_the_gate_up_entry_points(lib):
    """The reference's "GATE+UP" kernels of a layer whose gate and up tensors differ in format (a Q4_K_M layer with
    a Q4_K gate and a Q6_K up, S/gen_llm.py:5335-5336): g_gemm_{fmt}_{fmt2}_swiglu (S/gen_gemm.py:535-547),
    g_moe_ggu_{fg}_{fu}_k{H} (S/gen_moe.py:1126-1141) and g_moe_gu_{fg}_{fu}_k{H}_r{R} (S/gen_moe.py:535-552) call the
    gate/up entry points with QMM_GATE_UP(gate, up); a second format anywhere else is refused."""
    from qmm import launch
    from qmm.formats import CODE
    names = {"g_gemm_q4_k_q6_k_swiglu": "qmm_gemm", "g_gemm_q6_k_q4_k_swiglu_m256": "qmm_gemm",
             "g_moe_ggu_q4_k_q6_k_k2048": "qmm_moe_grouped", "g_moe_gu_q4_k_q6_k_k2048_r2": "qmm_moe_expert_mv",
             "g_moe_gu_q4_0_mxfp4_k2880_r2": "qmm_moe_expert_mv"}
    for name, ep in names.items():
        assert launch.entry_point(name) == ep and hasattr(lib, ep), name
        fam, f = launch.parse(name)
        assert launch._fcode(f) == CODE[f["fmt"]] | ((CODE[f["fmt2"]] + 1) << 8), name
    for bad in ("g_gemm_q4_k_q6_k_store", "g_moe_dn_q4_k_q6_k_k768_r4", "g_moe_gdn_q4_k_q6_k_k768",
                "g_moe_gu_q4_k_q6_k_q8_k2048_r2", "g_moe_ggu_q4_k_q6_k_fused_k2048"):
        with pytest.raises(KeyError):
            launch.entry_point(bad)


def test_malformed_launches_fail_before_any_device_call():
    """Argument counts and grids are checked against the reference's launch lists first (ints stand in for
    buffers: a check that came later would fail on them with another error)."""
    from qmm import launch
    L = launch.Launcher(launch.Config(experts=128, used=8))
    with pytest.raises(ValueError, match="arguments"):
        L.launch("g_mv_q4_k_k4096_q8", [4096, 1], [4096, 1, 0, 1, 2])
    with pytest.raises(ValueError, match="grid"):
        L.launch("g_mv_q4_k_k4096_q8", [4096, 2], [4096, 1, 0, 1, 2, 3])
    with pytest.raises(ValueError, match="arguments"):
        L.launch("g_moe_ggu_q4_k_k2048", [8704, 768], [8704, 2048, 768, 64, 1, 2, 3, 4, 5, 6])
    with pytest.raises(ValueError, match="K 2048"):
        L.launch("g_moe_ggu_q4_k_k2048", [8704, 768], [8704, 1024, 768, 64, 1, 2, 3, 4, 5, 6, 7])
    with pytest.raises(ValueError, match="grid"):
        L.launch("g_moe_bucket", [63], [64, 136, 1, 2, 3, 4, 5])
    with pytest.raises(ValueError, match="Config"):
        launch.Launcher().launch("g_moe_bucket", [64], [64, 136, 1, 2, 3, 4, 5])
