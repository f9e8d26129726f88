"""Pins the oracle's weight decoders (oracle/formats.py) -- CPU only.

Each decoder is checked against something other than itself:

* Q4_0   the reference's exhaustive construction over every finite f16 scale x all 16 codes
         (.github/devlab/kbench/moe_q4_0/gen_bench.py:51-63, tests/test_moe_q4_0.py:90-112), with the required f16
         bit patterns; the f16 half-multiply property (tests/test_moe_q4_0.py:24-33); a float64 decoder written from
         the closed form; the nibble-swap negative control (tests/test_moe_q4_0.py:77-84).
* Q4_K   a scalar decoder that follows ggml's dequantize_row_q4_K loop (two sub-blocks per 32-byte page, low nibbles
         then high nibbles, get_scale_min_k4 for the 6-bit fields) against the vectorized one, bit for bit; a
         hand-built known-answer block; the scale packer's round trip over all 64 x 64 (sc, m) pairs at every
         sub-block; the reference's real Q4_K bytes (Qwen3-0.6B ffn_gate / ffn_up).
* Q6_K   no Q6_K bytes or vectors exist in the reference: a scalar decoder that follows ggml's
         dequantize_row_q6_K loop (four values per ql / qh lane, then the pointer advance) against the vectorized
         one (group formula of S/gen_llm.py:320-325), bit for bit; two hand-built known-answer blocks; the sign of
         the int8 scales and the single rounding of the value.
* MXFP4  the reference's split-plane KAT (tests/test_safetensors_source.py:200-206) and its scalar vLLM-table
         decoder (:92-103) on random planes; GGUF blocks against a scalar ggml decoder (kvalues x 2^(e-128) with
         the e < 2 subnormal rule), and GGUF <-> split equivalence up to the sign of zero.
"""
import json
import os

import numpy as np
import pytest

from oracle import formats as of

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
with open(os.path.join(GOLDEN, "kats.json")) as _f:
    KATS = json.load(_f)


# ------------------------------------------------------------------------------------------------------- Q4_0
def q4_0_all_scales():
    bits = np.arange(65536, dtype=np.uint16)
    bits = bits[(bits & 0x7C00) != 0x7C00]
    raw = np.empty((bits.size, 18), np.uint8)
    raw[:, :2] = bits.astype("<u2").view(np.uint8).reshape(-1, 2)
    codes = np.arange(16, dtype=np.uint8)
    raw[:, 2:] = codes | ((15 - codes) << 4)
    return bits, raw


def q4_0_f64(raw):
    """Closed form in float64: d * (q - 8), element j < 16 = low nibble of qs[j], j >= 16 = high nibble of qs[j-16]."""
    b = raw.reshape(-1, 18)
    d = b[:, :2].copy().view("<f2").reshape(-1).astype(np.float64)
    out = np.empty((b.shape[0], 32))
    for j in range(16):
        out[:, j] = d * ((b[:, 2 + j] & 15).astype(np.float64) - 8)
        out[:, 16 + j] = d * ((b[:, 2 + j] >> 4).astype(np.float64) - 8)
    return out


def test_q4_0_every_finite_scale_and_code():
    bits, raw = q4_0_all_scales()
    assert bits.size == KATS["q4_0_scale_count"]
    got = of.dequant_q4_0(raw, bits.size, 32)
    exact = q4_0_f64(raw)
    # the f32 product of an f16 scale and a 4-bit integer is exact
    assert np.array_equal(got.astype(np.float64), exact)
    with np.errstate(over="ignore"):
        h = got.astype(np.float16).view(np.uint16)
    for pattern in KATS["q4_0_required_f16_bits"]:
        assert np.any(h == pattern), hex(pattern)
    for pattern in KATS["q4_0_never_f16_bits"]:
        assert not np.any(h == pattern)


def test_q4_0_half_multiply_property():
    """f16(f32(d) * c) == f16(d * c) for every finite f16 d and c in -8..7: one rounding of the exact product."""
    scales = np.arange(65536, dtype=np.uint16).view(np.float16)
    scales = scales[np.isfinite(scales)][:, None]
    codes = np.arange(-8, 8, dtype=np.float16)[None, :]
    with np.errstate(over="ignore", invalid="ignore"):
        half = (scales * codes).astype(np.float16)
        wide = (scales.astype(np.float32) * codes.astype(np.float32)).astype(np.float16)
    assert np.array_equal(half.view(np.uint16), wide.view(np.uint16))


def test_q4_0_signed_scales_and_nibble_swap_negative_control():
    rng = np.random.default_rng(47)
    nb = 3 * 64 * 704 // 32
    raw = np.empty((nb, 18), np.uint8)
    scale = (rng.uniform(.0005, .003, nb) * rng.choice([-1, 1], nb)).astype("<f2")
    raw[:, :2] = scale.view(np.uint8).reshape(-1, 2)
    raw[:, 2:] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    got = of.dequant_q4_0(raw, 3 * 64, 704)
    exact = q4_0_f64(raw).reshape(3 * 64, 704)
    assert np.array_equal(got.astype(np.float64), exact)
    swapped = raw.copy()
    swapped[:, 2:] = (swapped[:, 2:] << 4) | (swapped[:, 2:] >> 4)
    assert np.max(np.abs(of.dequant_q4_0(swapped, 3 * 64, 704) - exact)) > .01


# ------------------------------------------------------------------------------------------------------- Q4_K
def get_scale_min_k4(j, q):
    """ggml get_scale_min_k4, written from its published definition (12 scale bytes q, sub-block j)."""
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def q4_k_scalar(raw):
    """ggml dequantize_row_q4_K's loop, element by element in float32: per 64-value step, sub-blocks is and is+1
    share 32 code bytes (low nibbles, then high nibbles); y = d1 * q - m1 with d1 = d * sc, m1 = dmin * m."""
    b = np.asarray(raw, np.uint8).reshape(-1, 144)
    out = np.empty((b.shape[0], 256), np.float32)
    for i in range(b.shape[0]):
        d = np.float32(b[i, 0:2].copy().view("<f2")[0])
        dmin = np.float32(b[i, 2:4].copy().view("<f2")[0])
        sc = [int(v) for v in b[i, 4:16]]
        q = b[i, 16:144]
        o = 0
        for step in range(4):
            s1, m1 = get_scale_min_k4(2 * step, sc)
            s2, m2 = get_scale_min_k4(2 * step + 1, sc)
            d1, mm1 = np.float32(d * np.float32(s1)), np.float32(dmin * np.float32(m1))
            d2, mm2 = np.float32(d * np.float32(s2)), np.float32(dmin * np.float32(m2))
            page = q[32 * step: 32 * step + 32]
            for l in range(32):
                out[i, o + l] = np.float32(d1 * np.float32(page[l] & 0xF)) - mm1
            for l in range(32):
                out[i, o + 32 + l] = np.float32(d2 * np.float32(page[l] >> 4)) - mm2
            o += 64
    return out


def random_q4_k(rng, nb, extreme=False):
    raw = np.empty((nb, 144), np.uint8)
    if extreme:   # any f16 bit pattern that is finite, both signs
        d = rng.integers(0, 65536, nb).astype(np.uint16)
        d = np.where((d & 0x7C00) == 0x7C00, d & 0x83FF, d)
        dm = rng.integers(0, 65536, nb).astype(np.uint16)
        dm = np.where((dm & 0x7C00) == 0x7C00, dm & 0x83FF, dm)
        raw[:, 0:2] = d.astype("<u2").view(np.uint8).reshape(-1, 2)
        raw[:, 2:4] = dm.astype("<u2").view(np.uint8).reshape(-1, 2)
        raw[:, 4:] = rng.integers(0, 256, (nb, 140), dtype=np.uint8)
    else:
        raw[:] = rng.integers(0, 256, (nb, 144), dtype=np.uint8)
        raw[:, 0:2] = np.abs(rng.normal(0, .01, nb)).astype("<f2").view(np.uint8).reshape(-1, 2)
        raw[:, 2:4] = np.abs(rng.normal(0, .01, nb)).astype("<f2").view(np.uint8).reshape(-1, 2)
    return raw.reshape(-1)


@pytest.mark.parametrize("extreme", [False, True])
def test_q4_k_vectorized_equals_scalar_ggml_loop(extreme):
    rng = np.random.default_rng(3 + extreme)
    raw = random_q4_k(rng, 48, extreme)
    got = of.dequant_q4_k(raw, 3, 16 * 256)
    want = q4_k_scalar(raw).reshape(3, -1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q4_k_known_answer_block():
    """d = 0.5, dmin = 0.25, sub-block g has scale g + 1 (g odd: + 32) and minimum 2 g + 1, codes (l + g) % 16;
    value = 0.5 sc q - 0.25 m, every one exactly representable."""
    sc = np.array([g + 1 + (32 if g % 2 else 0) for g in range(8)])
    m = np.array([2 * g + 1 for g in range(8)])
    raw = np.zeros(144, np.uint8)
    raw[0:2] = np.array([0.5], "<f2").view(np.uint8)
    raw[2:4] = np.array([0.25], "<f2").view(np.uint8)
    raw[4:16] = of.q4_k_pack_scale_min(sc, m)
    codes = np.array([[(l + g) % 16 for l in range(32)] for g in range(8)], np.uint8)
    for p in range(4):
        raw[16 + 32 * p: 48 + 32 * p] = codes[2 * p] | (codes[2 * p + 1] << 4)
    want = np.array([[0.5 * sc[g] * codes[g, l] - 0.25 * m[g] for l in range(32)] for g in range(8)]).reshape(-1)
    assert np.array_equal(of.dequant_q4_k(raw, 1, 256).reshape(-1).astype(np.float64), want)


def test_q4_k_scale_packing_round_trip_all_values():
    v = np.arange(64)
    sc_all, m_all = np.meshgrid(v, v, indexing="ij")
    sc_all, m_all = sc_all.reshape(-1), m_all.reshape(-1)
    for g in range(8):
        sc = np.zeros((sc_all.size, 8), np.int32)
        m = np.zeros_like(sc)
        sc[:, g] = sc_all
        m[:, g] = m_all
        sc[:, (g + 3) % 8] = 63 - sc_all      # a neighbour with other bits, so crosstalk would show
        m[:, (g + 5) % 8] = m_all[::-1]
        S = of.q4_k_pack_scale_min(sc, m)
        rsc, rm = of.q4_k_scale_min(S)
        assert np.array_equal(rsc, sc) and np.array_equal(rm, m)
        # and the scalar get_scale_min_k4 agrees on a sample
        for i in range(0, sc_all.size, 397):
            assert get_scale_min_k4(g, [int(x) for x in S[i]]) == (sc[i, g], m[i, g])


@pytest.mark.parametrize("name", ["q4k_real_gate_64rows", "q4k_real_up_64rows"])
def test_q4_k_real_weights(name):
    """The reference's real Q4_K bytes (Qwen3-0.6B layer 3): scalar and vectorized decoders agree bit for bit and the
    values look like trained weights (finite, centred, every sub-block within its d*sc*15 - dmin*m range)."""
    raw = np.load(os.path.join(GOLDEN, name + ".npy"), allow_pickle=False)
    rows, k = KATS["real_q4k"]["rows"], KATS["real_q4k"]["k"]
    got = of.dequant_q4_k(raw, rows, k)
    assert np.array_equal(got.view(np.uint32), q4_k_scalar(raw).reshape(rows, k).view(np.uint32))
    assert np.all(np.isfinite(got))
    assert abs(float(got.mean())) < 0.01 and 0.005 < float(got.std()) < 0.2
    d, dmin, sc, m, q = of.q4_k_fields(raw)
    lo = -(dmin[:, None] * m)
    hi = d[:, None] * sc * 15 - dmin[:, None] * m
    g = got.reshape(-1, 8, 32)
    assert np.all(g >= lo[:, :, None] - 1e-7) and np.all(g <= hi[:, :, None] + 1e-7)


# ------------------------------------------------------------------------------------------------------- Q6_K
def q6_k_scalar(raw):
    """ggml's dequantize_row_q6_K, element by element: per 128-value half, the lane l of 32 yields four values
    l, l+32, l+64, l+96 from ql[l] and ql[l+32] (low nibbles, then high nibbles) and the four 2-bit fields of
    qh[l], with the scale sc[l/16 + 0, 2, 4, 6]; pointers then advance by 64 ql, 32 qh and 8 scale bytes."""
    b = np.asarray(raw, np.uint8).reshape(-1, 210)
    out = np.zeros((b.shape[0], 256), np.float32)
    for i, blk in enumerate(b):
        d = np.frombuffer(blk[208:210].tobytes(), "<f2")[0].astype(np.float32)
        sc = blk[192:208].view(np.int8)
        for n in range(2):
            ql, qh, s = blk[64 * n:64 * n + 64], blk[128 + 32 * n:160 + 32 * n], sc[8 * n:8 * n + 8]
            for l in range(32):
                i16 = l // 16
                h = int(qh[l])
                q1 = (int(ql[l]) & 15) | ((h >> 0) & 3) << 4
                q2 = (int(ql[l + 32]) & 15) | ((h >> 2) & 3) << 4
                q3 = (int(ql[l]) >> 4) | ((h >> 4) & 3) << 4
                q4 = (int(ql[l + 32]) >> 4) | ((h >> 6) & 3) << 4
                for off, q, si in ((0, q1, 0), (32, q2, 2), (64, q3, 4), (96, q4, 6)):
                    out[i, 128 * n + l + off] = np.float32(d * np.float32(s[i16 + si])) * np.float32(q - 32)
    return out


@pytest.mark.parametrize("seed", [0, 1])
def test_q6_k_vectorized_equals_scalar_ggml_loop(seed):
    from qmm import synth
    rng = np.random.default_rng(900 + seed)
    raw = synth.q6_k_weights(rng, 3, 512, sigma=0.5 if seed else 0.002)
    got = of.dequant_q6_k(raw, 3, 512)
    assert np.array_equal(got.view(np.uint32), q6_k_scalar(raw).reshape(3, 512).view(np.uint32))


def test_q6_k_known_answer_blocks():
    """Hand-built blocks. (1) every ql byte 0x21, every qh byte 0xE4 (fields 0, 1, 2, 3), scales 1..16, d = 0.5:
    group j of either half has code 1, 17, 34, 50 (values -31, -15, 2, 18 times 0.5 sc). (2) ql[i] = i, qh = 0,
    scales 1, d = 1: value c = 128 h + 32 j + l is ((64 h + 32 (j % 2) + l) >> 4 (j // 2) & 15) - 32."""
    blk = np.zeros(210, np.uint8)
    blk[0:128] = 0x21
    blk[128:192] = 0xE4
    blk[192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)
    blk[208:210] = np.array([0.5], "<f2").view(np.uint8)
    got = of.dequant_q6_k(blk, 1, 256).reshape(2, 4, 32)
    for h in range(2):
        for j in range(4):
            for l in range(32):
                want = 0.5 * (8 * h + 2 * j + l // 16 + 1) * (-31, -15, 2, 18)[j]
                assert got[h, j, l] == want, (h, j, l)
    blk = np.zeros(210, np.uint8)
    blk[0:128] = np.arange(128, dtype=np.uint8)
    blk[192:208] = 1
    blk[208:210] = np.array([1.0], "<f2").view(np.uint8)
    got = of.dequant_q6_k(blk, 1, 256).reshape(2, 4, 32)
    for h in range(2):
        for j in range(4):
            for l in range(32):
                assert got[h, j, l] == (((64 * h + 32 * (j % 2) + l) >> (4 * (j // 2))) & 15) - 32


def test_q6_k_signed_scales_and_single_rounding():
    """A negated int8 scale negates its 16 values; the second product rounds once in f32 (d sc exact, then x q)."""
    from qmm import synth
    rng = np.random.default_rng(901)
    raw = synth.q6_k_weights(rng, 1, 256, sigma=3.0)
    blk = raw.reshape(210).copy()
    sc = blk[192:208].view(np.int8).copy()
    sc[sc == -128] = 5
    blk[192:208] = sc.view(np.uint8)
    neg = blk.copy()
    neg[192:208] = (-sc).astype(np.int8).view(np.uint8)
    a, b = of.dequant_q6_k(blk, 1, 256), of.dequant_q6_k(neg, 1, 256)
    assert np.array_equal(a, -b)
    d, s, q = of.q6_k_fields(blk)
    exact = np.float64(d[0]) * np.repeat(s[0], 16).astype(np.float64) * (q[0] - 32)
    assert np.array_equal(a.reshape(-1), exact.astype(np.float32))   # one rounding of the exact product


# ------------------------------------------------------------------------------------------------------ MXFP4
def mxfp4s_scalar(nibbles, scales):
    """The reference test's scalar decoder (vLLM kE2M1x2 table, tests/test_safetensors_source.py:92-103)."""
    tab = [0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12]
    rows, half = nibbles.shape
    out = np.zeros((rows, half * 2), np.float32)
    for r in range(rows):
        for k in range(half * 2):
            byte = int(nibbles[r, k // 2])
            code = (byte >> 4) & 15 if k & 1 else byte & 15
            out[r, k] = tab[code] * 0.5 * 2.0 ** (int(scales[r, k // 32]) - 127)
    return out


def test_mxfp4s_kat():
    kat = KATS["mxfp4_split"]
    nib = np.zeros((1, 16), np.uint8)
    nib[0, :2] = kat["nibbles"]
    out = of.dequant_mxfp4s(nib, np.array([[kat["e8m0"]]], np.uint8), 1, 32)
    assert out[0, :4].tolist() == kat["values"]


def test_mxfp4s_matches_scalar_table_decoder():
    rng = np.random.default_rng(1)
    nib = rng.integers(0, 256, (7, 96), dtype=np.uint8)
    sc = rng.integers(100, 130, (7, 6), dtype=np.uint8)
    assert np.array_equal(of.dequant_mxfp4s(nib, sc, 7, 192), mxfp4s_scalar(nib, sc))


def mxfp4_ggml_scalar(raw):
    """ggml dequantize_row_mxfp4: y = kvalues_mxfp4[code] * GGML_E8M0_TO_FP32_HALF(e), codes in split16 order;
    2^(e-128) is built as an f32 bit pattern, with 0x00200000 << e for e < 2 (subnormals)."""
    b = np.asarray(raw, np.uint8).reshape(-1, 17)
    kv = [0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12]
    out = np.empty((b.shape[0], 32), np.float32)
    for i in range(b.shape[0]):
        e = int(b[i, 0])
        bits = (0x00200000 << e) if e < 2 else ((e - 1) << 23)
        half = np.array([bits], np.uint32).view(np.float32)[0]
        for j in range(16):
            out[i, j] = np.float32(kv[b[i, 1 + j] & 15]) * half
            out[i, j + 16] = np.float32(kv[b[i, 1 + j] >> 4]) * half
    return out


def test_mxfp4s_icodes_times_scale_is_the_weight_exactly():
    """The int8 weight codes of the opt-in MXFP4S_Q8 decode (of.mxfp4s_icodes) against the split-plane dequantization:
    codes x d equals the decoded value exactly for every nibble byte (all 16 x 16 low / high pairs, so every code in
    both halves) and every E8M0 byte whose values stay finite in f32 (0 .. 250, both subnormal scale bytes included);
    d itself is 2^(e - 128) for all 256 bytes. Negative control: the low / high nibbles swapped (the "split16" order of
    GGUF blocks) breaks the equality."""
    nib = np.arange(256, dtype=np.uint8)
    for e in range(256):
        assert of.mxfp4s_icodes(nib[:16], e)[1] == np.float32(np.ldexp(1.0, e - 128)), e
    for e in range(251):
        for b0 in range(0, 256, 16):
            blk = nib[b0:b0 + 16]
            codes, d = of.mxfp4s_icodes(blk, e)
            got = codes.astype(np.float64) * np.float64(d)
            want = of.dequant_mxfp4s(blk, np.array([e], np.uint8), 1, 32).reshape(32).astype(np.float64)
            assert np.array_equal(got, want), (e, b0)
    blk = nib[16:32]
    codes, d = of.mxfp4s_icodes(blk, 127)
    swapped = np.concatenate([codes[0::2], codes[1::2]]).astype(np.float64) * np.float64(d)
    assert not np.array_equal(swapped, of.dequant_mxfp4s(blk, np.array([127], np.uint8), 1, 32).reshape(32))


def test_mxfp4_gguf_matches_scalar_ggml_decoder_all_exponents():
    rng = np.random.default_rng(9)
    raw = np.empty((254 * 2, 17), np.uint8)
    raw[:, 0] = np.repeat(np.arange(254), 2)          # every exponent byte except the NaN encoding 255
    raw[:, 1:] = rng.integers(0, 256, (raw.shape[0], 16), dtype=np.uint8)
    with np.errstate(over="ignore"):
        got = of.dequant_mxfp4(raw, raw.shape[0], 32)
        want = mxfp4_ggml_scalar(raw)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.all(np.isfinite(got[raw[:, 0] <= 252]))   # 8 * 2^(253-128) overflows f32, in ggml as here


def test_mxfp4_gguf_and_split_agree_up_to_the_sign_of_zero():
    rng = np.random.default_rng(4)
    rows, k = 5, 2880
    raw = np.empty((rows * k // 32, 17), np.uint8)
    raw[:, 0] = 127 + rng.integers(-8, 1, raw.shape[0])
    raw[:, 1:] = rng.integers(0, 256, (raw.shape[0], 16), dtype=np.uint8)
    g = of.dequant_mxfp4(raw, rows, k)
    nib, sc = of.mxfp4_to_split(raw, rows, k)
    s = of.dequant_mxfp4s(nib, sc, rows, k)
    assert np.array_equal(g, s)                       # == treats -0 and +0 as equal
    zeros = g == 0
    assert np.all(~np.signbit(g[zeros]))              # GGUF code 8 -> +0
    codes = np.concatenate([raw[:, 1:] & 15, raw[:, 1:] >> 4], axis=1).reshape(rows, k)
    assert np.all(np.signbit(s[codes == 8]))          # split convention: code 8 -> -0


def test_row_bytes_table():
    assert of.row_bytes("q4_0", 2816) == 1584           # tests/test_moe_q4_0.py:36
    assert of.row_bytes("q4_k", 4096) == 2304
    assert of.row_bytes("mxfp4", 2880) == 1530
    assert of.row_bytes("mxfp4s", 2880) == 1440
    with pytest.raises(AssertionError):
        of.row_bytes("q4_k", 100)


# --------------------------------------------------------------------------------------- MXFP4 MFMA-tiled planes
def _split_planes(rng, rows, k):
    nib = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
    sc = (127 + rng.integers(-8, 1, (rows, k // 32))).astype(np.uint8)
    return nib, sc


def test_mxfp4t_byte_addresses_follow_the_layout_definition():
    """Every nibble byte and scale byte lands at the address the layout defines, computed here as a flat offset:
    nibble byte j of row r -> ((r // 32 * C + j // 32) * 64 + 32 * ((j % 32) // 16) + r % 32) * 16 + j % 16;
    scale of block b of row r -> ((r // 32 * C4 + b // 8) * 64 + 32 * (b % 2) + r % 32) * 4 + (b // 2) % 4."""
    rng = np.random.default_rng(11)
    rows, k = 64, 2880                        # C = 45 chunks: the last group of four holds one real chunk
    C, C4 = k // 64, (k // 64 + 3) // 4
    nib, sc = _split_planes(rng, rows, k)
    nt, st = of.mxfp4s_to_tiled(nib, sc, rows, k)
    assert nt.size == rows * k // 2 and st.size == rows // 32 * C4 * 256
    r, j = np.meshgrid(np.arange(rows), np.arange(k // 2), indexing="ij")
    off = ((r // 32 * C + j // 32) * 64 + 32 * ((j % 32) // 16) + r % 32) * 16 + j % 16
    assert np.array_equal(nt[off], nib)
    r, b = np.meshgrid(np.arange(rows), np.arange(k // 32), indexing="ij")
    soff = ((r // 32 * C4 + b // 8) * 64 + 32 * (b % 2) + r % 32) * 4 + (b // 2) % 4
    assert np.array_equal(st[soff], sc)
    used = np.zeros(st.size, bool)
    used[soff.ravel()] = True
    assert np.all(st[~used] == 0)             # chunks past K carry scale 0


def test_mxfp4t_round_trip_and_values():
    rng = np.random.default_rng(12)
    for rows, k in ((32, 64), (96, 2880), (64, 768)):
        nib, sc = _split_planes(rng, rows, k)
        nt, st = of.mxfp4s_to_tiled(nib, sc, rows, k)
        n2, s2 = of.mxfp4t_to_split(nt, st, rows, k)
        assert np.array_equal(n2, nib) and np.array_equal(s2, sc)
        want = of.dequant_mxfp4s(nib, sc, rows, k)
        got = of.dequant_mxfp4t(nt, st, rows, k)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_mxfp4t_lane_half_swap_negative_control():
    """Swapping the two lane halves of every tile (K values 0..31 <-> 32..63 of each chunk) must change the values."""
    rng = np.random.default_rng(13)
    rows, k = 32, 256
    nib, sc = _split_planes(rng, rows, k)
    nt, st = of.mxfp4s_to_tiled(nib, sc, rows, k)
    bad = nt.reshape(-1, 2, 32, 16)[:, ::-1].reshape(-1)
    assert not np.array_equal(of.dequant_mxfp4t(bad, st, rows, k), of.dequant_mxfp4s(nib, sc, rows, k))


# ------------------------------------------------------------------------------------------- Q4_K tiled layout
@pytest.mark.parametrize("k", [1536, 1280, 256])
def test_q4_kt_byte_addresses_follow_the_layout_definition(k):
    """Every byte of every GGUF Q4_K block lands where the tiled layout puts it, computed as a flat offset: for row
    r, super-block b and byte j of its 144, row block base B = (r // 16) 16 (K / 256) 144, i = r % 16; in a full
    unit (b < 2 (K // 512)): u = b // 2, sb = b % 2, header byte j < 16 -> B + 4608 u + 16 (2 i + sb) + j, code
    byte c = j - 16 -> B + 4608 u + 512 + 1024 ((c // 16) % 4) + 16 (4 i + 2 sb + c // 64) + c % 16; in the half
    unit of K % 512 == 256 (the last super-block): header -> B + 4608 F + 16 i + j, code -> B + 4608 F + 256
    + 512 ((c // 16) % 4) + 16 (2 i + c // 64) + c % 16 (F = K // 512)."""
    from qmm import synth
    rng = np.random.default_rng(21)
    rows = 32
    raw = synth.q4_k_weights(rng, rows, k).reshape(rows, k // 256, 144)
    t = of.q4_k_to_tiled(raw, rows, k)
    assert t.size == raw.size
    r, b, j = np.meshgrid(np.arange(rows), np.arange(k // 256), np.arange(144), indexing="ij")
    F = k // 512
    B = (r // 16) * 16 * (k // 256) * 144
    u, sb, i, c = b // 2, b % 2, r % 16, j - 16
    full = np.where(j < 16, B + 4608 * u + 16 * (2 * i + sb) + j,
                    B + 4608 * u + 512 + 1024 * ((c // 16) % 4) + 16 * (4 * i + 2 * sb + c // 64) + c % 16)
    tail = np.where(j < 16, B + 4608 * F + 16 * i + j,
                    B + 4608 * F + 256 + 512 * ((c // 16) % 4) + 16 * (2 * i + c // 64) + c % 16)
    off = np.where(b < 2 * F, full, tail)
    assert np.array_equal(np.sort(off.ravel()), np.arange(raw.size))    # a permutation
    assert np.array_equal(t[off], raw)


def test_q4_kt_round_trip_and_values():
    from qmm import synth
    rng = np.random.default_rng(22)
    for rows, k in ((16, 512), (48, 4096), (32, 768), (16, 256)):
        raw = synth.q4_k_weights(rng, rows, k)
        t = of.q4_k_to_tiled(raw, rows, k)
        assert np.array_equal(of.q4_kt_to_gguf(t, rows, k), np.asarray(raw).reshape(-1))
        want = of.dequant_q4_k(raw, rows, k)
        assert np.array_equal(of.dequant_q4_kt(t, rows, k).view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------------------------------- Q4_0 tiled layout
def _q4_0_signed(rng, rows, k):
    """Q4_0 blocks with scales of both signs (synth draws positive ones)."""
    from qmm import synth
    raw = synth.q4_0_weights(rng, rows, k).reshape(-1, 18).copy()
    raw[::3, 1] |= 0x80
    return raw.reshape(-1)


@pytest.mark.parametrize("rows,k", [(16, 512), (32, 1024)])
def test_q4_0t_addresses_follow_the_layout_definition(rows, k):
    """Every scale byte and every code nibble of every GGUF Q4_0 block lands where the tiled layout puts it, as a flat
    offset: row r, block b, code i (value 32 b + i); rb = r // 16, s = r % 16, unit u = b // 16, span sb = (b // 8)
    % 2, j = b % 8, unit base B = 4608 (rb (K / 512) + u); d byte e -> B + 16 (2 s + sb) + 2 j + e; span byte
    c = 32 (j // 2) + i -> B + 512 + 1024 ((c // 16) % 4) + 16 (4 s + 2 sb + c // 64) + c % 16, low nibble for even j."""
    rng = np.random.default_rng(31)
    raw = _q4_0_signed(rng, rows, k)
    t = of.q4_0_to_tiled(raw, rows, k)
    assert t.size == raw.size
    blk = raw.reshape(rows, k // 32, 18)
    r, b, i = np.meshgrid(np.arange(rows), np.arange(k // 32), np.arange(32), indexing="ij")
    s, u, sb, j = r % 16, b // 16, (b // 8) % 2, b % 8
    B = 4608 * ((r // 16) * (k // 512) + u)
    c = 32 * (j // 2) + i
    off = B + 512 + 1024 * ((c // 16) % 4) + 16 * (4 * s + 2 * sb + c // 64) + c % 16
    nib = np.where(j % 2 == 0, t[off] & 15, t[off] >> 4)
    code = np.where(i < 16, blk[r, b, 2 + i % 16] & 15, blk[r, b, 2 + i % 16] >> 4)
    assert np.array_equal(nib, code)
    for e in range(2):
        doff = B[..., 0] + 16 * (2 * s[..., 0] + sb[..., 0]) + 2 * j[..., 0] + e
        assert np.array_equal(t[doff], blk[:, :, e])
    # the code planes are a permutation of nibbles: every plane byte is named exactly twice, once per nibble
    cnt = np.bincount((2 * off + j % 2).ravel(), minlength=2 * t.size).reshape(-1, 4608, 2)
    assert (cnt[:, 512:] == 1).all() and (cnt[:, :512] == 0).all()


def test_q4_0t_round_trip_and_values():
    rng = np.random.default_rng(32)
    for rows, k in ((16, 512), (48, 2048), (32, 1536)):
        raw = _q4_0_signed(rng, rows, k)
        t = of.q4_0_to_tiled(raw, rows, k)
        assert np.array_equal(of.q4_0t_to_gguf(t, rows, k), raw)
        want = of.dequant_q4_0(raw, rows, k)
        assert np.array_equal(of.dequant_q4_0t(t, rows, k).view(np.uint32), want.view(np.uint32))


def test_q4_0t_span_page_swap_negative_control():
    """Swapping the two nibbles of every code byte (blocks 2 p <-> 2 p + 1 of a page) must change the values."""
    rng = np.random.default_rng(33)
    rows, k = 16, 512
    raw = _q4_0_signed(rng, rows, k)
    t = of.q4_0_to_tiled(raw, rows, k)
    bad = t.copy().reshape(-1, 4608)
    bad[:, 512:] = (bad[:, 512:] >> 4) | (bad[:, 512:] << 4)
    assert not np.array_equal(of.dequant_q4_0t(bad.reshape(-1), rows, k), of.dequant_q4_0(raw, rows, k))
