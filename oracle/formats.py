"""Bit-exact CPU decoders of the weight formats on the quantized matmul path (oracle; test infrastructure only).

All byte orders are little endian. Every decoder returns float32 values produced with at most one rounding, exactly
as the reference's decoders do, so any correct implementation reproduces them bit for bit:

* Q4_0  (18 B / 32 values)   S/quant_values.loom:386-408, S/moe_q4_0.py:1-38,
                             .github/devlab/kbench/moe_q4_0/gen_bench.py:19-25
* Q4_K  (144 B / 256 values) S/gen_llm.py:234-326 (@g_k_scale_minimum, @g_k_metadata, @g_q4_k_values)
* Q6_K  (210 B / 256 values) S/gen_llm.py:320-397 (@g_q6_k_values); ggml's dequantize_row_q6_K (gguf-py
                             quants.Q6_K, the reference's oracle dependency, make_kernel_tests.py:44-55) restated
* MXFP4 GGUF (17 B / 32)     S/gen_llm.py:786-841 (@g_mxfp4_values)
* MXFP4 split planes         S/gen_llm.py:844-895 (@g_mxfp4s_values), S/st_tensors.py:17-33 (dequant_mxfp4)
* MXFP4 MFMA-tiled planes    this library's load-time layout of the split planes (no reference counterpart); a byte
                             permutation, so its values are the split planes' values
* Q4_K tiled                 this library's load-time layout of GGUF Q4_K for the decode GEMV (lane-ordered units of
                             16 rows x 512 values); a byte permutation of the GGUF blocks
"""
import numpy as np

# bytes per block and values per block (S/formats.py:5-19)
BLOCK_BYTES = {"q4_0": 18, "q4_k": 144, "mxfp4": 17, "mxfp4s": 16, "q6_k": 210}
BLOCK_VALUES = {"q4_0": 32, "q4_k": 256, "mxfp4": 32, "mxfp4s": 32, "q6_k": 256}

# E2M1 magnitudes; bit 3 of a code is the sign (S/st_tensors.py:17-22)
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float64)
# ggml's kvalues_mxfp4: twice the E2M1 values, code 8 is +0 (S/gen_llm.py:821-829)
KVALUES_MXFP4 = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], np.int8)


def row_bytes(fmt, k):
    """Bytes of one weight row of K values (S/gen_llm.py:182-183)."""
    assert k % BLOCK_VALUES[fmt] == 0, (fmt, k)
    return k // BLOCK_VALUES[fmt] * BLOCK_BYTES[fmt]


def _blocks(raw, fmt):
    b = np.ascontiguousarray(np.asarray(raw).view(np.uint8).reshape(-1))
    assert b.size % BLOCK_BYTES[fmt] == 0, (fmt, b.size)
    return b.reshape(-1, BLOCK_BYTES[fmt])


def _f16(two_bytes):
    return np.ascontiguousarray(two_bytes).view("<f2").reshape(-1).astype(np.float32)


def dequant_q4_0(raw, rows, k):
    """Q4_0: d = f16 bytes 0..1, qs = bytes 2..17; value j = f32(d) * (q_j - 8), q_j the low nibble of qs[j] for
    j < 16 and the high nibble of qs[j-16] otherwise (S/quant_values.loom:386-408). The product is exact in f32."""
    b = _blocks(raw, "q4_0")
    d = _f16(b[:, 0:2])
    qs = b[:, 2:18]
    q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.int32) - 8
    return (d[:, None] * q.astype(np.float32)).astype(np.float32).reshape(rows, k)


def q4_k_scale_min(S):
    """The 6-bit (scale, minimum) of the 8 sub-blocks from the 12 packed scale bytes S [..., 12] (ggml
    get_scale_min_k4, restated from S/gen_llm.py:234-267): g < 4: sc = S[g] & 63, m = S[g+4] & 63; g >= 4:
    sc = (S[g+4] & 15) | (S[g-4] >> 6) << 4, m = (S[g+4] >> 4) | (S[g] >> 6) << 4."""
    S = np.asarray(S).astype(np.int32)
    sc = np.empty(S.shape[:-1] + (8,), np.int32)
    m = np.empty_like(sc)
    sc[..., :4] = S[..., 0:4] & 63
    m[..., :4] = S[..., 4:8] & 63
    sc[..., 4:] = (S[..., 8:12] & 15) | ((S[..., 0:4] >> 6) << 4)
    m[..., 4:] = (S[..., 8:12] >> 4) | ((S[..., 4:8] >> 6) << 4)
    return sc, m


def q4_k_pack_scale_min(sc, m):
    """Inverse of q4_k_scale_min: 8 six-bit scales and minima -> the 12 packed bytes (used to build synthetic and
    known-answer blocks; the round trip over all 64 x 64 values is a test)."""
    sc = np.asarray(sc).astype(np.int32)
    m = np.asarray(m).astype(np.int32)
    S = np.empty(sc.shape[:-1] + (12,), np.int32)
    S[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    S[..., 4:8] = (m[..., 0:4] & 63) | ((m[..., 4:8] >> 4) << 6)
    S[..., 8:12] = (sc[..., 4:8] & 15) | ((m[..., 4:8] & 15) << 4)
    return S.astype(np.uint8)


def q4_k_fields(raw):
    """(d f32 [nb], dmin f32 [nb], sc i32 [nb,8], m i32 [nb,8], q u8 [nb,8,32]) of Q4_K super-blocks: sub-block
    g = 2p + h holds the nibble h (0 low, 1 high) of qs[32p .. 32p+31] (S/gen_llm.py:288-326)."""
    b = _blocks(raw, "q4_k")
    d, dmin = _f16(b[:, 0:2]), _f16(b[:, 2:4])
    sc, m = q4_k_scale_min(b[:, 4:16])
    qs = b[:, 16:144].reshape(-1, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32)
    return d, dmin, sc, m, q


def dequant_q4_k(raw, rows, k):
    """Q4_K: value = (f32(d) * sc_g) * q - f32(dmin) * m_g. Both products are exact in f32 (at most 21 significant
    bits), so the single rounding is the subtraction (S/gen_llm.py:269-326)."""
    d, dmin, sc, m, q = q4_k_fields(raw)
    scale = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
    minimum = (dmin[:, None] * m.astype(np.float32)).astype(np.float32)
    v = scale[:, :, None] * q.astype(np.float32) - minimum[:, :, None]
    return v.astype(np.float32).reshape(rows, k)


def e8m0_half_scale(e):
    """ggml GGML_E8M0_TO_FP32_HALF: 2^(e - 128) as f32 bits, (0x00200000 << e) for e < 2 (S/gen_llm.py:797-806)."""
    e = np.asarray(e).astype(np.uint32)
    bits = np.where(e < 2, np.uint32(0x00200000) << e, (e - np.uint32(1)) << np.uint32(23)).astype(np.uint32)
    return bits.view(np.float32)


def dequant_mxfp4(raw, rows, k):
    """MXFP4 GGUF block (17 B): e = byte 0, codes = bytes 1..16 in split16 order (value j < 16: low nibble of
    qs[j], j >= 16: high nibble of qs[j-16]); value = kvalues_mxfp4[code] * 2^(e-128) (S/gen_llm.py:786-841).
    Code 8 decodes to +0."""
    b = _blocks(raw, "mxfp4")
    half = e8m0_half_scale(b[:, 0])
    qs = b[:, 1:17]
    codes = np.concatenate([qs & 15, qs >> 4], axis=1)
    v = KVALUES_MXFP4[codes].astype(np.float32) * half[:, None]
    return v.astype(np.float32).reshape(rows, k)


def dequant_mxfp4s(nibbles, scales, rows, k):
    """MXFP4 split planes: nibbles [rows, K/2] in pairs order (byte j = element 2j low nibble, 2j+1 high nibble),
    scales [rows, K/32] E8M0; value = E2M1(code) * 2^(e - 127) (S/st_tensors.py:26-33). Code 8 decodes to -0, as the
    reference's numpy decoder does."""
    nib = np.asarray(nibbles).view(np.uint8).reshape(rows, k // 2)
    sc = np.asarray(scales).view(np.uint8).reshape(rows, k // 32)
    lut = np.concatenate([E2M1, -E2M1])
    v = np.stack([lut[nib & 15], lut[nib >> 4]], axis=-1).reshape(rows, k)
    s = np.exp2(sc.astype(np.float64) - 127.0)
    return (v.reshape(rows, -1, 32) * s[:, :, None]).reshape(rows, k).astype(np.float32)


def mxfp4s_icodes(nibbles16, e):
    """@g_mxfp4s_icodes (S/gen_mxfp4s.py:1113-1160), the weight side of the reference's opt-in int8 decode of MXFP4
    split planes (MXFP4S_Q8): a 32-value block's 16 nibble bytes (pairs order: value 2j is the low nibble of byte j,
    2j+1 the high nibble) give signed codes kvalues_mxfp4 (twice the E2M1 values; code 8 is 0), and its E8M0 byte e
    the block scale 2^(e - 128) (the codes carry the factor 2). Returns (codes int8 [32], d f32)."""
    b = np.asarray(nibbles16, np.uint8).reshape(16)
    codes = np.stack([KVALUES_MXFP4[b & 15], KVALUES_MXFP4[b >> 4]], axis=-1).reshape(32)
    return codes, e8m0_half_scale(np.uint8(e))[()]


def mxfp4_to_split(raw, rows, k):
    """GGUF MXFP4 blocks -> (nibbles [rows, K/2] pairs order, scales [rows, K/32]): the same codes and exponents in
    the split-plane layout (S/formats.py:12-15). Values are preserved except that code 8 reads as -0 in the split
    convention and +0 in the GGUF one."""
    b = _blocks(raw, "mxfp4").reshape(rows, k // 32, 17)
    e = b[:, :, 0].copy()
    qs = b[:, :, 1:17]
    codes = np.concatenate([qs & 15, qs >> 4], axis=2)          # [rows, nb, 32] in element order
    pairs = (codes[:, :, 0::2] | (codes[:, :, 1::2] << 4)).astype(np.uint8)
    return pairs.reshape(rows, k // 2), e


def mxfp4s_to_tiled(nibbles, scales, rows, k):
    """Split planes -> MFMA-tiled planes, written element by element from the layout's definition:
    nib_t[rb, c, l, :] = nibbles[32 rb + l % 32, 32 c + 16 (l // 32) : +16] and byte q of sc_t[rb, g, l, :] =
    scales[32 rb + l % 32, 2 (4 g + q) + l // 32] (0 when chunk 4 g + q lies past K). rows % 32 == 0, k % 64 == 0."""
    assert rows % 32 == 0 and k % 64 == 0, (rows, k)
    nib = np.asarray(nibbles).view(np.uint8).reshape(rows, k // 2)
    sc = np.asarray(scales).view(np.uint8).reshape(rows, k // 32)
    RB, C = rows // 32, k // 64
    C4 = (C + 3) // 4
    lanes = np.arange(64)
    li, lh = lanes % 32, lanes // 32
    nt = np.empty((RB, C, 64, 16), np.uint8)
    st = np.zeros((RB, C4, 64, 4), np.uint8)
    for rb in range(RB):
        r = 32 * rb + li
        for c in range(C):
            cols = 32 * c + 16 * lh[:, None] + np.arange(16)[None, :]
            nt[rb, c] = nib[r[:, None], cols]
            st[rb, c // 4, :, c % 4] = sc[r, 2 * c + lh]
    return nt.reshape(-1), st.reshape(-1)


def mxfp4t_to_split(nib_t, sc_t, rows, k):
    """Inverse of mxfp4s_to_tiled (vectorized, an independent construction: index arithmetic instead of loops)."""
    RB, C = rows // 32, k // 64
    C4 = (C + 3) // 4
    nt = np.asarray(nib_t).view(np.uint8).reshape(RB, C, 2, 32, 16)       # [rb, c, h, i, byte]
    nib = nt.transpose(0, 3, 1, 2, 4).reshape(rows, k // 2)                # row 32 rb + i, byte 32 c + 16 h + j
    st = np.asarray(sc_t).view(np.uint8).reshape(RB, C4, 2, 32, 4)        # [rb, g, h, i, q]
    s = st.transpose(0, 3, 1, 4, 2).reshape(rows, C4 * 4 * 2)[:, : k // 32]  # block 2 (4 g + q) + h
    return np.ascontiguousarray(nib), np.ascontiguousarray(s)


def dequant_mxfp4t(nib_t, sc_t, rows, k):
    """MXFP4 MFMA-tiled planes: the values of the split planes they permute."""
    nib, sc = mxfp4t_to_split(nib_t, sc_t, rows, k)
    return dequant_mxfp4s(nib, sc, rows, k)


def q4_k_to_tiled(raw, rows, k):
    """GGUF Q4_K rows -> the lane-ordered tiled layout of the decode GEMV and the grouped expert GEMMs, written from
    the layout's definition. Each block of 16 rows keeps its 16 x k / 256 super-blocks in its own byte range, cut
    into units of 512 values (two super-blocks a row), 4608 bytes each: the 32 16-byte headers ([f16 d][f16 dmin]
    [12 scale bytes]) of super-block sb of row r at 16 (2 r + sb), then four 1 KB code planes, plane q holding at
    16 l (l = 4 r + 2 sb + h) code bytes 16 (4 h + q) .. +16 of that super-block. When k % 512 == 256 the row
    block ends in a half unit of 2304 bytes (its last super-block of each row): the 16 headers at 16 r, then four
    512-byte planes, plane q holding at 16 (2 r + h) code bytes 16 (4 h + q) .. +16. rows % 16 == 0, k % 256 == 0."""
    assert rows % 16 == 0 and k % 256 == 0, (rows, k)
    b = _blocks(raw, "q4_k").reshape(rows, k // 256, 144)
    F, half = k // 512, (k // 256) % 2
    rbb = 16 * (k // 256) * 144
    out = np.empty(rows * k // 256 * 144, np.uint8)
    for rb in range(rows // 16):
        for sl in range(F):
            u = rb * rbb + sl * 4608
            for r in range(16):
                for sb in range(2):
                    blk = b[16 * rb + r, 2 * sl + sb]
                    out[u + 16 * (2 * r + sb): u + 16 * (2 * r + sb) + 16] = blk[0:16]
                    for h in range(2):
                        lane = 4 * r + 2 * sb + h
                        for q in range(4):
                            o = u + 512 + 1024 * q + 16 * lane
                            c = 16 + 16 * (4 * h + q)
                            out[o: o + 16] = blk[c: c + 16]
        if half:
            u = rb * rbb + F * 4608
            for r in range(16):
                blk = b[16 * rb + r, 2 * F]
                out[u + 16 * r: u + 16 * r + 16] = blk[0:16]
                for h in range(2):
                    for q in range(4):
                        o = u + 256 + 512 * q + 16 * (2 * r + h)
                        c = 16 + 16 * (4 * h + q)
                        out[o: o + 16] = blk[c: c + 16]
    return out


def q4_kt_to_gguf(raw_t, rows, k):
    """Inverse of q4_k_to_tiled (vectorized: an independent construction by index arithmetic)."""
    F, half = k // 512, (k // 256) % 2
    rbb = 16 * (k // 256) * 144
    t = np.asarray(raw_t).view(np.uint8).reshape(rows // 16, rbb)
    full = t[:, :F * 4608].reshape(rows // 16, F, 4608)
    hdr = full[:, :, :512].reshape(rows // 16, F, 16, 2, 16)                  # [rb, sl, r, sb, 16]
    codes = full[:, :, 512:].reshape(rows // 16, F, 4, 16, 2, 2, 16)          # [rb, sl, q, r, sb, h, 16]
    codes = codes.transpose(0, 1, 3, 4, 5, 2, 6).reshape(rows // 16, F, 16, 2, 128)   # [rb, sl, r, sb, (h q 16)]
    blk = np.concatenate([hdr, codes], axis=-1)                               # [rb, sl, r, sb, 144]
    blk = blk.transpose(0, 2, 1, 3, 4).reshape(rows // 16, 16, 2 * F, 144)    # [rb, r, super-block, 144]
    if half:
        tail = t[:, F * 4608:]
        th = tail[:, :256].reshape(rows // 16, 16, 1, 16)                     # [rb, r, -, 16]
        tc = tail[:, 256:].reshape(rows // 16, 4, 16, 2, 16)                  # [rb, q, r, h, 16]
        tc = tc.transpose(0, 2, 3, 1, 4).reshape(rows // 16, 16, 1, 128)      # [rb, r, -, (h q 16)]
        blk = np.concatenate([blk, np.concatenate([th, tc], axis=-1)], axis=2)
    return np.ascontiguousarray(blk).reshape(-1)    # rows in order, super-blocks in order


def q4_0_to_tiled(raw, rows, k):
    """GGUF Q4_0 rows -> the tiled layout of the decode GEMV (qmm_tile_q40), written from the layout's definition:
    per block of 16 rows, units of 512 values, 4608 bytes each; at 16 (2 r + sb) the eight f16 d of blocks 8 sb ..
    8 sb + 7 of the unit's row r (a 256-value span), then four 1 KB code planes, plane q holding at 16 l
    (l = 4 r + 2 sb + h) bytes 16 (4 h + q) .. +16 of the span's 128 code bytes. Span byte 32 p + i holds code i of
    block 2 p in its low nibble and code i of block 2 p + 1 in its high nibble (code i of a block: qs[i] & 15 for
    i < 16, qs[i - 16] >> 4 otherwise). rows % 16 == 0, k % 512 == 0."""
    assert rows % 16 == 0 and k % 512 == 0, (rows, k)
    b = _blocks(raw, "q4_0").reshape(rows, k // 32, 18)
    out = np.empty(rows * k // 32 * 18, np.uint8)
    for rb in range(rows // 16):
        for u in range(k // 512):
            base = (rb * (k // 512) + u) * 4608
            for r in range(16):
                for sb in range(2):
                    blks = b[16 * rb + r, 16 * u + 8 * sb: 16 * u + 8 * sb + 8]     # [8, 18]
                    out[base + 16 * (2 * r + sb): base + 16 * (2 * r + sb) + 16] = blks[:, 0:2].reshape(-1)
                    codes = [[int(bk[2 + i] & 15) if i < 16 else int(bk[2 + i - 16] >> 4) for i in range(32)]
                             for bk in blks]
                    span = bytes(codes[2 * (c // 32)][c % 32] | (codes[2 * (c // 32) + 1][c % 32] << 4)
                                 for c in range(128))
                    for h in range(2):
                        for q in range(4):
                            o = base + 512 + 1024 * q + 16 * (4 * r + 2 * sb + h)
                            out[o: o + 16] = np.frombuffer(span[16 * (4 * h + q): 16 * (4 * h + q) + 16], np.uint8)
    return out


def q4_0t_to_gguf(raw_t, rows, k):
    """Inverse of q4_0_to_tiled (vectorized: an independent construction by index arithmetic)."""
    U = k // 512
    t = np.asarray(raw_t).view(np.uint8).reshape(rows // 16, U, 4608)
    d = t[:, :, :512].reshape(rows // 16, U, 16, 2, 8, 2)                     # [rb, u, r, sb, block, 2 bytes]
    span = t[:, :, 512:].reshape(rows // 16, U, 4, 16, 2, 2, 16)              # [rb, u, q, r, sb, h, 16]
    span = span.transpose(0, 1, 3, 4, 5, 2, 6).reshape(rows // 16, U, 16, 2, 4, 32)   # [rb, u, r, sb, page, i]
    lo, hi = span & 15, span >> 4                                             # codes i of blocks 2 p, 2 p + 1
    codes = np.stack([lo, hi], axis=5).reshape(rows // 16, U, 16, 2, 8, 32)   # [rb, u, r, sb, block, i]
    qs = codes[..., :16] | (codes[..., 16:] << 4)
    blk = np.concatenate([d, qs.astype(np.uint8)], axis=-1)                   # [rb, u, r, sb, block, 18]
    return np.ascontiguousarray(blk.transpose(0, 2, 1, 3, 4, 5)).reshape(-1)


def dequant_q4_0t(raw_t, rows, k):
    """Q4_0 in the tiled GEMV layout: the values of the GGUF blocks it permutes."""
    return dequant_q4_0(q4_0t_to_gguf(raw_t, rows, k), rows, k)


def q6_k_fields(raw):
    """(d f32 [nb], sc i32 [nb, 16], q i32 [nb, 256]) of Q6_K super-blocks: ql = bytes 0..127, qh = 128..191, int8
    scales = 192..207, f16 d = 208..209. Value c = 128 half + 32 j + l (group g = 4 half + j) has the 6-bit code
    q = ((ql[64 half + 32 (j % 2) + l] >> 4 (j // 2)) & 15) | (((qh[32 half + l] >> 2 j) & 3) << 4) and the scale
    sc[8 half + 2 j + l // 16] (S/gen_llm.py:320-325)."""
    b = _blocks(raw, "q6_k")
    ql = b[:, 0:128].reshape(-1, 2, 2, 32).astype(np.int32)      # [nb, half, j % 2, l]
    qh = b[:, 128:192].reshape(-1, 2, 1, 32).astype(np.int32)    # [nb, half, -, l]
    j = np.arange(4).reshape(1, 1, 4, 1)
    low = (ql[:, :, j[0, 0, :, 0] % 2, :] >> (4 * (j // 2))) & 15  # [nb, half, j, l]
    high = (qh >> (2 * j)) & 3
    q = (low | (high << 4)).reshape(-1, 256)
    sc = b[:, 192:208].view(np.int8).astype(np.int32)
    return _f16(b[:, 208:210]), sc, q


def dequant_q6_k(raw, rows, k):
    """Q6_K: value = (f32(d) * sc) * (q - 32), the two products in that order in f32 (S/gen_llm.py:386-396); the
    first is exact (11 x 8 bits), the second rounds once."""
    d, sc, q = q6_k_fields(raw)
    scale = (d[:, None] * sc.astype(np.float32)).astype(np.float32)            # [nb, 16], exact
    s = np.repeat(scale, 16, axis=1)                                            # 16 consecutive values share one
    return (s * (q - 32).astype(np.float32)).astype(np.float32).reshape(rows, k)


def dequant_q4_kt(raw_t, rows, k):
    """Q4_K in the tiled GEMV layout: the values of the GGUF blocks it permutes."""
    return dequant_q4_k(q4_kt_to_gguf(raw_t, rows, k), rows, k)


def dequantize(fmt, raw, rows, k, scales=None):
    if fmt == "q4_0":
        return dequant_q4_0(raw, rows, k)
    if fmt == "q4_k":
        return dequant_q4_k(raw, rows, k)
    if fmt == "mxfp4":
        return dequant_mxfp4(raw, rows, k)
    if fmt == "mxfp4s":
        return dequant_mxfp4s(raw, scales, rows, k)
    if fmt == "mxfp4t":
        return dequant_mxfp4t(raw, scales, rows, k)
    if fmt == "q4_kt":
        return dequant_q4_kt(raw, rows, k)
    if fmt == "q6_k":
        return dequant_q6_k(raw, rows, k)
    if fmt == "q4_0t":
        return dequant_q4_0t(raw, rows, k)
    raise ValueError(fmt)
