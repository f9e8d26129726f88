"""Pins the oracle's reference arithmetic (oracle/ref.py) -- CPU only.

* matmuls       brute-force Python loops on tiny inputs (a transposed operand or dropped row scale fails)
* Q8_1          closed-form properties of llama.cpp quantize_q8_1 (make_kernel_tests.py:32-39): the group maximum maps
                to +-127, halves round away from zero, an all-zero group stays zero
* E4M3          every one of the 254 finite E4M3FN numbers is a fixed point and encodes to its own byte; midpoints
                round to even; saturation at 448; torch's float8_e4m3fn conversion agrees on in-range values
* MXFP8         the shared exponent keeps every scaled element in [128, 256) for the block maximum, never saturating
* row scale     the exponent rule of g_row_scale_f16 (S/gen_llm.py:1843-1915) on powers of two
* routing       brute-force loops per gating mode, ties to the lower id, and the identity that gating 1 + norm and
                gating 3 give the same weights (softmax over the picked logits)
* bucket        the invariants of S/gen_moe.py:829-955 (segment sizes, tile table, rowmap/pos inverse, -1 padding) and
                a second construction by stable argsort
* combine       an explicit loop (S/gen_moe.py:1231-1280)
* activations   the swiglu_oai clamps at their limits (S/gen_moe.py:33-46)
* MoE chain     a per-token, per-slot loop in the shape of experts_ref (make_kernel_tests.py:3197-3221)
"""
import numpy as np
import pytest

from oracle import ref


# ---------------------------------------------------------------------------------------------------- matmuls
def test_gemv_and_gemm_brute_force():
    rng = np.random.default_rng(0)
    x, w, inv = rng.standard_normal((3, 5)), rng.standard_normal((4, 5)), rng.uniform(.25, 2, 3)
    want = [[sum(x[t, k] * w[n, k] for k in range(5)) for n in range(4)] for t in range(3)]
    assert np.allclose(ref.gemv(x, w), want, rtol=1e-14, atol=0)
    assert np.allclose(ref.gemm(x, w, inv), np.array(want) * inv[:, None], rtol=1e-14, atol=0)
    assert ref.rel_l2(ref.gemv(x, w), np.array(want)) < 1e-15
    assert ref.rel_l2(ref.gemv(x, w[::-1]), np.array(want)) > 0.1


# ------------------------------------------------------------------------------------------------------- Q8_1
def test_q8_1_closed_form():
    x = np.zeros((1, 64), np.float32)
    x[0, :32] = np.linspace(-1, 2.54, 32, dtype=np.float32)
    x[0, 3] = 1.27 * 2.5 / 127 * 100 / 100       # some value
    got = ref.q8_1(x)
    d = np.float32(np.abs(x[0, :32]).max()) / np.float32(127)
    dq = np.float32(np.float16(d))
    q = got[0, :32] / dq
    assert np.allclose(q, np.rint(q)) and np.abs(q).max() == 127
    assert np.all(got[0, 32:] == 0)
    # round half away from zero: x/d = +-2.5 -> +-3
    y = np.zeros((1, 32), np.float32)
    y[0, 0], y[0, 1], y[0, 2] = 127.0, 2.5, -2.5
    g = ref.q8_1(y)[0]
    assert g[1] == 3 * np.float32(np.float16(1.0)) and g[2] == -3.0


def test_q8_1_codes_and_planar_layout():
    """codes * f16(d) is q8_1; the group sum is the sum of codes; a zero group has d = 0 and zero codes; the planar
    buffer holds the codes first and the (d, sum) pairs after rows * K bytes (S/gen_llm.py:684-690)."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((3, 96)) * np.exp(rng.uniform(-4, 4, (3, 1)))).astype(np.float32)
    x[1, 32:64] = 0.0
    codes, d16, sums = ref.q8_1_codes(x)
    assert codes.dtype == np.int8 and codes.shape == x.shape and d16.shape == sums.shape == (3, 3)
    assert np.array_equal(ref.q8_1(x), (codes.astype(np.float32).reshape(3, 3, 32) * d16[..., None]).reshape(3, 96))
    assert np.array_equal(sums, codes.reshape(3, 3, 32).sum(-1).astype(np.float32))
    assert d16[1, 1] == 0 and not codes[1, 32:64].any()
    assert np.abs(codes.reshape(3, 3, 32)).max(-1).tolist() == [[127] * 3, [127, 0, 127], [127] * 3]
    buf = ref.q8_planar(x)
    assert buf.size == 3 * 96 + 3 * 3 * 8
    assert np.array_equal(buf[:288].view(np.int8).reshape(3, 96), codes)
    meta = buf[288:].view(np.float32).reshape(3, 3, 2)
    assert np.array_equal(meta[..., 0], d16) and np.array_equal(meta[..., 1], sums)
    # a plausible mistake -- rounding half to even -- changes the codes of exact halves
    y = np.zeros((1, 32), np.float32)
    y[0, 0], y[0, 1] = 127.0, 0.5
    assert ref.q8_1_codes(y)[0][0, 1] == 1 and np.rint(np.float32(0.5)) == 0


# ------------------------------------------------------------------------------------------------------- E4M3
def all_e4m3():
    b = np.arange(256, dtype=np.uint8)
    b = b[(b & 0x7F) != 0x7F]                       # drop the two NaN encodings
    return b, ref.e4m3_decode(b)


def test_e4m3_fixed_points_and_bytes():
    b, v = all_e4m3()
    assert v.max() == 448 and v.min() == -448 and np.unique(v).size == 253   # +0 and -0 share a value
    assert np.array_equal(ref.e4m3_round(v), v)
    nz = v != 0
    assert np.array_equal(ref.e4m3_bytes(v[nz]), b[nz])
    assert ref.e4m3_bytes(np.array([-0.0]))[0] == 0x80


def test_e4m3_rounding_even_and_saturation():
    _, v = all_e4m3()
    pos = np.unique(v[v > 0])
    mid = (pos[:-1] + pos[1:]) / 2
    r = ref.e4m3_round(mid)
    lo_b, hi_b = ref.e4m3_bytes(pos[:-1]), ref.e4m3_bytes(pos[1:])
    even = np.where(lo_b % 2 == 0, pos[:-1], pos[1:])
    assert np.array_equal(r, even)
    assert ref.e4m3_round(np.array([1e6, -500.0]))[0] == 448 and ref.e4m3_round(np.array([-500.0]))[0] == -448
    assert ref.e4m3_round(np.array([2.0 ** -10]))[0] == 0.0        # below half the smallest subnormal 2^-9


def test_e4m3_against_torch_conversion():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(20000) * 10, rng.standard_normal(5000) * 0.01, [0.0, 447.0, -447.9]])
    x = x.astype(np.float32)
    t = torch.from_numpy(x).to(torch.float8_e4m3fn).to(torch.float64).numpy()
    assert np.array_equal(ref.e4m3_round(x), t)


def test_mxfp8_exponent_choice():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((16, 256)) * np.exp(rng.uniform(-20, 20, (16, 1)))
    x[0, :32] = 0.0
    codes, sc, vals = ref.mxfp8_quantize(x)
    s = sc.astype(np.int64) - 127
    g = np.abs(x.reshape(16, 8, 32)).max(-1)
    scaled = g * 2.0 ** -s
    live = g > 0
    assert np.all((scaled[live] >= 128) & (scaled[live] < 256))
    assert sc[0, 0] == 0 and np.all(codes[0, :32] == 0)
    assert np.array_equal(ref.e4m3_decode(codes).reshape(16, 8, 32) * 2.0 ** s[..., None], vals.reshape(16, 8, 32))
    assert ref.rel_l2(vals, x) < 0.04
    c64, s64, v64 = ref.mxfp8_quantize(x, block=64)  # a coarser block shares the larger exponent
    assert s64.shape == (16, 4) and np.all(s64 == np.maximum(sc[:, 0::2], sc[:, 1::2]))
    assert ref.rel_l2(v64, x) < 0.04


def test_row_scale_exponent():
    x = np.ones((4, 8))
    x[1] *= 2.0 ** 13
    x[2] *= 2.0 ** 14
    x[3] *= 2.0 ** 200
    assert ref.row_scale_exponent(x).tolist() == [0, 0, 1, 100]
    f = ref.f16_rows(np.array([[1.0 + 2 ** -12, 3.0]]))
    assert f[0, 0] == 1.0 and f[0, 1] == 3.0


# ---------------------------------------------------------------------------------------------------- routing
def route_loop(logits, KU, gating, norm, bias=None):
    T, E = logits.shape
    b = np.zeros(E) if bias is None else bias
    ids = np.zeros((T, KU), np.int32)
    wts = np.zeros((T, KU))
    for t in range(T):
        l = [float(v) for v in logits[t]]
        if gating == 1:
            m = max(l)
            ex = [np.exp(v - m) for v in l]
            p = [v / sum(ex) for v in ex]
            sel = [p[e] + b[e] for e in range(E)]
        elif gating == 2:
            p = [1 / (1 + np.exp(-v)) for v in l]
            sel = [p[e] + b[e] for e in range(E)]
        else:
            p = [l[e] + b[e] for e in range(E)]
            sel = p
        order = sorted(range(E), key=lambda e: (-sel[e], e))[:KU]
        w = [p[e] for e in order]
        if gating == 3:
            mx = max(w)
            w = [np.exp(v - mx) for v in w]
            w = [v / sum(w) for v in w]
        if norm:
            s = max(sum(w), ref.NORM_FLOOR)
            w = [v / s for v in w]
        ids[t], wts[t] = order, w
    return ids, wts


@pytest.mark.parametrize("gating,norm,bias", [(1, True, False), (1, False, False), (2, True, True), (3, False, True)])
def test_route_matches_loop(gating, norm, bias):
    rng = np.random.default_rng(gating * 10 + norm)
    logits = rng.standard_normal((9, 12)).astype(np.float32)
    logits[2, [1, 5, 7]] = logits[2].max() + 1     # a three-way tie at the top
    b = rng.standard_normal(12) * 0.1 if bias else None
    ids, wts = ref.route(logits, 4, gating, norm, bias=b)
    eids, ewts = route_loop(logits, 4, gating, norm, b)
    assert np.array_equal(ids, eids)
    assert np.allclose(wts, ewts, rtol=1e-12, atol=1e-15)
    if b is None:
        assert ids[2, :3].tolist() == [1, 5, 7]          # the tie goes to the lower ids in order


def test_gating_1_norm_equals_gating_3():
    rng = np.random.default_rng(3)
    logits = rng.standard_normal((50, 32))
    i1, w1 = ref.route(logits, 4, 1, True)
    i3, w3 = ref.route(logits, 4, 3, False)
    assert np.array_equal(i1, i3)
    assert np.allclose(w1, w3, rtol=1e-12)
    assert np.allclose(w1.sum(-1), 1.0)


def test_route_margin():
    logits = np.array([[3.0, 2.0, 2.0, 1.0], [4.0, 3.0, 2.0, 1.0]])
    m = ref.route_margin(logits, 2, 3)
    assert m[0] == 0.0 and m[1] == pytest.approx(1 / 3)     # (3 - 2) / 3


# ----------------------------------------------------------------------------------------------------- bucket
def test_bucket_invariants_and_argsort_construction():
    rng = np.random.default_rng(2)
    T, KU, E = 150, 4, 8
    ids = rng.integers(0, E, (T, KU)).astype(np.int32)
    ids[:40, 0] = 3                        # expert 3 gets more than 64 rows
    live = np.ones(T, np.int32)
    live[-5:] = 0
    mt = ref.max_tiles(T, KU, E)
    ti, rm, pos = ref.bucket(ids, E, mt, live=live)
    flat = ids.reshape(-1)
    alive = np.repeat(live != 0, KU)
    counts = np.bincount(flat[alive], minlength=E)
    # tile table: experts ascending, 64-row tiles, the last one partial, unused tiles (-1, 0)
    used = ti[:, 0] >= 0
    assert np.all(ti[~used] == [-1, 0]) and np.all(used[:used.sum()])
    assert np.all(np.diff(ti[used, 0]) >= 0)
    for e in range(E):
        assert ti[ti[:, 0] == e, 1].sum() == counts[e]
        assert np.all(ti[ti[:, 0] == e, 1][:-1] == 64) if counts[e] else True
    # rowmap / pos are inverse; dead assignments are -1
    live_a = np.flatnonzero(alive)
    assert np.array_equal(rm[pos[live_a]], live_a)
    assert np.all(pos[~alive] == -1)
    assert np.sum(rm >= 0) == alive.sum()
    # second construction: stable argsort by expert gives the same rows
    order = live_a[np.argsort(flat[live_a], kind="stable")]
    rows = []
    for e in range(E):
        seg = order[flat[order] == e]
        base = int(np.flatnonzero(ti[:, 0] == e)[0]) * 64 if seg.size else 0
        rows += list(zip(seg, base + np.arange(seg.size)))
    for a, r in rows:
        assert pos[a] == r
    # ids out of range are clamped (S/gen_moe.py:868-870)
    bad = ids.copy()
    bad[0, 0] = 99
    assert ref.bucket(bad, E, mt)[2][0] == ref.bucket(np.where(bad > E - 1, E - 1, bad), E, mt)[2][0]


# ---------------------------------------------------------------------------------------------------- combine
def test_combine_loop():
    rng = np.random.default_rng(4)
    T, KU, H = 5, 3, 7
    ys = rng.standard_normal((40, H))
    pos = rng.integers(-1, 40, (T, KU))
    wts = rng.random((T, KU))
    y0 = rng.standard_normal((T, H))
    want = y0.copy()
    for t in range(T):
        for k in range(KU):
            if pos[t, k] >= 0:
                want[t] += wts[t, k] * ys[pos[t, k]]
    assert np.allclose(ref.combine(ys, pos.reshape(-1), wts, y0), want, rtol=1e-14)
    dec = ref.combine(ys[:T * KU], None, wts)
    assert np.allclose(dec, (wts[:, :, None] * ys[:T * KU].reshape(T, KU, H)).sum(1))


def test_swiglu_oai_clamps():
    assert ref.swiglu_oai(10.0, 0.0) == pytest.approx(7.0 / (1 + np.exp(-1.702 * 7.0)))
    assert ref.swiglu_oai(1.0, -10.0) == pytest.approx(1.0 / (1 + np.exp(-1.702)) * -6.0)
    assert ref.silu_mul(2.0, 3.0) == pytest.approx(2.0 / (1 + np.exp(-2.0)) * 3.0)


def test_moe_chain_matches_loop():
    rng = np.random.default_rng(6)
    T, KU, E, H, FE = 6, 2, 4, 8, 5
    x = rng.standard_normal((T, H))
    Wg, Wu, Wd = rng.standard_normal((E, FE, H)), rng.standard_normal((E, FE, H)), rng.standard_normal((E, H, FE))
    ids, wts = ref.route(rng.standard_normal((T, E)), KU, 1, True)
    y, acts = ref.moe(x, ids, wts, lambda e: (Wg[e], Wu[e]), lambda e: Wd[e], act="silu")
    want = np.zeros((T, H))
    for t in range(T):
        for k in range(KU):
            e = ids[t, k]
            g, u = Wg[e] @ x[t], Wu[e] @ x[t]
            a = g / (1 + np.exp(-g)) * u
            assert np.allclose(acts[t * KU + k], a)
            want[t] += wts[t, k] * (Wd[e] @ a)
    assert np.allclose(y, want, rtol=1e-12)


def test_moe_chain_with_expert_biases():
    """The gpt-oss expert biases: with zero weights the chain reduces to y[t] = sum_k w (Wd act(bg, bu) + bd), and a
    random case matches the per-assignment loop of make_kernel_tests.py:3204-3215 (bias before the activation,
    down bias inside the weighted sum)."""
    rng = np.random.default_rng(16)
    T, KU, E, H, FE = 5, 2, 4, 6, 3
    x = rng.standard_normal((T, H))
    bg, bu, bd = rng.standard_normal((E, FE)), rng.standard_normal((E, FE)), rng.standard_normal((E, H))
    ids, wts = ref.route(rng.standard_normal((T, E)), KU, 3, False)
    Z = np.zeros((E, FE, H))
    Wd = rng.standard_normal((E, H, FE))
    y0, _ = ref.moe(x, ids, wts, lambda e: (Z[e], Z[e]), lambda e: Wd[e], act="swiglu_oai", bias=(bg, bu, bd))
    want0 = np.zeros((T, H))
    for t in range(T):
        for k in range(KU):
            e = ids[t, k]
            want0[t] += wts[t, k] * (Wd[e] @ ref.swiglu_oai(bg[e], bu[e]) + bd[e])
    assert np.allclose(y0, want0, rtol=1e-13)
    Wg, Wu = rng.standard_normal((E, FE, H)), rng.standard_normal((E, FE, H))
    y, _ = ref.moe(x, ids, wts, lambda e: (Wg[e], Wu[e]), lambda e: Wd[e], act="silu", bias=(bg, bu, bd))
    want = np.zeros((T, H))
    for t in range(T):
        for k in range(KU):
            e = ids[t, k]
            g, u = Wg[e] @ x[t] + bg[e], Wu[e] @ x[t] + bu[e]
            want[t] += wts[t, k] * (Wd[e] @ (g / (1 + np.exp(-g)) * u) + bd[e])
    assert np.allclose(y, want, rtol=1e-12)


def test_router_logits_and_shared_gate_brute_force():
    rng = np.random.default_rng(17)
    T, E, H = 3, 5, 7
    x, w = rng.standard_normal((T, H)), rng.standard_normal((E, H))
    lg = ref.router_logits(x, w)
    for t in range(T):
        for e in range(E):
            assert lg[t, e] == pytest.approx(sum(float(x[t, k]) * float(w[e, k]) for k in range(H)), rel=1e-12)
    sg = ref.shared_gate(x, w[0])
    assert np.allclose(sg, 1 / (1 + np.exp(-lg[:, 0])), rtol=1e-14)
    assert ref.shared_gate(np.full((1, 2), -800.0), np.ones(2))[0] == 0.0      # no overflow: the limit
    assert ref.shared_gate(np.zeros((1, 2)), np.ones(2))[0] == 0.5


def test_wscale_clamps_ids():
    """ktest_more.py:99-111: ids out of range use the first / last expert's scale."""
    rng = np.random.default_rng(18)
    E, T, KU = 6, 3, 4
    ids = rng.integers(0, E, (T, KU)).astype(np.int32)
    ids[0, 0], ids[1, 1] = -1, E + 5
    wts = rng.random((T, KU))
    sc = 0.5 + rng.random(E)
    out = ref.wscale(ids, wts, sc)
    assert out[0, 0] == wts[0, 0] * sc[0] and out[1, 1] == wts[1, 1] * sc[E - 1]
    assert out[2, 3] == wts[2, 3] * sc[ids[2, 3]]


def test_gated_combine():
    """shared_gated (S/gen_moe.py:765-779): y = sg y0 + sum_k w ys; sg = 1 is the plain accumulate."""
    rng = np.random.default_rng(19)
    T, KU, H = 4, 2, 5
    ys = rng.standard_normal((T * KU, H))
    wts, y0, sg = rng.random((T, KU)), rng.standard_normal((T, H)), rng.random(T)
    got = ref.combine(ys, None, wts, y0, sg=sg)
    assert np.allclose(got, sg[:, None] * y0 + (wts[:, :, None] * ys.reshape(T, KU, H)).sum(1), rtol=1e-14)
    assert np.array_equal(ref.combine(ys, None, wts, y0, sg=np.ones(T)), ref.combine(ys, None, wts, y0))
