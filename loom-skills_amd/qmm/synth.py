"""Seeded synthetic inputs of the five benchmark workloads (numpy, host side).

Seeds are ``default_rng(20261200 + index)`` with index 0..4 for the workloads below, and every generator draws in
the same order: the weights' scale fields, then the code bytes, then the activations, then the router logits.

0 ``q4_0_gemv``   Q4_0 W [4096, 4096], d = f16(|N(0, 0.02)|), code bytes uniform; x f32 [1, 4096] ~ N(0, 1)
1 ``q4_k_gemv``   Q4_K W [12288, 4096], d, dmin = f16(|N(0, 0.01)|), 6-bit sc / m uniform 0..63, code bytes uniform;
                  x bf16 [M, 4096] ~ N(0, 1) for M in {1, 4, 8}
2 ``q4_k_gemm``   Q4_K W [4096, 4096] as above; x bf16 [512, 4096]
3 ``mxfp4_moe``   32 experts, top-4, H = FE = 2880; fused gate_up [32, 5760, 2880] and down [32, 2880, 2880] MXFP4
                  (GGUF 17-byte blocks: E8M0 = 127 + U{-8..0}, code bytes uniform); x bf16 [T, 2880]; logits f32 [T, 32]
4 ``q4_k_moe``    128 experts, top-8, H = 2048, FE = 768; gate / up [128, 768, 2048], down [128, 2048, 768] Q4_K;
                  x bf16 [64, 2048]; logits f32 [64, 128]
"""
import numpy as np

SEED_BASE = 20261200


def rng_for(index):
    return np.random.default_rng(SEED_BASE + index)


def to_bf16_bits(x):
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(np.asarray(x, np.float32)).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _abs_f16(rng, sigma, n):
    return np.abs(rng.normal(0.0, sigma, n)).astype(np.float16)


def pack_q4_k_scales(sc, m):
    """8 six-bit scales and minima -> the 12 packed bytes of a Q4_K super-block (the inverse of ggml's
    get_scale_min_k4, skills/loom-port-llm/starter/gen_llm.py:234-267)."""
    sc = np.asarray(sc).astype(np.int32)
    m = np.asarray(m).astype(np.int32)
    S = np.empty(sc.shape[:-1] + (12,), np.int32)
    S[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    S[..., 4:8] = (m[..., 0:4] & 63) | ((m[..., 4:8] >> 4) << 6)
    S[..., 8:12] = (sc[..., 4:8] & 15) | ((m[..., 4:8] & 15) << 4)
    return S.astype(np.uint8)


def q4_0_weights(rng, rows, k, sigma=0.02):
    """Q4_0 bytes [rows * k/32 * 18]: f16 d then 16 code bytes per block."""
    nb = rows * k // 32
    d = _abs_f16(rng, sigma, nb)
    qs = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    raw = np.empty((nb, 18), np.uint8)
    raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    raw[:, 2:] = qs
    return raw.reshape(-1)


def q4_k_weights(rng, rows, k, sigma=0.01):
    """Q4_K bytes [rows * k/256 * 144]: f16 d, f16 dmin, 12 packed scale bytes, 128 code bytes per super-block."""
    nb = rows * k // 256
    d = _abs_f16(rng, sigma, nb)
    dmin = _abs_f16(rng, sigma, nb)
    sc = rng.integers(0, 64, (nb, 8))
    m = rng.integers(0, 64, (nb, 8))
    qs = rng.integers(0, 256, (nb, 128), dtype=np.uint8)
    raw = np.empty((nb, 144), np.uint8)
    raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    raw[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    raw[:, 4:16] = pack_q4_k_scales(sc, m)
    raw[:, 16:] = qs
    return raw.reshape(-1)


def q6_k_weights(rng, rows, k, sigma=0.002):
    """Q6_K bytes [rows * k/256 * 210]: ql[128], qh[64], 16 int8 scales, f16 d per super-block (code bytes and
    scales uniform)."""
    nb = rows * k // 256
    raw = rng.integers(0, 256, (nb, 210), dtype=np.uint8)
    raw[:, 208:210] = _abs_f16(rng, sigma, nb).view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


def mxfp4_weights(rng, rows, k, e_lo=-8, e_hi=0):
    """MXFP4 GGUF bytes [rows * k/32 * 17]: E8M0 byte 127 + U{e_lo..e_hi} then 16 code bytes per block."""
    nb = rows * k // 32
    e = (127 + rng.integers(e_lo, e_hi + 1, nb)).astype(np.uint8)
    qs = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    raw = np.empty((nb, 17), np.uint8)
    raw[:, 0] = e
    raw[:, 1:] = qs
    return raw.reshape(-1)


def weights(fmt, rng, rows, k):
    return {"q4_0": q4_0_weights, "q4_k": q4_k_weights, "mxfp4": mxfp4_weights, "q6_k": q6_k_weights}[fmt](rng, rows, k)


def normal_f32(rng, shape):
    return rng.standard_normal(shape).astype(np.float32)


def _weights(index, rng, kw):
    """The weights (and shape fields) of workload `index`, drawn first from its generator."""
    if index == 0:
        n, k = kw.get("n", 4096), kw.get("k", 4096)
        return {"fmt": "q4_0", "n": n, "k": k, "w": q4_0_weights(rng, n, k)}
    if index in (1, 2):
        n, k = (12288, 4096) if index == 1 else (4096, 4096)
        n, k = kw.get("n", n), kw.get("k", k)
        return {"fmt": "q4_k", "n": n, "k": k, "w": q4_k_weights(rng, n, k)}
    if index == 3:
        E, KU, H, FE = kw.get("E", 32), kw.get("KU", 4), kw.get("H", 2880), kw.get("FE", 2880)
        gate_up = mxfp4_weights(rng, E * 2 * FE, H)
        down = mxfp4_weights(rng, E * H, FE)
        return {"fmt": "mxfp4", "E": E, "KU": KU, "H": H, "FE": FE, "gate_up": gate_up, "down": down, "gating": 3,
                "norm": False, "act": "swiglu_oai", "fused": True}
    if index == 4:
        E, KU, H, FE = kw.get("E", 128), kw.get("KU", 8), kw.get("H", 2048), kw.get("FE", 768)
        gate = q4_k_weights(rng, E * FE, H)
        up = q4_k_weights(rng, E * FE, H)
        down = q4_k_weights(rng, E * H, FE)
        return {"fmt": "q4_k", "E": E, "KU": KU, "H": H, "FE": FE, "gate": gate, "up": up, "down": down,
                "gating": 1, "norm": True, "act": "silu", "fused": False}
    raise ValueError(index)


def _inputs(index, rng, w, kw):
    """The activations (and router logits) of workload `index`, drawn after its weights."""
    if index == 0:
        return {"x": normal_f32(rng, (kw.get("m", 1), w["k"]))}
    if index in (1, 2):
        m = kw.get("m", 1 if index == 1 else 512)
        return {"x_bf16": to_bf16_bits(normal_f32(rng, (m, w["k"])))}
    T = kw.get("T", 256 if index == 3 else 64)
    x = to_bf16_bits(normal_f32(rng, (T, w["H"])))
    return {"T": T, "x_bf16": x, "logits": normal_f32(rng, (T, w["E"]))}


def workload(index, cache=None, **kw):
    """Inputs of one workload as host numpy arrays (see the module docstring). cache: a dict owned by the caller that
    keeps the weights of a workload (keyed by index and shape) with the generator's state after drawing them, so a
    second call with another token count (m / T) reuses them and draws the same inputs as a fresh call would."""
    shape = tuple(sorted((k, v) for k, v in kw.items() if k not in ("m", "T")))
    key = (index, shape)
    if cache is not None and key in cache:
        w, state = cache[key]
        rng = np.random.default_rng()
        rng.bit_generator.state = state
    else:
        rng = rng_for(index)
        w = _weights(index, rng, kw)
        if cache is not None:
            cache[key] = (w, rng.bit_generator.state)
    d = dict(w)
    d.update(_inputs(index, rng, w, kw))
    return d
