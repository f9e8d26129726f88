"""Shared test helpers: numpy <-> device tensors and the oracle comparisons used by the GPU parity tests."""
import numpy as np

from oracle import formats as of
from oracle import ref


def dev_u8(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a).view(np.uint8).reshape(-1))).to(device)


def dev_f32(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)


def dev_bf16(bits, device):
    """bf16 tensor from uint16 bit patterns."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).to(device)
    return t.view(torch.bfloat16)


def host(t):
    import torch
    if t.dtype == torch.bfloat16:
        return (t.view(torch.int16).cpu().numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    return t.cpu().numpy()


def bf16_values(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_close_rel_l2(actual, expected, tol, what=""):
    err = ref.rel_l2(actual, expected)
    assert err <= tol, f"{what}: rel-L2 {err:.3e} > {tol:.1e}"
    return err


def assert_bits_equal(a, b, what=""):
    a = np.ascontiguousarray(a, np.float32).view(np.uint32)
    b = np.ascontiguousarray(b, np.float32).view(np.uint32)
    bad = np.flatnonzero(a.reshape(-1) != b.reshape(-1))
    assert bad.size == 0, f"{what}: {bad.size} of {a.size} values differ in bits (first at {bad[:5]})"


def dequant_oracle(fmt, raw, rows, k):
    return of.dequantize(fmt, raw, rows, k)
