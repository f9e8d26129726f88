"""GGUF tensor binding: the weights of a GGUF file as device tensors, by tensor name.

The reference binds a weight with ``command.parameter %weights, "<tensor name>" : view<...>`` (S/gen_llm.py:5356-5371
for the MoE tensors) and reads the raw block bytes in place. Here a GGUF file is parsed on the host (numpy memmap:
nothing is read beyond the header until a tensor is asked for) and its data region goes to the device once, as one
uint8 buffer; every tensor is then a view of that buffer at its offset, in the GGUF's own block layout, which is the
layout the qmm entry points take (Q4_0, Q4_K, Q6_K, MXFP4 blocks). GGUF aligns tensor data to ``general.alignment``
(32 by default), so the views meet the 16-byte alignment of the Q4_K kernels as long as the device buffer is 32-byte
aligned (torch allocations are 512-byte aligned).

File layout (GGUF v2 / v3, little endian): magic "GGUF", u32 version, u64 tensor count, u64 KV count; the KV pairs
(u64-length key, u32 type, value); the tensor infos (u64-length name, u32 n_dims, n_dims u64 dims with ne0 the
fastest-varying, u32 ggml type, u64 offset from the data start); padding to the alignment; the data.
"""
import struct

import numpy as np

MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# KV value types
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
KV_STRING, KV_ARRAY = 8, 9

# ggml tensor types: (name, values per block, bytes per block). The quantized ones this library computes on carry
# the qmm format name (GGML type ids 2 = Q4_0, 12 = Q4_K, 14 = Q6_K, 39 = MXFP4).
GGML_TYPES = {
    0: ("f32", 1, 4), 1: ("f16", 1, 2), 2: ("q4_0", 32, 18), 3: ("q4_1", 32, 20), 6: ("q5_0", 32, 22),
    7: ("q5_1", 32, 24), 8: ("q8_0", 32, 34), 10: ("q2_k", 256, 84), 11: ("q3_k", 256, 110), 12: ("q4_k", 256, 144),
    13: ("q5_k", 256, 176), 14: ("q6_k", 256, 210), 15: ("q8_k", 256, 292), 20: ("iq4_nl", 32, 18),
    23: ("iq4_xs", 256, 136), 24: ("i8", 1, 1), 25: ("i16", 1, 2), 26: ("i32", 1, 4), 27: ("i64", 1, 8),
    28: ("f64", 1, 8), 30: ("bf16", 1, 2), 39: ("mxfp4", 32, 17),
}
QMM_FORMATS = {"q4_0", "q4_k", "q6_k", "mxfp4"}


class GGUFError(ValueError):
    pass


class TensorInfo:
    """One tensor of the file: dims in GGUF order (ne0 first: the row length K of a matrix), its ggml type, its byte
    offset from the data start and its size."""

    __slots__ = ("name", "dims", "ggml_type", "offset", "nbytes")

    def __init__(self, name, dims, ggml_type, offset):
        if ggml_type not in GGML_TYPES:
            raise GGUFError(f"{name}: unknown ggml type {ggml_type}")
        tname, bv, bb = GGML_TYPES[ggml_type]
        n = int(np.prod(dims, dtype=np.int64)) if dims else 1
        if dims[0] % bv:
            raise GGUFError(f"{name}: row length {dims[0]} is not a multiple of the {tname} block ({bv})")
        self.name, self.dims, self.ggml_type, self.offset = name, tuple(int(d) for d in dims), ggml_type, int(offset)
        self.nbytes = n // bv * bb

    @property
    def type_name(self):
        return GGML_TYPES[self.ggml_type][0]

    @property
    def fmt(self):
        """The qmm format name of a quantized tensor this library computes on, else None."""
        t = self.type_name
        return t if t in QMM_FORMATS else None

    @property
    def k(self):
        """Values per row (ne0)."""
        return self.dims[0]

    @property
    def rows(self):
        """Rows of all matrices together (ne1 * ne2 * ...: an expert tensor [E, n, K] has E * n rows)."""
        return int(np.prod(self.dims[1:], dtype=np.int64)) if len(self.dims) > 1 else 1

    def __repr__(self):
        return f"TensorInfo({self.name!r}, {self.type_name}, dims={list(self.dims)}, offset={self.offset})"


class _Cursor:
    def __init__(self, buf, pos=0):
        self.buf, self.pos = buf, pos

    def take(self, n):
        if self.pos + n > len(self.buf):
            raise GGUFError("truncated GGUF header")
        b = bytes(self.buf[self.pos:self.pos + n])
        self.pos += n
        return b

    def unpack(self, fmt):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self):
        return self.take(self.unpack("<Q")).decode("utf-8", errors="replace")

    def value(self, t):
        if t in _SCALAR:
            return self.unpack(_SCALAR[t])
        if t == KV_STRING:
            return self.string()
        if t == KV_ARRAY:
            et, n = self.unpack("<I"), self.unpack("<Q")
            if et in _SCALAR:
                fmt = _SCALAR[et]
                size = struct.calcsize(fmt)
                return np.frombuffer(self.take(size * n), dtype=np.dtype(fmt)).copy()
            return [self.value(et) for _ in range(n)]
        raise GGUFError(f"unknown KV type {t}")


class GGUFFile:
    """A parsed GGUF file: ``kv`` (key -> value), ``tensors`` (name -> TensorInfo, file order), ``data_start``."""

    def __init__(self, path):
        self.path = path
        self._map = np.memmap(path, dtype=np.uint8, mode="r")
        c = _Cursor(self._map)
        if c.take(4) != MAGIC:
            raise GGUFError(f"{path}: not a GGUF file")
        self.version = c.unpack("<I")
        if self.version not in (2, 3):
            raise GGUFError(f"{path}: GGUF version {self.version} is not supported")
        n_tensors, n_kv = c.unpack("<Q"), c.unpack("<Q")
        self.kv = {}
        for _ in range(n_kv):
            key = c.string()
            self.kv[key] = c.value(c.unpack("<I"))
        self.tensors = {}
        for _ in range(n_tensors):
            name = c.string()
            nd = c.unpack("<I")
            dims = [c.unpack("<Q") for _ in range(nd)]
            tt, off = c.unpack("<I"), c.unpack("<Q")
            self.tensors[name] = TensorInfo(name, dims, tt, off)
        self.header_bytes = c.pos
        self.alignment = int(self.kv.get("general.alignment", DEFAULT_ALIGNMENT))
        a = self.alignment
        self.data_start = (c.pos + a - 1) // a * a
        self.size = len(self._map)
        for t in self.tensors.values():
            if t.offset % a:
                raise GGUFError(f"{t.name}: offset {t.offset} is not {a}-byte aligned")
            if self.data_start + t.offset + t.nbytes > self.size:
                raise GGUFError(f"{t.name}: data past the end of the file")
        self._device = None

    def __getitem__(self, name):
        return self.tensors[name]

    def raw(self, name):
        """The tensor's bytes as a read-only uint8 view of the file (no copy)."""
        t = self.tensors[name]
        lo = self.data_start + t.offset
        return self._map[lo:lo + t.nbytes]

    def to_device(self, device, stage_bytes=1 << 28):
        """Copy the data region to the device once (one uint8 buffer); later ``view`` calls slice it. The file is
        streamed through one pinned staging buffer of at most stage_bytes (host memory stays bounded)."""
        import torch
        if self._device is None or self._device.device != torch.device(device):
            n = self.size - self.data_start
            buf = torch.empty(n, dtype=torch.uint8, device=device)
            stage = torch.empty(max(1, min(n, stage_bytes)), dtype=torch.uint8, pin_memory=True)
            sv = stage.numpy()
            for lo in range(0, n, len(sv)):
                m = min(len(sv), n - lo)
                sv[:m] = self._map[self.data_start + lo:self.data_start + lo + m]
                buf[lo:lo + m].copy_(stage[:m])          # synchronous: the staging buffer is reused next
            self._device = buf
        return self._device

    def view(self, name, device):
        """The tensor as a uint8 device tensor in the file's block layout (a view of the device copy of the data)."""
        t = self.tensors[name]
        buf = self.to_device(device)
        return buf[t.offset:t.offset + t.nbytes]

    def upload(self, name, device):
        """The tensor alone as its own uint8 device tensor (when the whole data region is not wanted on the device)."""
        import torch
        return torch.from_numpy(np.array(self.raw(name))).to(device)


def moe_layer_tensors(g, layer):
    """The names and formats of one MoE layer's expert tensors (moe_routed's command.parameter names,
    S/gen_llm.py:5318, :5356-5371): router, gate / up (or the fused gate_up), down, and the optional biases and scales."""
    b = f"blk.{layer}."
    out = {}
    for key, name in (("router", "ffn_gate_inp.weight"), ("router_bias", "ffn_gate_inp.bias"),
                      ("probs_bias", "exp_probs_b.bias"), ("gate", "ffn_gate_exps.weight"),
                      ("up", "ffn_up_exps.weight"), ("gate_up", "ffn_gate_up_exps.weight"),
                      ("down", "ffn_down_exps.weight"), ("gate_bias", "ffn_gate_exps.bias"),
                      ("up_bias", "ffn_up_exps.bias"), ("down_bias", "ffn_down_exps.bias"),
                      ("down_scale", "ffn_down_exps.scale"), ("shared_gate", "ffn_gate_inp_shexp.weight")):
        if b + name in g.tensors:
            out[key] = g.tensors[b + name]
    return out
