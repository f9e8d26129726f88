"""A minimal GGUF writer for the tests (v3, little endian): header bytes from KV entries and a tensor table, and
small files with tensor data."""
import base64
import struct

import numpy as np

ALIGN = 32


def kv_bytes(key, t, raw):
    k = key.encode()
    return struct.pack("<Q", len(k)) + k + struct.pack("<I", t) + raw


def stand_in(t, n):
    """A valid KV value of type t (string or array of strings) that takes exactly n bytes."""
    if t == 8:
        return struct.pack("<Q", n - 8) + b"x" * (n - 8)
    if t == 9:
        assert n >= 20
        return struct.pack("<IQQ", 8, 1, n - 20) + b"x" * (n - 20)
    raise ValueError(t)


def header(kv, tensors, version=3):
    """kv: [(key, type, raw value bytes)]; tensors: [(name, dims, ggml type, offset)]."""
    out = [b"GGUF", struct.pack("<IQQ", version, len(tensors), len(kv))]
    out += [kv_bytes(k, t, raw) for k, t, raw in kv]
    for name, dims, tt, off in tensors:
        nb = name.encode()
        out.append(struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims)))
        out += [struct.pack("<Q", int(d)) for d in dims]
        out.append(struct.pack("<IQ", tt, off))
    return b"".join(out)


def fixture_kv(model):
    return [(e["key"], e["type"], base64.b64decode(e["raw"]) if "raw" in e else stand_in(e["type"], e["len"]))
            for e in model["kv"]]


def write(path, kv, tensors_with_data):
    """tensors_with_data: [(name, dims, ggml type, uint8 bytes)]; offsets are assigned with 32-byte padding."""
    table, off = [], 0
    for name, dims, tt, data in tensors_with_data:
        table.append((name, dims, tt, off))
        off = (off + len(data) + ALIGN - 1) // ALIGN * ALIGN
    h = header(kv, table)
    start = (len(h) + ALIGN - 1) // ALIGN * ALIGN
    with open(path, "wb") as f:
        f.write(h + b"\0" * (start - len(h)))
        for (name, dims, tt, o), (_, _, _, data) in zip(table, tensors_with_data):
            f.seek(start + o)
            f.write(np.ascontiguousarray(data, np.uint8).tobytes())
    return table
