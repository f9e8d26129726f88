"""Writes tests/golden/gguf_headers.json.gz from the reference's GGUF header dumps (fleet/*/gguf/*.json.gz).

    python tests/golden/make_gguf_fixtures.py [REFERENCE_ROOT]      (default /root/reference)

The dumps keep a GGUF's header (KV values as raw bytes, large ones in the content-addressed store fleet/blobs/*.xz),
its tensor table [name, dims, ggml type, offset] and the layout facts (version, alignment, data_start, size). The
fixture keeps, for three models of the benchmark workloads, the tensor table, the layout facts and every KV entry;
values of 4 KiB or more are reduced to their key, type and byte length (enough to rebuild a header of the same
length, so data_start and every tensor offset stay those of the real file). Nothing of the reference is imported or
executed: the dumps are gzip'd JSON, the blobs xz files.
"""
import base64
import gzip
import json
import lzma
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
MODELS = {
    "qwen3_8b_q4_k_m": "fleet/unsloth-Qwen3-8B-loom/gguf/Qwen3-8B-Q4_K_M.gguf.json.gz",
    "qwen3_coder_30b_a3b_q4_k_m": None,   # found by name below
    "gpt_oss_20b": None,
}
PATTERNS = {"qwen3_coder_30b_a3b_q4_k_m": "Qwen3-Coder-30B-A3B-Instruct-Q4_K_M.gguf.json.gz",
            "gpt_oss_20b": "gpt-oss-20b-Q4_K_M.gguf.json.gz"}
SMALL = 4096


def find(root, name):
    for dp, _, fs in os.walk(os.path.join(root, "fleet")):
        if name in fs:
            return os.path.join(dp, name)
    raise FileNotFoundError(name)


def main(root):
    out = {}
    for key, rel in MODELS.items():
        path = os.path.join(root, rel) if rel else find(root, PATTERNS[key])
        d = json.load(gzip.open(path))
        kv = []
        for e in d["kv"]:
            if "blob" in e:
                raw = lzma.decompress(open(os.path.join(root, "fleet", "blobs", e["blob"] + ".xz"), "rb").read())
            else:
                raw = base64.b64decode(e["raw"])
            if len(raw) < SMALL:
                kv.append({"key": e["key"], "type": e["type"], "raw": base64.b64encode(raw).decode()})
            else:
                kv.append({"key": e["key"], "type": e["type"], "len": len(raw)})
        out[key] = {"source": os.path.relpath(path, root), "version": d["version"], "alignment": d["alignment"],
                    "size": d["size"], "data_start": d["data_start"], "kv": kv, "tensors": d["tensors"]}
    with gzip.GzipFile(os.path.join(HERE, "gguf_headers.json.gz"), "wb", mtime=0) as f:
        f.write(json.dumps(out, separators=(",", ":")).encode())


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
