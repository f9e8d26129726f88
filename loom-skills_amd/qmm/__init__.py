"""qmm: MI355X (gfx950) quantized-weight matmul path — GGUF Q4_0 / Q4_K and OCP MXFP4 weights dequantized inside the
decode GEMV, the prefill GEMM and the MoE routed-expert chain, as hand-written HIP kernels in libqmm.so.

    import qmm                      # host-side op surface over the C ABI (include/qmm.h)
    qmm.ops.mv("q4_k", w, x, n, k)  # g_mv_q4_k_k{K}: y = x W^T
    qmm.launch.launch("g_mv_q4_k_k4096_q8", [n, t], [n, t, 0, xq, w, y])   # a reference kernel launch by name

The library is loaded on first use and must have been built (qmm.build.build()); there is no CPU fallback.
"""
from . import formats  # noqa: F401

__version__ = "0.1.0"


def __getattr__(name):
    if name in ("ops", "launch", "gguf", "synth", "build"):
        import importlib
        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(name)
