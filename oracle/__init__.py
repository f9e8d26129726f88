"""CPU oracle for the quantized-weight matmul path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of loom-skills' quantized dense and MoE matmul path so that the
HIP kernels can be checked against it. It is never the thing measured or shipped:

* only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it;
* the product path (``loom-skills_amd/qmm``) never imports it and fails loudly when its HIP library is missing.

Modules
-------
``formats``  block layouts and bit-exact decoders of GGUF Q4_0, Q4_K, MXFP4 (17-byte GGUF blocks) and MXFP4 split
             planes, plus the inverse Q4_K scale packer used to build known-answer blocks.
``ref``      float64 reference matmuls (GEMV, GEMM), the activation quantizers (Q8_1, row-scale f16, E4M3/MXFP8),
             routing (top-k, gating 1/2/3), the canonical bucket/permutation, expert activations, combine and the
             whole MoE chain.

Every function cites the reference file:line it restates (paths relative to the reference root; ``S/`` is
``skills/loom-port-llm/starter/``). How each function is pinned (known-answer tests, the reference's own fixtures,
closed forms, brute force) is recorded in the docstring of its test in ``tests/test_oracle_*.py``.
"""
