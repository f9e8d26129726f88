#!/usr/bin/env python3
"""Throughput of the quantized-weight matmul path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--m M] [--no-cpu] [--no-secondary]

A step is one pass of the hot path over one batch of synthetic input. The default run measures the headline workload
(`value`), then every other workload of the metric as a compact entry of `secondary` (skipped when --workload names
one workload, or with --no-secondary):

    q4_k_gemv_q8  (headline) Q4_K decode GEMV, W [12288, 4096] (Qwen3-8B FFN gate/up), x bf16 [M, 4096], y f32, on
                the int8-activation path the reference takes by default: the bf16 rows are quantized to Q8_1 inside
                the kernel and multiplied with exact int32 group dot products; the weights are repacked once (before
                timing) into the lane-ordered tiled layout (qmm_tile_q4k), a byte permutation of the GGUF blocks.
                Secondary at M = 4 and 8.
    q4_k_swiglu_q8 the int8 swiglu matvec silu(x Wg^T) (x Wu^T), Wg, Wu [12288, 4096] Q4_K tiled, x bf16 [M, 4096]
    q4_k_gemv_q8_gguf the int8 GEMV reading the GGUF Q4_K blocks as they are
    q4_k_gemv   the Q4_K GEMV on the f16-activation path (x bf16 staged as f16, v_dot2_f32_f16)
    q4_k_gemv_q8p the int8 GEMV on its reference boundary: x is the planar Q8_1 buffer qmm_quant_q8 makes
    q4_0_gemv   Q4_0 decode GEMV, W [4096, 4096], x f32 [1, 4096], y f32 (the weights repacked once into the tiled
                layout; f32 activations, the reference's default Q4_0 decode)
    q4_0_gemv_q8 the same GEMV on the int8-activation path, the weights repacked once into the tiled layout
                (qmm_tile_q40) the Q4_K int8 kernel streams
    q4_k_gemm   Q4_K prefill GEMM, x bf16 [512, 4096] (row scale to f16, then the MFMA GEMM), W [4096, 4096],
                y bf16 [512, 4096] (Qwen3-8B attn o_proj)
    mxfp4_moe   MXFP4 MoE at the gpt-oss-20b shape (32 experts, top-4, H = FE = 2880), T tokens (--m): T < 64 the
                decode chain (top-k, gate/up and down expert matvecs, combine), else the prefill chain
                (top-k, bucket, MXFP8 quantize, grouped gate_up on the scaled MFMA + swiglu_oai with the MXFP8
                quantization of its output fused, grouped down, combine). Secondary at T = 1, 256, 1024 and 4096.
    q4_k_moe    Q4_K MoE prefill chain at the Qwen3-30B-A3B shape (128 experts, top-8, H = 2048, FE = 768), T = 64
    hbm_copy    calibration: a 256 MiB device copy, whose counter readings scale FETCH_SIZE / WRITE_SIZE to bytes

Consecutive steps read different copies of the weights (more than 300 MB in rotation), so the 256 MB MALL cannot
serve them and the figures are HBM figures. The W warm-up steps run first, repeated until 30 ms of GPU time has
passed (the clocks leave their idle state during the host-side setup). The K timed steps are launched one by one
behind a GPU spin kernel that outlasts the host's enqueueing and 3 ms of warm-up steps queued behind it (--graph:
captured in one HIP graph, which adds a launch overhead of its own on this stack), so every step is queued on the
device before the first timed kernel starts, the GPU has run the workload right up to it, and the two HIP events on
the launching stream see the kernels and the dispatch gaps between them, not the host. The region of K steps is
timed 5 times and its median taken; value = algorithmic work x K / that median. `roofline` is the dominant
kernel's: algorithmic bytes (or FLOPs) per launch over its average launch time, K eager launches of that kernel
alone back to back between two HIP events (kernel time plus the dispatch gap; the step's own timing where a step is
one launch of it). `cpu_baseline` times the numpy oracle on this host's cores on the same workload (dequant and
matmul separately and together), at least 5 runs.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "loom-skills_amd"))

import numpy as np  # noqa: E402

METRIC = "Q4_K GEMV GB/s (% HBM peak); MXFP4 MoE prefill TFLOP/s (% MFMA peak)"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "fp16": 2500.0, "fp8": 5000.0, "fp4": 10100.0}
ROTATE_BYTES = 300 * 2 ** 20
SPIN_CYCLES = 4_000_000   # the spin ahead of a timed graph: about 2 ms, longer than the host's graph submission

# (workload, M or T) measured after the headline by the default run
SECONDARY = [("q4_k_gemv_q8", 4), ("q4_k_gemv_q8", 8), ("q4_k_swiglu_q8", 1), ("q4_k_gemv", 1), ("q4_0_gemv", 1),
             ("q4_0_gemv_q8", 1),
             ("q4_k_gemm", 512), ("mxfp4_moe", 1), ("mxfp4_moe", 256), ("mxfp4_moe", 1024), ("mxfp4_moe", 4096),
             ("q4_k_moe", 64)]


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", default=None, choices=sorted(WORKLOADS))
    p.add_argument("--m", type=int, default=None, help="tokens (GEMV: M; MoE: T)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    p.add_argument("--no-secondary", action="store_true", help="measure the headline workload only")
    p.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work (headline)")
    p.add_argument("--cpu-budget-secondary", type=float, default=3.0, help="seconds of CPU work per secondary")
    p.add_argument("--graph", action="store_true",
                   help="capture the timed steps in one HIP graph instead of launching them one by one")
    return p.parse_args()


def traffic_from_profile(name):
    """HBM bytes per launch recorded by the rocprofv3 --pmc runs summarised in profiles/<name>.txt
    (a line 'traffic_bytes_per_launch: <int>'), or None."""
    path = os.path.join(ROOT, "profiles", name + ".txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    return None


_WEIGHTS = {}


def cached_workload(index, **kw):
    """synth.workload with the weights of each workload generated once per process (every token count of a workload
    sees the same weights and the inputs a fresh call would draw)."""
    from qmm import synth
    return synth.workload(index, cache=_WEIGHTS, **kw)


def cpu_entry(res, work, unit, scale, kind_sample):
    """cpu_baseline dict from a cpu_baseline timing result: value = work / total time in `unit` (work / scale)."""
    out = {"value": round(work / res["total_s"] / scale, 6), "unit": unit, "cores": res["threads"], "kind": "port",
           "dequant_ms": round(res["dequant_s"] * 1e3, 3), "matmul_ms": round(res["matmul_s"] * 1e3, 3),
           "total_ms": round(res["total_s"] * 1e3, 3), "sample": kind_sample}
    return out


# ------------------------------------------------------------------------------------------------ workloads
class GemvWorkload:
    """Decode GEMV y = x W^T over rotated weight copies; one step = one qmm_mv / qmm_mv_q8 launch (or the swiglu
    matvec over a gate and an up matrix)."""
    metric, unit, bound = METRIC, "GB/s", "hbm"

    def __init__(self, name, index, fmt, n, k, m, x_dtype, traffic_name, q8=False, tiled=False, swiglu=False):
        self.name, self.index, self.fmt, self.n, self.k, self.m = name, index, fmt, n, k, m
        self.x_dtype, self.traffic_name, self.q8, self.tiled = x_dtype, traffic_name, q8, tiled
        self.swiglu = swiglu
        # the weights the kernel reads (tiled: repacked once at load)
        self.kfmt = {"q4_k": "q4_kt", "q4_0": "q4_0t"}[fmt] if tiled else fmt

    def setup(self, dev):
        import torch
        from qmm import ops, synth
        d = cached_workload(self.index, m=self.m)
        self.raw = d["w"]
        if self.x_dtype == "bf16":
            self.x_host = synth.bf16_bits_to_f32(d["x_bf16"])
            x = torch.from_numpy(d["x_bf16"].view(np.int16)).to(dev).view(torch.bfloat16)
        else:
            self.x_host = d["x"]
            x = torch.from_numpy(d["x"]).to(dev)
        w0 = torch.from_numpy(self.raw).to(dev)
        if self.swiglu:   # the up matrix: the gate matrix's code bytes in reverse order (same distributions)
            self.raw_up = np.ascontiguousarray(self.raw.reshape(-1, 144)[::-1]).reshape(-1)
            w0 = torch.cat([w0, torch.from_numpy(self.raw_up).to(dev)])
        if self.tiled:   # one-time weight preparation: GGUF blocks -> the lane-ordered tiled layout
            tile = ops.tile_q4k if self.fmt == "q4_k" else ops.tile_q40
            parts = [tile(p, self.n, self.k) for p in w0.chunk(2 if self.swiglu else 1)]
            w0 = torch.cat(parts) if len(parts) > 1 else parts[0]
        self.wbytes = w0.numel()
        copies = max(2, -(-ROTATE_BYTES // self.wbytes))
        self.ws = [w0] + [w0.clone() for _ in range(copies - 1)]
        self.x = x
        self.y = torch.empty((self.m, self.n), dtype=torch.float32, device=dev)
        self.ops = ops
        self.copies = copies
        # more than two rows of activations are quantized by a quant_q8 pass ahead of the matvec (ops.mv_q8); the
        # dominant kernel is then the matvec over that planar buffer, timed alone
        self.split = bool(self.q8) and (self.q8 == "planar" or (self.tiled and self.m > 2))
        if self.split:
            self.xq = ops.quant_q8(self.x)

    def step(self, i):
        w = self.ws[i % self.copies]
        if self.swiglu:
            g, u = w.chunk(2)
            self.ops.mv_swiglu_q8(self.kfmt, g, u, self.x, self.n, self.k, y=self.y)
        elif self.q8 == "planar":
            self.ops.mv_q8(self.kfmt, w, self.xq, self.n, self.k, tokens=self.m, y=self.y)
        elif self.q8:
            self.ops.mv_q8(self.kfmt, w, self.x, self.n, self.k, y=self.y)
        else:
            self.ops.mv(self.kfmt, w, self.x, self.n, self.k, y=self.y)

    @property
    def kernel_is_step(self):
        return not self.split

    def kernel_step(self, i):
        if not self.split:
            return self.step(i)
        w = self.ws[i % self.copies]
        if self.swiglu:
            g, u = w.chunk(2)
            self.ops.mv_swiglu_q8(self.kfmt, g, u, self.xq, self.n, self.k, tokens=self.m, y=self.y)
        else:
            self.ops.mv_q8(self.kfmt, w, self.xq, self.n, self.k, tokens=self.m, y=self.y)

    def kernel_bytes(self):
        if not self.split:
            return self.alg_bytes()
        return self.wbytes + self.m * (self.k + self.k // 32 * 8) + self.m * self.n * 4

    def value(self, sec):
        return self.alg_bytes() / sec / 1e9

    def dtype(self):
        if self.q8 == "planar":
            return f"{self.fmt} x int8 (planar Q8_1 from qmm_quant_q8) -> f32, int32 group dots"
        if self.q8:
            return f"{self.fmt} x int8 (Q8_1 of {self.x_dtype}, quantized in the kernel) -> f32, int32 group dots"
        return "q4_k x f16 (bf16 x) -> f32" if self.fmt == "q4_k" else "q4_0 x f32 -> f32"

    def alg_bytes(self):
        if self.q8 == "planar":   # the planar Q8_1 buffer: a code byte per value and 8 bytes per 32 values
            return self.wbytes + self.m * (self.k + self.k // 32 * 8) + self.m * self.n * 4
        xb = 2 if self.x_dtype == "bf16" else 4
        return self.wbytes + self.m * self.k * xb + self.m * self.n * 4

    def alg_flops(self):
        return 2 * self.m * self.n * self.k * (2 if self.swiglu else 1)

    def cpu_baseline(self, budget):
        from oracle import cpu_baseline, ref
        x = ref.q8_1(self.x_host) if self.q8 else self.x_host
        n = self.n * (2 if self.swiglu else 1)
        raw = np.concatenate([self.raw, self.raw_up]) if self.swiglu else self.raw
        res = cpu_baseline.time_gemv(self.fmt, raw, n, self.k, x, budget_s=budget)
        return cpu_entry(res, self.alg_bytes(), "GB/s", 1e9,
                         f"{res['runs']} full {self.fmt} GEMVs (N={n}, K={self.k}, M={self.m}): numpy oracle, "
                         f"dequant fused in 256-row chunks + f32 matmul on {res['threads']} threads")

    def tokens(self):
        return self.m

    def config(self):
        return {"workload": self.name, "format": self.fmt, "layout": f"tiled ({self.kfmt})" if self.tiled else "gguf",
                "N": self.n, "K": self.k, "M": self.m,
                "x_dtype": "q8_1 planar" if self.q8 == "planar" else self.x_dtype,
                "activations": "q8_1" if self.q8 else self.x_dtype, "y_dtype": "f32",
                "weight_copies_rotated": self.copies, "rotated_bytes": self.copies * self.wbytes}


class GemmWorkload:
    """Q4_K prefill GEMM: one step = row-scale bf16 x to f16 + the GEMM (bf16 out) on the next weight copy."""
    metric, unit, bound = "Q4_K prefill GEMM TFLOP/s (Qwen3-8B o_proj, 512 x 4096 x 4096)", "TFLOP/s", "mfma"
    peak_key = "fp16"
    name = "q4_k_gemm"

    def __init__(self, m):
        self.m, self.n, self.k = m or 512, 4096, 4096
        self.traffic_name = f"q4k_dense_kernel.q4_k_gemm_m{self.m}_n4096_k4096"

    def setup(self, dev):
        import torch
        from qmm import ops
        d = cached_workload(2, m=self.m)
        self.raw, self.x_bits = d["w"], d["x_bf16"]
        w0 = torch.from_numpy(self.raw).to(dev)
        self.wbytes = w0.numel()
        self.copies = max(2, -(-ROTATE_BYTES // self.wbytes))
        self.ws = [w0] + [w0.clone() for _ in range(self.copies - 1)]
        self.x = torch.from_numpy(self.x_bits.view(np.int16)).to(dev).view(torch.bfloat16)
        self.x16 = torch.empty((self.m, self.k), dtype=torch.float16, device=dev)
        self.scales = torch.empty((self.m, 2), dtype=torch.float32, device=dev)
        self.y = torch.empty((self.m, self.n), dtype=torch.bfloat16, device=dev)
        self.ops = ops
        self.ops.row_scale_f16(self.x, x16=self.x16, scales=self.scales)

    def step(self, i):
        self.ops.row_scale_f16(self.x, x16=self.x16, scales=self.scales)
        self.kernel_step(i)

    def kernel_step(self, i):
        self.ops.gemm("q4_k", "store", self.x16, self.ws[i % self.copies], self.n, self.k, scales=self.scales,
                      y=self.y)

    def alg_bytes(self):
        return self.wbytes + self.m * self.k * 2 + self.m * self.n * 2

    def alg_flops(self):
        return 2 * self.m * self.n * self.k

    def library_setup(self, dev):
        """Context, not a baseline of this path: the same GEMM shape with plain f16 weights through torch.matmul
        (hipBLASLt), two weight copies in turn."""
        import torch
        g = torch.Generator(device=dev).manual_seed(0)
        self.lib_b = [torch.randn((self.n, self.k), generator=g, device=dev, dtype=torch.float16) for _ in range(2)]
        self.lib_y = torch.empty((self.m, self.n), dtype=torch.float16, device=dev)

    def library_step(self, i):
        import torch
        torch.matmul(self.x16, self.lib_b[i % 2].t(), out=self.lib_y)

    def value(self, sec):
        return self.alg_flops() / sec / 1e12

    def dtype(self):
        return "q4_k x f16 (row-scaled bf16) -> bf16, fp32 accumulate"

    def cpu_baseline(self, budget):
        from oracle import cpu_baseline
        from qmm import synth
        x = synth.bf16_bits_to_f32(self.x_bits)
        res = cpu_baseline.time_gemv("q4_k", self.raw, self.n, self.k, x, budget_s=budget)
        return cpu_entry(res, self.alg_flops(), "TFLOP/s", 1e12,
                         f"{res['runs']} full GEMMs (M={self.m}, N={self.n}, K={self.k}): numpy oracle, dequant "
                         f"fused in 256-row chunks + f32 matmul on {res['threads']} threads")

    def tokens(self):
        return self.m

    def config(self):
        return {"workload": self.name, "format": "q4_k", "M": self.m, "N": self.n, "K": self.k, "x_dtype": "bf16",
                "y_dtype": "bf16", "weight_copies_rotated": self.copies, "rotated_bytes": self.copies * self.wbytes}


class MoeWorkload:
    """The routed-expert chain (ops.moe_routed: the decode chain for T < 64, the prefill chain from 64 tokens); one
    step = the whole chain over one batch of T tokens, on one of several copies of the expert weights in turn."""
    unit = "TFLOP/s"

    def __init__(self, name, index, m):
        self.name, self.index = name, index
        if index == 3:
            self.T = m or 256
            self.metric = METRIC
        else:
            self.T = m or 64
            chain = "decode" if self.T < 64 else "prefill"
            self.metric = f"Q4_K MoE {chain} TFLOP/s (Qwen3-30B-A3B, 128 experts, top-8)"
        self.decode = self.T < 64
        # the Q4_K prefill chain streams the tiled layout through the narrow grouped kernel
        kern = ("mxt_expert_kernel" if self.decode else "mxfp4_grouped_kernel_gu8") if index == 3 else \
            ("expert_mv_q8_kernel" if self.decode else "q4k_narrow_kernel_gu")
        model = "mxfp4_moe_gpt_oss_20b" if index == 3 else "q4_k_moe_qwen3_30b_a3b"
        self.traffic_name = f"{kern}.{model}_t{self.T}"

    def setup(self, dev):
        import torch
        from qmm import ops
        d = cached_workload(self.index, T=self.T)
        self.d = d
        self.E, self.KU, self.H, self.FE = d["E"], d["KU"], d["H"], d["FE"]
        u8 = lambda a: torch.from_numpy(a).to(dev)
        self.x = torch.from_numpy(d["x_bf16"].view(np.int16)).to(dev).view(torch.bfloat16)
        self.logits = torch.from_numpy(d["logits"]).to(dev)
        E, H, FE = self.E, self.H, self.FE
        if d["fmt"] == "mxfp4":
            # one-time weight preparation: GGUF blocks -> split planes -> MFMA-tiled planes, the one copy the decode
            # expert matvecs and the prefill grouped GEMMs both read
            gn, gs = ops.repack_mxfp4(u8(d["gate_up"]), E * 2 * FE, H)
            dn, ds = ops.repack_mxfp4(u8(d["down"]), E * H, FE)
            gn, gs = ops.tile_mxfp4(gn, gs, E * 2 * FE, H)
            dn, ds = ops.tile_mxfp4(dn, ds, E * H, FE)
            self.fmt = "mxfp4t"
            self.kw = dict(w_gate=gn, ws_gate=gs, w_down=dn, ws_down=ds, fused=True, act=d["act"])
            self.wbytes_expert = (2 * FE * H + H * FE) // 2 + (2 * FE * H + H * FE) // 32
            self.peak_key = "fp8"
        else:
            # prefill: one-time weight preparation, GGUF blocks -> the tiled Q4_K layout the grouped GEMMs stream
            self.kw = dict(w_gate=u8(d["gate"]), w_up=u8(d["up"]), w_down=u8(d["down"]), fused=False, act=d["act"])
            self.fmt = "q4_k"
            if not self.decode:
                for m, rows, k in (("w_gate", E * FE, H), ("w_up", E * FE, H), ("w_down", E * H, FE)):
                    self.kw[m] = ops.tile_q4k(self.kw[m], rows, k)
                self.fmt = "q4_kt"
            self.wbytes_expert = (2 * FE * H + H * FE) // 256 * 144
            self.peak_key = "fp16"
        self.ops = ops
        # a second copy of every expert tensor, alternated from step to step: one layer's experts (441 MB MXFP4,
        # 340 MB Q4_K) are close to the 256 MB MALL, and a kernel timed on the same copy again would partly be
        # served from it
        self.kws = [self.kw]
        self.copies = 1
        y, mid = self.run_chain()
        torch.cuda.synchronize()
        self.experts_hit = int(torch.unique(mid["ids"]).numel())
        self.mid = mid
        # copies of every expert tensor, taken in turn from step to step, so that more than 300 MB of expert weights
        # pass between two reads of one copy and the 256 MB MALL cannot serve them: one layer's experts (441 MB MXFP4,
        # 340 MB Q4_K) at prefill, 6 copies of the 4 x 13.2 MB the MXFP4 decode chain reads at one token
        touched = self.experts_hit * self.wbytes_expert
        self.copies = max(2, -(-ROTATE_BYTES // touched))
        while len(self.kws) < self.copies:
            self.kws.append({k: (v.clone() if hasattr(v, "clone") else v) for k, v in self.kw.items()})
        self.rotated_bytes = self.copies * touched
        # inputs of the dominant kernel (the gate/up GEMM or expert matvec) for its own timing; the decode chain
        # routes inside its gate/up matvecs where ops.moe_decode does
        # int8 decode (the reference's MOE_Q8 default for Q4_K / Q6_K): the Q8_1 gate/up matvecs on the quantized x
        kw0 = self.kw
        self.q8 = self.decode and ops._moe_q8("auto", self.fmt, kw0.get("fmt_down") or ops.gate_format(self.fmt),
                                              kw0.get("expert_bias"))
        self.route_gu = (self.decode and not self.q8 and self.E <= ops.ROUTE_GU_MAX_E
                         and self.T * self.KU <= ops.ROUTE_GU_MAX_A)
        if self.decode:
            self.gu_y = torch.empty_like(mid["act"])
            if self.q8:
                self.gu_xq = ops.quant_q8(self.x)
        elif self.fmt == "mxfp4t":   # prefill
            self.gu_x, self.gu_xs = ops.quant_mxfp8(self.x)
            self.gu_y = (torch.empty_like(mid["act8"]), torch.empty_like(mid["act_scales"]))
        else:
            self.gu_x, self.gu_xs = ops.row_scale_f16(self.x)
            self.gu_y = torch.empty_like(mid["act"])

    def run_chain(self, i=0):
        return self.ops.moe_routed(self.fmt, self.x, self.logits, self.E, self.KU, self.H, self.FE, self.d["gating"],
                                   self.d["norm"], **self.kws[i % self.copies])

    def step(self, i):
        self.run_chain(i)

    def kernel_step(self, i):
        kw = self.kws[i % self.copies]
        if self.decode and self.route_gu:   # the decode chain's gate/up expert matvecs, routing their own tokens
            self.ops.moe_topk_expert_mv(self.fmt, self.logits, self.KU, self.d["gating"], self.d["norm"], self.x,
                                        kw["w_gate"], self.FE, self.H, self.E, w2=kw.get("w_up"), ws=kw.get("ws_gate"),
                                        fused=kw["fused"], act=kw["act"], y=self.gu_y)
        elif self.decode and self.q8:   # the int8 gate/up expert matvecs of the decode chain
            self.ops.moe_expert_mv_q8(self.fmt, "gu", self.mid["ids"], self.gu_xq, kw["w_gate"], self.FE, self.H,
                                      self.E, self.KU, w2=kw.get("w_up"), fused=kw["fused"], act=kw["act"],
                                      y=self.gu_y)
        elif self.decode:   # the gate/up expert matvecs of the decode chain
            self.ops.moe_expert_mv(self.fmt, "gu", self.mid["ids"], self.x, kw["w_gate"], self.FE, self.H, self.E,
                                   self.KU, w2=kw.get("w_up"), ws=kw.get("ws_gate"), fused=kw["fused"],
                                   act=kw["act"], y=self.gu_y)
        elif self.fmt == "mxfp4t":   # prefill: the gate/up GEMM with its activation written as MXFP8 (the chain's kernel)
            self.ops.moe_grouped_mxfp8(self.fmt, self.mid["tile_info"], self.mid["rowmap"], self.gu_x, kw["w_gate"],
                                       self.FE, self.H, self.E, self.KU, ws=kw.get("ws_gate"), x_scales=self.gu_xs,
                                       fused=kw["fused"], act=kw["act"], codes=self.gu_y[0], scales=self.gu_y[1])
        else:
            self.ops.moe_grouped(self.fmt, "gu", self.mid["tile_info"], self.mid["rowmap"], self.gu_x, kw["w_gate"],
                                 self.FE, self.H, self.E, self.KU, w2=kw.get("w_up"), ws=kw.get("ws_gate"),
                                 x_scales=self.gu_xs, fused=kw["fused"], act=kw["act"], y=self.gu_y)

    @property
    def bound(self):
        # arithmetic intensity of the whole chain against the MFMA / HBM balance point
        ai = self.alg_flops() / self.alg_bytes()
        return "mfma" if ai > MFMA_PEAK_TFLOPS[self.peak_key] * 1e12 / (HBM_PEAK_GBS * 1e9) else "hbm"

    def alg_bytes(self):
        T, H, E = self.T, self.H, self.E
        return self.experts_hit * self.wbytes_expert + T * H * 2 + T * H * 4 + T * E * 4

    def alg_flops(self):
        return 2 * self.T * self.KU * (self.H * 2 * self.FE + self.FE * self.H)

    def kernel_bytes(self):
        """weights of the experts hit, the activation rows in, the activation out (MXFP8 codes + scales for the
        MXFP4 grouped GEMM, f32 otherwise)"""
        T, H, A = self.T, self.H, self.T * self.KU
        wgu = self.experts_hit * (self.wbytes_expert * 2 // 3)
        if self.fmt == "mxfp4t" and not self.decode:
            return wgu + T * H + T * H // 32 + A * self.FE * 33 // 32
        return wgu + T * H * 2 + A * self.FE * 4

    def kernel_flops(self):
        return 2 * self.T * self.KU * self.H * 2 * self.FE

    def value(self, sec):
        return self.alg_flops() / sec / 1e12

    def dtype(self):
        if self.fmt == "mxfp4t" and self.decode:
            return "mxfp4 (MFMA-tiled planes) x bf16 -> f32 (expert matvecs)"
        if self.fmt == "mxfp4t":
            return "mxfp4 x mxfp8 (E4M3, E8M0 per 32) -> f32"
        if self.fmt == "q4_kt":
            return "q4_k (tiled layout) x f16 (row-scaled) -> f32"
        return "q4_k x f16 (row-scaled) -> f32"

    def cpu_baseline(self, budget):
        from oracle import cpu_baseline
        from oracle import formats as of
        from oracle import ref
        from qmm import synth
        d = self.d
        gfmt = "mxfp4" if self.fmt.startswith("mxfp4") else "q4_k"
        E, KU, H, FE = self.E, self.KU, self.H, self.FE
        rb_h, rb_f = of.row_bytes(gfmt, H), of.row_bytes(gfmt, FE)

        def experts(e):
            if gfmt == "mxfp4":
                gu = d["gate_up"][2 * FE * e * rb_h:2 * FE * (e + 1) * rb_h]
                g = of.dequantize(gfmt, gu[:FE * rb_h], FE, H)
                u = of.dequantize(gfmt, gu[FE * rb_h:], FE, H)
            else:
                g = of.dequantize(gfmt, d["gate"][FE * e * rb_h:FE * (e + 1) * rb_h], FE, H)
                u = of.dequantize(gfmt, d["up"][FE * e * rb_h:FE * (e + 1) * rb_h], FE, H)
            return g, u, of.dequantize(gfmt, d["down"][H * e * rb_f:H * (e + 1) * rb_f], H, FE)

        x = synth.bf16_bits_to_f32(d["x_bf16"])
        rnd = {"mxfp4t": ref.mxfp8_values, "q4_k": ref.f16_rows, "q4_kt": ref.f16_rows}.get(self.fmt)
        res = cpu_baseline.time_moe(x, d["logits"], KU, d["gating"], d["norm"], d["act"], experts, budget_s=budget,
                                    x_round=rnd, act_round=rnd)
        return cpu_entry(res, self.alg_flops(), "TFLOP/s", 1e12,
                         f"{res['runs']} full chains (T={self.T}, {res['experts_hit']} experts hit): numpy oracle, "
                         f"per-expert dequant + f32 matmuls on {res['threads']} threads")

    def config(self):
        return {"workload": self.name, "format": self.fmt, "chain": "decode" if self.decode else "prefill",
                "E": self.E, "top_k": self.KU, "H": self.H, "FE": self.FE, "T": self.T, "gating": self.d["gating"],
                "act": self.d["act"], "experts_hit": self.experts_hit, "weight_copies_rotated": self.copies,
                "rotated_expert_bytes": self.rotated_bytes}

    def tokens(self):
        return self.T


class CopyWorkload:
    """Calibration: a plain device-to-device copy of a known size (256 MiB, torch's copy kernel). Its FETCH_SIZE and
    WRITE_SIZE counter readings against the bytes it must move give the factors that turn those counters into HBM
    bytes for the other kernels."""
    metric, unit, bound = "HBM copy GB/s (counter calibration)", "GB/s", "hbm"
    name, traffic_name, kernel_step = "hbm_copy", "copy.hbm_copy_256mib", None

    def __init__(self, m):
        self.nbytes = (m or 256) * 2 ** 20

    def setup(self, dev):
        import torch
        self.src = [torch.randint(0, 255, (self.nbytes,), dtype=torch.uint8, device=dev) for _ in range(2)]
        self.dst = torch.empty_like(self.src[0])

    def step(self, i):
        self.dst.copy_(self.src[i % 2])

    def value(self, sec):
        return self.alg_bytes() / sec / 1e9

    def dtype(self):
        return "u8"

    def alg_bytes(self):
        return 2 * self.nbytes

    def alg_flops(self):
        return 0

    def cpu_baseline(self, budget):
        a = np.ones(self.nbytes // 4, np.uint8)
        b = np.empty_like(a)
        t0, runs = time.perf_counter(), 0
        while runs < 3 or time.perf_counter() - t0 < min(budget, 2.0):
            np.copyto(b, a)
            runs += 1
        sec = (time.perf_counter() - t0) / runs
        return {"value": round(2 * a.nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{runs} numpy copies of {a.nbytes >> 20} MiB"}

    def config(self):
        return {"workload": self.name, "bytes": self.nbytes}


def _q4k_gemv(m):
    return GemvWorkload("q4_k_gemv", 1, "q4_k", 12288, 4096, m or 1, "bf16",
                        f"mv_q4k_kernel.q4_k_gemv_n12288_k4096_m{m or 1}")


def _q4k_gemv_q8(m):
    return GemvWorkload("q4_k_gemv_q8", 1, "q4_k", 12288, 4096, m or 1, "bf16",
                        f"mv_q4kt_q8_kernel.q4_k_gemv_q8_n12288_k4096_m{m or 1}", q8=True, tiled=True)


def _q4k_swiglu_q8(m):
    return GemvWorkload("q4_k_swiglu_q8", 1, "q4_k", 12288, 4096, m or 1, "bf16",
                        f"mv_q4kt_q8_kernel.q4_k_swiglu_q8_n12288_k4096_m{m or 1}", q8=True, tiled=True, swiglu=True)


def _q4k_gemv_q8_gguf(m):
    return GemvWorkload("q4_k_gemv_q8_gguf", 1, "q4_k", 12288, 4096, m or 1, "bf16",
                        f"mv_q4k_q8s_kernel.q4_k_gemv_q8_gguf_n12288_k4096_m{m or 1}", q8=True)


def _q4k_gemv_q8p(m):
    return GemvWorkload("q4_k_gemv_q8p", 1, "q4_k", 12288, 4096, m or 1, "bf16",
                        f"mv_q4kt_q8_kernel.q4_k_gemv_q8p_n12288_k4096_m{m or 1}", q8="planar", tiled=True)


def _q40_gemv(m):
    return GemvWorkload("q4_0_gemv", 0, "q4_0", 4096, 4096, m or 1, "f32",
                        f"mv_q40t_f32_kernel.q4_0_gemv_n4096_k4096_m{m or 1}", tiled=True)


def _q40_gemv_q8(m):
    return GemvWorkload("q4_0_gemv_q8", 0, "q4_0", 4096, 4096, m or 1, "f32",
                        f"mv_q4kt_q8_kernel.q4_0_gemv_q8_n4096_k4096_m{m or 1}", q8=True, tiled=True)


WORKLOADS = {"q4_k_gemv": _q4k_gemv, "q4_k_gemv_q8": _q4k_gemv_q8, "q4_k_gemv_q8_gguf": _q4k_gemv_q8_gguf,
             "q4_k_gemv_q8p": _q4k_gemv_q8p, "q4_k_swiglu_q8": _q4k_swiglu_q8, "q4_0_gemv": _q40_gemv,
             "q4_0_gemv_q8": _q40_gemv_q8,
             "q4_k_gemm": GemmWorkload, "mxfp4_moe": lambda m: MoeWorkload("mxfp4_moe", 3, m),
             "q4_k_moe": lambda m: MoeWorkload("q4_k_moe", 4, m), "hbm_copy": CopyWorkload}


# ---------------------------------------------------------------------------------------------------- timing
RAMP_MS = 30.0   # untimed GPU work before a timed region: the warm-up steps repeated until this much has run
PRE_MS = 3.0     # warm-up steps queued right ahead of the first timed step (behind the spin), in GPU time
MAX_SPIN_CYCLES = 1_000_000_000


def _ramp(run_once):
    """Repeats run_once() (the warm-up steps) until RAMP_MS of GPU time has passed, so the timed region starts at the
    clocks the workload runs at, not at the idle clocks of the host-side setup before it. Returns the GPU ms of one
    run_once()."""
    import torch
    total, n = 0.0, 0
    while total < RAMP_MS and n < 1000:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        run_once()
        b.record()
        torch.cuda.synchronize()
        total += a.elapsed_time(b)
        n += 1
    return total / n


def _spin_for(host_s_per_step, steps):
    """Spin cycles that outlast the host's enqueueing of `steps` steps (about 2.4 cycles a ns, twice the estimate)."""
    return int(min(max(SPIN_CYCLES, 2.0 * host_s_per_step * steps * 2.4e9), MAX_SPIN_CYCLES))


REPEATS = 5   # timed regions of K steps each; their median is reported (a region of 20 short steps varies by 5-10 %)


def timed(step_fn, steps, warmup, no_graph=False, repeats=REPEATS):
    """ms for `steps` steps between two HIP events on the launching stream (the median over `repeats` such regions),
    and the wall time of all of them.
    Graph mode captures the steps in one HIP graph; eager mode launches them one by one. Either way the warm-up steps
    run first (repeated for RAMP_MS of GPU time), then a spin kernel holds the stream while the host submits PRE_MS
    of warm-up steps and the timed steps behind it, so the events time the kernels and the gaps between them only,
    and the GPU has run the workload at full load right up to the first timed step (a spin alone, one wave, would
    let the clocks fall before it)."""
    import torch
    stream = torch.cuda.current_stream()

    def run(count, start):
        for i in range(count):
            step_fn(start + i)

    torch.cuda.synchronize()
    w = max(warmup, 1)
    times, wall = [], 0.0
    if no_graph:
        # the host's enqueue time a step, from a second warm-up pass (the first carries one-time costs: code object
        # loads, first calls)
        run(w, 0)
        torch.cuda.synchronize()
        h0 = time.perf_counter()
        run(w, 0)
        host = (time.perf_counter() - h0) / w
        gpu_ms = _ramp(lambda: run(w, 0)) / w
        pre = int(min(max(w, PRE_MS / max(gpu_ms, 1e-4)), 5000))
    else:
        gw, gt = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
        with torch.cuda.graph(gw):
            run(w, 0)
        with torch.cuda.graph(gt):
            run(steps, w)
        torch.cuda.synchronize()
        gpu_ms = _ramp(gw.replay)
    for _ in range(repeats):
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        if no_graph:
            torch.cuda._sleep(_spin_for(host, steps + pre))
            run(pre, 0)
            wall0 = time.perf_counter()
            t0.record(stream)
            run(steps, w)
            t1.record(stream)
        else:
            torch.cuda._sleep(SPIN_CYCLES)
            for _ in range(int(min(max(1, PRE_MS / max(gpu_ms, 1e-4)), 200))):
                gw.replay()
            wall0 = time.perf_counter()
            t0.record(stream)
            gt.replay()
            t1.record(stream)
        torch.cuda.synchronize()
        wall += time.perf_counter() - wall0
        times.append(t0.elapsed_time(t1))
    return float(np.median(times)), wall


KERNEL_LAUNCHES = 200   # launches of the dominant kernel a timed region for roofline.avg_launch_us


def kernel_time(fn, steps, warmup):
    """Average launch time (ms) of the dominant kernel: `steps` eager launches fn(warmup) .. back to back between two
    HIP events on the launching stream, after the warm-up launches and the ramp, queued behind a spin that outlasts
    the host's enqueueing (so the GPU runs them without idling: each launch's time is its kernel plus the dispatch
    gap to the next). The launches are eager because a captured graph adds its own launch overhead on this stack."""
    return timed(fn, steps, warmup, no_graph=True)[0] / steps


def measure(wl, args, cpu_budget):
    """Times one set-up workload; returns its result fields (the headline line's, or a secondary entry's)."""
    ms, wall = timed(wl.step, args.steps, args.warmup, no_graph=not args.graph)
    per_step_s = ms / 1e3 / args.steps
    if getattr(wl, "kernel_is_step", False) and not args.graph:
        per_launch_s = per_step_s   # the step is one launch of the dominant kernel: the same measurement
    else:
        # at least KERNEL_LAUNCHES launches a region, whatever --steps is: a short burst of a long kernel reads a few
        # per cent slow (the first launches after the host-side setup), and the profiles trace 200 launches
        per_launch_s = kernel_time(wl.kernel_step or wl.step, max(args.steps, KERNEL_LAUNCHES), args.warmup) / 1e3
    kb = wl.kernel_bytes() if hasattr(wl, "kernel_bytes") else wl.alg_bytes()
    kf = wl.kernel_flops() if hasattr(wl, "kernel_flops") else wl.alg_flops()
    if wl.bound == "hbm":
        achieved, peak, unit = kb / per_launch_s / 1e9, HBM_PEAK_GBS, "GB/s"
    else:
        achieved, peak, unit = kf / per_launch_s / 1e12, MFMA_PEAK_TFLOPS[wl.peak_key], "TFLOP/s"
    roof = {"bound": wl.bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic_from_profile(wl.traffic_name),
            "kernel": wl.traffic_name.split(".")[0], "avg_launch_us": round(per_launch_s * 1e6, 3),
            "alg_bytes_per_launch": kb, "alg_flops_per_launch": kf}
    res = {"value": round(wl.value(per_step_s), 3), "unit": wl.unit, "ms_per_step": round(ms / args.steps, 6),
           "roofline": roof, "gbs": round(wl.alg_bytes() / per_step_s / 1e9, 2),
           "tflops": round(wl.alg_flops() / per_step_s / 1e12, 3), "wall_s_timed_region": round(wall, 4),
           "timed_regions": REPEATS}
    if hasattr(wl, "tokens"):   # tokens through the step (decode rows, prefill rows, MoE tokens) a second
        res["tokens_per_s"] = round(wl.tokens() / per_step_s, 1)
    if getattr(wl, "peak_key", None) == "fp8":
        # the scaled MFMA runs E4M3 x E2M1 at the FP8 rate; the MXFP4 figure is the fraction of the FP4 peak
        res["chain_frac_fp4_peak"] = round(res["tflops"] / MFMA_PEAK_TFLOPS["fp4"], 4)
        res["chain_frac_fp8_rate"] = round(res["tflops"] / MFMA_PEAK_TFLOPS["fp8"], 4)
    if hasattr(wl, "library_step"):
        wl.library_setup(torch_device())
        lib_s = kernel_time(wl.library_step, max(args.steps, KERNEL_LAUNCHES), args.warmup) / 1e3
        lib_tf = wl.alg_flops() / lib_s / 1e12
        res["library_f16_gemm"] = {"what": "torch.matmul of the same shape, f16 x f16 (hipBLASLt), no dequantization",
                                   "us": round(lib_s * 1e6, 3), "tflops": round(lib_tf, 3),
                                   "frac": round(lib_tf / MFMA_PEAK_TFLOPS["fp16"], 4)}
    if cpu_budget:
        res["cpu_baseline"] = wl.cpu_baseline(cpu_budget)
    return res


def torch_device():
    import torch
    return torch.device("cuda:0")


def secondary_entry(name, m, wl, res):
    """The compact form of a secondary workload's result."""
    r = res["roofline"]
    out = {"workload": name, "m": m, "value": res["value"], "unit": res["unit"],
           "us_per_step": round(res["ms_per_step"] * 1e3, 3), "gbs": res["gbs"], "tflops": res["tflops"],
           "tokens_per_s": res.get("tokens_per_s"),
           "roofline": {k: r[k] for k in ("bound", "achieved", "unit", "frac", "traffic", "kernel", "avg_launch_us")}}
    if "chain_frac_fp4_peak" in res:
        out["chain_frac_fp4_peak"] = res["chain_frac_fp4_peak"]
    if "library_f16_gemm" in res:
        out["library_f16_gemm"] = res["library_f16_gemm"]
    if "cpu_baseline" in res:
        c = res["cpu_baseline"]
        out["cpu"] = {k: c[k] for k in ("value", "unit", "cores", "dequant_ms", "matmul_ms", "total_ms") if k in c}
    return out


# ---------------------------------------------------------------------------------------------------- main
def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this path has no multi-GPU code (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world})", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU (torch.cuda.is_available() is False)", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    name = args.workload or "q4_k_gemv_q8"
    wl = WORKLOADS[name](args.m)
    wl.setup(dev)
    res = measure(wl, args, 0 if args.no_cpu else args.cpu_budget)
    out = {
        "metric": wl.metric,
        "value": res["value"],
        "unit": wl.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.dtype(),
        "data": "synthetic (seeded generators of the workload's distributions)",
        "config": wl.config(),
        "roofline": res["roofline"],
    }
    out.update({k: v for k, v in res.items() if k not in out and k != "cpu_baseline"})
    if "cpu_baseline" in res:
        out["cpu_baseline"] = res["cpu_baseline"]
    del wl
    if args.workload is None and not args.no_secondary:
        sec = []
        for sname, m in SECONDARY:
            torch.cuda.empty_cache()
            w2 = WORKLOADS[sname](m)
            try:
                w2.setup(dev)
                r2 = measure(w2, args, 0 if args.no_cpu else args.cpu_budget_secondary)
            except Exception as e:   # a failing secondary is reported in its entry, not fatal to the line
                sec.append({"workload": sname, "m": m, "error": f"{type(e).__name__}: {str(e)[:120]}"})
                print(f"secondary {sname} m={m}: {e}", file=sys.stderr, flush=True)
                continue
            sec.append(secondary_entry(sname, m, w2, r2))
            print(f"secondary {sname} m={m}: {r2['value']} {r2['unit']} frac {r2['roofline']['frac']}",
                  file=sys.stderr, flush=True)
            del w2
        out["secondary"] = sec
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
