#!/usr/bin/env python3
"""Throughput of the quantized-weight matmul path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--m M] [--no-cpu]

A step is one launch of the hot path over one batch of synthetic input:

    q4_k_gemv_q8  (default) Q4_K decode GEMV, W [12288, 4096] (Qwen3-8B FFN gate/up), x bf16 [M, 4096], y f32, on
                the int8-activation path the reference takes by default: the bf16 rows are quantized to Q8_1 inside
                the kernel and multiplied with exact int32 group dot products; the weights are repacked once (before
                timing) into the lane-ordered tiled layout (qmm_tile_q4k), a byte permutation of the GGUF blocks
    q4_k_gemv_q8_gguf the same GEMV reading the GGUF Q4_K blocks as they are
    q4_k_gemv   the same GEMV on the f16-activation path (x staged as f16, v_dot2_f32_f16)
    q4_k_gemv_q8p the int8-activation GEMV on its reference boundary: x is the planar Q8_1 buffer qmm_quant_q8 makes
                (once per layer input, shared by the matvecs that read it), quantized before the timed region
    q4_0_gemv   Q4_0 decode GEMV, W [4096, 4096], x f32 [1, 4096], y f32
    q4_k_gemm   Q4_K prefill GEMM, x bf16 [512, 4096] (row scale to f16, then the MFMA GEMM), W [4096, 4096],
                y bf16 [512, 4096] (Qwen3-8B attn o_proj)
    mxfp4_moe   MXFP4 MoE prefill chain at the gpt-oss-20b shape (32 experts, top-4, H = FE = 2880), T tokens
                (--m, default 256): top-k, bucket, MXFP8 quantize, grouped gate_up (scaled MFMA) + swiglu_oai,
                quantize, grouped down, combine
    q4_k_moe    Q4_K MoE prefill chain at the Qwen3-30B-A3B shape (128 experts, top-8, H = 2048, FE = 768), T = 64
    hbm_copy    calibration: a 256 MiB device copy, whose counter readings scale FETCH_SIZE / WRITE_SIZE to bytes

Consecutive steps read different copies of the weight (more than 300 MB in rotation), so the 256 MB MALL cannot
serve them and the figure is an HBM figure. The K timed steps are captured in one HIP graph and replayed on the
launching stream between two HIP events; value = algorithmic bytes x K / elapsed. The JSON line also carries the
roofline of the kernel (achieved = algorithmic bytes per launch / average launch time from the same events) and
a CPU baseline: the numpy oracle timed on this host's cores on a bounded sample of the same workload.
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


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--workload", default="q4_k_gemv_q8", choices=sorted(WORKLOADS))
    p.add_argument("--m", type=int, default=None, help="tokens per GEMV (q4_k_gemv: 1, 4 or 8)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work")
    p.add_argument("--no-graph", action="store_true", help="launch steps one by one instead of a HIP graph")
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


# ------------------------------------------------------------------------------------------------ workloads
class GemvWorkload:
    """Decode GEMV y = x W^T over rotated weight copies; one step = one qmm_mv launch."""
    metric, unit, bound = METRIC, "GB/s", "hbm"

    def __init__(self, name, index, fmt, n, k, m, x_dtype, traffic_name, q8=False, tiled=False):
        self.name, self.index, self.fmt, self.n, self.k, self.m = name, index, fmt, n, k, m
        self.x_dtype, self.traffic_name, self.q8, self.tiled = x_dtype, traffic_name, q8, tiled
        self.kfmt = "q4_kt" if tiled else fmt   # the weights the kernel reads (tiled: repacked once at load)

    def setup(self, dev):
        import torch
        from qmm import ops, synth
        d = synth.workload(self.index, m=self.m)
        self.raw = d["w"]
        if self.x_dtype == "bf16":
            self.x_host = synth.bf16_bits_to_f32(d["x_bf16"])
            x = torch.from_numpy(d["x_bf16"].view(np.int16)).to(dev).view(torch.bfloat16)
        else:
            self.x_host = d["x"]
            x = torch.from_numpy(d["x"]).to(dev)
        w0 = torch.from_numpy(self.raw).to(dev)
        if self.tiled:   # one-time weight preparation: GGUF Q4_K blocks -> the lane-ordered tiled layout
            w0 = ops.tile_q4k(w0, self.n, self.k)
        self.wbytes = w0.numel()
        copies = max(2, -(-ROTATE_BYTES // self.wbytes))
        self.ws = [w0] + [w0.clone() for _ in range(copies - 1)]
        self.x = x
        self.y = torch.empty((self.m, self.n), dtype=torch.float32, device=dev)
        self.ops = ops
        self.copies = copies
        if self.q8 == "planar":
            self.xq = ops.quant_q8(self.x)

    def step(self, i):
        if self.q8 == "planar":
            self.ops.mv_q8(self.kfmt, self.ws[i % self.copies], self.xq, self.n, self.k, tokens=self.m, y=self.y)
        elif self.q8:
            self.ops.mv_q8(self.kfmt, self.ws[i % self.copies], self.x, self.n, self.k, y=self.y)
        else:
            self.ops.mv(self.fmt, self.ws[i % self.copies], self.x, self.n, self.k, y=self.y)

    kernel_step = None

    def value(self, sec):
        return self.alg_bytes() / sec / 1e9

    def dtype(self):
        if self.q8 == "planar":
            return f"{self.fmt} x int8 (planar Q8_1 from qmm_quant_q8) -> f32, int32 group dots"
        if self.q8:
            return f"{self.fmt} x int8 (Q8_1 of {self.x_dtype}, quantized in the kernel) -> f32, int32 group dots"
        return "q4_k x bf16 -> f32" if self.fmt == "q4_k" else "q4_0 x f32 -> f32"

    def alg_bytes(self):
        if self.q8 == "planar":   # the planar Q8_1 buffer: a code byte per value and 8 bytes per 32 values
            return self.wbytes + self.m * (self.k + self.k // 32 * 8) + self.m * self.n * 4
        xb = 2 if self.x_dtype == "bf16" else 4
        return self.wbytes + self.m * self.k * xb + self.m * self.n * 4

    def alg_flops(self):
        return 2 * self.m * self.n * self.k

    def cpu_baseline(self, budget):
        from oracle import cpu_baseline, ref
        x = ref.q8_1(self.x_host) if self.q8 else self.x_host
        sec, runs, threads = cpu_baseline.time_gemv(self.fmt, self.raw, self.n, self.k, x, budget_s=budget)
        return {"value": round(self.alg_bytes() / sec / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": f"{runs} full {self.fmt} GEMVs (N={self.n}, K={self.k}, M={self.m}): numpy oracle dequant "
                          f"in 256-row chunks + f32 matmul on {threads} threads, median {sec * 1e3:.1f} ms per GEMV"}

    def config(self):
        return {"workload": self.name, "format": self.fmt, "layout": "tiled (q4_kt)" if self.tiled else "gguf",
                "N": self.n, "K": self.k, "M": self.m,
                "x_dtype": "q8_1 planar" if self.q8 == "planar" else self.x_dtype,
                "activations": "q8_1" if self.q8 else self.x_dtype, "y_dtype": "f32",
                "weight_copies_rotated": self.copies,
                "rotated_bytes": self.copies * self.wbytes}


class GemmWorkload:
    """Q4_K prefill GEMM: one step = row-scale bf16 x to f16 + the GEMM (bf16 out) on the next weight copy."""
    metric, unit, bound = "Q4_K prefill GEMM TFLOP/s (Qwen3-8B o_proj, 512 x 4096 x 4096)", "TFLOP/s", "mfma"
    peak_key = "fp16"
    name, traffic_name = "q4_k_gemm", "q4k_mfma_kernel_dense.q4_k_gemm_m512_n4096_k4096"

    def __init__(self, m):
        self.m, self.n, self.k = m or 512, 4096, 4096

    def setup(self, dev):
        import torch
        from qmm import ops, synth
        d = synth.workload(2, m=self.m)
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

    def value(self, sec):
        return self.alg_flops() / sec / 1e12

    def dtype(self):
        return "q4_k x f16 (row-scaled bf16) -> bf16, fp32 accumulate"

    def cpu_baseline(self, budget):
        from oracle import cpu_baseline
        from qmm import synth
        x = synth.bf16_bits_to_f32(self.x_bits)
        sec, runs, threads = cpu_baseline.time_gemv("q4_k", self.raw, self.n, self.k, x, budget_s=budget)
        return {"value": round(self.alg_flops() / sec / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
                "kind": "port",
                "sample": f"{runs} full GEMMs (M={self.m}, N={self.n}, K={self.k}): numpy oracle dequant in 256-row "
                          f"chunks + f32 matmul on {threads} threads, median {sec * 1e3:.1f} ms per GEMM"}

    def config(self):
        return {"workload": self.name, "format": "q4_k", "M": self.m, "N": self.n, "K": self.k, "x_dtype": "bf16",
                "y_dtype": "bf16", "weight_copies_rotated": self.copies, "rotated_bytes": self.copies * self.wbytes}


class MoeWorkload:
    """MoE prefill chain; one step = the whole chain over one batch of T tokens, on one of two copies of the expert
    weights in turn (see setup)."""
    unit, higher = "TFLOP/s", True

    def __init__(self, name, index, m):
        self.name, self.index = name, index
        if index == 3:
            self.T = m or 256
            self.metric = METRIC
            self.traffic_name = f"mxfp4_grouped_kernel_gu8.mxfp4_moe_gpt_oss_20b_t{self.T}"
        else:
            self.T = m or 64
            self.metric = "Q4_K MoE prefill TFLOP/s (Qwen3-30B-A3B, 128 experts, top-8, T = 64)"
            self.traffic_name = f"q4k_mfma_kernel_gu.q4_k_moe_qwen3_30b_a3b_t{self.T}"

    def setup(self, dev):
        import torch
        from qmm import ops, synth
        d = synth.workload(self.index, T=self.T)
        self.d = d
        self.E, self.KU, self.H, self.FE = d["E"], d["KU"], d["H"], d["FE"]
        u8 = lambda a: torch.from_numpy(a).to(dev)
        self.x = torch.from_numpy(d["x_bf16"].view(np.int16)).to(dev).view(torch.bfloat16)
        self.logits = torch.from_numpy(d["logits"]).to(dev)
        if d["fmt"] == "mxfp4":
            E, H, FE = self.E, self.H, self.FE
            # one-time weight preparation: GGUF blocks -> split planes -> MFMA-tiled planes
            gn, gs = ops.repack_mxfp4(u8(d["gate_up"]), E * 2 * FE, H)
            dn, ds = ops.repack_mxfp4(u8(d["down"]), E * H, FE)
            gn, gs = ops.tile_mxfp4(gn, gs, E * 2 * FE, H)
            dn, ds = ops.tile_mxfp4(dn, ds, E * H, FE)
            self.fmt = "mxfp4t"
            self.kw = dict(w_gate=gn, ws_gate=gs, w_down=dn, ws_down=ds, fused=True, act=d["act"])
            self.wbytes_expert = (2 * FE * H + H * FE) // 2 + (2 * FE * H + H * FE) // 32
            self.peak_key = "fp8"
        else:
            self.fmt = "q4_k"
            self.kw = dict(w_gate=u8(d["gate"]), w_up=u8(d["up"]), w_down=u8(d["down"]), fused=False, act=d["act"])
            self.wbytes_expert = (2 * self.FE * self.H + self.H * self.FE) // 256 * 144
            self.peak_key = "fp16"
        self.ops = ops
        # a second copy of every expert tensor, alternated from step to step: one layer's experts (441 MB MXFP4,
        # 340 MB Q4_K) are close to the 256 MB MALL, and a kernel timed on the same copy again would partly be
        # served from it
        self.kws = [self.kw, {k: (v.clone() if hasattr(v, "clone") else v) for k, v in self.kw.items()}]
        self.copies = 2
        y, mid = self.run_chain()
        torch.cuda.synchronize()
        self.experts_hit = int(torch.unique(mid["ids"]).numel())
        # inputs of the dominant kernel (the grouped gate/up GEMM) for its own timing
        self.mid = mid
        if self.fmt == "mxfp4t":
            self.gu_x, self.gu_xs = ops.quant_mxfp8(self.x)
            self.gu_y = (torch.empty_like(mid["act8"]), torch.empty_like(mid["act_scales"]))
        else:
            self.gu_x, self.gu_xs = ops.row_scale_f16(self.x)
            self.gu_y = torch.empty_like(mid["act"])

    def run_chain(self, i=0):
        return self.ops.moe_prefill(self.fmt, self.x, self.logits, self.E, self.KU, self.H, self.FE, self.d["gating"],
                                    self.d["norm"], **self.kws[i % self.copies])

    def step(self, i):
        self.run_chain(i)

    def kernel_step(self, i):
        kw = self.kws[i % self.copies]
        if self.fmt == "mxfp4t":   # the gate/up GEMM with its activation written as MXFP8 (the chain's kernel)
            self.ops.moe_grouped_mxfp8(self.fmt, self.mid["tile_info"], self.mid["rowmap"], self.gu_x, kw["w_gate"],
                                       self.FE, self.H, self.E, self.KU, ws=kw.get("ws_gate"), x_scales=self.gu_xs,
                                       fused=kw["fused"], act=kw["act"], codes=self.gu_y[0], scales=self.gu_y[1])
            return
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

    def gu_bytes(self):
        """weights of the experts hit, the activation rows in, the activation out (MXFP8 codes + scales for MXFP4,
        f32 for Q4_K)"""
        T, H, A = self.T, self.H, self.T * self.KU
        if self.fmt == "mxfp4t":
            return self.experts_hit * (self.wbytes_expert * 2 // 3) + T * H + T * H // 32 + A * self.FE * 33 // 32
        return self.experts_hit * ((2 * self.FE * H) // 256 * 144) + T * H * 2 + A * self.FE * 4

    def gu_flops(self):
        return 2 * self.T * self.KU * self.H * 2 * self.FE

    def value(self, sec):
        return self.alg_flops() / sec / 1e12

    def dtype(self):
        return ("mxfp4 x mxfp8 (E4M3, E8M0 per 32) -> f32" if self.fmt == "mxfp4t"
                else "q4_k x f16 (row-scaled) -> f32")

    def cpu_baseline(self, budget):
        from oracle import formats as of
        from oracle import ref
        from qmm import synth
        import time as _t
        d = self.d
        gfmt = "mxfp4" if self.fmt == "mxfp4t" else "q4_k"
        E, KU, H, FE = self.E, self.KU, self.H, self.FE
        rb_h, rb_f = of.row_bytes(gfmt, H), of.row_bytes(gfmt, FE)
        def gate_up(e):
            if self.fmt == "mxfp4t":
                g = of.dequantize(gfmt, d["gate_up"][2 * FE * e * rb_h:(2 * FE * e + FE) * rb_h], FE, H)
                u = of.dequantize(gfmt, d["gate_up"][(2 * FE * e + FE) * rb_h:2 * FE * (e + 1) * rb_h], FE, H)
                return g, u
            return (of.dequantize(gfmt, d["gate"][FE * e * rb_h:FE * (e + 1) * rb_h], FE, H),
                    of.dequantize(gfmt, d["up"][FE * e * rb_h:FE * (e + 1) * rb_h], FE, H))
        def down(e):
            return of.dequantize(gfmt, d["down"][H * e * rb_f:H * (e + 1) * rb_f], H, FE)
        x = synth.bf16_bits_to_f32(d["x_bf16"])
        ids, wts = ref.route(d["logits"], KU, d["gating"], d["norm"])
        rnd = ref.mxfp8_values if self.fmt == "mxfp4t" else ref.f16_rows
        # bounded sample: the first tokens whose experts fit the time budget (the whole chain on them)
        tokens = 0
        t0 = _t.perf_counter()
        while tokens < self.T and _t.perf_counter() - t0 < budget:
            n = min(self.T - tokens, max(1, self.T // 16))
            ref.moe(x[tokens:tokens + n], ids[tokens:tokens + n], wts[tokens:tokens + n], gate_up, down,
                    act=d["act"], x_round=rnd, act_round=rnd)
            tokens += n
        sec = _t.perf_counter() - t0
        flops = 2 * tokens * KU * (H * 2 * FE + FE * H)
        return {"value": round(flops / sec / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
                "sample": f"{tokens} of {self.T} tokens through the numpy oracle's MoE chain (per-expert exact "
                          f"dequant + float64 matmuls, single-threaded numpy), {sec:.1f} s"}

    def config(self):
        return {"workload": self.name, "format": self.fmt, "E": self.E, "top_k": self.KU, "H": self.H,
                "FE": self.FE, "T": self.T, "gating": self.d["gating"], "act": self.d["act"],
                "experts_hit": self.experts_hit, "weight_copies_rotated": self.copies}


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


def _q4k_gemv_q8_gguf(m):
    return GemvWorkload("q4_k_gemv_q8_gguf", 1, "q4_k", 12288, 4096, m or 1, "bf16",
                        f"mv_q4k_q8s_kernel.q4_k_gemv_q8_gguf_n12288_k4096_m{m or 1}", q8=True)


def _q4k_gemv_q8p(m):
    return GemvWorkload("q4_k_gemv_q8p", 1, "q4_k", 12288, 4096, m or 1, "bf16",
                        f"mv_q4kt_q8_kernel.q4_k_gemv_q8p_n12288_k4096_m{m or 1}", q8="planar", tiled=True)


def _q40_gemv(m):
    return GemvWorkload("q4_0_gemv", 0, "q4_0", 4096, 4096, m or 1, "f32",
                        f"mv_kernel_q4_0.q4_0_gemv_n4096_k4096_m{m or 1}")


WORKLOADS = {"q4_k_gemv": _q4k_gemv, "q4_k_gemv_q8": _q4k_gemv_q8, "q4_k_gemv_q8_gguf": _q4k_gemv_q8_gguf,
             "q4_k_gemv_q8p": _q4k_gemv_q8p, "q4_0_gemv": _q40_gemv, "q4_k_gemm": GemmWorkload,
             "mxfp4_moe": lambda m: MoeWorkload("mxfp4_moe", 3, m), "q4_k_moe": lambda m: MoeWorkload("q4_k_moe", 4, m),
             "hbm_copy": CopyWorkload}


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
    wl = WORKLOADS[args.workload](args.m)
    wl.setup(dev)
    stream = torch.cuda.current_stream()

    def timed(step_fn):
        """ms for args.steps steps (HIP-graph replay between two events on the launching stream) and the wall time"""
        def run(count, start):
            for i in range(count):
                step_fn(start + i)
        torch.cuda.synchronize()
        if args.no_graph:
            run(args.warmup, 0)
            torch.cuda.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            wall0 = time.perf_counter()
            t0.record(stream)
            run(args.steps, args.warmup)
            t1.record(stream)
        else:
            gw, gt = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
            with torch.cuda.graph(gw):
                run(max(args.warmup, 1), 0)
            with torch.cuda.graph(gt):
                run(args.steps, args.warmup)
            torch.cuda.synchronize()
            if args.warmup:
                gw.replay()
            torch.cuda.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            wall0 = time.perf_counter()
            t0.record(stream)
            gt.replay()
            t1.record(stream)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1), time.perf_counter() - wall0

    ms, wall = timed(wl.step)
    per_step_s = ms / 1e3 / args.steps
    value = wl.value(per_step_s)
    kms = timed(wl.kernel_step)[0] if wl.kernel_step is not None else ms
    per_launch_s = kms / 1e3 / args.steps
    kb = wl.gu_bytes() if hasattr(wl, "gu_bytes") else wl.alg_bytes()
    kf = wl.gu_flops() if hasattr(wl, "gu_flops") else wl.alg_flops()
    if wl.bound == "hbm":
        achieved, peak, unit = kb / per_launch_s / 1e9, HBM_PEAK_GBS, "GB/s"
    else:
        achieved, peak, unit = kf / per_launch_s / 1e12, MFMA_PEAK_TFLOPS[wl.peak_key], "TFLOP/s"
    traffic = traffic_from_profile(wl.traffic_name)
    out = {
        "metric": wl.metric,
        "value": round(value, 3),
        "unit": wl.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.dtype(),
        "data": "synthetic (seeded generators of the workload's distributions)",
        "config": wl.config(),
        "roofline": {"bound": wl.bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
                     "frac": round(achieved / peak, 4), "traffic": traffic,
                     "alg_bytes_per_launch": kb, "alg_flops_per_launch": kf,
                     "avg_launch_us": round(per_launch_s * 1e6, 3),
                     "mfma_frac": round(kf / per_launch_s / 1e12 / MFMA_PEAK_TFLOPS.get(getattr(wl, "peak_key", "fp16"), 2500.0), 4)},
        "gbs": round(wl.alg_bytes() / per_step_s / 1e9, 2),
        "tflops": round(wl.alg_flops() / per_step_s / 1e12, 3),
        "wall_s_timed_region": round(wall, 4),
    }
    if getattr(wl, "fmt", None) == "mxfp4t":
        # the scaled MFMA runs E4M3 x E2M1 at the FP8 rate; the MXFP4 figure is the fraction of the FP4 peak
        out["roofline"]["mfma_frac_fp4_peak"] = round(kf / per_launch_s / 1e12 / MFMA_PEAK_TFLOPS["fp4"], 4)
        out["chain_frac_fp4_peak"] = round(out["tflops"] / MFMA_PEAK_TFLOPS["fp4"], 4)
    if not args.no_cpu:
        out["cpu_baseline"] = wl.cpu_baseline(args.cpu_budget)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
