"""Timed CPU baseline of the quantized matmul path (oracle; test infrastructure only).

The same algorithm as ``oracle.formats`` + ``oracle.ref`` -- exact dequantization of the GGUF blocks to float32,
then float32 matmuls -- run the way a CPU implementation would, on every core of the host:

* GEMV / GEMM: the weight rows are split into 256-row chunks that are dequantized into a buffer and multiplied right
  away (the fused figure), spread over a thread pool (numpy releases the GIL inside its kernels); the dequantization
  alone (every chunk into one f32 matrix) and the matmul alone (on that matrix, BLAS threads = cores) are timed too.
* MoE: top-k routing, then per hit expert the dequantization of its gate / up / down rows (one task per expert on the
  thread pool) and its two matmuls over the tokens routed to it (BLAS single-threaded inside each task, the experts
  in parallel), then the weighted combine. The dequant phase and the matmul phase are timed separately.

Only ``bench.py``'s ``cpu_baseline`` leg calls this module. Every figure is the median of repeated runs after a
warm-up, bounded by a time budget.
"""
import concurrent.futures
import os
import time

import numpy as np

from . import formats
from . import ref


def cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def _blas_limit(n):
    """A context that caps the BLAS thread count at n (threadpoolctl when importable, else nothing)."""
    try:
        from threadpoolctl import threadpool_limits
        return threadpool_limits(limits=n, user_api="blas")
    except ImportError:   # pragma: no cover - threadpoolctl ships with the image
        import contextlib
        return contextlib.nullcontext()


def _median_runs(fn, budget_s, min_runs=5, max_runs=50):
    """fn() once as a warm-up, then at least min_runs times and on for about budget_s seconds; (median seconds,
    runs)."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or (time.perf_counter() < t_end and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def gemv(fmt, raw, n, k, x, threads=None, chunk_rows=256, pool=None):
    """y [t, n] = x [t, k] W^T with W dequantized chunk by chunk (float32 accumulate, numpy matmul)."""
    threads = threads or cores()
    rb = formats.row_bytes(fmt, k)
    raw = np.ascontiguousarray(np.asarray(raw).view(np.uint8).reshape(-1))
    x = np.asarray(x, np.float32)
    y = np.empty((x.shape[0], n), np.float32)

    def work(r0):
        r1 = min(n, r0 + chunk_rows)
        w = formats.dequantize(fmt, raw[r0 * rb:r1 * rb], r1 - r0, k)
        y[:, r0:r1] = x @ w.T

    if pool is not None:
        list(pool.map(work, range(0, n, chunk_rows)))
        return y
    with concurrent.futures.ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(work, range(0, n, chunk_rows)))
    return y


def dequant_all(fmt, raw, n, k, pool, out=None, chunk_rows=256):
    """f32 W [n, k] of the whole matrix, chunks dequantized on the pool."""
    rb = formats.row_bytes(fmt, k)
    raw = np.ascontiguousarray(np.asarray(raw).view(np.uint8).reshape(-1))
    out = np.empty((n, k), np.float32) if out is None else out

    def work(r0):
        r1 = min(n, r0 + chunk_rows)
        out[r0:r1] = formats.dequantize(fmt, raw[r0 * rb:r1 * rb], r1 - r0, k)

    list(pool.map(work, range(0, n, chunk_rows)))
    return out


def time_gemv(fmt, raw, n, k, x, budget_s=12.0, threads=None):
    """The GEMV / GEMM y = x W^T on the CPU, timed three ways. Returns a dict: total_s (dequant fused with the
    matmul chunk by chunk, median), dequant_s (the whole matrix to f32), matmul_s (x W^T on the f32 matrix), runs and
    threads."""
    threads = threads or cores()
    x = np.asarray(x, np.float32)
    with concurrent.futures.ThreadPoolExecutor(max_workers=threads) as pool, _blas_limit(1):
        total_s, runs = _median_runs(lambda: gemv(fmt, raw, n, k, x, pool=pool), budget_s * 0.5)
        W = np.empty((n, k), np.float32)
        dequant_s, _ = _median_runs(lambda: dequant_all(fmt, raw, n, k, pool, out=W), budget_s * 0.25)
    with _blas_limit(threads):
        matmul_s, _ = _median_runs(lambda: x @ W.T, budget_s * 0.25)
    return {"total_s": total_s, "dequant_s": dequant_s, "matmul_s": matmul_s, "runs": runs, "threads": threads}


def moe_chain(x, logits, KU, gating, norm, act, experts_fn, pool, x_round=None, act_round=None, dequantized=None):
    """The routed-expert chain on the CPU in float32: route, per-expert gate/up, activation, down, combine.
    experts_fn(e) -> (Wg [FE, H], Wu [FE, H], Wd [H, FE]) f32 (dequantized here unless `dequantized` holds them).
    Returns (y [T, H], seconds in the dequant phase, seconds in the matmul phase)."""
    t0 = time.perf_counter()
    ids, wts = ref.route(logits, KU, gating, norm)
    hit = [int(e) for e in np.unique(ids)]
    W = dequantized if dequantized is not None else dict(zip(hit, pool.map(experts_fn, hit)))
    t1 = time.perf_counter()
    xr = np.asarray(x if x_round is None else x_round(x), np.float32)
    fn = ref.ACTIVATIONS[act]

    def expert(e):
        tok, slot = np.nonzero(ids == e)
        Wg, Wu, Wd = W[e]
        with _blas_limit(1):
            a = fn(xr[tok] @ Wg.T, xr[tok] @ Wu.T).astype(np.float32)
            if act_round is not None:
                a = np.asarray(act_round(a), np.float32)
            return tok, slot, a @ Wd.T

    y = np.zeros((x.shape[0], W[hit[0]][2].shape[0]), np.float32)
    for tok, slot, out in pool.map(expert, hit):
        np.add.at(y, tok, wts[tok, slot][:, None].astype(np.float32) * out)
    return y, t1 - t0, time.perf_counter() - t1


def time_moe(x, logits, KU, gating, norm, act, experts_fn, budget_s=12.0, threads=None, x_round=None,
             act_round=None):
    """The MoE chain timed on all cores: a dict of total_s (route + dequant + matmuls + combine, median), dequant_s
    (the hit experts' weights to f32), matmul_s (route + matmuls + combine on dequantized weights), runs and
    threads."""
    threads = threads or cores()
    with concurrent.futures.ThreadPoolExecutor(max_workers=threads) as pool:
        ids, _ = ref.route(logits, KU, gating, norm)
        hit = [int(e) for e in np.unique(ids)]
        total_s, runs = _median_runs(
            lambda: moe_chain(x, logits, KU, gating, norm, act, experts_fn, pool, x_round, act_round),
            budget_s * 0.5, max_runs=20)
        W = dict(zip(hit, pool.map(experts_fn, hit)))
        dequant_s, _ = _median_runs(lambda: list(pool.map(experts_fn, hit)), budget_s * 0.25, max_runs=20)
        matmul_s, _ = _median_runs(
            lambda: moe_chain(x, logits, KU, gating, norm, act, experts_fn, pool, x_round, act_round, dequantized=W),
            budget_s * 0.25, max_runs=20)
    return {"total_s": total_s, "dequant_s": dequant_s, "matmul_s": matmul_s, "runs": runs, "threads": threads,
            "experts_hit": len(hit)}
