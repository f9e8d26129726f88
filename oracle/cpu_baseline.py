"""Timed CPU baseline of the quantized matmul path (oracle; test infrastructure only).

The same algorithm as ``oracle.formats`` + ``oracle.ref`` -- exact dequantization of the GGUF blocks to float32,
then a float32 matmul -- run the way a CPU implementation would: the weight rows are split into chunks that are
dequantized into a reused buffer and multiplied right away, and the chunks are spread over a thread pool (numpy
releases the GIL inside its kernels). Only ``bench.py``'s ``cpu_baseline`` leg calls this module.
"""
import concurrent.futures
import os
import time

import numpy as np

from . import formats


def cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def gemv(fmt, raw, n, k, x, threads=None, chunk_rows=256):
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

    with concurrent.futures.ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(work, range(0, n, chunk_rows)))
    return y


def time_gemv(fmt, raw, n, k, x, budget_s=12.0, min_runs=2, threads=None):
    """Runs gemv repeatedly for about budget_s seconds (at least min_runs, one warm-up first); returns
    (median seconds per call, runs, threads)."""
    threads = threads or cores()
    gemv(fmt, raw, n, k, x, threads)
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        gemv(fmt, raw, n, k, x, threads)
        times.append(time.perf_counter() - t0)
        if len(times) >= 50:
            break
    return float(np.median(times)), len(times), threads
