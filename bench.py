#!/usr/bin/env python3
"""Benchmark: Q4_0 matvec throughput at 11008x4096 on one MI355X.

One step = one y = W x over a resident 11008x4096 GGUF Q4_0 matrix (the
reference's asm_matmul_q4 contract, src/kernels/x86_64/matmul_q4_avx2.asm:57,
with the weights read in their 18-byte block layout).  Each step reads a
different copy of the weights: 32 copies (813 MB) rotate, more than three
times the 256 MB MALL, so HBM and not the last-level cache serves them.

`value` is whole-job throughput: algorithmic bytes (M*(K/32)*18 + 4K + 4M per
step) over the wall time of K steps replayed from a captured HIP graph,
bracketed by device synchronizations.  `roofline.achieved` uses the matvec
kernel's average duration measured with HIP events around single launches on
the launch stream.  The CPU baseline times the oracle's restatement of the
reference's AVX2 kernel and threadpool on the host cores on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "Q4_0 matvec GB/s (% HBM peak) at 11008x4096; decode tokens/sec"
HBM_PEAK_GBPS = 8000.0
M_MAIN, K_MAIN = 11008, 4096


def q4_algorithmic_bytes(M: int, K: int) -> int:
    return M * (K // 32) * 18 + 4 * K + 4 * M


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_cores() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def make_q4_problem(M: int, K: int, seed: int = 42):
    from asmllm_amd import gguf

    rng = np.random.default_rng(seed)
    w = rng.standard_normal((M, K), dtype=np.float32) * np.float32(0.02)
    x = rng.standard_normal(K, dtype=np.float32)
    return gguf.quantize_q4_0(w), x


def bench_matvec(steps: int, warmup: int, copies: int) -> dict:
    from asmllm_amd import native
    from asmllm_amd.device import DeviceBuffer, Event, Graph, Stream, synchronize
    from oracle import native as oracle

    lib = native.lib()
    M, K = M_MAIN, K_MAIN
    blocks, x = make_q4_problem(M, K)
    nbytes = blocks.nbytes
    log(f"uploading {copies} copies of the {M}x{K} Q4_0 matrix ({copies * nbytes / 1e6:.0f} MB)")
    bufs = [DeviceBuffer.from_numpy(blocks)]
    for _ in range(copies - 1):
        b = DeviceBuffer(nbytes)
        b.copy_from(bufs[0])
        bufs.append(b)
    dx, dy = DeviceBuffer.from_numpy(x), DeviceBuffer(M * 4)
    stream = Stream()

    def launch(i: int) -> None:
        rc = lib.asmhip_matmul_q4_0(bufs[i % copies].ptr, dx.ptr, dy.ptr, M, K, stream.handle)
        if rc:
            native.check(rc, "asmhip_matmul_q4_0")

    # correctness gate on the first and last copy
    y_ref = oracle.matmul_q4_0_gguf(blocks, x, host_cores())
    l1 = np.abs(oracle.dequantize_q4_0(blocks).astype(np.float64)) @ np.abs(x.astype(np.float64))
    worst = 0.0
    for i in (0, copies - 1):
        launch(i)
        stream.synchronize()
        y = dy.download(np.float32, M)
        worst = max(worst, float(np.max(np.abs(y.astype(np.float64) - y_ref) / l1)))
    if worst > 1e-4:
        raise SystemExit(f"matvec parity failed: max err / row L1 = {worst:.3e}")
    log(f"parity ok (max err / row L1 {worst:.2e})")

    # one graph replays one pass over all copies
    graph = Graph.capture(stream, lambda: [launch(i) for i in range(copies)])
    reps_warm = max(1, warmup // copies)
    reps = max(1, steps // copies)
    for _ in range(reps_warm):
        graph.launch(stream)
    synchronize()
    e0, e1 = Event(), Event()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(reps):
        graph.launch(stream)
    e1.record(stream)
    e1.synchronize()
    synchronize()
    wall_s = time.perf_counter() - t0
    total_ms = e0.elapsed_ms(e1)
    n_steps = reps * copies
    bytes_step = q4_algorithmic_bytes(M, K)

    # per-launch kernel duration (events around single launches on the launch stream)
    n_single = 256
    evs = [(Event(), Event()) for _ in range(n_single)]
    for i, (a, b) in enumerate(evs):
        a.record(stream)
        launch(i)
        b.record(stream)
    stream.synchronize()
    durs = np.array([a.elapsed_ms(b) for a, b in evs]) * 1e3  # us
    kernel_us = float(np.mean(durs))

    value = bytes_step * n_steps / (total_ms / 1e3) / 1e9
    return {
        "value": value,
        "ms_per_step": total_ms / n_steps,
        "steps": n_steps,
        "wall_s": wall_s,
        "kernel_us_mean": kernel_us,
        "kernel_us_median": float(np.median(durs)),
        "kernel_us_min": float(np.min(durs)),
        "bytes_per_step": bytes_step,
        "parity_max_err_over_l1": worst,
    }


def bench_cpu_baseline(seconds: float) -> dict:
    from asmllm_amd import gguf
    from oracle import native as oracle

    M, K = M_MAIN, K_MAIN
    blocks, x = make_q4_problem(M, K)
    qs, sc = gguf.split_q4_0(blocks)  # generate.py:91-99: the reference kernel's split layout
    cores = host_cores()
    out = {}
    for nt in (cores, 1):
        for _ in range(3):
            oracle.matmul_q4_mt(qs, sc, x, nt, 0)
        times = []
        t_end = time.perf_counter() + seconds / 2
        while time.perf_counter() < t_end or len(times) < 10:
            t0 = time.perf_counter()
            oracle.matmul_q4_mt(qs, sc, x, nt, 0)
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        out[nt] = (q4_algorithmic_bytes(M, K) / med / 1e9, len(times), med)
    oracle.threadpool_shutdown()
    gbps, calls, med = out[cores]
    return {
        "value": gbps,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"Q4_0 {M}x{K} matvec, split layout (qs + fp32 scales widened from fp16), oracle restatement "
                   f"of asm_matmul_q4 AVX2 + threadpool tiling, {calls} calls, median {med * 1e3:.3f} ms"),
        "single_thread_value": out[1][0],
        "avx512_host": bool(oracle.has_avx512()),
    }


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4096)
    ap.add_argument("--warmup", type=int, default=256)
    ap.add_argument("--copies", type=int, default=32)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this build has no multi-GPU path)",
              file=sys.stderr)
        raise SystemExit(2)

    from asmllm_amd.device import device_info

    info = device_info()
    log(f"device {info['arch']} with {info['compute_units']} CUs")
    mv = bench_matvec(args.steps, args.warmup, args.copies)
    achieved = mv["bytes_per_step"] / (mv["kernel_us_mean"] * 1e-6) / 1e9
    cpu = None if args.no_cpu else bench_cpu_baseline(args.cpu_seconds)

    result = {
        "metric": METRIC,
        "value": round(mv["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": mv["steps"],
        "warmup": args.warmup,
        "ms_per_step": mv["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: W ~ N(0, 0.02) quantized to GGUF Q4_0, x ~ N(0, 1), numpy default_rng(42)",
        "config": {
            "workload": f"Q4_0 matvec y = W x, W {M_MAIN}x{K_MAIN} GGUF Q4_0 blocks resident in HBM, x/y fp32, batch 1",
            "weight_copies": args.copies,
            "weight_bytes_rotated": args.copies * M_MAIN * (K_MAIN // 32) * 18,
            "device": info["arch"],
        },
        "pct_hbm_peak": round(100.0 * mv["value"] / HBM_PEAK_GBPS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": None,
            "kernel": "q4_matvec_pairs (GGUF)",
            "kernel_us_mean": round(mv["kernel_us_mean"], 3),
            "kernel_us_median": round(mv["kernel_us_median"], 3),
            "bytes_per_launch": mv["bytes_per_step"],
        },
        "cpu_baseline": cpu,
        "parity_max_err_over_l1": mv["parity_max_err_over_l1"],
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
