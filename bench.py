#!/usr/bin/env python3
"""Benchmark: Q4_0 matvec throughput at 11008x4096 on one MI355X.

One step = one y = W x over a resident 11008x4096 GGUF Q4_0 matrix (the
reference's asm_matmul_q4 contract, src/kernels/x86_64/matmul_q4_avx2.asm:57,
with the weights read in their 18-byte block layout).  Each step reads a
different copy of the weights: 32 copies (813 MB) rotate, more than three
times the 256 MB MALL, so HBM and not the last-level cache serves them.

`value` is whole-job throughput: algorithmic bytes (M*(K/32)*18 + 4K + 4M per
step) over the GPU time of exactly K steps replayed from captured HIP graphs,
bracketed by HIP events and device synchronizations.  `roofline.achieved` uses
the matvec kernel's average duration over that timed region (the graphs hold
nothing else), which the rocprofv3 kernel trace of the same command matches;
`roofline.traffic` comes from two rocprofv3 counter passes (FETCH_SIZE,
WRITE_SIZE) scaled by a calibration kernel of known traffic.  The CPU baseline times the oracle's restatement of the
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

    def timed(n_steps: int) -> tuple[float, float]:
        """GPU ms and wall s of exactly `n_steps` launches: graphs over all
        copies plus one graph for the remainder, bracketed by HIP events on
        the launch stream and device synchronizations."""
        graph = Graph.capture(stream, lambda: [launch(i) for i in range(copies)])
        rem = n_steps % copies
        graph_rem = Graph.capture(stream, lambda: [launch(i) for i in range(rem)]) if rem else None
        for _ in range(max(1, -(-warmup // copies))):
            graph.launch(stream)
        synchronize()
        e0, e1 = Event(), Event()
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(n_steps // copies):
            graph.launch(stream)
        if graph_rem:
            graph_rem.launch(stream)
        e1.record(stream)
        e1.synchronize()
        synchronize()
        wall = time.perf_counter() - t0
        ms = e0.elapsed_ms(e1)
        graph.close()
        if graph_rem:
            graph_rem.close()
        return ms, wall

    total_ms, wall_s = timed(steps)
    bytes_step = q4_algorithmic_bytes(M, K)
    selected = lib.asmhip_get_q4_kernel()
    # the fp32 VALU kernel on the same copies, for reference
    native.check(lib.asmhip_set_q4_kernel(native.Q4_KERNEL_FP32), "asmhip_set_q4_kernel")
    n_ref = min(steps, 1024)
    fp32_ms, _ = timed(n_ref)
    native.check(lib.asmhip_set_q4_kernel(selected), "asmhip_set_q4_kernel")

    return {
        "value": bytes_step * steps / (total_ms / 1e3) / 1e9,
        "ms_per_step": total_ms / steps,
        "steps": steps,
        "wall_s": wall_s,
        "kernel_us_mean": total_ms * 1e3 / steps,
        "fp32_kernel_us_mean": fp32_ms * 1e3 / n_ref,
        "bytes_per_step": bytes_step,
        "parity_max_err_over_l1": worst,
    }


def bench_cpu_baseline(seconds: float, copies: int = 4) -> dict:
    """The oracle's restatement of asm_matmul_q4 (AVX2) + threadpool tiling on
    the host cores.  `copies` split-layout copies of the weights rotate
    (4 x 27 MB), more than the host's last-level cache, so DRAM serves them
    as HBM serves the GPU."""
    from asmllm_amd import gguf
    from oracle import native as oracle

    M, K = M_MAIN, K_MAIN
    blocks, x = make_q4_problem(M, K)
    qs, sc = gguf.split_q4_0(blocks)  # generate.py:91-99: the reference kernel's split layout
    qs_c = [qs] + [qs.copy() for _ in range(copies - 1)]
    sc_c = [sc] + [sc.copy() for _ in range(copies - 1)]
    cores = host_cores()
    out = {}
    for nt in (cores, 1):
        for i in range(3):
            oracle.matmul_q4_mt(qs_c[i % copies], sc_c[i % copies], x, nt, 0)
        times = []
        t_end = time.perf_counter() + seconds / 2
        i = 0
        while time.perf_counter() < t_end or len(times) < 10:
            t0 = time.perf_counter()
            oracle.matmul_q4_mt(qs_c[i % copies], sc_c[i % copies], x, nt, 0)
            times.append(time.perf_counter() - t0)
            i += 1
        med = float(np.median(times))
        out[nt] = (q4_algorithmic_bytes(M, K) / med / 1e9, len(times), med)
    oracle.threadpool_shutdown()
    gbps, calls, med = out[cores]
    return {
        "value": round(gbps, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"Q4_0 {M}x{K} matvec, split layout (qs + fp32 scales widened from fp16), oracle restatement "
                   f"of asm_matmul_q4 AVX2 + threadpool tiling over {copies} rotating weight copies, "
                   f"{calls} calls in ~{seconds / 2:.0f} s, median {med * 1e3:.3f} ms per call"),
        "single_thread_value": round(out[1][0], 3),
        "avx512_host": bool(oracle.has_avx512()),
    }


def profile_pass(copies: int, launches: int = 64) -> None:
    """A short fixed workload for hardware-counter runs: `launches` matvecs
    over rotating weight copies, then the calibration kernel (exact Q4_0
    dequantization of a 1024x4096 matrix: 2,359,296 bytes read, 16,777,216
    bytes written per launch) whose counter readings scale the matvec's."""
    from asmllm_amd import native
    from asmllm_amd.device import DeviceBuffer, Stream

    lib = native.lib()
    M, K = M_MAIN, K_MAIN
    blocks, x = make_q4_problem(M, K)
    bufs = [DeviceBuffer.from_numpy(blocks)]
    for _ in range(copies - 1):
        b = DeviceBuffer(blocks.nbytes)
        b.copy_from(bufs[0])
        bufs.append(b)
    dx, dy = DeviceBuffer.from_numpy(x), DeviceBuffer(M * 4)
    cal_rows = CAL_ROWS
    dcal = DeviceBuffer(cal_rows * K * 4)
    stream = Stream()
    for i in range(launches):
        native.check(lib.asmhip_matmul_q4_0(bufs[i % copies].ptr, dx.ptr, dy.ptr, M, K, stream.handle), "matvec")
    for i in range(8):
        native.check(lib.asmhip_dequantize_q4_0(bufs[i].ptr, dcal.ptr, cal_rows, K, stream.handle), "dequantize")
    stream.synchronize()
    log(f"profile pass: {launches} matvec launches ({M}x{K}), 8 calibration dequantize launches ({cal_rows}x{K})")


CAL_ROWS = 1024  # calibration dequantize: CAL_ROWS x K_MAIN Q4_0 -> fp32
CAL_READ_BYTES = CAL_ROWS * (K_MAIN // 32) * 18
CAL_WRITE_BYTES = CAL_ROWS * K_MAIN * 4


def measure_traffic(timeout_s: int = 150) -> dict | None:
    """HBM bytes per matvec launch from two rocprofv3 counter passes
    (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch) over `--profile-pass`, each
    scaled by what the same counter reads for the calibration dequantize
    (CAL_READ_BYTES read, CAL_WRITE_BYTES written per launch).  Runs rocprofv3
    as a child process; returns None when it is unavailable or fails."""
    import csv
    import shutil
    import subprocess
    import tempfile

    exe = shutil.which("rocprofv3")
    if exe is None:
        log("rocprofv3 not found: traffic not measured")
        return None
    out: dict = {}
    env = dict(os.environ, TMPDIR="/tmp")
    with tempfile.TemporaryDirectory(dir="/tmp") as tmp:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            cmd = [exe, "--pmc", counter, "--output-format", "csv", "-d", tmp, "-o", counter, "--",
                   sys.executable, str(ROOT / "bench.py"), "--profile-pass"]
            try:
                subprocess.run(cmd, cwd="/tmp", env=env, timeout=timeout_s, check=True,
                               stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
            except (subprocess.SubprocessError, OSError) as e:
                log(f"rocprofv3 --pmc {counter} failed ({e}): traffic not measured")
                return None
            files = list(Path(tmp).rglob(f"{counter}_counter_collection.csv"))
            if not files:
                log(f"rocprofv3 --pmc {counter} wrote no counter file: traffic not measured")
                return None
            vals: dict[str, list[float]] = {"matvec": [], "cal": []}
            with open(files[0]) as f:
                for row in csv.DictReader(f):
                    if row.get("Counter_Name") != counter:
                        continue
                    name = row["Kernel_Name"]
                    if "q4_0_mfma" in name or "q4_matvec" in name:
                        vals["matvec"].append(float(row["Counter_Value"]))
                    elif "dequant_kernel" in name:
                        vals["cal"].append(float(row["Counter_Value"]))
            if not vals["matvec"] or not vals["cal"]:
                log(f"rocprofv3 --pmc {counter}: kernels not found in the counter file")
                return None
            out[counter] = (float(np.mean(vals["matvec"])), float(np.mean(vals["cal"])))
    fetch_kib, cal_fetch_kib = out["FETCH_SIZE"]
    write_kib, cal_write_kib = out["WRITE_SIZE"]
    read_scale = CAL_READ_BYTES / (cal_fetch_kib * 1024)
    write_scale = CAL_WRITE_BYTES / (cal_write_kib * 1024)
    return {
        "bytes": fetch_kib * 1024 * read_scale + write_kib * 1024 * write_scale,
        "fetch_kib_raw": fetch_kib,
        "write_kib_raw": write_kib,
        "fetch_scale": read_scale,
        "write_scale": write_scale,
    }


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4096)
    ap.add_argument("--warmup", type=int, default=256)
    ap.add_argument("--copies", type=int, default=32)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--profile-pass", action="store_true",
                    help="run only a short fixed workload for hardware-counter collection")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 counter passes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this build has no multi-GPU path)",
              file=sys.stderr)
        raise SystemExit(2)

    if args.profile_pass:
        profile_pass(args.copies)
        return

    from asmllm_amd.device import device_info

    info = device_info()
    log(f"device {info['arch']} with {info['compute_units']} CUs")
    mv = bench_matvec(args.steps, args.warmup, args.copies)
    achieved = mv["bytes_per_step"] / (mv["kernel_us_mean"] * 1e-6) / 1e9
    cpu = None if args.no_cpu else bench_cpu_baseline(args.cpu_seconds)
    traffic = None if args.no_traffic else measure_traffic()

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
            "traffic": round(traffic["bytes"]) if traffic else None,
            "traffic_detail": traffic,
            "kernel": "q4_0_mfma_stream (int8 MFMA, GGUF Q4_0)",
            "kernel_us_mean": round(mv["kernel_us_mean"], 3),
            "fp32_valu_kernel_us_mean": round(mv["fp32_kernel_us_mean"], 3),
            "bytes_per_launch": mv["bytes_per_step"],
        },
        "cpu_baseline": cpu,
        "parity_max_err_over_l1": mv["parity_max_err_over_l1"],
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
