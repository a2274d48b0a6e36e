#!/usr/bin/env python3
"""Benchmark: Q4_0 matvec throughput at 11008x4096 on one MI355X.

One step = one y = W x over a resident 11008x4096 GGUF Q4_0 matrix (the
reference's asm_matmul_q4 contract, src/kernels/x86_64/matmul_q4_avx2.asm:57,
with the weights read in their 18-byte block layout).  Each step reads a
different copy of the weights: 32 copies (813 MB) rotate, more than three
times the 256 MB MALL, so HBM and not the last-level cache serves them.

`value` is whole-job throughput: algorithmic bytes (M*(K/32)*18 + 4K + 4M per
step) over the GPU time of exactly K steps (stream launches, or replays of
captured HIP graphs past 512 steps), bracketed by HIP events and device
synchronizations.  `roofline.achieved` uses the matvec kernel's average duration
over that timed region (it holds nothing else) less what the two events add to
the region on their own (timed with nothing between them); the rocprofv3 kernel
trace of the same timed launches (`roofline.kernel_trace`) agrees with it;
`roofline.traffic` comes from two rocprofv3 counter passes (the L2's memory read
and write requests by size).  The CPU baseline times the oracle's restatements of
the reference's AVX2 and AVX-512 kernels with its threadpool tiling on the host
cores, swept over thread counts, on a bounded sample.
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
    """Threads for the CPU legs: the cores this process may run on, capped by the
    reference's MAX_WORKERS (64, threadpool.c:99) and by OMP_NUM_THREADS where the
    host sets it (a shared GPU host allots each GPU its share of the cores)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    share = os.environ.get("OMP_NUM_THREADS", "")
    if share.isdigit() and int(share) > 0:
        n = min(n, int(share))
    return max(1, min(64, n))


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def l3_bytes() -> int:
    """Last-level cache the process can fill: the sizes of the distinct L3 instances
    (sysfs shared_cpu_list) of the cores it may run on, summed (an EPYC's L3 is per
    CCD, and the allowed cores can span several); 0 if unknown."""
    try:
        cpus = sorted(os.sched_getaffinity(0))
    except AttributeError:
        cpus = list(range(os.cpu_count() or 1))
    seen: dict[str, int] = {}
    for cpu in cpus:
        for idx in Path(f"/sys/devices/system/cpu/cpu{cpu}/cache").glob("index*"):
            try:
                if (idx / "level").read_text().strip() != "3":
                    continue
                shared = (idx / "shared_cpu_list").read_text().strip()
                txt = (idx / "size").read_text().strip().upper()
                mult = {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}.get(txt[-1], 1)
                seen[shared] = int(txt.rstrip("KMG")) * mult
            except (OSError, ValueError):
                continue
    return sum(seen.values())


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
    cov, sink = DeviceBuffer(1 << 30), DeviceBuffer(4096)  # untimed cover reads (see timed)
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
        """GPU ms and wall s of exactly `n_steps` launches between two HIP
        events on the launch stream, with device synchronizations before the
        last untimed round and after the timed steps.

        A HIP graph launch costs ~7 us before its first kernel starts, also when
        it is queued behind running work (measured: 640 steps as 20 graphs of 32
        launches 7.06 us a step, as one graph 6.79), so the timed region keeps
        graph boundaries out or few: up to 512 steps are plain stream launches,
        enqueued while the GPU still runs untimed single-launch reads
        (asmhip_stream_read, one host call each) long enough (~40 us of host
        time per launch) that all K launches are queued before the start event
        fires (after one untimed pass of the same launches: the first such pass
        runs slower); more steps are graphs of 512 launches (one
        boundary per 512 steps, ~0.01 us a step; one graph serves every full
        block of 512, cycling over the copies), each graph launched once
        untimed first (a graph's first launch also sets it up).  The
        events are timing-only (hipEventDisableSystemFence, HIP's flag for
        events that only measure time: no system-scope cache writeback and
        invalidate at record)."""
        e0, e1 = Event(timing=True), Event(timing=True)
        warm = Graph.capture(stream, lambda: [launch(i) for i in range(copies)])

        def cover() -> None:
            # untimed single-launch reads (~160 us per GiB) that keep the GPU busy
            # while the host enqueues the timed launches (~40 us of host time
            # each), at least 400 (~64 ms): the GPU reaches its steady speed only
            # after tens of ms of load (20 steps behind 3 / 16 / 64 ms of reads:
            # 6.95 / 6.80 / 6.74 us a step, the last as in 4096-step runs)
            for _ in range(max(400, 1 + -(-n_steps * 40 // 150))):
                native.check(lib.asmhip_stream_read(cov.ptr, cov.nbytes, sink.ptr, stream.handle), "cover read")

        big = []  # graphs of the timed region, in order
        if n_steps > 512:
            full = Graph.capture(stream, lambda: [launch(i % copies) for i in range(512)])
            big = [full] * (n_steps // 512)
            rem = n_steps % 512
            if rem:
                big.append(Graph.capture(stream, lambda: [launch((n_steps - rem + i) % copies) for i in range(rem)]))
        for _ in range(max(1, -(-warmup // copies))):
            warm.launch(stream)
        for g in dict.fromkeys(big):  # each graph once
            g.launch(stream)
        synchronize()
        if not big:  # one untimed pass of the same stream launches (first passes run slower)
            cover()
            for i in range(n_steps):
                launch(i % copies)
            synchronize()
        t0 = time.perf_counter()
        if big:
            warm.launch(stream)
        else:
            cover()
        e0.record(stream)
        if big:
            for g in big:
                g.launch(stream)
        else:
            for i in range(n_steps):
                launch(i % copies)
        e1.record(stream)
        e1.synchronize()
        synchronize()
        wall = time.perf_counter() - t0
        ms = e0.elapsed_ms(e1)
        warm.close()
        for g in dict.fromkeys(big):
            g.close()
        return ms, wall

    # the same bracketing with no launch between the events: what recording the two
    # events adds to the region (~3-4 us: a few percent of 20 steps, nothing at 4096);
    # taken first, so that the timed launches are the last headline dispatches of a
    # run (the kernel-trace leg reads them from the end of the trace)
    bracket_ms = min(timed(0)[0] for _ in range(3))
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
        # per-launch time of the matvec over the timed region without the events'
        # own bracketing cost (roofline.achieved); `value` keeps the whole region
        "kernel_us_mean": max(total_ms - bracket_ms, 0.5 * total_ms) * 1e3 / steps,
        "event_bracket_us": bracket_ms * 1e3,
        "fp32_kernel_us_mean": fp32_ms * 1e3 / n_ref,
        "bytes_per_step": bytes_step,
        "parity_max_err_over_l1": worst,
    }


def bench_cpu_baseline(seconds: float) -> dict:
    """The oracle's restatements of asm_matmul_q4 (AVX2, matmul_q4_avx2.asm; and the
    AVX-512 variant where the host has it) with the threadpool's row tiling
    (threadpool.c:390-486) on the host cores, swept over 1, 2, 4, ... threads as
    bench/harness/bench_mt_throughput.py:49-112 does: 5 warmups, then timed calls for
    a bounded time (at least 10), median and interquartile range.  Distinct weight
    copies in the split layout rotate, at least twice the host's L3 in total, so
    DRAM and not the cache serves them, as HBM serves the GPU."""
    from asmllm_amd import gguf
    from oracle import native as oracle

    M, K = M_MAIN, K_MAIN
    blocks, x = make_q4_problem(M, K)
    qs, sc = gguf.split_q4_0(blocks)  # generate.py:91-99: the reference kernel's split layout
    per_copy = qs.nbytes + sc.nbytes
    l3 = l3_bytes()
    copies = int(min(64, max(4, -(-2 * l3 // per_copy) if l3 else 16)))
    qs_c = [qs] + [qs.copy() for _ in range(copies - 1)]
    sc_c = [sc] + [sc.copy() for _ in range(copies - 1)]
    cores = host_cores()
    threads = sorted({1 << i for i in range(7) if (1 << i) <= cores} | {cores})
    kinds = [("avx2", 0)] + ([("avx512", 1)] if oracle.has_avx512() else [])
    per_point = seconds / (len(threads) * len(kinds))
    nbytes = q4_algorithmic_bytes(M, K)
    sweep = []
    for kind, variant in kinds:
        for nt in threads:
            for i in range(5):
                oracle.matmul_q4_mt(qs_c[i % copies], sc_c[i % copies], x, nt, variant)
            times = []
            t_end = time.perf_counter() + per_point
            i = 0
            while time.perf_counter() < t_end or len(times) < 10:
                t0 = time.perf_counter()
                oracle.matmul_q4_mt(qs_c[i % copies], sc_c[i % copies], x, nt, variant)
                times.append(time.perf_counter() - t0)
                i += 1
            med = float(np.median(times))
            q1, q3 = (float(v) for v in np.percentile(times, [25, 75]))
            sweep.append({"kernel": kind, "threads": nt, "calls": len(times), "median_ms": round(med * 1e3, 4),
                          "iqr_ms": [round(q1 * 1e3, 4), round(q3 * 1e3, 4)],
                          "GBps": round(nbytes / med / 1e9, 3)})
            log(f"cpu {kind} {nt} threads: {med * 1e3:.3f} ms, {nbytes / med / 1e9:.1f} GB/s")
    oracle.threadpool_shutdown()
    best = max(sweep, key=lambda p: p["GBps"])  # the fastest configuration of the sweep is the baseline
    return {
        "value": best["GBps"],
        "unit": "GB/s",
        "cores": best["threads"],
        "kind": "port",
        "sample": (f"Q4_0 {M}x{K} matvec, split layout (qs + fp32 scales widened from fp16): the oracle's op-for-op "
                   f"restatement of asm_matmul_{'q4_avx512' if best['kernel'] == 'avx512' else 'q4'} with the "
                   f"threadpool's row tiling, fastest of the sweep over 1..{cores} threads ({best['threads']}), "
                   f"{copies} rotating weight copies ({copies * per_copy / 1e6:.0f} MB, L3 {l3 / 1e6:.0f} MB), "
                   f"median of {best['calls']} calls ({best['median_ms']} ms)"),
        "host_cores": cores,
        "cpu_model": cpu_model(),
        "l3_bytes": l3,
        "weight_copies": copies,
        "avx512_host": bool(oracle.has_avx512()),
        "sweep": sweep,
    }


def _cpu_time(call, copies: int, seconds: float) -> tuple[float, int]:
    """Median seconds of `call(i)` cycling over `copies` operand sets: 5 warm-ups,
    then timed calls for `seconds` (at least 10), as bench_mt_throughput.py:82-96."""
    for i in range(5):
        call(i % copies)
    times = []
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end or len(times) < 10:
        t0 = time.perf_counter()
        call(i % copies)
        times.append(time.perf_counter() - t0)
        i += 1
    return float(np.median(times)), len(times)


def cpu_table_baselines(rows: list[dict], threads: int, variant: int, seconds: float = 0.5) -> dict:
    """A CPU baseline beside every row of the matvec table: the oracle's op-for-op
    restatement of the reference kernel for the row's format (asm_matmul_q4 AVX2 or
    AVX-512 (`variant`), asm_matmul_q8, asm_matmul_q5 on their split planes, with the
    threadpool's row tiling, threadpool.c:390-486, 588-665, 667-787) at the shape of
    the row, on `threads` host threads (the headline sweep's fastest), operands rotating
    over at least twice the host's L3.  GB/s uses the row's own algorithmic bytes, so
    the GPU and CPU figures of a row compare the same work.  The Llama-3 layer rows
    get the sum of their matvecs.  Annotates `rows` in place; returns the settings."""
    from oracle import native as oracle

    l3 = l3_bytes()
    fmt_of = {name: (qt, M, K) for name, qt, M, K in MATVEC_TABLE}
    cache: dict[tuple, float] = {}

    def time_shape(qt: str, M: int, K: int) -> float:
        fam = {"q4": "q4", "q4s": "q4", "q8": "q8", "q8s": "q8", "q5": "q5", "q5s": "q5"}[qt]
        key = (fam, M, K)
        if key in cache:
            return cache[key]
        # random planes of the format (the kernels' time does not depend on the values)
        rng = np.random.default_rng(M * 7 + K)
        nb = K // 32
        x = rng.standard_normal(K, dtype=np.float32)
        sc = rng.uniform(1e-3, 2e-3, (M, nb)).astype(np.float32)
        if fam == "q4":
            planes = (rng.integers(0, 256, (M, nb, 16), dtype=np.uint8), sc)
            fn = lambda pl: oracle.matmul_q4_mt(pl[0], pl[1], x, threads, variant)  # noqa: E731
        elif fam == "q8":
            planes = (rng.integers(-127, 128, (M, nb, 32), dtype=np.int8), sc)
            fn = lambda pl: oracle.matmul_q8_mt(pl[0], pl[1], x, threads)  # noqa: E731
        else:
            planes = (rng.integers(0, 256, (M, nb, 16), dtype=np.uint8),
                      rng.integers(0, 256, (M, nb, 4), dtype=np.uint8), sc)
            fn = lambda pl: oracle.matmul_q5_mt(pl[0], pl[1], pl[2], x, threads)  # noqa: E731
        per_copy = sum(a.nbytes for a in planes)
        copies = int(min(64, max(2, -(-2 * l3 // per_copy) if l3 else 4)))
        sets = [planes] + [tuple(a.copy() for a in planes) for _ in range(copies - 1)]
        med, calls = _cpu_time(lambda i: fn(sets[i]), copies, seconds)
        cache[key] = med
        log(f"cpu {fam} {M}x{K} on {threads} threads: {med * 1e3:.3f} ms ({copies} copies, {calls} calls)")
        return med

    kind = "asm_matmul_q4_avx512" if variant == 1 else "asm_matmul_q4"
    names = {"q4": kind, "q4s": kind, "q8": "asm_matmul_q8", "q8s": "asm_matmul_q8", "q5": "asm_matmul_q5",
             "q5s": "asm_matmul_q5"}

    def attach(row: dict, sec: float, what: str) -> None:
        row["cpu_baseline"] = {"us": round(sec * 1e6, 2), "GBps": round(row["bytes"] / sec / 1e9, 3),
                               "cores": threads, "kind": "port", "sample": what,
                               "gpu_speedup": round(sec * 1e6 / row["us"], 1)}

    layer_sec = 0.0
    for row in rows:
        if row["op"] not in fmt_of:
            continue
        qt, M, K = fmt_of[row["op"]]
        sec = time_shape(qt, M, K)
        attach(row, sec, f"{names[qt]} restatement, {M}x{K}, split planes, threadpool row tiling")
        if row["op"].startswith("llama3 "):
            layer_sec += sec
    for row in rows:
        if row["op"].startswith("llama3 layer"):
            attach(row, layer_sec, "sum of the 7 Llama-3 matvecs' CPU times (q, k, v, o, gate, up, down)")
    oracle.threadpool_shutdown()
    return {"threads": threads, "cpu_model": cpu_model(), "l3_bytes": l3, "seconds_per_shape": seconds,
            "rotation": "operand copies >= 2x L3 per shape"}


def cpu_gemm_baseline(gemm: dict, threads: int, T: int = 512, M: int = 11008, K: int = 4096,
                      sample_rows: int = 16, seconds: float = 3.0) -> None:
    """The oracle's Q8_0 GEMM (the matmul_q4_neon.S:190-255 recipe per block: int32
    dot, product of the fp16 scales, fma, in block order) on the host threads, on a
    bounded sample of the workload: `sample_rows` of the 512 activation rows against
    the whole 11008x4096 weight matrix, scaled to 512 rows.  Annotates `gemm`."""
    from asmllm_amd import gguf
    from oracle import native as oracle

    rng = np.random.default_rng(99)
    w_blocks = gguf.quantize_q8_0(rng.standard_normal((M, K), dtype=np.float32) * np.float32(0.02))
    a_blocks = gguf.quantize_q8_0(rng.standard_normal((sample_rows, K), dtype=np.float32))
    med, calls = _cpu_time(lambda i: oracle.gemm_q8_0(w_blocks, a_blocks, threads), 1, seconds)
    full = med * T / sample_rows
    ops = 2 * T * M * K
    oracle.threadpool_shutdown()
    log(f"cpu GEMM {sample_rows}x{M}x{K} on {threads} threads: {med * 1e3:.1f} ms -> {full * 1e3:.1f} ms for {T} rows")
    gemm["cpu_baseline"] = {"value": round(ops / full / 1e12, 4), "unit": "TOP/s", "us": round(full * 1e6, 1),
                            "cores": threads, "kind": "port",
                            "sample": f"{sample_rows} of the {T} activation rows x the {M}x{K} Q8_0 weights "
                                      f"(oracle_gemm_q8_0, {calls} calls, median {med * 1e3:.1f} ms), scaled to {T} rows",
                            "gpu_speedup": round(full * 1e6 / gemm["us"], 1)}


def bench_host_pointer(seconds: float = 2.0) -> list[dict]:
    """asm_matmul_q4 as the reference's unchanged callers use it (numpy buffers in
    host memory, tests/correctness/test_runner.py:84-117, src/runtime/generate.py:255-259):
    every call copies the split weights, x and y across PCIe and synchronizes."""
    from asmllm_amd import gguf, native

    lib = native.lib()
    out = []
    for M, K in ((M_MAIN, K_MAIN), (4, 64)):
        blocks, x = make_q4_problem(M, K, seed=7)
        qs, sc = gguf.split_q4_0(blocks)
        y = np.zeros(M, np.float32)
        args = [a.ctypes.data for a in (qs, sc, x, y)] + [M, K]
        for _ in range(3):
            lib.asm_matmul_q4(*args)
        times = []
        t_end = time.perf_counter() + seconds / 2
        while time.perf_counter() < t_end or len(times) < 10:
            t0 = time.perf_counter()
            lib.asm_matmul_q4(*args)
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        moved = qs.nbytes + sc.nbytes + x.nbytes + y.nbytes
        out.append({"shape": f"{M}x{K}", "us_per_call": round(med * 1e6, 2), "host_bytes_per_call": moved,
                    "GBps_host_bytes": round(moved / med / 1e9, 3), "calls": len(times)})
        log(f"host-pointer asm_matmul_q4 {M}x{K}: {med * 1e6:.1f} us per call")
    return out


def _rotating_blocks(qtype: int, M: int, K: int, copies: int, seed: int):
    """`copies` device copies of one synthetic GGUF matrix, generated on the GPU."""
    from asmllm_amd import gguf, native
    from asmllm_amd.device import DeviceBuffer

    lib = native.lib()
    nbytes = gguf.q4_0_nbytes(M, K) if qtype == native.Q4_0 else gguf.q8_0_nbytes(M, K)
    first = DeviceBuffer(nbytes)
    native.check(lib.asmhip_random_blocks(qtype, first.ptr, M, K, seed, 0.02, None), "random blocks")
    bufs = [first]
    for _ in range(copies - 1):
        b = DeviceBuffer(nbytes)
        b.copy_from(first)
        bufs.append(b)
    return bufs, nbytes


EAGER = False  # --eager: launch directly instead of replaying graphs


def time_launches(enqueue, copies: int, reps: int) -> float:
    """Mean GPU microseconds of one launch: `enqueue(i)` cycling over i < copies,
    at least reps x copies launches, between timing-only HIP events.  The
    launches are captured into graphs of at least 512 (a whole number of
    rounds over the copies), since every graph launch costs ~7 us before its
    first kernel starts: in graphs of `copies` launches that would add
    7 us / copies to each launch."""
    from asmllm_amd.device import Event, Graph, Stream, synchronize

    stream = Stream()
    rounds = max(1, -(-512 // copies))  # rounds over the copies per graph
    if EAGER:
        def run():
            for _ in range(rounds):
                for i in range(copies):
                    enqueue(i, stream.handle)
    else:
        graph = Graph.capture(stream, lambda: [enqueue(i, stream.handle) for _ in range(rounds)
                                               for i in range(copies)])

        def run():
            graph.launch(stream)
    for _ in range(2):
        run()
    synchronize()
    runs = max(1, -(-reps // rounds))
    e0, e1 = Event(timing=True), Event(timing=True)
    e0.record(stream)
    for _ in range(runs):
        run()
    e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_ms(e1) * 1e3 / (runs * rounds * copies)
    if not EAGER:
        graph.close()
    return us


# Matvec shapes of the benchmark configurations: the Q8_0 4096x4096 matvec, the
# Llama-7B decode set and the Llama-3-8B layer sweep (GQA: k/v 1024 rows).
MATVEC_TABLE = [
    ("q8_0 4096x4096", "q8", 4096, 4096),
    ("q4_0 4096x4096", "q4", 4096, 4096),
    ("q4_0 11008x4096", "q4", 11008, 4096),
    ("q4_0 4096x11008", "q4", 4096, 11008),
    ("llama3 q 4096x4096", "q4", 4096, 4096),
    ("llama3 k 1024x4096", "q4", 1024, 4096),
    ("llama3 v 1024x4096", "q4", 1024, 4096),
    ("llama3 o 4096x4096", "q4", 4096, 4096),
    ("llama3 gate 14336x4096", "q4", 14336, 4096),
    ("llama3 up 14336x4096", "q4", 14336, 4096),
    ("llama3 down 4096x14336", "q4", 4096, 14336),
    ("q4 split 11008x4096", "q4s", 11008, 4096),
    ("q5_0 11008x4096", "q5", 11008, 4096),
    ("q5 split 11008x4096", "q5s", 11008, 4096),
    # the reference's quant-format sweep (bench/harness/bench_quant_formats.py:41-138):
    # split-layout Q4/Q8/Q5 at M = 32 and 1024, K = 4096; GGUF Q4_0/Q8_0 beside them
    ("formats q4 split 32x4096", "q4s", 32, 4096),
    ("formats q8 split 32x4096", "q8s", 32, 4096),
    ("formats q5 split 32x4096", "q5s", 32, 4096),
    ("formats q4_0 32x4096", "q4", 32, 4096),
    ("formats q8_0 32x4096", "q8", 32, 4096),
    ("formats q4 split 1024x4096", "q4s", 1024, 4096),
    ("formats q8 split 1024x4096", "q8s", 1024, 4096),
    ("formats q5 split 1024x4096", "q5s", 1024, 4096),
    ("formats q8_0 1024x4096", "q8", 1024, 4096),
]


def _rotating_q5(M: int, K: int, copies: int, seed: int, split: bool, q4: bool = False, q8: bool = False):
    """`copies` device copies of one synthetic Q5_0 matrix (random nibbles and
    fifth bits, fp16 scales of N(0, 0.02^2) weights' size): GGUF blocks, or
    the split ql / qh / fp32 scales planes (q4: the Q4 split qs / scales planes;
    q8: the Q8 split int8 qs / scales planes)."""
    from asmllm_amd import gguf
    from asmllm_amd.device import DeviceBuffer

    rng = np.random.default_rng(seed)
    nb = K // 32
    ql = rng.integers(0, 256, (M, nb, 16), dtype=np.uint8)
    qh = rng.integers(0, 256, (M, nb, 4), dtype=np.uint8)
    d = (rng.uniform(0.001, 0.004, (M, nb)) * rng.choice([-1.0, 1.0], (M, nb))).astype(np.float16)
    if q8:
        planes = (rng.integers(-127, 128, (M, nb, 32), dtype=np.int8), d.astype(np.float32))
    elif q4:
        planes = (ql, d.astype(np.float32))
    else:
        planes = (ql, qh, d.astype(np.float32)) if split else (gguf.pack_q5_0(ql, qh, d),)
    first = [DeviceBuffer.from_numpy(a) for a in planes]
    sets = [first]
    for _ in range(copies - 1):
        bs = []
        for f in first:
            b = DeviceBuffer(f.nbytes)
            b.copy_from(f)
            bs.append(b)
        sets.append(bs)
    return sets, sum(a.nbytes for a in planes)


def bench_matvec_table(min_rotated_bytes: int = 600_000_000) -> list[dict]:
    """GB/s of every configured matvec shape, weights rotating over enough
    copies (>= 600 MB) that HBM serves them."""
    from asmllm_amd import native
    from asmllm_amd.device import DeviceBuffer

    lib = native.lib()
    rows = []
    for name, qt, M, K in MATVEC_TABLE:
        blk = {"q4": 18, "q8": 34, "q5": 22, "q5s": 24, "q4s": 20, "q8s": 36}[qt]
        copies = max(8, -(-min_rotated_bytes // (M * (K // 32) * blk)))
        dx, dy = DeviceBuffer(4 * K), DeviceBuffer(4 * M)
        native.check(lib.asmhip_fill_f32(dx.ptr, K, 0.5, None), "fill")
        if qt in ("q5", "q5s", "q4s", "q8s"):
            sets, _ = _rotating_q5(M, K, copies, seed=M * 7 + K, split=qt != "q5", q4=qt == "q4s", q8=qt == "q8s")
            if qt in ("q4s", "q8s"):
                fn = lib.asmhip_matmul_q4_split if qt == "q4s" else lib.asmhip_matmul_q8_split

                def enqueue(i, st, sets=sets, dx=dx, dy=dy, M=M, K=K, name=name, fn=fn):
                    qs, sc = sets[i % len(sets)]
                    native.check(fn(qs.ptr, sc.ptr, dx.ptr, dy.ptr, M, K, st), name)
            elif qt == "q5":
                def enqueue(i, st, sets=sets, dx=dx, dy=dy, M=M, K=K, name=name):
                    w = sets[i % len(sets)]
                    native.check(lib.asmhip_matmul_q5_0(w[0].ptr, dx.ptr, dy.ptr, M, K, st), name)
            else:
                def enqueue(i, st, sets=sets, dx=dx, dy=dy, M=M, K=K, name=name):
                    ql, qh, sc = sets[i % len(sets)]
                    native.check(lib.asmhip_matmul_q5_split(ql.ptr, qh.ptr, sc.ptr, dx.ptr, dy.ptr, M, K, st), name)
            bufs = [b for bs in sets for b in bs]
        else:
            qtype = native.Q4_0 if qt == "q4" else native.Q8_0
            bufs, nbytes = _rotating_blocks(qtype, M, K, copies, seed=M * 7 + K)
            fn = lib.asmhip_matmul_q4_0 if qt == "q4" else lib.asmhip_matmul_q8_0

            def enqueue(i, st, fn=fn, bufs=bufs, dx=dx, dy=dy, M=M, K=K, name=name):
                native.check(fn(bufs[i % len(bufs)].ptr, dx.ptr, dy.ptr, M, K, st), name)

        us = time_launches(enqueue, copies, reps=max(4, 4000 // copies))
        algo = M * (K // 32) * blk + 4 * K + 4 * M
        rows.append({"op": name, "us": round(us, 3), "GBps": round(algo / us / 1e3, 1),
                     "frac": round(algo / us / 1e3 / HBM_PEAK_GBPS, 4), "bytes": algo})
        for b in bufs:
            b.close()
        log(f"{name}: {us:.3f} us, {algo / us / 1e3:.0f} GB/s")
    layer = [r for r in rows if r["op"].startswith("llama3 ")]
    us = sum(r["us"] for r in layer)
    nbytes = sum(r["bytes"] for r in layer)
    rows.append({"op": "llama3 layer (7 matvecs)", "us": round(us, 3), "GBps": round(nbytes / us / 1e3, 1),
                 "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBPS, 4), "bytes": nbytes})

    # The same layer's matvecs as the decode engine launches them (asmllm_amd/engine.py):
    # q/k/v stacked into one matrix with the attention RMSNorm fused into its read of x,
    # o with the residual add, gate/up interleaved into one matrix with the FFN RMSNorm
    # and SwiGLU fused (h = silu(gate) * up), down with the residual add: 4 launches.
    d, ffn, kv = 4096, 14336, 1024
    norm = DeviceBuffer(4 * ffn)
    native.check(lib.asmhip_fill_f32(norm.ptr, ffn, 1.0, None), "fill")
    hx, hh, work = DeviceBuffer(4 * ffn), DeviceBuffer(4 * ffn), DeviceBuffer(8 * ffn)
    native.check(lib.asmhip_fill_f32(hx.ptr, ffn, 0.5, None), "fill")
    native.check(lib.asmhip_fill_f32(hh.ptr, ffn, 0.5, None), "fill")
    eps = 1e-5
    engine_ops = [
        ("llama3.engine q/k/v stacked 6144x4096 (RMSNorm)", d + 2 * kv, d,
         lambda w, st, M, K: lib.asmhip_matmul_fused(native.Q4_0, w, hx.ptr, work.ptr, M, K, native.PRE_RMSNORM,
                                                     norm.ptr, eps, 0, st)),
        ("llama3.engine o 4096x4096 (residual add)", d, d,
         lambda w, st, M, K: lib.asmhip_matmul_fused(native.Q4_0, w, hh.ptr, hx.ptr, M, K, native.PRE_NONE,
                                                     None, eps, 1, st)),
        ("llama3.engine gate/up 28672x4096 (RMSNorm, SwiGLU)", 2 * ffn, d,
         lambda w, st, M, K: lib.asmhip_matmul_swiglu(native.Q4_0, w, hx.ptr, hh.ptr, M // 2, K, native.PRE_RMSNORM,
                                                      norm.ptr, eps, work.ptr, st)),
        ("llama3.engine down 4096x14336 (residual add)", d, ffn,
         lambda w, st, M, K: lib.asmhip_matmul_fused(native.Q4_0, w, hh.ptr, hx.ptr, M, K, native.PRE_NONE,
                                                     None, eps, 1, st)),
    ]
    eng_rows = []
    for name, M, K, call in engine_ops:
        copies = max(8, -(-min_rotated_bytes // (M * (K // 32) * 18)))
        bufs, _ = _rotating_blocks(native.Q4_0, M, K, copies, seed=M * 5 + K)

        def enqueue(i, st, bufs=bufs, M=M, K=K, name=name, call=call):
            native.check(call(bufs[i % len(bufs)].ptr, st, M, K), name)

        us = time_launches(enqueue, copies, reps=max(4, 4000 // copies))
        algo = M * (K // 32) * 18 + 4 * K + 4 * M
        eng_rows.append({"op": name, "us": round(us, 3), "GBps": round(algo / us / 1e3, 1),
                         "frac": round(algo / us / 1e3 / HBM_PEAK_GBPS, 4), "bytes": algo})
        for b in bufs:
            b.close()
        log(f"{name}: {us:.3f} us, {algo / us / 1e3:.0f} GB/s")
    rows += eng_rows
    us = sum(r["us"] for r in eng_rows)
    nbytes = sum(r["bytes"] for r in eng_rows)
    rows.append({"op": "llama3 layer (engine form: 4 launches)", "us": round(us, 3),
                 "GBps": round(nbytes / us / 1e3, 1), "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBPS, 4),
                 "bytes": nbytes})
    return rows


def bench_read_floor(multiples=(1, 2, 4, 8)) -> dict:
    """The single-launch read floor: asmhip_stream_read (every workgroup one
    contiguous chunk, all loads up front) over m times the 11008x4096 matvec's
    bytes per launch, rotating over a 1.6 GB region so HBM serves every launch.
    A straight-line fit of time against bytes splits a launch into a fixed part
    (ramp, first-load latency, drain, launch gap) and a sustained rate; the time
    at m = 1 is the fastest any one launch reads the matvec's bytes."""
    from asmllm_amd import native
    from asmllm_amd.device import DeviceBuffer

    lib = native.lib()
    unit = q4_algorithmic_bytes(M_MAIN, K_MAIN)
    region = 64 * unit
    buf, sink = DeviceBuffer(region + (1 << 20)), DeviceBuffer(4096)
    native.check(lib.asmhip_fill_f32(buf.ptr, region // 4, 0.5, None), "fill")
    native.check(lib.asmhip_fill_f32(sink.ptr, 1024, 0.0, None), "fill")
    points = []
    for m in multiples:
        nbytes = m * unit
        launches = region // nbytes

        def enqueue(i, st, nbytes=nbytes):
            native.check(lib.asmhip_stream_read(buf.ptr + i * nbytes, nbytes, sink.ptr, st), "stream read")

        us = time_launches(enqueue, launches, reps=max(4, 2000 // launches))
        points.append({"bytes": nbytes, "us": round(us, 3), "GBps": round(nbytes / us / 1e3, 1)})
        log(f"stream read {nbytes / 1e6:.1f} MB: {us:.3f} us, {nbytes / us / 1e3:.0f} GB/s")
    xs = np.array([p["bytes"] for p in points], np.float64)
    ys = np.array([p["us"] for p in points], np.float64)
    slope, fixed = np.polyfit(xs, ys, 1)

    # the same kernel on 4 KB (one 16-byte load per workgroup): what a dependent
    # graph node costs with next to no work (64 addresses cycled in graphs of 512 launches)
    def enqueue_tiny(i, st):
        native.check(lib.asmhip_stream_read(buf.ptr + i * 4096, 4096, sink.ptr, st), "stream read")

    launch_us = time_launches(enqueue_tiny, 64, reps=50)
    log(f"stream read 4 KB (launch floor): {launch_us:.3f} us")

    # an empty kernel as a dependent graph node, at the matvec's launch shape
    # (256 workgroups of 1024 threads, 155 KB of dynamic LDS) and two small ones
    empty = []
    for grid, threads, lds in ((256, 1024, 155 * 1024), (256, 256, 0), (64, 64, 0)):
        def enqueue_empty(i, st, grid=grid, threads=threads, lds=lds):
            native.check(lib.asmhip_empty_launch(grid, threads, lds, st), "empty launch")

        us = time_launches(enqueue_empty, 64, reps=50)
        empty.append({"grid": grid, "threads": threads, "lds_bytes": lds, "us": round(us, 3)})
        log(f"empty launch {grid}x{threads}, {lds} B LDS: {us:.3f} us")

    # the read floor in the matvec's launch shape, its structural pieces added one at a time
    cus = device_info_cus()
    x = DeviceBuffer(4 * K_MAIN)
    native.check(lib.asmhip_fill_f32(x.ptr, K_MAIN, 0.5, None), "fill")
    y_floats = 1 << 16
    y = DeviceBuffer(4 * y_floats)
    shaped = []
    launches = region // unit
    for flags, what in ((0, "one 1024-thread workgroup per CU, all loads up front"),
                        (1, "+ the matvec's 155 KB of dynamic LDS"),
                        (3, "+ x (16 KB) read and a workgroup barrier first"),
                        (7, "+ 16 floats stored per workgroup at the end")):
        def enqueue_shaped(i, st, flags=flags):
            native.check(lib.asmhip_stream_read_shaped(buf.ptr + i * unit, unit, x.ptr, K_MAIN, y.ptr, y_floats,
                                                       flags, 155 * 1024, sink.ptr, st), "shaped read")

        us = time_launches(enqueue_shaped, launches, reps=max(4, 2000 // launches))
        shaped.append({"flags": flags, "shape": what, "us": round(us, 3), "GBps": round(unit / us / 1e3, 1)})
        log(f"shaped read ({what}): {us:.3f} us")
    x.close()
    y.close()
    buf.close()
    sink.close()
    return {"points": points, "fixed_us_per_launch": round(float(fixed), 3),
            "sustained_GBps": round(1e-3 / float(slope), 1),
            "floor_us_at_matvec_bytes": points[0]["us"],
            "floor_frac_of_peak": round(points[0]["GBps"] / HBM_PEAK_GBPS, 4),
            "launch_floor_us_4KB": round(launch_us, 3),
            "empty_launch": empty,
            "matvec_shaped_read": shaped,
            "grid_barrier": bench_grid_barrier(cus)}


STAMP_EVENTS = ("entry", "first weight loads issued", "x digits ready", "first unit landed", "last unit landed",
                "stream done", "all waves done", "y written")


def bench_stamps(launches: int = 64, copies: int = 32) -> dict:
    """Where one 11008x4096 launch spends its time, from inside the kernel: the
    headline matvec in its stamped instantiation (asmhip_matmul_q4_0_stamped: every
    wave records the 100 MHz real-time counter at 8 points), `launches` back-to-back
    launches replayed from one graph over rotating weight copies behind untimed
    cover reads.  Per event: percentiles over all waves of the time since the
    launch's first wave started; per launch: the span from the first wave's start to
    the last wave's completed y write, and the gap from there to the next launch's
    first wave.  The stamps cost time of their own (their scalar reads of the
    counter and stores): the stamped and plain launches are timed side by side."""
    from asmllm_amd import native
    from asmllm_amd.device import DeviceBuffer, Event, Graph, Stream, synchronize

    lib = native.lib()
    M, K = M_MAIN, K_MAIN
    bufs, _ = _rotating_blocks(native.Q4_0, M, K, copies, seed=7)
    x, y, y2 = DeviceBuffer(4 * K), DeviceBuffer(4 * M), DeviceBuffer(4 * M)
    native.check(lib.asmhip_fill_f32(x.ptr, K, 0.5, None), "fill")
    grid = min((M + 15) // 16, device_info_cus())
    per = grid * 16 * len(STAMP_EVENTS)
    st_buf = DeviceBuffer(8 * per * launches)
    cov, sink = DeviceBuffer(1 << 30), DeviceBuffer(4096)
    stream = Stream()

    def stamped(i: int) -> None:
        native.check(lib.asmhip_matmul_q4_0_stamped(bufs[i % copies].ptr, x.ptr, y.ptr, M, K, st_buf.ptr + 8 * per * i,
                                                    per, stream.handle), "stamped matvec")

    def plain(i: int) -> None:
        native.check(lib.asmhip_matmul_q4_0(bufs[i % copies].ptr, x.ptr, y2.ptr, M, K, stream.handle), "matvec")

    stamped(0)
    plain(0)
    stream.synchronize()
    same = bool(np.array_equal(y.download(np.uint32, M), y2.download(np.uint32, M)))
    g_st = Graph.capture(stream, lambda: [stamped(i) for i in range(launches)])
    g_pl = Graph.capture(stream, lambda: [plain(i) for i in range(launches)])
    e0, e1 = Event(timing=True), Event(timing=True)

    def timed(g) -> float:
        g.launch(stream)
        synchronize()
        for _ in range(200):  # ~30 ms of untimed reads: the GPU busy while the graph is queued
            native.check(lib.asmhip_stream_read(cov.ptr, cov.nbytes, sink.ptr, stream.handle), "cover")
        e0.record(stream)
        g.launch(stream)
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_ms(e1) * 1e3 / launches

    t_pl = min(timed(g_pl) for _ in range(3))
    t_st = min(timed(g_st) for _ in range(3))
    a = st_buf.download(np.uint64, (launches, grid * 16, len(STAMP_EVENTS))).astype(np.int64)
    g_st.close()
    g_pl.close()
    first = a[:, :, 0].min(axis=1)
    last = a[:, :, -1].max(axis=1)
    rel = (a - first[:, None, None]) * 0.01  # 100 MHz ticks -> us
    keep = slice(4, launches)  # the first launches of a replay start the stream
    events = []
    for i, name in enumerate(STAMP_EVENTS):
        v = rel[keep, :, i]
        v = v[a[keep, :, i] > 0]
        events.append({"event": name, "p10_us": round(float(np.percentile(v, 10)), 3),
                       "median_us": round(float(np.median(v)), 3), "p90_us": round(float(np.percentile(v, 90)), 3),
                       "max_us": round(float(v.max()), 3)})
    span = (last - first)[keep] * 0.01
    gap = (first[1:] - last[:-1])[keep.start:] * 0.01
    tiles = -(-((M + 15) // 16 - np.arange(grid)) // grid)
    wg_end = rel[keep, :, -1].reshape(-1, grid, 16).max(axis=2)
    by_tiles = {int(t): round(float(np.median(wg_end[:, tiles == t])), 3) for t in sorted(set(tiles.tolist()))}
    for b in bufs:
        b.close()
    log(f"stamps: plain {t_pl:.3f} us/launch, stamped {t_st:.3f}; span {span.mean():.3f}, gap {gap.mean():.3f}")
    return {"workload": f"Q4_0 matvec {M}x{K}, {launches} back-to-back launches from one graph, {copies} weight copies",
            "kernel": "gguf_mfma_stream<0,1,16,1,1,0,false,16,false,true,false,false> (stamped instantiation)",
            "stamped_y_bitwise_equal_plain": same,
            "plain_us_per_launch": round(t_pl, 3), "stamped_us_per_launch": round(t_st, 3),
            "events_us_since_first_wave": events,
            "span_us_mean": round(float(span.mean()), 3), "gap_us_mean": round(float(gap.mean()), 3),
            "gap_us_min": round(float(gap.min()), 3),
            "workgroup_end_median_us_by_tiles": by_tiles}


def device_info_cus() -> int:
    from asmllm_amd.device import device_info

    return int(device_info()["compute_units"])


def bench_grid_barrier(cus: int) -> dict | None:
    """What a grid-wide handoff inside one launch costs: n barriers in one
    cooperative launch of one 1024-thread workgroup per compute unit (a counter
    added to and polled at agent scope, coherent across the XCDs), timed at
    n = 200 and 1000; the difference over 800 is the cost of one barrier, to set
    beside a dependent launch (`empty_launch`)."""
    from asmllm_amd import native
    from asmllm_amd.device import DeviceBuffer, Event, Stream

    lib = native.lib()
    counter, err = DeviceBuffer(256), DeviceBuffer(256)
    zero = np.zeros(64, np.uint32)
    counter.upload(zero)
    err.upload(zero)
    stream = Stream()
    e0, e1 = Event(timing=True), Event(timing=True)

    def run(n: int) -> float | None:
        e0.record(stream)
        rc = lib.asmhip_grid_barrier(counter.ptr, n, err.ptr, stream.handle)
        if rc:
            log(f"grid barrier not measured: {native.last_error()}")
            return None
        e1.record(stream)
        e1.synchronize()
        if int(err.download(np.uint32, 1)[0]):
            log("grid barrier: a barrier hit its poll bound")
            return None
        return e0.elapsed_ms(e1) * 1e3

    times = {}
    for n in (0, 200, 1000, 200, 1000):
        t = run(n)
        if t is None:
            return None
        times.setdefault(n, []).append(t)
    per = (min(times[1000]) - min(times[200])) / 800
    log(f"grid barrier: {per:.3f} us per barrier ({cus} workgroups)")
    counter.close()
    err.close()
    return {"workgroups": cus, "us_per_barrier": round(per, 3), "launch_us_n0": round(min(times[0]), 2),
            "us_n200": round(min(times[200]), 1), "us_n1000": round(min(times[1000]), 1)}


def bench_matvec_phases(K: int = K_MAIN, rows=(1024, 2048, 4096, 8192, 11008, 16384, 22016, 32000),
                        min_rotated_bytes: int = 600_000_000) -> dict:
    """Ramp and tail against the steady stream of the Q4_0 matvec: the same kernel
    (K = 4096) timed at several row counts, weights rotating over >= 32 copies and
    >= 600 MB, and a straight-line fit of time against bytes over the rows that
    fill the grid (M >= 4096: one 16-row tile or more per compute unit).  The
    slope is the steady streaming rate; the intercept is what a launch costs
    besides streaming (dispatch, x read and digitization before the first
    multiply, the last tiles' tail, the partial-sum reduction and store).  Set
    beside the read floor's fit (`--only floor`) it says whether the gap to the
    floor is rate or fixed cost."""
    from asmllm_amd import native
    from asmllm_amd.device import DeviceBuffer

    lib = native.lib()
    points = []
    for M in rows:
        nbytes_w = M * (K // 32) * 18
        copies = max(32, -(-min_rotated_bytes // nbytes_w))
        bufs, _ = _rotating_blocks(native.Q4_0, M, K, copies, seed=M + 5)
        dx, dy = DeviceBuffer(4 * K), DeviceBuffer(4 * M)
        native.check(lib.asmhip_fill_f32(dx.ptr, K, 0.5, None), "fill")

        def enqueue(i, st, bufs=bufs, dx=dx, dy=dy, M=M):
            native.check(lib.asmhip_matmul_q4_0(bufs[i % len(bufs)].ptr, dx.ptr, dy.ptr, M, K, st), "matvec")

        us = time_launches(enqueue, copies, reps=max(4, 4000 // copies))
        algo = q4_algorithmic_bytes(M, K)
        points.append({"M": M, "bytes": algo, "us": round(us, 3), "GBps": round(algo / us / 1e3, 1)})
        log(f"matvec {M}x{K}: {us:.3f} us, {algo / us / 1e3:.0f} GB/s")
        for b in bufs:
            b.close()
        dx.close()
        dy.close()
    full = [p for p in points if p["M"] >= 4096]
    xs = np.array([p["bytes"] for p in full], np.float64)
    ys = np.array([p["us"] for p in full], np.float64)
    slope, fixed = np.polyfit(xs, ys, 1)
    resid = ys - (fixed + slope * xs)
    return {"K": K, "points": points, "fit_rows": "M >= 4096", "fixed_us_per_launch": round(float(fixed), 3),
            "steady_GBps": round(1e-3 / float(slope), 1), "fit_max_residual_us": round(float(np.max(np.abs(resid))), 3)}


INT8_MFMA_PEAK_TOPS = 5000.0


def bench_gemm(T: int = 512, M: int = 11008, K: int = 4096, copies: int = 12) -> dict:
    """Q8_0 x Q8_0 prefill GEMM: activations 512x4096 fp32 quantized per row on
    the GPU, weights 11008x4096 Q8_0; ops = 2*T*M*K.  The headline form takes
    both operands in the GEMM tile layout (the same Q8_0 blocks, permuted): the
    weights arranged once (a load-time cost, reported, not timed per call), the
    activations quantized straight into it.  The GGUF-block form and the split
    form are timed on the same blocks."""
    from asmllm_amd import gguf, native
    from asmllm_amd.device import DeviceBuffer, Event, Stream

    lib = native.lib()
    wbufs, _ = _rotating_blocks(native.Q8_0, M, K, copies, seed=99)
    da = DeviceBuffer(4 * T * K)
    native.check(lib.asmhip_fill_f32(da.ptr, T * K, 0.25, None), "fill")
    dq = DeviceBuffer(gguf.q8_0_nbytes(T, K))
    native.check(lib.asmhip_random_blocks(native.Q8_0, dq.ptr, T, K, 5, 1.0, None), "random activations")
    dc = DeviceBuffer(4 * T * M)

    # the tile layout: weights arranged once per copy, activations from the same blocks
    wt_bytes = lib.asmhip_gemm_q8_0_tiled_weight_bytes(M, K)
    wtiled = [DeviceBuffer(wt_bytes) for _ in range(copies)]
    st = Stream()
    e0, e1 = Event(timing=True), Event(timing=True)
    e0.record(st)
    native.check(lib.asmhip_gemm_q8_0_tile_weights(wbufs[0].ptr, wtiled[0].ptr, M, K, st.handle), "tile weights")
    e1.record(st)
    e1.synchronize()
    tile_us = e0.elapsed_ms(e1) * 1e3
    for b in wtiled[1:]:
        b.copy_from(wtiled[0])
    dqt = DeviceBuffer(lib.asmhip_gemm_q8_0_tiled_activation_bytes(T, K))
    native.check(lib.asmhip_gemm_q8_0_tile_activations(dq.ptr, dqt.ptr, T, K, None), "tile activations")

    def gemm_tiled(i, st):
        native.check(lib.asmhip_gemm_q8_0_tiled(wtiled[i % copies].ptr, dqt.ptr, dc.ptr, T, M, K, st), "gemm tiled")

    def quant_tiled(i, st):
        native.check(lib.asmhip_quantize_q8_0_tiled(da.ptr, dqt.ptr, T, K, st), "quantize tiled")

    def gemm(i, st):
        native.check(lib.asmhip_gemm_q8_0(wbufs[i % copies].ptr, dq.ptr, dc.ptr, T, M, K, st), "gemm")

    def quant(i, st):
        native.check(lib.asmhip_quantize(native.Q8_0, da.ptr, dq.ptr, T, K, st), "quantize")

    us = time_launches(gemm_tiled, copies, reps=20)
    us_qt = time_launches(quant_tiled, copies, reps=20)  # (overwrites dqt; the block form reads dq)
    us_b = time_launches(gemm, copies, reps=20)
    us_q = time_launches(quant, copies, reps=20)
    ops = 2 * T * M * K
    nbytes = gguf.q8_0_nbytes(M, K) + gguf.q8_0_nbytes(T, K) + 4 * T * M
    log(f"GEMM {T}x{M}x{K} tile layout: {us:.2f} us, {ops / us / 1e6:.0f} TOP/s; GGUF blocks: {us_b:.2f} us")

    # the same operands in the split layout (int8 qs planes + fp32 scale planes);
    # the results are bitwise those of the block-form GEMM
    nb = K // 32
    w0 = wbufs[0].download(np.uint8, (M, nb, 34))
    wq = DeviceBuffer.from_numpy(np.ascontiguousarray(w0[:, :, 2:]).view(np.int8))
    ws = DeviceBuffer.from_numpy(w0[:, :, 0:2].copy().view(np.float16).reshape(M, nb).astype(np.float32))
    wsplit = [(wq, ws)] + [(DeviceBuffer(wq.nbytes), DeviceBuffer(ws.nbytes)) for _ in range(copies - 1)]
    for q, s in wsplit[1:]:
        q.copy_from(wq)
        s.copy_from(ws)
    a0 = dq.download(np.uint8, (T, nb, 34))  # the same activation blocks
    aq = DeviceBuffer.from_numpy(np.ascontiguousarray(a0[:, :, 2:]).view(np.int8))
    as_ = DeviceBuffer.from_numpy(a0[:, :, 0:2].copy().view(np.float16).reshape(T, nb).astype(np.float32))

    def gemm_split(i, st):
        q, s = wsplit[i % copies]
        native.check(lib.asmhip_gemm_q8_split(q.ptr, s.ptr, aq.ptr, as_.ptr, dc.ptr, T, M, K, st), "gemm split")

    us_s = time_launches(gemm_split, copies, reps=20)
    nbytes_s = M * K + 4 * M * nb + T * K + 4 * T * nb + 4 * T * M
    log(f"GEMM split layout: {us_s:.2f} us, {ops / us_s / 1e6:.0f} TOP/s")

    def form(us_, nbytes_):
        return {"us": round(us_, 3), "TOPs": round(ops / us_ / 1e6, 1),
                "frac_int8_mfma_peak": round(ops / us_ / 1e6 / INT8_MFMA_PEAK_TOPS, 4), "bytes": nbytes_}

    return {"workload": f"Q8_0 GEMM C[{T}][{M}] = A_q8[{T}][{K}] . W_q8[{M}][{K}]^T, operands in the GEMM tile "
                        f"layout (the same Q8_0 blocks; weights arranged once, activations quantized into it)",
            **form(us, nbytes), "GBps": round(nbytes / us / 1e3, 1), "ops": ops,
            "activation_quantize_us": round(us_qt, 3), "weight_tiling_us_once": round(tile_us, 3),
            "block_layout": {"layout": "GGUF Q8_0 blocks [rows][K/32] as given (asmhip_gemm_q8_0)",
                             **form(us_b, nbytes), "activation_quantize_us": round(us_q, 3)},
            "split_layout": {"layout": "int8 qs [rows][K] + fp32 scales [rows][K/32] (asm_matmul_q8's operands)",
                             **form(us_s, nbytes_s)}}


def decode_cpu_baseline(eng, context: int, seconds: float) -> dict:
    """The oracle's decode step (the reference's forward_token sequence over the
    oracle's restated kernels, generate.py:261-326) on the host cores, on the
    engine's own weights and cache read back from HBM: tokens from position
    `context` until `seconds` have passed (at least two)."""
    from oracle.decode_ref import DecodeRef

    s = eng.shape
    d, h, kv = s.dim, s.hidden_dim, s.kv_dim

    def blocks(buf, rows, K):
        return buf.download(np.uint8, (rows, K // 32, 18))

    layers, kcs, vcs = [], [], []
    for i, ly in enumerate(eng.layers):
        qkv, (gate, up) = blocks(ly.wqkv, s.qkv_rows, d), eng.gate_up_blocks(i)
        layers.append({"attn_norm": ly.attn_norm.download(np.float32, d),
                       "ffn_norm": ly.ffn_norm.download(np.float32, d),
                       "wq": qkv[:d], "wk": qkv[d:d + kv], "wv": qkv[d + kv:], "wo": blocks(ly.wo, d, d),
                       "w_gate": gate, "w_up": up, "w_down": blocks(ly.wdown, d, h)})
        kcs.append(ly.k_cache.download(np.uint16, (s.n_kv_heads, eng.max_ctx, s.head_dim)))
        vcs.append(ly.v_cache.download(np.uint16, (s.n_kv_heads, eng.max_ctx, s.head_dim)))
    cores = host_cores()
    ref = DecodeRef(dim=d, n_heads=s.n_heads, n_kv_heads=s.n_kv_heads, hidden_dim=h, vocab=s.vocab, eps=s.eps,
                    theta=s.theta, embed=blocks(eng.embed, s.vocab, d),
                    final_norm=eng.final_norm.download(np.float32, d), output=blocks(eng.output, s.vocab, d),
                    layers=layers, k_caches=kcs, v_caches=vcs, nt=cores)
    del kcs, vcs
    token, times = 1, []
    t_end = time.perf_counter() + seconds
    while len(times) < 2 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        logits = ref.forward_token(token, context + len(times))
        times.append(time.perf_counter() - t0)
        token = int(np.argmax(logits))
    from oracle import native as oracle

    oracle.threadpool_shutdown()
    med = float(np.median(times))
    return {"value": round(1.0 / med, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": (f"{len(times)} greedy decode tokens of the same 7B-shape model from position {context}: "
                       f"oracle forward_token (restated AVX2 Q4_0 kernel + threadpool tiling over GGUF blocks, "
                       f"fp16-cache attention) on {cores} threads, median {med:.3f} s per token")}


def bench_decode(steps: int = 128, context: int = 2048, warmup: int = 4, eager: bool = False,
                 cpu_seconds: float = 0.0) -> dict:
    """Greedy single-token decode of the 32-layer 7B-shape Q4_0 model, fp16 KV
    cache prefilled to `context`: `steps` tokens from position `context` through
    the engine's own generation path (DecodeEngine.enqueue_generate): replays of
    a captured graph of 16 consecutive token steps (token, position and the
    history of chosen tokens stay on the GPU between steps; one graph launch per
    16 tokens, since a graph launch costs ~7 us before its first kernel) plus
    single-step replays for the remainder; every generated token is read back
    from the device history after the timed region.  `eager` enqueues the
    launches directly instead (for tracing tools that do not follow graph
    launches)."""
    from asmllm_amd.device import Event, synchronize
    from asmllm_amd.engine import LLAMA_7B, DecodeEngine

    s = LLAMA_7B
    eng = DecodeEngine(s, max_ctx=context + steps)
    eng.init_random(seed=42)
    per_graph = eng.STEPS_PER_GRAPH
    # warm-up: every graph the timed steps replay is launched once (a graph's
    # first launch also sets it up on the device)
    eng.set_position(1, context)
    eng.enqueue_generate(max(warmup, per_graph + 1) if not eager else warmup, use_graph=not eager)
    eng.stream.synchronize()
    eng.set_position(1, context)
    synchronize()
    e0, e1 = Event(timing=True), Event(timing=True)
    e0.record(eng.stream)
    # the engine's own generation path: graphs of 16 token steps, then one-step
    # graphs for the rest; every token is kept in the device history
    eng.enqueue_generate(steps, use_graph=not eager)
    e1.record(eng.stream)
    e1.synchronize()
    ms = e0.elapsed_ms(e1)
    tokens = eng.read_history(context, steps)
    if len(tokens) != steps or not all(0 <= t < s.vocab for t in tokens):
        raise SystemExit("decode: the token history is not a list of vocabulary ids")
    end_pos = eng.read_position()
    if end_pos != context + steps:
        raise SystemExit(f"decode: position {end_pos} after {steps} steps from {context}")
    # HBM bytes per token: all Q4_0 weights + one embedding row + the KV cache
    # read (positions 0..pos, k and v, every layer) + the new k/v row written
    kv_read = sum((p + 1) for p in range(context, context + steps)) / steps * s.kv_bytes_per_position()
    per_token = s.weight_bytes() + (s.dim // 32) * 18 + kv_read + s.kv_bytes_per_position()
    tok_s = steps / (ms / 1e3)
    cpu = decode_cpu_baseline(eng, context, cpu_seconds) if cpu_seconds > 0 else None
    eng.close()
    log(f"decode: {tok_s:.1f} tokens/s ({ms / steps:.3f} ms/token)")
    return {"workload": f"7B-shape Q4_0 Llama greedy decode, {s.n_layers} layers, d {s.dim}, {s.n_heads}x"
                        f"{s.head_dim} heads, FFN {s.hidden_dim}, vocab {s.vocab}, fp16 KV prefilled to {context}",
            "launch": "eager" if eager else "graph", "tokens_per_s": round(tok_s, 2), "ms_per_token": round(ms / steps, 4), "steps": steps,
            "context": context, "bytes_per_token": int(per_token),
            "GBps": round(per_token * tok_s / 1e9, 1), "frac": round(per_token * tok_s / 1e9 / HBM_PEAK_GBPS, 4),
            "cpu_baseline": cpu}


def bench_decode_launches(context: int = 2048, reps: int = 8, per_graph: int = 256) -> dict:
    """Each launch kind of the 7B decode step timed on its own, back to back in
    graph replay, in the state of a real token step at position `context`: one
    whole step runs first (every buffer then holds that step's values), then
    the launches of one kind (qkv, attention, o, gate_up, down over the 32
    layers' own weights and caches; lm_head, embed, argmax once a step) are
    captured `per_graph` launches to a graph and replayed `reps` times.  The
    attention reads positions 0..context of the layer's cache; argmax runs last
    (it advances the position).  bytes: what the launch reads from HBM."""
    from asmllm_amd.device import Event, Graph, synchronize
    from asmllm_amd.engine import LLAMA_7B, DecodeEngine
    from asmllm_amd.gguf import q4_0_nbytes

    s = LLAMA_7B
    d, h, hd = s.dim, s.hidden_dim, s.head_dim
    eng = DecodeEngine(s, max_ctx=context + 128)
    eng.init_random(seed=42)
    eng.set_position(1, context)
    eng.enqueue_step()
    eng.stream.synchronize()
    launches = list(eng.step_launches())
    kv = s.n_kv_heads * (context + 1) * hd * 2 * 2  # k and v rows 0..context of one layer, fp16
    nbytes = {
        "qkv": q4_0_nbytes(s.qkv_rows, d) + 4 * d, "attention": kv,
        "o": q4_0_nbytes(d, d) + 4 * s.n_heads * attn_splits_of(context + 128) * (hd + 4),
        "gate_up": q4_0_nbytes(2 * h, d) + 4 * d, "down": q4_0_nbytes(d, h) + 4 * h,
        "lm_head": q4_0_nbytes(s.vocab, d) + 4 * d, "embed": (d // 32) * 18, "argmax": 4 * s.vocab,
    }
    out = {}
    for kind in ("qkv", "attention", "o", "gate_up", "down", "lm_head", "embed", "argmax"):
        eng.set_position(1, context)
        fns = [f for k, _, f in launches if k == kind]
        rounds = max(1, per_graph // len(fns))
        graph = Graph.capture(eng.stream, lambda: [f() for _ in range(rounds) for f in fns])
        graph.launch(eng.stream)
        eng.stream.synchronize()
        if kind == "argmax":
            eng.set_position(1, context)
        synchronize()
        e0, e1 = Event(timing=True), Event(timing=True)
        e0.record(eng.stream)
        for _ in range(reps):
            graph.launch(eng.stream)
        e1.record(eng.stream)
        e1.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / (reps * rounds * len(fns))
        graph.close()
        out[kind] = {"us": round(us, 3), "per_token": len(fns), "bytes": int(nbytes[kind]),
                     "GBps": round(nbytes[kind] / (us * 1e-6) / 1e9, 1)}
    eng.close()
    layer = sum(out[k]["us"] for k in ("qkv", "attention", "o", "gate_up", "down"))
    token = sum(v["us"] * v["per_token"] for v in out.values())
    log(f"decode launches: layer {layer:.2f} us, token {token:.1f} us (sum of the launches, one kind at a time)")
    return {"workload": f"7B-shape Q4_0 decode step at position {context}, each launch kind back to back in "
                        f"graphs of {per_graph}; lm_head / embed / argmax repeat the one launch of a step "
                        "(its weights then stay in the MALL)",
            "launches": out, "layer_us": round(layer, 2), "token_us_sum": round(token, 1)}


def attn_splits_of(max_ctx: int) -> int:
    """Splits of the decode attention at this cache length (384 positions up to 3072, else 512)."""
    sl = 384 if max_ctx <= 3072 else 512
    return -(-max_ctx // sl)


def profile_pass(copies: int, launches: int = 64) -> None:
    """A short fixed workload for hardware-counter runs: `launches` matvecs over
    rotating weight copies, then the calibration kernel (exact Q4_0 dequantization
    of a 1024x4096 matrix: 2,359,296 bytes read, 16,777,216 bytes written per
    launch), whose readings check the counters' byte accounting."""
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

# rocprofv3 passes (each within one pass's limit of 4 TCC counters): the L2's read
# requests to memory by size, then its write requests and FETCH_SIZE's own inputs
TRAFFIC_PASSES = (
    ("TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum", "TCC_EA0_RDREQ_sum"),
    ("TCC_EA0_WRREQ_sum", "TCC_EA0_WRREQ_64B_sum", "TCC_BUBBLE_sum", "TCC_EA0_RDREQ_DRAM_sum"),
)


def _pmc_passes(passes, workload: list[str], kinds: dict, timeout_s: int = 150) -> dict | None:
    """Runs `bench.py <workload>` once per counter pass under rocprofv3 --pmc (a
    child process each) and returns, per kernel kind, the mean of every counter
    over that kind's dispatches and the mean dispatch duration in microseconds
    (`kinds` maps a kind to a predicate on the kernel name).  None when
    rocprofv3 is unavailable or a pass fails."""
    import csv
    import shutil
    import subprocess
    import tempfile

    exe = shutil.which("rocprofv3")
    if exe is None:
        log("rocprofv3 not found: counters not collected")
        return None
    vals: dict[str, dict[str, float]] = {k: {} for k in kinds}
    durs: dict[str, list[float]] = {k: [] for k in kinds}
    env = dict(os.environ, TMPDIR="/tmp")
    with tempfile.TemporaryDirectory(dir="/tmp") as tmp:
        for n, counters in enumerate(passes):
            cmd = [exe, "--pmc", *counters, "--output-format", "csv", "-d", tmp, "-o", f"pass{n}", "--",
                   sys.executable, str(ROOT / "bench.py"), *workload]
            try:
                subprocess.run(cmd, cwd="/tmp", env=env, timeout=timeout_s, check=True,
                               stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
            except (subprocess.SubprocessError, OSError) as e:
                log(f"rocprofv3 pass {n} failed ({e}): counters not collected")
                return None
            files = list(Path(tmp).rglob(f"pass{n}_counter_collection.csv"))
            if not files:
                log(f"rocprofv3 pass {n} wrote no counter file: counters not collected")
                return None
            acc: dict[str, dict[str, list[float]]] = {k: {} for k in kinds}
            seen: set = set()
            with open(files[0]) as f:
                for row in csv.DictReader(f):
                    name, ctr = row["Kernel_Name"], row.get("Counter_Name", "")
                    kind = next((k for k, match in kinds.items() if match(name)), None)
                    if kind is None or ctr not in counters:
                        continue
                    acc[kind].setdefault(ctr, []).append(float(row["Counter_Value"]))
                    if (kind, row["Dispatch_Id"]) not in seen:
                        seen.add((kind, row["Dispatch_Id"]))
                        durs[kind].append((int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3)
            for kind in acc:
                for ctr in counters:
                    if ctr not in acc[kind]:
                        log(f"rocprofv3 pass {n}: {ctr} missing for the {kind} kernel")
                        return None
                    vals[kind][ctr] = float(np.mean(acc[kind][ctr]))
    return {k: {"counters": vals[k], "us": float(np.mean(durs[k])), "dispatches": len(durs[k])} for k in kinds}


HEADLINE_KERNEL = "gguf_mfma_stream<0, 1, 16, 1, 1, 0, false, 16, false, false, false, false>"


def kernel_trace(steps: int = 20, timeout_s: int = 300) -> dict | None:
    """rocprofv3 kernel trace of bench.py's own timed region: the default matvec
    run (`steps` launches queued behind the untimed cover reads, no other legs) in
    a child process under `rocprofv3 --kernel-trace`.  The last `steps` dispatches
    of the headline kernel are the timed launches; their begin/end timestamps give
    each launch's duration in the same back-to-back regime as bench.py's events
    (the tracer's own host work per launch runs while the cover keeps the GPU
    busy, so the timed launches still start back to back).  Returns their mean
    duration next to the child's own HIP-event figure, or None without rocprofv3."""
    import csv
    import shutil
    import subprocess
    import tempfile

    exe = shutil.which("rocprofv3")
    if exe is None:
        log("rocprofv3 not found: kernel trace not taken")
        return None
    env = dict(os.environ, TMPDIR="/tmp")
    workload = ["--steps", str(steps), "--warmup", "5", "--no-extra", "--no-cpu", "--no-traffic", "--no-trace"]
    with tempfile.TemporaryDirectory(dir="/tmp") as tmp:
        cmd = [exe, "--kernel-trace", "--output-format", "csv", "-d", tmp, "-o", "trace", "--",
               sys.executable, str(ROOT / "bench.py"), *workload]
        try:
            out = subprocess.run(cmd, cwd="/tmp", env=env, timeout=timeout_s, check=True, capture_output=True,
                                 text=True).stdout
        except (subprocess.SubprocessError, OSError) as e:
            log(f"rocprofv3 kernel trace failed ({e})")
            return None
        files = list(Path(tmp).rglob("trace_kernel_trace.csv"))
        if not files:
            log("rocprofv3 wrote no kernel trace")
            return None
        with open(files[0]) as f:
            rows = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in csv.DictReader(f)
                    if HEADLINE_KERNEL in r["Kernel_Name"]]
    rows.sort()
    if len(rows) < steps:
        log(f"kernel trace holds {len(rows)} headline dispatches, fewer than {steps}")
        return None
    try:
        child = json.loads(out.strip().splitlines()[-1])
    except (ValueError, IndexError):
        child = {}
    timed = rows[-steps:]
    dur = np.array([(e - b) / 1e3 for b, e in timed])
    gaps = np.array([(timed[i + 1][0] - timed[i][1]) / 1e3 for i in range(steps - 1)])
    bytes_step = q4_algorithmic_bytes(M_MAIN, K_MAIN)
    mean = float(dur.mean())
    return {"command": "rocprofv3 --kernel-trace -- python3 bench.py " + " ".join(workload),
            "kernel": HEADLINE_KERNEL, "dispatches_traced": len(rows), "timed_dispatches": steps,
            "us_mean": round(mean, 3), "us_median": round(float(np.median(dur)), 3),
            "us_min": round(float(dur.min()), 3), "us_max": round(float(dur.max()), 3),
            "gap_us_mean": round(float(gaps.mean()), 3), "gap_us_max": round(float(gaps.max()), 3),
            "frac_at_trace_mean": round(bytes_step / mean / 1e3 / HBM_PEAK_GBPS, 4),
            "child_events_us_per_step": round(child["ms_per_step"] * 1e3, 3) if "ms_per_step" in child else None}


def measure_traffic(timeout_s: int = 150) -> dict | None:
    """HBM bytes per matvec launch from the L2's memory requests counted by size:
    read = 32 RDREQ_32B + 64 RDREQ_64B + 128 RDREQ_128B, written = 64 WRREQ_64B +
    32 (WRREQ - WRREQ_64B), per dispatch (two rocprofv3 --pmc passes over
    `--profile-pass`, run as child processes).  FETCH_SIZE's own formula
    (128 TCC_BUBBLE + 64 (RDREQ - BUBBLE - RDREQ_32B) + 32 RDREQ_32B) is evaluated
    from the same counts beside it: it prices a 128-byte request at 64 bytes when
    the request is not counted as a bubble, which is where FETCH_SIZE's shortfall
    comes from.  The calibration dequantize (known bytes) checks the accounting.
    Returns None when rocprofv3 is unavailable or fails."""
    res = _pmc_passes(TRAFFIC_PASSES, ["--profile-pass"],
                      {"matvec": lambda n: "gguf_mfma_stream" in n or "q4_matvec" in n,
                       "cal": lambda n: "dequant_kernel" in n}, timeout_s)
    if res is None:
        log("traffic not measured")
        return None
    vals = {k: res[k]["counters"] for k in res}

    def account(v):
        read = 32 * v["TCC_EA0_RDREQ_32B_sum"] + 64 * v["TCC_EA0_RDREQ_64B_sum"] + 128 * v["TCC_EA0_RDREQ_128B_sum"]
        written = 64 * v["TCC_EA0_WRREQ_64B_sum"] + 32 * (v["TCC_EA0_WRREQ_sum"] - v["TCC_EA0_WRREQ_64B_sum"])
        fetch = (128 * v["TCC_BUBBLE_sum"] + 64 * (v["TCC_EA0_RDREQ_sum"] - v["TCC_BUBBLE_sum"] -
                                                   v["TCC_EA0_RDREQ_32B_sum"]) + 32 * v["TCC_EA0_RDREQ_32B_sum"])
        return read, written, fetch

    read, written, fetch = account(vals["matvec"])
    cal_read, cal_written, cal_fetch = account(vals["cal"])
    return {
        "bytes": read + written,
        "read_bytes": read,
        "written_bytes": written,
        "fetch_size_formula_bytes": fetch,
        "rdreq_dram": vals["matvec"]["TCC_EA0_RDREQ_DRAM_sum"],
        "counters": vals["matvec"],
        "calibration": {"read_bytes": cal_read, "expected_read": CAL_READ_BYTES, "written_bytes": cal_written,
                        "expected_written": CAL_WRITE_BYTES, "fetch_size_formula_bytes": cal_fetch},
    }


def gemm_profile_pass(T: int = 512, M: int = 11008, K: int = 4096, copies: int = 6, launches: int = 24) -> None:
    """A short fixed GEMM workload for hardware-counter runs: `launches` Q8_0
    GEMMs C[T][M] = A_q8[T][K] . W_q8[M][K]^T over rotating weight copies."""
    from asmllm_amd import gguf, native
    from asmllm_amd.device import DeviceBuffer, Stream

    lib = native.lib()
    wbufs, _ = _rotating_blocks(native.Q8_0, M, K, copies, seed=99)
    dq = DeviceBuffer(gguf.q8_0_nbytes(T, K))
    native.check(lib.asmhip_random_blocks(native.Q8_0, dq.ptr, T, K, 5, 1.0, None), "random activations")
    dc = DeviceBuffer(4 * T * M)
    stream = Stream()
    # the tile layout (the headline form)
    wtiled = [DeviceBuffer(lib.asmhip_gemm_q8_0_tiled_weight_bytes(M, K)) for _ in range(copies)]
    for b, wt in zip(wbufs, wtiled):
        native.check(lib.asmhip_gemm_q8_0_tile_weights(b.ptr, wt.ptr, M, K, stream.handle), "tile weights")
    dqt = DeviceBuffer(lib.asmhip_gemm_q8_0_tiled_activation_bytes(T, K))
    native.check(lib.asmhip_gemm_q8_0_tile_activations(dq.ptr, dqt.ptr, T, K, stream.handle), "tile activations")
    for i in range(launches):
        native.check(lib.asmhip_gemm_q8_0_tiled(wtiled[i % copies].ptr, dqt.ptr, dc.ptr, T, M, K, stream.handle),
                     "gemm tiled")
    stream.synchronize()
    for b in wtiled:
        b.close()
    for i in range(launches):
        native.check(lib.asmhip_gemm_q8_0(wbufs[i % copies].ptr, dq.ptr, dc.ptr, T, M, K, stream.handle), "gemm")
    # the same product on split operands (int8 qs planes + fp32 scale planes)
    nb = K // 32
    w0 = wbufs[0].download(np.uint8, (M, nb, 34))
    a0 = dq.download(np.uint8, (T, nb, 34))
    planes = [DeviceBuffer.from_numpy(v) for v in (
        np.ascontiguousarray(w0[:, :, 2:]).view(np.int8), w0[:, :, 0:2].copy().view(np.float16).reshape(M, nb).astype(np.float32),
        np.ascontiguousarray(a0[:, :, 2:]).view(np.int8), a0[:, :, 0:2].copy().view(np.float16).reshape(T, nb).astype(np.float32))]
    for b in wbufs[1:]:
        b.close()
    wsplit = [(planes[0], planes[1])]
    for _ in range(copies - 1):
        q, sc = DeviceBuffer(planes[0].nbytes), DeviceBuffer(planes[1].nbytes)
        q.copy_from(planes[0])
        sc.copy_from(planes[1])
        wsplit.append((q, sc))
    for i in range(launches):
        q, sc = wsplit[i % copies]
        native.check(lib.asmhip_gemm_q8_split(q.ptr, sc.ptr, planes[2].ptr, planes[3].ptr, dc.ptr, T, M, K,
                                              stream.handle), "gemm split")
    stream.synchronize()
    log(f"GEMM profile pass: {launches} launches of each form ({T}x{M}x{K})")


# rocprofv3 passes for the GEMM (each within one pass's limit of 8 SQ and 2 GRBM
# counters): matrix-core and VALU issue, then the VALU mix, LDS and waits
GEMM_PASSES = (
    ("SQ_BUSY_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU", "SQ_INSTS_VALU_MFMA_MOPS_I8", "SQ_INSTS_MFMA",
     "SQ_ACTIVE_INST_VALU", "SQ_WAVES", "SQ_INSTS_LDS", "GRBM_GUI_ACTIVE"),
    ("SQ_INSTS_VALU_CVT", "SQ_INSTS_VALU_FMA_F32", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_WAIT_INST_ANY",
     "SQ_WAVE_CYCLES", "SQ_INSTS_SALU", "SQ_INSTS_VALU_MFMA_MOPS_F16", "GRBM_GUI_ACTIVE"),
    # the staging path: L1 -> L2 read requests (64-byte lines), L2 hits and misses, texture-address busy
    ("TCP_TCC_READ_REQ_sum", "TCC_HIT_sum", "TCC_MISS_sum", "TA_TA_BUSY_sum", "GRBM_GUI_ACTIVE"),
)


def gemm_counters(T: int = 512, M: int = 11008, K: int = 4096, timeout_s: int = 150) -> dict | None:
    """Hardware counters of the Q8_0 GEMM per dispatch and what they give:
    matrix-core busy fraction, int8 ops counted by the hardware (MOPS_I8 x 512)
    against 2 T M K, VALU instructions per 32x32 output tile and block, the shader
    clock (GUI-active cycles per XCD over the dispatch's duration); for the
    tile-layout kernel and, under "block_layout" and "split_layout", the GGUF-block
    and split-operand ones."""
    res = _pmc_passes(GEMM_PASSES, ["--gemm-profile-pass"],
                      {"gemm": lambda n: "gemm_q8_0_tiled" in n, "block": lambda n: "gemm_q8_0_coalesced" in n,
                       "split": lambda n: "gemm_q8_split" in n}, timeout_s)
    if res is None:
        return None
    out = _gemm_derived(res["gemm"], T, M, K)
    for key, name, bb in (("block", "block_layout", 34), ("split", "split_layout", 36)):
        if key in res:
            out[name] = _gemm_derived(res[key], T, M, K, bb)
    return out


def _gemm_derived(r: dict, T: int, M: int, K: int, block_bytes: int = 34) -> dict:
    from asmllm_amd.device import device_info

    v, us = r["counters"], r["us"]
    cus = device_info()["compute_units"]
    simds, xcds = 4 * cus, 8
    gui = v["GRBM_GUI_ACTIVE"] / xcds  # summed over the XCDs' GRBMs
    block_tiles = (T // 32) * (M // 32) * (K // 32)
    ops = 2 * T * M * K
    return {
        "workload": f"Q8_0 GEMM C[{T}][{M}] = A_q8[{T}][{K}] . W_q8[{M}][{K}]^T, eager launches",
        "dispatch_us": round(us, 3),
        "dispatches": r["dispatches"],
        "counters": {k: round(x, 1) for k, x in v.items()},
        "gui_cycles": round(gui, 0),
        "shader_clock_ghz": round(gui / us / 1e3, 3),
        "mfma_busy_frac": round(v["SQ_VALU_MFMA_BUSY_CYCLES"] / (gui * simds), 4),
        "int8_ops_counted": v["SQ_INSTS_VALU_MFMA_MOPS_I8"] * 512,
        "int8_ops_expected": ops,
        "int8_TOPs": round(ops / us / 1e6, 1),
        "valu_insts_per_block_tile": round(v["SQ_INSTS_VALU"] / block_tiles, 2),
        "cvt_per_block_tile": round(v["SQ_INSTS_VALU_CVT"] / block_tiles, 2),
        "fma_f32_per_block_tile": round(v["SQ_INSTS_VALU_FMA_F32"] / block_tiles, 2),
        "mfma_per_block_tile": round(v["SQ_INSTS_MFMA"] / block_tiles, 2),
        "lds_insts_per_block_tile": round(v["SQ_INSTS_LDS"] / block_tiles, 2),
        "valu_issue_frac": round(4 * v["SQ_INSTS_VALU"] / (gui * simds), 4),
        "lds_bank_conflict_frac_of_lds_active": round(v["SQ_LDS_BANK_CONFLICT"] / max(v["SQ_LDS_IDX_ACTIVE"], 1), 4),
        "l2_read_requests": round(v["TCP_TCC_READ_REQ_sum"], 0),
        "l2_read_requests_per_64_staged_bytes": round(
            64 * v["TCP_TCC_READ_REQ_sum"] / _gemm_staged_bytes(T, M, K, block_bytes), 3),
        "l2_hit_rate": round(v["TCC_HIT_sum"] / max(v["TCC_HIT_sum"] + v["TCC_MISS_sum"], 1), 4),
        "ta_busy_frac": round(v["TA_TA_BUSY_sum"] / (cus * gui), 4),
    }


def _gemm_staged_bytes(T: int, M: int, K: int, block_bytes: int = 34, tt: int = 64, tm: int = 128) -> int:
    """Operand bytes the 64 x 128 workgroup tiles stage from L2 in all: every
    tile reads its 64 A rows and 128 W rows over the whole of K (block_bytes a
    block: 34 in GGUF blocks, 36 as split int8 qs + an fp32 scale)."""
    tiles = -(-T // tt) * -(-M // tm)
    return tiles * (tt + tm) * (K // 32) * block_bytes


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
    ap.add_argument("--gemm-profile-pass", action="store_true",
                    help="run only a short fixed GEMM workload for hardware-counter collection")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 counter passes")
    ap.add_argument("--no-trace", action="store_true", help="skip the rocprofv3 kernel trace of the timed region")
    ap.add_argument("--no-extra", action="store_true", help="skip the shape table, GEMM and decode legs")
    ap.add_argument("--only", choices=["decode", "gemm", "table", "floor", "host", "cpu", "traffic", "gemm_counters",
                                       "phases", "trace", "stamps", "decode_launches"],
                    help="run one extra leg and print its JSON")
    ap.add_argument("--eager", action="store_true", help="with --only: launch without graphs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this build has no multi-GPU path)",
              file=sys.stderr)
        raise SystemExit(2)

    if args.profile_pass:
        profile_pass(args.copies)
        return
    if args.gemm_profile_pass:
        gemm_profile_pass()
        return

    from asmllm_amd.device import device_info

    if args.only:
        global EAGER
        EAGER = args.eager
        if args.only == "decode":
            res = bench_decode(eager=args.eager, cpu_seconds=0.0 if args.no_cpu else args.cpu_seconds)
        elif args.only == "cpu":
            res = bench_cpu_baseline(args.cpu_seconds)
        else:
            res = {"gemm": bench_gemm, "table": bench_matvec_table, "floor": bench_read_floor,
                   "host": bench_host_pointer, "traffic": measure_traffic,
                   "gemm_counters": gemm_counters, "phases": bench_matvec_phases,
                   "trace": kernel_trace, "stamps": bench_stamps,
                   "decode_launches": bench_decode_launches}[args.only]()
        print(json.dumps({args.only: res}), flush=True)
        return

    info = device_info()
    log(f"device {info['arch']} with {info['compute_units']} CUs")
    mv = bench_matvec(args.steps, args.warmup, args.copies)
    achieved = mv["bytes_per_step"] / (mv["kernel_us_mean"] * 1e-6) / 1e9
    extra = {}
    if not args.no_extra:
        extra["read_floor"] = bench_read_floor()
        extra["decode"] = bench_decode(cpu_seconds=0.0 if args.no_cpu else args.cpu_seconds)
        extra["gemm"] = bench_gemm()
        extra["matvec_table"] = bench_matvec_table()
        extra["host_pointer"] = bench_host_pointer()
    cpu = None if args.no_cpu else bench_cpu_baseline(args.cpu_seconds)
    if cpu is not None and not args.no_extra:
        best = max(cpu["sweep"], key=lambda p: p["GBps"])
        variant = 1 if best["kernel"] == "avx512" else 0
        extra["cpu_table"] = cpu_table_baselines(extra["matvec_table"], best["threads"], variant)
        cpu_gemm_baseline(extra["gemm"], best["threads"])
    traffic = None if args.no_traffic else measure_traffic()
    trace = None if args.no_trace else kernel_trace()

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
            "kernel": "gguf_mfma_stream<0,1,16,1,1,0,false,16,false,false,false,false> (int8 MFMA, GGUF Q4_0)",
            "kernel_us_mean": round(mv["kernel_us_mean"], 3),
            "event_bracket_us": round(mv["event_bracket_us"], 3),
            "fp32_valu_kernel_us_mean": round(mv["fp32_kernel_us_mean"], 3),
            "bytes_per_launch": mv["bytes_per_step"],
            "kernel_trace": trace,
        },
        "cpu_baseline": cpu,
        "parity_max_err_over_l1": mv["parity_max_err_over_l1"],
    }
    result.update(extra)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
