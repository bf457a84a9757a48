"""Benchmark of the MI355X hip backend on BASELINE.json's metric.

Headline (``value``): fp32 GEMM 8192^3 GFLOP/s through ``a @ b`` (config 4),
inputs resident in HBM, one step = one product. ``extra`` holds the other
hot-path workloads of the metric ("+ GEMV/norm HBM GB/s") and the remaining
configs (GEMV/DOT, scaled norms, RNG, fp64/padded/batched GEMM, compiled MLP),
each with its roofline fraction. Kernel durations come from HIP events
recorded on the library's stream around the timed region.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu] [--only NAME,...]
Prints ONE JSON line on stdout; progress goes to stderr.
"""

import argparse
import ctypes
import gc
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _path in (str(ROOT / "open-pacho_amd"), str(ROOT)):
    if _path not in sys.path:
        sys.path.insert(0, _path)

import numpy as np  # noqa: E402

METRIC = "fp32 GEMM GFLOP/s @8192³ + GEMV/norm HBM GB/s, % of MI355X roofline"
PEAK_HBM_GBS = 8000.0
PEAK_FP32_TFLOPS = 157.3
PEAK_FP64_TFLOPS = 78.6
# Untimed load before each extra workload. The MI355X raises its compute
# clock only after some tens of milliseconds of sustained work: after an idle
# second, 2 warm-up calls left fp64 4096^3 at 77-79% of peak against 85% once
# warm, and the RNG at ~700 against ~900 Gsample/s.
WARM_MS = 100.0


def log(message):
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def warm(fn, synchronize, calls):
    """Untimed calls: at least ``calls`` of them and at least WARM_MS of
    device work, so that the timed region starts at the sustained clock.

    Calls are queued in batches of about 5 ms of device work, synchronized
    only between batches: with a synchronization after every call a ~0.3 ms
    kernel left the device idle a tenth of the time, and the timed region
    then started below the sustained clock (2^28 float32 uniform samples:
    kernels of 321 us right after such a warm-up, 293 us once loaded)."""
    t0 = time.perf_counter()
    fn()
    synchronize()
    batch = max(1, int(5e-3 / max(time.perf_counter() - t0, 1e-6)))
    done = 1
    while done < calls or (time.perf_counter() - t0) * 1e3 < WARM_MS:
        for _ in range(batch):
            fn()
        done += batch
        synchronize()


class Timer:
    """HIP events on the backend stream around a region of repeated calls.

    One untimed call is queued ahead of the start event, so the device is
    busy when the region opens: the first timed call's host-side preparation
    overlaps device work, and the events bracket the device time of exactly
    the timed calls. (Opened on an idle device, the region also counted that
    preparation: about 160 us of a 15 ms region of the odd-shape product
    under a kernel trace.) A host-bound call still measures its host time:
    the device then waits for each submission. ``wall`` is the host time per
    call over the untimed call and the timed ones.
    """

    def __init__(self, backend):
        self.backend = backend
        lib, ctx = backend._lib, backend._ctx
        self.start, self.stop = ctypes.c_void_p(), ctypes.c_void_p()
        assert lib.hp_event_create(ctx, ctypes.byref(self.start)) == 0
        assert lib.hp_event_create(ctx, ctypes.byref(self.stop)) == 0

    def run(self, fn, reps, warmup=2):
        lib, ctx = self.backend._lib, self.backend._ctx
        warm(fn, self.backend.synchronize, warmup)
        # As timeit does: no garbage-collection pass inside the timed region
        # (a pass while the stream is empty shows up as device idle time).
        gc.collect()
        gc.disable()
        try:
            wall0 = time.perf_counter()
            fn()
            lib.hp_event_record(ctx, self.start)
            for _ in range(reps):
                fn()
            lib.hp_event_record(ctx, self.stop)
            self.backend.synchronize()
        finally:
            gc.enable()
        wall = (time.perf_counter() - wall0) * 1e3 / (reps + 1)
        ms = ctypes.c_float()
        assert lib.hp_event_elapsed_ms(self.start, self.stop, ctypes.byref(ms)) == 0
        return ms.value / reps, wall


def roofline(bound, work, ms, traffic=None):
    if bound == "hbm":
        achieved = work / (ms * 1e-3) / 1e9
        peak, unit = PEAK_HBM_GBS, "GB/s"
    else:
        achieved = work / (ms * 1e-3) / 1e12
        peak, unit = (PEAK_FP64_TFLOPS if bound == "mfma_fp64" else PEAK_FP32_TFLOPS), "TFLOP/s"
        bound = "mfma"
    return {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit, "frac": round(achieved / peak, 4), "traffic": traffic}


def _traffic(name):
    """HBM bytes per launch measured by rocprofv3 --pmc (profiles/traffic.json), if recorded."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(name, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


# Vector-ALU issue peak: 256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz, in lane
# instructions per second (a wave64 instruction occupies a SIMD 4 cycles).
# Transcendental instructions (v_log/v_sqrt/v_cos) run on gfx950's separate
# transcendental unit while the VALU keeps issuing, so only the other VALU
# instructions count against this peak (PMC: counting the transcendentals too
# puts the normal kernel at 102% of issue, without them at 96%).
PEAK_VALU_TINSTR = 256 * 4 * 16 * 2.4e9 / 1e12


def _valu(name, samples, ms):
    """Vector-ALU issue roofline of an RNG kernel from its PMC instruction
    counts (profiles/valu.json): non-transcendental VALU instructions per
    sample x samples / time, against the issue peak."""
    path = ROOT / "profiles" / "valu.json"
    try:
        entry = json.loads(path.read_text())[name]
        per_sample = entry["valu_issue_per_sample"]
    except (OSError, ValueError, KeyError):
        return None
    achieved = per_sample * samples / (ms * 1e-3) / 1e12
    return {"bound": "valu", "instr_per_sample": per_sample, "trans_per_sample": entry.get("valu_trans_per_sample"),
            "achieved": round(achieved, 2), "peak": round(PEAK_VALU_TINSTR, 2), "unit": "Tinstr/s",
            "frac": round(achieved / PEAK_VALU_TINSTR, 4)}


def cpu_threads():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_timed(fn, min_calls=7, min_seconds=0.0):
    """The CPU baseline protocol: warm-up of at least 3 calls and 0.25 s, then
    the median of at least ``min_calls`` timed calls (and ``min_seconds``)."""
    t0, calls = time.perf_counter(), 0
    while calls < 3 or time.perf_counter() - t0 < 0.25:
        fn()
        calls += 1
    times, t1 = [], time.perf_counter()
    while len(times) < min_calls or time.perf_counter() - t1 < min_seconds:
        start = time.perf_counter()
        fn()
        times.append(time.perf_counter() - start)
    return statistics.median(times), len(times)


def blas_threads(count):
    """Limit NumPy's BLAS to ``count`` threads inside a with-block."""
    from threadpoolctl import threadpool_limits

    return threadpool_limits(limits=count, user_api="blas")


def cpu_blas_seconds(fn, min_seconds=0.0):
    """Median seconds per call of a BLAS-backed ``fn`` at every core the
    process may use and at 1 thread: (cores, seconds, calls, seconds_1, calls_1)."""
    cores = cpu_threads()
    with blas_threads(cores):
        sec, calls = cpu_timed(fn, min_seconds=min_seconds)
    with blas_threads(1):
        sec1, calls1 = cpu_timed(fn)
    return cores, sec, calls, sec1, calls1


def cpu_blas(fn, work, unit, sample, min_seconds=0.0):
    """A BLAS-backed CPU leg at every core the process may use and at 1 thread.
    ``work`` is the algorithmic flop or byte count of one call of ``fn``."""
    scale = 1e9
    cores, sec, calls, sec1, calls1 = cpu_blas_seconds(fn, min_seconds)
    return {
        "value": round(work / sec / scale, 3),
        "unit": unit,
        "cores": cores,
        "kind": "port",
        "sample": f"{sample}; median of {calls} calls",
        "one_thread": {"value": round(work / sec1 / scale, 3), "unit": unit, "cores": 1, "calls": calls1},
    }


def cpu_single(fn, work, unit, sample, scale=1e9):
    """A single-threaded NumPy elementwise CPU leg (the norm and RNG restatements)."""
    sec, calls = cpu_timed(fn)
    return {
        "value": round(work / sec / scale, 4),
        "unit": unit,
        "cores": 1,
        "kind": "port",
        "sample": f"{sample}; single-threaded NumPy; median of {calls} calls",
    }


def strict_json(value):
    """Non-finite floats become strings, so the line is strict JSON (the
    convention of reference benchmarks/numerical_metrics.py:13-18)."""
    if isinstance(value, dict):
        return {k: strict_json(v) for k, v in value.items()}
    if isinstance(value, (list, tuple)):
        return [strict_json(v) for v in value]
    if isinstance(value, float) and not np.isfinite(value):
        return str(value)
    return value


def bench_gemm(p, hip, steps, warmup):
    n = 8192
    rng = p.random.default_rng(3, backend=hip)
    a = rng.uniform(-1, 1, (n, n), dtype="float32")
    b = rng.uniform(-1, 1, (n, n), dtype="float32")
    timer = Timer(hip)
    for _ in range(warmup):
        a @ b
    hip.synchronize()
    gc.collect()
    gc.disable()
    try:
        wall0 = time.perf_counter()
        lib, ctx = hip._lib, hip._ctx
        lib.hp_event_record(ctx, timer.start)
        for _ in range(steps):
            c = a @ b
        lib.hp_event_record(ctx, timer.stop)
        hip.synchronize()
    finally:
        gc.enable()
    wall_ms = (time.perf_counter() - wall0) * 1e3 / steps
    ms = ctypes.c_float()
    lib.hp_event_elapsed_ms(timer.start, timer.stop, ctypes.byref(ms))
    kernel_ms = ms.value / steps
    flops = 2.0 * n**3
    del c
    return {"a": a, "b": b, "flops": flops, "kernel_ms": kernel_ms, "wall_ms": wall_ms}


def cpu_gemm_baseline(p, gemm):
    """np.matmul (the reference NumPy backend's path) on a row sample of the
    same product: about 10 s at every core, plus a 64-row sample at 1 thread."""
    from oracle import numpy_backend

    rows = int(os.environ.get("PACHO_BENCH_CPU_ROWS", "1024"))
    a = p.asnumpy(gemm["a"][:rows])
    b = p.asnumpy(gemm["b"])
    cores = cpu_threads()
    with blas_threads(cores):
        sec, calls = cpu_timed(lambda: numpy_backend.matmul(a, b), min_seconds=10.0)
    with blas_threads(1):
        sec1, calls1 = cpu_timed(lambda: numpy_backend.matmul(a[:64], b))
    return {
        "value": round(2.0 * rows * 8192 * 8192 / sec / 1e9, 2),
        "unit": "GFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": f"np.matmul float32 A[:{rows}] @ B (8192x8192) at {cores} BLAS threads; median of {calls} calls",
        "one_thread": {"value": round(2.0 * 64 * 8192 * 8192 / sec1 / 1e9, 2), "unit": "GFLOP/s", "cores": 1, "sample": "A[:64] @ B", "calls": calls1},
    }


def vendor_gemm():
    """The vendor BLAS on the headline shapes, for comparison only.

    Runs ``bench.py --vendor-child`` as a child process: PyTorch's ROCm build
    brings its own HIP runtime, which finds no GPU in a process that has
    already loaded the hip backend's library (built against /opt/rocm). Never
    feeds ``value``.
    """
    import subprocess

    try:
        child = subprocess.run(
            [sys.executable, os.path.abspath(__file__), "--vendor-child"],
            capture_output=True, text=True, timeout=240,
        )
    except subprocess.TimeoutExpired:
        log("vendor: child timed out; skipped")
        return {}
    if child.returncode != 0 or not child.stdout.strip():
        log(f"vendor: child exited {child.returncode}: {child.stderr.strip()[-300:]}")
        return {}
    return json.loads(child.stdout.strip().splitlines()[-1])


def vendor_gemm_child():
    """PyTorch's fp32/fp64 matmul on ROCm (hipBLASLt or rocBLAS; full fp32,
    TF32 off) on 8192^3 / 4096^3, timed with events on torch's stream."""
    try:
        import torch
    except ImportError as error:
        log(f"vendor: torch not importable ({error}); skipped")
        return {}
    if not torch.cuda.is_available():
        log("vendor: torch sees no GPU; skipped")
        return {}
    torch.backends.cuda.matmul.allow_tf32 = False
    out = {}
    for name, n, dtype, peak in (
        ("vendor_gemm_f32_8192", 8192, torch.float32, PEAK_FP32_TFLOPS),
        ("vendor_gemm_f64_4096", 4096, torch.float64, PEAK_FP64_TFLOPS),
    ):
        generator = torch.Generator(device="cuda").manual_seed(3)
        a = torch.rand((n, n), device="cuda", dtype=dtype, generator=generator) * 2 - 1
        b = torch.rand((n, n), device="cuda", dtype=dtype, generator=generator) * 2 - 1
        warm(lambda: torch.matmul(a, b), torch.cuda.synchronize, 3)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 10
        c = torch.matmul(a, b)  # untimed, queued ahead of the start event (as Timer.run)
        start.record()
        for _ in range(reps):
            c = torch.matmul(a, b)
        stop.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(stop) / reps
        tflops = 2.0 * n**3 / (ms * 1e-3) / 1e12
        out[name] = {
            "value": round(tflops * 1e3, 1),
            "unit": "GFLOP/s",
            "kernel_ms": round(ms, 4),
            "frac_of_peak": round(tflops / peak, 4),
            "library": "torch.matmul on ROCm (hipBLASLt/rocBLAS), full precision",
        }
        del a, b, c
        torch.cuda.empty_cache()
    return out


def bench_extras(p, hip, only, skip_cpu):
    from oracle import numpy_backend

    timer = Timer(hip)
    extra = {}
    # CPU legs run after every GPU timing: a BLAS call leaves its threads
    # spinning for a while, which slowed the launching thread of the next
    # GPU workload (the compiled MLP: 85% against 90% of peak). Host copies
    # of the inputs are taken right away, the CPU work is queued here.
    legs = []

    def later(fn):
        legs.append(fn)

    def begin(name):
        # Whether workload `name` is selected; a selected workload starts
        # from an empty allocation cache: its operands
        # are then fresh allocations whatever ran before (after the whole
        # bench had cached ~11 GB of other sizes, the compiled MLP measured
        # 86-90% of peak from one run to the next, 90% from an empty cache).
        selected = not only or name in only
        if selected:
            hip.release_cached_memory()
        return selected

    def hbm(key, bytes_moved, ms, wall, traffic_key):
        extra[key] = {
            "value": round(bytes_moved / (ms * 1e-3) / 1e9, 1),
            "unit": "GB/s",
            "kernel_us": round(ms * 1e3, 2),
            "wall_us": round(wall * 1e3, 2),
            "roofline": roofline("hbm", bytes_moved, ms, _traffic(traffic_key)),
        }

    def mfma(key, flops, ms, traffic_key, bound="mfma"):
        extra[key] = {
            "value": round(flops / (ms * 1e-3) / 1e9, 1),
            "unit": "GFLOP/s",
            "kernel_ms": round(ms, 4),
            "roofline": roofline(bound, flops, ms, _traffic(traffic_key)),
        }

    if begin("gemv"):
        n = 16384
        rng = p.random.default_rng(1, backend=hip)
        A = rng.uniform(-1, 1, (n, n), dtype="float32")
        x = rng.normal(0, 1, n, dtype="float32")
        ms, wall = timer.run(lambda: A @ x, 50)
        hbm("gemv_f32_16384", n * n * 4 + 2 * n * 4, ms, wall, "gemv")
        ms, wall = timer.run(lambda: p.dot(x, x), 1000)  # ~4.5 ms of host-bound calls
        extra["dot_f32_16384"] = {"value": round(ms * 1e3, 2), "unit": "us", "wall_us": round(wall * 1e3, 2)}
        if not skip_cpu:
            rows = 4096
            host_a, host_x = p.asnumpy(A[:rows]), p.asnumpy(x)

            def gemv_legs(host_a=host_a, host_x=host_x, rows=rows, n=n):
                extra["gemv_f32_16384"]["cpu_baseline"] = cpu_blas(
                    lambda: numpy_backend.matmul(host_a, host_x), rows * n * 4 + (rows + n) * 4, "GB/s",
                    f"np.matmul float32 A[:{rows}] @ x (n=16384)")
                batch = 100  # calls per timing: one call is a few microseconds
                cores, sec, calls, sec1, calls1 = cpu_blas_seconds(
                    lambda: [numpy_backend.matmul(host_x, host_x) for _ in range(batch)])
                extra["dot_f32_16384"]["cpu_baseline"] = {
                    "value": round(sec / batch * 1e6, 3), "unit": "us", "cores": cores, "kind": "port",
                    "sample": f"np.matmul(x, x), n=16384; median of {calls} timings of {batch} calls",
                    "one_thread": {"value": round(sec1 / batch * 1e6, 3), "unit": "us", "cores": 1, "calls": calls1},
                }

            later(gemv_legs)
            del host_a, host_x
        del A
    if begin("norm"):
        n = 1 << 28
        for dtype, decades in (("float32", 30.0), ("float64", 300.0)):
            rng = p.random.default_rng(2, backend=hip)
            mags = p.power(10.0 if dtype == "float64" else np.float32(10.0), rng.uniform(-decades, decades, n, dtype=dtype))
            signs = rng.random(n, dtype=dtype) < 0.5
            x = p.where(signs, -mags, mags)
            del mags, signs
            ms, wall = timer.run(lambda: p.linalg.norm(x), 30)
            key = f"norm_flat_{dtype}_2^28"
            hbm(key, n * np.dtype(dtype).itemsize, ms, wall, f"norm_{dtype}")
            if not skip_cpu:
                sample = p.asnumpy(x[: 1 << 22])
                later(lambda key=key, sample=sample, dtype=dtype: extra[key].__setitem__("cpu_baseline", cpu_single(
                    lambda: numpy_backend.norm(sample), sample.nbytes, "GB/s", f"two-pass NumPy norm of 2^22 {dtype}")))
            del x
        rows = p.random.default_rng(2, backend=hip).uniform(-1, 1, (65536, 4096), dtype="float32")
        ms, wall = timer.run(lambda: p.linalg.norm(rows, axis=1), 30)
        hbm("norm_rows_f32_65536x4096", 65536 * 4096 * 4 + 65536 * 4, ms, wall, "norm_rows")
        if not skip_cpu:
            sample = p.asnumpy(rows[:1024])
            later(lambda sample=sample: extra["norm_rows_f32_65536x4096"].__setitem__("cpu_baseline", cpu_single(
                lambda: numpy_backend.norm(sample, axis=1), sample.nbytes + 1024 * 4, "GB/s",
                "two-pass NumPy norm, axis=1, of 1024x4096 float32")))
        del rows
    if begin("strided"):
        rows, cols = 262144, 1024
        data = p.random.default_rng(3, backend=hip).uniform(-1, 1, (rows, cols), dtype="float32")
        bytes_moved = rows * cols * 4 + cols * 4
        sample = p.asnumpy(data[:16384]) if not skip_cpu else None
        for name, fn, host_fn in (
            ("sum", lambda: p.sum(data, axis=0), lambda: np.sum(sample, axis=0)),
            ("max", lambda: p.max(data, axis=0), lambda: np.max(sample, axis=0)),
            ("norm", lambda: p.linalg.norm(data, axis=0), lambda: numpy_backend.norm(sample, axis=0)),
        ):
            ms, wall = timer.run(fn, 30)
            key = f"{name}_axis0_f32_262144x1024"
            hbm(key, bytes_moved, ms, wall, f"strided_{name}")
            if sample is not None:
                later(lambda key=key, host_fn=host_fn, name=name, nbytes=sample.nbytes + cols * 4: extra[key].__setitem__(
                    "cpu_baseline", cpu_single(host_fn, nbytes, "GB/s", f"NumPy {name} over axis 0 of a 16384x1024 float32 sample")))
        del data
    if begin("rng"):
        n = 1 << 28
        for dist in ("uniform", "normal", "exponential"):
            rng = p.random.default_rng(42, backend=hip)
            ms, wall = timer.run(lambda: getattr(rng, dist)(size=n, dtype="float32"), 100)
            key = f"rng_{dist}_f32_2^28"
            extra[key] = {
                "value": round(n / (ms * 1e-3) / 1e9, 2),
                "unit": "Gsample/s",
                "kernel_us": round(ms * 1e3, 2),
                "roofline": roofline("hbm", n * 4, ms, _traffic(f"rng_{dist}")),
                "valu_roofline": _valu(f"rng_{dist}", n, ms),
                "alu_bound_note": "vector-ALU issue bound: one Philox4x32-10 block per sample = ~17 v_mad_u64_u32 + ~17 three-input XORs (v_bitop3_b32) per sample",
            }
            if not skip_cpu:
                count = 1 << 20
                later(lambda key=key, dist=dist, count=count: extra[key].__setitem__("cpu_baseline", cpu_single(
                    lambda: numpy_backend.random(dist, "float32", (count,), 42), count, "Gsample/s",
                    f"NumPy Philox {dist} float32, 2^20 samples")))
    if begin("gemm_f64"):
        n = 4096
        rng = p.random.default_rng(3, backend=hip)
        a = rng.uniform(-1, 1, (n, n), dtype="float64")
        b = rng.uniform(-1, 1, (n, n), dtype="float64")
        ms, wall = timer.run(lambda: a @ b, 10)
        mfma("gemm_f64_4096", 2.0 * n**3, ms, "gemm_f64", bound="mfma_fp64")
        if not skip_cpu:
            ha, hb = p.asnumpy(a[:512]), p.asnumpy(b)
            later(lambda ha=ha, hb=hb, n=n: extra["gemm_f64_4096"].__setitem__("cpu_baseline", cpu_blas(
                lambda: numpy_backend.matmul(ha, hb), 2.0 * 512 * n * n, "GFLOP/s", "np.matmul float64 A[:512] @ B (4096x4096)")))
        del a, b
    if begin("gemm_padded"):
        m, k, n = 4097, 3001, 2049
        rng = p.random.default_rng(3, backend=hip)
        a = rng.uniform(-1, 1, (m, k), dtype="float32")
        b = rng.uniform(-1, 1, (k, n), dtype="float32")
        flops = 2.0 * m * n * k
        ms, wall = timer.run(lambda: p.matmul(a, b, padding=True), 40)
        mfma("gemm_f32_4097x3001x2049_padded", flops, ms, "gemm_padded")
        ms, wall = timer.run(lambda: a @ b, 40)
        mfma("gemm_f32_4097x3001x2049_unpadded", flops, ms, "gemm_unpadded")
        if not skip_cpu:
            ha, hb = p.asnumpy(a[:1024]), p.asnumpy(b)

            def padded_leg(ha=ha, hb=hb, n=n, k=k):
                leg = cpu_blas(lambda: numpy_backend.matmul(ha, hb), 2.0 * 1024 * n * k, "GFLOP/s",
                               "np.matmul float32 A[:1024] @ B (3001x2049)")
                extra["gemm_f32_4097x3001x2049_padded"]["cpu_baseline"] = leg
                extra["gemm_f32_4097x3001x2049_unpadded"]["cpu_baseline"] = leg

            later(padded_leg)
        del a, b
    if begin("gemm_batched"):
        rng = p.random.default_rng(3, backend=hip)
        a = rng.uniform(-1, 1, (64, 512, 1024), dtype="float32")
        b = rng.uniform(-1, 1, (1024, 768), dtype="float32")
        ms, wall = timer.run(lambda: a @ b, 40)
        mfma("gemm_f32_batched_64x512x1024x768", 2.0 * 64 * 512 * 768 * 1024, ms, "gemm_batched")
        if not skip_cpu:
            ha, hb = p.asnumpy(a[:8]), p.asnumpy(b)
            later(lambda ha=ha, hb=hb: extra["gemm_f32_batched_64x512x1024x768"].__setitem__("cpu_baseline", cpu_blas(
                lambda: numpy_backend.matmul(ha, hb), 2.0 * 8 * 512 * 768 * 1024, "GFLOP/s",
                "np.matmul float32 A[:8] @ B, batch of 8")))
        del a, b
    if begin("gemm_small"):
        # Config 1's shape: 1024^3 float32, seed 0 host inputs; the GPU product
        # beside the reference CPU path itself (NumPy's BLAS) and its error.
        gen = np.random.default_rng(0)
        ha = gen.uniform(-1, 1, (1024, 1024)).astype(np.float32)
        hb = gen.uniform(-1, 1, (1024, 1024)).astype(np.float32)
        a, b = p.asarray(ha, backend=hip), p.asarray(hb, backend=hip)
        ms, wall = timer.run(lambda: a @ b, 400)  # ~8 ms of ~21 us products
        flops = 2.0 * 1024**3
        mfma("gemm_f32_1024", flops, ms, "gemm_1024")
        exact64 = ha.astype(np.float64) @ hb.astype(np.float64)
        got = p.asnumpy(a @ b).astype(np.float64)
        extra["gemm_f32_1024"]["rel_l2_vs_float64"] = float(np.linalg.norm(got - exact64) / np.linalg.norm(exact64))
        if not skip_cpu:

            def config1_leg(ha=ha, hb=hb, flops=flops, exact64=exact64):
                leg = cpu_blas(lambda: numpy_backend.matmul(ha, hb), flops, "GFLOP/s",
                               "config 1: np.matmul float32 1024x1024x1024, seed 0")
                cpu_c = numpy_backend.matmul(ha, hb).astype(np.float64)
                leg["rel_l2_vs_float64"] = float(np.linalg.norm(cpu_c - exact64) / np.linalg.norm(exact64))
                extra["gemm_f32_1024"]["cpu_baseline"] = leg
                extra["config1_cpu_gemm_f32_1024"] = dict(
                    leg, note="BASELINE config 1 (the reference NumPy backend path), measured on this host")

            later(config1_leg)
        del a, b
    if only and "copy" in only:
        # Calibration for rocprofv3 --pmc: a plain 1 GiB float32 copy
        # (hipRTC elementwise cast kernel) moves exactly 2^30 B each way.
        n = 1 << 28
        src = p.random.default_rng(9, backend=hip).random(n, dtype="float32")
        ms, wall = timer.run(lambda: src.copy(), 5)
        extra["copy_f32_2^28"] = {"value": round(2 * n * 4 / (ms * 1e-3) / 1e9, 1), "unit": "GB/s", "kernel_us": round(ms * 1e3, 2)}
        del src
    if begin("mlp"):
        rng = p.random.default_rng(42, backend=hip)
        widths = (4096, 4096, 4096, 1024)
        params = []
        for fan_in, fan_out in zip(widths[:-1], widths[1:]):
            params.append(rng.normal(0, (1 / fan_in) ** 0.5, (fan_in, fan_out), dtype="float32"))
            params.append(p.zeros(fan_out, dtype=np.float32, backend=hip))
        x = rng.uniform(-1, 1, (8192, 4096), dtype="float32")

        @p.compile
        def mlp(x, w1, b1, w2, b2, w3, b3):
            h = p.tanh(x @ w1 + b1)
            h = p.tanh(h @ w2 + b2)
            out = p.tanh(h @ w3 + b3)
            return p.mean(out, axis=1)

        ms, wall = timer.run(lambda: mlp(x, *params), 10)
        flops = 2.0 * 8192 * (4096 * 4096 * 2 + 4096 * 1024)
        mfma("mlp_forward_f32_8192x4096", flops, ms, "mlp")
        extra["mlp_forward_f32_8192x4096"]["wall_ms"] = round(wall, 4)
        extra["mlp_forward_f32_8192x4096"]["steps"] = [s["kind"] for s in mlp.explain(x, *params)["steps"]]
        if not skip_cpu:
            rows = 256
            hx = p.asnumpy(x[:rows])
            hosts = [p.asnumpy(v) for v in params]

            def forward():
                h = hx
                for w, bias in zip(hosts[0::2], hosts[1::2]):
                    h = np.tanh(numpy_backend.matmul(h, w) + bias)
                return h.mean(axis=1)

            later(lambda work=flops * rows / 8192, rows=rows: extra["mlp_forward_f32_8192x4096"].__setitem__(
                "cpu_baseline", cpu_blas(forward, work, "GFLOP/s", f"NumPy forward of {rows} rows (np.matmul + np.tanh + mean)")))
    if begin("vendor"):
        extra.update(vendor_gemm())
    for leg in legs:
        leg()
    return extra


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=10)
    parser.add_argument("--warmup", type=int, default=15)
    parser.add_argument("--skip-cpu", action="store_true", help="omit the CPU baselines")
    parser.add_argument("--vendor-child", action="store_true", help=argparse.SUPPRESS)
    parser.add_argument("--only", default="", help="comma-separated extras to run (gemv,norm,strided,rng,gemm_f64,gemm_padded,gemm_batched,gemm_small,mlp,vendor; copy = PMC calibration, only when named); 'none' for the headline only")
    args = parser.parse_args(argv)
    if args.vendor_child:
        print(json.dumps(vendor_gemm_child()), flush=True)
        return 0
    if args.gpus != 1:
        print(
            f"bench.py measures one MI355X: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
            "Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2
    import openpacho as p

    hip = p.get_backend("hip", device=0)
    log(f"device {hip.device}; GEMM 8192^3 fp32, warmup {args.warmup}, steps {args.steps}")
    gemm = bench_gemm(p, hip, args.steps, args.warmup)
    gflops = gemm["flops"] / (gemm["wall_ms"] * 1e-3) / 1e9
    log(f"gemm: kernel {gemm['kernel_ms']:.3f} ms, wall {gemm['wall_ms']:.3f} ms, {gflops:.0f} GFLOP/s")
    only = set() if not args.only else {s.strip() for s in args.only.split(",") if s.strip()}
    extra = {} if only == {"none"} else bench_extras(p, hip, only, args.skip_cpu)
    # The CPU legs run after every GPU timing (see bench_extras).
    cpu = None
    if not args.skip_cpu:
        log("cpu baseline: np.matmul row sample")
        cpu = cpu_gemm_baseline(p, gemm)
    del gemm["a"], gemm["b"]
    vendor = extra.get("vendor_gemm_f32_8192")
    if vendor:
        vendor["hip_over_vendor"] = round(vendor["kernel_ms"] / gemm["kernel_ms"], 4)
    for name, entry in extra.items():
        log(f"{name}: {entry['value']} {entry['unit']}" + (f" ({entry['roofline']['frac']:.1%} of roofline)" if "roofline" in entry else ""))
    result = {
        "metric": METRIC,
        "value": round(gflops, 1),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gemm["wall_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: on-device Philox4x32-10 U[-1,1) float32, seed 3 (inputs resident in HBM)",
        "config": {"workload": "fp32 GEMM C = A @ B, 8192x8192x8192, row-major (BASELINE config 4)", "parallelism": "single GPU"},
        "roofline": roofline("mfma", gemm["flops"], gemm["kernel_ms"], _traffic("gemm_f32")),
        "cpu_baseline": cpu,
        "kernel_ms_per_step": round(gemm["kernel_ms"], 4),
        "extra": extra,
    }
    print(json.dumps(strict_json(result)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
