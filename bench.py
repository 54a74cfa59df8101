"""Benchmark of the HIP backend on one MI355X.

Headline workload: row-wise stable softmax, f32,
8192 x 4096, x ~ N(0, 2) from seed; one step = one launch of the artifact
over the batch with inputs resident in HBM. The metric is achieved GB/s over
the algorithmic bytes (one read + one write of the matrix, 268,435,456 B),
with the fraction of MI355X peak HBM bandwidth (8 TB/s) in ``roofline``.
The other configs are reported under ``configs`` (same protocol).

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--only c2]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, AMD datasheet
PEAK_F16_TFLOPS = 2500.0       # dense FP16 MFMA
PEAK_F32_TFLOPS = 157.3        # FP32 matrix
PROFILE_PMC = os.path.join(ROOT, "profiles", "softmax_c2_8192x4096_pmc.txt")
# Back-to-back launches of a config before it is timed. Under sustained load
# the chip's clock settles within about 30 ms; a few launches alone time the
# ramp instead (4096^3 f16 GEMM: 130-150 us cold, 119 us settled).
SETTLE_MS = 100.0
# Each config's duration is the median of SPANS event-timed spans of back-to-
# back launches, each at least SPAN_MS long: the runtime now and then leaves a
# gap of tens of microseconds between two launches, which a single short
# span of a 20 us kernel would spread over its average.
SPANS, SPAN_MS = 5, 2.0


def median_span(art, bufs, reps: int) -> float:
    """Median over SPANS spans of `reps` back-to-back launches (ms per launch)."""
    return float(np.median([art.time_device_span(bufs, reps=reps, warmup=0) for _ in range(SPANS)]))


def _cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the machine type."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _stats(ms: np.ndarray) -> dict:
    return {"median_ms": float(np.median(ms)), "mean_ms": float(ms.mean()), "min_ms": float(ms.min())}


def _pmc_traffic():
    """HBM bytes per softmax launch from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration), or None."""
    if not os.path.exists(PROFILE_PMC):
        return None
    for line in open(PROFILE_PMC):
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return int(float(line.split(":", 1)[1].strip()))
            except ValueError:
                return None
    return None


def bench_config(be, name: str, steps: int, warmup: int) -> dict:
    from mlk2_amd import fixtures as fx
    from mlk2_amd import inputs
    from mlk2_amd.backend import DeviceBuffer

    if name == "copy":
        # Calibration for the PMC counters: y = x + 0 over 2^26 f32 (a plain
        # streaming copy through the elementwise template, 512 MiB moved).
        from mlk2_amd.kernel_ir import KernelExpr, const, elem_a
        n = 1 << 26
        km = fx.lower_elementwise([("x", [n], "f32")], [KernelExpr("add", elem_a(), const(0.0))], [n])
        bufs = {0: DeviceBuffer.from_array(np.zeros(n, np.float32), "f32"), 1: DeviceBuffer(n, "f32")}
        work, unit, peak, bound = 8 * n, "GB/s", PEAK_HBM_GBS, "hbm"
        wl = "copy y = x + 0, f32, 2^26"
    elif name == "c1":
        n = 1 << 24
        km = fx.config1_module(n=n)
        d = inputs.config_inputs("c1")
        bufs = {0: DeviceBuffer.from_array(d["x"], "f32"), 1: DeviceBuffer(n, "f32")}
        work, unit, peak, bound = 8 * n, "GB/s", PEAK_HBM_GBS, "hbm"
        wl = "sin(x^2+3x) poly7, f32, 2^24"
    elif name == "c2":
        m, k = 8192, 4096
        km = fx.config2_module(m, k, tier=1)
        d = inputs.config_inputs("c2")
        bufs = {0: DeviceBuffer.from_array(d["x"], "f32"), 1: DeviceBuffer(m * k, "f32")}
        work, unit, peak, bound = 8 * m * k, "GB/s", PEAK_HBM_GBS, "hbm"
        wl = "row softmax, f32, 8192x4096"
    elif name == "c3":
        r, c = 4096, 4096
        km = fx.config3_module(r, c, tier=2)
        d = inputs.config_inputs("c3")
        bufs = {0: DeviceBuffer.from_array(d["x"], "f32"), 1: DeviceBuffer.from_array(d["b"], "f32"),
                2: DeviceBuffer(r * c, "f32")}
        work, unit, peak, bound = 4 * r * c * 2 + 4 * c, "GB/s", PEAK_HBM_GBS, "hbm"
        wl = "exp(0.5*x+b[j])*x, f32, 4096x4096"
    elif name == "c4a":
        m = k = n = 1024
        km = fx.config4_module(m, k, n, "f32", tier=2)
        d = inputs.config_inputs("c4a")
        bufs = {0: DeviceBuffer.from_array(d["A"], "f32"), 1: DeviceBuffer.from_array(d["B"], "f32"),
                2: DeviceBuffer(m * n, "f32")}
        work, unit, peak, bound = 2 * m * n * k, "TFLOP/s", PEAK_F32_TFLOPS, "mfma"
        wl = "gemm f32 1024^3"
    elif name == "c4b":
        m = k = n = 4096
        km = fx.config4_module(m, k, n, "f16", tier=2)
        d = inputs.config_inputs("c4b")
        bufs = {0: DeviceBuffer.from_array(d["A"], "f16"), 1: DeviceBuffer.from_array(d["B"], "f16"),
                2: DeviceBuffer(m * n, "f32")}
        work, unit, peak, bound = 2 * m * n * k, "TFLOP/s", PEAK_F16_TFLOPS, "mfma"
        wl = "gemm f16 in / f32 acc 4096^3"
    elif name == "c4b_call":
        # The Tier-1 Call(MatMul) form the reference's bench builds and times
        # first (tools/mlk-poly/poly_bench.cpp:123-160, :314-366): C += A*B
        # with the executor's skip of A[i,p] == 0: one MFMA launch whose
        # waves check their accumulators for non-finite values (none here).
        m = k = n = 4096
        km = fx.config4_module(m, k, n, "f16", tier=1)
        d = inputs.config_inputs("c4b")
        bufs = {0: DeviceBuffer.from_array(d["A"], "f16"), 1: DeviceBuffer.from_array(d["B"], "f16"),
                2: DeviceBuffer(m * n, "f32")}
        bufs[2].fill_zero()
        work, unit, peak, bound = 2 * m * n * k, "TFLOP/s", PEAK_F16_TFLOPS, "mfma"
        wl = "Call(MatMul) f16 in / f32 acc 4096^3, C += A*B with skip-zero-A"
    elif name == "c5":
        b, s, dm = 16, 2048, 128
        km = fx.score_softmax_module(b, s, dm)
        d = inputs.config_inputs("c5")
        bufs = {0: DeviceBuffer.from_array(d["Q"], "f16"), 1: DeviceBuffer.from_array(d["K"], "f16"),
                2: DeviceBuffer.from_array(d["bias"], "f32"), 3: DeviceBuffer(b * s * s, "f32")}
        work, unit, peak, bound = 2 * b * s * dm * 2 + 4 * s + 4 * b * s * s, "GB/s", PEAK_HBM_GBS, "hbm"
        wl = "softmax(QK^T/sqrt(128)+bias), 16x2048x2048"
    else:
        raise KeyError(name)
    art = be.build(km)
    # Settle: at least SETTLE_MS of back-to-back launches, then the timed span.
    est = art.time_device_span(bufs, reps=3, warmup=1)
    settle_reps = max(warmup, int(SETTLE_MS / max(est, 1e-3)) + 1)
    settled_ms = art.time_device_span(bufs, reps=settle_reps, warmup=0) * settle_reps
    span_reps = max(steps, int(SPAN_MS / max(est, 1e-3)) + 1)
    span_ms = median_span(art, bufs, span_reps)
    st = _stats(art.time_device(bufs, reps=steps, warmup=1))
    scale = 1e9 if unit == "GB/s" else 1e12
    achieved = work / (span_ms * 1e-3) / scale
    kernels = [art.step_kernel_name(i) for i in range(art.num_steps())]
    out = {"workload": wl, "class": art.class_name, "policy": art.policy, "kernels": kernels, "unit": unit,
           "bound": bound, "algorithmic_work": work, "achieved": round(achieved, 2),
           "peak": peak, "frac": round(achieved / peak, 4), "kernel_ms": round(span_ms, 5),
           "per_launch_event": {k: round(v, 5) for k, v in st.items()},
           "settle": {"launches": settle_reps, "ms": round(settled_ms, 1)},
           "spans": {"count": SPANS, "launches_each": span_reps}}
    if name == "c5":
        # The second fraction: the score GEMM's flops against the f16 MFMA
        # peak (each pass recomputes the scores, so the MFMAs run it twice).
        flops = 2 * 16 * 2048 * 2048 * 128
        out["mfma"] = {"algorithmic_flops": flops,
                       "achieved_tflops": round(flops / (span_ms * 1e-3) / 1e12, 2),
                       "peak_tflops": PEAK_F16_TFLOPS,
                       "frac": round(flops / (span_ms * 1e-3) / 1e12 / PEAK_F16_TFLOPS, 4),
                       "frac_with_recompute": round(2 * flops / (span_ms * 1e-3) / 1e12 / PEAK_F16_TFLOPS, 4)}
    return out


def _time_cpu(fn, warmup: int = 5, reps: int = 30, budget_s: float = 15.0):
    """The reference bench's protocol (bench/math/math_bench.cpp:142-185,
    constants.h:50-51): `warmup` untimed runs, then the median of `reps`
    timed ones, cut short only past `budget_s` of timed work (the count
    taken is reported)."""
    for _ in range(warmup):
        fn()
    times = []
    end = time.perf_counter() + budget_s
    while len(times) < reps and (not times or time.perf_counter() < end):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_baseline_softmax() -> dict:
    """The oracle's Call(Softmax) (serial, f64, as kernel_buffers.cpp:290-340)
    on a bounded sample of the same workload: 512 rows x 4096."""
    import oracle
    from mlk2_amd import fixtures as fx
    from mlk2_amd import inputs
    rows, k = 512, 4096
    x = inputs.normal(inputs.SEEDS["c2_x"], rows * k, 0.0, 2.0).astype(np.float64)
    km = fx.config2_module(rows, k, tier=1)
    y = np.zeros(rows * k)
    text = km.to_json()
    med, n_reps = _time_cpu(lambda: oracle.execute(text, [x], [y]), 5, 30)
    gbs = 8 * rows * k / med / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"oracle Call(Softmax) f64, {rows}x{k} rows of the config-2 input, "
                      f"warmup 5, median of {n_reps} reps ({med * 1e3:.1f} ms), bytes counted as f32 read+write",
            "host": _cpu_model(), "nproc": os.cpu_count()}


def cpu_baseline_config(name: str) -> dict:
    """The oracle's restatement of the reference CPU path for one config, on a
    bounded sample, timed on this host: the Tier-1 1-D path and Call(MatMul)
    with the executor's default thread count min(hardware threads, 4)
    (kernel_buffers.cpp:183-199) and once with the module's "threads"
    parameter at the host's thread count; the serial walker for the nests."""
    import oracle
    from mlk2_amd import fixtures as fx
    from mlk2_amd import inputs
    nproc = os.cpu_count() or 1
    default_threads = min(nproc, 4)
    out = {"kind": "port", "nproc": nproc, "host": _cpu_model()}

    def run(km, ins, outs, threads):
        text = km.to_json()
        return lambda: oracle.execute(text, ins, outs, (), 0, threads)

    if name == "c1":
        n = 1 << 22
        x = inputs.uniform(inputs.SEEDS["c1_x"], n, -4.0, 4.0, "f32").astype(np.float64)
        km = fx.config1_module(n=n)
        y = np.zeros(n)
        med, reps = _time_cpu(run(km, [x], [y], default_threads))
        km.schedule["threads"] = nproc
        med_all, _ = _time_cpu(run(km, [x], [y], nproc))
        work, unit, scale = 8 * n, "GB/s", 1e9
        sample = "1-D path (poly7) over 2^22 of the 2^24 elements, warmup 5"
    elif name == "c3":
        rows, cols = 256, 4096
        d = inputs.config_inputs("c3", {"rows": rows, "cols": cols})
        km = fx.config3_module(rows, cols, tier=2)
        y = np.zeros(rows * cols)
        med, reps = _time_cpu(run(km, [d["x"].astype(np.float64), d["b"].astype(np.float64)], [y], default_threads))
        med_all = None
        default_threads = 1
        work, unit, scale = 8 * rows * cols + 4 * cols, "GB/s", 1e9
        sample = (f"Tier-2 walker (serial: the synthesized nest carries no parallel marks), {rows} of 4096 rows, "
                  "warmup 5")
    elif name in ("c4a", "c4b", "c4b_call"):
        m, k, n = (1024, 1024, 1024) if name == "c4a" else (256, 4096, 4096)
        dt = "f32" if name == "c4a" else "f16"
        # The config's own seeded inputs; C4b takes the first 256 rows of A.
        d = inputs.config_inputs("c4a" if name == "c4a" else "c4b")
        a = d["A"].astype(np.float64).reshape(-1)[: m * k].copy()
        b = d["B"].astype(np.float64).reshape(-1)
        km = fx.config4_module(m, k, n, dt, tier=1)
        c = np.zeros(m * n)
        wu, nr = (5, 30) if name == "c4a" else (1, 5)
        med, reps = _time_cpu(run(km, [a, b], [c], default_threads), wu, nr)
        km.schedule["threads"] = nproc
        med_all, _ = _time_cpu(run(km, [a, b], [c], nproc), wu, nr)
        work, unit, scale = 2 * m * n * k, "TFLOP/s", 1e12
        sample = (f"Call(MatMul) blocked 64/64/32 (f64), {m}x{k}x{n}"
                  + ("" if name == "c4a" else " (the first 256 of the 4096 rows)")
                  + f", warmup {wu}")
    elif name == "c5":
        b_, s_, d_ = 1, 512, 128
        d = inputs.config_inputs("c5", {"batch": b_, "seq": s_, "dim": d_})
        km = fx.score_softmax_module(b_, s_, d_)
        y = np.zeros(b_ * s_ * s_)
        med, reps = _time_cpu(run(km, [d["Q"].astype(np.float64), d["K"].astype(np.float64),
                                       d["bias"].astype(np.float64)], [y], default_threads), 1, 5)
        med_all = None
        default_threads = 1
        work, unit, scale = 2 * b_ * s_ * d_ * 2 + 4 * s_ + 4 * b_ * s_ * s_, "GB/s", 1e9
        sample = "walker over the composed module (serial), 1 batch x 512 x 512 x 128, warmup 1"
    else:
        return {}
    out.update({"value": round(work / med / scale, 4), "unit": unit, "cores": default_threads,
                "sample": f"{sample}; median of {reps} ({med * 1e3:.1f} ms)"})
    if med_all is not None:
        out["value_threads_nproc"] = round(work / med_all / scale, 4)
    return out


def probe_mfma() -> dict:
    """Settled f16 MFMA rates of register-only loops (no memory traffic in the
    loop), one workgroup per CU: the ceiling the power limit leaves a GEMM
    and the calibration of the MFMA-busy counters (rocprofv3 --pmc of this
    command reads what those counters show at each measured rate)."""
    import ctypes

    from mlk2_amd.backend import lib

    fn = lib().mlkd_probe_mfma_rate
    fn.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_int,
                   ctypes.POINTER(ctypes.c_double), ctypes.c_void_p]
    fn.restype = ctypes.c_int
    out = {}
    for shape, sname in ((0, "16x16x32"), (1, "32x32x16")):
        for random in (1, 0):
            for wps in (1, 2):
                r = ctypes.c_double()
                rc = fn(shape, random, wps, 100.0, 10, ctypes.byref(r), None)
                key = f"{sname} {'random' if random else 'ones'} {wps}w/SIMD"
                out[key] = None if rc != 0 else round(r.value / 1e12, 1)
                print(f"[probe] {key}: {out[key]} TFLOP/s", file=sys.stderr, flush=True)
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default="")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--probe-mfma", action="store_true",
                    help="only time the register-only f16 MFMA probes (TFLOP/s) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the kernels shard by rows/batches across GPUs by design, but no multi-GPU "
              "path is built or measured)", file=sys.stderr)
        return 2

    from mlk2_amd import fixtures as fx
    from mlk2_amd import inputs
    from mlk2_amd.backend import DeviceBuffer, HipBackend, lib

    be = HipBackend("gfx950")
    if not be.device_available():
        print("bench.py: no gfx950 device visible", file=sys.stderr)
        return 3
    if args.probe_mfma:
        print(json.dumps({"probe": "register-only f16 MFMA, TFLOP/s", "rates": probe_mfma()}), flush=True)
        return 0

    # Headline: C2 softmax, K timed steps bracketed by device synchronization.
    m, k = 8192, 4096
    km = fx.config2_module(m, k, tier=1)
    x = inputs.config_inputs("c2")["x"]
    xb = DeviceBuffer.from_array(x, "f32")
    yb = DeviceBuffer(m * k, "f32")
    art = be.build(km)
    bufs = {0: xb, 1: yb}
    for _ in range(args.warmup):
        art.run_device(bufs, sync=False)
    lib().mlkhip_synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        art.run_device(bufs, sync=False)
    lib().mlkhip_synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    bytes_alg = 2 * 4 * m * k
    value = bytes_alg / (ms_per_step * 1e-3) / 1e9
    # Kernel duration: HIP event pairs on the launch stream around K
    # back-to-back launches (the span the wall clock covers above), the
    # median of SPANS such spans.
    kernel_ms = median_span(art, bufs, args.steps)
    achieved = bytes_alg / (kernel_ms * 1e-3) / 1e9

    configs = {}
    names = [n for n in ("copy", "c1", "c3", "c4a", "c4b", "c4b_call", "c5")
             if (not args.only and n != "copy") or n in args.only.split(",")]
    for name in names:
        try:
            configs[name] = bench_config(be, name, max(10, args.steps // 2), 5)
            if not args.no_cpu:
                prior = configs.get("c4b", {}).get("cpu_baseline")
                # C4b's CPU baseline is the Call(MatMul) form already.
                configs[name]["cpu_baseline"] = (prior if name == "c4b_call" and prior
                                                 else cpu_baseline_config(name))
        except Exception as e:  # a config failing must not hide the headline line
            configs[name] = {"error": str(e)}

    line = {
        "metric": "achieved GB/s (row softmax f32 8192x4096) as % of MI355X HBM roofline",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (SplitMix64 seed 0x5EED0002, N(0,2))",
        "config": {"workload": "config 2: row-wise stable softmax, f32, 8192x4096",
                   "rows": m, "cols": k, "class": art.class_name, "policy": art.policy},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": _pmc_traffic(), "kernel_ms": round(kernel_ms, 5),
                     "algorithmic_bytes": bytes_alg,
                     "traffic_source": "profiles/softmax_c2_8192x4096_pmc.txt (rocprofv3 FETCH_SIZE and "
                                       "WRITE_SIZE runs of this workload, copy-calibrated); not measured "
                                       "in this run"},
        "cpu_baseline": None if args.no_cpu else cpu_baseline_softmax(),
        # Each config is timed after >= SETTLE_MS of back-to-back launches
        # (its "settle" field); the headline's steps follow --warmup steps.
        "config_settle_ms": SETTLE_MS,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
