"""`mlk-poly autotune` over the HIP backend, for the five configs.

The reference's verb (tools/mlk-poly/mlk_poly.cpp:389-600) builds an f64
MatMul graph of M x K x N (64 x 48 x 56 by default), runs the fast-kernel
search over its declared variant space and prints one line per candidate:
its identity certificate, its benchmarked runtime upper bound, the winner
and the gap over the roofline lower bound. `--json-out` writes the full
report. Here the searched space is each step's gfx950 launch forms
(`mlkhip_autotune`: identity certificates under the plan's tolerance
policy, runtime bounds, the roofline bound and the cache), and the verb
covers the five configs as well as the reference's GEMM:

    python -m mlk2_amd.autotune [--config=gemm|c1|c2|c3|c4a|c4b|c5|all]
        [--m=M --k=K --n=N] [--dtype=f64|f32|f16]   gemm (f64 64x48x56 by default)
        [--elements=N]                              c1 (2^24)
        [--rows=R --cols=C]                         c2 (8192x4096), c3 (4096x4096)
        [--batch=B --seq=S --dim=D]                 c5 (16x2048x128)
        [--tier=1|2] [--reps=R] [--cache-dir=D] [--arch=gfx950] [--json-out=F]

c4a and c4b take --m/--k/--n too (1024^3 and 4096^3 by default). The
inputs are the configs' seeded synthetic data (mlk2_amd.inputs).
`--module=doc.json` searches any mlk-kernel document instead (seeded
uniform [-1, 1] inputs; `--elements` for a dynamic extent, `--scalar` for
scalar parameters). Exit codes: 0 done, 1 a search failed, 2 usage error or
no device.
"""
from __future__ import annotations

import argparse
import json
import sys
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import backend as be
from . import fixtures as fx
from . import inputs
from .kernel_ir import KernelBuffer, KernelModule

CONFIGS = ("gemm", "c1", "c2", "c3", "c4a", "c4b", "c5")


class UsageError(Exception):
    pass


@dataclass
class TuneArgs:
    configs: List[str]
    m: Optional[int] = None
    k: Optional[int] = None
    n: Optional[int] = None
    dtype: str = "f64"
    elements: Optional[int] = None
    rows: Optional[int] = None
    cols: Optional[int] = None
    batch: Optional[int] = None
    seq: Optional[int] = None
    dim: Optional[int] = None
    tier: Optional[int] = None
    reps: int = 10
    cache_dir: Optional[str] = None
    arch: str = "gfx950"
    json_out: Optional[str] = None
    module: Optional[str] = None
    scalars: Sequence[float] = ()


def parse_args(argv: Sequence[str]) -> TuneArgs:
    """Parses the command line; raises UsageError on anything malformed."""
    p = argparse.ArgumentParser(prog="mlk2_amd.autotune", add_help=True)
    p.add_argument("--config", default="gemm")
    for name in ("m", "k", "n", "elements", "rows", "cols", "batch", "seq", "dim", "tier"):
        p.add_argument(f"--{name}", type=int, default=None)
    p.add_argument("--dtype", default="f64")
    p.add_argument("--reps", type=int, default=10)
    p.add_argument("--cache-dir", default=None)
    p.add_argument("--arch", default="gfx950")
    p.add_argument("--json-out", default=None)
    p.add_argument("--module", default=None)
    p.add_argument("--scalar", action="append", default=[], type=float)
    try:
        ns = p.parse_args(list(argv))
    except SystemExit as e:
        raise UsageError(f"bad arguments ({e.code})")
    configs = ["module"] if ns.module else (list(CONFIGS) if ns.config == "all" else ns.config.split(","))
    for c in configs:
        if c not in CONFIGS and c != "module":
            raise UsageError(f"unknown --config {c} (one of {', '.join(CONFIGS)} or all)")
    if ns.dtype not in ("f64", "f32", "f16"):
        raise UsageError("--dtype must be f64, f32 or f16")
    if ns.tier is not None and ns.tier not in (1, 2):
        raise UsageError("--tier must be 1 or 2")
    if ns.reps <= 0:
        raise UsageError("--reps must be positive")
    for name in ("m", "k", "n", "elements", "rows", "cols", "batch", "seq", "dim"):
        v = getattr(ns, name)
        if v is not None and v <= 0:
            raise UsageError(f"--{name} must be positive")
    return TuneArgs(configs=configs, m=ns.m, k=ns.k, n=ns.n, dtype=ns.dtype, elements=ns.elements, rows=ns.rows,
                    cols=ns.cols, batch=ns.batch, seq=ns.seq, dim=ns.dim, tier=ns.tier, reps=ns.reps,
                    cache_dir=ns.cache_dir, arch=ns.arch, json_out=ns.json_out, module=ns.module,
                    scalars=tuple(ns.scalar))


def _pick(v: Optional[int], default: int) -> int:
    return default if v is None else v


class DocumentModule:
    """An mlk-kernel document as written: its text goes to the library
    unchanged, and its buffer table says what the search binds."""

    def __init__(self, text: str):
        try:
            doc = json.loads(text)
        except ValueError as e:
            raise UsageError(f"not JSON: {e}")
        if not isinstance(doc, dict) or doc.get("format") != "mlk-kernel" or "buffers" not in doc:
            raise UsageError("not an mlk-kernel document")
        self.text = text
        self.buffers = [KernelBuffer(name=str(b.get("name", f"b{i}")), dtype=str(b.get("dtype", "f64")),
                                     is_input=bool(b.get("input", False)), is_output=bool(b.get("output", False)),
                                     is_temp=bool(b.get("temp", False)), elements=int(b.get("elements", -1)),
                                     dims=[int(d) for d in b.get("dims", [])])
                        for i, b in enumerate(doc["buffers"])]

    def to_json(self) -> str:
        return self.text

    def bindable_ids(self) -> List[int]:
        return [i for i, b in enumerate(self.buffers) if b.is_input or b.is_output or b.is_temp]


def _document_case(a: TuneArgs) -> Tuple[str, DocumentModule, List[np.ndarray]]:
    try:
        with open(a.module, "r", encoding="utf-8") as f:
            km = DocumentModule(f.read())
    except OSError as e:
        raise UsageError(f"cannot read {a.module}: {e}")
    arrays = []
    for i, b in enumerate(km.buffers):
        n = int(np.prod(b.dims)) if b.dims else (b.elements if b.elements >= 0 else (a.elements or -1))
        if n < 0:
            raise UsageError(f"buffer {i} has a dynamic extent: give --elements")
        b.elements = n
        if b.is_input and not b.is_temp:
            arrays.append(inputs.uniform(0x5EED0200 + i, n, -1.0, 1.0, b.dtype))
    return f"module {a.module}", km, arrays


def config_case(name: str, a: TuneArgs) -> Tuple[str, KernelModule, List[np.ndarray]]:
    """(description, module, input arrays in the module's input order) of
    config `name` at the shape the arguments give."""
    if name == "module":
        return _document_case(a)
    if name == "gemm":
        m, k, n = _pick(a.m, 64), _pick(a.k, 48), _pick(a.n, 56)
        tier = _pick(a.tier, 2)
        out_dt = "f64" if a.dtype == "f64" else "f32"
        call = fx.matmul_call_module(m, k, n, a.dtype, out_dt)
        km = fx.synth_gemm(call) if tier == 2 else call
        A = inputs.uniform(0x5EED0101, m * k, -1.0, 1.0, a.dtype).reshape(m, k)
        B = inputs.uniform(0x5EED0102, k * n, -1.0, 1.0, a.dtype).reshape(k, n)
        return f"gemm {a.dtype} {m}x{k}x{n}, tier {tier}", km, [A, B]
    if name == "c1":
        n = _pick(a.elements, 1 << 24)
        return f"c1 sin(x^2+3x) poly7, f32, {n}", fx.config1_module(n=n), \
            [inputs.config_inputs("c1", {"n": n})["x"]]
    if name == "c2":
        m, k = _pick(a.rows, 8192), _pick(a.cols, 4096)
        tier = _pick(a.tier, 1)
        return f"c2 row softmax f32 {m}x{k}, tier {tier}", fx.config2_module(m, k, tier=tier), \
            [inputs.config_inputs("c2", {"m": m, "k": k})["x"]]
    if name == "c3":
        r, c = _pick(a.rows, 4096), _pick(a.cols, 4096)
        tier = _pick(a.tier, 2)
        d = inputs.config_inputs("c3", {"rows": r, "cols": c})
        return f"c3 exp(0.5x+b[j])*x f32 {r}x{c}, tier {tier}", fx.config3_module(r, c, tier=tier), \
            [d["x"], d["b"]]
    if name in ("c4a", "c4b"):
        default = 1024 if name == "c4a" else 4096
        m, k, n = _pick(a.m, default), _pick(a.k, default), _pick(a.n, default)
        tier = _pick(a.tier, 2)
        dt = "f32" if name == "c4a" else "f16"
        d = inputs.config_inputs(name, {"m": m, "k": k, "n": n})
        return f"{name} gemm {dt} {m}x{k}x{n}, tier {tier}", fx.config4_module(m, k, n, dt, tier), \
            [d["A"], d["B"]]
    if name == "c5":
        b, s, dm = _pick(a.batch, 16), _pick(a.seq, 2048), _pick(a.dim, 128)
        d = inputs.config_inputs("c5", {"batch": b, "seq": s, "dim": dm})
        return f"c5 softmax(QK^T/sqrt({dm})+bias) {b}x{s}x{s}", fx.score_softmax_module(b, s, dm), \
            [d["Q"], d["K"], d["bias"]]
    raise UsageError(f"unknown config {name}")


def bind(km: KernelModule, arrays: Sequence[np.ndarray]) -> Dict[int, be.DeviceBuffer]:
    """Device buffers for every non-temp buffer of `km`: inputs from
    `arrays` in order, outputs zeroed."""
    bufs: Dict[int, be.DeviceBuffer] = {}
    it = iter(arrays)
    for i, b in enumerate(km.buffers):
        if b.is_temp:
            continue
        if b.is_input:
            bufs[i] = be.DeviceBuffer.from_array(np.asarray(next(it)).reshape(-1), b.dtype)
        else:
            bufs[i] = be.DeviceBuffer(b.elements, b.dtype)
    return bufs


def summary(title: str, art: "be.LoadedKernel", rep: dict) -> List[str]:
    """The human summary of one search: every line traces to a field of
    the report."""
    env = rep.get("environment", {})
    out = [f"== fast-kernel search: {title} ==",
           f"class: {art.class_name}   policy: {art.policy}   fingerprint: {rep.get('fingerprint', '')}",
           f"environment: HBM {env.get('measured_bytes_per_sec', 0) / 1e12:.2f} TB/s measured, "
           f"f16 MFMA {env.get('measured_f16_flops_per_sec', 0) / 1e12:.0f} TFLOP/s measured"]
    work = rep.get("work", {})
    if rep.get("roofline_lower_sec", 0) > 0:
        out.append(f"roofline lower bound: {rep['roofline_lower_sec'] * 1e3:.4f} ms "
                   f"(B_min={work.get('min_bytes', 0)} B, O_min={work.get('min_ops', 0)} ops); "
                   f"winner gap: {1.0 + rep.get('winner_gap_over_lower', 0.0):.2f}x over L")
    if not rep.get("steps"):
        out.append("no step declares more than one launch form: defaults kept, nothing timed")
    for st in rep.get("steps", []):
        out.append(f"step {st.get('step', 0)} ({st.get('class', '')}): launch "
                   f"{'covered' if st.get('launch', {}).get('covered') else 'NOT covered'}, "
                   f"{st.get('launch', {}).get('workgroups', 0)} workgroups")
        out.append(f"  {'form':<6} {'identity':<11} {'U_run(ms)':<11} {'min(ms)':<10} status")
        for c in st.get("candidates", []):
            if c.get("admissible"):
                rt = c["certificate"]["runtime"]
                ident = "certified" if c["certificate"]["identity"]["certified"] else "-"
                mark = "  <- chosen" if c["variant"] == st.get("chosen") else ""
                out.append(f"  {c['variant']:<6} {ident:<11} {rt['upper_bound_sec'] * 1e3:<11.4f} "
                           f"{rt['min_sec'] * 1e3:<10.4f} admissible{mark}")
            else:
                out.append(f"  {c['variant']:<6} {'-':<11} {'-':<11} {'-':<10} "
                           f"{c.get('rejected', {}).get('reason', 'rejected')}")
    if rep.get("winner_sec", 0) > 0:
        out.append(f"winner: forms {rep.get('variants')} (U_run = {rep['winner_sec'] * 1e3:.4f} ms), "
                   f"combined certified: {rep.get('combined_certified')}")
    cache = rep.get("cache", {}).get("file", "")
    out.append(f"cache: {cache if cache else '-'}")
    return out


def main(argv: Optional[Sequence[str]] = None) -> int:
    try:
        a = parse_args(sys.argv[1:] if argv is None else argv)
    except UsageError as e:
        print(f"mlk2_amd.autotune: {e}", file=sys.stderr)
        return 2
    hip = be.HipBackend(a.arch)
    if not hip.device_available():
        print(f"mlk2_amd.autotune: no {a.arch} device visible", file=sys.stderr)
        return 2
    reports = {}
    rc = 0
    for name in a.configs:
        try:
            title, km, arrays = config_case(name, a)
        except UsageError as e:
            print(f"mlk2_amd.autotune: {e}", file=sys.stderr)
            return 2
        bufs = bind(km, arrays)
        try:
            art = hip.build(km, cache_dir=a.cache_dir)
            # --elements is the run's element count only for a document (for
            # c1 it is the config's size).
            rep = art.autotune(bufs, scalars=a.scalars, elements=(a.elements or 0) if name == "module" else 0,
                               reps=a.reps, cache_dir=a.cache_dir)
        except be.MlkHipError as e:
            print(f"mlk2_amd.autotune: {name}: search failed: {e}", file=sys.stderr)
            rc = 1
            continue
        finally:
            for b in bufs.values():
                b.free()
        reports[name] = rep
        print("\n".join(summary(title, art, rep)), flush=True)
        print(flush=True)
    if a.json_out:
        with open(a.json_out, "w") as f:
            json.dump(reports, f, indent=1)
        print(f"report: {a.json_out}")
    return rc


if __name__ == "__main__":
    sys.exit(main())
