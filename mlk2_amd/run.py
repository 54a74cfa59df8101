"""`mlkc run` over the HIP backend, for a module already lowered to Kernel IR.

The reference's `mlkc run <graph.mlk> --tier=N` (tools/mlkc/mlkc.cpp:206-263)
parses a graph, executes it on the CPU engine and prints `out[i] = %.17g`.
Its graph front end and passes stay in the reference; this route starts at
the mlk-kernel JSON that `mlkc compile --emit=kernel` writes and runs it on
the declared AMD target through the C ABI's run-route entries:

    python -m mlk2_amd.run module.json --backend=hip [--arch=gfx950]
        [--x=2.0 ...]               scalar kernels: ScalarParams in order
        [--input=x.npy ...]         tensor kernels: input buffers in order
        [--scalar=0.5 ...]          tensor kernels: ScalarParams in order
        [--elements=N]              dynamic loop bound (legacy 1-D form)
        [--out=DIR]                 tensor outputs saved as DIR/out<i>.npy

Scalar kernels print `out[i] = %.17g` per output, like `mlkc run`; tensor
kernels print each output's element count, its first values and a checksum.
Exit codes follow `mlkc`: 0 done, 1 execution failed (the status code and
message of the library), 2 usage or input error. There is no silent
fallback: a caller that wants Tier 0 on failure takes it on exit code 1.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

from . import backend as be


@dataclass
class RunArgs:
    module: str
    backend: str = "hip"
    arch: str = "gfx950"
    xs: List[float] = field(default_factory=list)
    inputs: List[str] = field(default_factory=list)
    scalars: List[float] = field(default_factory=list)
    elements: int = 0
    out: Optional[str] = None


class UsageError(Exception):
    pass


def parse_args(argv: Sequence[str]) -> RunArgs:
    """Parses the command line; raises UsageError on anything malformed."""
    p = argparse.ArgumentParser(prog="mlk2_amd.run", add_help=True)
    p.add_argument("module")
    p.add_argument("--backend", default="hip")
    p.add_argument("--arch", default="gfx950")
    p.add_argument("--x", action="append", default=[], type=float)
    p.add_argument("--input", action="append", default=[])
    p.add_argument("--scalar", action="append", default=[], type=float)
    p.add_argument("--elements", type=int, default=0)
    p.add_argument("--out", default=None)
    try:
        ns = p.parse_args(list(argv))
    except SystemExit as e:
        raise UsageError(f"bad arguments (exit {e.code})")
    if ns.backend != "hip":
        raise UsageError(f"--backend={ns.backend}: this route runs the HIP backend only")
    if not be.lib().mlkhip_valid_arch(ns.arch.encode()):
        raise UsageError(f"--arch={ns.arch}: not a gfx target")
    if ns.elements < 0:
        raise UsageError("--elements must be >= 0")
    if ns.x and (ns.input or ns.scalar):
        raise UsageError("--x is for scalar kernels; tensor kernels take --input and --scalar")
    return RunArgs(ns.module, ns.backend, ns.arch, ns.x, ns.input, ns.scalar, ns.elements, ns.out)


@dataclass
class BufferRole:
    is_input: bool
    is_output: bool
    elements: int
    dims: List[int]


class ModuleText:
    """An mlk-kernel document as written: the text goes to the library
    unchanged; the buffer table tells the route what to bind."""

    def __init__(self, text: str):
        doc = json.loads(text)
        if doc.get("format") != "mlk-kernel":
            raise ValueError("not an mlk-kernel document")
        self.text = text
        self.buffers = [BufferRole(bool(b.get("input", False)), bool(b.get("output", False)),
                                   int(b.get("elements", 0)), [int(d) for d in b.get("dims", [])])
                        for b in doc["buffers"]]

    def to_json(self) -> str:
        return self.text


def load_module(path: str) -> ModuleText:
    with open(path, "r", encoding="utf-8") as f:
        return ModuleText(f.read())


def _numel(km: ModuleText, bid: int, elements: int) -> int:
    b = km.buffers[bid]
    if b.dims:
        n = 1
        for d in b.dims:
            n *= int(d)
        return n
    return int(b.elements) if b.elements >= 0 else int(elements)


def run(args: RunArgs, stdout=None, stderr=None) -> int:
    stdout = stdout or sys.stdout
    stderr = stderr or sys.stderr
    try:
        km = load_module(args.module)
    except (OSError, ValueError, KeyError) as e:
        print(f"mlkc: cannot read module: {e}", file=stderr)
        return 2
    in_ids = [i for i, b in enumerate(km.buffers) if b.is_input]
    out_ids = [i for i, b in enumerate(km.buffers) if b.is_output]
    try:
        if not in_ids:
            values = be.execute_kernel(km, args.xs, args.arch)
            for i, v in enumerate(values):
                print(f"out[{i}] = {v:.17g}", file=stdout)
        else:
            if len(args.inputs) != len(in_ids):
                print(f"mlkc: module has {len(in_ids)} input buffers, got {len(args.inputs)} --input",
                      file=stderr)
                return 2
            arrays = []
            for path, bid in zip(args.inputs, in_ids):
                a = np.load(path, allow_pickle=False).astype(np.float64).reshape(-1)
                want = _numel(km, bid, args.elements)
                if a.size != want:
                    print(f"mlkc: {path}: {a.size} elements, buffer {bid} needs {want}", file=stderr)
                    return 2
                arrays.append(a)
            outs = [np.zeros(_numel(km, bid, args.elements), dtype=np.float64) for bid in out_ids]
            be.execute_kernel_on_buffers(km, arrays, outs, args.scalars, args.elements, args.arch)
            for i, o in enumerate(outs):
                head = ", ".join(f"{v:.9g}" for v in o[:4])
                print(f"out[{i}]: {o.size} elements [{head}{', ...' if o.size > 4 else ''}] "
                      f"sum = {float(np.sum(o)):.17g}", file=stdout)
                if args.out:
                    os.makedirs(args.out, exist_ok=True)
                    np.save(os.path.join(args.out, f"out{i}.npy"), o)
    except be.MlkHipError as e:
        print(f"mlkc: execution failed: status {e.code}: {e.message}", file=stderr)
        return 1
    print(f"mlkc: executed backend=hip arch={args.arch}", file=stderr)
    return 0


def main(argv: Optional[Sequence[str]] = None) -> int:
    try:
        args = parse_args(sys.argv[1:] if argv is None else argv)
    except UsageError as e:
        print(f"mlkc: {e}", file=sys.stderr)
        return 2
    return run(args)


if __name__ == "__main__":
    sys.exit(main())
