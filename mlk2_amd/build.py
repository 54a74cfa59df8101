"""Builds libmlk_hip.so for gfx950 in-tree (mlk2_amd/lib/).

Device code (*.hip) is compiled with hipcc for --offload-arch=gfx950 and
-ffp-contract=off (f64 chains round like the reference's x86-64 build);
host code (host/*.cpp) is C++26 without exceptions or RTTI, compiled with
ROCm's clang against the C launch ABI only. The elementwise kernel template
is embedded into the library (it is instantiated with hipRTC per module) and
also compiled once standalone here, so a template that does not compile
fails the build rather than a run.

    python -m mlk2_amd.build        # or __graft_entry__.build()
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(ROOT, "_build", "mlk_hip")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libmlk_hip.so")
ARCH = "gfx950"

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
CLANG = os.path.join(ROCM, "llvm", "bin", "clang++")

DEVICE_SOURCES = ["runtime.hip", "jit.hip", "softmax.hip", "gemm.hip", "score_softmax.hip", "probe.hip"]
HOST_SOURCES = ["kernel_ir.cpp", "planner.cpp", "codegen.cpp", "nestgen.cpp", "canonical.cpp", "driver.cpp", "tune.cpp",
                "artifact.cpp"]

HIP_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
             "-Wall", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
HOST_FLAGS = ["-std=c++2c", "-O2", "-fPIC", "-fno-exceptions", "-fno-rtti", "-Wall", "-Wextra",
              "-Werror"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _embed(gen_dir: str, source: str, symbol: str, inc: str) -> None:
    src = open(os.path.join(CSRC, "device", source)).read()
    if ")MLKTPL" in src:
        raise RuntimeError(f"{source} contains the raw-string delimiter")
    text = f'static const char {symbol}[] = R"MLKTPL(' + src + ')MLKTPL";\n'
    path = os.path.join(gen_dir, inc)
    if not os.path.exists(path) or open(path).read() != text:
        with open(path, "w") as f:
            f.write(text)


def _embed_template(gen_dir: str) -> None:
    """The hipRTC sources the host code instantiates: the device math header
    (prepended to every instance) and the elementwise template."""
    _embed(gen_dir, "mlk_device_math.h", "kDeviceMathHeader", "device_math.inc")
    _embed(gen_dir, "elementwise_template.hip", "kElementwiseTemplate", "elementwise_template.inc")


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    gen = os.path.join(BUILD, "gen")
    os.makedirs(gen, exist_ok=True)
    _embed_template(gen)
    jobs = []
    objs = []
    for s in DEVICE_SOURCES:
        o = os.path.join(BUILD, s.replace(".hip", ".o"))
        jobs.append([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, "device", s), "-o", o])
        objs.append(o)
    for s in HOST_SOURCES:
        o = os.path.join(BUILD, s.replace(".cpp", ".host.o"))
        jobs.append([CLANG] + HOST_FLAGS + ["-I", gen, "-c", os.path.join(CSRC, "host", s), "-o", o])
        objs.append(o)
    # The template, standalone (its built-in sample instance).
    jobs.append([HIPCC] + HIP_FLAGS + ["--cuda-device-only", "-c",
                                       os.path.join(CSRC, "device", "elementwise_template.hip"),
                                       "-o", os.path.join(BUILD, "elementwise_template.check.o")])
    workers = min(8, os.cpu_count() or 4)
    with ThreadPoolExecutor(max_workers=workers) as ex:
        for out in ex.map(_run, jobs):
            if verbose and out.strip():
                print(out)
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs +
         [f"-L{ROCM}/lib", "-lhiprtc", f"-Wl,-rpath,{ROCM}/lib"])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> None:
    """Compiles the CPU oracle (test infrastructure) and, where the reference
    tree is mounted, the reference's own poly7 header into oracle/_ref."""
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle")])


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    build_oracle()
