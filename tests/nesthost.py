"""CPU execution of generated loop-nest kernels, for tests.

The HIP backend's generic loop-nest path emits one kernel per forest root
(``mlk2_amd/csrc/host/nestgen.cpp``). This helper takes that source (through
``mlkhip_compile_check``), compiles it for the host with ROCm's clang under
AddressSanitizer together with ``tests/nest_host/harness.cpp``, and runs every
thread of the launch grid sequentially over numpy buffers. Every index the
kernel forms is thereby checked against exact-size host allocations before the
kernel ever runs on a GPU, and its results can be compared with the oracle.
"""
from __future__ import annotations

import hashlib
import os
import re
import struct
import subprocess
import tempfile
from typing import Dict, List, Sequence, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SHIM = os.path.join(HERE, "nest_host", "hip_host_shim.h")
HARNESS = os.path.join(HERE, "nest_host", "harness.cpp")
CLANG = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", "clang++")
CACHE = os.path.join(tempfile.gettempdir(), "mlk_nest_host")
DT = {"f32": (0, np.float32), "f16": (1, np.float16), "f64": (2, np.float64)}


def parse_header(src: str) -> Tuple[List[int], int]:
    slots = [int(x) for x in re.search(r"// mlk-nest slots:([ 0-9]*)\n", src).group(1).split()]
    total = int(re.search(r"// mlk-nest instances: (\d+)\n", src).group(1))
    return slots, total


def workgroup_size(src: str) -> int:
    """Threads per workgroup of an instance: 256, or what its launch form's
    leading `#define MLK_NEST_WG` sets."""
    m = re.match(r"#define MLK_NEST_WG (\d+)\n", src)
    return int(m.group(1)) if m else 256


def grid_for(threads: int, wg: int = 256) -> int:
    """The driver's launch grid for `threads` instances (gridFor)."""
    return max(1, min((threads + wg - 1) // wg, 16384))


def build(src: str) -> str:
    os.makedirs(CACHE, exist_ok=True)
    h = hashlib.sha256((src + open(SHIM).read() + open(HARNESS).read()).encode()).hexdigest()[:20]
    exe = os.path.join(CACHE, f"nest_{h}")
    if os.path.exists(exe):
        return exe
    # Per-process file names, then an atomic rename: test workers running in
    # parallel may build the same kernel at once.
    tag = f"{os.getpid()}"
    path = os.path.join(CACHE, f"nest_{h}.{tag}.hip.inc")
    with open(path, "w") as f:
        f.write(src)
    tmp = f"{exe}.{tag}.tmp"
    cmd = [CLANG, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-ffp-contract=off",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-include", SHIM, f'-DMLK_NEST_SRC="{path}"', HARNESS, "-o", tmp]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    os.remove(path)
    if r.returncode != 0:
        raise RuntimeError("host build of the nest kernel failed:\n" + r.stdout[-4000:])
    os.replace(tmp, exe)
    return exe


def run(src: str, dtypes: Dict[int, str], arrays: Dict[int, np.ndarray], scalars: Sequence[float] = (),
        elements: int = 0, reverse: bool = False) -> Tuple[int, Dict[int, np.ndarray]]:
    """Runs the kernel over `arrays` (buffer id -> values, converted to the
    buffer's device dtype). Returns (status word, buffer id -> result).
    ``reverse`` runs the grid's threads last to first."""
    slots, total = parse_header(src)
    exe = build(src)
    blob = bytearray(struct.pack("<i", len(slots)))
    conv = {}
    for b in slots:
        code, npdt = DT[dtypes[b]]
        a = np.ascontiguousarray(np.asarray(arrays[b]).astype(npdt))
        conv[b] = a
        blob += struct.pack("<iq", code, a.size) + a.tobytes()
    sc = list(scalars)[:8] + [0.0] * (8 - min(8, len(scalars)))
    blob += struct.pack("<8d", *sc)
    blob += struct.pack("<qqq", elements, total, grid_for(total, workgroup_size(src)))
    with tempfile.TemporaryDirectory() as td:
        fin, fout = os.path.join(td, "in.bin"), os.path.join(td, "out.bin")
        with open(fin, "wb") as f:
            f.write(bytes(blob))
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:exitcode=23",
                   UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=24")
        # Inside the host-sanitizer run the parent preloads clang's ASan
        # runtime; this harness links gcc's, and two runtimes refuse to mix.
        pre = [e for e in env.get("LD_PRELOAD", "").split(":") if e and "libclang_rt.asan" not in e]
        if pre:
            env["LD_PRELOAD"] = ":".join(pre)
        else:
            env.pop("LD_PRELOAD", None)
        r = subprocess.run([exe, fin, fout] + (["r"] if reverse else []), stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                           text=True, env=env, timeout=300)
        if r.returncode != 0:
            raise RuntimeError(f"nest kernel failed on the host (rc={r.returncode}):\n" + r.stdout[-6000:])
        raw = open(fout, "rb").read()
    status = struct.unpack_from("<i", raw, 0)[0]
    off = 4
    out = {}
    for b in slots:
        a = conv[b]
        n = a.nbytes
        out[b] = np.frombuffer(raw[off:off + n], dtype=a.dtype).copy()
        off += n
    return status, out


def run_module(km, arrays: Dict[int, np.ndarray], scalars: Sequence[float] = (), elements: int = 0,
               reverse: bool = False, skip_other: bool = False, wg: int = 0) -> Tuple[int, Dict[int, np.ndarray]]:
    """Runs every step of a module whose plan is all loop-nest steps, in order,
    the way the artifact does (temps zeroed first, held in f64). Returns the
    first nonzero status (or 0) and every buffer as f64. ``skip_other`` skips
    steps of other classes instead of refusing (an address check of the
    loop-nest kernels only: the values are then not the module's). ``wg``
    runs launch forms 2 and 3 (512 or 64 threads per workgroup): the form-0
    source behind a leading `#define MLK_NEST_WG`, as the driver builds it."""
    from mlk2_amd import backend
    cls, _, nsteps = backend.plan(km)
    kinds = cls.split("+")
    dtypes = {i: ("f64" if b.is_temp else b.dtype) for i, b in enumerate(km.buffers)}
    cur = {}
    for i, b in enumerate(km.buffers):
        n = b.elements if b.elements >= 0 else elements
        if b.dims:
            n = int(np.prod(b.dims))
        cur[i] = (np.asarray(arrays[i], dtype=np.float64).reshape(-1).copy() if i in arrays
                  else np.zeros(max(n, 0)))
    for s in range(nsteps):
        if kinds[s] == "empty":
            continue
        if kinds[s] != "loop-nest" and skip_other:
            continue
        if kinds[s] != "loop-nest":
            raise ValueError(f"step {s} is a {kinds[s]} step, not a loop-nest step")
        _, src = backend.compile_check(km, s)
        if wg:
            src = f"#define MLK_NEST_WG {wg}\n" + src
        st, out = run(src, dtypes, cur, scalars, elements, reverse)
        for b, v in out.items():
            cur[b] = v.astype(np.float64)
        if st != 0:
            return st, cur
    return 0, cur
