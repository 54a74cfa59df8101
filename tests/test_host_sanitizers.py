"""The host half of libmlk_hip.so under AddressSanitizer and UBSan.

The host sources (the mlk-kernel reader, class recognition and the planner,
the canonical rewrite, the loop-nest generator, the driver, the launch-form
search and the artifact emitter) are compiled with
-fsanitize=address,undefined and linked with the regular build's device
objects into a library of the same name in a temporary directory. The CPU
suite then runs against it in a subprocess (MLK_HIP_LIB), with clang's ASan
runtime preloaded ahead of whatever the environment already preloads. Any
sanitizer report fails the run. CPU only; GPU kernels are not instrumented.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

import pytest

from mlk2_amd import build as mb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-g"]


def _host_flags():
    return [f for f in mb.HOST_FLAGS if f != "-O2"] + ["-O1"] + SAN


def test_cpu_suite_under_host_sanitizers(tmp_path):
    if os.environ.get("MLK_HIP_LIB"):
        pytest.skip("this run already uses the sanitized library")
    dev = [os.path.join(mb.BUILD, s.replace(".hip", ".o")) for s in mb.DEVICE_SOURCES]
    gen = os.path.join(mb.BUILD, "gen")
    if not all(os.path.exists(o) for o in dev) or not os.path.isdir(gen):
        pytest.skip("the regular build's device objects are not there (run __graft_entry__.build())")
    rt = subprocess.run([mb.CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], stdout=subprocess.PIPE,
                        text=True).stdout.strip()
    if not os.path.isabs(rt) or not os.path.exists(rt):
        pytest.skip("clang's shared ASan runtime is not installed")
    objs = []
    jobs = []
    for s in mb.HOST_SOURCES:
        o = str(tmp_path / s.replace(".cpp", ".o"))
        jobs.append([mb.CLANG] + _host_flags() + ["-I", gen, "-c", os.path.join(mb.CSRC, "host", s), "-o", o])
        objs.append(o)
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        for out in ex.map(mb._run, jobs):
            pass
    libdir = tmp_path / "lib"
    libdir.mkdir()
    lib = str(libdir / "libmlk_hip.so")   # the artifact emitter links -lmlk_hip from here
    mb._run([mb.CLANG, "-shared", "-fPIC", "-fsanitize=address,undefined", "-shared-libasan", "-o", lib] + dev + objs +
            [f"-L{mb.ROCM}/lib", "-lamdhip64", "-lhiprtc", f"-Wl,-rpath,{mb.ROCM}/lib"])
    env = dict(os.environ, MLK_HIP_LIB=lib,
               LD_PRELOAD=":".join([rt] + [e for e in os.environ.get("LD_PRELOAD", "").split(":") if e]),
               ASAN_OPTIONS="detect_leaks=0:verify_asan_link_order=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([sys.executable, "-m", "pytest", "tests", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
                        "--deselect", "tests/test_host_sanitizers.py"],
                       cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=1200)
    tail = r.stdout[-6000:]
    assert "ERROR: AddressSanitizer" not in r.stdout and "runtime error:" not in r.stdout, tail
    assert r.returncode == 0, tail
    print(r.stdout.strip().splitlines()[-1], flush=True)
