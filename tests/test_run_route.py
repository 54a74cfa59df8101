"""The run route: `mlkc run` on the HIP backend (mlk2_amd/run.py) over the C
ABI's execute entries, which stand in for executeKernel / executeKernelOnBuffers
(runtime/src/execution/execution.cpp:195-256, kernel_buffers.cpp:839-1106)
behind an ExecutionEngine hook.

CPU tests cover argument handling and error paths (no device: exit code 1
with the library's status). GPU tests pin results: the sin graph at x = 2
(examples/scalar/README.md:9, tests/differential/differential_test.cpp:44-48:
-0.5440211108893698, <= 1e-13) and bit-exact f64 tensor kernels against the
oracle, through the library entries and through the command line.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from mlk2_amd import backend as be
from mlk2_amd import fixtures as fx
from mlk2_amd import run as route

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = json.load(open(os.path.join(ROOT, "tests", "golden", "oracle_golden.json")))


def _write(tmp_path, km, name="module.json"):
    p = tmp_path / name
    p.write_text(km.to_json())
    return str(p)


@pytest.mark.parametrize("argv", [
    ["m.json", "--backend=cpu"],
    ["m.json", "--arch=sm_90"],
    ["m.json", "--elements=-1"],
    ["m.json", "--x=1", "--input=a.npy"],
    ["m.json", "--bogus"],
    [],
])
def test_bad_command_lines_are_usage_errors(argv):
    with pytest.raises(route.UsageError):
        route.parse_args(argv)


def test_good_command_line():
    a = route.parse_args(["m.json", "--backend=hip", "--arch=gfx950", "--x=2.0", "--x=-1"])
    assert (a.module, a.arch, a.xs) == ("m.json", "gfx950", [2.0, -1.0])


def test_module_text_keeps_the_document(tmp_path):
    km = fx.config1_module(1 << 10, dtype="f64")
    mt = route.load_module(_write(tmp_path, km))
    assert mt.to_json() == km.to_json()
    assert [(b.is_input, b.is_output) for b in mt.buffers] == [(True, False), (False, True)]
    with pytest.raises(ValueError):
        route.ModuleText(json.dumps({"format": "other", "buffers": []}))


def test_missing_module_is_exit_2(tmp_path, capsys):
    rc = route.run(route.parse_args([str(tmp_path / "none.json")]))
    assert rc == 2


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="checks the no-device path")
def test_no_device_is_exit_1_with_status(tmp_path, capsys):
    rc = route.main([_write(tmp_path, fx.sin_graph_scalar_module()), "--x=2"])
    err = capsys.readouterr().err
    assert rc == 1 and "status 4" in err


# ---------------------------------------------------------------- GPU ----
@pytest.mark.gpu
def test_scalar_sin_graph_known_answer(hip):
    ka = GOLDEN["known_answers"]["sin_graph_at_2"]
    km = fx.sin_graph_scalar_module()
    (y,) = be.execute_kernel(km, [ka["x"]])
    ref = oracle.run(km, {}, scalars=[ka["x"]])[0][0]
    assert abs(y - ka["y"]) <= ka["tol"]
    assert np.float64(y).view(np.int64) == np.float64(ref).view(np.int64)


@pytest.mark.gpu
def test_buffers_entry_bit_exact_and_cached(hip):
    be.lib().mlkhip_execute_cache_clear()
    n = 5000
    x = np.linspace(-30.0, 30.0, n)
    km = fx.config1_module(n, dtype="f64")
    y = np.zeros(n)
    be.execute_kernel_on_buffers(km, [x], [y])
    ref = oracle.run(km, {0: x})[1]
    assert np.array_equal(y.view(np.int64), ref.view(np.int64))
    assert be.lib().mlkhip_execute_cache_size() == 1
    y2 = np.zeros(n)
    be.execute_kernel_on_buffers(km, [x], [y2])        # same module: cached artifact
    assert be.lib().mlkhip_execute_cache_size() == 1
    assert np.array_equal(y2, y)
    # Call(MatMul) reads and writes its output (C += A B): the reference GEMM
    # fixture (unit_poly.cpp:2024-2056) starting from C = 0.
    M, K, N = 8, 6, 7
    A = np.array([((i * 7) % 13) * 0.25 for i in range(M * K)])
    B = np.array([((i * 5) % 11) * 0.5 for i in range(K * N)])
    C = np.zeros(M * N)
    be.execute_kernel_on_buffers(fx.matmul_call_module(M, K, N, "f64", "f64"), [A, B], [C])
    assert [float(v).hex() for v in C] == GOLDEN["known_answers"]["gemm_8x6x7_unit_poly"]["C"]
    assert be.lib().mlkhip_execute_cache_size() == 2


@pytest.mark.gpu
def test_buffers_entry_rejects_missing_output(hip):
    km = fx.config1_module(64, dtype="f64")
    with pytest.raises(be.MlkHipError) as ei:
        be.execute_kernel_on_buffers(km, [np.zeros(64)], [])
    assert ei.value.code == be.BAD_BINDING


@pytest.mark.gpu
def test_command_line_scalar_and_tensor(hip, tmp_path):
    env = dict(os.environ, PYTHONPATH=ROOT)
    ka = GOLDEN["known_answers"]["sin_graph_at_2"]
    mod = _write(tmp_path, fx.sin_graph_scalar_module(), "sin.json")
    r = subprocess.run([sys.executable, "-m", "mlk2_amd.run", mod, "--backend=hip", f"--x={ka['x']}"],
                       capture_output=True, text=True, env=env, cwd=ROOT, timeout=120)
    assert r.returncode == 0, r.stderr
    y = float(r.stdout.strip().split("=")[1])
    assert abs(y - ka["y"]) <= ka["tol"]
    assert "executed backend=hip" in r.stderr
    n = 1000
    x = np.linspace(-5.0, 5.0, n)
    np.save(tmp_path / "x.npy", x)
    km = fx.config1_module(n, dtype="f64")
    mod = _write(tmp_path, km, "c1.json")
    r = subprocess.run([sys.executable, "-m", "mlk2_amd.run", mod, f"--input={tmp_path / 'x.npy'}",
                        f"--out={tmp_path / 'o'}"], capture_output=True, text=True, env=env, cwd=ROOT,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    got = np.load(tmp_path / "o" / "out0.npy")
    assert np.array_equal(got.view(np.int64), oracle.run(km, {0: x})[1].view(np.int64))
