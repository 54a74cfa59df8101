"""The per-module artifact (mlkhip_emit_artifact): libmlk_kernel.so exporting
`mlk_kernel` exactly as the reference's LoadedKernel::run binds it.

The reference's driver dlsym's `mlk_kernel` (backends/cpu/src/
backend_driver.cpp:427) and calls it through a function pointer typed by the
bindable count (callMultiDim / callLegacy, :223-232, :932-1042): one
(const double*, const int64_t*) pair per bindable buffer in table order and
the scalars pair for multi-dim modules, returning int; the buffer pointers, n
and the scalars pair for legacy 1-D modules, returning void. Temp slots carry
dummies (:853-865). Every module here is serialized exactly as the reference's
writer does (no Call "math", -inf written as -1e308, NaN as null), and the
results are compared with the oracle run on the same module.
"""
import ctypes
import os
import sys

import numpy as np
import pytest

import oracle
from mlk2_amd import backend as be
from mlk2_amd import fixtures as fx
from mlk2_amd import inputs
from mlk2_amd.kernel_ir import is_multidim_module
from mlk2_amd.parity import max_rel, ulp_distance_f32

_PD = ctypes.POINTER(ctypes.c_double)
_PI = ctypes.POINTER(ctypes.c_int64)


def say(msg):
    print(f"[artifact] {msg}", flush=True)
    sys.stdout.flush()


def emit(km, out_dir) -> str:
    text = km.to_reference_json().encode()
    path = ctypes.create_string_buffer(4096)
    rc = be.lib().mlkhip_emit_artifact(text, len(text), b"gfx950", None, str(out_dir).encode(), path, 4096)
    if rc != 0:
        raise be.MlkHipError(rc, be.last_error())
    return path.value.decode()


def bind_mlk_kernel(so_path: str, km):
    """`mlk_kernel` of the artifact with the exact prototype LoadedKernel::run
    calls it through, and whether it is the multi-dim form."""
    lib = ctypes.CDLL(so_path)
    fn = lib.mlk_kernel
    n = len(km.bindable_ids())
    multi = is_multidim_module(km)
    if multi:
        fn.restype = ctypes.c_int
        fn.argtypes = [_PD, _PI] * n + [_PD, ctypes.c_int64]
    else:
        fn.restype = None
        fn.argtypes = [_PD] * n + [ctypes.c_int64, _PD, ctypes.c_int64]
    lib.mlk_kernel_status.restype = ctypes.c_int
    lib.mlk_kernel_status.argtypes = []
    return lib, fn, multi


def call(lib, fn, multi, km, arrays, scalars=(), n_elements=0):
    """Binds like backend_driver.cpp:840-930: table-order (ptr, dims) pairs,
    dummies for temps, the module's own dims; returns outputs and status."""
    keep = []
    args = []
    dummy = (ctypes.c_double * 1)(0.0)
    zero_dim = (ctypes.c_int64 * 1)(0)
    outs = {}
    for bid in km.bindable_ids():
        b = km.buffers[bid]
        if b.is_temp:
            args.append(ctypes.cast(dummy, _PD))
            if multi:
                args.append(ctypes.cast(zero_dim, _PI))
            continue
        n = int(np.prod(b.dims)) if b.dims else (b.elements if b.elements >= 0 else n_elements)
        a = np.ascontiguousarray(np.asarray(arrays.get(bid, np.zeros(n)), dtype=np.float64).reshape(-1)).copy()
        keep.append(a)
        if b.is_output:
            outs[bid] = a
        args.append(a.ctypes.data_as(_PD))
        if multi:
            d = np.asarray(b.dims or [n], dtype=np.int64)
            keep.append(d)
            args.append(d.ctypes.data_as(_PI))
    sc = np.asarray(list(scalars) or [0.0], dtype=np.float64)
    if multi:
        rc = fn(*args, sc.ctypes.data_as(_PD), len(scalars))
    else:
        fn(*args, int(n_elements), sc.ctypes.data_as(_PD), len(scalars))
        rc = lib.mlk_kernel_status()
    return outs, rc


def config_modules():
    """(label, module, inputs, tolerance check) at parity-test sizes."""
    c1 = fx.config1_module(n=1 << 14)
    x1 = inputs.config_inputs("c1", {"n": 1 << 14})["x"]
    c2 = fx.config2_module(64, 512, tier=2)
    x2 = inputs.config_inputs("c2", {"m": 64, "k": 512})["x"]
    c3 = fx.config3_module(64, 512, tier=2)
    d3 = inputs.config_inputs("c3", {"rows": 64, "cols": 512})
    c4 = fx.config4_module(256, 128, 256, "f32", tier=1)
    d4 = inputs.config_inputs("c4a", {"m": 256, "k": 128, "n": 256})
    c4b = fx.config4_module(256, 256, 256, "f16", tier=2)
    d4b = inputs.config_inputs("c4b", {"m": 256, "k": 256, "n": 256})
    c5 = fx.score_softmax_module(2, 256, 128)
    d5 = inputs.config_inputs("c5", {"batch": 2, "seq": 256, "dim": 128})
    return [
        ("c1", c1, {0: x1}, lambda g, r: float(ulp_distance_f32(g.astype(np.float32), r).max()) <= 4.0),
        ("c2", c2, {0: x2}, lambda g, r: max_rel(g, r) <= 1e-6),
        ("c3", c3, {0: d3["x"], 1: d3["b"]}, lambda g, r: max_rel(g, r) <= 1e-6),
        ("c4a", c4, {0: d4["A"], 1: d4["B"]}, lambda g, r: max_rel(g, r) <= 1e-5 * np.sqrt(128)),
        ("c4b", c4b, {0: d4b["A"], 1: d4b["B"]}, lambda g, r: max_rel(g, r) <= 1e-2),
        ("c5", c5, {0: d5["Q"], 1: d5["K"], 2: d5["bias"]}, lambda g, r: max_rel(g, r) <= 1e-2),
    ]


@pytest.mark.parametrize("label,km", [(c[0], c[1]) for c in config_modules()])
def test_artifact_exports_the_reference_prototype(tmp_path, label, km):
    so = emit(km, tmp_path)
    src = open(os.path.join(tmp_path, "mlk_kernel.cpp")).read()
    lib, fn, multi = bind_mlk_kernel(so, km)
    n = len(km.bindable_ids())
    proto = [l for l in src.splitlines() if l.startswith('extern "C" ') and "mlk_kernel(" in l][0]
    if multi:
        assert proto.startswith('extern "C" int mlk_kernel(')
        assert proto.count("const int64_t* p") == n
        assert proto.endswith("const double* mlk_scalars, int64_t mlk_n_scalars) {")
    else:
        assert proto.startswith('extern "C" void mlk_kernel(')
        assert "int64_t n, const double* mlk_scalars, int64_t mlk_n_scalars) {" in proto
    # Stored, output and temp buffers are double*, pure inputs const double*.
    for i, bid in enumerate(km.bindable_ids()):
        b = km.buffers[bid]
        want = "double* " if (b.is_output or b.is_temp) else "const double* "
        assert f"{want}p{i} " in proto or f"{want}p{i}," in proto, (label, i, proto)
    assert hasattr(lib, "mlk_kernel_status")


def test_artifact_reports_no_device_through_its_status(tmp_path):
    # On a host without a HIP device the first call reports ABI code 4, the
    # reference artifact's "no device" (docs/kernel_abi.md:25-40): as the
    # multi-dim return value and through the legacy form's side channel.
    if os.path.exists("/dev/kfd"):
        pytest.skip("a device is present")
    for km, arrays in ((fx.config2_module(4, 8, 2), {0: np.zeros(32)}), (fx.config1_module(64), {0: np.zeros(64)})):
        d = tmp_path / km.name / str(len(km.nodes))
        d.mkdir(parents=True)
        lib, fn, multi = bind_mlk_kernel(emit(km, d), km)
        _, rc = call(lib, fn, multi, km, arrays, n_elements=64)
        assert rc == 4 and lib.mlk_kernel_status() == 4


def test_artifact_refuses_what_the_planner_refuses(tmp_path):
    with pytest.raises(be.MlkHipError) as e:
        emit(fx.config3_tier1_module(64, 128), tmp_path)
    assert "outside its buffer" in e.value.message


@pytest.mark.gpu
@pytest.mark.parametrize("idx", range(6))
def test_artifact_runs_reference_documents_gpu(tmp_path, hip, idx):
    label, km, arrays, ok = config_modules()[idx]
    so = emit(km, tmp_path)
    lib, fn, multi = bind_mlk_kernel(so, km)
    say(f"{label}: {'int' if multi else 'void'} mlk_kernel over {len(km.bindable_ids())} bindables")
    # The legacy form's n is the run's element count (io.elements).
    n = 0 if multi else int(np.asarray(arrays[0]).size)
    outs, rc = call(lib, fn, multi, km, arrays, n_elements=n)
    assert rc == 0, (label, rc)
    ref = oracle.run(km, {i: arrays[i] for i in km.input_ids()})
    for bid, got in outs.items():
        assert ok(got, ref[bid]), (label, bid, max_rel(got, ref[bid]))
    # A second call reuses the process's artifact and gives the same bits.
    outs2, rc2 = call(lib, fn, multi, km, arrays, n_elements=n)
    assert rc2 == 0 and all(np.array_equal(outs2[b], outs[b], equal_nan=True) for b in outs)


@pytest.mark.gpu
def test_artifact_multidim_status_codes_gpu(tmp_path, hip):
    # The walker's negative store address comes back as ABI code 1.
    import test_nest as tn
    km = tn.neg_store_module()
    lib, fn, multi = bind_mlk_kernel(emit(km, tmp_path), km)
    assert multi
    _, rc = call(lib, fn, multi, km, {0: np.arange(4.0)})
    assert rc == 1 and lib.mlk_kernel_status() == 1
