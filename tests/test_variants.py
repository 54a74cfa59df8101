"""Launch-form search (the fastkernel analogue) on the device, through the C
ABI: every declared form of every searched kernel meets the path's
tolerance against the oracle; the search certifies, times and picks among
them without disturbing the caller's buffers; its choice is cached under the
artifact's fingerprint and applied by a later build.

Tolerances as in test_gpu_parity: softmax <= 1e-6 relative; f16 GEMM and
score+softmax <= 1e-2 relative (|got-ref|/max(|ref|,1)); the loop-nest
kernel's forms (with and without LDS slabs) are bit-exact.
"""
import math
import sys

import numpy as np
import pytest

import oracle
from mlk2_amd import fixtures as fx
from mlk2_amd import inputs
from mlk2_amd import backend as be
from mlk2_amd.backend import DeviceBuffer, MlkHipError, lib
from mlk2_amd.parity import max_rel

pytestmark = pytest.mark.gpu


def launched_workgroups(name, v):
    """Workgroups the launcher of form `v` starts for the autotune cases, from
    the launchers: softmax form 5 two rows per wave (4 waves a workgroup),
    form 1 a grid of min(rows, 2048) waves, the others a row per wave; f16
    GEMM forms 5 and 6 on 128 x 256 tiles, the others 256 x 256; f32 GEMM
    64 x 64; score-softmax form 0 128 rows x 2 key halves per pass, form 1
    64 x 128 score tiles. The launch certificate must name the chosen form's
    geometry."""
    if name == "softmax-512x4096":
        return {5: (256 + 3) // 4, 1: (512 + 3) // 4}.get(v, (512 + 3) // 4)
    if name == "gemm-f16-512x1024x512":
        return (512 // 128) * (512 // 256) if v in (5, 6) else (512 // 256) ** 2
    if name == "gemm-f32-256x1024x512":
        return (256 // 64) * (512 // 64)
    if name == "score-2x512x128":
        return 2 * (512 // 128) * 2 if v != 1 else 2 * (512 // 64) * (512 // 128)
    return None

def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def _gemm_ref(A, B):
    m, k = A.shape
    call = fx.matmul_call_module(m, k, B.shape[1], "f64", "f64")
    return oracle.run(call, {0: A, 1: B}, hw_threads=8)[2].reshape(m, B.shape[1])


def _score_ref(Q, K, bias):
    B, S, D = Q.shape
    out = []
    for b in range(B):
        sc = _gemm_ref(Q[b].astype(np.float64), np.ascontiguousarray(K[b].astype(np.float64).T))
        sc = sc / math.sqrt(D) + bias.astype(np.float64)
        out.append(oracle.run(fx.softmax_call_module(S, S, "f64"), {0: sc})[1].reshape(S, S))
    return np.concatenate(out)


def _softmax_case(m=512, k=4096):
    x = inputs.normal(inputs.SEEDS["c2_x"], m * k, 0.0, 2.0).reshape(m, k)
    km = fx.config2_module(m, k, 2)
    ref = oracle.run(fx.config2_module(m, k, 1), {0: x})[1]
    bufs = {0: DeviceBuffer.from_array(x, "f32"), 1: DeviceBuffer(m * k, "f32")}
    return km, bufs, 1, ref, 1e-6


def _gemm_case(m=512, k=1024, n=512):
    d = inputs.config_inputs("c4b", {"m": m, "k": k, "n": n})
    km = fx.config4_module(m, k, n, "f16", 2)
    ref = _gemm_ref(d["A"].astype(np.float64), d["B"].astype(np.float64)).reshape(-1)
    bufs = {0: DeviceBuffer.from_array(d["A"], "f16"), 1: DeviceBuffer.from_array(d["B"], "f16"),
            2: DeviceBuffer(m * n, "f32")}
    return km, bufs, 2, ref, 1e-2


def _gemm_f32_case(m=256, k=1024, n=512):
    # f32 forms 0 (direct to the LDS ring, k permuted within a step) and 1
    # (register-staged, k ascending): within 1e-5 sqrt(k) of the f64 product.
    d = inputs.config_inputs("c4a", {"m": m, "k": k, "n": n})
    km = fx.config4_module(m, k, n, "f32", 2)
    ref = _gemm_ref(d["A"].astype(np.float64), d["B"].astype(np.float64)).reshape(-1)
    bufs = {0: DeviceBuffer.from_array(d["A"], "f32"), 1: DeviceBuffer.from_array(d["B"], "f32"),
            2: DeviceBuffer(m * n, "f32")}
    return km, bufs, 2, ref, 1e-5 * math.sqrt(k)


def _score_case(b=2, s=512, dm=128):
    d = inputs.config_inputs("c5", {"batch": b, "seq": s, "dim": dm})
    km = fx.score_softmax_module(b, s, dm)
    ref = _score_ref(d["Q"], d["K"], d["bias"]).reshape(-1)
    bufs = {0: DeviceBuffer.from_array(d["Q"], "f16"), 1: DeviceBuffer.from_array(d["K"], "f16"),
            2: DeviceBuffer.from_array(d["bias"], "f32"), 3: DeviceBuffer(b * s * s, "f32")}
    return km, bufs, 3, ref, 1e-2


def _gemm_call_acc_case(m=256, k=128, n=512):
    # Call(MatMul) adds into C (kernel_buffers.cpp:406-432): the accumulate
    # form of every kernel.
    d = inputs.config_inputs("c4b", {"m": m, "k": k, "n": n})
    c0 = inputs.uniform(9, m * n, -1, 1)
    km = fx.matmul_call_module(m, k, n, "f16", "f32")
    ref = oracle.run(km, {0: d["A"], 1: d["B"]}, init={2: c0})[2]

    class InitialC(DeviceBuffer):
        """The output buffer; "zeroing" it restores the initial C."""

        def fill_zero(self):
            host = np.ascontiguousarray(c0.astype(np.float32))
            assert lib().mlkhip_memcpy_h2d(self.ptr, host.ctypes.data, self.nbytes) == 0

    out = InitialC(m * n, "f32")
    bufs = {0: DeviceBuffer.from_array(d["A"], "f16"), 1: DeviceBuffer.from_array(d["B"], "f16"), 2: out}
    return km, bufs, 2, ref, 1e-2


def _nest_case(m=64, n=256, k=41):
    # The generic loop-nest kernel with LDS slabs (form 0), without them (1),
    # at 512 and 64 threads per workgroup (2, 3) and with one fewer collapsed
    # loop (4): each instance computed with the same operations, so every
    # form is bit-exact.
    from test_nest import generic, weighted_rows_inputs, weighted_rows_module
    km = generic(weighted_rows_module(M=m, N=n, K=k, off=7, dtype="f32"))
    arr = weighted_rows_inputs(km)
    ref = oracle.run(km, arr)[2].astype(np.float32).astype(np.float64)
    bufs = {0: DeviceBuffer.from_array(arr[0], "f32"), 1: DeviceBuffer.from_array(arr[1], "f32"),
            2: DeviceBuffer(m * n, "f32")}
    return km, bufs, 2, ref, 0.0


CASES = {
    "gemm-f16-call-accumulate": _gemm_call_acc_case,
    "softmax-512x4096": _softmax_case,
    "softmax-333x1000": lambda: _softmax_case(333, 1000),
    "softmax-70001x8": lambda: _softmax_case(70001, 8),
    "gemm-f16-512x1024x512": _gemm_case,
    "gemm-f32-256x1024x512": _gemm_f32_case,
    "score-2x512x128": _score_case,
    "score-1x2048x128": lambda: _score_case(1, 2048, 128),
    "nest-slabs-64x256x41": _nest_case,
}


@pytest.mark.parametrize("name", list(CASES))
def test_every_declared_form_meets_tolerance(hip, name):
    km, bufs, out, ref, tol = CASES[name]()
    art = hip.build(km)
    space = art.step_variants(0)
    assert len(space) >= 2, name
    for v in space:
        say(f"variants {name} form {v}")
        art.set_step_variant(0, v)
        assert art.step_variant(0) == v
        bufs[out].fill_zero()
        art.run_device(bufs)
        e = max_rel(bufs[out].to_numpy(), ref)
        say(f"variants {name} form {v} max_rel={e:.3e}")
        assert e <= tol, (name, v)


@pytest.mark.parametrize("m,k", [(512, 4096), (333, 1000), (70001, 8)])
def test_softmax_forms_with_one_arithmetic_agree_bitwise(hip, m, k):
    # Forms 5, 0 and 3 share the v_exp_f32 / grouped-sum row body and differ
    # only in launch shape and store kind; forms 2, 4 and 1 share the expf /
    # per-element-f64 body. Within each family the outputs are identical.
    km, bufs, out, _, _ = _softmax_case(m, k)
    art = hip.build(km)
    got = {}
    for v in art.step_variants(0):
        art.set_step_variant(0, v)
        bufs[out].fill_zero()
        art.run_device(bufs)
        got[v] = bufs[out].to_numpy().astype(np.float32).view(np.uint32)
    for family in ([5, 0, 3], [2, 4, 1]):
        for v in family[1:]:
            assert np.array_equal(got[family[0]], got[v]), (m, k, family[0], v)


def test_set_variant_outside_space_refused(hip):
    km, _, _, _, _ = _softmax_case(64, 256)
    art = hip.build(km)
    with pytest.raises(MlkHipError):
        art.set_step_variant(0, 99)
    with pytest.raises(MlkHipError):
        art.set_step_variant(5, 0)
    art.set_step_variant(0, -1)
    assert art.step_variant(0) == -1
    assert art.step_variant(7) == -2


@pytest.mark.parametrize("name", ["softmax-512x4096", "gemm-f16-512x1024x512", "gemm-f32-256x1024x512",
                                  "score-2x512x128", "nest-slabs-64x256x41"])
def test_autotune_certifies_restores_and_caches(hip, name, tmp_path):
    km, bufs, out, ref, tol = CASES[name]()
    # A sentinel in the output: the search must hand the buffer back as it was.
    n_out = bufs[out].elements
    sentinel = np.full(n_out, 0.75, dtype=np.float32)
    bufs[out].free()
    bufs[out] = DeviceBuffer.from_array(sentinel, "f32")
    art = hip.build(km, cache_dir=str(tmp_path))
    assert not art.variants_from_cache
    fp = art.fingerprint
    assert len(fp) == 16
    say(f"autotune {name} start")
    rep = art.autotune(bufs, reps=5, cache_dir=str(tmp_path))
    say(f"autotune {name} chose {rep['variants']}")
    assert rep["fingerprint"] == fp
    assert rep["combined_certified"] is True
    assert np.array_equal(bufs[out].to_numpy(), sentinel)
    (step,) = rep["steps"]
    space = art.step_variants(0)
    assert [c["variant"] for c in step["candidates"]] == space
    assert step["chosen"] in space
    chosen = [c for c in step["candidates"] if c["variant"] == step["chosen"]][0]
    assert chosen["admissible"] and chosen["certificate"]["identity"]["certified"]
    rt = chosen["certificate"]["runtime"]
    assert 0 < rt["min_sec"] <= rt["upper_bound_sec"] <= rt["max_sec"]
    for c in step["candidates"]:
        if c["admissible"]:
            assert c["certificate"]["runtime"]["upper_bound_sec"] >= rt["upper_bound_sec"]
        else:
            assert c["rejected"]["reason"] in ("identity-mismatch", "build-failed")
    assert art.step_variant(0) == step["chosen"]
    # Work model, roofline bound and the winner's gap over it; the step's
    # launch-coverage certificate.
    assert rep["work"]["bytes_known"] and rep["work"]["min_bytes"] > 0
    assert rep["roofline_lower_sec"] > 0 and rep["winner_sec"] > rep["roofline_lower_sec"]
    assert abs(rep["winner_gap_over_lower"] - (rep["winner_sec"] / rep["roofline_lower_sec"] - 1)) < 1e-3
    assert step["launch"]["covered"] and step["launch"]["workgroups"] > 0
    expect = launched_workgroups(name, step["chosen"])
    if expect is not None:
        assert step["launch"]["workgroups"] == expect, (name, step["chosen"], step["launch"])
    env = rep["environment"]
    assert 1e12 < env["measured_bytes_per_sec"] < 1e13 and 1e14 < env["measured_f16_flops_per_sec"] < 3e15
    assert rep["roofline_lower_sec_measured"] >= rep["roofline_lower_sec"]
    # The chosen form meets the path's tolerance against the oracle.
    bufs[out].fill_zero()
    art.run_device(bufs)
    assert max_rel(bufs[out].to_numpy(), ref) <= tol
    # A second build with the same cache directory applies the choice.
    assert rep["cache"]["file"].endswith(f"fk-{fp}.json")
    art2 = hip.build(km, cache_dir=str(tmp_path))
    assert art2.fingerprint == fp
    assert art2.variants_from_cache
    assert art2.step_variant(0) == step["chosen"]
    # Another shape has another fingerprint and ignores the entry.
    km3, _, _, _, _ = (_softmax_case(256, 4096) if name.startswith("softmax") else
                       _gemm_case(256, 1024, 512) if name.startswith("gemm") else
                       _nest_case(32, 256, 41) if name.startswith("nest") else _score_case(1, 512, 128))
    art3 = hip.build(km3, cache_dir=str(tmp_path))
    assert art3.fingerprint != fp
    assert not art3.variants_from_cache


def test_autotune_without_variants_is_a_no_op(hip):
    # A 1-D elementwise chain has one form: the search times nothing and
    # keeps defaults.
    n = 1 << 16
    d = inputs.config_inputs("c1", {"n": n})
    km = fx.config1_module(n=n)
    art = hip.build(km)
    bufs = {0: DeviceBuffer.from_array(d["x"], "f32"), 1: DeviceBuffer(n, "f32")}
    rep = art.autotune(bufs, reps=3)
    assert rep["steps"] == [] and rep["variants"] == [-1]
    assert rep["cache"]["file"] == ""


def test_measured_environment(hip):
    env = be.measure_environment()
    say(f"environment: {env['bytes_per_sec'] / 1e12:.2f} TB/s HBM, "
        f"{env['f16_flops_per_sec'] / 1e12:.0f} TFLOP/s f16 MFMA")
    assert 1e12 < env["bytes_per_sec"] < 1e13
    assert 1e14 < env["f16_flops_per_sec"] < 3e15
    assert be.measure_environment() == env           # probed once per process
