"""mlkhip_run_device_noalloc: the allocation-free variant of mlkhip_run_device.

Its scratch (materialized temps, score-softmax row statistics) comes from one
file-scope device array. Each case runs twice in a row on that array, the
second time on a smaller input, and must match mlkhip_run_device on the same
buffers bit for bit: both run the same kernels. Call(MatMul) takes its
skip-zero-A decision inside its one kernel and needs none of the array; its
case runs a B with infinities (exact blocks) and then a finite one.
"""
import math
import sys

import numpy as np
import pytest

from mlk2_amd import backend
from mlk2_amd import fixtures as fx
from mlk2_amd import inputs
from mlk2_amd.backend import DeviceBuffer
from mlk2_amd.parity import max_rel

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[noalloc] {msg}", flush=True)
    sys.stdout.flush()


def _device_bufs(km, host):
    bufs = {}
    for bid in km.bindable_ids():
        b = km.buffers[bid]
        if b.is_temp:
            continue
        n = int(np.prod(b.dims)) if b.dims else b.elements
        a = host.get(bid, np.zeros(n))
        bufs[bid] = DeviceBuffer.from_array(np.asarray(a, dtype=np.float64).reshape(-1), b.dtype)
    return bufs


def _both(hip, km, host):
    """Outputs of run_device and of run_device_noalloc on fresh buffers."""
    art = hip.build(km)
    ref_bufs = _device_bufs(km, host)
    art.run_device(ref_bufs)
    na_bufs = _device_bufs(km, host)
    art.run_device_noalloc(na_bufs)
    outs = km.output_ids()
    return art, {i: ref_bufs[i].to_numpy() for i in outs}, {i: na_bufs[i].to_numpy() for i in outs}


def test_scratch_array_size(hip):
    assert backend.lib().mlkhip_noalloc_scratch_bytes() == 32 << 20


@pytest.mark.parametrize("m,k", [(256, 512), (64, 256)])
def test_noalloc_materialized_temps(hip, m, k):
    # The generic loop-nest path materializes the softmax temps (row max,
    # exponentials, sums); the smaller second case reuses the array, whose
    # temps must be cleared again.
    km = fx.softmax_rowmax_reader_module(m, k)
    x = inputs.config_inputs("c2", {"m": m, "k": k})["x"]
    art, ref, got = _both(hip, km, {0: x})
    assert art.class_name.startswith("loop-nest")
    for i in ref:
        assert np.array_equal(ref[i].view(np.uint32), got[i].view(np.uint32)), (m, k, i)
    say(f"materialized temps {m}x{k} ({art.class_name}): bit-identical to run_device")


@pytest.mark.parametrize("b,s", [(2, 512), (1, 256)])
def test_noalloc_score_softmax_statistics(hip, b, s):
    km = fx.score_softmax_module(b, s, 128)
    d = inputs.config_inputs("c5", {"batch": b, "seq": s, "dim": 128})
    art, ref, got = _both(hip, km, {0: d["Q"], 1: d["K"], 2: d["bias"]})
    assert art.class_name == "score-softmax"
    for i in ref:
        assert np.array_equal(ref[i].view(np.uint32), got[i].view(np.uint32)), (b, s, i)
    say(f"score-softmax {b}x{s}: bit-identical to run_device")


@pytest.mark.parametrize("m,k,n,bad", [(256, 64, 512, True), (128, 32, 128, False)])
def test_noalloc_matmul_call(hip, m, k, n, bad):
    # The first run has inf in B where A is zero, and a row that reads it:
    # the waves over columns 400-402 recompute their blocks exactly. The
    # second, smaller run has B finite and stores the MFMA result everywhere.
    km = fx.config4_module(m, k, n, "f32", tier=1)
    d = inputs.config_inputs("c4a", {"m": m, "k": k, "n": n})
    A, B = d["A"].astype(np.float64).reshape(m, k), d["B"].astype(np.float64).reshape(k, n)
    if bad:
        B[3, 400:403] = np.inf
        A[:, 3] = 0.0
        A[11, 3] = 0.5
    c0 = inputs.uniform(9, m * n, -1, 1)
    art, ref, got = _both(hip, km, {0: A, 1: B, 2: c0})
    for i in ref:
        assert np.array_equal(ref[i].view(np.uint32), got[i].view(np.uint32)), (m, k, n, i)
        assert int(np.isinf(got[i]).sum()) == (3 if bad else 0)
    say(f"Call(MatMul) {m}x{k}x{n} (non-finite B: {bad}): bit-identical to run_device")


@pytest.mark.parametrize("case", ["score 4x1000", "score 64x128", "gemm f16 1000x600x1000"])
def test_noalloc_padded_shapes(hip, case):
    # Shapes off the fast forms' blocks run on zero-padded copies; here the
    # copies sit in the array (2.1 MiB, 8.3 MiB and 6.5 MiB of its 32 MiB).
    # Bit-identity with run_device shows the padded kernels ran: the general
    # kernels sum in another order.
    if case.startswith("score"):
        b, s = (int(v) for v in case.split()[1].split("x"))
        km = fx.score_softmax_module(b, s, 128)
        d = inputs.config_inputs("c5", {"batch": b, "seq": s, "dim": 128})
        host = {0: d["Q"], 1: d["K"], 2: d["bias"]}
    else:
        m, k, n = 1000, 600, 1000
        km = fx.config4_module(m, k, n, "f16", tier=2)
        d = inputs.config_inputs("c4b", {"m": m, "k": k, "n": n})
        host = {0: d["A"], 1: d["B"]}
    art, ref, got = _both(hip, km, host)
    for i in ref:
        assert np.array_equal(ref[i].view(np.uint32), got[i].view(np.uint32)), (case, i)
    say(f"{case} ({art.step_kernel_name(0)}): bit-identical to run_device")


def test_noalloc_refusals(hip):
    # More scratch than the array holds: refused before anything runs.
    km = fx.softmax_rowmax_reader_module(4096, 1024)
    art = hip.build(km)
    x = np.zeros(4096 * 1024)
    bufs = _device_bufs(km, {0: x})
    with pytest.raises(backend.MlkHipError) as e:
        art.run_device_noalloc(bufs)
    assert e.value.code == backend.REFUSED and "device scratch" in e.value.message
    # A loop nest whose bounds checks report through a host read-back.
    import test_nest as tn
    km = tn.dynamic_end_module()
    art = hip.build(km)
    bufs = _device_bufs(km, {0: np.arange(8.0)})
    with pytest.raises(backend.MlkHipError) as e:
        art.run_device_noalloc(bufs, elements=7)
    assert e.value.code == backend.REFUSED and "read-back" in e.value.message
    say("refusals: oversized scratch, checked loop nest")
