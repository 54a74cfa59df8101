"""Executor semantics at the boundary, on the device, against the oracle.

* Call(MatMul) skips A[i,p] == 0 (gemmRowBlock, runtime/src/execution/
  kernel_buffers.cpp:422): 0 * inf or 0 * NaN in B must not reach C. Only
  there can the skip change C, and there the MFMA accumulators of every row
  of those columns come out non-finite; inside the one MFMA launch, a wave
  whose block holds such a value recomputes it exactly with the skip, and
  the other waves store the MFMA result.
* A fused class keeps its temps on chip only when no other root reads them;
  a later root that reads the softmax row max, or the scaled scores, makes
  the nest run with the walker's materialized temps (kernel_buffers.cpp:
  902-920).
* Modules serialized exactly as the reference's writer does them (Call
  targets without "math", -inf as -1e308, NaN as null) run like the
  lossless document, all-(-inf) softmax rows included.
* Each stream gets its own artifact scratch, so runs of one artifact on two
  streams at once do not share temps.
* The host-buffer ABI moves buffers through the artifact's page-locked
  staging chunk by chunk, one call at a time per artifact.
"""
import math
import sys

import numpy as np
import pytest

import oracle
from mlk2_amd import backend
from mlk2_amd import fixtures as fx
from mlk2_amd import inputs
from mlk2_amd.backend import DeviceBuffer
from mlk2_amd.parity import max_rel

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[boundary] {msg}", flush=True)
    sys.stdout.flush()


def same_class_close(got, ref, tol):
    """Same NaN positions, same infinities, |got-ref|/max(|ref|,1) <= tol."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "NaN positions differ"
    inf = np.isinf(ref)
    assert np.array_equal(got[inf], ref[inf]), "infinities differ"
    fin = np.isfinite(ref)
    return max_rel(got[fin], ref[fin]) <= tol


def test_skip_zero_a_reference_fixture(hip):
    # The oracle's own fixture (2x2, f64): C stays finite where A[i,p] == 0
    # meets B[p,j] = inf, and is inf where A[i,p] != 0 does.
    A = np.array([0.0, 1.0, 2.0, 3.0])
    B = np.array([np.inf, 1.0, 1.0, 1.0])
    C0 = np.array([10.0, 20.0, 30.0, 40.0])
    call = fx.matmul_call_module(2, 2, 2, "f64", "f64")
    got = hip.build(call).run({0: A, 1: B, 2: C0})[2]
    ref = oracle.run(call, {0: A, 1: B}, init={2: C0})[2]
    say(f"skip-zero-A 2x2 f64: {got.tolist()} (oracle {ref.tolist()})")
    assert got.tolist() == [11.0, 21.0, np.inf, 45.0]
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("dt_in,dt_out,m,k,n", [("f32", "f32", 256, 64, 256), ("f16", "f32", 256, 256, 256),
                                                ("f64", "f64", 70, 33, 65), ("f32", "f32", 1024, 1024, 1024)])
def test_skip_zero_a_with_nonfinite_b(hip, dt_in, dt_out, m, k, n):
    # Shapes that take the MFMA forms when B is finite. A holds zeros in some
    # columns p whose B rows hold inf, -inf or NaN; the rows of A that are
    # non-zero there make those C entries non-finite, the rest stay finite.
    rng = np.random.default_rng(5)
    A = rng.uniform(-1, 1, (m, k))
    B = rng.uniform(-1, 1, (k, n))
    for p, bad in ((3, np.inf), (k // 2, -np.inf), (k - 1, np.nan)):
        B[p, rng.integers(0, n, 8)] = bad
        A[:, p] = 0.0
        A[rng.integers(0, m, 2), p] = 0.5     # two rows read the non-finite values
    np_dt = {"f32": np.float32, "f16": np.float16, "f64": np.float64}[dt_in]
    A = A.astype(np_dt).astype(np.float64)
    B = B.astype(np_dt).astype(np.float64)
    C0 = rng.uniform(-1, 1, m * n)
    call = fx.matmul_call_module(m, k, n, dt_in, dt_out)
    ref = oracle.run(call, {0: A.reshape(-1), 1: B.reshape(-1)}, init={2: C0})[2]
    got = hip.build(call).run({0: A, 1: B, 2: C0})[2]
    nonfinite = int((~np.isfinite(ref)).sum())
    tol = 1e-12 if dt_in == "f64" else (1e-5 * math.sqrt(k) if dt_in == "f32" else 1e-2)
    ok = same_class_close(got, ref, tol)
    say(f"skip-zero-A {dt_in} {m}x{k}x{n}: {nonfinite} non-finite outputs, all finite ones within {tol:g}: {ok}")
    assert 0 < nonfinite < m * n // 4 and ok
    # The same inputs with B finite run the MFMA forms and still match.
    Bf = np.where(np.isfinite(B), B, 0.25)
    ref2 = oracle.run(call, {0: A.reshape(-1), 1: Bf.reshape(-1)}, init={2: C0})[2]
    got2 = hip.build(call).run({0: A, 1: Bf, 2: C0})[2]
    assert np.isfinite(got2).all() and max_rel(got2, ref2) <= tol


@pytest.mark.parametrize("dt_in,m,k,n,variant", [("f16", 512, 256, 1024, None), ("f16", 512, 256, 1024, 7),
                                                  ("f16", 256, 128, 1024, 5), ("f32", 256, 128, 512, None)])
def test_skip_zero_a_mixes_mfma_and_exact_tiles(hip, dt_in, m, k, n, variant):
    # Non-finite values of B only in columns 300-309. The waves whose blocks
    # hold those columns recompute them exactly; every other wave stores its
    # MFMA result, in one run, with C accumulated from a non-zero start.
    rng = np.random.default_rng(6)
    A = rng.uniform(-1, 1, (m, k))
    B = rng.uniform(-1, 1, (k, n))
    B[5, 300:305] = np.inf
    B[k - 2, 305:310] = np.nan
    A[:, 5] = 0.0
    A[:, k - 2] = 0.0
    A[7, 5] = 0.25                               # row 7 reads the infinities
    np_dt = {"f32": np.float32, "f16": np.float16}[dt_in]
    A = A.astype(np_dt).astype(np.float64)
    B = B.astype(np_dt).astype(np.float64)
    C0 = rng.uniform(-1, 1, m * n)
    call = fx.matmul_call_module(m, k, n, dt_in, "f32")
    art = hip.build(call)
    if variant is not None:
        art.set_step_variant(0, variant)
    ref = oracle.run(call, {0: A.reshape(-1), 1: B.reshape(-1)}, init={2: C0})[2]
    got = art.run({0: A, 1: B, 2: C0})[2]
    tol = 1e-5 * math.sqrt(k) if dt_in == "f32" else 1e-2
    nonfinite = int((~np.isfinite(ref)).sum())
    ok = same_class_close(got, ref, tol)
    say(f"skip-zero-A mixed {dt_in} {m}x{k}x{n} form {variant}: {nonfinite} non-finite outputs, close: {ok}")
    assert nonfinite == 5 and ok


@pytest.mark.parametrize("dt_in,m,k,n", [("f16", 512, 256, 512), ("f32", 128, 128, 128)])
def test_skip_zero_a_every_declared_form(hip, dt_in, m, k, n):
    # Every launch form of the Call(MatMul) step takes the skip inside its
    # own kernel: the waves whose blocks hold columns 300-302 (f16) or 70-72
    # (f32) of B, where inf meets A[i,p] == 0, recompute exactly; the rest
    # store their MFMA result. Each form is held to the oracle.
    rng = np.random.default_rng(8)
    A = rng.uniform(-1, 1, (m, k))
    B = rng.uniform(-1, 1, (k, n))
    c0 = 300 if n > 300 else 70
    B[9, c0:c0 + 3] = np.inf
    B[k - 3, c0 + 1] = np.nan
    A[:, 9] = 0.0
    A[:, k - 3] = 0.0
    A[5, 9] = -0.75                              # row 5 reads the infinities
    np_dt = {"f32": np.float32, "f16": np.float16}[dt_in]
    A = A.astype(np_dt).astype(np.float64)
    B = B.astype(np_dt).astype(np.float64)
    C0 = rng.uniform(-1, 1, m * n)
    call = fx.matmul_call_module(m, k, n, dt_in, "f32")
    ref = oracle.run(call, {0: A.reshape(-1), 1: B.reshape(-1)}, init={2: C0})[2]
    art = hip.build(call)
    forms = art.step_variants(0)
    assert forms, "the Call(MatMul) step declares its launch forms"
    tol = 1e-5 * math.sqrt(k) if dt_in == "f32" else 1e-2
    for form in forms:
        art.set_step_variant(0, form)
        got = art.run({0: A, 1: B, 2: C0})[2]
        ok = same_class_close(got, ref, tol)
        say(f"skip-zero-A {dt_in} {m}x{k}x{n} form {form}: {int((~np.isfinite(got)).sum())} non-finite, close: {ok}")
        assert ok, form
    art.set_step_variant(0, -1)
    assert int((~np.isfinite(ref)).sum()) == 3


def test_skip_zero_a_f32_overflow_takes_the_exact_path(hip):
    # Finite f32 operands whose products overflow make non-finite
    # accumulators with B finite; those blocks take the exact path, which
    # computes the same overflow the reference does.
    m = k = n = 128
    rng = np.random.default_rng(9)
    A = rng.uniform(-1, 1, (m, k)).astype(np.float32).astype(np.float64)
    B = rng.uniform(-1, 1, (k, n)).astype(np.float32).astype(np.float64)
    A[3, 0] = 3e38
    B[0, 7] = 2.0                                # 6e38: +inf in f32
    A[4, 1] = -3e38
    B[1, 8] = 4.0                                # -inf
    C0 = np.zeros(m * n)
    call = fx.matmul_call_module(m, k, n, "f32", "f32")
    ref = oracle.run(call, {0: A.reshape(-1), 1: B.reshape(-1)}, init={2: C0})[2]
    got = hip.build(call).run({0: A, 1: B, 2: C0})[2]
    # The oracle accumulates in f64, where these sums stay finite; the f32
    # output rounds them to inf. Compare in f32.
    ref32 = ref.astype(np.float32).astype(np.float64)
    assert np.isposinf(got.reshape(m, n)[3, 7]) and np.isneginf(got.reshape(m, n)[4, 8])
    ok = same_class_close(got, ref32, 1e-5 * math.sqrt(k))
    say(f"f32 overflow: {int(np.isinf(got).sum())} infinities, finite ones close: {ok}")
    assert ok


def test_fused_softmax_temps_read_by_a_later_root(hip):
    km = fx.softmax_rowmax_reader_module(32, 256)
    x = inputs.config_inputs("c2", {"m": 32, "k": 256})["x"]
    art = hip.build(km)
    say(f"softmax + row-max reader: {art.class_name}")
    assert not art.class_name.startswith("softmax-nest")
    got = art.run({0: x})
    ref = oracle.run(km, {0: x})
    ids = km.output_ids()
    assert max_rel(got[ids[0]], ref[ids[0]]) <= 1e-6
    # The row max read back is the walker's, bit for bit (an f32 buffer's max).
    assert np.array_equal(got[ids[1]], ref[ids[1]])
    assert np.array_equal(got[ids[1]], x.astype(np.float64).max(axis=1))


def test_fused_score_temps_read_by_a_later_root(hip):
    km = fx.score_reader_module(1, 256, 128)
    d = inputs.config_inputs("c5", {"batch": 1, "seq": 256, "dim": 128})
    arrays = {0: d["Q"], 1: d["K"], 2: d["bias"]}
    art = hip.build(km)
    say(f"score-softmax + score reader: {art.class_name}")
    assert "score-softmax" not in art.class_name
    got = art.run(arrays)
    ref = oracle.run(km, arrays)
    for i in km.output_ids():
        assert max_rel(got[i], ref[i]) <= 1e-5, (i, max_rel(got[i], ref[i]))


@pytest.mark.parametrize("km_name", ["c2_call", "c2_synth", "c4_call", "c5", "rowsum_call"])
def test_reference_documents_run_like_lossless_ones(hip, km_name):
    m, k = 64, 512
    x = inputs.config_inputs("c2", {"m": m, "k": k})["x"].astype(np.float64)
    x[3, :] = -np.inf                              # all -inf row: NaN in the walker (-inf - -inf)
    x[7, :] = np.nan
    x[9, 5] = np.inf
    if km_name == "c2_call":
        km, arrays = fx.config2_module(m, k, 1), {0: x}
    elif km_name == "c2_synth":
        km, arrays = fx.config2_module(m, k, 2), {0: x}
    elif km_name == "rowsum_call":
        km, arrays = fx.reducesum_call_module(m, k), {0: x}
    elif km_name == "c4_call":
        d = inputs.config_inputs("c4a", {"m": 256, "k": 128, "n": 256})
        km, arrays = fx.config4_module(256, 128, 256, "f32", 1), {0: d["A"], 1: d["B"]}
    else:
        d = inputs.config_inputs("c5", {"batch": 2, "seq": 256, "dim": 128})
        km, arrays = fx.score_softmax_module(2, 256, 128), {0: d["Q"], 1: d["K"], 2: d["bias"]}
    a_ref = hip.build(km, reference_document=True)
    a_ext = hip.build(km)
    assert a_ref.class_name == a_ext.class_name
    got = a_ref.run(arrays)
    ext = a_ext.run(arrays)
    ref = oracle.run(km, {i: arrays[i] for i in km.input_ids()})
    tol = {"c2_call": 1e-6, "c2_synth": 1e-6, "rowsum_call": 1e-6, "c4_call": 1e-5 * math.sqrt(128),
           "c5": 1e-2}[km_name]
    for i in km.output_ids():
        assert np.array_equal(got[i], ext[i], equal_nan=True)
        assert same_class_close(got[i], ref[i], tol), (km_name, i)
    say(f"reference document {km_name}: {a_ref.class_name}, same bits as the lossless document")


def test_runs_on_two_streams_use_separate_scratch(hip):
    # The generic loop-nest path materializes the softmax temps; two runs of
    # one artifact in flight on two streams must not share them.
    km = fx.softmax_rowmax_reader_module(256, 512)
    art = hip.build(km)
    assert art.class_name.startswith("loop-nest")
    xs = [inputs.config_inputs("c2", {"m": 256, "k": 512})["x"], None]
    xs[1] = (xs[0][::-1] * 0.5).copy()
    lib = backend.lib()
    import ctypes
    streams = []
    for _ in range(2):
        s = ctypes.c_void_p()
        assert lib.mlkhip_stream_create(ctypes.byref(s)) == 0
        streams.append(s.value)
    ids = km.output_ids()
    bufs = []
    for x in xs:
        b = {0: DeviceBuffer.from_array(x, "f32")}
        for i in ids:
            b[i] = DeviceBuffer(km.buffers[i].elements, "f32")
        bufs.append(b)
    for rep in range(3):
        for b, s in zip(bufs, streams):
            art.run_device(b, stream=s, sync=False)
    assert lib.mlkhip_synchronize() == 0
    for x, b in zip(xs, bufs):
        ref = oracle.run(km, {0: x})
        assert max_rel(b[ids[0]].to_numpy(), ref[ids[0]]) <= 1e-6
        assert np.array_equal(b[ids[1]].to_numpy().astype(np.float64), ref[ids[1]])
    # Each stream's set is released before its stream is destroyed; a run
    # after a release allocates a new set, with its temps cleared as ever.
    for s in streams:
        art.release_stream_scratch(s)
    art.run_device(bufs[1], stream=streams[0], sync=False)
    assert lib.mlkhip_synchronize() == 0
    ref = oracle.run(km, {0: xs[1]})
    assert max_rel(bufs[1][ids[0]].to_numpy(), ref[ids[0]]) <= 1e-6
    for s in streams:
        art.release_stream_scratch(s)
        lib.mlkhip_stream_destroy(s)
    art.release_stream_scratch(streams[0])          # not held: nothing to do
    say("two streams, separate scratch: both runs match the oracle; sets released")


def test_step_kernel_names_name_the_launched_kernels(hip):
    # Profiles name kernels by these; bench.py reports them per config.
    cases = [
        (fx.config2_module(64, 4096, tier=1), ["softmaxWaveRowPair<16, true>"]),
        (fx.config2_module(64, 1001, tier=1), ["softmaxWaveRowScalar<4>"]),
        (fx.config4_module(256, 256, 256, "f16", tier=1), ["gemmF16Dma8s<true>"]),
        (fx.config4_module(256, 192, 256, "f16", tier=1), ["gemmF16Dma8s<true>"]),   # K % 128 == 64
        (fx.config4_module(256, 256, 256, "f16", tier=2), ["gemmF16Dma8s<false>"]),
        (fx.config4_module(256, 128, 256, "f32", tier=1), ["gemmF32Dma<true>"]),
        (fx.config4_module(70, 33, 65, "f64", tier=1), ["gemmGeneral<double>"]),
        (fx.score_softmax_module(1, 256, 128), ["scoreStatsQ+scoreStoreQ"]),
    ]
    for km, want in cases:
        art = hip.build(km)
        got = [art.step_kernel_name(i) for i in range(art.num_steps())]
        say(f"{art.class_name}: {got}")
        assert got == want, (art.class_name, got)
    art = hip.build(fx.config4_module(256, 256, 256, "f16", tier=1))
    art.set_step_variant(0, 7)
    assert art.step_kernel_name(0) == "gemmF16Dma<true>"
    # Shapes the MFMA forms do not tile run on zero-padded copies (named by
    # the MFMA form); thin ones, padded more than 8 times their work, stay
    # on the general kernel.
    assert hip.build(fx.config4_module(1000, 600, 1000, "f16", tier=2)).step_kernel_name(0) == "gemmF16Dma8s<false>"
    assert hip.build(fx.config4_module(700, 1000, 900, "f32", tier=1)).step_kernel_name(0) == "gemmF32Dma<true>"
    assert hip.build(fx.config4_module(300, 50, 70, "f16", tier=2)).step_kernel_name(0) == "gemmF16Dma8s<false>"
    assert hip.build(fx.config4_module(100, 100, 100, "f32", tier=2)).step_kernel_name(0) == "gemmF32Dma<false>"
    assert hip.build(fx.config4_module(8, 512, 512, "f16", tier=2)).step_kernel_name(0) == "gemmGeneral<float>"
    art = hip.build(fx.config1_module(n=4096))
    assert art.step_kernel_name(0).startswith("mlk_elementwise_")


@pytest.mark.parametrize("dt_in,dt_out,n", [("f32", "f32", (1 << 24) + 3),    # 64 MiB + 12 B on the device
                                            ("f16", "f32", (1 << 25) + 5),    # f16 input: 64 MiB + 10 B
                                            ("f64", "f64", (1 << 23) + 7)])   # f64 both ways, 64 MiB + 56 B
def test_host_abi_stages_large_buffers_in_chunks(hip, dt_in, dt_out, n):
    # The host-buffer ABI (mlk_kernel's f64 arrays) converts and copies each
    # buffer through at most 64 MiB of page-locked staging, chunk by chunk;
    # these buffers need a second, short chunk both ways. y = x + 0 returns
    # x rounded once to the input dtype, widened exactly: a misplaced or
    # stale chunk shows as a mismatch.
    from mlk2_amd.kernel_ir import KernelExpr, const, elem_a
    say(f"host abi chunks {dt_in}->{dt_out} n={n}")
    km = fx.lower_elementwise([("x", [n], dt_in)], [KernelExpr("add", elem_a(), const(0.0))], [n], dt_out)
    art = hip.build(km)
    x = inputs.normal(77, n, 0.0, 3.0, "f64")
    got = art.run({0: x})[km.output_ids()[0]]
    want = {"f32": x.astype(np.float32), "f16": x.astype(np.float16), "f64": x}[dt_in].astype(np.float64)
    assert np.array_equal(got, want)
    say(f"host abi chunks {dt_in}->{dt_out}: every element exact")


def test_host_abi_calls_from_two_threads(hip):
    # Two host threads call the host-buffer ABI of one artifact at once (ctypes
    # releases the GIL during the call); the calls share the artifact's
    # page-locked staging one at a time, so each gets its own result.
    import threading
    from mlk2_amd.kernel_ir import KernelExpr, const, elem_a
    n = (1 << 22) + 9
    km = fx.lower_elementwise([("x", [n], "f32")], [KernelExpr("mul", elem_a(), const(2.0))], [n], "f32")
    art = hip.build(km)
    out_id = km.output_ids()[0]
    xs = [inputs.normal(80 + t, n, 0.0, 1.0, "f64") for t in range(2)]
    got = [None, None]

    def work(t):
        for _ in range(3):
            got[t] = art.run({0: xs[t]})[out_id]

    threads = [threading.Thread(target=work, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    for t in range(2):
        assert np.array_equal(got[t], xs[t].astype(np.float32).astype(np.float64) * 2.0)
    say("host abi from two threads: both results exact")


def test_1d_roots_resolve_buffers_by_position(hip):
    # The 1-D executor path indexes its bindings (the inputs, then the
    # outputs) by buffer id (kernel_buffers.cpp resolveInput/resolveOutput).
    # With a temp between the input and the output, a store to the temp (not
    # an output) and a store to y (output 1 of 1) both resolve to no binding,
    # so neither root runs and y stays as given. With the output right after
    # the input, x -> y and y -> y run, and a root reading the temp after
    # them (output 1 of 1 again) is skipped.
    from mlk2_amd.kernel_ir import KernelModule, KernelBuffer, KernelNode, KernelExpr, const, elem_a

    def module(order, roots):
        km = KernelModule()
        ids = {}
        for name in order:
            kind = {"x": dict(is_input=True), "t": dict(is_temp=True), "y": dict(is_output=True)}[name]
            ids[name] = km.add_buffer(KernelBuffer(name=name, dtype="f32", elements=4096, dims=[4096], **kind))
        for src, dst, op, c in roots:
            cid = km.add_node(KernelNode(op="compute", math=op, exprs=[KernelExpr(op, elem_a(), const(c))],
                                         a=ids[src], b=0xFFFFFFFF))
            sid = km.add_node(KernelNode(op="store", out=ids[dst]))
            km.add_node(KernelNode(op="loop", var="i", begin=0, end=4096, children=[cid, sid]))
        return km, ids

    x = inputs.uniform(6, 4096, -4.0, 4.0)
    y0 = inputs.uniform(7, 4096, -1.0, 1.0)
    cases = [(("x", "t", "y"), (("x", "t", "mul", 2.0), ("t", "y", "add", 1.0)), False),
             (("x", "y", "t"), (("x", "y", "mul", 2.0), ("y", "y", "add", 1.0), ("t", "y", "mul", 5.0)), True)]
    for order, roots, runs in cases:
        km, ids = module(order, roots)
        got = hip.build(km).run({ids["x"]: x, ids["y"]: y0})[ids["y"]].astype(np.float32)
        ref = oracle.run(km, {ids["x"]: x}, init={ids["y"]: y0})[ids["y"]].astype(np.float32)
        assert np.array_equal(got, ref), order
        want = (x.astype(np.float32).astype(np.float64) * 2.0 + 1.0).astype(np.float32) if runs else \
            y0.astype(np.float32)
        assert np.array_equal(got, want), order
        say(f"1-D position resolution {order}: same as the executor")


@pytest.mark.parametrize("m,k,n,dt,tier", [(1000, 600, 1000, "f16", 2), (1000, 600, 1000, "f16", 1),
                                           (700, 1000, 900, "f32", 2), (700, 1000, 900, "f32", 1),
                                           (4000, 4000, 4000, "f16", 2)])
def test_ragged_gemm_runs_padded(hip, m, k, n, dt, tier):
    # M, N or K off the MFMA tiles: A, B (and C for the Call form) are copied
    # into zero-padded blocks, the MFMA form runs there, and C is copied
    # back. The extra products are 0 * 0, so each output is the product's.
    # The Call form accumulates into a non-zero C.
    rng = np.random.default_rng(21)
    A = rng.uniform(-1, 1, (m, k))
    B = rng.uniform(-1, 1, (k, n))
    np_dt = {"f32": np.float32, "f16": np.float16}[dt]
    A = A.astype(np_dt).astype(np.float64)
    B = B.astype(np_dt).astype(np.float64)
    km = fx.config4_module(m, k, n, dt, tier)
    art = hip.build(km)
    name = art.step_kernel_name(0)
    assert name.startswith("gemmF16Dma8s" if dt == "f16" else "gemmF32Dma"), name
    rows = slice(0, m) if m <= 1000 else slice(0, m, 97)       # the oracle on sampled rows at 4000^3
    C0 = rng.uniform(-1, 1, m * n) if tier == 1 else np.zeros(m * n)
    got = (art.run({0: A, 1: B, 2: C0}) if tier == 1 else art.run({0: A, 1: B}))[2].reshape(m, n)
    Ar = np.ascontiguousarray(A[rows])
    ref = oracle.run(fx.matmul_call_module(Ar.shape[0], k, n, "f64", "f64"), {0: Ar.reshape(-1), 1: B.reshape(-1)},
                     init={2: np.ascontiguousarray(C0.reshape(m, n)[rows]).reshape(-1)},
                     hw_threads=8)[2].reshape(-1, n)
    tol = 1e-2 if dt == "f16" else 1e-5 * math.sqrt(k)
    e = max_rel(got[rows], ref)
    say(f"ragged gemm {dt} {m}x{k}x{n} tier {tier} on {name}: max_rel {e:.3e}")
    assert e <= tol
