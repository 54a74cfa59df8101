"""Parity of the HIP backend against the CPU oracle, through the C ABI.

Tolerances of the path: poly7 sin chain <= 4 f32 ULP; softmax <= 1e-6
relative; f32 GEMM <= 1e-5*sqrt(K) relative; f16 GEMM <= 1e-2 relative;
score+softmax <= 1e-2 relative; "relative" is |got-ref|/max(|ref|,1)
(bench/math/math_bench.cpp:172-181). Chains of IEEE add/sub/mul/div over
f64 buffers are bit-exact. The general kernels are held tighter on f64
buffers (1e-12), and f16 outputs of f64 arithmetic must equal the oracle's
value rounded once.
"""
import math
import sys

import numpy as np
import pytest

import oracle
from mlk2_amd import backend as be
from mlk2_amd import fixtures as fx
from mlk2_amd import inputs
from mlk2_amd.backend import DeviceBuffer, MlkHipError
from mlk2_amd.kernel_ir import (KernelBuffer, KernelExpr, KernelModule, KernelNode, elem_a, elem_b,
                                 scalar, temp)
from mlk2_amd.parity import max_rel, ulp_distance_f32

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


# ------------------------------------------------------------------ C1 ----
@pytest.mark.parametrize("n", [1, 1000, 1 << 20, 1 << 24])
def test_c1_sin_chain_ulp(hip, n):
    say(f"c1 sin(x^2+3x) poly7 n={n}")
    km = fx.config1_module(n=n)
    x = inputs.config_inputs("c1", {"n": n})["x"]
    art = hip.build(km)
    assert art.class_name == "elementwise-1d"
    got = art.run({0: x})[1].astype(np.float32)
    ref = oracle.run(km, {0: x}, hw_threads=4)[1]
    d = ulp_distance_f32(got, ref)
    say(f"c1 n={n} max_ulp={d.max()} mean_ulp={d.mean():.3f}")
    assert d.max() <= 4.0


def test_c1_quadrant_edges_and_specials(hip):
    say("c1 quadrant edges / specials")
    xs = []
    for q in range(-6, 7):
        # x with x^2+3x near (2q+1)*pi/4: solve, then take f32 neighbours.
        t = (2 * q + 1) * math.pi / 4
        disc = 9 + 4 * t
        if disc < 0:
            continue
        r = (-3 + math.sqrt(disc)) / 2
        f = np.float32(r)
        xs += [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    xs += [0.0, -0.0, -3.0, 2.0, 4.0, -4.0, np.inf, -np.inf, np.nan]
    x = np.array(xs, dtype=np.float32)
    km = fx.config1_module(n=x.size)
    got = hip.build(km).run({0: x})[1].astype(np.float32)
    ref = oracle.run(km, {0: x})[1]
    assert ulp_distance_f32(got, ref).max() <= 4.0


def test_c1_f64_buffers_bit_exact(hip):
    # Every op of the chain (mul, add, the poly7 reduction and polynomial) is
    # an IEEE f64 operation evaluated in the reference's order.
    say("c1 f64 bit-exact")
    n = 100000
    x = inputs.uniform(inputs.SEEDS["c1_x"], n, -40.0, 40.0, "f64")
    km = fx.config1_module(n=n, dtype="f64")
    art = hip.build(km)
    assert art.policy == "bitexact-rne-gfx950-v1"
    got = art.run({0: x})[1]
    ref = oracle.run(km, {0: x})[1]
    assert np.array_equal(got.view(np.int64), ref.view(np.int64))


@pytest.mark.parametrize("n", [1000, 1 << 20])
def test_c1_f16_buffers_bit_exact(hip, n):
    # An f16 output keeps the exact f64 chain, so its one rounding gives the
    # reference's value rounded to f16, bit for bit. The split-precision sine
    # would move about one value in a thousand to the neighbouring f16.
    say(f"c1 f16 bit-exact n={n}")
    x = inputs.uniform(inputs.SEEDS["c1_x"], n, -40.0, 40.0, "f64").astype(np.float16).astype(np.float64)
    km = fx.config1_module(n=n, dtype="f16")
    art = hip.build(km)
    assert art.policy == "bitexact-rne-gfx950-v1"
    got = art.run({0: x})[1]
    want = oracle.run(fx.config1_module(n=n, dtype="f64"), {0: x})[1].astype(np.float16).astype(np.float64)
    assert np.array_equal(got, want), int((got != want).sum())


def test_c1_dynamic_bound_legacy_form(hip):
    # loop end = kKernelLoopDynamicBound: the extent comes from io.elements
    # (kernel_buffers.cpp:966-969), through the legacy 1-D ABI.
    say("c1 dynamic bound, legacy ABI")
    km = fx.config1_module(n=1)
    km.nodes[2].end = -1
    km.buffers[0].elements = -1
    km.buffers[0].dims = []
    km.buffers[1].elements = -1
    km.buffers[1].dims = []
    n = 3001
    x = inputs.uniform(5, n, -4.0, 4.0)
    art = hip.build(km)
    got = art.run({0: x}, elements=n, legacy=True)[1].astype(np.float32)
    ref = oracle.run(km, {0: x}, elements=n)[1]
    assert ulp_distance_f32(got, ref).max() <= 4.0


def test_scalar_param_and_two_inputs_1d(hip):
    # y = (x * s0 - y) / s1 with ScalarParams (lower.to_kernel_ir.cpp:295-307)
    say("1-D chain with scalar params, f64 bit-exact")
    n = 5000
    chain = [KernelExpr("mul", elem_a(), scalar(0)), KernelExpr("sub", temp(0), elem_b()),
             KernelExpr("div", temp(1), scalar(1))]
    km = fx.lower_elementwise([("x", [n], "f64"), ("z", [n], "f64")], chain, [n], "f64")
    a = inputs.uniform(1, n, -3, 3, "f64")
    b = inputs.uniform(2, n, -3, 3, "f64")
    art = hip.build(km)
    for sc in ([1.5, 0.25], [2.0, 0.0], [-1.0]):
        got = art.run({0: a, 1: b}, scalars=sc)[2]
        ref = oracle.run(km, {0: a, 1: b}, scalars=sc)[2]
        assert np.array_equal(got.view(np.int64), ref.view(np.int64)), sc


# ------------------------------------------------------------------ C2 ----
@pytest.mark.parametrize("shape,tier", [((8192, 4096), 1), ((512, 4096), 2), ((33, 100), 1),
                                        ((7, 9000), 1), ((64, 256), 2),
                                        # odd row counts on the guard-free pair kernel
                                        # (the last row pairs with itself)
                                        ((3, 4096), 1), ((1, 256), 1), ((4097, 1024), 2),
                                        # more rows than the capped grid has waves (each
                                        # wave walks several pairs); a row length that is
                                        # not a multiple of 4 (block-per-row kernel)
                                        ((70001, 8), 1), ((33, 101), 2),
                                        # the wave path's longest rows (32 float4 a lane)
                                        ((5, 8192), 1), ((2, 8192), 2)])
def test_c2_softmax(hip, shape, tier):
    m, k = shape
    say(f"c2 softmax {m}x{k} tier{tier}")
    x = inputs.normal(inputs.SEEDS["c2_x"], m * k, 0.0, 2.0).reshape(m, k)
    km = fx.config2_module(m, k, tier)
    art = hip.build(km)
    got = art.run({0: x})[1]
    ref = oracle.run(fx.config2_module(m, k, 1), {0: x})[1]
    e = max_rel(got, ref)
    say(f"c2 {m}x{k} max_rel={e:.3e}")
    assert e <= 1e-6
    rows = got.reshape(m, k).sum(axis=1)
    assert np.abs(rows - 1.0).max() < 1e-5


def test_softmax_adversarial_rows(hip):
    # unit_poly.cpp:3820-3835: NaN row, +/-0 rows, K=1.
    say("softmax adversarial rows")
    M, K = 24, 16
    x = np.array([((i * 13) % 19) * 0.25 - 2.0 for i in range(M * K)])
    x[9 * K + 2] = np.nan
    x[10 * K:11 * K] = [(-0.0 if k % 2 == 0 else 0.0) for k in range(K)]
    x[11 * K:11 * K + 4] = [-1.0, -0.0, 0.0, -2.0]
    for tier in (1, 2):
        km = fx.config2_module(M, K, tier)
        got = hip.build(km).run({0: x})[1]
        ref = oracle.run(fx.config2_module(M, K, 1), {0: x})[1]
        assert np.array_equal(np.isnan(got), np.isnan(ref))
        assert max_rel(got[~np.isnan(ref)], ref[~np.isnan(ref)]) <= 1e-6
    km = fx.softmax_call_module(5, 1)
    got = hip.build(km).run({0: np.array([-3.0, 0.0, 7.5, 1e30, -1e30])})[1]
    assert np.array_equal(got, np.ones(5))


@pytest.mark.parametrize("K", [256, 4096, 1000])
def test_softmax_infinite_and_nan_rows(hip, K):
    # Rows whose max is +inf, rows of -inf, all-NaN rows, and a lone finite
    # element among -inf: the reference yields NaN rows for the first three
    # (inf - inf, NaN) and a one-hot row for the last. Whole rows of
    # 256 * CH columns take the guard-free kernels, K = 1000 the guarded ones.
    say(f"softmax inf/nan rows K={K}")
    rows = []
    base = np.array([((i * 7) % 23) * 0.5 - 5.0 for i in range(K)])
    r = base.copy(); r[K // 3] = np.inf; rows.append(r)
    r = base.copy(); r[1] = np.inf; r[K - 1] = np.inf; rows.append(r)
    rows.append(np.full(K, -np.inf))
    rows.append(np.full(K, np.nan))
    r = np.full(K, -np.inf); r[K // 2] = 3.0; rows.append(r)
    r = base.copy(); r[5] = -np.inf; rows.append(r)
    rows.append(base.copy())
    x = np.concatenate(rows)
    M = len(rows)
    ref = oracle.run(fx.config2_module(M, K, 1), {0: x})[1]
    art = hip.build(fx.config2_module(M, K, 1))
    for v in art.step_variants(0):
        art.set_step_variant(0, v)
        got = art.run({0: x})[1]
        assert np.array_equal(np.isnan(got), np.isnan(ref)), v
        ok = ~np.isnan(ref)
        assert max_rel(got[ok], ref[ok]) <= 1e-6, v
    assert np.isnan(ref.reshape(M, K)[:4]).all() and ref.reshape(M, K)[4, K // 2] == 1.0


# ------------------------------------------------------------------ C3 ----
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (37, 100), (3, 5)])
def test_c3_broadcast_chain(hip, rows, cols):
    say(f"c3 exp(a*x+b)*x {rows}x{cols}")
    d = inputs.config_inputs("c3", {"rows": rows, "cols": cols})
    km = fx.config3_module(rows, cols, tier=2)
    art = hip.build(km)
    assert art.class_name == "elementwise-nd"
    got = art.run({0: d["x"], 1: d["b"]})[2]
    ref = oracle.run(km, {0: d["x"], 1: d["b"]}, hw_threads=4)[2]
    e = max_rel(got, ref)
    u = ulp_distance_f32(got.astype(np.float32), ref)
    say(f"c3 max_rel={e:.3e} max_ulp={u.max()}")
    assert e <= 1e-6


def test_elementwise_nd_f16_buffers(hip):
    # The n-D template on f16 buffers: the poly7 chain lifted to a nest and
    # the C3 broadcast chain. Each keeps its f64 chain and rounds once to
    # f16, so the outputs equal the oracle's f64 values rounded to f16 (the
    # exp chain within one f64 ULP before that rounding, which moves no f16
    # value at these sizes).
    say("elementwise n-D f16 buffers")
    n = 1 << 16
    x = inputs.uniform(inputs.SEEDS["c1_x"], n, -40.0, 40.0, "f64").astype(np.float16).astype(np.float64)
    km = fx.lift_1d(fx.config1_module(n=n, dtype="f16"))
    art = hip.build(km)
    assert art.class_name == "elementwise-nd" and art.policy == "bitexact-rne-gfx950-v1"
    want = oracle.run(fx.config1_module(n=n, dtype="f64"), {0: x})[1].astype(np.float16).astype(np.float64)
    got = art.run({0: x})[1]
    assert np.array_equal(got, want), int((got != want).sum())
    rows, cols = 300, 1000
    d = inputs.config_inputs("c3", {"rows": rows, "cols": cols})
    xs = d["x"].astype(np.float16).astype(np.float64)
    bs = d["b"].astype(np.float16).astype(np.float64)
    km = fx.synth_elementwise(fx.config3_tier1_module(rows, cols, "f16"))
    art = hip.build(km)
    assert art.class_name == "elementwise-nd"
    got = art.run({0: xs, 1: bs})[2]
    want = oracle.run(fx.synth_elementwise(fx.config3_tier1_module(rows, cols, "f64")), {0: xs, 1: bs},
                      hw_threads=4)[2].astype(np.float16).astype(np.float64)
    assert np.array_equal(got, want), int((got != want).sum())


def test_c3_tier1_form_refused(hip):
    # The Tier-1 1-D path reads b[i] (kernel_buffers.cpp:110-113): with
    # b[4096] under a 4096^2 loop that is out of bounds; the backend refuses.
    km = fx.config3_module(64, 128, tier=1)
    with pytest.raises(MlkHipError) as ei:
        hip.build(km)
    assert ei.value.code == 7


def test_c3_scalar_param_a(hip):
    say("c3 with a as ScalarParam")
    rows, cols = 64, 256
    d = inputs.config_inputs("c3", {"rows": rows, "cols": cols})
    km = fx.config3_module(rows, cols, tier=2, a_operand=scalar(0))
    art = hip.build(km)
    for a in (0.5, -1.25):
        got = art.run({0: d["x"], 1: d["b"]}, scalars=[a])[2]
        ref = oracle.run(km, {0: d["x"], 1: d["b"]}, scalars=[a])[2]
        assert max_rel(got, ref) <= 1e-6


# ------------------------------------------------------------------ C4 ----
def _gemm_ref(A, B):
    m, k = A.shape
    n = B.shape[1]
    call = fx.matmul_call_module(m, k, n, "f64", "f64")
    return oracle.run(call, {0: A, 1: B}, hw_threads=8)[2].reshape(m, n)


@pytest.mark.parametrize("m,k,n,tier", [(1024, 1024, 1024, 2), (1024, 1024, 1024, 1),
                                        (64, 64, 64, 2),      # f32 form 0: one K step
                                        (192, 128, 320, 2),   # form 0: two steps, 3 x 5 tiles
                                        (128, 96, 64, 2),     # K % 64 != 0: form 1
                                        (64, 32, 64, 2), (100, 70, 33, 2)])
def test_c4a_gemm_f32(hip, m, k, n, tier):
    say(f"c4a gemm f32 {m}x{k}x{n} tier{tier}")
    d = inputs.config_inputs("c4a", {"m": m, "k": k, "n": n})
    km = fx.config4_module(m, k, n, "f32", tier)
    art = hip.build(km)
    got = art.run({0: d["A"], 1: d["B"]})[2].reshape(m, n)
    ref = _gemm_ref(d["A"].astype(np.float64), d["B"].astype(np.float64))
    e = max_rel(got, ref)
    say(f"c4a max_rel={e:.3e} (tol {1e-5 * math.sqrt(k):.3e})")
    assert e <= 1e-5 * math.sqrt(k)


@pytest.mark.parametrize("m,k,n", [(512, 4096, 512), (256, 64, 256), (300, 50, 70),
                                   (768, 128, 1280),   # 3 x 5 tiles: the row-major tile map
                                   (256, 4160, 512)])  # 130 K steps of 32
def test_c4b_gemm_f16(hip, m, k, n):
    say(f"c4b gemm f16 {m}x{k}x{n}")
    d = inputs.config_inputs("c4b", {"m": m, "k": k, "n": n})
    km = fx.config4_module(m, k, n, "f16", 2)
    art = hip.build(km)
    got = art.run({0: d["A"], 1: d["B"]})[2].reshape(m, n)
    ref = _gemm_ref(d["A"].astype(np.float64), d["B"].astype(np.float64))
    e = max_rel(got, ref)
    say(f"c4b max_rel={e:.3e}")
    assert e <= 1e-2


@pytest.mark.parametrize("m,k,n,tier", [(512, 4096, 256, 2), (256, 192, 512, 2), (512, 640, 256, 1),
                                        (256, 320, 256, 1)])
def test_c4b_form8_kernels_match_form7_bitwise(hip, m, k, n, tier):
    # Form 8 runs gemmF16Dma8s (its loop unrolled over the 4 ring slots, with
    # a two-step tail when K % 128 == 64); it takes every output's products
    # in form 7's k order, so the two agree bit for bit, for the nest
    # (C = A*B) and for the Call form (C += A*B over a nonzero C).
    say(f"c4b form 8 vs form 7 bitwise {m}x{k}x{n} tier {tier}")
    d = inputs.config_inputs("c4b", {"m": m, "k": k, "n": n})
    km = fx.config4_module(m, k, n, "f16", tier)
    art = hip.build(km)
    c0 = inputs.uniform(13, m * n, -1, 1).astype(np.float32)
    outs = {}
    for form in (8, 7):
        art.set_step_variant(0, form)
        arrays = {0: d["A"], 1: d["B"]}
        if tier == 1:
            arrays[2] = c0
        outs[form] = art.run(arrays)[2]
    art.set_step_variant(0, -1)
    assert art.step_kernel_name(0).startswith("gemmF16Dma8s")
    bits = {f: o.astype(np.float32).view(np.uint32) for f, o in outs.items()}   # f32 results, carried in f64
    assert np.array_equal(bits[8], bits[7])
    ref = _gemm_ref(d["A"].astype(np.float64), d["B"].astype(np.float64)).reshape(-1)
    if tier == 1:
        ref = ref + c0.astype(np.float64)
    e = max_rel(outs[8], ref)
    say(f"c4b form 8 == form 7 bitwise, max_rel={e:.3e}")
    assert e <= 1e-2


@pytest.mark.parametrize("m,k,n", [(100, 70, 33), (128, 256, 64)])
def test_gemm_f64_buffers(hip, m, k, n):
    # f64 operands and output take the general tiled kernel in f64, k
    # ascending per output element: 1e-12 relative, where an f32 accumulator
    # anywhere would show near 1e-6. Both the Call and the poly.synth nest.
    say(f"gemm f64 {m}x{k}x{n}")
    A = inputs.normal(11, m * k).reshape(m, k)
    B = inputs.normal(12, k * n).reshape(k, n)
    ref = _gemm_ref(A, B)
    call = fx.matmul_call_module(m, k, n, "f64", "f64")
    for km in (call, fx.synth_gemm(call)):
        got = hip.build(km).run({0: A, 1: B})[2].reshape(m, n)
        e = max_rel(got, ref)
        say(f"gemm f64 {m}x{k}x{n} max_rel={e:.3e}")
        assert e <= 1e-12


def test_c4b_full_size_sampled_rows(hip):
    # 4096^3 on the device; 32 sampled rows recomputed by the oracle's GEMM.
    m = k = n = 4096
    say("c4b gemm f16 4096^3, sampled rows")
    d = inputs.config_inputs("c4b", {"m": m, "k": k, "n": n})
    km = fx.config4_module(m, k, n, "f16", 2)
    art = hip.build(km)
    bufs = {0: DeviceBuffer.from_array(d["A"], "f16"), 1: DeviceBuffer.from_array(d["B"], "f16"),
            2: DeviceBuffer(m * n, "f32")}
    art.run_device(bufs)
    got = bufs[2].to_numpy().reshape(m, n)
    rows = np.random.default_rng(4).choice(m, 32, replace=False)
    ref = _gemm_ref(d["A"][rows].astype(np.float64), d["B"].astype(np.float64))
    e = max_rel(got[rows], ref)
    say(f"c4b full max_rel(sampled)={e:.3e}")
    assert e <= 1e-2


def test_c4b_blocked_tile_map_non_square(hip):
    # 8 x 32 tiles of 256 x 256: a multiple of 256 tiles, so each XCD takes
    # 4 x 8 blocks of tiles, here over a grid four blocks wide; sampled rows
    # from every block row against the oracle's GEMM.
    m, k, n = 2048, 256, 8192
    say(f"c4b gemm f16 {m}x{k}x{n}, blocked tile map, sampled rows")
    d = inputs.config_inputs("c4b", {"m": m, "k": k, "n": n})
    km = fx.config4_module(m, k, n, "f16", 2)
    art = hip.build(km)
    bufs = {0: DeviceBuffer.from_array(d["A"], "f16"), 1: DeviceBuffer.from_array(d["B"], "f16"),
            2: DeviceBuffer(m * n, "f32")}
    art.run_device(bufs)
    got = bufs[2].to_numpy().reshape(m, n)
    rows = np.concatenate([np.arange(b * 1024, b * 1024 + 1024, 97) for b in range(2)])
    ref = _gemm_ref(d["A"][rows].astype(np.float64), d["B"].astype(np.float64))
    e = max_rel(got[rows], ref)
    say(f"c4b blocked map max_rel(sampled)={e:.3e}")
    assert e <= 1e-2
    for bb in bufs.values():
        bb.free()


def test_matmul_call_accumulates_into_c(hip):
    # Call(MatMul) adds into C (kernel_buffers.cpp:406-432); the nest form
    # initializes it (poly.synth.cpp:75-95).
    say("matmul call accumulates")
    m, k, n = 256, 64, 256
    d = inputs.config_inputs("c4a", {"m": m, "k": k, "n": n})
    c0 = inputs.uniform(9, m * n, -1, 1)
    call = fx.config4_module(m, k, n, "f32", 1)
    got = hip.build(call).run({0: d["A"], 1: d["B"], 2: c0})[2]
    ref = oracle.run(call, {0: d["A"], 1: d["B"]}, init={2: c0})[2]
    assert max_rel(got, ref) <= 1e-5 * math.sqrt(k)


@pytest.mark.parametrize("m,n", [(64, 1001), (33, 4095), (8, 8191), (5, 1), (7, 3), (16, 257), (2, 4097)])
def test_c2_ragged_rows(hip, m, n):
    # Row lengths off the float4 path (n % 4 != 0) take one wave per row
    # with 4-byte loads (softmaxWaveRowScalar) up to 8192 columns, with the
    # float4 path's arithmetic and the class bound of 1e-6; longer rows take
    # the workgroup-per-row kernel. Rows of -inf, a NaN and +inf give the
    # reference's NaN rows.
    say(f"c2 ragged rows {m}x{n}")
    km = fx.config2_module(m, n, tier=1)
    x = inputs.config_inputs("c2", {"m": m, "k": n})["x"].astype(np.float64).reshape(m, n)
    if m >= 8:
        x[1, :] = -np.inf
        x[2, n // 2] = np.nan
        x[3, n - 1] = np.inf
    art = hip.build(km)
    assert art.step_kernel_name(0) == ("softmaxBlockRow" if n > 8192 else
                                       "softmaxWaveRowScalar<%d>" % max(1, 1 << max(0, (n - 1).bit_length() - 8)))
    got = art.run({0: x.reshape(-1)})[1].reshape(m, n)
    ref = oracle.run(km, {0: x.reshape(-1)}, hw_threads=8)[1].reshape(m, n)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = np.isfinite(ref)
    e = max_rel(got[fin], ref[fin])
    say(f"c2 ragged {m}x{n} max_rel={e:.3e}")
    assert e <= 1e-6


# ------------------------------------------------------------------ C5 ----
@pytest.mark.parametrize("b,s,dm", [(2, 128, 128), (1, 24, 8)])
def test_c5_score_softmax(hip, b, s, dm):
    say(f"c5 score softmax b={b} s={s} d={dm}")
    d = inputs.config_inputs("c5", {"batch": b, "seq": s, "dim": dm})
    km = fx.score_softmax_module(b, s, dm)
    art = hip.build(km)
    assert art.class_name == "score-softmax"
    got = art.run({0: d["Q"], 1: d["K"], 2: d["bias"]})[3]
    ref = oracle.run(km, {0: d["Q"], 1: d["K"], 2: d["bias"]}, hw_threads=8)[3]
    e = max_rel(got, ref)
    say(f"c5 max_rel={e:.3e}")
    assert e <= 1e-2


@pytest.mark.parametrize("b,s,dm", [(2, 128, 128), (1, 24, 8), (1, 300, 20)])
def test_c5_score_softmax_f64_operands(hip, b, s, dm):
    # Q and K held as f64 take the general score kernel (f64 dot products,
    # one thread per score) and then the row softmax in place over S. S is
    # an f32 buffer, so each score (|score| < 6 here) is rounded to f32
    # before its exponential, about 1e-7 in the outputs. Held to 1e-5, where
    # operands rounded to f16 would be off by about 1e-4.
    say(f"c5 score softmax f64 operands b={b} s={s} d={dm}")
    km = fx.score_softmax_module(b, s, dm, "f64")
    Q = inputs.normal(21, b * s * dm)
    K = inputs.normal(22, b * s * dm)
    bias = inputs.uniform(23, s, -1, 1)
    art = hip.build(km)
    assert art.class_name == "score-softmax"
    got = art.run({0: Q, 1: K, 2: bias})[3]
    ref = oracle.run(km, {0: Q, 1: K, 2: bias.astype(np.float32).astype(np.float64)}, hw_threads=8)[3]
    e = max_rel(got, ref)
    say(f"c5 f64 operands max_rel={e:.3e}")
    assert e <= 1e-5


@pytest.mark.parametrize("dtype_in", ["f16", "f64"])
def test_c5_score_softmax_f16_output(hip, dtype_in):
    # S held as f16 takes the general score kernel, which stores each score
    # to S with one rounding, then the row softmax in place over S (f64
    # arithmetic, one rounding per output). Rounding the scores to f16
    # first moves the outputs by about 2^-11 of a score times the output;
    # the score+softmax bound of 1e-2 holds.
    b, s, dm = 2, 96, 32
    say(f"c5 score softmax f16 S, {dtype_in} operands")
    km = fx.score_softmax_module(b, s, dm, dtype_in, dtype_out="f16")
    Q = inputs.normal(31, b * s * dm)
    K = inputs.normal(32, b * s * dm)
    if dtype_in == "f16":
        Q = Q.astype(np.float16).astype(np.float64)
        K = K.astype(np.float16).astype(np.float64)
    bias = inputs.uniform(33, s, -1, 1).astype(np.float32).astype(np.float64)
    art = hip.build(km)
    assert art.class_name == "score-softmax"
    got = art.run({0: Q, 1: K, 2: bias})[3]
    ref = oracle.run(km, {0: Q, 1: K, 2: bias}, hw_threads=8)[3]
    e = max_rel(got, ref)
    say(f"c5 f16 S max_rel={e:.3e}")
    assert e <= 1e-2
    assert np.abs(got.reshape(b * s, s).sum(axis=1) - 1.0).max() < 0.05


def _score_ref(Q, K, bias, rows=None):
    """Config-5 reference composed from oracle pieces: k-ascending f64 GEMM
    Q_b K_b^T (Call(MatMul) with K^T materialized, as Transpose is rank-2),
    then Div by the f64 constant sqrt(dim) and Add bias[j] (IEEE f64, the
    walker's operations), then Call(Softmax)."""
    B, S, D = Q.shape
    out = []
    for b in range(B):
        q = Q[b].astype(np.float64) if rows is None else Q[b][rows].astype(np.float64)
        sc = _gemm_ref(q, np.ascontiguousarray(K[b].astype(np.float64).T))
        sc = sc / math.sqrt(D) + bias.astype(np.float64)
        m = sc.shape[0]
        km = fx.softmax_call_module(m, S, "f64")
        out.append(oracle.run(km, {0: sc})[1].reshape(m, S))
    return np.concatenate(out)


@pytest.mark.parametrize("b,s,dm", [(1, 2048, 128), (2, 512, 64), (1, 384, 16), (2, 512, 128), (3, 256, 128)])
def test_c5_fused_shapes(hip, b, s, dm):
    say(f"c5 fused b={b} s={s} d={dm}")
    d = inputs.config_inputs("c5", {"batch": b, "seq": s, "dim": dm})
    km = fx.score_softmax_module(b, s, dm)
    art = hip.build(km)
    got = art.run({0: d["Q"], 1: d["K"], 2: d["bias"]})[3].reshape(b * s, s)
    ref = _score_ref(d["Q"], d["K"], d["bias"])
    e = max_rel(got, ref)
    say(f"c5 fused max_rel={e:.3e}")
    assert e <= 1e-2


def test_c5_full_size_sampled_rows(hip):
    b, s, dm = 16, 2048, 128
    say("c5 full size 16x2048x2048, sampled rows")
    d = inputs.config_inputs("c5")
    km = fx.score_softmax_module(b, s, dm)
    art = hip.build(km)
    bufs = {0: DeviceBuffer.from_array(d["Q"], "f16"), 1: DeviceBuffer.from_array(d["K"], "f16"),
            2: DeviceBuffer.from_array(d["bias"], "f32"), 3: DeviceBuffer(b * s * s, "f32")}
    art.run_device(bufs)
    got = bufs[3].to_numpy().reshape(b, s, s)
    rows = np.random.default_rng(5).choice(s, 24, replace=False)
    for bb in (0, 15):
        ref = _score_ref(d["Q"][bb:bb + 1], d["K"][bb:bb + 1], d["bias"], rows=rows)
        e = max_rel(got[bb][rows], ref)
        say(f"c5 full batch {bb} max_rel={e:.3e}")
        assert e <= 1e-2
    sums = got.reshape(b * s, s)[::97].astype(np.float64).sum(axis=1)
    assert np.abs(sums - 1.0).max() < 1e-3


@pytest.mark.parametrize("s,two_pass", [(4096, True), (8192, True), (8448, False)])
def test_c5_long_rows_sampled(hip, s, two_pass):
    # The two-pass form up to its largest row (seq <= 8192: pass 1 keeps a
    # key half's bias in LDS), and one row length past it, which takes the
    # scores-then-softmax form with the workgroup-per-row softmax (rows
    # longer than the wave path's 8192).
    b, dm = 1, 128
    say(f"c5 long rows b={b} s={s}, sampled rows")
    d = inputs.config_inputs("c5", {"batch": b, "seq": s, "dim": dm})
    km = fx.score_softmax_module(b, s, dm)
    assert be.plan_variants(km, 0) == ([0, 1] if two_pass else [])
    art = hip.build(km)
    bufs = {0: DeviceBuffer.from_array(d["Q"], "f16"), 1: DeviceBuffer.from_array(d["K"], "f16"),
            2: DeviceBuffer.from_array(d["bias"], "f32"), 3: DeviceBuffer(b * s * s, "f32")}
    art.run_device(bufs)
    got = bufs[3].to_numpy().reshape(s, s)
    rows = np.random.default_rng(6).choice(s, 12, replace=False)
    rows[0], rows[1] = 0, s - 1
    ref = _score_ref(d["Q"], d["K"], d["bias"], rows=rows)
    e = max_rel(got[rows], ref)
    say(f"c5 long rows s={s} max_rel={e:.3e}")
    assert e <= 1e-2
    sums = got[::131].astype(np.float64).sum(axis=1)
    assert np.abs(sums - 1.0).max() < 1e-3
    for bb in bufs.values():
        bb.free()


@pytest.mark.parametrize("b,s", [(1, 2000), (4, 1000), (16, 300), (64, 128), (1, 8000), (2, 1500), (8, 700),
                                 (32, 257), (1, 100), (3, 129)])
def test_c5_ragged_seq_runs_padded(hip, b, s):
    # A sequence length off the two-pass form's 256-row blocks runs on
    # zero-padded copies of Q and K (padded keys take a -inf bias, so they
    # add exp(-inf) = 0 to each row's sum; padded query rows are dropped).
    # At 64x128 the padded length is 256 and pass 1's second key half is
    # all padding; 1x8000 pads to the longest two-pass row (8192); 32x257
    # pads 257 rows to 512, the most padding per row. Sampled rows of the first and last batch are held to the
    # composed oracle reference; a fully masked bias gives NaN rows, as the
    # reference does.
    dm = 128
    say(f"c5 ragged seq b={b} s={s}")
    d = inputs.config_inputs("c5", {"batch": b, "seq": s, "dim": dm})
    km = fx.score_softmax_module(b, s, dm)
    art = hip.build(km)
    assert art.step_kernel_name(0) == "scoreStatsQ+scoreStoreQ"
    got = art.run({0: d["Q"], 1: d["K"], 2: d["bias"]})[3].reshape(b, s, s)
    rows = np.random.default_rng(7).choice(s, min(s, 16), replace=False)
    rows[0], rows[1] = 0, s - 1
    for bb in sorted({0, b - 1}):
        ref = _score_ref(d["Q"][bb:bb + 1], d["K"][bb:bb + 1], d["bias"], rows=rows)
        e = max_rel(got[bb][rows], ref)
        say(f"c5 ragged b={b} s={s} batch {bb} max_rel={e:.3e}")
        assert e <= 1e-2
    sums = got.reshape(b * s, s)[::37].astype(np.float64).sum(axis=1)
    assert np.abs(sums - 1.0).max() < 1e-3
    masked = art.run({0: d["Q"], 1: d["K"], 2: np.full(s, -np.inf)})[3]
    assert np.isnan(masked).all()


def test_c5_ragged_seq_forms(hip):
    # Padded at any size with dim 128 up to the longest two-pass row; other
    # head dims and longer rows take the general kernels.
    assert hip.build(fx.score_softmax_module(1, 100, 128)).step_kernel_name(0) == "scoreStatsQ+scoreStoreQ"
    assert hip.build(fx.score_softmax_module(1, 300, 64)).step_kernel_name(0).startswith("scoresGeneral+")
    assert hip.build(fx.score_softmax_module(1, 8200, 128)).step_kernel_name(0).startswith("scoresGeneral+")


# ------------------------------------------------------------- entries ----
def test_device_entry_matches_host_entry(hip):
    say("device entry vs host entry")
    n = 1 << 18
    x = inputs.config_inputs("c1", {"n": n})["x"]
    km = fx.config1_module(n=n)
    art = hip.build(km)
    host = art.run({0: x})[1].astype(np.float32)
    bufs = {0: DeviceBuffer.from_array(x, "f32"), 1: DeviceBuffer(n, "f32")}
    art.run_device(bufs)
    dev = bufs[1].to_numpy()
    assert np.array_equal(host.view(np.int32), dev.view(np.int32))


def test_bad_binding_rejected(hip):
    km = fx.config1_module(n=1024)
    art = hip.build(km)
    bufs = {0: DeviceBuffer(100, "f32"), 1: DeviceBuffer(1024, "f32")}
    with pytest.raises(MlkHipError) as ei:
        art.run_device(bufs)
    assert ei.value.code == 6
    bufs = {0: DeviceBuffer(1024, "f16"), 1: DeviceBuffer(1024, "f32")}
    with pytest.raises(MlkHipError) as ei:
        art.run_device(bufs)
    assert ei.value.code == 6


def test_reducesum_call_and_nest(hip):
    say("reducesum")
    M, K = 300, 1000
    x = inputs.normal(3, M * K)
    for km in (fx.reducesum_call_module(M, K), fx.synth_reducesum(fx.reducesum_call_module(M, K))):
        got = hip.build(km).run({0: x})[1]
        ref = oracle.run(fx.reducesum_call_module(M, K), {0: x})[1]
        assert max_rel(got, ref) <= 1e-6


@pytest.mark.parametrize("dtype", ["f64", "f16"])
@pytest.mark.parametrize("m,k", [(37, 300), (5, 9001), (16, 4096)])
def test_softmax_and_rowsum_on_f64_and_f16_buffers(hip, dtype, m, k):
    # Buffers other than f32 take the general block-per-row softmax and the
    # wave row sum, both in f64 like the reference (kernel_buffers.cpp:237-340).
    # The device rounds inputs to the buffer dtype on upload and outputs once
    # on store, so the oracle sees the rounded inputs and its outputs are
    # rounded the same way. f64 buffers are held to 1e-12 (an f32 intermediate
    # anywhere would show at 1e-7). f16 outputs must equal the oracle's f64
    # result rounded once: an f64 -> f32 -> f16 store misrounds about one
    # value in 8192, which these shapes hit.
    say(f"softmax/rowsum {dtype} {m}x{k}")
    x = inputs.normal(inputs.SEEDS["c2_x"], m * k, 0.0, 2.0)
    if dtype == "f16":
        x = x.astype(np.float16).astype(np.float64)
    tol = 1e-12 if dtype == "f64" else 0.0

    def rounded(v):
        return v.astype(np.float16).astype(np.float64) if dtype == "f16" else v

    call = fx.softmax_call_module(m, k, dtype)
    ref = rounded(oracle.run(fx.softmax_call_module(m, k, "f64"), {0: x})[1])
    for km in (call, fx.synth_softmax(call)):
        got = hip.build(km).run({0: x})[1]
        e = max_rel(got, ref)
        say(f"softmax {dtype} {m}x{k} max_rel={e:.3e}")
        assert e <= tol
    rs = fx.reducesum_call_module(m, k, dtype)
    ref = rounded(oracle.run(fx.reducesum_call_module(m, k, "f64"), {0: x})[1])
    for km in (rs, fx.synth_reducesum(rs)):
        got = hip.build(km).run({0: x})[1]
        e = max_rel(got, ref)
        say(f"rowsum {dtype} {m}x{k} max_rel={e:.3e}")
        assert e <= tol


def _tie_neighbours():
    # Values just above, just below and exactly on the midpoint between f16
    # neighbours (normal, smallest-normal and subnormal). Rounding f64 -> f32
    # -> f16 lands 11 of them on the tie and then rounds to even, the wrong way.
    h = np.array([1.0, 1.0009765625, 3.140625, 1000.0, 6.103515625e-05, 1.7881393432617188e-07,
                  0.25 + 2.0 ** -12], dtype=np.float16)
    lo = h.astype(np.float64)
    hi = np.nextafter(h, np.float16(np.inf)).astype(np.float64)
    t = (lo + hi) / 2
    v = np.concatenate([t * (1 + 2.0 ** -40), t * (1 - 2.0 ** -40), t, -t * (1 + 2.0 ** -40)])
    assert (v.astype(np.float16) != v.astype(np.float32).astype(np.float16)).sum() == 11
    return v


def test_f64_results_stored_to_f16_round_once(hip):
    # The artifact ABI's f64 -> f16 store is one round-to-nearest-even of the
    # f64 value (numpy's astype(float16) is that rounding). A k = 1 GEMM
    # (C = A * 1) and a one-column row sum hand each value to the store as is.
    say("f16 stores round once")
    v = _tie_neighbours()
    m = len(v)
    want = v.astype(np.float16).astype(np.float64)
    km = fx.matmul_call_module(m, 1, 1, "f64", "f16")
    got = hip.build(km).run({0: v, 1: np.ones(1)})[2]
    assert np.array_equal(got, want), np.c_[v, got, want][got != want]
    km = KernelModule()
    x = km.add_buffer(KernelBuffer("X", "f64", True, False, False, m, [m, 1]))
    y = km.add_buffer(KernelBuffer("Y", "f16", False, True, False, m, [m]))
    km.add_node(KernelNode(op="call", math="reduce_sum", a=x, out=y))
    got = hip.build(km).run({0: v})[1]
    assert np.array_equal(got, want), np.c_[v, got, want][got != want]


@pytest.mark.parametrize("s", [512, 384])
def test_c5_masked_keys_every_form(hip, s):
    # An attention-style mask: bias = -inf over whole key ranges (a full
    # 64/128-key panel and a ragged span). Those scores contribute exp(-inf)
    # = 0 and the other keys' softmax is unchanged; with every key masked
    # each row is NaN, as the reference's exp(-inf - -inf) makes it. Every
    # declared launch form is held to the oracle, NaN positions included.
    b, dm = 2, 128
    d = inputs.config_inputs("c5", {"batch": b, "seq": s, "dim": dm})
    km = fx.score_softmax_module(b, s, dm)
    art = hip.build(km)
    forms = art.step_variants(0) or [-1]
    for label, bias in (("masked spans", d["bias"].astype(np.float32).copy()), ("all masked", None)):
        if bias is None:
            bias = np.full(s, -np.inf, dtype=np.float32)
        else:
            bias[0:128] = -np.inf
            bias[200:230] = -np.inf
        arrays = {0: d["Q"], 1: d["K"], 2: bias}
        ref = oracle.run(km, arrays, hw_threads=8)[3]
        for form in forms:
            art.set_step_variant(0, form)
            got = art.run(arrays)[3]
            assert np.array_equal(np.isnan(got), np.isnan(ref)), (s, label, form)
            fin = np.isfinite(ref)
            e = max_rel(got[fin], ref[fin]) if fin.any() else 0.0
            say(f"c5 {label} seq={s} form {form}: NaN positions match, max_rel={e:.3e}")
            assert e <= 1e-2, (s, label, form, e)
    art.set_step_variant(0, -1)
