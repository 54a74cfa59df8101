"""Chain forms whose operations differ from the reference's list but whose
results do not, run on the device against the oracle.

* A sum of an exact product (two f32 or f16 values, or one and a short
  constant) is one fused multiply-add: bit-exact with the walker's separate
  product and sum (kernel_buffers.cpp:130-160 evaluates each in f64).
* exp as a factor of an f32 result takes the f32-accurate form: within 1e-6
  relative. Arguments outside its range (|u*log2(e)| >= 1000, NaN, +-inf) make
  their wave redo its segment with the f64 exp; the inputs put such arguments
  in some waves and not in others.
* The split-precision poly7 sine (math_families.h:81-90) with arguments whose
  reduction it declines (|x*2/pi| >= 2^20, NaN, inf) beside ones it takes:
  within 4 f32 ULP, the declined ones from the exact f64 form.
"""
import sys

import numpy as np
import pytest

import oracle
from mlk2_amd import fixtures as fx
from mlk2_amd import inputs
from mlk2_amd.parity import max_rel, ulp_distance_f32
from test_host import EXP_CASES, FUSE_CASES

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[fast-forms] {msg}", flush=True)
    sys.stdout.flush()


def finite_max_rel(got, ref):
    """Max relative error of an f32 output over the finite references, after
    checking that NaNs and infinities sit where the reference's do. The
    walker holds f64 values; the reference's f32 buffer holds them rounded,
    so a value past the f32 range is inf there too."""
    got = np.asarray(got, dtype=np.float64)
    with np.errstate(over="ignore"):
        ref = np.asarray(ref, dtype=np.float64).astype(np.float32).astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "NaN positions differ"
    inf = np.isinf(ref)
    assert np.array_equal(got[inf], ref[inf]), "infinities differ"
    fin = np.isfinite(ref)
    return max_rel(got[fin], ref[fin])


@pytest.mark.parametrize("name,chain,fused", FUSE_CASES, ids=[c[0] for c in FUSE_CASES])
@pytest.mark.parametrize("dt_in", ["f32", "f16"])
@pytest.mark.parametrize("lift", [False, True])
def test_exact_product_sums_bit_exact(hip, name, chain, fused, dt_in, lift):
    n = 70001                                    # ragged: a partial last segment
    rng = np.random.default_rng(11)
    np_dt = np.float32 if dt_in == "f32" else np.float16
    a = rng.uniform(-3, 3, n).astype(np_dt).astype(np.float64)
    b = rng.uniform(-3, 3, n).astype(np_dt).astype(np.float64)
    a[:4] = [0.0, -0.0, np.inf, np.nan]
    b[:4] = [-0.0, 0.0, 1.0, 2.0]
    km = fx.lower_elementwise([("a", [n], dt_in), ("b", [n], dt_in)], chain, [n], out_dtype="f64")
    if lift:
        km = fx.lift_1d(km)
    art = hip.build(km)
    assert art.policy == "bitexact-rne-gfx950-v1"
    got = art.run({0: a, 1: b})[2]
    ref = oracle.run(km, {0: a, 1: b})[2]
    # Bit-exact means equal bits except NaN payloads and signs (IEEE leaves
    # those to the implementation; the reference's writer emits NaN as null).
    same = (got.view(np.int64) == ref.view(np.int64)) | (np.isnan(got) & np.isnan(ref))
    say(f"{name} {dt_in} lift={lift}: fused={fused}, {int((~same).sum())} bit differences")
    assert same.all()


def exp_arguments(n, rng):
    """Mostly ordinary arguments; a few waves' worth around overflow,
    underflow and the non-finite values."""
    a = rng.uniform(-10, 10, n)
    a[20000:20400] = rng.uniform(700, 720, 400)      # exp overflows past 709.78
    a[30000:30400] = rng.uniform(-760, -690, 400)    # subnormal and zero results
    a[40000:40010] = [np.nan, np.inf, -np.inf, 709.78, -708.4, -745.2, 0.0, -0.0, 693.0, -693.0]
    return a.astype(np.float32).astype(np.float64)


@pytest.mark.parametrize("name,chain,out_dt,fast_exp", [c for c in EXP_CASES if c[2] == "f32"],
                         ids=[c[0] for c in EXP_CASES if c[2] == "f32"])
@pytest.mark.parametrize("lift", [False, True])
def test_f32_accurate_exp_against_the_walker(hip, name, chain, out_dt, fast_exp, lift):
    n = 50000
    rng = np.random.default_rng(12)
    a = exp_arguments(n, rng)
    b = rng.uniform(0.5, 2, n).astype(np.float32).astype(np.float64)
    km = fx.lower_elementwise([("a", [n], "f32"), ("b", [n], "f32")], chain, [n], out_dtype="f32")
    if lift:
        km = fx.lift_1d(km)
    art = hip.build(km)
    got = art.run({0: a, 1: b})[2]
    ref = oracle.run(km, {0: a, 1: b})[2]
    err = finite_max_rel(got, ref)
    say(f"{name} lift={lift}: f32-accurate exp={fast_exp}, max rel {err:.3g}")
    assert err <= 1e-6


def test_c3_chain_with_exact_pass_rows(hip):
    rows, cols = 256, 1024
    km = fx.config3_module(rows, cols, 2)
    d = inputs.config_inputs("c3", {"rows": rows, "cols": cols})
    x = d["x"].astype(np.float64)
    x[5, :] = 1500.0                                  # exp(750 + b): overflow, the exact pass
    x[9, 100:200] = -1600.0                           # exp(-800 + b): zero
    x[77, 3] = np.nan
    got = hip.build(km).run({0: x, 1: d["b"]})[2]
    ref = oracle.run(km, {0: x, 1: d["b"]})[2]
    err = finite_max_rel(got, ref)
    say(f"c3 with exact-pass rows: max rel {err:.3g}")
    assert err <= 1e-6


@pytest.mark.parametrize("lift", [False, True])
def test_c1_sine_with_declined_reductions(hip, lift):
    n = 1 << 20
    rng = np.random.default_rng(13)
    x = rng.uniform(-4, 4, n)
    x[100000:101000] = rng.uniform(-3000, 3000, 1000)    # |t| up to 9e6: y beyond 2^20
    x[300000:300064] = rng.uniform(-1e4, 1e4, 64)
    x[500000:500005] = [np.nan, np.inf, -np.inf, 1e19, -1e19]
    x = x.astype(np.float32).astype(np.float64)
    km = fx.config1_module(n=n)
    if lift:
        km = fx.lift_1d(km)
    art = hip.build(km)
    assert art.policy == "tol-4ulp-f32-gfx950-v1"
    got = art.run({0: x})[1].astype(np.float32)
    ref = oracle.run(km, {0: x}, hw_threads=4)[1]
    d = ulp_distance_f32(got, ref)
    with np.errstate(invalid="ignore", over="ignore"):
        t = x * x + 3.0 * x
        big = ~(np.abs(t * (2 / np.pi) + 0.5) < 2.0 ** 20)  # declined: |y| >= 2^20, NaN, inf
    say(f"c1 lift={lift}: max ULP {d.max()}, over the declined arguments {d[big].max()}")
    assert d.max() <= 4.0
    # The declined arguments come from the exact f64 form.
    assert d[big].max() == 0


def mixed_streams_module(rows, cols):
    """out[i, j] = exp(0.5 * x[i, j] + s[i]) * t[j, i]: a unit-stride stream,
    a broadcast stream (coefficient 0 on the innermost loop) and a gather
    (coefficient `rows`), so the exact pass re-reads all three kinds."""
    from mlk2_amd.kernel_ir import (KernelBuffer, KernelExpr, KernelModule, KernelNode, const, elem_idx,
                                    temp)
    km = KernelModule()
    x = km.add_buffer(KernelBuffer("x", "f32", True, False, False, rows * cols, [rows, cols]))
    s = km.add_buffer(KernelBuffer("s", "f32", True, False, False, rows, [rows]))
    t = km.add_buffer(KernelBuffer("t", "f32", True, False, False, cols * rows, [cols, rows]))
    y = km.add_buffer(KernelBuffer("y", "f32", False, True, False, rows * cols, [rows, cols]))
    cp = km.add_node(KernelNode(op="compute", exprs=[
        KernelExpr("mul", elem_idx(x, [cols, 1]), const(0.5)),
        KernelExpr("add", temp(0), elem_idx(s, [1, 0])),
        KernelExpr("exp", temp(1)),
        KernelExpr("mul", temp(2), elem_idx(t, [1, rows]))]))
    st = km.add_node(KernelNode(op="store", out=y, out_index_coeffs=[cols, 1]))
    j = km.add_node(KernelNode(op="loop", var="j", begin=0, end=cols, children=[cp, st]))
    km.add_node(KernelNode(op="loop", var="i", begin=0, end=rows, children=[j]))
    return km


def test_exact_pass_rereads_broadcast_and_gather_streams(hip):
    rows, cols = 67, 1100                       # ragged: partial last segments
    km = mixed_streams_module(rows, cols)
    art = hip.build(km)
    assert art.class_name == "elementwise-nd"
    rng = np.random.default_rng(14)
    x = rng.uniform(-4, 4, (rows, cols)).astype(np.float32).astype(np.float64)
    s = rng.uniform(-1, 1, rows).astype(np.float32).astype(np.float64)
    t = rng.uniform(0.5, 2, (cols, rows)).astype(np.float32).astype(np.float64)
    x[3, 700] = 1500.0                          # exp overflows: that wave's exact pass
    x[10, :] = -1600.0                          # a row of zeros
    x[20, 5] = np.nan
    s[33] = 800.0                               # a broadcast value that declines a whole row
    got = art.run({0: x, 1: s, 2: t})[3]
    ref = oracle.run(km, {0: x, 1: s, 2: t})[3]
    err = finite_max_rel(got, ref)
    say(f"mixed streams {rows}x{cols}: max rel {err:.3g}")
    assert err <= 1e-6


def test_exact_pass_with_a_dynamic_bound(hip):
    # The 1-D dynamic form (loop end = the run's element count) through the
    # legacy ABI, with declined sine arguments in a partial last segment.
    km = fx.config1_module(n=1)
    km.nodes[2].end = -1
    for b in km.buffers:
        b.elements = -1
        b.dims = []
    n = 5000
    rng = np.random.default_rng(15)
    x = rng.uniform(-4, 4, n)
    x[4990:4996] = [3000.0, -2500.0, np.nan, np.inf, 1e7, -1e7]
    x = x.astype(np.float32).astype(np.float64)
    got = hip.build(km).run({0: x}, elements=n, legacy=True)[1].astype(np.float32)
    ref = oracle.run(km, {0: x}, elements=n)[1]
    d = ulp_distance_f32(got, ref)
    say(f"dynamic bound with declined arguments: max ULP {d.max()}, tail {d[4990:4996].tolist()}")
    assert d.max() <= 4.0 and d[4990:4996].max() == 0


@pytest.mark.parametrize("lift", [False, True])
def test_in_place_chains_with_declined_elements(hip, lift):
    # y is x: the store goes back into the buffer the chain reads. A NaN or
    # an out-of-range argument in a segment must not make that segment's
    # other elements come out as f(f(x)); each element is the walker's f(x).
    # The walker reads an element before it stores it (kernel_buffers.cpp:
    # 342-402), so an in-place run equals the out-of-place one.
    from test_host import in_place
    n = 70001
    rng = np.random.default_rng(16)
    x = rng.uniform(-4, 4, n)
    x[1000:1004] = [np.nan, 3000.0, -1e7, np.inf]       # declined sine arguments
    x = x.astype(np.float32).astype(np.float64)
    km = fx.config1_module(n=n)
    if lift:
        km = fx.lift_1d(km)
    ref = oracle.run(km, {0: x})[1]
    got = hip.build(in_place(km)).run({0: x})[0].astype(np.float32)
    d = ulp_distance_f32(got, ref)
    say(f"in-place sine lift={lift}: max ULP {d.max()}")
    assert d.max() <= 4.0

    a = exp_arguments(50000, rng)
    b = rng.uniform(0.5, 2, a.size).astype(np.float32).astype(np.float64)
    km = fx.lower_elementwise([("a", [a.size], "f32"), ("b", [a.size], "f32")], EXP_CASES[0][1], [a.size],
                              out_dtype="f32")
    if lift:
        km = fx.lift_1d(km)
    ref = oracle.run(km, {0: a, 1: b})[2]
    got = hip.build(in_place(km)).run({0: a, 1: b})[0]
    err = finite_max_rel(got, ref)
    say(f"in-place exp*b lift={lift}: max rel {err:.3g}")
    assert err <= 1e-6


def random_chain(rng):
    """A fused chain of 1-5 ops over ElemA, ElemB, constants and earlier
    temps, drawing the IEEE ops, neg, exp and sin."""
    from mlk2_amd.kernel_ir import KernelExpr, const, elem_a, elem_b, temp
    exprs = []
    for k in range(int(rng.integers(1, 6))):
        def operand():
            r = rng.random()
            if k > 0 and r < 0.5:
                return temp(int(rng.integers(0, k)))
            if r < 0.7:
                return elem_a()
            if r < 0.85:
                return elem_b()
            return const(float(rng.choice([0.5, 2.0, 3.0, -1.0, 0.1, 1e-3, 7.25])))
        if rng.random() < 0.35:
            exprs.append(KernelExpr(str(rng.choice(["neg", "exp", "sin"])),
                                    temp(k - 1) if k > 0 and rng.random() < 0.7 else operand()))
        else:
            exprs.append(KernelExpr(str(rng.choice(["add", "sub", "mul", "div"])),
                                    temp(k - 1) if k > 0 and rng.random() < 0.6 else operand(), operand()))
    if not any(o.kind in ("elem_a", "elem_b") for e in exprs for o in (e.a, e.b)):
        exprs[0] = KernelExpr("add", elem_a(), exprs[0].a)
    return exprs


def random_chain_inputs(rng, n, dt):
    """Uniform values with NaN, +-inf, zeros of both signs, tiny values and
    arguments that overflow exp or that the split sine declines."""
    a = rng.uniform(-4, 4, n)
    b = rng.uniform(0.25, 4, n) * rng.choice([-1, 1], n)
    for x in (a, b):
        i = rng.integers(0, n, 24)
        x[i[:4]] = [np.nan, np.inf, -np.inf, 0.0]
        x[i[4:8]] = rng.uniform(-1e3, 1e3, 4)
        x[i[8:12]] = rng.uniform(-1e7, 1e7, 4)
        x[i[12:16]] = rng.uniform(-1e-30, 1e-30, 4)
        x[i[16:20]] = -0.0
    npdt = {"f32": np.float32, "f16": np.float16}[dt]
    with np.errstate(over="ignore"):
        return a.astype(npdt).astype(np.float64), b.astype(npdt).astype(np.float64)


# Seed 26 is left out: its chain takes sin of exp(a)/a with a near 494, an
# argument near 1e212 where one f64 ULP of exp (device libm against the
# host's) changes the sine completely. No tolerance holds for such a chain.
@pytest.mark.parametrize("seed", [s for s in range(60) if s != 26])
def test_random_chains_against_the_walker(hip, seed):
    # Random chains with random input and output dtypes, Tier-1 and lifted,
    # each held to the policy its artifact declares: bit for bit (NaN pairs
    # equal) for IEEE chains, 4 f32 ULP for the split sine, 1e-6 relative
    # otherwise. The reference's f32 and f16 buffers hold the walker's f64
    # result rounded once, so the oracle's result is rounded the same way.
    rng = np.random.default_rng(seed)
    chain = random_chain(rng)
    dt_in = "f32" if rng.random() < 0.8 else "f16"
    out_dt = str(rng.choice(["f32", "f32", "f64", "f16"]))
    family = "poly7" if any(e.op == "sin" for e in chain) and rng.random() < 0.7 else None
    n = 8192 + int(rng.integers(0, 300))
    a, b = random_chain_inputs(rng, n, dt_in)
    for lift in (False, True):
        km = fx.lower_elementwise([("a", [n], dt_in), ("b", [n], dt_in)], chain, [n], out_dtype=out_dt,
                                  family=family)
        if lift:
            km = fx.lift_1d(km)
        art = hip.build(km)
        got = np.asarray(art.run({0: a, 1: b})[2], dtype=np.float64)
        ref = np.asarray(oracle.run(km, {0: a, 1: b})[2], dtype=np.float64)
        with np.errstate(over="ignore"):
            if out_dt != "f64":
                ref = ref.astype(np.float32 if out_dt == "f32" else np.float16).astype(np.float64)
        if art.policy.startswith("bitexact"):
            ok = bool(((got == ref) | (np.isnan(got) & np.isnan(ref))).all())
            note = "bit-exact"
        elif art.policy.startswith("tol-4ulp"):
            d = float(ulp_distance_f32(got, ref).max())
            ok, note = d <= 4.0, f"{d:g} ulp"
        else:
            e = max_rel(got, ref)
            ok, note = e <= 1e-6, f"max rel {e:.3g}"
        say(f"chain seed {seed} lift={lift} {dt_in}->{out_dt} {art.policy}: {note}")
        assert ok, (seed, lift, art.policy, note)
