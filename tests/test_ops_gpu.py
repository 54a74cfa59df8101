"""Device parity of every operation the chain code generator emits.

The reference evaluator's op table (runtime/src/execution/kernel_buffers.cpp:
130-160) is what a chain computes, in f64, whatever the buffer dtype: Add,
Sub, Mul, Div with its b != 0 guard, Neg, Pow with the (2, 2) -> a*a form,
Exp, Log with its a > 0 guard, Sin (poly7 or libm family), Cos, Tan, Tanh,
Sqrt with its a >= 0 guard, Rsqrt with its a > 0 guard, Erf and the tanh form
of Gelu. Each op runs here as a one-op chain over inputs that reach every arm
(zeros of both signs, negatives, infinities, NaN, tiny and huge values), on
f64 and on f32 buffers, through the elementwise template (Tier-1 module) and
through the generic loop-nest kernel (the same chain lifted to a multi-dim
nest), against the oracle.

Bars, per op:
* IEEE ops and the guards (add, sub, mul, div, neg, sqrt, rsqrt, poly7 sin,
  pow at (2, 2)): bit-exact on f64 buffers, and so on f32 buffers too (the f64
  result is the same, and rounds to f32 the same way). The poly7 sine on an
  f32 output is the split-precision form, held to its 4-ULP policy.
* Device libm against the host glibc (the oracle's exp/log/sin/cos/tan/
  tanh/erf/pow; their bits are pinned by no reference fixture): f64 buffers
  within 4 f64 ULP, f32 buffers within 1 f32 ULP (the two f64 values round to
  the same or an adjacent f32). Non-finite results must match in class.
  exp into an f32 buffer through the template takes the f32-accurate form
  (hardware exp2 on the reduced fraction, about 1.4e-7 relative): within 2
  f32 ULP.
* Gelu: 0.5 a (1 + tanh(u)) cancels for a below about -3, where an f64 ULP of
  tanh is many ULP of the result, so it is held to the reference's relative
  measure |got - ref| / max(|ref|, 1) <= 1e-14 on f64 buffers and 1e-7 on f32.
"""
import sys

import numpy as np
import pytest

import oracle
from mlk2_amd import fixtures as fx
from mlk2_amd.kernel_ir import KernelExpr, const, elem_a, elem_b
from mlk2_amd.parity import max_rel, ulp_distance_f32, ulp_distance_f64

N = 4096

EXACT = {"add", "sub", "mul", "div", "neg", "sqrt", "rsqrt"}
LIBM = {"exp", "log", "sin", "cos", "tan", "tanh", "erf", "pow"}
UNARY = {"neg", "exp", "log", "sin", "cos", "tan", "tanh", "sqrt", "rsqrt", "erf", "gelu"}


def say(msg):
    print(f"[ops] {msg}", flush=True)
    sys.stdout.flush()


def _specials():
    return np.array([0.0, -0.0, 1.0, -1.0, 2.0, -2.0, 0.5, -0.5, np.inf, -np.inf, np.nan,
                     1e-30, -1e-30, 1e30, -1e30, 3.0, 0.25, 1.5707963267948966, 3.141592653589793])


def op_inputs(op: str, dtype: str, seed: int = 0):
    """x (and y for binary ops): the specials, then values drawn over the
    op's interesting domain, rounded to the buffer dtype."""
    rng = np.random.default_rng(seed + sum(map(ord, op)))
    sp = _specials()
    m = N - sp.size
    if op == "exp":
        body = rng.uniform(-745.0, 710.0, m) if dtype == "f64" else rng.uniform(-104.0, 89.0, m)
    elif op in ("log", "sqrt", "rsqrt"):
        mag = 10.0 ** rng.uniform(-300, 300, m) if dtype == "f64" else 10.0 ** rng.uniform(-37, 38, m)
        body = mag * np.where(rng.random(m) < 0.15, -1.0, 1.0)
        body[:16] = 0.0
    elif op in ("sin", "cos", "tan"):
        body = np.concatenate([rng.uniform(-10.0, 10.0, m // 2), rng.uniform(-1e5, 1e5, m - m // 2)])
    elif op == "tanh":
        body = rng.uniform(-25.0, 25.0, m)
    elif op == "erf":
        body = rng.uniform(-7.0, 7.0, m)
    elif op == "gelu":
        body = rng.uniform(-12.0, 12.0, m)
    else:
        body = rng.uniform(-8.0, 8.0, m) * 10.0 ** rng.integers(-3, 4, m)
    x = np.concatenate([sp, body])
    y = rng.uniform(-8.0, 8.0, N) * 10.0 ** rng.integers(-2, 2, N)
    if op == "div":
        y[::7] = 0.0
        y[3::7] = -0.0
    if op == "pow":
        x = np.concatenate([sp, rng.uniform(-6.0, 6.0, m)])
        y = rng.uniform(-6.0, 6.0, N)
        y[::5] = np.round(y[::5])                 # integer exponents of negative bases
        x[::11] = 2.0                             # the (2, 2) fast form
        y[::11] = 2.0
        y[1::13] = 0.5
        y[:sp.size] = np.resize([2.0, -1.0, 0.5, 3.0, 0.0, -0.5], sp.size)
    if dtype == "f32":
        with np.errstate(over="ignore"):
            x = x.astype(np.float32).astype(np.float64)
            y = y.astype(np.float32).astype(np.float64)
    return x, y


def op_module(op: str, dtype: str, family=None):
    if op in UNARY:
        chain = [KernelExpr(op, elem_a(), const(0.0))]
        ins = [("x", [N], dtype)]
    else:
        chain = [KernelExpr(op, elem_a(), elem_b())]
        ins = [("x", [N], dtype), ("y", [N], dtype)]
    return fx.lower_elementwise(ins, chain, [N], dtype, family=family)


def generic(km):
    g = fx.lift_1d(km)
    g.schedule["hip_generic"] = 1
    return g


def check(op, dtype, family, got, ref, f32_ulps=1.0):
    """Asserts the per-op bar; returns the measure for the log line."""
    finite_ref = np.isfinite(ref)
    # Non-finite results match in class (NaN with NaN, inf with the same inf).
    assert np.array_equal(np.isnan(got), np.isnan(ref)), (op, dtype, "NaN class")
    inf = ~finite_ref & ~np.isnan(ref)
    assert np.array_equal(got[inf], ref[inf]), (op, dtype, "infinity")
    if op in EXACT or (op == "sin" and family == "poly7" and dtype == "f64"):
        same = (got.view(np.int64) == ref.view(np.int64)) | (np.isnan(got) & np.isnan(ref))
        # +0 and -0 compare equal under the reference's own gates; bit-exact here
        # means equal bits except for NaN payloads.
        bad = np.nonzero(~same)[0]
        assert bad.size == 0, (op, dtype, int(bad[0]), got[bad[0]], ref[bad[0]])
        return "bit-exact"
    if op == "sin" and family == "poly7":
        d = float(ulp_distance_f32(got, ref).max())
        assert d <= 4.0, (op, dtype, d)
        return f"{d:g} f32 ULP (split-precision poly7, bound 4)"
    if op == "gelu":
        r = max_rel(got[finite_ref], ref[finite_ref])
        tol = 1e-14 if dtype == "f64" else 1e-7
        assert r <= tol, (op, dtype, r)
        return f"rel {r:.2e} (bound {tol:g})"
    if dtype == "f64":
        d = ulp_distance_f64(got, ref)
        worst = float(d.max())
        assert worst <= 4.0, (op, dtype, worst, int(d.argmax()))
        return f"{worst:g} f64 ULP (bound 4)"
    d = ulp_distance_f32(got.astype(np.float32), ref)
    worst = float(d.max())
    assert worst <= f32_ulps, (op, dtype, worst, int(d.argmax()))
    return f"{worst:g} f32 ULP (bound {f32_ulps:g})"


CASES = [(op, None) for op in ["add", "sub", "mul", "div", "neg", "pow", "exp", "log", "sin", "cos",
                               "tan", "tanh", "sqrt", "rsqrt", "erf", "gelu"]] + [("sin", "poly7")]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f64", "f32"])
@pytest.mark.parametrize("op,family", CASES)
def test_op_parity_gpu(hip, op, family, dtype):
    x, y = op_inputs(op, dtype)
    km = op_module(op, dtype, family)
    arrays = {0: x} if op in UNARY else {0: x, 1: y}
    out = 1 if op in UNARY else 2
    ref = oracle.run(km, arrays)[out]
    for path, mod in (("template", km), ("generic", generic(km))):
        art = hip.build(mod)
        got = art.run(arrays)[out]
        # Exact ops on f32 buffers: the f64 result rounded once to f32.
        with np.errstate(over="ignore"):
            cmp_ref = ref.astype(np.float32).astype(np.float64) if (dtype == "f32" and op in EXACT) else ref
        fast_exp = op == "exp" and dtype == "f32" and path == "template"
        note = check(op, dtype, family, got, cmp_ref, 2.0 if fast_exp else 1.0)
        say(f"{op}{'/' + family if family else ''} {dtype} {path} ({art.class_name}): {note}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f64", "f32"])
def test_guard_arms_gpu(hip, dtype):
    # Each guard's taken and untaken arm, exactly: div by +-0 -> 0, log of
    # <= 0 -> 0, sqrt of < 0 -> 0 (and sqrt(-0) = -0), rsqrt of <= 0 -> 0, and
    # pow(2, 2) -> 4 by the a * a form.
    vals = np.array([-4.0, -0.0, 0.0, 4.0, 0.25, -np.inf, np.inf, np.nan])
    for op, y, want in (
            ("div", np.array([0.0, -0.0, 0.0, 2.0, -0.0, 1.0, 0.0, 1.0]),
             [0.0, 0.0, 0.0, 2.0, 0.0, -np.inf, 0.0, np.nan]),
            ("log", None, [0.0, 0.0, 0.0, np.log(4.0), np.log(0.25), 0.0, np.inf, 0.0]),
            ("sqrt", None, [0.0, -0.0, 0.0, 2.0, 0.5, 0.0, np.inf, 0.0]),
            ("rsqrt", None, [0.0, 0.0, 0.0, 0.5, 2.0, 0.0, 0.0, 0.0])):
        km = fx.lower_elementwise([("x", [8], dtype)] + ([("y", [8], dtype)] if y is not None else []),
                                  [KernelExpr(op, elem_a(), elem_b() if y is not None else const(0.0))],
                                  [8], dtype)
        arrays = {0: vals} if y is None else {0: vals, 1: y}
        got = hip.build(km).run(arrays)[2 if y is not None else 1]
        ref = oracle.run(km, arrays)[2 if y is not None else 1]
        # The oracle states the reference's arms; NaN compared as NaN.
        assert np.array_equal(ref, np.asarray(want), equal_nan=True), (op, ref)
        if dtype == "f32":
            ref = ref.astype(np.float32).astype(np.float64)   # one rounding of the f64 value
        same = (got.view(np.int64) == ref.view(np.int64)) | (np.isnan(got) & np.isnan(ref))
        assert same.all(), (op, dtype, got, ref)
        say(f"guard {op} {dtype}: {got.tolist()}")
    km = fx.lower_elementwise([("x", [4], dtype), ("y", [4], dtype)], [KernelExpr("pow", elem_a(), elem_b())],
                              [4], dtype)
    got = hip.build(km).run({0: np.array([2.0, 2.0, -2.0, 3.0]), 1: np.array([2.0, 3.0, 2.0, 2.0])})[2]
    assert got.tolist() == [4.0, 8.0, 4.0, 9.0]
