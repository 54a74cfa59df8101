"""Pins the CPU oracle (oracle/oracle.cpp) before anything is compared to it.

Every check below can fail for a plausible mistake in the restatement: the
poly7 polynomial is compared bit-for-bit with the reference's own header, the
GEMM / ReduceSum results with exact rational sums, softmax with a hand-computed
stable form and the reference's adversarial rows, the walker with the Call
path and brute-force enumeration.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle
from mlk2_amd import fixtures as fx
from mlk2_amd.kernel_ir import (KernelBuffer, KernelExpr, KernelModule, KernelNode,
                                const, elem_idx)
from mlk2_amd.parity import ulp_distance_f64


def test_poly7_bit_exact_vs_reference_header():
    ref = oracle.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference tree absent on this host)")
    rng = np.random.default_rng(7)
    xs = np.concatenate([rng.uniform(-40, 40, 20000), np.linspace(-30, 30, 4001),
                         np.array([0.0, -0.0, math.pi / 4, -math.pi / 4, math.pi / 2,
                                   math.pi, 3 * math.pi / 2, 28.0, -2.25, 1e-300])])
    got = oracle.poly_sin(xs)
    want = np.array([ref.ref_poly_sin(float(x)) for x in xs])
    assert np.array_equal(got.view(np.int64), want.view(np.int64))


def test_poly7_known_answer_sin_graph_at_2():
    # examples/scalar/README.md:9 and tests/differential/differential_test.cpp:44-48.
    km = fx.config1_module(n=1, dtype="f64")
    out = oracle.run(km, {0: np.array([2.0])})
    assert abs(out[1][0] - (-0.5440211108893698)) <= 1e-13


def test_poly7_certificate_vs_libm():
    # README.md:34: <= 2 ULP vs libm on [-pi, pi] incl. quadrant edges
    # (sample set of math_families.h:113-137, constants.h kUlpVerify*).
    n = 512
    xs = [-math.pi + 2.0 * math.pi * i / n for i in range(n)]
    edges = [-math.pi, -math.pi / 2, -math.pi / 4, 0.0, math.pi / 4, math.pi / 2, math.pi]
    xs += [edges[i % 7] for i in range(64)]
    xs = np.array(xs)
    d = ulp_distance_f64(oracle.poly_sin(xs), np.array([math.sin(x) for x in xs]))
    assert d.max() <= 2.0
    ref = oracle.ref_lib()
    if ref is not None:
        assert ref.ref_measured_poly_sin_max_ulps() == d.max()


def test_poly7_quadrant_edges():
    # unit_poly.cpp:3331-3346 uses quadrant boundaries; the polynomial must
    # stay continuous across every boundary x = (2q+1) pi/4.
    for q in range(-8, 9):
        b = (2 * q + 1) * math.pi / 4
        lo, hi = np.nextafter(b, -np.inf), np.nextafter(b, np.inf)
        y = oracle.poly_sin(np.array([lo, b, hi]))
        assert abs(y[0] - math.sin(lo)) < 4e-16 and abs(y[2] - math.sin(hi)) < 4e-16


def _gemm_fixture(M, K, N):
    A = np.array([((i * 7) % 13) * 0.25 for i in range(M * K)])
    B = np.array([((i * 5) % 11) * 0.5 for i in range(K * N)])
    exact = np.zeros(M * N)
    for i in range(M):
        for j in range(N):
            s = Fraction(0)
            for k in range(K):
                s += Fraction(A[i * K + k]) * Fraction(B[k * N + j])
            exact[i * N + j] = float(s)
    return A, B, exact


@pytest.mark.parametrize("shape", [(8, 6, 7), (4, 3, 5), (70, 33, 65)])
def test_gemm_call_and_nest_exact(shape):
    # unit_poly.cpp:2024-2056 (8x6x7) and :680-682 (4x3x5): dyadic entries,
    # every partial sum exact in f64, so k-ascending must equal the exact sum.
    M, K, N = shape
    A, B, exact = _gemm_fixture(M, K, N)
    call = fx.matmul_call_module(M, K, N, "f64", "f64")
    got_call = oracle.run(call, {0: A, 1: B})[2]
    got_nest = oracle.run(fx.synth_gemm(call), {0: A, 1: B})[2]
    assert np.array_equal(got_call, exact)
    assert np.array_equal(got_nest, exact)


def test_gemm_call_accumulates_into_c_and_skips_zero_a():
    # kernel_buffers.cpp:406-432: C += A*B and A[i,p]==0 skips the product
    # (so 0*inf never reaches C); the synthesized nest initializes C.
    A = np.array([0.0, 1.0, 2.0, 3.0])          # 2x2
    B = np.array([np.inf, 1.0, 1.0, 1.0])       # 2x2
    C0 = np.array([10.0, 20.0, 30.0, 40.0])
    call = fx.matmul_call_module(2, 2, 2, "f64", "f64")
    out = oracle.run(call, {0: A, 1: B}, init={2: C0})[2]
    assert out[0] == 10.0 + 1.0 and out[1] == 20.0 + 1.0
    assert math.isinf(out[2]) and out[3] == 40.0 + 2.0 + 3.0
    nest = oracle.run(fx.synth_gemm(call), {0: A, 1: B}, init={2: C0})[2]
    assert math.isnan(nest[0]) and nest[1] == 1.0


def test_gemm_threads_bit_identical():
    M, K, N = 80, 50, 70
    rng = np.random.default_rng(3)
    A, B = rng.standard_normal(M * K), rng.standard_normal(K * N)
    call = fx.matmul_call_module(M, K, N, "f64", "f64")
    one = oracle.run(call, {0: A, 1: B}, hw_threads=1)[2]
    four = oracle.run(call, {0: A, 1: B}, hw_threads=4)[2]
    assert np.array_equal(one, four)
    # k-ascending per cell (independent of tiles): numpy float64 dot in the
    # same order.
    ref = np.zeros(M * N)
    for k in range(K):
        ref += np.repeat(A.reshape(M, K)[:, k], N) * np.tile(B.reshape(K, N)[k], M)
    assert np.array_equal(one, ref)


def _softmax_rows(x, M, K):
    x = x.reshape(M, K)
    out = np.empty_like(x)
    for i in range(M):
        r = -math.inf
        for v in x[i]:
            r = v if v > r else r
        e = [math.exp(v - r) for v in x[i]]
        s = 0.0
        for v in e:
            s += v
        out[i] = [v / s if s != 0.0 else 0.0 for v in e]
    return out.reshape(-1)


def test_softmax_hand_computed_and_synth_bit_exact():
    # unit_poly.cpp:3521-3525 input, 24x16, plus the adversarial rows of
    # :3820-3835 (NaN row, +/-0 rows).
    M, K = 24, 16
    x = np.array([((i * 13) % 19) * 0.25 - 2.0 for i in range(M * K)])
    x[9 * K + 2] = np.nan
    x[10 * K:11 * K] = [(-0.0 if k % 2 == 0 else 0.0) for k in range(K)]
    x[11 * K:11 * K + 4] = [-1.0, -0.0, 0.0, -2.0]
    call = fx.softmax_call_module(M, K, "f64")
    got = oracle.run(call, {0: x})[1]
    want = _softmax_rows(x, M, K)
    assert np.isnan(got[9 * K:10 * K]).all()
    mask = ~np.isnan(want)
    assert np.array_equal(got[mask], want[mask])
    synth = oracle.run(fx.synth_softmax(call), {0: x})[1]
    assert np.array_equal(np.isnan(synth), np.isnan(got))
    assert np.array_equal(synth[mask].view(np.int64), got[mask].view(np.int64))


def test_softmax_k1_is_exactly_one():
    # unit_poly.cpp:3612-3615.
    call = fx.softmax_call_module(5, 1, "f64")
    got = oracle.run(call, {0: np.array([-3.0, 0.0, 7.5, 1e300, -1e300])})[1]
    assert np.array_equal(got, np.ones(5))
    assert np.array_equal(oracle.run(fx.synth_softmax(call), {0: np.array([-3.0, 0.0, 7.5, 1e300, -1e300])})[1], np.ones(5))


def test_max_accumulate_store_semantics():
    # unit_poly.cpp:3685-3776: NaN never replaces, -0.0 replaces -inf.
    km = KernelModule()
    a = km.add_buffer(KernelBuffer("A", "f64", True, dims=[3, 1], elements=3))
    o = km.add_buffer(KernelBuffer("O", "f64", False, True, dims=[3, 1], elements=3))
    km.nodes = [
        KernelNode(op="compute", exprs=[KernelExpr("add", const(-math.inf), const(0.0))]),
        KernelNode(op="store", out=o, out_index_coeffs=[1]),
        KernelNode(op="compute", exprs=[KernelExpr("sub", elem_idx(a, [1, 0]), const(0.0))]),
        KernelNode(op="store", out=o, out_index_coeffs=[1, 0], accum="max"),
        KernelNode(op="loop", var="k", begin=0, end=1, children=[2, 3]),
        KernelNode(op="loop", var="m", begin=0, end=3, children=[0, 1, 4]),
    ]
    out = oracle.run(km, {0: np.array([np.nan, -0.0, 2.5])}, elements=3)[1]
    assert out[0] == -math.inf
    assert out[1] == 0.0 and math.copysign(1.0, out[1]) < 0
    assert out[2] == 2.5


def test_reducesum_call_and_nest_exact():
    M, K = 9, 37
    x = np.array([((i * 13) % 19) * 0.25 - 2.0 for i in range(M * K)])
    call = fx.reducesum_call_module(M, K, "f64")
    exact = np.array([float(sum(Fraction(v) for v in x[i * K:(i + 1) * K])) for i in range(M)])
    assert np.array_equal(oracle.run(call, {0: x})[1], exact)
    assert np.array_equal(oracle.run(fx.synth_reducesum(call), {0: x})[1], exact)


def test_broadcast_index_identity():
    # poly.synth.cpp:258-291: y[i,j] uses b[j] (coefficients {0,1}).
    R, C = 7, 12
    x = np.linspace(-2, 2, R * C)
    b = np.linspace(-1, 1, C)
    km = fx.config3_module(R, C, tier=2)
    y = oracle.run(km, {0: x, 1: b})[2].reshape(R, C)
    for i in range(R):
        for j in range(C):
            want = math.exp(0.5 * x[i * C + j] + b[j]) * x[i * C + j]
            assert y[i, j] == want


def test_elementwise_1d_threads_bit_identical_and_threshold():
    n = 40000   # above kParallelChunkElements (16384) -> threaded chunks
    x = np.linspace(-4, 4, n)
    km = fx.config1_module(n=n, dtype="f64")
    one = oracle.run(km, {0: x}, hw_threads=1)[1]
    four = oracle.run(km, {0: x}, hw_threads=4)[1]
    assert np.array_equal(one, four)
    assert np.array_equal(one, oracle.poly_sin(x * x + 3.0 * x))


def test_temp_limit_rejects_oversized_synth_softmax():
    # kernel_buffers.cpp:852-878 with kKernelTempElementsLimit = 2^24: the
    # synthesized softmax at 8192x4096 needs a 2^25-element exp temp.
    km = fx.config2_module(8192, 4096, tier=2)
    with pytest.raises(oracle.OracleError) as ei:
        oracle.execute(km.to_json(), [np.zeros(1)], [np.zeros(1)])
    assert ei.value.code == 2


def test_negative_store_flat_is_invalid_graph():
    km = KernelModule()
    o = km.add_buffer(KernelBuffer("O", "f64", False, True, dims=[4], elements=4))
    km.nodes = [KernelNode(op="compute", exprs=[KernelExpr("add", const(1.0), const(0.0))]),
                KernelNode(op="store", out=o, out_index_coeffs=[1], out_index_offset=-2),
                KernelNode(op="loop", var="i", begin=0, end=4, children=[0, 1])]
    with pytest.raises(oracle.OracleError) as ei:
        oracle.run(km, {}, elements=4)
    assert ei.value.code == 2


def test_affine_bounds_and_guard_vs_brute_force():
    # Triangular nest i{ j in [0, i] } plus a guard (j - 3 == 0): the walker's
    # inclusive affine bounds (kernel_buffers.cpp:579-601) and guard
    # predicate (:670-700) against direct enumeration.
    N = 6
    km = KernelModule()
    o = km.add_buffer(KernelBuffer("O", "f64", False, True, dims=[N, N], elements=N * N))
    g = km.add_buffer(KernelBuffer("G", "f64", False, True, dims=[N], elements=N))
    km.nodes = [
        KernelNode(op="compute", exprs=[KernelExpr("add", const(1.0), const(0.0))]),          # 0
        KernelNode(op="store", out=o, out_index_coeffs=[N, 1], accum="add"),                  # 1
        KernelNode(op="compute", exprs=[KernelExpr("add", const(5.0), const(0.0))]),          # 2
        KernelNode(op="store", out=g, out_index_coeffs=[1, 0], accum="add"),                  # 3
        KernelNode(op="guard", guard_coeffs=[0, 1], guard_offset=-3, children=[2, 3]),        # 4
        KernelNode(op="loop", var="j", begin_coeffs=[0], begin_offset=0, end_coeffs=[1],
                   end_offset=0, children=[0, 1, 4]),                                         # 5
        KernelNode(op="loop", var="i", begin=0, end=N, children=[5]),                        # 6
    ]
    out = oracle.run(km, {}, elements=N * N)
    want = np.zeros((N, N))
    wg = np.zeros(N)
    for i in range(N):
        for j in range(0, i + 1):
            want[i, j] += 1.0
            if j == 3:
                wg[i] += 5.0
    assert np.array_equal(out[0].reshape(N, N), want)
    assert np.array_equal(out[1], wg)


def test_div_log_sqrt_rsqrt_guards():
    # kernel_buffers.cpp:135-153 special cases.
    ops = [("div", 1.0, 0.0, 0.0), ("log", -1.0, 0.0, 0.0), ("sqrt", -4.0, 0.0, 0.0),
           ("rsqrt", 0.0, 0.0, 0.0), ("pow", 2.0, 2.0, 4.0), ("rsqrt", 4.0, 0.0, 0.5)]
    for op, a, b, want in ops:
        km = fx.lower_elementwise([], [KernelExpr(op, const(a), const(b))], [1], "f64")
        assert oracle.run(km, {})[0][0] == want, op


def test_score_softmax_composition_matches_numpy():
    B, S, D = 2, 8, 4
    rng = np.random.default_rng(11)
    Q = rng.standard_normal((B, S, D))
    K = rng.standard_normal((B, S, D))
    bias = rng.standard_normal(S) * 0.1
    km = fx.score_softmax_module(B, S, D, "f64")
    out = oracle.run(km, {0: Q, 1: K, 2: bias})[3].reshape(B * S, S)
    sc = np.einsum("bid,bjd->bij", Q, K).reshape(B * S, S) / math.sqrt(D) + bias
    sc = sc - sc.max(axis=1, keepdims=True)
    e = np.exp(sc)
    want = e / e.sum(axis=1, keepdims=True)
    assert np.abs(out - want).max() < 1e-14


# Op table of the evaluator (kernel_buffers.cpp:130-160): each op name maps to
# the host libm function of that name, which Python's math module calls too,
# so the oracle must agree with it bit for bit (a swapped or mis-dispatched
# op fails). Guard arms are covered above and below.
_LIBM = {"exp": math.exp, "cos": math.cos, "tan": math.tan, "tanh": math.tanh, "erf": math.erf}


def _oracle_unary(op, xs, family=None):
    km = fx.lower_elementwise([("x", [len(xs)], "f64")], [KernelExpr(op, fx.elem_a(), const(0.0))],
                              [len(xs)], "f64", family=family)
    return oracle.run(km, {0: np.asarray(xs, dtype=np.float64)})[1]


@pytest.mark.parametrize("op", sorted(_LIBM))
def test_transcendental_ops_dispatch_to_libm(op):
    xs = np.linspace(-3.0, 3.0, 97)
    got = _oracle_unary(op, xs)
    want = np.array([_LIBM[op](x) for x in xs])
    assert np.array_equal(got.view(np.int64), want.view(np.int64)), op


def test_log_sqrt_rsqrt_sin_libm_family_dispatch():
    xs = np.geomspace(1e-3, 1e3, 61)
    assert np.array_equal(_oracle_unary("log", xs), np.log(xs))
    assert np.array_equal(_oracle_unary("sqrt", xs), np.sqrt(xs))
    assert np.array_equal(_oracle_unary("rsqrt", xs), 1.0 / np.sqrt(xs))
    # Without the poly7 family, Sin is the libm sine (kernel_buffers.cpp:143).
    ys = np.linspace(-20.0, 20.0, 81)
    assert np.array_equal(_oracle_unary("sin", ys), np.array([math.sin(y) for y in ys]))
    # And with it, the polynomial, which differs from libm somewhere here.
    assert not np.array_equal(_oracle_unary("sin", ys, "poly7"), _oracle_unary("sin", ys))


def test_pow_general_arm_and_fast_form():
    # Pow: (2, 2) -> a * a, otherwise std::pow, including its special cases.
    pairs = [(2.0, 2.0, 4.0), (2.0, 0.5, math.sqrt(2.0)), (-2.0, 3.0, -8.0), (0.0, -1.0, math.inf),
             (9.0, 0.5, 3.0), (4.0, -0.5, 0.5)]
    for a, b, want in pairs:
        km = fx.lower_elementwise([], [KernelExpr("pow", const(a), const(b))], [1], "f64")
        assert oracle.run(km, {})[0][0] == want, (a, b)
    km = fx.lower_elementwise([], [KernelExpr("pow", const(-2.0), const(0.5))], [1], "f64")
    assert math.isnan(oracle.run(km, {})[0][0])


def test_gelu_closed_forms():
    # Gelu is the tanh form 0.5 a (1 + tanh(sqrt(2/pi) (a + 0.044715 a^3)))
    # (kernel_buffers.cpp:152-154). Closed forms it must satisfy:
    xs = np.linspace(-6.0, 6.0, 241)
    g = _oracle_unary("gelu", xs)
    gm = _oracle_unary("gelu", -xs)
    # gelu(0) = 0 exactly.
    assert _oracle_unary("gelu", [0.0])[0] == 0.0
    # The tanh is odd, so gelu(x) - gelu(-x) = x (to rounding).
    assert np.max(np.abs((g - gm) - xs)) <= 8 * np.finfo(np.float64).eps * 6.0
    # Limits: the tanh saturates to +-1 in f64, so gelu(x) = x and gelu(-x) = 0.
    big = _oracle_unary("gelu", [10.0, 30.0, -10.0, -30.0])
    assert big[0] == 10.0 and big[1] == 30.0 and big[2] == 0.0 and big[3] == 0.0
    # It approximates x * Phi(x) (the erf form) within 4.8e-4, the accuracy of
    # the tanh approximation; 0.8 in place of sqrt(2/pi) gives 6.4e-4 and a
    # dropped cubic term 2e-2.
    exact = np.array([0.5 * x * (1.0 + math.erf(x / math.sqrt(2.0))) for x in xs])
    assert np.max(np.abs(g - exact)) < 4.8e-4
    wrong_cubic = np.array([0.5 * x * (1.0 + math.tanh(0.7978845608028654 * x)) for x in xs])
    assert np.max(np.abs(wrong_cubic - exact)) > 1e-2 > np.max(np.abs(g - exact))
