"""The generic loop-nest path (mlk2_amd/csrc/host/nestgen.cpp).

Any multi-dim forest root no hand-written class claims (poly.codegen's tiled,
guarded and split forms, triangular bounds, recurrences) runs as one generated
kernel with the reference walker's semantics
(runtime/src/execution/kernel_buffers.cpp:453-835).

CPU tests compile each generated kernel for the host under AddressSanitizer
and UndefinedBehaviorSanitizer and run its whole grid one thread at a time, in
reverse order (``tests/nesthost.py``), against the oracle. That checks every
address the kernel forms, and the host's parallelization proof, before the
kernel runs on a GPU. GPU tests run the same modules through the C ABI.

Bar: f64 buffers with IEEE operations are bit-exact with the walker (any NaN
matches any NaN). f32 outputs of a register-held accumulation equal the
walker's f64 value rounded once (round to nearest even), so they are
bit-exact against the oracle's result rounded to f32. Chains with exp use
the elementwise tolerance of 1e-6 relative.
"""
import copy
import sys

import numpy as np
import pytest

import nest_fuzz as nf
import nesthost
import oracle
from mlk2_amd import backend
from mlk2_amd import fixtures as fx
from mlk2_amd import inputs
from mlk2_amd.kernel_ir import (KernelBuffer, KernelExpr, KernelModule, KernelNode, const, elem_idx)
from mlk2_amd.parity import max_rel


def say(msg):
    print(f"[nest] {msg}", flush=True)
    sys.stdout.flush()


def gemm_inputs(m, k, n, seed=7):
    rng = np.random.default_rng(seed)
    a = rng.uniform(-1, 1, m * k).astype(np.float32).astype(np.float64)
    b = rng.uniform(-1, 1, k * n).astype(np.float32).astype(np.float64)
    return a, b


def expected(ref: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f32":
        return ref.astype(np.float32).astype(np.float64)
    return ref


def generic(km, canonical: bool = True):
    """The module with the schedule parameters that select the generic
    loop-nest kernel for every root (and, with canonical=False, plan the
    module as written, without the canonical rewrite)."""
    out = fx.KernelModule(buffers=list(km.buffers), nodes=list(km.nodes), name=km.name,
                          schedule=dict(km.schedule))
    out.schedule["hip_generic"] = 1
    if not canonical:
        out.schedule["hip_canonical"] = 0
    return out


def collapsed(km, step=0) -> int:
    _, src = backend.compile_check(km, step)
    line = src.splitlines()[0]
    return int(line.split(",")[1].split()[0])


def neg_store_module() -> KernelModule:
    """i in [0,4): y[i-2] = x[i]; z[i] = 2*x[i] (two statements: no perfect
    nest, so the generic path runs it). The walker fails at i = 0."""
    km = KernelModule()
    x = km.add_buffer(KernelBuffer("x", "f64", True, False, False, 4, [4]))
    y = km.add_buffer(KernelBuffer("y", "f64", False, True, False, 4, [4]))
    z = km.add_buffer(KernelBuffer("z", "f64", False, True, False, 4, [4]))
    c0 = km.add_node(KernelNode(op="compute", exprs=[KernelExpr("add", elem_idx(x, [1]), const(0.0))]))
    s0 = km.add_node(KernelNode(op="store", out=y, out_index_coeffs=[1], out_index_offset=-2))
    c1 = km.add_node(KernelNode(op="compute", exprs=[KernelExpr("mul", elem_idx(x, [1]), const(2.0))]))
    s1 = km.add_node(KernelNode(op="store", out=z, out_index_coeffs=[1]))
    km.add_node(KernelNode(op="loop", var="i", begin=0, end=4, children=[c0, s0, c1, s1]))
    return km


def dynamic_end_module(n=8) -> KernelModule:
    """i in [0, elements): y[i] = x[i] + x[i+1]: the loop end is the run's
    element count, so the addresses are bounded only at run time."""
    km = KernelModule()
    x = km.add_buffer(KernelBuffer("x", "f64", True, False, False, n, [n]))
    y = km.add_buffer(KernelBuffer("y", "f64", False, True, False, n, [n]))
    c0 = km.add_node(KernelNode(op="compute", exprs=[KernelExpr("add", elem_idx(x, [1]), elem_idx(x, [1], 1))]))
    s0 = km.add_node(KernelNode(op="store", out=y, out_index_coeffs=[1]))
    km.add_node(KernelNode(op="loop", var="i", begin=0, end=-1, children=[c0, s0]))
    return km


def prefix_sum_module(n=300) -> KernelModule:
    """y[0] = x[0]; i in [1,n): y[i] = y[i-1] + x[i] -- a recurrence: no loop
    is parallel, the whole root runs in one thread, in order."""
    km = KernelModule()
    x = km.add_buffer(KernelBuffer("x", "f64", True, False, False, n, [n]))
    y = km.add_buffer(KernelBuffer("y", "f64", False, True, False, n, [n]))
    c0 = km.add_node(KernelNode(op="compute", exprs=[KernelExpr("add", elem_idx(x, [0]), const(0.0))]))
    s0 = km.add_node(KernelNode(op="store", out=y, out_index_coeffs=[0]))
    c1 = km.add_node(KernelNode(op="compute", exprs=[KernelExpr("add", elem_idx(y, [0, 1], -1),
                                                                 elem_idx(x, [0, 1]))]))
    s1 = km.add_node(KernelNode(op="store", out=y, out_index_coeffs=[0, 1]))
    l1 = km.add_node(KernelNode(op="loop", var="i", begin=1, end=n, children=[c1, s1]))
    km.add_node(KernelNode(op="loop", var="z", begin=0, end=1, children=[c0, s0, l1]))
    return km


def triangular_module(n=37) -> KernelModule:
    """i in [0,n): { y[i] = 0; j in [0, i]: y[i] += L[i,j] * x[j];
    guard j == i: d[i] = L[i,i] } -- lower-triangular product."""
    km = KernelModule()
    L = km.add_buffer(KernelBuffer("L", "f64", True, False, False, n * n, [n, n]))
    x = km.add_buffer(KernelBuffer("x", "f64", True, False, False, n, [n]))
    y = km.add_buffer(KernelBuffer("y", "f64", False, True, False, n, [n]))
    d = km.add_buffer(KernelBuffer("d", "f64", False, True, False, n, [n]))
    c0 = km.add_node(KernelNode(op="compute", exprs=[KernelExpr("add", const(0.0), const(0.0))]))
    s0 = km.add_node(KernelNode(op="store", out=y, out_index_coeffs=[1]))
    c1 = km.add_node(KernelNode(op="compute", exprs=[KernelExpr("mul", elem_idx(L, [n, 1]), elem_idx(x, [0, 1]))]))
    s1 = km.add_node(KernelNode(op="store", out=y, out_index_coeffs=[1, 0], accum="add"))
    c2 = km.add_node(KernelNode(op="compute", exprs=[KernelExpr("add", elem_idx(L, [n, 1]), const(0.0))]))
    s2 = km.add_node(KernelNode(op="store", out=d, out_index_coeffs=[1, 0]))
    g = km.add_node(KernelNode(op="guard", guard_coeffs=[1, -1], guard_offset=0, children=[c2, s2]))
    lj = km.add_node(KernelNode(op="loop", var="j", begin=0, end=-1, begin_coeffs=[0], begin_offset=0,
                                end_coeffs=[1], end_offset=0, children=[c1, s1, g]))
    km.add_node(KernelNode(op="loop", var="i", begin=0, end=n, children=[c0, s0, lj]))
    return km


def weighted_rows_module(M=24, N=40, K=19, off=5, dtype="f64", stored_w=False) -> KernelModule:
    """i, j parallel; k in [0,K): y[i,j] += w[k + off] * x[i,k]. Every (i, j)
    re-reads w[off, off + K), and every j re-reads row i of x. With
    ``stored_w`` a first root rewrites the input w in place (w[t] = w[t] * 1),
    so w is no longer read-only anywhere in the module."""
    km = KernelModule()
    nw = K + off + 3
    w = km.add_buffer(KernelBuffer("w", dtype, True, False, False, nw, [nw]))
    x = km.add_buffer(KernelBuffer("x", dtype, True, False, False, M * K, [M, K]))
    y = km.add_buffer(KernelBuffer("y", dtype, False, True, False, M * N, [M, N]))
    if stored_w:
        c0 = km.add_node(KernelNode(op="compute", exprs=[KernelExpr("mul", elem_idx(w, [1]), const(1.0))]))
        s0 = km.add_node(KernelNode(op="store", out=w, out_index_coeffs=[1]))
        km.add_node(KernelNode(op="loop", var="t", begin=0, end=nw, children=[c0, s0]))
    c = km.add_node(KernelNode(op="compute", exprs=[KernelExpr("mul", elem_idx(w, [0, 0, 1], off),
                                                                elem_idx(x, [K, 0, 1]))]))
    s = km.add_node(KernelNode(op="store", out=y, out_index_coeffs=[N, 1, 0], accum="add"))
    kl = km.add_node(KernelNode(op="loop", var="k", begin=0, end=K, children=[c, s]))
    jl = km.add_node(KernelNode(op="loop", var="j", begin=0, end=N, children=[kl], parallel=True))
    km.add_node(KernelNode(op="loop", var="i", begin=0, end=M, children=[jl], parallel=True))
    return km


def weighted_rows_inputs(km):
    # Multiples of 1/8 in [-4, 4): exact in f16, f32 and f64.
    rng = np.random.default_rng(11)
    return {b: rng.integers(-32, 32, km.buffers[b].elements).astype(np.float64) / 8.0 for b in (0, 1)}


def slab_lines(km, step=0):
    _, src = backend.compile_check(km, step)
    return [ln for ln in src.splitlines() if ln.startswith("// mlk-nest slab:")]


def host_vs_oracle(km, arrays, scalars=(), elements=0):
    st, cur = nesthost.run_module(km, arrays, scalars, elements, reverse=True)
    ref = oracle.run(km, {i: arrays[i] for i in km.input_ids()}, scalars, elements,
                     init={i: arrays[i] for i in km.output_ids() if i in arrays})
    return st, cur, ref


# ---------------------------------------------------------------- CPU ----
@pytest.mark.parametrize("init", ["hoist", "guard", "split"])
@pytest.mark.parametrize("dtype", ["f64", "f32"])
@pytest.mark.parametrize("canonical", [False, True])
def test_tiled_gemm_generic_host(init, dtype, canonical):
    # canonical=False: the tiled form itself on the generic kernel;
    # canonical=True: its canonical rewrite on the generic kernel (checks
    # that the rewrite keeps the walker's order: bit-exact in f64).
    m, k, n = 70, 45, 37
    km = fx.tiled_gemm_module(m, k, n, dtype, tile=16, init=init, out_dtype=dtype)
    g = generic(km, canonical)
    cls, pol, _ = backend.plan(g)
    assert set(cls.split("+")) == {"loop-nest"} and pol == "bitexact-rne-gfx950-v1"
    a, b = gemm_inputs(m, k, n)
    st, cur, ref = host_vs_oracle(g, {0: a, 1: b, 2: np.full(m * n, 7.0)})
    assert st == 0
    assert nf.same_bits(cur[2], expected(ref[2], dtype))


@pytest.mark.parametrize("init", ["hoist", "guard", "split"])
@pytest.mark.parametrize("shape", [(70, 45, 37, 16), (64, 32, 64, 16), (256, 160, 192, 32)])
def test_tiled_gemm_canonicalizes_to_gemm_class(init, shape):
    m, k, n, t = shape
    km = fx.tiled_gemm_module(m, k, n, "f32", tile=t, init=init)
    assert backend.plan(km) == ("gemm-nest", "tol-rel1e-5sqrtk-gfx950-v1", 1)
    km16 = fx.tiled_gemm_module(m, k, n, "f16", tile=t, init=init)
    assert backend.plan(km16)[0] == "gemm-nest"


def test_tiled_elementwise_canonicalizes_to_template_class():
    km = fx.tiled_elementwise_module(fx.config3_module(37, 100, tier=2), tile=32)
    assert backend.plan(km)[0] == "elementwise-nd"
    km = fx.tiled_elementwise_module(fx.lift_1d(fx.config1_module(n=1 << 20)), tile=32)
    assert backend.plan(km)[:2] == ("elementwise-nd", "tol-4ulp-f32-gfx950-v1")


def test_slab_plan_follows_reuse_budget_and_stores():
    # GEMM tiles re-read both operands within a workgroup: both staged whole.
    km = generic(fx.tiled_gemm_module(70, 45, 37, "f32", tile=16, init="split", out_dtype="f32"))
    assert slab_lines(km) == ["// mlk-nest slab: buffer 0 elements [0, 3150)",
                              "// mlk-nest slab: buffer 1 elements [0, 1665)"]
    # Hulls above the 64 KiB budget stay in global memory.
    big = generic(fx.tiled_gemm_module(256, 160, 192, "f32", tile=32, init="split", out_dtype="f32"))
    assert slab_lines(big) == []
    # C3 tiled: the bias row is re-read by every row, x once. Tile indices
    # only move the point loops' windows, so they are no reuse: x stays out.
    c3 = generic(fx.tiled_elementwise_module(fx.config3_module(37, 100, tier=2), tile=32), False)
    assert slab_lines(c3) == ["// mlk-nest slab: buffer 1 elements [0, 100)"]
    # The hull starts where the reads start.
    wr = generic(weighted_rows_module())
    assert slab_lines(wr) == ["// mlk-nest slab: buffer 0 elements [5, 24)",
                              "// mlk-nest slab: buffer 1 elements [0, 456)"]
    # A buffer that any Store of the module targets is never staged, even in
    # a root that only reads it.
    ws = generic(weighted_rows_module(stored_w=True))
    assert backend.plan(ws)[2] == 2
    assert slab_lines(ws, 1) == ["// mlk-nest slab: buffer 1 elements [0, 456)"]
    # The schedule parameter hip_slabs = 0 turns them off.
    off = generic(weighted_rows_module())
    off.schedule["hip_slabs"] = 0
    assert slab_lines(off) == []


@pytest.mark.parametrize("dtype", ["f64", "f32", "f16"])
@pytest.mark.parametrize("stored_w", [False, True])
def test_slabs_host(dtype, stored_w):
    # Under AddressSanitizer every redirected read lands inside its slab's
    # static copy; results stay bit-exact with the walker (inputs are exact
    # in every dtype and the sums are held in f64).
    km = generic(weighted_rows_module(dtype=dtype, stored_w=stored_w))
    arrays = weighted_rows_inputs(km)
    st, cur, ref = host_vs_oracle(km, arrays)
    assert st == 0
    want = ref[2].astype(np.float16).astype(np.float64) if dtype == "f16" else expected(ref[2], dtype)
    assert nf.same_bits(cur[2], want)


@pytest.mark.parametrize("wg", [64, 512])
@pytest.mark.parametrize("case", ["slabs-f64", "slabs-f16", "fuzz-3", "fuzz-11"])
def test_workgroup_forms_host(case, wg):
    # Launch forms 2 and 3 (512 and 64 threads per workgroup): the slab copy
    # loop strides by the workgroup size and the grid-stride loop by the
    # grid's thread count; under AddressSanitizer every access stays in
    # bounds, and the bits are form 0's and the walker's.
    if case.startswith("slabs"):
        km = generic(weighted_rows_module(dtype=case.split("-")[1]))
        arrays, scalars = weighted_rows_inputs(km), ()
    else:
        seed = int(case.split("-")[1])
        km = generic(nf.random_module(seed))
        arrays, scalars = nf.random_inputs(km, seed)
    assert {2, 3} <= set(backend.plan_variants(km, 0))
    st0, cur0 = nesthost.run_module(km, arrays, scalars)
    st, cur = nesthost.run_module(km, arrays, scalars, reverse=True, wg=wg)
    assert st == st0 == 0
    ref = oracle.run(km, {i: arrays[i] for i in km.input_ids()}, scalars,
                     init={i: arrays[i] for i in km.output_ids() if i in arrays})
    for i in km.output_ids():
        assert nf.same_bits(cur[i], cur0[i]), (case, wg, i)
        if km.buffers[i].dtype == "f64":
            assert nf.same_bits(cur[i], ref[i]), (case, wg, i)


@pytest.mark.parametrize("case", ["slabs-f64", "slabs-f16", "tiled-hoist", "tiled-split"])
def test_less_collapse_form_host(case):
    # Launch form 4 runs the innermost collapsed loop inside each thread: the
    # module planned with hip_collapse_max = (collapsed loops - 1) gives its
    # source. Under AddressSanitizer every access stays in bounds, and the
    # bits are form 0's and the walker's.
    if case.startswith("slabs"):
        km = generic(weighted_rows_module(dtype=case.split("-")[1]))
        arrays, scalars = weighted_rows_inputs(km), ()
    else:
        km = generic(fx.tiled_gemm_module(70, 45, 37, "f64", tile=16, init=case.split("-")[1], out_dtype="f64"),
                     canonical=False)
        rng = np.random.default_rng(3)
        arrays, scalars = {b: rng.integers(-32, 32, km.buffers[b].elements).astype(np.float64) / 8.0
                           for b in (0, 1)}, ()
    assert 4 in backend.plan_variants(km, 0)
    less = copy.deepcopy(km)
    less.schedule["hip_collapse_max"] = collapsed(km) - 1
    assert collapsed(less) == collapsed(km) - 1
    st0, cur0 = nesthost.run_module(km, arrays, scalars)
    st, cur = nesthost.run_module(less, arrays, scalars, reverse=True)
    assert st == st0 == 0
    ref = oracle.run(km, {i: arrays[i] for i in km.input_ids()}, scalars,
                     init={i: arrays[i] for i in km.output_ids() if i in arrays})
    for i in km.output_ids():
        assert nf.same_bits(cur[i], cur0[i]), (case, i)
        if km.buffers[i].dtype == "f64":
            assert nf.same_bits(cur[i], ref[i]), (case, i)


def test_tiled_gemm_collapses_all_parallel_levels():
    # Divisible sizes: one full tile part per level, i_t/i/j_t/j collapse.
    km = generic(fx.tiled_gemm_module(64, 32, 64, "f32", tile=16, init="split"), canonical=False)
    assert collapsed(km) == 4
    _, src = backend.compile_check(km)
    assert "double r0 = " in src  # C[i,j] held in an f64 register over the k band


# ------------------------------------------- anchors in the reference ----
def _loop(km, nid):
    n = km.nodes[nid]
    assert n.op == "loop", n.op
    return n


def test_split_gemm_fixture_is_the_spec_form():
    # docs/polyhedral_spec.md:252-267 writes the piecewise-split GEMM out as
    # for i { for k in [0,1) { for j { init; acc } } for k in [1,K) { for j
    # { acc } } }: the split k segments are sibling subtrees under i, the
    # init (a plain store of 0) runs only in the singleton segment, before
    # the accumulation in the same j body.
    m, k, n = 5, 7, 3
    km = fx.split_gemm_module(m, k, n)
    (root,) = km.roots()
    i = _loop(km, root)
    assert (i.var, i.begin, i.end, i.parallel) == ("i", 0, m, True)
    assert len(i.children) == 2
    segs = [_loop(km, c) for c in i.children]
    assert [(s_.var, s_.begin, s_.end) for s_ in segs] == [("k", 0, 1), ("k", 1, k)]
    bodies = []
    for seg in segs:
        (jid,) = seg.children
        j = _loop(km, jid)
        assert (j.var, j.begin, j.end, j.parallel) == ("j", 0, n, True)
        bodies.append([km.nodes[c] for c in j.children])
    assert [b.op for b in bodies[0]] == ["compute", "store", "compute", "store"]
    assert [b.op for b in bodies[1]] == ["compute", "store"]
    assert bodies[0][1].accum in (None, "none") and bodies[0][3].accum == "add" and bodies[1][1].accum == "add"


def test_split_gemm_collapse_chain_is_one_level():
    # tests/unit/unit_poly.cpp:4279-4286: the untiled scheduled GEMM's
    # collapse chain is ONE level [i], because the split k segments are
    # sibling subtrees (j duplicated per segment) and the interior
    # single-loop-child rule stops the collapse at i. The generic kernel
    # applies the same rule.
    km = fx.split_gemm_module(70, 45, 37)
    assert collapsed(generic(km, canonical=False)) == 1
    assert collapsed(generic(km, canonical=True)) == 1


@pytest.mark.parametrize("dtype", ["f64", "f32"])
def test_split_gemm_spec_form_host(dtype):
    # In this form C[i,j] is reloaded for every k (the k segments enclose the
    # j loops): an f32 C is rounded at each k step where the walker keeps
    # f64, so the plan claims bit-exactness for f64 buffers only.
    m, k, n = 70, 45, 37
    km = generic(fx.split_gemm_module(m, k, n, dtype, dtype), canonical=False)
    assert backend.plan(km)[1] == ("bitexact-rne-gfx950-v1" if dtype == "f64" else "tol-rel1e-6-gfx950-v1")
    a, b = gemm_inputs(m, k, n)
    st, cur, ref = host_vs_oracle(km, {0: a, 1: b, 2: np.full(m * n, 7.0)})
    assert st == 0
    if dtype == "f64":
        assert nf.same_bits(cur[2], ref[2])
    else:
        assert not nf.same_bits(cur[2], expected(ref[2], dtype))  # the per-step rounding shows
        assert max_rel(cur[2], ref[2]) <= 1e-6
    # The init overwrote the 7.0 everywhere: C = A B exactly as the walker sums it.
    assert np.array_equal(ref[2], oracle.run(fx.matmul_call_module(m, k, n, "f64", "f64"),
                                             {0: a, 1: b}, init={2: np.zeros(m * n)})[2])


def _chained_roots_module(dtype, overlap=True):
    """Root 1: y[i] = 0.1 x[i]; root 2: z[i] = 3 y[i + s] (s = 0, or past
    root 1's writes when overlap is False)."""
    n = 64
    km = KernelModule()
    x = km.add_buffer(KernelBuffer("x", dtype, True, False, False, 2 * n, [2 * n]))
    y = km.add_buffer(KernelBuffer("y", dtype, False, True, False, 2 * n, [2 * n]))
    z = km.add_buffer(KernelBuffer("z", dtype, False, True, False, n, [n]))
    for src, dst, c, off in ((x, y, 0.1, 0), (y, z, 3.0, 0 if overlap else n)):
        ex = KernelExpr("mul", elem_idx(src, [1], off), const(c))
        cp = km.add_node(KernelNode(op="compute", exprs=[ex]))
        st = km.add_node(KernelNode(op="store", out=dst, out_index_coeffs=[1]))
        km.add_node(KernelNode(op="loop", var="i", begin=0, end=n, children=[cp, st]))
    return km


@pytest.mark.parametrize("dtype", ["f64", "f32", "f16"])
def test_later_root_reading_a_narrow_output_is_not_bit_exact(dtype):
    # The walker keeps y in f64 between the roots; the device stores it in
    # y's dtype, so root 2 reads the rounded value. The plan says so.
    km = _chained_roots_module(dtype)
    want = {"f64": "bitexact-rne-gfx950-v1", "f32": "tol-rel1e-6-gfx950-v1", "f16": "tol-rel1e-2-gfx950-v1"}
    assert backend.plan(km)[1] == want[dtype]
    xs = np.random.default_rng(1).uniform(-1, 1, 128)
    ref = oracle.run(km, {0: xs})
    if dtype == "f32":
        xs32 = xs.astype(np.float32).astype(np.float64)
        ref = oracle.run(km, {0: xs32})
        y_dev = (ref[1][:64]).astype(np.float32).astype(np.float64)
        assert not np.array_equal((3.0 * y_dev).astype(np.float32), ref[2].astype(np.float32))
    # Reads of elements no earlier root wrote keep the claim.
    assert backend.plan(_chained_roots_module(dtype, overlap=False))[1] == "bitexact-rne-gfx950-v1"


@pytest.mark.parametrize("lo,hi,t", [(0, 44, 16), (0, 63, 16), (0, 15, 16), (0, 9, 16), (3, 40, 8)])
def test_tiled_level_parts_follow_the_spec(lo, hi, t):
    # docs/polyhedral_spec.md:275-282: a tiled band level is a TILE loop with
    # constant bounds floor(lo/t) .. floor(hi/t) and a POINT loop with affine
    # bounds t*ti .. t*ti + t - 1; a trailing partial tile, present exactly
    # when (hi + 1) % t != 0, is a sibling part whose point loop carries the
    # constant clipped end hi. Each point loop's begin is the tile
    # coefficient at the tile index's stack slot.
    km = fx.KernelModule()
    parts = fx._emit_tiled_levels(km, [("x", lo, hi, True, False)], lambda p, d: [], t)
    tiles = [_loop(km, pid) for pid in parts]
    covered = []
    for tl in tiles:
        assert tl.var == "x_t" and not tl.begin_coeffs and not tl.end_coeffs
        covered += list(range(tl.begin, tl.end))
        (pid,) = tl.children
        pt = _loop(km, pid)
        assert pt.var == "x" and pt.begin_coeffs == [t] and pt.begin_offset == 0
    assert covered == list(range(lo // t, hi // t + 1))
    partial = (hi + 1) % t != 0
    assert len(tiles) == (1 if not partial or (hi + 1) // t - 1 < lo // t else 2) or (partial and len(tiles) == 2)
    last_point = _loop(km, tiles[-1].children[0])
    if partial:
        assert tiles[-1].begin == hi // t and tiles[-1].end == hi // t + 1
        assert not last_point.end_coeffs and last_point.end == hi + 1
    else:
        assert last_point.end_coeffs == [t] and last_point.end_offset == t - 1


@pytest.mark.parametrize("canonical", [False, True])
def test_tiled_elementwise_generic_host(canonical):
    km = generic(fx.tiled_elementwise_module(fx.config3_module(37, 100, tier=2), tile=32), canonical)
    d = inputs.config_inputs("c3", {"rows": 37, "cols": 100})
    st, cur, ref = host_vs_oracle(km, {0: d["x"], 1: d["b"]})
    assert st == 0
    assert max_rel(cur[2], ref[2]) <= 1e-6


@pytest.mark.parametrize("canonical", [False, True])
@pytest.mark.parametrize("seed", range(24))
def test_fuzz_host(seed, canonical):
    km = generic(nf.random_module(seed), canonical)
    arrays, scalars = nf.random_inputs(km, seed)
    st, cur, ref = host_vs_oracle(km, arrays, scalars)
    assert st == 0
    for i in km.output_ids():
        assert nf.same_bits(cur[i], ref[i]), (seed, i)


@pytest.mark.parametrize("seed", range(16))
def test_tiled_fuzz_canonical_host(seed):
    # A random forest and the same forest strip-mined as poly codegen tiles
    # bands: the walker gives the same bits for both, the canonical rewrite
    # of the tiled form runs bit-exact on the generic kernel, and in most
    # seeds the canonical form plans to the untiled form's classes.
    km0 = nf.random_module(seed)
    km = nf.tiled_random_module(seed)
    arrays, scalars = nf.random_inputs(km0, seed)
    r0 = oracle.run(km0, {i: arrays[i] for i in km0.input_ids()}, scalars,
                    init={i: arrays[i] for i in km0.output_ids()})
    st, cur, ref = host_vs_oracle(generic(km, True), arrays, scalars)
    assert st == 0
    for i in km.output_ids():
        assert nf.same_bits(ref[i], r0[i]) and nf.same_bits(cur[i], ref[i]), (seed, i)


def test_recurrence_runs_serially_host():
    km = prefix_sum_module()
    assert collapsed(km) == 0
    x = np.arange(300, dtype=np.float64) * 0.5 - 20
    st, cur, ref = host_vs_oracle(km, {0: x})
    assert st == 0 and nf.same_bits(cur[1], ref[1])


def test_triangular_and_guard_host():
    km = triangular_module()
    assert collapsed(km) == 1  # i proven parallel: y[i], d[i] move with i only
    rng = np.random.default_rng(3)
    arrays = {0: rng.uniform(-1, 1, 37 * 37), 1: rng.uniform(-1, 1, 37)}
    st, cur, ref = host_vs_oracle(km, arrays)
    assert st == 0 and nf.same_bits(cur[2], ref[2]) and nf.same_bits(cur[3], ref[3])


def test_negative_store_reports_status_host():
    km = neg_store_module()
    assert backend.plan(km)[0] == "loop-nest"
    st, _ = nesthost.run_module(km, {0: np.arange(4.0)})
    assert st == 1
    with pytest.raises(oracle.OracleError):
        oracle.run(km, {0: np.arange(4.0)})


def test_dynamic_end_bounds_checked_host():
    km = dynamic_end_module()
    x = np.arange(8.0)
    st, cur, ref = host_vs_oracle(km, {0: x}, elements=7)
    assert st == 0 and nf.same_bits(cur[1], ref[1])
    # elements past the buffers: every out-of-range access is caught by the
    # kernel's own checks (AddressSanitizer sees none) and reported as 6.
    st, _ = nesthost.run_module(km, {0: x}, elements=12)
    assert st == 6


def test_nest_refusals():
    # A Call inside a loop nest has no walker semantics the kernel can mirror.
    km = KernelModule()
    a = km.add_buffer(KernelBuffer("A", "f32", True, False, False, 4, [2, 2]))
    y = km.add_buffer(KernelBuffer("Y", "f32", False, True, False, 4, [2, 2]))
    call = km.add_node(KernelNode(op="call", math="softmax", a=a, out=y))
    c = km.add_node(KernelNode(op="compute", exprs=[KernelExpr("add", elem_idx(a, [1]), const(0.0))]))
    s = km.add_node(KernelNode(op="store", out=y, out_index_coeffs=[1]))
    km.add_node(KernelNode(op="loop", var="i", begin=0, end=2, children=[call, c, s]))
    with pytest.raises(backend.MlkHipError):
        backend.plan(km)


# ---------------------------------------------------------------- GPU ----
@pytest.mark.gpu
@pytest.mark.parametrize("init", ["hoist", "guard", "split"])
@pytest.mark.parametrize("shape", [(70, 45, 37, 16), (256, 160, 192, 32)])
def test_tiled_gemm_gpu(hip, init, shape):
    m, k, n, t = shape
    say(f"tiled gemm {init} {m}x{k}x{n} tile {t}")
    a, b = gemm_inputs(m, k, n)
    c0 = np.full(m * n, 7.0)
    for dtype in ("f64", "f32"):
        km = fx.tiled_gemm_module(m, k, n, dtype, tile=t, init=init, out_dtype=dtype)
        ref = oracle.run(km, {0: a, 1: b}, init={2: c0})[2]
        # The generic kernel on the tiled form and on its canonical rewrite:
        # the walker's f64 sums, bit-exact (f32: rounded once).
        for canonical in (False, True):
            got = hip.build(generic(km, canonical)).run({0: a, 1: b, 2: c0})[2]
            assert nf.same_bits(got, expected(ref, dtype)), (dtype, canonical)
        # As planned: the canonical form on the GEMM class.
        art = hip.build(km)
        assert art.class_name == "gemm-nest"
        got = art.run({0: a, 1: b, 2: c0})[2]
        r = max_rel(got, ref)
        say(f"  {dtype} gemm-nest max_rel={r:.3e}")
        assert r <= 1e-5 * np.sqrt(k)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f64", "f32", "f16"])
def test_later_root_reading_a_narrow_output_gpu(hip, dtype):
    # Root 2 reads root 1's output: bit-exact on f64 buffers, and within the
    # plan's tolerance where the device rounds the intermediate buffer.
    km = _chained_roots_module(dtype)
    xs = np.random.default_rng(2).uniform(-1, 1, 128)
    np_dt = {"f64": np.float64, "f32": np.float32, "f16": np.float16}[dtype]
    xs = xs.astype(np_dt).astype(np.float64)
    art = hip.build(km)
    got = art.run({0: xs})
    ref = oracle.run(km, {0: xs})
    tol = {"bitexact-rne-gfx950-v1": 0.0, "tol-rel1e-6-gfx950-v1": 1e-6, "tol-rel1e-2-gfx950-v1": 1e-2}[art.policy]
    for bid in km.output_ids():
        want = ref[bid].astype(np_dt).astype(np.float64)
        err = max_rel(got[bid][:64], want[:64])
        say(f"chained roots {dtype} buffer {bid}: {art.policy}, max rel {err:.2e}")
        assert err <= tol if tol else nf.same_bits(got[bid][:64], want[:64])


@pytest.mark.gpu
def test_split_gemm_spec_form_gpu(hip):
    # The spec's piecewise-split GEMM on the generic kernel (chain [i] only):
    # the walker's f64 sums, bit-exact on f64 buffers; an f32 C is reloaded
    # per k step, so it is held to its plan's 1e-6.
    m, k, n = 70, 45, 37
    a, b = gemm_inputs(m, k, n)
    c0 = np.full(m * n, 7.0)
    for dtype in ("f64", "f32"):
        km = fx.split_gemm_module(m, k, n, dtype, dtype)
        ref = oracle.run(km, {0: a, 1: b}, init={2: c0})[2]
        for canonical in (False, True):
            art = hip.build(generic(km, canonical))
            got = art.run({0: a, 1: b, 2: c0})[2]
            if dtype == "f64":
                assert art.policy == "bitexact-rne-gfx950-v1"
                assert nf.same_bits(got, ref), canonical
            else:
                assert art.policy == "tol-rel1e-6-gfx950-v1"
                assert max_rel(got, ref) <= 1e-6, canonical
        say(f"split gemm (spec form) {dtype}: within its policy")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f64", "f32", "f16"])
def test_slabs_gpu(hip, dtype):
    say(f"lds slabs weighted rows {dtype}")
    for stored_w in (False, True):
        km = weighted_rows_module(M=64, N=256, K=41, off=7, dtype=dtype, stored_w=stored_w)
        g = generic(km)
        assert any("buffer 1" in ln for ln in slab_lines(g, 1 if stored_w else 0))
        arrays = weighted_rows_inputs(km)
        ref = oracle.run(km, arrays)
        got = hip.build(g).run(arrays)
        want = ref[2].astype(np.float16).astype(np.float64) if dtype == "f16" else expected(ref[2], dtype)
        assert nf.same_bits(got[2], want), (dtype, stored_w)


@pytest.mark.gpu
def test_tiled_c1_gpu(hip):
    say("tiled 1-D sin chain (poly7), 2^20")
    n = 1 << 20
    km = fx.tiled_elementwise_module(fx.lift_1d(fx.config1_module(n=n)), tile=32)
    x = inputs.config_inputs("c1", {"n": n})["x"]
    ref = oracle.run(km, {0: x})[1]
    # Generic kernel: exact f64 poly7, one rounding to f32.
    got = hip.build(generic(km, canonical=False)).run({0: x})[1]
    assert nf.same_bits(got, expected(ref, "f32"))
    # As planned: the elementwise template (split-precision sin, <= 4 ULP).
    from mlk2_amd.parity import ulp_distance_f32
    art = hip.build(km)
    assert art.class_name == "elementwise-nd"
    assert ulp_distance_f32(art.run({0: x})[1].astype(np.float32), ref).max() <= 4.0


@pytest.mark.gpu
def test_tiled_c3_gpu(hip):
    say("tiled broadcast exp chain 4096x4096")
    km = fx.tiled_elementwise_module(fx.config3_module(4096, 4096, tier=2), tile=32)
    d = inputs.config_inputs("c3")
    ref = oracle.run(km, {0: d["x"], 1: d["b"]})[2]
    for mod in (km, generic(km, canonical=False)):
        art = hip.build(mod)
        got = art.run({0: d["x"], 1: d["b"]})[2]
        r = max_rel(got, ref)
        say(f"tiled c3 {art.class_name} max_rel={r:.3e}")
        assert r <= 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(60))
def test_fuzz_gpu(hip, seed):
    km = nf.random_module(seed)
    say(f"fuzz seed {seed}: {backend.plan(km)[0]}")
    arrays, scalars = nf.random_inputs(km, seed)
    ref = oracle.run(km, {i: arrays[i] for i in km.input_ids()}, scalars,
                     init={i: arrays[i] for i in km.output_ids()})
    for mod in (km, generic(km, canonical=False)):
        got = hip.build(mod).run(arrays, scalars)
        for i in km.output_ids():
            assert nf.same_bits(got[i], ref[i]), (seed, i)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["fuzz-0", "fuzz-2", "fuzz-5", "fuzz-11", "tiled-split", "tiled-guard"])
def test_fuzz_every_nest_form_gpu(hip, case):
    # Every loop-nest launch form (slabs, no slabs, 512 and 64 threads per
    # workgroup, one fewer collapsed loop) pinned on every loop-nest step that
    # declares it: the bits are the walker's for each.
    if case.startswith("fuzz"):
        seed = int(case.split("-")[1])
        km = generic(nf.random_module(seed), canonical=False)
        arrays, scalars = nf.random_inputs(km, seed)
    else:
        seed = case
        km = generic(fx.tiled_gemm_module(70, 45, 37, "f64", tile=16, init=case.split("-")[1], out_dtype="f64"),
                     canonical=False)
        rng = np.random.default_rng(3)
        arrays = {b: rng.integers(-32, 32, km.buffers[b].elements).astype(np.float64) / 8.0 for b in (0, 1)}
        arrays[2] = np.zeros(km.buffers[2].elements)
        scalars = ()
    ref = oracle.run(km, {i: arrays[i] for i in km.input_ids()}, scalars,
                     init={i: arrays[i] for i in km.output_ids()})
    art = hip.build(km)
    steps = art.num_steps()
    for form in (0, 1, 2, 3, 4):
        pinned = 0
        for s in range(steps):
            space = art.step_variants(s)
            if space:
                art.set_step_variant(s, form if form in space else 0)
                pinned += form in space
        if form != 0 and pinned == 0:
            continue
        say(f"fuzz seed {seed}: nest form {form} on {pinned} step(s)")
        got = art.run(arrays, scalars)
        for i in km.output_ids():
            assert nf.same_bits(got[i], ref[i]), (seed, form, i)


def close_to_walker(got, ref, tol):
    """NaN where the walker has NaN, the same infinities, and
    |got - ref| / max(|ref|, 1) <= tol elsewhere."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if not np.array_equal(np.isnan(got), np.isnan(ref)):
        return False
    inf = np.isinf(ref)
    if not np.array_equal(got[inf], ref[inf]):
        return False
    return max_rel(got, ref) <= tol


@pytest.mark.gpu
@pytest.mark.parametrize("seed", list(range(24)) + [1009, 1195, 1249])   # the last three store infinities
def test_fuzz_transcendental_gpu(hip, seed):
    # The fuzz forests with chains that also draw exp, log, sin, cos, tan,
    # tanh, sqrt, rsqrt, erf, gelu and pow: device libm against the host's,
    # within 1e-9 of the reference's relative measure (a few f64 ULP per op,
    # grown through at most three ops per pair and the accumulations).
    km = nf.random_module(seed, exact_ops=False)
    say(f"transcendental fuzz seed {seed}: {backend.plan(km)[0]}")
    arrays, scalars = nf.random_inputs(km, seed)
    ref = oracle.run(km, {i: arrays[i] for i in km.input_ids()}, scalars,
                     init={i: arrays[i] for i in km.output_ids()})
    for mod in (km, generic(km, canonical=False)):
        got = hip.build(mod).run(arrays, scalars)
        for i in km.output_ids():
            assert close_to_walker(got[i], ref[i], 1e-9), (seed, i, max_rel(got[i], ref[i]))


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(24))
def test_tiled_fuzz_gpu(hip, seed):
    km = nf.tiled_random_module(seed)
    say(f"tiled fuzz seed {seed}: {backend.plan(km)[0]}")
    arrays, scalars = nf.random_inputs(km, seed)
    ref = oracle.run(km, {i: arrays[i] for i in km.input_ids()}, scalars,
                     init={i: arrays[i] for i in km.output_ids()})
    got = hip.build(km).run(arrays, scalars)
    for i in km.output_ids():
        assert nf.same_bits(got[i], ref[i]), (seed, i)


@pytest.mark.gpu
def test_serial_triangular_gpu(hip):
    say("recurrence + triangular/guard nests")
    km = prefix_sum_module()
    x = np.arange(300, dtype=np.float64) * 0.5 - 20
    assert nf.same_bits(hip.build(km).run({0: x})[1], oracle.run(km, {0: x})[1])
    km = triangular_module()
    rng = np.random.default_rng(3)
    arrays = {0: rng.uniform(-1, 1, 37 * 37), 1: rng.uniform(-1, 1, 37)}
    got = hip.build(km).run(arrays)
    ref = oracle.run(km, arrays)
    assert nf.same_bits(got[2], ref[2]) and nf.same_bits(got[3], ref[3])


@pytest.mark.gpu
def test_error_status_gpu(hip):
    say("nest run-time checks: negative store, dynamic end past the buffers")
    art = hip.build(neg_store_module())
    with pytest.raises(backend.MlkHipError) as e:
        art.run({0: np.arange(4.0)})
    assert e.value.code == 1
    art = hip.build(dynamic_end_module())
    x = np.arange(8.0)
    got = art.run({0: x}, elements=7)[1]
    assert nf.same_bits(got, oracle.run(dynamic_end_module(), {0: x}, elements=7)[1])
    with pytest.raises(backend.MlkHipError) as e:
        art.run({0: x}, elements=12)
    assert e.value.code == 6
