"""CPU-side checks of the product library: it loads, exports the C ABI of
include/mlk_hip.h, recognizes every hot-path module form, refuses what no
kernel covers, and its template instances compile for gfx950 (hipRTC needs no
device). No compute call runs here."""
import ctypes
import json
import math
import os
import re

import pytest

from mlk2_amd import backend as be
from mlk2_amd import fixtures as fx
import test_nest as tn
import numpy as np
import oracle

from mlk2_amd.kernel_ir import (INVALID_ID, KernelBuffer, KernelExpr, KernelModule, KernelNode, const,
                                elem_a, elem_b, elem_idx, temp)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "mlk_hip.h")).read()
    return sorted(set(re.findall(r"\b(mlkhip_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = be.lib()
    syms = declared_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(L, s), s


def test_valid_arch():
    L = be.lib()
    for ok in ("gfx950", "gfx90a", "gfx942", "gfx1100"):
        assert L.mlkhip_valid_arch(ok.encode()) == 1, ok
    for bad in ("sm_90", "gfx", "gfx95", "gfx9500a", "GFX950", "gfx95z", ""):
        assert L.mlkhip_valid_arch(bad.encode()) == 0, bad


@pytest.mark.parametrize("name,km,cls,policy", [
    ("c1", fx.config1_module(1 << 12), "elementwise-1d", "tol-4ulp-f32-gfx950-v1"),
    ("c1f64", fx.config1_module(1 << 12, dtype="f64"), "elementwise-1d", "bitexact-rne-gfx950-v1"),
    # f16 output: the exact f64 sine, rounded once.
    ("c1f16", fx.config1_module(1 << 12, dtype="f16"), "elementwise-1d", "bitexact-rne-gfx950-v1"),
    ("c2-call", fx.config2_module(64, 128, 1), "softmax-call", "tol-rel1e-6-gfx950-v1"),
    ("c2-nest", fx.config2_module(64, 128, 2), "softmax-nest", "tol-rel1e-6-gfx950-v1"),
    ("c2-full-nest", fx.config2_module(8192, 4096, 2), "softmax-nest", "tol-rel1e-6-gfx950-v1"),
    ("c3-nest", fx.config3_module(64, 128, 2), "elementwise-nd", "tol-rel1e-6-gfx950-v1"),
    ("c4a-nest", fx.config4_module(1024, 1024, 1024, "f32", 2), "gemm-nest", "tol-rel1e-5sqrtk-gfx950-v1"),
    ("c4b-call", fx.config4_module(64, 64, 64, "f16", 1), "gemm-call", "tol-rel1e-2-gfx950-v1"),
    ("c5", fx.score_softmax_module(16, 2048, 128), "score-softmax", "tol-rel1e-2-gfx950-v1"),
    ("reducesum", fx.synth_reducesum(fx.reducesum_call_module(8, 16)), "reducesum-nest", "tol-rel1e-6-gfx950-v1"),
])
def test_plan_classes(name, km, cls, policy):
    got_cls, got_pol, steps = be.plan(km)
    assert (got_cls, got_pol, steps) == (cls, policy, 1), name


def test_full_size_synth_softmax_plans_without_temps():
    # The reference walker refuses this module (2^25-element exp temp above
    # kKernelTempElementsLimit, kernel_buffers.cpp:852-878); the softmax
    # class keeps the row in registers and materializes no temp.
    cls, _, _ = be.plan(fx.config2_module(8192, 4096, 2))
    assert cls == "softmax-nest"


def test_tier1_broadcast_module_refused():
    with pytest.raises(be.MlkHipError) as ei:
        be.plan(fx.config3_module(64, 128, tier=1))
    assert ei.value.code == be.REFUSED
    assert "outside its buffer" in ei.value.message


def test_unrecognized_nest_takes_generic_path():
    km = fx.config3_module(8, 8, tier=2)
    km.nodes[2].begin_coeffs = [0]          # affine bound: no hand-written class
    km.nodes[2].end_coeffs = [1]
    cls, policy, steps = be.plan(km)
    assert (cls, steps) == ("loop-nest", 1)
    # A loop with a non-unit step has no walker semantics: refused.
    km.nodes[2].step = 2
    with pytest.raises(be.MlkHipError):
        be.plan(km)


def _plan_text(text: bytes):
    cls = ctypes.create_string_buffer(256)
    pol = ctypes.create_string_buffer(64)
    n = ctypes.c_int()
    rc = be.lib().mlkhip_plan(text, len(text), cls, 256, pol, 64, ctypes.byref(n))
    return rc, cls.value.decode(), pol.value.decode(), n.value


def test_reference_writer_quirks_parse():
    # The reference writer clamps -inf to -1e308 and writes NaN as null
    # (compiler/src/core/json.cpp:300-312). The synthesized softmax's -inf
    # init therefore arrives as -1e308 and must still be the softmax class.
    km = fx.config2_module(4, 8, 2)
    text = km.to_reference_json()
    assert '"value":-1e308' in text and "Infinity" not in text
    rc, cls, _, _ = _plan_text(text.encode())
    assert rc == 0 and cls == "softmax-nest"


@pytest.mark.parametrize("km", [
    fx.config1_module(1 << 12), fx.config2_module(64, 128, 1), fx.config2_module(64, 128, 2),
    fx.config3_module(64, 128, 2),
    fx.config4_module(64, 32, 48, "f32", 1), fx.config4_module(256, 64, 256, "f16", 2),
    fx.reducesum_call_module(8, 16), fx.synth_reducesum(fx.reducesum_call_module(8, 16)),
    fx.score_softmax_module(2, 256, 128),
])
def test_reference_document_plans_like_the_extended_one(km):
    # Every configuration's module, serialized exactly as the reference
    # writer would (no Call "math", clamped infinities, null NaN), plans to
    # the same class and policy as the lossless document.
    ref = _plan_text(km.to_reference_json().encode())
    ext = _plan_text(km.to_json().encode())
    assert ref[0] == 0 and ref == ext


@pytest.mark.parametrize("math_name,with_b,out_rank", [("matmul", True, 2), ("softmax", False, 2),
                                                       ("reduce_sum", False, 1)])
def test_call_target_inferred_from_operands(math_name, with_b, out_rank):
    # tools/mlk-poly/poly_bench.cpp:121-158: MatMul binds B; Softmax is rank-2
    # in and out; ReduceSum is rank-2 in, rank-1 out.
    km = KernelModule()
    a = km.add_buffer(KernelBuffer("A", "f32", is_input=True, elements=8 * 4, dims=[8, 4]))
    b = km.add_buffer(KernelBuffer("B", "f32", is_input=True, elements=4 * 6, dims=[4, 6])) if with_b else INVALID_ID
    dims = [8, 6] if with_b else ([8, 4] if out_rank == 2 else [8])
    o = km.add_buffer(KernelBuffer("Y", "f32", is_output=True, elements=int(np.prod(dims)), dims=dims))
    km.add_node(KernelNode(op="call", math=math_name, a=a, b=b, out=o))
    rc, cls, _, _ = _plan_text(km.to_reference_json().encode())
    assert '"math"' not in km.to_reference_json()
    want = {"matmul": "gemm-call", "softmax": "softmax-call", "reduce_sum": "reducesum-call"}[math_name]
    assert rc == 0 and cls == want


def test_fused_softmax_refused_when_a_later_root_reads_its_temps():
    # The softmax class keeps the row max, exponentials and sum on chip. A
    # later root that reads the row-max temp makes the nest run on the
    # generic loop-nest path, whose temps are materialized as the walker's.
    km = fx.softmax_rowmax_reader_module(4, 8)
    cls, _, _ = be.plan(km)
    assert not cls.startswith("softmax-nest"), cls
    assert cls.startswith("loop-nest"), cls
    # Without the reader the same nest is the softmax class.
    cls2, _, _ = be.plan(fx.config2_module(4, 8, 2))
    assert cls2 == "softmax-nest"


def test_fused_score_softmax_refused_when_a_later_root_reads_the_scores():
    km = fx.score_softmax_module(1, 256, 128)
    cls, _, _ = be.plan(km)
    assert cls == "score-softmax"
    km2 = fx.score_reader_module(1, 256, 128)
    cls2, _, _ = be.plan(km2)
    assert "score-softmax" not in cls2, cls2


def test_hiprtc_options_disable_packed_fp32():
    buf = ctypes.create_string_buffer(512)
    n = be.lib().mlkhip_jit_options(b"gfx950", buf, 512)
    opts = buf.value.decode().split(" ")
    assert n == len(opts)
    assert opts[0] == "--offload-arch=gfx950"
    assert "-ffp-contract=off" in opts
    i = opts.index("-packed-fp32-ops")
    assert opts[i - 3:i + 1] == ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def test_elementwise_instances_have_distinct_kernel_names():
    _, s1 = be.compile_check(fx.config1_module(1 << 12), 0, "gfx950")
    _, s3 = be.compile_check(fx.config3_module(64, 128, 2), 0, "gfx950")
    n1 = [l for l in s1.splitlines() if l.startswith("#define MLK_KERNEL_NAME ")][0].split()[-1]
    n3 = [l for l in s3.splitlines() if l.startswith("#define MLK_KERNEL_NAME ")][0].split()[-1]
    assert n1.startswith("mlk_elementwise_") and n3.startswith("mlk_elementwise_")
    assert len(n1) == len("mlk_elementwise_") + 12 and n1 != n3


@pytest.mark.parametrize("km", [fx.config1_module(1 << 24), fx.config3_module(4096, 4096, 2),
                                fx.config1_module(1 << 10, dtype="f64")])
def test_template_instances_compile_for_gfx950(km):
    n, src = be.compile_check(km, 0, "gfx950")
    assert n > 0
    assert "#define MLK_GENERATED 1" in src
    assert "mlk_chain" in src


def test_chain_codegen_exact_constants():
    km = fx.lower_elementwise([("x", [16], "f64")],
                              [KernelExpr("mul", elem_a(), const(0.1)),
                               KernelExpr("add", temp(0), const(-math.inf))], [16], "f64")
    _, src = be.compile_check(km, 0, "gfx950")
    assert "0x1.999999999999ap-4" in src
    assert "(-__builtin_inf())" in src


@pytest.mark.parametrize("km,space", [
    (fx.config2_module(8192, 4096, 2), [5, 0, 2, 3, 4, 1]),
    (fx.config4_module(4096, 4096, 4096, "f16", 2), [8, 7, 0, 1, 2, 3, 5, 6]),
    (fx.score_softmax_module(16, 2048, 128), [0, 1]),
    (fx.score_softmax_module(2, 4096, 128), [0, 1]),
    (fx.score_softmax_module(2, 256, 128), [0, 1]),
    (fx.score_softmax_module(2, 384, 128), []),
    (fx.config4_module(1024, 1024, 1024, "f32", 2), [0, 1]),
    (fx.config4_module(64, 32, 64, "f32", 2), []),      # K below the 64-deep ring steps
    (fx.config1_module(1 << 12), []),
    (fx.config4_module(64, 64, 64, "f16", 1), []),     # below the 256-multiple tiles
    (tn.generic(tn.weighted_rows_module()), [0, 1, 2, 3, 4]),  # slabs, none, 512/64 threads, one fewer collapse
    (tn.generic(fx.tiled_gemm_module(70, 45, 37, "f32", tile=16, init="split", out_dtype="f32"), False),
     [0, 1, 2, 3]),   # f32 sums stored between k bands: no form 4
    (tn.generic(fx.lift_1d(fx.config1_module(n=1 << 12)), False), [0, 2, 3]),   # loop nest without slabs
])
def test_declared_variant_space(km, space):
    assert be.plan_variants(km, 0) == space


def test_variant_space_step_out_of_range():
    with pytest.raises(be.MlkHipError):
        be.plan_variants(fx.config2_module(64, 128, 2), 3)


def chain_bodies(km):
    """(fast body, exact body or "") of the instance's chain prelude."""
    _, src = be.compile_check(km)
    prelude = src.split("// Fused elementwise kernel template")[0]

    def body(name):
        if f"#define {name} " not in prelude:
            return ""
        return prelude.split(f"#define {name} ")[1].split("\n\n")[0]
    return body("MLK_CHAIN_BODY"), body("MLK_CHAIN_EXACT")


# Chains over two streams a, b: (name, chain, fused?) -- a sum of an exact
# product becomes one fused multiply-add (the product of two f32 or f16
# values, or of one and a short constant, is exact in f64).
FUSE_CASES = [
    ("t+X", [KernelExpr("mul", elem_a(), elem_b()), KernelExpr("add", temp(0), elem_b())], True),
    ("X+t", [KernelExpr("mul", elem_a(), elem_b()), KernelExpr("add", elem_a(), temp(0))], True),
    ("t-X", [KernelExpr("mul", elem_a(), elem_b()), KernelExpr("sub", temp(0), elem_a())], True),
    ("X-t", [KernelExpr("mul", elem_a(), elem_b()), KernelExpr("sub", elem_b(), temp(0))], True),
    ("c1-form", [KernelExpr("mul", elem_a(), elem_a()), KernelExpr("mul", const(3.0), elem_a()),
                 KernelExpr("add", temp(0), temp(1))], True),
    ("long-const", [KernelExpr("mul", const(0.1), elem_a()), KernelExpr("add", temp(0), elem_b())], False),
    ("product-read-twice", [KernelExpr("mul", elem_a(), elem_b()), KernelExpr("add", temp(0), elem_a()),
                            KernelExpr("mul", temp(1), temp(0))], False),
]


@pytest.mark.parametrize("name,chain,fused", FUSE_CASES, ids=[c[0] for c in FUSE_CASES])
@pytest.mark.parametrize("dt_in", ["f32", "f16", "f64"])
@pytest.mark.parametrize("lift", [False, True])
def test_exact_product_sums_fuse(name, chain, fused, dt_in, lift):
    n = 4096
    km = fx.lower_elementwise([("a", [n], dt_in), ("b", [n], dt_in)], chain, [n], out_dtype="f64")
    if lift:
        km = fx.lift_1d(km)
    fast, exact = chain_bodies(km)
    want = fused and dt_in != "f64"
    assert ("__builtin_fma(" in fast) == want, (name, dt_in, fast)
    assert exact == ""          # no form here declines an element
    assert be.plan(km)[1] == "bitexact-rne-gfx950-v1"


# (name, chain, output dtype, whether the exp takes the f32-accurate form)
EXP_CASES = [
    ("exp*b", [KernelExpr("exp", elem_a()), KernelExpr("mul", temp(0), elem_b())], "f32", True),
    ("b/exp", [KernelExpr("exp", elem_a()), KernelExpr("div", elem_b(), temp(0))], "f32", True),
    ("-exp/b", [KernelExpr("exp", elem_a()), KernelExpr("neg", temp(0)), KernelExpr("div", temp(1), elem_b())],
     "f32", True),
    ("exp", [KernelExpr("exp", elem_a())], "f32", True),
    ("exp+b", [KernelExpr("exp", elem_a()), KernelExpr("add", temp(0), elem_b())], "f32", False),
    ("exp*exp-same", [KernelExpr("exp", elem_a()), KernelExpr("mul", temp(0), temp(0))], "f32", False),
    # The outer exp is the result itself; the inner one feeds its argument
    # (absolute error there becomes relative error of the result) and stays f64.
    ("exp(exp)", [KernelExpr("exp", elem_a()), KernelExpr("exp", temp(0))], "f32", True),
    ("exp*b-f64", [KernelExpr("exp", elem_a()), KernelExpr("mul", temp(0), elem_b())], "f64", False),
    ("exp*b-f16", [KernelExpr("exp", elem_a()), KernelExpr("mul", temp(0), elem_b())], "f16", False),
]


@pytest.mark.parametrize("name,chain,out_dt,fast_exp", EXP_CASES, ids=[c[0] for c in EXP_CASES])
def test_f32_accurate_exp_only_as_a_factor_of_an_f32_result(name, chain, out_dt, fast_exp):
    n = 4096
    km = fx.lower_elementwise([("a", [n], "f32"), ("b", [n], "f32")], chain, [n], out_dtype=out_dt)
    fast, exact = chain_bodies(km)
    assert fast.count("mlk_exp_f32acc(") == (1 if fast_exp else 0), (name, fast)
    if name == "exp(exp)":
        assert "t0 = exp(a0)" in fast and "t1 = mlk_exp_f32acc(a1, slow)" in fast
    # A declining form always comes with the exact chain for its elements.
    assert (exact != "") == fast_exp
    assert "mlk_exp_f32acc(" not in exact and "slow" not in exact
    if fast_exp:
        assert be.plan(km)[1] == "tol-rel1e-6-gfx950-v1"


def test_f32_accurate_exp_once_per_chain():
    n = 4096
    chain = [KernelExpr("exp", elem_a()), KernelExpr("exp", elem_b()), KernelExpr("mul", temp(0), temp(1))]
    km = fx.lower_elementwise([("a", [n], "f32"), ("b", [n], "f32")], chain, [n])
    fast, _ = chain_bodies(km)
    assert fast.count("mlk_exp_f32acc(") == 1 and fast.count(" exp(") == 1


@pytest.mark.parametrize("lift", [False, True])
def test_split_precision_sine_only_for_f32_outputs(lift):
    # The split-precision poly7 sine is chosen only where its result is
    # rounded to f32; f16 and f64 outputs keep the exact f64 form, in the
    # 1-D template and the n-D one alike.
    for dtype, split in (("f32", True), ("f16", False), ("f64", False)):
        km = fx.config1_module(1 << 12, dtype=dtype)
        if lift:
            km = fx.lift_1d(km)
        _, src = be.compile_check(km)
        # The instance's chain is the prelude, ahead of the template text
        # (whose comments show an example chain).
        body = [line for line in src.splitlines() if "mlk_p7_sin" in line and "const double" in line]
        assert body, dtype
        assert ("mlk_p7_sin_f32out(" in body[0]) == split, (dtype, body[0])


def in_place(km):
    """The chain's store pointed back at its first input: y is x. The input
    stays an input only, so the reference's executor, which looks buffers up
    by position (kernel_buffers.cpp resolveOutput), writes through it."""
    root = km.nodes[km.roots()[0]]
    while True:
        kids = [km.nodes[c] for c in root.children]
        store = next((n for n in kids if n.op == "store"), None)
        if store is not None:
            break
        root = kids[0]
    src = 0
    store.out = src
    return km


IN_PLACE_CASES = [
    ("sin", lambda: fx.config1_module(1 << 12)),
    ("exp*b", lambda: fx.lower_elementwise([("a", [4096], "f32"), ("b", [4096], "f32")],
                                           EXP_CASES[0][1], [4096], out_dtype="f32")),
    ("c3", lambda: fx.config3_module(64, 1024, 2)),
]


@pytest.mark.parametrize("name,make", IN_PLACE_CASES, ids=[c[0] for c in IN_PLACE_CASES])
@pytest.mark.parametrize("lift", [False, True])
def test_in_place_chains_plan_the_exact_forms(name, make, lift):
    # A chain that stores into the buffer it reads cannot take the forms
    # whose declined elements are redone from re-read inputs: by then the
    # inputs hold results. It plans the exact f64 forms, with no second pass.
    km = make()
    if lift and name != "c3":
        km = fx.lift_1d(km)
    fast, exact = chain_bodies(km)
    assert exact != ""                   # out of place: a declining form
    fast, exact = chain_bodies(in_place(km))
    assert exact == "", fast
    assert "f32acc" not in fast and "f32out" not in fast and "slow" not in fast.replace("(void)slow", "")


def _roots_module(order, roots):
    km = KernelModule()
    ids = {}
    for name in order:
        kind = {"x": dict(is_input=True), "t": dict(is_temp=True), "y": dict(is_output=True)}[name]
        ids[name] = km.add_buffer(KernelBuffer(name=name, dtype="f32", elements=64, dims=[64], **kind))
    for src, dst in roots:
        cid = km.add_node(KernelNode(op="compute", math="mul", exprs=[KernelExpr("mul", elem_a(), const(2.0))],
                                     a=ids[src], b=INVALID_ID))
        sid = km.add_node(KernelNode(op="store", out=ids[dst]))
        km.add_node(KernelNode(op="loop", var="i", begin=0, end=64, children=[cid, sid]))
    return km


def test_1d_path_resolves_buffers_by_position():
    # kernel_buffers.cpp resolveInput/resolveOutput: the 1-D executor looks
    # an input up as inputs[id], anything else it reads as outputs[id -
    # #inputs], an output it stores as outputs[id - #inputs], anything else
    # as inputs[id]. A temp between x and y leaves both roots without a
    # binding (the reference skips them); with y right after x both run.
    assert be.plan(_roots_module(("x", "t", "y"), (("x", "t"), ("t", "y"))))[2] == 0
    assert be.plan(_roots_module(("x", "y", "t"), (("x", "y"), ("y", "y"))))[2] == 2
    # A store into the input writes through the caller's array: it runs.
    assert be.plan(_roots_module(("x", "y"), (("x", "x"),)))[2] == 1


def test_call_buffers_resolved_by_position():
    # The Tier-1 call executors use the same lookup for their data: a
    # binding it cannot find is the reference's InvalidArgument; one that
    # lands on another buffer than the id is refused, not run on mismatched
    # shapes.
    km = KernelModule()
    a = km.add_buffer(KernelBuffer("A", "f32", is_input=True, elements=8 * 4, dims=[8, 4]))
    km.add_buffer(KernelBuffer("T", "f32", is_temp=True, elements=8, dims=[8]))   # between A and Y
    y = km.add_buffer(KernelBuffer("Y", "f32", is_output=True, elements=8 * 4, dims=[8, 4]))
    km.add_node(KernelNode(op="call", math="softmax", a=a, b=INVALID_ID, out=y))
    with pytest.raises(be.MlkHipError) as ei:
        be.plan(km)
    assert "not bound" in ei.value.message


def _nd_module(order, dst, reads=("x",)):
    # y[i] = sum of the read buffers at i, over a multi-dim (elem_idx) nest.
    km = KernelModule()
    ids = {}
    for name in order:
        kind = {"x": dict(is_input=True), "t": dict(is_temp=True)}.get(name, dict(is_output=True))
        ids[name] = km.add_buffer(KernelBuffer(name=name, dtype="f32", elements=64, dims=[64], **kind))
    ops = [elem_idx(ids[r], [1]) for r in reads] + [const(0.0)] * (2 - len(reads))
    cid = km.add_node(KernelNode(op="compute", exprs=[KernelExpr("add", ops[0], ops[1])]))
    sid = km.add_node(KernelNode(op="store", out=ids[dst], out_index_coeffs=[1]))
    km.add_node(KernelNode(op="loop", var="i", begin=0, end=64, children=[cid, sid]))
    return km


def test_multi_dim_path_checks_buffer_positions():
    # The walker looks non-temp buffers up by position as the 1-D executor
    # does (kernel_buffers.cpp elemPtr :85-103, execPair :730-737) and temps
    # by id. The lowering's tables (inputs, outputs, temps) resolve to the
    # ids themselves and plan as usual.
    assert be.plan(_nd_module(("x", "y", "t"), "y"))[2] == 1
    assert be.plan(_nd_module(("x", "y", "t"), "t"))[2] == 1
    # A temp between x and y leaves y's store without a binding: the
    # walker's InvalidArgument.
    for order, dst in ((("x", "t", "y"), "y"), (("x", "t", "y", "z"), "z")):
        km = _nd_module(order, dst)
        with pytest.raises(be.MlkHipError) as ei:
            be.plan(km)
        assert "walker: output buffer not bound" in ei.value.message
        with pytest.raises(RuntimeError, match="walker: output buffer not bound"):
            oracle.run(km, {0: np.zeros(64)})
    # With a second output after it, y's position reaches z's binding: the
    # module is declined rather than run on the wrong array.
    with pytest.raises(be.MlkHipError) as ei:
        be.plan(_nd_module(("x", "t", "y", "z"), "y"))
    assert "resolves by position" in ei.value.message
    # Stores into temps go by id wherever the temp sits.
    assert be.plan(_nd_module(("x", "t", "y"), "t"))[2] == 1
