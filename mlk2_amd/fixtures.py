"""KernelModule builders: the module shapes the reference compiler hands to a
backend for the hot-path classes.

Tier-1 forms mirror ``lower.to_kernel_ir``
(``compiler/src/passes/lower/lower.to_kernel_ir.cpp:20-428``): buffers for the
placeholder inputs in value-id order, then the outputs; a fused elementwise
chain becomes ``[compute, store, loop]`` with ElemA/ElemB operands in
first-touch order; ``MatMul`` becomes a ``Call`` node. Softmax and ReduceSum
``Call`` modules are hand-built exactly like ``tools/mlk-poly/poly_bench.cpp:123-160``.

Tier-2 forms mirror ``poly.synth`` (``compiler/src/passes/poly/poly.synth.cpp``):
``buildGemmNodes`` (:58-147), ``buildReduceSumNodes`` (:153-229),
``buildElementwiseNodes`` (:231-353) and ``buildSoftmaxNodes`` (:363-523), node
emission order included, since node ids are part of the module.
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence

from .kernel_ir import (KernelBuffer, KernelExpr, KernelModule,
                        KernelNode, KernelOperand, const, elem_a, elem_b,
                        elem_idx, scalar, temp)


def _numel(dims: Sequence[int]) -> int:
    n = 1
    for d in dims:
        n *= int(d)
    return n


def _stride_of(dims: Sequence[int], idx: int) -> int:
    """poly.synth.cpp:44-51 strideOf."""
    s = 1
    for d in range(idx + 1, len(dims)):
        s *= dims[d] if dims[d] > 0 else 1
    return s


# ----------------------------------------------------------------- Tier 1 --
def lower_elementwise(inputs: Sequence[tuple], chain: List[KernelExpr],
                      out_dims: Sequence[int], out_dtype: str = "f32",
                      family: Optional[str] = None, elem_bufs=(0, 1),
                      vector_width: int = 8) -> KernelModule:
    """Fused elementwise chain as lower.to_kernel_ir emits it (:146-425).

    ``inputs`` are ``(name, dims, dtype)`` placeholder tensors in value-id
    order; ``elem_bufs`` gives the buffer ids bound to ElemA / ElemB (the
    first-touch order of the chain)."""
    km = KernelModule()
    for name, dims, dt in inputs:
        km.add_buffer(KernelBuffer(name=name, dtype=dt, is_input=True,
                                   elements=_numel(dims), dims=list(dims)))
    out_id = km.add_buffer(KernelBuffer(name="y", dtype=out_dtype, is_output=True,
                                        elements=_numel(out_dims), dims=list(out_dims)))
    uses_a = any(o.kind == "elem_a" for e in chain for o in (e.a, e.b))
    uses_b = any(o.kind == "elem_b" for e in chain for o in (e.a, e.b))
    compute = KernelNode(op="compute", math=chain[-1].op, family=family,
                         exprs=list(chain),
                         a=elem_bufs[0] if uses_a else 0xFFFFFFFF,
                         b=elem_bufs[1] if uses_b else 0xFFFFFFFF)
    store = KernelNode(op="store", out=out_id)
    cid = km.add_node(compute)
    sid = km.add_node(store)
    km.add_node(KernelNode(op="loop", var="i", begin=0, end=_numel(out_dims),
                           children=[cid, sid]))
    km.schedule["vector_width"] = vector_width
    return km


def sin_chain() -> List[KernelExpr]:
    """y = sin(x^2 + 3x) as lowered from examples/scalar/sin_graph.mlk:12-17
    (Mul(x,x), Mul(3,x), Add, Sin; ScalarToTensor is transparent,
    lower.to_kernel_ir.cpp:251-258)."""
    return [KernelExpr("mul", elem_a(), elem_a()),
            KernelExpr("mul", const(3.0), elem_a()),
            KernelExpr("add", temp(0), temp(1)),
            KernelExpr("sin", temp(2), const(0.0))]


def exp_affine_chain(a_operand: Optional[KernelOperand] = None) -> List[KernelExpr]:
    """y = exp(a*x + b) * x: Mul(a,x), Add(t0,b), Exp, Mul(t2,x). x touches
    ElemA first, b is ElemB; a is a Const (or ScalarParam 0)."""
    a = a_operand if a_operand is not None else const(0.5)
    return [KernelExpr("mul", a, elem_a()),
            KernelExpr("add", temp(0), elem_b()),
            KernelExpr("exp", temp(1), const(0.0)),
            KernelExpr("mul", temp(2), elem_a())]


def scalar_kernel_module(chain: List[KernelExpr], family: Optional[str] = None) -> KernelModule:
    """A scalar graph as lower.to_kernel_ir emits it (:355-425): ScalarParam
    operands, one f64 output slot, a loop of exactly one instance."""
    km = KernelModule()
    out_id = km.add_buffer(KernelBuffer(name="out", dtype="f64", is_output=True, elements=1))
    cid = km.add_node(KernelNode(op="compute", math=chain[-1].op, family=family, exprs=list(chain)))
    sid = km.add_node(KernelNode(op="store", out=out_id))
    km.add_node(KernelNode(op="loop", var="i", begin=0, end=1, children=[cid, sid]))
    km.schedule["vector_width"] = 8
    return km


def sin_graph_scalar_module() -> KernelModule:
    """examples/scalar/sin_graph.mlk:12-17 lowered as a scalar kernel: x is
    ScalarParam 0, y = sin(x*x + 3*x) with the poly7 family."""
    x = scalar(0)
    return scalar_kernel_module([KernelExpr("mul", x, x), KernelExpr("mul", const(3.0), x),
                                 KernelExpr("add", temp(0), temp(1)), KernelExpr("sin", temp(2), const(0.0))],
                                family="poly7")


def config1_module(n: int = 1 << 24, family: str = "poly7", dtype: str = "f32") -> KernelModule:
    """Config 1, Tier-1 form: 1-D fused sin(x^2+3x), family poly7."""
    return lower_elementwise([("x", [n], dtype)], sin_chain(), [n], dtype, family=family)


def config3_tier1_module(rows: int = 4096, cols: int = 4096, dtype: str = "f32",
                         a_operand=None) -> KernelModule:
    """Config 3, Tier-1 form. The 1-D path reads ElemB as b[i]
    (kernel_buffers.cpp:110-113), so with b[cols] this module reads out of
    bounds on the reference: the HIP backend rejects it (see the recognizer)."""
    return lower_elementwise([("x", [rows, cols], dtype), ("b", [cols], dtype)],
                             exp_affine_chain(a_operand), [rows, cols], dtype)


def matmul_call_module(m: int, k: int, n: int, dtype_in: str = "f32",
                       dtype_out: str = "f32", tiles: Optional[dict] = None) -> KernelModule:
    """MatMul lowered to Call (lower.to_kernel_ir.cpp:114-144): buffers A[M,K],
    B[K,N] (placeholders), C[M,N] (output)."""
    km = KernelModule()
    a = km.add_buffer(KernelBuffer("A", dtype_in, True, False, False, m * k, [m, k]))
    b = km.add_buffer(KernelBuffer("B", dtype_in, True, False, False, k * n, [k, n]))
    c = km.add_buffer(KernelBuffer("C", dtype_out, False, True, False, m * n, [m, n]))
    km.add_node(KernelNode(op="call", math="matmul", a=a, b=b, out=c))
    for key, v in (tiles or {}).items():
        km.schedule[key] = v
    return km


def softmax_call_module(m: int, k: int, dtype: str = "f32") -> KernelModule:
    """Call(Softmax) module as hand-built by poly_bench.cpp:123-160."""
    km = KernelModule()
    a = km.add_buffer(KernelBuffer("X", dtype, True, False, False, m * k, [m, k]))
    y = km.add_buffer(KernelBuffer("Y", dtype, False, True, False, m * k, [m, k]))
    km.add_node(KernelNode(op="call", math="softmax", a=a, out=y))
    return km


def reducesum_call_module(m: int, k: int, dtype: str = "f32") -> KernelModule:
    """Call(ReduceSum) module (poly_bench.cpp:123-160)."""
    km = KernelModule()
    a = km.add_buffer(KernelBuffer("X", dtype, True, False, False, m * k, [m, k]))
    y = km.add_buffer(KernelBuffer("Y", dtype, False, True, False, m, [m]))
    km.add_node(KernelNode(op="call", math="reduce_sum", a=a, out=y))
    return km


# ----------------------------------------------------------------- Tier 2 --
def synth_gemm(km: KernelModule) -> KernelModule:
    """poly.synth buildGemmNodes (:58-147): i{ j{ C=0; k{ C += A*B } } }."""
    call = km.nodes[km.roots()[0]]
    da, db = km.buffers[call.a].dims, km.buffers[call.b].dims
    M, K, N = da[0], da[1], db[1]
    c1 = KernelNode(op="compute", exprs=[
        KernelExpr("add", elem_idx(call.a, [K, 0, 1])),
        KernelExpr("add", elem_idx(call.b, [0, 1, N])),
        KernelExpr("mul", temp(0), temp(1))])
    s1 = KernelNode(op="store", out=call.out, out_index_coeffs=[N, 1, 0], accum="add")
    c0 = KernelNode(op="compute", exprs=[KernelExpr("add", const(0.0))])
    s0 = KernelNode(op="store", out=call.out, out_index_coeffs=[N, 1])
    k_loop = KernelNode(op="loop", var="pk", begin=0, end=K, children=[0, 1])
    j_loop = KernelNode(op="loop", var="pj", begin=0, end=N, children=[2, 3, 4])
    i_loop = KernelNode(op="loop", var="pi", begin=0, end=M, children=[5])
    out = KernelModule(buffers=list(km.buffers), name=km.name, schedule=dict(km.schedule))
    out.nodes = [c1, s1, c0, s0, k_loop, j_loop, i_loop]
    return out


def synth_reducesum(km: KernelModule) -> KernelModule:
    """poly.synth buildReduceSumNodes (:153-229): i{ Y=0; k{ Y += A } }."""
    call = km.nodes[km.roots()[0]]
    M, K = km.buffers[call.a].dims
    c1 = KernelNode(op="compute", a=call.a, exprs=[
        KernelExpr("add", elem_idx(call.a, [K, 1]), const(0.0))])
    s1 = KernelNode(op="store", out=call.out, out_index_coeffs=[1, 0], accum="add")
    k_loop = KernelNode(op="loop", var="rk", begin=0, end=K, children=[0, 1])
    c0 = KernelNode(op="compute", exprs=[KernelExpr("add", const(0.0), const(0.0))])
    s0 = KernelNode(op="store", out=call.out, out_index_coeffs=[1])
    i_loop = KernelNode(op="loop", var="ri", begin=0, end=M, children=[3, 4, 2])
    out = KernelModule(buffers=list(km.buffers), name=km.name, schedule=dict(km.schedule))
    out.nodes = [c1, s1, k_loop, c0, s0, i_loop]
    return out


def synth_elementwise(km: KernelModule) -> KernelModule:
    """poly.synth buildElementwiseNodes (:231-353): the 1-D chain becomes an
    R-dim nest over the output dims with broadcast-aware ElemIdx operands
    (trailing-dim alignment; size-1 and leading dims get coefficient 0)."""
    root = km.nodes[km.roots()[0]]
    compute = store = None
    for c in root.children:
        if km.nodes[c].op == "compute":
            compute = km.nodes[c]
        elif km.nodes[c].op == "store" and compute is not None:
            store = km.nodes[c]
            break
    od = km.buffers[store.out].dims
    rank = len(od)
    if rank < 2:
        return km

    def map_operand(o: KernelOperand) -> KernelOperand:
        if o.kind not in ("elem_a", "elem_b"):
            return o
        buf = compute.a if o.kind == "elem_a" else compute.b
        idims = km.buffers[buf].dims
        irank = len(idims)
        coeffs = [0] * rank
        for d in range(rank):
            if d + irank < rank:
                continue
            aligned = d - (rank - irank)
            if idims[aligned] == 1:
                continue
            coeffs[d] = _stride_of(idims, aligned)
        return elem_idx(buf, coeffs)

    exprs = compute.exprs or [KernelExpr(compute.math, elem_a(), elem_b())]
    new_compute = KernelNode(op="compute", family=compute.family, exprs=[
        KernelExpr(e.op, map_operand(e.a), map_operand(e.b)) for e in exprs])
    new_store = KernelNode(op="store", out=store.out,
                           out_index_coeffs=[_stride_of(od, d) for d in range(rank)],
                           accum=store.accum)
    nodes = [new_compute, new_store]
    ids = [0, 1]
    for d in range(rank - 1, -1, -1):
        nodes.append(KernelNode(op="loop", var=f"e{d}", begin=0, end=od[d]))
        ids.append(len(nodes) - 1)
    nodes[ids[2]].children = [ids[0], ids[1]]
    for k in range(2, len(ids) - 1):
        nodes[ids[k + 1]].children.append(ids[k])
    out = KernelModule(buffers=list(km.buffers), name=km.name, schedule=dict(km.schedule))
    out.nodes = nodes
    return out


def synth_softmax(km: KernelModule) -> KernelModule:
    """poly.synth buildSoftmaxNodes (:363-523): six statements over four
    sibling k-bands under m, with temps rowmax[M], exp[M,K], sum[M]."""
    call = km.nodes[km.roots()[0]]
    M, K = km.buffers[call.a].dims
    out = KernelModule(buffers=list(km.buffers), name=km.name, schedule=dict(km.schedule))
    rm = out.add_buffer(KernelBuffer("softmax_rowmax", "f32", is_temp=True, elements=M, dims=[M]))
    e = out.add_buffer(KernelBuffer("softmax_exp", "f32", is_temp=True, elements=M * K, dims=[M, K]))
    s = out.add_buffer(KernelBuffer("softmax_sum", "f32", is_temp=True, elements=M, dims=[M]))
    fam = call.family
    c0 = KernelNode(op="compute", family=fam, exprs=[KernelExpr("add", const(-math.inf), const(0.0))])
    s0 = KernelNode(op="store", out=rm, out_index_coeffs=[1])
    c1 = KernelNode(op="compute", family=fam, exprs=[KernelExpr("sub", elem_idx(call.a, [K, 1]), const(0.0))])
    s1 = KernelNode(op="store", out=rm, out_index_coeffs=[1, 0], accum="max")
    c2 = KernelNode(op="compute", family=fam, exprs=[
        KernelExpr("sub", elem_idx(call.a, [K, 1]), elem_idx(rm, [1, 0])),
        KernelExpr("exp", temp(0), const(0.0))])
    s2 = KernelNode(op="store", out=e, out_index_coeffs=[K, 1])
    c3 = KernelNode(op="compute", family=fam, exprs=[KernelExpr("add", const(0.0), const(0.0))])
    s3 = KernelNode(op="store", out=s, out_index_coeffs=[1])
    c4 = KernelNode(op="compute", family=fam, exprs=[KernelExpr("sub", elem_idx(e, [K, 1]), const(0.0))])
    s4 = KernelNode(op="store", out=s, out_index_coeffs=[1, 0], accum="add")
    c5 = KernelNode(op="compute", family=fam, exprs=[KernelExpr("div", elem_idx(e, [K, 1]), elem_idx(s, [1, 0]))])
    s5 = KernelNode(op="store", out=call.out, out_index_coeffs=[K, 1])

    def kloop(name, c, st):
        return KernelNode(op="loop", var=name, begin=0, end=K, children=[c, st])

    out.nodes = [c1, s1, kloop("sk_rm", 0, 1), c2, s2, kloop("sk_e", 3, 4), c3, s3,
                 kloop("sk_s", 9, 10), c4, s4, kloop("sk_d", 12, 13), c5, s5, c0, s0,
                 KernelNode(op="loop", var="sm", begin=0, end=M,
                            children=[14, 15, 2, 5, 6, 7, 8, 11])]
    return out


def config2_module(m: int = 8192, k: int = 4096, tier: int = 1) -> KernelModule:
    km = softmax_call_module(m, k, "f32")
    return synth_softmax(km) if tier == 2 else km


def config3_module(rows: int = 4096, cols: int = 4096, tier: int = 2, a_operand=None) -> KernelModule:
    km = config3_tier1_module(rows, cols, "f32", a_operand)
    return synth_elementwise(km) if tier == 2 else km


def config4_module(m: int, k: int, n: int, dtype_in: str, tier: int = 2) -> KernelModule:
    km = matmul_call_module(m, k, n, dtype_in, "f32")
    return synth_gemm(km) if tier == 2 else km


# ------------------------------------------------------ score + softmax --
def score_softmax_module(batch: int, seq: int, dim: int, dtype_in: str = "f16",
                         scale_div: Optional[float] = None, dtype_out: str = "f32",
                         reader_output: bool = False) -> KernelModule:
    """Config 5 as a Kernel IR composition of reference pieces (no single
    reference class covers it): a batched QK^T init+accumulate nest written
    like buildGemmNodes (:58-147) with the K operand read transposed through
    its ElemIdx coefficients, then the broadcast elementwise chain
    Add(Div(S, sqrt(dim)), bias[j]) as buildElementwiseNodes emits it
    (:231-353), then the stable softmax nest of buildSoftmaxNodes (:363-523)
    over the [batch*seq, seq] score rows into S (`dtype_out`). The score
    matrix is a temp."""
    c = float(math.sqrt(dim)) if scale_div is None else scale_div
    R = batch * seq
    km = KernelModule()
    q = km.add_buffer(KernelBuffer("Q", dtype_in, True, False, False, batch * seq * dim, [batch, seq, dim]))
    kb = km.add_buffer(KernelBuffer("K", dtype_in, True, False, False, batch * seq * dim, [batch, seq, dim]))
    bias = km.add_buffer(KernelBuffer("bias", "f32", True, False, False, seq, [seq]))
    y = km.add_buffer(KernelBuffer("S", dtype_out, False, True, False, R * seq, [R, seq]))
    if reader_output:  # a second output, filled by a root the caller appends
        km.add_buffer(KernelBuffer("scores_out", "f32", False, True, False, R * seq, [R, seq]))
    sc = km.add_buffer(KernelBuffer("scores", "f32", is_temp=True, elements=R * seq, dims=[R, seq]))
    # Root 1: b{ i{ j{ SC=0; k{ SC += Q[b,i,k] * K[b,j,k] } } } }
    n = []
    n.append(KernelNode(op="compute", exprs=[
        KernelExpr("add", elem_idx(q, [seq * dim, dim, 0, 1])),
        KernelExpr("add", elem_idx(kb, [seq * dim, 0, dim, 1])),
        KernelExpr("mul", temp(0), temp(1))]))                                  # 0
    n.append(KernelNode(op="store", out=sc, out_index_coeffs=[seq * seq, seq, 1, 0], accum="add"))  # 1
    n.append(KernelNode(op="compute", exprs=[KernelExpr("add", const(0.0))]))  # 2
    n.append(KernelNode(op="store", out=sc, out_index_coeffs=[seq * seq, seq, 1]))  # 3
    n.append(KernelNode(op="loop", var="qk", begin=0, end=dim, children=[0, 1]))    # 4
    n.append(KernelNode(op="loop", var="qj", begin=0, end=seq, children=[2, 3, 4]))  # 5
    n.append(KernelNode(op="loop", var="qi", begin=0, end=seq, children=[5]))        # 6
    n.append(KernelNode(op="loop", var="qb", begin=0, end=batch, children=[6]))      # 7
    # Root 2: r{ j{ SC[r,j] = Add(Div(SC[r,j], c), bias[j]) } }
    n.append(KernelNode(op="compute", exprs=[
        KernelExpr("div", elem_idx(sc, [seq, 1]), const(c)),
        KernelExpr("add", temp(0), elem_idx(bias, [0, 1]))]))                  # 8
    n.append(KernelNode(op="store", out=sc, out_index_coeffs=[seq, 1]))         # 9
    n.append(KernelNode(op="loop", var="e1", begin=0, end=seq, children=[8, 9]))    # 10
    n.append(KernelNode(op="loop", var="e0", begin=0, end=R, children=[10]))        # 11
    km.nodes = n
    # Root 3: stable softmax over the score rows into S.
    tmp = KernelModule(buffers=[], nodes=[])
    soft = synth_softmax(_softmax_over(km, sc, y, R, seq))
    base = len(km.nodes)
    for b in soft.buffers[len(km.buffers):]:
        km.add_buffer(b)
    for node in soft.nodes:
        node.children = [c_ + base for c_ in node.children]
        km.nodes.append(node)
    del tmp
    return km


def _append_copy_root(km: KernelModule, src: int, dims: Sequence[int], out: int) -> KernelModule:
    """Appends a last root that copies temp `src` into output buffer `out`
    (Add(src[...], 0) over a perfect nest): a later reader of a temp that a
    fused class would otherwise keep on chip."""
    coeffs = [_stride_of(dims, d) for d in range(len(dims))]
    c = km.add_node(KernelNode(op="compute", exprs=[KernelExpr("add", elem_idx(src, coeffs), const(0.0))]))
    st = km.add_node(KernelNode(op="store", out=out, out_index_coeffs=coeffs))
    child = [c, st]
    for d in range(len(dims) - 1, -1, -1):
        child = [km.add_node(KernelNode(op="loop", var=f"r{d}", begin=0, end=dims[d], children=child))]
    return km


def softmax_rowmax_reader_module(m: int, k: int) -> KernelModule:
    """Config 2's synthesized softmax followed by a root that copies the
    row-max temp into a second output. Outputs precede the temps in the
    table, as the reference's binding requires (an output id indexes the
    outputs after the input count, kernel_buffers.cpp:200-230)."""
    km = softmax_call_module(m, k, "f32")
    r = km.add_buffer(KernelBuffer("rowmax_out", "f32", False, True, False, m, [m]))
    km = synth_softmax(km)
    rm = next(i for i, b in enumerate(km.buffers) if b.name == "softmax_rowmax")
    return _append_copy_root(km, rm, [m], r)


def score_reader_module(batch: int, seq: int, dim: int) -> KernelModule:
    """Config 5's composition followed by a root that copies the scaled
    score temp into a second output (placed before the temps)."""
    km = score_softmax_module(batch, seq, dim, reader_output=True)
    sc = next(i for i, b in enumerate(km.buffers) if b.name == "scores")
    out = next(i for i, b in enumerate(km.buffers) if b.name == "scores_out")
    return _append_copy_root(km, sc, [batch * seq, seq], out)


def _softmax_over(km: KernelModule, x: int, y: int, rows: int, cols: int) -> KernelModule:
    view = KernelModule(buffers=list(km.buffers))
    view.nodes = [KernelNode(op="call", math="softmax", a=x, out=y)]
    return view


# ------------------------------------------- poly.codegen tiled forms --
def _stack_coeffs(depth: int, pos: dict, terms: dict) -> List[int]:
    """Stack-position coefficient vector (codegen.cpp mapCoeffs): `terms` maps
    a loop name to its coefficient, placed at that loop's stack position."""
    c = [0] * depth
    for name, v in terms.items():
        c[pos[name]] = v
    return c


def _emit_tiled_levels(km: KernelModule, levels: Sequence[tuple], body, tile: int,
                       depth: int = 0, pos: Optional[dict] = None) -> List[int]:
    """Tiled band emission following poly codegen's emitLoop/emitPointBody
    (polyhedral/src/codegen.cpp:296-420): per level a TILE loop over
    [floor(lo/t), (hi+1)/t - 1] holding a POINT loop with the affine inclusive
    bounds [t*ti, t*ti + t-1], plus a sibling partial tile whose point loop
    ends at the constant hi when t does not divide hi+1; the inner levels are
    replayed under each part. Tile and point loops carry the level's parallel
    mark, the point loop its vector hint. ``levels`` are (name, lo, hi,
    parallel, vector); ``body(pos, depth)`` returns the innermost children."""
    pos = dict(pos or {})
    if not levels:
        return body(pos, depth)
    name, lo, hi, par, vec = levels[0]
    t = tile
    first, full_last, last = lo // t, (hi + 1) // t - 1, hi // t
    parts = []
    if full_last >= first:
        parts.append(("full", first, full_last))
    if (hi + 1) % t != 0:
        parts.append(("partial", last, last))
    ids = []
    for kind, t0, t1 in parts:
        tile_id = km.add_node(KernelNode(op="loop", var=name + "_t", begin=t0, end=t1 + 1, parallel=par))
        inner = dict(pos)
        inner[name] = depth + 1
        children = _emit_tiled_levels(km, levels[1:], body, tile, depth + 2, inner)
        bc = [0] * (depth + 1)
        bc[depth] = t
        point = KernelNode(op="loop", var=name, begin_coeffs=bc, begin_offset=0, parallel=par,
                           vector_hint=vec, children=children)
        if kind == "full":
            ec = [0] * (depth + 1)
            ec[depth] = t
            point.end_coeffs = ec
            point.end_offset = t - 1
        else:
            point.end = hi + 1
        km.nodes[tile_id].children.append(km.add_node(point))
        ids.append(tile_id)
    return ids


def lift_1d(km: KernelModule) -> KernelModule:
    """A Tier-1 1-D chain (Loop{Compute; Store} over ElemA/ElemB) written as
    the one-level multi-dim nest the polyhedral scop models it as
    (polyhedral/src/scop.cpp:107-149): each legacy operand becomes an ElemIdx
    access with coefficient 1 on the loop, the store gets coefficient 1."""
    root = km.nodes[km.roots()[0]]
    compute = next(km.nodes[c] for c in root.children if km.nodes[c].op == "compute")
    store = next(km.nodes[c] for c in root.children if km.nodes[c].op == "store")

    def lift(o: KernelOperand) -> KernelOperand:
        if o.kind == "elem_a":
            return elem_idx(compute.a, [1])
        if o.kind == "elem_b":
            return elem_idx(compute.b, [1])
        return o

    out = KernelModule(buffers=list(km.buffers), name=km.name, schedule=dict(km.schedule))
    c = out.add_node(KernelNode(op="compute", family=compute.family,
                                exprs=[KernelExpr(e.op, lift(e.a), lift(e.b)) for e in compute.exprs]))
    st = out.add_node(KernelNode(op="store", out=store.out, out_index_coeffs=[1]))
    out.add_node(KernelNode(op="loop", var="i", begin=root.begin, end=root.end, children=[c, st]))
    return out


def tiled_elementwise_module(synth: KernelModule, tile: int = 32) -> KernelModule:
    """A poly.synth broadcast elementwise nest (one perfect nest ending in
    Compute+Store) re-emitted with every level tiled by ``tile`` and marked
    parallel, the innermost point loop vector-hinted: the shape poly.codegen
    gives a dependence-free band."""
    root = synth.nodes[synth.roots()[0]]
    dims = []
    cur = root
    while True:
        dims.append(cur.end)
        ch = [synth.nodes[c] for c in cur.children]
        if len(ch) == 1 and ch[0].op == "loop":
            cur = ch[0]
            continue
        compute, store = ch
        break
    rank = len(dims)
    names = [f"e{d}" for d in range(rank)]
    out = KernelModule(buffers=list(synth.buffers), name=synth.name, schedule=dict(synth.schedule))

    def remap(o: KernelOperand, pos, depth) -> KernelOperand:
        if o.kind != "elem_idx":
            return o
        return elem_idx(o.index, _stack_coeffs(depth, pos, {names[d]: c for d, c in enumerate(o.coeffs)
                                                            if d < rank}), o.offset)

    def body(pos, depth):
        c = KernelNode(op="compute", family=compute.family, exprs=[
            KernelExpr(e.op, remap(e.a, pos, depth), remap(e.b, pos, depth)) for e in compute.exprs])
        s = KernelNode(op="store", out=store.out, accum=store.accum, out_index_offset=store.out_index_offset,
                       out_index_coeffs=_stack_coeffs(depth, pos, {names[d]: c_ for d, c_ in
                                                                   enumerate(store.out_index_coeffs)}))
        return [out.add_node(c), out.add_node(s)]

    levels = [(names[d], 0, dims[d] - 1, True, d == rank - 1) for d in range(rank)]
    _emit_tiled_levels(out, levels, body, tile)
    return out


def tiled_gemm_module(m: int, k: int, n: int, dtype_in: str = "f32", tile: int = 32,
                      init: str = "split", out_dtype: str = "f32") -> KernelModule:
    """The poly.synth GEMM statements (S0: C[i,j] = 0 over (i,j); S1:
    C[i,j] += A[i,k]*B[k,j] over (i,j,k), poly.synth.cpp:58-147) in the tiled
    forms poly.codegen can give them, i and j parallel, k sequential. ``init``
    places S0 as codegen's three strategies do (codegen.cpp:1-30, :440-530):
    "hoist" emits it before the k band (its k value precedes the loop),
    "guard" re-enters it in the k loop under the guard k == 0, and "split" cuts
    the k range at 0 so S0 runs only in the singleton segment [0, 0] of the
    first k tile, with constant point segments."""
    km = KernelModule()
    a = km.add_buffer(KernelBuffer("A", dtype_in, True, False, False, m * k, [m, k]))
    b = km.add_buffer(KernelBuffer("B", dtype_in, True, False, False, k * n, [k, n]))
    c = km.add_buffer(KernelBuffer("C", out_dtype, False, True, False, m * n, [m, n]))

    def s0(pos, depth):
        cp = KernelNode(op="compute", exprs=[KernelExpr("add", const(0.0), const(0.0))])
        st = KernelNode(op="store", out=c, out_index_coeffs=_stack_coeffs(depth, pos, {"i": n, "j": 1}))
        return [km.add_node(cp), km.add_node(st)]

    def s1(pos, depth):
        cp = KernelNode(op="compute", exprs=[
            KernelExpr("add", elem_idx(a, _stack_coeffs(depth, pos, {"i": k, "k": 1})), const(0.0)),
            KernelExpr("add", elem_idx(b, _stack_coeffs(depth, pos, {"k": n, "j": 1})), const(0.0)),
            KernelExpr("mul", temp(0), temp(1))])
        st = KernelNode(op="store", out=c, accum="add",
                        out_index_coeffs=_stack_coeffs(depth, pos, {"i": n, "j": 1}))
        return [km.add_node(cp), km.add_node(st)]

    def k_band(pos, depth):
        if init == "hoist":
            return s0(pos, depth) + _emit_tiled_levels(km, [("k", 0, k - 1, False, False)], s1, tile, depth, pos)
        if init == "guard":
            def body(p, d):
                g = KernelNode(op="guard", guard_coeffs=_stack_coeffs(d, p, {"k": 1}), guard_offset=0,
                               children=s0(p, d))
                return [km.add_node(g)] + s1(p, d)
            return _emit_tiled_levels(km, [("k", 0, k - 1, False, False)], body, tile, depth, pos)
        # split: tile 0 holds the singleton point segment [0,0] with S0 and S1,
        # then [1, min(t,K)-1] with S1; later tiles as the standard parts.
        ids = []
        t0 = km.add_node(KernelNode(op="loop", var="k_t", begin=0, end=1))
        p = dict(pos)
        p["k"] = depth + 1
        seg0 = KernelNode(op="loop", var="k", begin=0, end=1, children=s0(p, depth + 2) + s1(p, depth + 2))
        km.nodes[t0].children.append(km.add_node(seg0))
        hi0 = min(tile, k) - 1
        if hi0 >= 1:
            seg1 = KernelNode(op="loop", var="k", begin=1, end=hi0 + 1, children=s1(p, depth + 2))
            km.nodes[t0].children.append(km.add_node(seg1))
        ids.append(t0)
        if k > tile:
            full_last = k // tile - 1
            if full_last >= 1:
                tf = km.add_node(KernelNode(op="loop", var="k_t", begin=1, end=full_last + 1))
                bc = [0] * (depth + 1)
                bc[depth] = tile
                ec = list(bc)
                pt = KernelNode(op="loop", var="k", begin_coeffs=bc, begin_offset=0, end_coeffs=ec,
                                end_offset=tile - 1, children=s1(p, depth + 2))
                km.nodes[tf].children.append(km.add_node(pt))
                ids.append(tf)
            if k % tile != 0:
                last = (k - 1) // tile
                tp = km.add_node(KernelNode(op="loop", var="k_t", begin=last, end=last + 1))
                bc = [0] * (depth + 1)
                bc[depth] = tile
                pt = KernelNode(op="loop", var="k", begin_coeffs=bc, begin_offset=0, end=k,
                                children=s1(p, depth + 2))
                km.nodes[tp].children.append(km.add_node(pt))
                ids.append(tp)
        return ids

    _emit_tiled_levels(km, [("i", 0, m - 1, True, False), ("j", 0, n - 1, True, True)], k_band, tile)
    return km


def split_gemm_module(m: int, k: int, n: int, dtype_in: str = "f32", out_dtype: str = "f32") -> KernelModule:
    """The untiled scheduled GEMM in the piecewise-split form the reference's
    spec writes out (docs/polyhedral_spec.md:252-267):
    `for i { for k in [0,1) { for j { init; acc } } for k in [1,K) { for j
    { acc } } }`. The k segments are sibling subtrees under i, so j appears
    once per segment (tests/unit/unit_poly.cpp:4279-4286). i and the j loops
    carry the parallel mark; the j loops carry the vector hint."""
    km = KernelModule()
    a = km.add_buffer(KernelBuffer("A", dtype_in, True, False, False, m * k, [m, k]))
    b = km.add_buffer(KernelBuffer("B", dtype_in, True, False, False, k * n, [k, n]))
    c = km.add_buffer(KernelBuffer("C", out_dtype, False, True, False, m * n, [m, n]))
    pos = {"i": 0, "k": 1, "j": 2}

    def init():
        cp = KernelNode(op="compute", exprs=[KernelExpr("add", const(0.0), const(0.0))])
        st = KernelNode(op="store", out=c, out_index_coeffs=_stack_coeffs(3, pos, {"i": n, "j": 1}))
        return [km.add_node(cp), km.add_node(st)]

    def acc():
        cp = KernelNode(op="compute", exprs=[
            KernelExpr("add", elem_idx(a, _stack_coeffs(3, pos, {"i": k, "k": 1})), const(0.0)),
            KernelExpr("add", elem_idx(b, _stack_coeffs(3, pos, {"k": n, "j": 1})), const(0.0)),
            KernelExpr("mul", temp(0), temp(1))])
        st = KernelNode(op="store", out=c, accum="add", out_index_coeffs=_stack_coeffs(3, pos, {"i": n, "j": 1}))
        return [km.add_node(cp), km.add_node(st)]

    segs = []
    for lo, hi, body in ((0, 1, init() + acc()), (1, k, acc())):
        j = km.add_node(KernelNode(op="loop", var="j", begin=0, end=n, parallel=True, vector_hint=True,
                                   children=body))
        segs.append(km.add_node(KernelNode(op="loop", var="k", begin=lo, end=hi, children=[j])))
    km.add_node(KernelNode(op="loop", var="i", begin=0, end=m, parallel=True, children=segs))
    return km
