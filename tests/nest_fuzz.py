"""Seeded random Kernel IR loop nests for the generic loop-nest path.

Each module is 1-3 forest roots of Loop / Guard / Compute+Store nodes with
constant, affine (including triangular) and buffer-dim loop bounds, equality
guards, chains of IEEE operations over ElemIdx / Const / ScalarParam / Temp
operands, and `=`, `+=` and max stores into outputs and temps. Addresses are
affine in the enclosing loop variables with small coefficients; every buffer is
sized so the walker's accesses stay in bounds (offsets are shifted so that the
smallest address is 0). No loop is marked parallel: which loops run on threads
is left to the backend's own proof, so a wrong proof shows up as a mismatch
against the oracle when the grid runs in another order.
"""
from __future__ import annotations

from typing import List, Tuple

import numpy as np

from mlk2_amd.kernel_ir import (KernelBuffer, KernelExpr, KernelModule, KernelNode,
                                const, elem_idx, scalar, temp)

BINARY = ["add", "sub", "mul", "div"]
UNARY = ["neg"]
# With exact_ops=False the chains also draw the device-libm operations and
# the guarded ones (kernel_buffers.cpp:130-160).
TRANS_BINARY = ["pow"]
TRANS_UNARY = ["exp", "log", "sin", "cos", "tan", "tanh", "sqrt", "rsqrt", "erf", "gelu"]


class _Gen:
    def __init__(self, seed: int, exact_ops: bool = True):
        self.rng = np.random.default_rng(seed)
        self.km = KernelModule(name=f"fuzz_{seed}")
        self.accesses: List[Tuple[int, list, list]] = []  # (buffer, coeffs, ranges) per access
        self.pending = []   # (node, field) whose offset is fixed after sizing
        # 2 inputs, 2 outputs, 1 temp; sizes set at the end.
        for name, inp, out, tmp in (("x0", 1, 0, 0), ("x1", 1, 0, 0), ("y0", 0, 1, 0), ("y1", 0, 1, 0),
                                    ("t0", 0, 0, 1)):
            self.km.add_buffer(KernelBuffer(name, "f64", bool(inp), bool(out), bool(tmp), 1, [1]))
        self.readable = [0, 1, 2, 3, 4]
        self.writable = [2, 3, 4]
        self.exact_ops = exact_ops

    def ri(self, lo, hi):
        return int(self.rng.integers(lo, hi + 1))

    def access(self, ranges):
        """Coefficients over the current stack; the offset is chosen so the
        smallest address over the ranges is 0..2."""
        depth = len(ranges)
        coeffs = [self.ri(-2, 3) if self.rng.random() < 0.7 else 0 for _ in range(depth)]
        lo = sum(min(c * r[0], c * r[1]) for c, r in zip(coeffs, ranges))
        off = -lo + self.ri(0, 2)
        return coeffs, off

    def operand(self, ranges, k):
        u = self.rng.random()
        if u < 0.55:
            b = int(self.rng.choice(self.readable))
            coeffs, off = self.access(ranges)
            self.accesses.append((b, coeffs, off, [tuple(r) for r in ranges]))
            return elem_idx(b, coeffs, off)
        if u < 0.7 and k > 0:
            return temp(self.ri(0, k - 1))
        if u < 0.8:
            return scalar(self.ri(0, 2))
        return const(float(self.rng.choice([0.0, 1.0, -0.5, 2.0, 3.25, -1.0])))

    def pair(self, ranges):
        n = self.ri(1, 3)
        exprs = []
        unary = UNARY if self.exact_ops else UNARY + TRANS_UNARY
        binary = BINARY if self.exact_ops else BINARY + TRANS_BINARY
        p_unary = 0.15 if self.exact_ops else 0.45
        for k in range(n):
            if self.rng.random() < p_unary:
                exprs.append(KernelExpr(str(self.rng.choice(unary)), self.operand(ranges, k), const(0.0)))
            else:
                exprs.append(KernelExpr(str(self.rng.choice(binary)), self.operand(ranges, k),
                                        self.operand(ranges, k)))
        c = self.km.add_node(KernelNode(op="compute", math=exprs[-1].op, exprs=exprs))
        b = int(self.rng.choice(self.writable))
        coeffs, off = self.access(ranges)
        self.accesses.append((b, coeffs, off, [tuple(r) for r in ranges]))
        acc = str(self.rng.choice(["none", "none", "add", "max"]))
        if not coeffs:
            coeffs = []
        s = self.km.add_node(KernelNode(op="store", out=b, out_index_coeffs=coeffs or [0],
                                        out_index_offset=off, accum=acc))
        return [c, s]

    def loop(self, ranges, depth):
        d = len(ranges)
        form = self.rng.random()
        node = KernelNode(op="loop", var=f"v{d}")
        if d > 0 and form < 0.35:
            # Affine: begin = b0 + c*v_p, inclusive end = begin + L - 1 (or v_p: triangular).
            p = self.ri(0, d - 1)
            c = self.ri(0, 1)
            b0 = self.ri(0, 1)
            bc = [0] * d
            bc[p] = c
            node.begin_coeffs, node.begin_offset = bc, b0
            if self.rng.random() < 0.5:
                ln = self.ri(0, 5)
                node.end_coeffs, node.end_offset = list(bc), b0 + ln - 1
                lo = b0 + c * ranges[p][0]
                hi = b0 + c * ranges[p][1] + ln - 1
            else:
                ec = [0] * d
                ec[p] = 1
                node.end_coeffs, node.end_offset = ec, self.ri(0, 1)
                lo = b0 + c * ranges[p][0]
                hi = ranges[p][1] + node.end_offset
        else:
            b = self.ri(0, 2)
            ln = self.ri(0, 7)
            node.begin, node.end = b, b + ln
            lo, hi = b, b + ln - 1
        if hi < lo:
            hi = lo  # the loop may be empty; ranges stay well-formed
        node.children = self.body(ranges + [(lo, hi)], depth + 1)
        return self.km.add_node(node)

    def guard(self, ranges, depth):
        d = len(ranges)
        p = self.ri(0, d - 1)
        c = int(self.rng.choice([1, -1]))
        v = self.ri(ranges[p][0], ranges[p][1])
        gc = [0] * d
        gc[p] = c
        node = KernelNode(op="guard", guard_coeffs=gc, guard_offset=-c * v)
        node.children = self.body(ranges, depth + 1)
        return self.km.add_node(node)

    def body(self, ranges, depth):
        out = []
        for _ in range(self.ri(1, 3)):
            u = self.rng.random()
            if depth < 4 and u < 0.4:
                out.append(self.loop(ranges, depth))
            elif ranges and depth < 6 and u < 0.5:
                out.append(self.guard(ranges, depth))
            else:
                out.extend(self.pair(ranges))
        return out

    def finish(self):
        size = {b: 1 for b in range(5)}
        for b, coeffs, off, ranges in self.accesses:
            hi = off + sum(max(c * r[0], c * r[1]) for c, r in zip(coeffs, ranges))
            size[b] = max(size[b], hi + 1)
        for b, kb in enumerate(self.km.buffers):
            kb.elements = size[b]
            kb.dims = [size[b]]
        return self.km


def random_module(seed: int, exact_ops: bool = True) -> KernelModule:
    g = _Gen(seed, exact_ops)
    for _ in range(g.ri(1, 3)):
        g.loop([], 0)
    return g.finish()


def random_inputs(km: KernelModule, seed: int):
    rng = np.random.default_rng(seed + 1000)
    arrays = {}
    for i, b in enumerate(km.buffers):
        if b.is_input or b.is_output:
            arrays[i] = rng.integers(-8, 9, b.elements).astype(np.float64) / 4.0
    scalars = [float(v) for v in rng.integers(-4, 5, 3) / 2.0]
    return arrays, scalars


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    """Bit-identical, except that any NaN matches any NaN."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.shape != b.shape:
        return False
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    return np.array_equal(a[~na].view(np.uint64), b[~nb].view(np.uint64))


def _insert_position(km: KernelModule, nid: int, p: int) -> None:
    """Shifts stack positions >= p of every affine form in the subtree up by
    one (a new loop level at position p encloses it)."""
    n = km.nodes[nid]

    def ins(c):
        return c[:p] + [0] + c[p:] if len(c) > p else c

    if n.begin_coeffs or n.end_coeffs:
        if n.begin_coeffs:
            n.begin_coeffs = ins(n.begin_coeffs)
        if n.end_coeffs:
            n.end_coeffs = ins(n.end_coeffs)
    if n.out_index_coeffs:
        n.out_index_coeffs = ins(n.out_index_coeffs)
    if n.guard_coeffs:
        n.guard_coeffs = ins(n.guard_coeffs)
    for e in n.exprs:
        for o in (e.a, e.b):
            if o.kind == "elem_idx" and o.coeffs:
                o.coeffs = ins(o.coeffs)
    for c in n.children:
        _insert_position(km, c, p)


def _copy_subtree(km: KernelModule, nid: int) -> int:
    import copy
    n = copy.deepcopy(km.nodes[nid])
    n.children = [_copy_subtree(km, c) for c in n.children]
    return km.add_node(n)


def _tile(km: KernelModule, nid: int, depth: int, t: int) -> List[int]:
    """Replaces loop `nid` (stack position `depth`, constant bounds, begin a
    multiple of t) by poly codegen's tile parts; returns the new node ids."""
    n = km.nodes[nid]
    lo, hi = n.begin, n.end - 1
    first, full_last, last = lo // t, (hi + 1) // t - 1, hi // t
    parts = []
    if full_last >= first:
        parts.append(("full", first, full_last))
    if (hi + 1) % t != 0:
        parts.append(("partial", last, last))
    out = []
    for kind, t0, t1 in parts:
        kids = [_copy_subtree(km, c) for c in n.children]
        for c in kids:
            _insert_position(km, c, depth)
        bc = [0] * (depth + 1)
        bc[depth] = t
        point = KernelNode(op="loop", var=(n.var or "v"), begin_coeffs=bc, begin_offset=0, children=kids)
        if kind == "full":
            point.end_coeffs, point.end_offset = list(bc), t - 1
        else:
            point.end = hi + 1
        pid = km.add_node(point)
        out.append(km.add_node(KernelNode(op="loop", var=(n.var or "v") + "_t", begin=t0, end=t1 + 1,
                                          children=[pid])))
    return out


def tiled_random_module(seed: int) -> KernelModule:
    """random_module(seed) with some constant-bound loops strip-mined the way
    poly codegen tiles a band (full tiles with affine point bounds, a partial
    tile with a constant end), nested tiles included."""
    km = random_module(seed)
    rng = np.random.default_rng(seed + 7)

    def visit(ids: List[int], depth: int) -> List[int]:
        out = []
        for nid in ids:
            n = km.nodes[nid]
            if n.op == "loop":
                n.children = visit(n.children, depth + 1)
                const = not n.begin_coeffs and not n.end_coeffs and n.end >= 0
                if const and n.end - n.begin >= 2 and rng.random() < 0.6:
                    t = int(rng.choice([1, 2, 3]))
                    if n.begin % t == 0:
                        out.extend(_tile(km, nid, depth, t))
                        continue
            elif n.op == "guard":
                n.children = visit(n.children, depth)
            out.append(nid)
        return out

    roots = km.roots()
    new_roots = visit(roots, 0)
    # Rebuild so the roots run in their original order.
    out = KernelModule(buffers=km.buffers, name=km.name, schedule=dict(km.schedule))

    def emit(nid: int) -> int:
        import copy
        n = copy.deepcopy(km.nodes[nid])
        n.children = [emit(c) for c in n.children]
        return out.add_node(n)

    for r in new_roots:
        emit(r)
    return out
