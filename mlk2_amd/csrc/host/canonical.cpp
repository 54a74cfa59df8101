// Canonical form of multi-dim forests before class recognition: undoes the
// loop shapes poly.codegen emits (polyhedral/src/codegen.cpp) where they are
// exact rewrites of the walker's iteration order
// (runtime/src/execution/kernel_buffers.cpp:453-835), so that a tiled,
// guarded or split band reaches the hand-written class of its untiled form:
//
//   strip-mine merge  T[a,b]{ P[t*T + o, t*T + o + t-1]{body} }
//                     -> P'[t*a + o, t*b + o + t-1]{body}   (also a single
//                     partial tile T[a,a]{ P[t*T + o, E-1] } -> P'[t*a + o, E-1])
//   sibling merge     L[a,b]{B}; L[b+1,c]{B}  -> L[a,c]{B}
//   split peel        L[v,v]{A; B}; L[v+1,e]{B} -> A(v); L[v,e]{B}
//   guard hoist       L[b,e]{ G(v == b){A}; rest } -> A(b); L[b,e]{rest}
//   singleton loop    L[a,a]{body} inside a loop -> body(a)
//
// Stack positions are absolute (coefficient p multiplies the p-th enclosing
// loop variable), so removing a loop level folds that variable's value into
// every affine form below it and shifts the deeper positions down by one.
// A form that was non-empty stays non-empty (an empty coefficient vector means
// "not affine" to the walker), so a folded form keeps a zero coefficient.
#include <algorithm>
#include <string>
#include <vector>

#include "planner.h"

namespace mlk::hip {

namespace {

struct TNode {
    KernelNode n;
    std::vector<TNode> kids;
};

bool buildTree(const KernelModule& km, uint32_t id, TNode& out, int level) {
    if (id >= km.nodes.size() || level > 64) return false;
    out.n = km.nodes[id];
    out.kids.clear();
    for (const uint32_t c : km.nodes[id].children) {
        TNode t;
        if (!buildTree(km, c, t, level + 1)) return false;
        out.kids.push_back(std::move(t));
    }
    out.n.children.clear();
    return true;
}

uint32_t emitTree(KernelModule& out, const TNode& t) {
    std::vector<uint32_t> ids;
    for (const TNode& k : t.kids) ids.push_back(emitTree(out, k));
    KernelNode n = t.n;
    n.children = ids;
    out.nodes.push_back(std::move(n));
    return static_cast<uint32_t>(out.nodes.size() - 1);
}

/// Folds position p = value into one affine form and removes the position.
void foldForm(std::vector<int64_t>& c, int64_t& off, size_t p, int64_t value) {
    if (p >= c.size()) return;
    const bool wasAffine = !c.empty();
    off += c[p] * value;
    c.erase(c.begin() + static_cast<std::ptrdiff_t>(p));
    if (wasAffine && c.empty()) c.push_back(0);
}

bool formUses(const std::vector<int64_t>& c, size_t p) { return p < c.size() && c[p] != 0; }

/// Applies f(coeffs, offset) to every affine form of the subtree.
template <class F>
void forEachForm(TNode& t, F&& f) {
    KernelNode& n = t.n;
    if (!n.beginCoeffs.empty()) f(n.beginCoeffs, n.beginOffset);
    if (!n.endCoeffs.empty()) f(n.endCoeffs, n.endOffset);
    if (!n.outIndexCoeffs.empty()) f(n.outIndexCoeffs, n.outIndexOffset);
    if (!n.guardCoeffs.empty()) f(n.guardCoeffs, n.guardOffset);
    for (KernelExpr& e : n.exprs) {
        for (KernelOperand* o : {&e.a, &e.b}) {
            if (o->kind == KernelOperand::Kind::ElemIdx && !o->idxCoeffs.empty()) f(o->idxCoeffs, o->idxOffset);
        }
    }
    for (TNode& k : t.kids) forEachForm(k, f);
}

void foldPosition(TNode& t, size_t p, int64_t value) {
    forEachForm(t, [&](std::vector<int64_t>& c, int64_t& off) { foldForm(c, off, p, value); });
}

bool usesPosition(TNode& t, size_t p) {
    bool used = false;
    forEachForm(t, [&](std::vector<int64_t>& c, int64_t&) { used = used || formUses(c, p); });
    return used;
}

bool isPlainLoop(const KernelNode& n) { return n.op == KernelOp::Loop && n.step == 1; }

/// Constant inclusive bounds of a loop (no affine forms, no dynamic end).
bool constRange(const KernelNode& n, int64_t& b, int64_t& e) {
    if (!isPlainLoop(n) || !n.beginCoeffs.empty() || !n.endCoeffs.empty() || n.end == kDynamicBound) return false;
    b = n.begin;
    e = n.end - 1;
    return true;
}

void setConstRange(KernelNode& n, int64_t b, int64_t e) {
    n.beginCoeffs.clear();
    n.endCoeffs.clear();
    n.beginOffset = 0;
    n.endOffset = 0;
    n.begin = b;
    n.end = e + 1;
    n.endBuf = kInvalidId;
    n.endDim = -1;
}

bool sameOperand(const KernelOperand& a, const KernelOperand& b) {
    if (a.kind != b.kind) return false;
    switch (a.kind) {
        case KernelOperand::Kind::Const:
            return a.constValue == b.constValue || (a.constValue != a.constValue && b.constValue != b.constValue);
        case KernelOperand::Kind::ScalarParam:
        case KernelOperand::Kind::Temp: return a.index == b.index;
        case KernelOperand::Kind::ElemIdx:
            return a.index == b.index && a.idxCoeffs == b.idxCoeffs && a.idxOffset == b.idxOffset;
        default: return true;
    }
}

bool sameTree(const TNode& x, const TNode& y) {
    const KernelNode& a = x.n;
    const KernelNode& b = y.n;
    if (a.op != b.op || a.math != b.math || a.begin != b.begin || a.end != b.end || a.step != b.step ||
        a.beginCoeffs != b.beginCoeffs || a.beginOffset != b.beginOffset || a.endCoeffs != b.endCoeffs ||
        a.endOffset != b.endOffset || a.endBuf != b.endBuf || a.endDim != b.endDim || a.bufferA != b.bufferA ||
        a.bufferB != b.bufferB || a.bufferOut != b.bufferOut || a.outIndexCoeffs != b.outIndexCoeffs ||
        a.outIndexOffset != b.outIndexOffset || a.accum != b.accum || a.guardCoeffs != b.guardCoeffs ||
        a.guardOffset != b.guardOffset || a.family != b.family || a.exprs.size() != b.exprs.size() ||
        x.kids.size() != y.kids.size()) {
        return false;
    }
    for (size_t i = 0; i < a.exprs.size(); ++i) {
        if (a.exprs[i].op != b.exprs[i].op || !sameOperand(a.exprs[i].a, b.exprs[i].a) ||
            !sameOperand(a.exprs[i].b, b.exprs[i].b)) {
            return false;
        }
    }
    for (size_t i = 0; i < x.kids.size(); ++i) {
        if (!sameTree(x.kids[i], y.kids[i])) return false;
    }
    return true;
}

bool sameList(const std::vector<TNode>& a, size_t a0, const std::vector<TNode>& b) {
    if (a.size() - a0 != b.size()) return false;
    for (size_t i = 0; i < b.size(); ++i) {
        if (!sameTree(a[a0 + i], b[i])) return false;
    }
    return true;
}

/// Strip-mine merge of a tile loop T at position p with its single point child.
bool mergeStripMine(TNode& t, size_t p) {
    int64_t a = 0, b = 0;
    if (!constRange(t.n, a, b) || b < a || t.kids.size() != 1) return false;
    TNode& pt = t.kids[0];
    const KernelNode& P = pt.n;
    if (!isPlainLoop(P) || P.beginCoeffs.size() != p + 1) return false;
    const int64_t tile = P.beginCoeffs[p];
    for (size_t q = 0; q < p; ++q) {
        if (P.beginCoeffs[q] != 0) return false;
    }
    if (tile <= 0) return false;
    int64_t lo = 0, hi = 0;
    if (!P.endCoeffs.empty()) {
        if (P.endCoeffs.size() != p + 1 || P.endCoeffs[p] != tile) return false;
        for (size_t q = 0; q < p; ++q) {
            if (P.endCoeffs[q] != 0) return false;
        }
        if (P.endOffset - P.beginOffset + 1 != tile) return false;  // consecutive tiles, no gap or overlap
        lo = tile * a + P.beginOffset;
        hi = tile * b + P.endOffset;
    } else {
        if (a != b || P.end == kDynamicBound) return false;  // constant end: only a single partial tile
        lo = tile * a + P.beginOffset;
        hi = P.end - 1;
        if (hi < lo) return false;
    }
    // The point body must not read the tile variable.
    for (TNode& k : pt.kids) {
        if (usesPosition(k, p)) return false;
    }
    TNode merged;
    merged.n = P;
    setConstRange(merged.n, lo, hi);
    merged.n.parallel = P.parallel && t.n.parallel;
    merged.kids = std::move(pt.kids);
    for (TNode& k : merged.kids) foldPosition(k, p, 0);  // removes position p (unused)
    t = std::move(merged);
    return true;
}

bool allPairsOrTrees(const std::vector<TNode>& v) {
    // Anything may be hoisted except a Store separated from its Compute.
    for (size_t i = 0; i < v.size(); ++i) {
        if (v[i].n.op == KernelOp::Compute) {
            if (i + 1 < v.size() && v[i + 1].n.op == KernelOp::Store) ++i;
            continue;
        }
        if (v[i].n.op == KernelOp::Store) return false;
    }
    return true;
}

/// One pass over a child list at stack depth `depth` (the list's nodes see
/// positions [0, depth)); `inLoop` when the list is a loop body.
bool canonList(std::vector<TNode>& list, size_t depth, bool inLoop, int budget);

bool canonNode(TNode& t, size_t depth, int budget) {
    bool changed = false;
    if (t.n.op == KernelOp::Loop) {
        changed = canonList(t.kids, depth + 1, true, budget) || changed;
        for (int i = 0; i < 8 && mergeStripMine(t, depth); ++i) {
            changed = true;
            canonList(t.kids, depth + 1, true, budget);
        }
    } else if (t.n.op == KernelOp::Guard) {
        changed = canonList(t.kids, depth, false, budget) || changed;
    }
    return changed;
}

bool canonList(std::vector<TNode>& list, size_t depth, bool inLoop, int budget) {
    if (budget <= 0) return false;
    bool changed = false;
    for (TNode& t : list) changed = canonNode(t, depth, budget - 1) || changed;
    for (bool again = true; again;) {
        again = false;
        for (size_t i = 0; i < list.size() && !again; ++i) {
            TNode& L = list[i];
            int64_t a = 0, b = 0;
            if (!constRange(L.n, a, b) || b < a) continue;
            // Sibling merge: L[a,b]{B}; L[b+1,c]{B}.
            if (i + 1 < list.size()) {
                TNode& M = list[i + 1];
                int64_t c0 = 0, c1 = 0;
                if (constRange(M.n, c0, c1) && c1 >= c0 && c0 == b + 1 && sameList(L.kids, 0, M.kids)) {
                    setConstRange(L.n, a, c1);
                    L.n.parallel = L.n.parallel && M.n.parallel;
                    list.erase(list.begin() + static_cast<std::ptrdiff_t>(i) + 1);
                    again = changed = true;
                    break;
                }
            }
            if (!inLoop) continue;  // hoisted statements must stay inside a loop
            // Split peel: L[v,v]{A; B}; L[v+1,e]{B}  ->  A(v); L[v,e]{B}.
            if (a == b && i + 1 < list.size()) {
                TNode& M = list[i + 1];
                int64_t c0 = 0, c1 = 0;
                if (constRange(M.n, c0, c1) && c1 >= c0 && c0 == a + 1 && M.kids.size() < L.kids.size()) {
                    const size_t na = L.kids.size() - M.kids.size();
                    std::vector<TNode> A(L.kids.begin(), L.kids.begin() + static_cast<std::ptrdiff_t>(na));
                    if (sameList(L.kids, na, M.kids) && allPairsOrTrees(A)) {
                        for (TNode& x : A) foldPosition(x, depth, a);
                        setConstRange(M.n, a, c1);
                        M.n.parallel = M.n.parallel && L.n.parallel;
                        list.erase(list.begin() + static_cast<std::ptrdiff_t>(i));
                        list.insert(list.begin() + static_cast<std::ptrdiff_t>(i), A.begin(), A.end());
                        again = changed = true;
                        break;
                    }
                }
            }
            // Guard hoist: L[b,e]{ G(v == b){A}; rest }  ->  A(b); L[b,e]{rest}.
            if (!L.kids.empty() && L.kids[0].n.op == KernelOp::Guard) {
                const KernelNode& G = L.kids[0].n;
                bool onlyThis = G.guardCoeffs.size() == depth + 1 && (G.guardCoeffs[depth] == 1 || G.guardCoeffs[depth] == -1);
                for (size_t q = 0; onlyThis && q < depth; ++q) onlyThis = G.guardCoeffs[q] == 0;
                if (onlyThis && G.guardCoeffs[depth] * a + G.guardOffset == 0 && allPairsOrTrees(L.kids[0].kids)) {
                    std::vector<TNode> A = std::move(L.kids[0].kids);
                    for (TNode& x : A) foldPosition(x, depth, a);
                    L.kids.erase(L.kids.begin());
                    list.insert(list.begin() + static_cast<std::ptrdiff_t>(i), A.begin(), A.end());
                    again = changed = true;
                    break;
                }
            }
            // Singleton loop inside a loop: body(a). A singleton level of a
            // perfect nest (one loop child, or one Compute+Store pair) stays,
            // so the nest keeps the shape of its class.
            const bool perfectLevel = L.kids.size() == 1 ||
                                      (L.kids.size() == 2 && L.kids[0].n.op == KernelOp::Compute &&
                                       L.kids[1].n.op == KernelOp::Store);
            if (a == b && !perfectLevel && allPairsOrTrees(L.kids)) {
                std::vector<TNode> body = std::move(L.kids);
                for (TNode& x : body) foldPosition(x, depth, a);
                list.erase(list.begin() + static_cast<std::ptrdiff_t>(i));
                list.insert(list.begin() + static_cast<std::ptrdiff_t>(i), body.begin(), body.end());
                again = changed = true;
                break;
            }
        }
        if (again) {
            for (TNode& t : list) canonNode(t, depth, budget - 1);
        }
    }
    return changed;
}

}  // namespace

KernelModule canonicalModule(const KernelModule& km, int* rewrites) {
    if (rewrites != nullptr) *rewrites = 0;
    const std::vector<uint32_t> roots = forestRoots(km);
    std::vector<TNode> trees;
    for (const uint32_t r : roots) {
        TNode t;
        if (!buildTree(km, r, t, 0)) return km;
        trees.push_back(std::move(t));
    }
    bool changed = false;
    for (TNode& t : trees) {
        // Roots run with an empty variable stack; only loops nest further.
        if (t.n.op == KernelOp::Loop || t.n.op == KernelOp::Guard) changed = canonNode(t, 0, 64) || changed;
    }
    // Root-level strip-mined bands, and root loops split into adjacent parts.
    std::vector<TNode> top = std::move(trees);
    changed = canonList(top, 0, false, 64) || changed;
    if (!changed) return km;
    KernelModule out;
    out.buffers = km.buffers;
    out.name = km.name;
    out.schedule = km.schedule;
    for (const TNode& t : top) emitTree(out, t);
    if (rewrites != nullptr) *rewrites = 1;
    return out;
}

}  // namespace mlk::hip
