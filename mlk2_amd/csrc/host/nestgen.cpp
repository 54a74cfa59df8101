// Generic loop-nest class: any multi-dim forest root built from Loop,
// Compute, Store and Guard nodes that no hand-written class claims runs as one
// hipRTC kernel with the reference walker's semantics
// (runtime/src/execution/kernel_buffers.cpp:453-835): inclusive affine loop
// bounds over the enclosing variable stack (:579-601), a Compute paired with
// the immediately next Store (:715-779), `=` / `+=` / max stores, equality
// guards, chains evaluated in f64. It takes the place of the reference's CUDA
// emitter (backends/cpu/src/cuda_emitter.cpp:631-1128): the outermost chain of
// parallel unit-step loops, each with a single loop child, is collapsed onto
// threads over padded trip counts and the rest of the subtree runs serially in
// each thread.
//
// Choices made for gfx950 rather than taken from that emitter:
//   * Trip counts are padded by interval arithmetic over the enclosing chain
//     variables and decomposed innermost-fastest, so the 64 lanes of a wave
//     walk 64 consecutive innermost iterations (one coalesced span for
//     row-major buffers). The grid is capped and strides over the instances.
//   * A loop without the `parallel` mark joins the chain when the host proves
//     it parallel: every buffer its subtree writes is addressed, by every
//     access of the subtree, with one common nonzero coefficient c on the loop
//     variable and identical coefficients on the enclosing ones, and all those
//     accesses stay, for one iteration, inside a window narrower than |c|.
//     Iterations then touch disjoint elements of every written buffer.
//   * An invariant-address accumulation lives in an f64 register: when every
//     access to a buffer inside a loop (or inside a thread's body) is a store
//     to one address that does not move with the inner loops, and one of those
//     stores runs whenever the region runs, the register takes the slot's
//     value on entry and writes it back once on exit. The register sees the
//     same f64 sequence the walker's slot sees; a narrow buffer is rounded
//     once instead of once per step.
//   * Every access is bounded on the host by interval arithmetic. Only an
//     access it cannot bound carries a run-time check, which reports through a
//     status word (1 = negative store address, the walker's InvalidGraph;
//     6 = outside a bound buffer) instead of touching memory out of bounds.
//   * LDS slabs, the counterpart of the reference's shared-memory slabs
//     (backends/cpu/src/slab_plan.cpp, contract in slab_plan.h:1-45): an input
//     that no Store of the module targets, whose every read in the root is
//     proven in bounds, is copied once per workgroup into LDS as the interval
//     hull of those reads, and the reads are redirected there. The copy holds
//     the buffer's own bits, so values and their order are unchanged. Unlike
//     the reference, which stages whenever the hull fits, a slab is taken only
//     when each workgroup is expected to read each staged element at least
//     twice, so the copy cannot cost more than the reads it replaces; slabs
//     share a 64 KiB budget per workgroup (two workgroups per CU).
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "planner.h"

namespace mlk::hip {

namespace {

using K = KernelOperand::Kind;

constexpr int kMaxSlots = 16;        // buffers one nest kernel binds (mlkd_nest_args)
constexpr int kMaxDepth = 32;        // loop nesting depth
constexpr int kMaxChain = 8;         // collapsed loops
constexpr int kMaxNodesVisited = 1 << 16;
constexpr __int128 kIndexLimit = static_cast<__int128>(1) << 62;
constexpr int64_t kMaxInstances = int64_t{1} << 40;
constexpr int64_t kSlabBudget = 64 * 1024;   // LDS bytes of slabs per workgroup
constexpr int64_t kSlabReuse = 2;            // reads per staged element per workgroup

/// Inclusive range of one loop variable; `unbounded` when it depends on the
/// run's element count (a dynamic loop end) and so is not known at build.
struct Range {
    int64_t lo{0}, hi{0};
    bool unbounded{false};
    bool steers{false};   // appears in the bounds of a deeper loop on the current path
};

/// off + sum c[p] * v[p] over stack positions p < min(|c|, depth).
struct Affine {
    std::vector<int64_t> c;
    int64_t off{0};
};

std::string intLit(int64_t v) {
    if (v == INT64_MIN) return "(-9223372036854775807LL - 1)";
    return std::to_string(v) + "LL";
}

int dtypeCode(Dtype d) { return d == Dtype::F32 ? 0 : (d == Dtype::F16 ? 1 : 2); }

int64_t coeffAt(const Affine& a, size_t p) { return p < a.c.size() ? a.c[p] : 0; }

/// [lo, hi] of `a` over the ranges of positions [0, depth). False when a term
/// leaves the +-2^62 index budget (the module is refused).
bool bound(const Affine& a, const std::vector<Range>& r, size_t depth, int64_t& lo, int64_t& hi,
           bool& unbounded) {
    __int128 L = a.off, H = a.off;
    unbounded = false;
    const size_t n = std::min({a.c.size(), r.size(), depth});
    for (size_t p = 0; p < n; ++p) {
        const int64_t c = a.c[p];
        if (c == 0) continue;
        if (r[p].unbounded) {
            unbounded = true;
            continue;
        }
        const __int128 x = static_cast<__int128>(c) * r[p].lo;
        const __int128 y = static_cast<__int128>(c) * r[p].hi;
        L += x < y ? x : y;
        H += x < y ? y : x;
        if (L < -kIndexLimit || H > kIndexLimit) return false;
    }
    if (L < -kIndexLimit || H > kIndexLimit) return false;
    lo = static_cast<int64_t>(L);
    hi = static_cast<int64_t>(H);
    return true;
}

std::string affineCode(const Affine& a, size_t depth) {
    std::string s = "(" + intLit(a.off);
    const size_t n = std::min(a.c.size(), depth);
    for (size_t p = 0; p < n; ++p) {
        if (a.c[p] == 0) continue;
        s += " + " + intLit(a.c[p]) + " * v" + std::to_string(p);
    }
    return s + ")";
}

/// Loop bounds as the walker reads them (:579-601): affine begin, affine
/// inclusive end, dims[endDim] of a buffer, the run's element count, or the
/// constant exclusive end.
struct LoopBounds {
    Affine begin;
    Affine endInc;
    bool dynamicEnd{false};
};

LoopBounds loopBounds(const KernelModule& km, const KernelNode& n) {
    LoopBounds b;
    if (!n.beginCoeffs.empty()) {
        b.begin.c = n.beginCoeffs;
        b.begin.off = n.beginOffset;
    } else {
        b.begin.off = n.begin;
    }
    if (!n.endCoeffs.empty()) {
        b.endInc.c = n.endCoeffs;
        b.endInc.off = n.endOffset;
    } else if (n.end == kDynamicBound && n.endBuf != kInvalidId && n.endBuf < km.buffers.size() &&
               n.endDim >= 0 && n.endDim < static_cast<int32_t>(km.buffers[n.endBuf].dims.size())) {
        b.endInc.off = km.buffers[n.endBuf].dims[static_cast<size_t>(n.endDim)] - 1;
    } else if (n.end == kDynamicBound) {
        b.dynamicEnd = true;
    } else {
        b.endInc.off = n.end - 1;
    }
    return b;
}

/// One read or write the host saw while walking a region.
struct Access {
    uint32_t buf{kInvalidId};
    bool store{false};
    AccumMode accum{AccumMode::None};
    Affine at;                 // coefficients trimmed to the access depth
    size_t depth{0};
    std::vector<Range> ranges; // positions [0, depth)
    bool definite{false};      // runs whenever the region runs
};

struct Ctx {
    const KernelModule& km;
    bool failed{false};
    ErrorCode code{ErrorCode::UnsupportedCapability};
    std::string why;
    int visited{0};

    void fail(ErrorCode c, const std::string& w) {
        if (failed) return;
        failed = true;
        code = c;
        why = w;
    }
    bool bindable(uint32_t b) const {
        return b < km.buffers.size() &&
               (km.buffers[b].isInput || km.buffers[b].isOutput || km.buffers[b].isTemp);
    }
    int64_t staticElems(uint32_t b) const { return bufferElements(km.buffers[b], -1); }
};

/// Variable range of a loop under the enclosing ranges. `dead`: the loop never
/// runs; `nonEmpty`: it runs at least once whenever it is reached.
bool loopRange(Ctx& cx, const LoopBounds& lb, const std::vector<Range>& r, Range& out, bool& dead,
               bool& nonEmpty) {
    int64_t bl = 0, bh = 0, el = 0, eh = 0;
    bool bu = false, eu = false;
    if (!bound(lb.begin, r, r.size(), bl, bh, bu)) {
        cx.fail(ErrorCode::UnsupportedCapability, "loop bound outside the index budget");
        return false;
    }
    if (lb.dynamicEnd) {
        eu = true;
    } else if (!bound(lb.endInc, r, r.size(), el, eh, eu)) {
        cx.fail(ErrorCode::UnsupportedCapability, "loop bound outside the index budget");
        return false;
    }
    out.unbounded = bu || eu;
    out.lo = bl;
    out.hi = eh;
    dead = !out.unbounded && eh < bl;
    nonEmpty = false;
    if (!lb.dynamicEnd && !out.unbounded) {
        Affine diff;
        const size_t n = std::max(lb.begin.c.size(), lb.endInc.c.size());
        diff.c.assign(n, 0);
        for (size_t p = 0; p < n; ++p) diff.c[p] = coeffAt(lb.endInc, p) - coeffAt(lb.begin, p);
        diff.off = lb.endInc.off - lb.begin.off;
        int64_t dl = 0, dh = 0;
        bool du = false;
        if (bound(diff, r, r.size(), dl, dh, du) && !du) nonEmpty = dl >= 0;
    }
    return true;
}

/// Guard refinement (the walker runs the children when off + sum c*v == 0,
/// :808-820). Returns false when the guard can never pass.
bool refineGuard(Ctx& cx, const KernelNode& g, std::vector<Range>& r, bool& constTrue) {
    constTrue = false;
    int nz = 0;
    size_t pos = 0;
    int64_t coef = 0;
    for (size_t p = 0; p < g.guardCoeffs.size(); ++p) {
        if (g.guardCoeffs[p] == 0) continue;
        if (p >= r.size()) {
            cx.fail(ErrorCode::InvalidGraph, "walker: guard references an unbound loop var");
            return false;
        }
        ++nz;
        pos = p;
        coef = g.guardCoeffs[p];
    }
    if (nz == 0) {
        constTrue = g.guardOffset == 0;
        return constTrue;
    }
    if (nz > 1) return true;
    if ((-static_cast<__int128>(g.guardOffset)) % coef != 0) return false;
    const int64_t v = static_cast<int64_t>(-static_cast<__int128>(g.guardOffset) / coef);
    if (!r[pos].unbounded && (v < r[pos].lo || v > r[pos].hi)) return false;
    r[pos].lo = r[pos].hi = v;
    r[pos].unbounded = false;
    return true;
}

Affine trimmed(const std::vector<int64_t>& c, int64_t off, size_t depth) {
    Affine a;
    a.c.assign(c.begin(), c.begin() + static_cast<std::ptrdiff_t>(std::min(c.size(), depth)));
    a.off = off;
    return a;
}

bool hasLegacyOperand(const KernelNode& cp) {
    for (const KernelExpr& e : cp.exprs) {
        for (const KernelOperand* o : {&e.a, &e.b}) {
            if (o->kind == K::ElemA || o->kind == K::ElemB) return true;
        }
    }
    return false;
}

/// Collects the accesses of a child list (the walker's pairing rule).
void collect(Ctx& cx, const std::vector<uint32_t>& children, std::vector<Range>& r, bool definite,
             std::vector<Access>& out, int level) {
    if (cx.failed) return;
    if (level > kMaxDepth || ++cx.visited > kMaxNodesVisited) {
        cx.fail(ErrorCode::UnsupportedCapability, "loop nest deeper or larger than the generic path takes");
        return;
    }
    const KernelModule& km = cx.km;
    for (size_t ci = 0; ci < children.size() && !cx.failed; ++ci) {
        const uint32_t id = children[ci];
        if (id >= km.nodes.size()) {
            cx.fail(ErrorCode::InvalidGraph, "walker: child id out of range");
            return;
        }
        const KernelNode& n = km.nodes[id];
        if (n.op == KernelOp::Compute) {
            if (ci + 1 >= children.size() || children[ci + 1] >= km.nodes.size() ||
                km.nodes[children[ci + 1]].op != KernelOp::Store) {
                continue;  // unpaired Compute: nothing executes
            }
            const KernelNode& so = km.nodes[children[++ci]];
            for (const KernelExpr& e : n.exprs) {
                for (const KernelOperand* o : {&e.a, &e.b}) {
                    if (o == &e.b && isUnaryMath(e.op)) continue;
                    if (o->kind != K::ElemIdx) continue;
                    if (o->index < 0 || static_cast<size_t>(o->index) >= km.buffers.size()) continue;
                    Access a;
                    a.buf = static_cast<uint32_t>(o->index);
                    a.at = trimmed(o->idxCoeffs, o->idxOffset, r.size());
                    a.depth = r.size();
                    a.ranges = r;
                    a.definite = definite;
                    out.push_back(std::move(a));
                }
            }
            Access s;
            s.buf = so.bufferOut;
            s.store = true;
            s.accum = so.accum;
            s.at = trimmed(so.outIndexCoeffs, so.outIndexOffset, r.size());
            s.depth = r.size();
            s.ranges = r;
            s.definite = definite;
            out.push_back(std::move(s));
            continue;
        }
        if (n.op == KernelOp::Loop) {
            if (r.size() >= static_cast<size_t>(kMaxDepth)) {
                cx.fail(ErrorCode::UnsupportedCapability, "loop nest deeper than the generic path takes");
                return;
            }
            const LoopBounds lb = loopBounds(km, n);
            Range vr;
            bool dead = false, nonEmpty = false;
            if (!loopRange(cx, lb, r, vr, dead, nonEmpty)) return;
            if (dead) continue;
            std::vector<size_t> marked;
            for (size_t p = 0; p < r.size(); ++p) {
                if (!r[p].steers && (coeffAt(lb.begin, p) != 0 || coeffAt(lb.endInc, p) != 0)) {
                    r[p].steers = true;
                    marked.push_back(p);
                }
            }
            r.push_back(vr);
            collect(cx, n.children, r, definite && nonEmpty, out, level + 1);
            r.pop_back();
            for (const size_t p : marked) r[p].steers = false;
            continue;
        }
        if (n.op == KernelOp::Guard) {
            if (n.guardCoeffs.empty()) continue;
            std::vector<Range> rr = r;
            bool constTrue = false;
            if (!refineGuard(cx, n, rr, constTrue)) continue;
            collect(cx, n.children, rr, definite && constTrue, out, level + 1);
            continue;
        }
        if (n.op == KernelOp::Call) {
            cx.fail(ErrorCode::UnsupportedCapability, "Call inside a loop nest");
            return;
        }
    }
}

/// Host proof that the loop at stack position d (range `self`) may run its
/// iterations in any order on different threads.
bool provablyParallel(Ctx& cx, const KernelNode& loop, std::vector<Range>& r, const Range& self) {
    if (self.unbounded) return false;
    const size_t d = r.size();
    std::vector<Access> acc;
    r.push_back(self);
    collect(cx, loop.children, r, true, acc, 1);
    r.pop_back();
    if (cx.failed) return false;
    std::vector<uint32_t> written;
    for (const Access& a : acc) {
        if (a.store && std::find(written.begin(), written.end(), a.buf) == written.end()) written.push_back(a.buf);
    }
    for (const uint32_t w : written) {
        const Access* first = nullptr;
        __int128 lo = 0, hi = 0;
        for (const Access& a : acc) {
            if (a.buf != w) continue;
            if (first == nullptr) first = &a;
            const int64_t c = coeffAt(a.at, d);
            if (c == 0 || c != coeffAt(first->at, d)) return false;
            for (size_t p = 0; p < d; ++p) {
                if (coeffAt(a.at, p) != coeffAt(first->at, p)) return false;
            }
            Affine inner;
            inner.off = a.at.off;
            inner.c.assign(a.depth, 0);
            for (size_t p = d + 1; p < a.depth; ++p) inner.c[p] = coeffAt(a.at, p);
            int64_t l = 0, h = 0;
            bool u = false;
            if (!bound(inner, a.ranges, a.depth, l, h, u) || u) return false;
            if (&a == first) {
                lo = l;
                hi = h;
            } else {
                lo = std::min<__int128>(lo, l);
                hi = std::max<__int128>(hi, h);
            }
        }
        const __int128 c = coeffAt(first->at, d);
        if (hi - lo >= (c < 0 ? -c : c)) return false;
    }
    return true;
}

/// One LDS slab: elements [lo, lo + span) of buffer `buf`.
struct Slab {
    uint32_t buf{kInvalidId};
    int64_t lo{0}, span{0};
};

/// Slabs for the root (buffer-id order), given the workgroups of its launch.
/// Planning never fails the nest: anything it cannot prove leaves the buffer
/// in global memory.
std::vector<Slab> planSlabs(const KernelModule& km, uint32_t root, int64_t workgroups) {
    std::vector<Slab> out;
    std::vector<bool> stored(km.buffers.size(), false);
    for (const KernelNode& n : km.nodes) {
        if (n.op == KernelOp::Store && n.bufferOut < km.buffers.size()) stored[n.bufferOut] = true;
    }
    Ctx cx{km, false, ErrorCode::UnsupportedCapability, std::string(), 0};
    std::vector<Range> r;
    std::vector<Access> acc;
    const std::vector<uint32_t> self{root};
    collect(cx, self, r, true, acc, 0);
    if (cx.failed) return out;
    int64_t used = 0;
    for (uint32_t b = 0; b < km.buffers.size(); ++b) {
        const KernelBuffer& kb = km.buffers[b];
        if (stored[b] || !kb.isInput || kb.isTemp) continue;
        const int64_t elems = cx.staticElems(b);
        if (elems <= 0) continue;
        int64_t lo = INT64_MAX, hi = INT64_MIN;
        // Reads over the loop hulls, and the distinct indices they can form:
        // an element is re-read only through loops whose coefficient in the
        // access is zero. A variable that steers a deeper loop's bounds (a
        // tile index) only moves that loop's window, already counted in the
        // deeper loop's hull, so it multiplies neither.
        __int128 reads = 0, distinct = 0;
        bool ok = true, any = false;
        for (const Access& a : acc) {
            if (a.buf != b || a.store) continue;
            int64_t l = 0, h = 0;
            bool u = false;
            if (!bound(a.at, a.ranges, a.depth, l, h, u) || u || l < 0 || h >= elems) {
                ok = false;
                break;
            }
            any = true;
            lo = std::min(lo, l);
            hi = std::max(hi, h);
            __int128 it = 1, dist = 1;
            for (size_t p = 0; p < a.ranges.size(); ++p) {
                const Range& x = a.ranges[p];
                if (x.unbounded) {
                    ok = false;
                    break;
                }
                if (x.steers) continue;
                const __int128 trips = static_cast<__int128>(x.hi - x.lo + 1);
                it = std::min<__int128>(it * trips, kIndexLimit);
                if (coeffAt(a.at, p) != 0) dist = std::min<__int128>(dist * trips, kIndexLimit);
            }
            reads += it;
            distinct += dist;
        }
        if (!ok || !any) continue;
        const int64_t span = hi - lo + 1;
        const int64_t bytes = (span * dtypeBytes(kb.dtype) + 15) / 16 * 16;   // each slab 16-byte aligned
        if (used + bytes > kSlabBudget) continue;
        if (reads < static_cast<__int128>(kSlabReuse) * distinct) continue;
        if (reads < static_cast<__int128>(kSlabReuse) * span * workgroups) continue;
        used += bytes;
        out.push_back(Slab{b, lo, span});
    }
    return out;
}

struct Reg {
    uint32_t buf;
    std::string name;
};

struct Emitter {
    Ctx& cx;
    const KernelModule& km;
    std::vector<uint32_t> slots;      // slot -> buffer id
    std::vector<int> slotOf;          // buffer id -> slot
    std::vector<Reg> regs;            // register-held buffers in scope
    std::vector<Slab> slabs;          // LDS-staged inputs
    std::vector<int> memReads, memStores, memAdds;
    // Register sites per buffer: opens emitted, closes emitted, and whether
    // an open can run more than once for one element (an enclosing loop
    // with a zero coefficient in the address, more than one iteration, and
    // no deeper loop bound on the path that it moves).
    std::vector<int> regOpens, regCloses;
    std::vector<char> regRepeats;
    // Each open site's in-thread element hull, with the address's
    // coefficients on the collapsed (thread) loops: other threads own other
    // elements, so two sites meet only with equal thread coefficients and
    // meeting hulls.
    struct RegSpan {
        std::vector<int64_t> threadCoeffs;
        int64_t lo, hi;
    };
    std::vector<std::vector<RegSpan>> regSpans;
    size_t chainLen{0};
    std::vector<int> steerCount;      // loop position -> deeper path loops whose bounds use it
    // Element hulls of the kernel's memory reads and writes, per buffer
    // (lo > hi: none), over every thread's iterations.
    std::vector<std::pair<int64_t, int64_t>> readHull, writeHull;
    std::string code;
    int nextReg{0};
    bool checked{false};
    bool transcendental{false};

    Emitter(Ctx& c)
        : cx(c), km(c.km), slotOf(c.km.buffers.size(), -1), memReads(c.km.buffers.size(), 0),
          memStores(c.km.buffers.size(), 0), memAdds(c.km.buffers.size(), 0), regOpens(c.km.buffers.size(), 0),
          regCloses(c.km.buffers.size(), 0), regRepeats(c.km.buffers.size(), 0), regSpans(c.km.buffers.size()),
          steerCount(kMaxDepth + 1, 0), readHull(c.km.buffers.size(), {INT64_MAX, INT64_MIN}),
          writeHull(c.km.buffers.size(), {INT64_MAX, INT64_MIN}) {}

    void widenHull(std::vector<std::pair<int64_t, int64_t>>& h, uint32_t b, const Affine& at,
                   const std::vector<Range>& r) {
        int64_t lo = 0, hi = 0;
        bool u = false;
        if (!bound(at, r, r.size(), lo, hi, u) || u) {
            lo = INT64_MIN;
            hi = INT64_MAX;
        }
        h[b].first = std::min(h[b].first, lo);
        h[b].second = std::max(h[b].second, hi);
    }

    /// Two register sites of buffer b can reach one element.
    bool regSitesOverlap(uint32_t b) const {
        const auto& v = regSpans[b];
        for (size_t i = 0; i < v.size(); ++i) {
            for (size_t j = i + 1; j < v.size(); ++j) {
                if (v[i].threadCoeffs != v[j].threadCoeffs) return true;
                if (v[i].lo <= v[j].hi && v[j].lo <= v[i].hi) return true;
            }
        }
        return false;
    }

    int slot(uint32_t b) {
        if (slotOf[b] >= 0) return slotOf[b];
        if (slots.size() >= static_cast<size_t>(kMaxSlots)) {
            cx.fail(ErrorCode::UnsupportedCapability, "loop nest binds more than 16 buffers");
            return 0;
        }
        slotOf[b] = static_cast<int>(slots.size());
        slots.push_back(b);
        return slotOf[b];
    }
    const Reg* regFor(uint32_t b) const {
        for (auto it = regs.rbegin(); it != regs.rend(); ++it) {
            if (it->buf == b) return &*it;
        }
        return nullptr;
    }
    /// In [0, static element count) for every variable value.
    bool inBounds(uint32_t b, const Affine& at, const std::vector<Range>& r) {
        const int64_t n = cx.staticElems(b);
        int64_t lo = 0, hi = 0;
        bool u = false;
        if (!bound(at, r, r.size(), lo, hi, u)) {
            cx.fail(ErrorCode::UnsupportedCapability, "index expression outside the index budget");
            return false;
        }
        return !u && n > 0 && lo >= 0 && hi < n;
    }
    bool negativePossible(const Affine& at, const std::vector<Range>& r) {
        int64_t lo = 0, hi = 0;
        bool u = false;
        if (!bound(at, r, r.size(), lo, hi, u)) return true;
        return u || lo < 0;
    }

    /// Buffers whose every access in the region is a store to one address
    /// that is invariant below position `inner` (loop variables from `inner`
    /// on have zero coefficients), with at least one store definite.
    std::vector<std::pair<uint32_t, Affine>> regCandidates(const std::vector<Access>& acc, size_t inner,
                                                          const std::vector<Range>& outer) {
        std::vector<std::pair<uint32_t, Affine>> out;
        std::vector<uint32_t> seen;
        for (const Access& a : acc) {
            if (std::find(seen.begin(), seen.end(), a.buf) != seen.end()) continue;
            seen.push_back(a.buf);
            if (a.buf >= km.buffers.size() || regFor(a.buf) != nullptr) continue;
            bool ok = true, definite = false;
            Affine at;
            at.off = a.at.off;
            at.c.assign(inner, 0);
            for (size_t p = 0; p < inner; ++p) at.c[p] = coeffAt(a.at, p);
            for (const Access& b : acc) {
                if (b.buf != a.buf) continue;
                if (!b.store || b.at.off != at.off) {
                    ok = false;
                    break;
                }
                for (size_t p = 0; p < std::max(b.at.c.size(), inner); ++p) {
                    const int64_t want = p < inner ? at.c[p] : 0;
                    if (coeffAt(b.at, p) != want) ok = false;
                }
                definite = definite || b.definite;
            }
            if (!ok || !definite) continue;
            if (!inBounds(a.buf, at, outer)) continue;
            out.emplace_back(a.buf, at);
        }
        return out;
    }

    std::string loadExpr(uint32_t b, const Affine& at, const std::vector<Range>& r) {
        const int s = slot(b);
        const std::string dt = std::to_string(dtypeCode(km.buffers[b].dtype));
        const std::string f = affineCode(at, r.size());
        ++memReads[b];
        widenHull(readHull, b, at, r);
        for (size_t k = 0; k < slabs.size(); ++k) {
            // The slab's hull covers every read of the buffer in the root.
            if (slabs[k].buf == b) {
                return "mlk::loadOne<" + dt + ">(mlk_slab" + std::to_string(k) + ", " + f + " - " +
                       intLit(slabs[k].lo) + ")";
            }
        }
        if (inBounds(b, at, r)) return "mlk::loadOne<" + dt + ">(mb" + std::to_string(s) + ", " + f + ")";
        checked = true;
        return "mlk_ld_chk<" + dt + ">(mb" + std::to_string(s) + ", " + f + ", a.n[" + std::to_string(s) +
               "], a.status, bad)";
    }

    void line(int ind, const std::string& s) { code += std::string(static_cast<size_t>(ind) * 4, ' ') + s + "\n"; }

    void pair(const KernelNode& cp, const KernelNode& so, std::vector<Range>& r, int ind) {
        if (hasLegacyOperand(cp)) {
            cx.fail(ErrorCode::InvalidGraph, "walker: legacy element operand in a multi-dim compute");
            return;
        }
        if (!cx.bindable(so.bufferOut)) {
            cx.fail(ErrorCode::InvalidArgument, "walker: output buffer not bound");
            return;
        }
        for (const KernelExpr& e : cp.exprs) {
            switch (e.op) {
                case MathOp::Exp: case MathOp::Log: case MathOp::Pow: case MathOp::Cos: case MathOp::Tan:
                case MathOp::Tanh: case MathOp::Erf: case MathOp::Gelu:
                    transcendental = true;
                    break;
                case MathOp::Sin:
                    if (cp.family != "poly7") transcendental = true;
                    break;
                default: break;
            }
        }
        auto elem = [&](const KernelOperand& o) -> std::string {
            if (o.kind != K::ElemIdx) return std::string();
            if (o.index < 0 || static_cast<size_t>(o.index) >= km.buffers.size()) return "0.0";  // elemPtr null
            const uint32_t b = static_cast<uint32_t>(o.index);
            if (!cx.bindable(b)) {
                cx.fail(ErrorCode::UnsupportedCapability, "operand buffer is not bindable");
                return std::string();
            }
            return loadExpr(b, trimmed(o.idxCoeffs, o.idxOffset, r.size()), r);
        };
        // An empty chain evaluates to 0.0 (kernel_buffers.cpp:176-177), still stored.
        std::string bodyText = "            val = 0.0;\n";
        if (!cp.exprs.empty()) {
            auto body = chainCode(cp.exprs, cp.family == "poly7", false, elem, "val = ");
            if (!body.has_value()) {
                cx.fail(body.error().code, body.error().message);
                return;
            }
            bodyText = *body;
        }
        line(ind, "{");
        line(ind + 1, "bool bad = false;");
        line(ind + 1, "(void)bad;");
        line(ind + 1, "double val;");
        line(ind + 1, "{");
        code += bodyText;
        line(ind + 1, "}");
        line(ind + 1, "if (bad) return;");
        const uint32_t w = so.bufferOut;
        const Affine at = trimmed(so.outIndexCoeffs, so.outIndexOffset, r.size());
        if (const Reg* rg = regFor(w)) {
            const std::string& x = rg->name;
            if (so.accum == AccumMode::Add) line(ind + 1, x + " = " + x + " + val;");
            else if (so.accum == AccumMode::Max) line(ind + 1, x + " = (val > " + x + ") ? val : " + x + ";");
            else line(ind + 1, x + " = val;");
        } else {
            const int s = slot(w);
            const std::string dt = std::to_string(dtypeCode(km.buffers[w].dtype));
            const std::string bs = "mb" + std::to_string(s);
            line(ind + 1, "const long long f = " + affineCode(at, r.size()) + ";");
            if (!inBounds(w, at, r)) {
                checked = true;
                if (negativePossible(at, r)) line(ind + 1, "if (f < 0) { *a.status = 1; return; }");
                line(ind + 1, "if (f >= a.n[" + std::to_string(s) + "]) { *a.status = 6; return; }");
            }
            ++memStores[w];
            widenHull(writeHull, w, at, r);
            if (so.accum != AccumMode::None) widenHull(readHull, w, at, r);
            if (so.accum == AccumMode::Add) {
                ++memAdds[w];
                ++memReads[w];
                line(ind + 1, "mlk::storeOne<" + dt + ">(" + bs + ", f, mlk::loadOne<" + dt + ">(" + bs + ", f) + val);");
            } else if (so.accum == AccumMode::Max) {
                line(ind + 1, "const double o = mlk::loadOne<" + dt + ">(" + bs + ", f);");
                line(ind + 1, "mlk::storeOne<" + dt + ">(" + bs + ", f, (val > o) ? val : o);");
            } else {
                line(ind + 1, "mlk::storeOne<" + dt + ">(" + bs + ", f, val);");
            }
        }
        line(ind, "}");
    }

    /// Opens registers for `cands` (loaded from their slots), returns how many.
    size_t openRegs(const std::vector<std::pair<uint32_t, Affine>>& cands, const std::vector<Range>& outer, int ind) {
        for (const auto& c : cands) {
            const int s = slot(c.first);
            const std::string dt = std::to_string(dtypeCode(km.buffers[c.first].dtype));
            const std::string name = "r" + std::to_string(nextReg++);
            line(ind, "const long long " + name + "f = " + affineCode(c.second, outer.size()) + ";");
            line(ind, "double " + name + " = mlk::loadOne<" + dt + ">(mb" + std::to_string(s) + ", " + name + "f);");
            regs.push_back(Reg{c.first, name});
            ++regOpens[c.first];
            widenHull(readHull, c.first, c.second, outer);
            widenHull(writeHull, c.first, c.second, outer);
            {
                RegSpan sp;
                Affine local = c.second;
                for (size_t p = 0; p < chainLen && p < local.c.size(); ++p) {
                    sp.threadCoeffs.push_back(local.c[p]);
                    local.c[p] = 0;
                }
                bool u = false;
                if (!bound(local, outer, outer.size(), sp.lo, sp.hi, u) || u) {
                    sp.lo = INT64_MIN;
                    sp.hi = INT64_MAX;
                }
                regSpans[c.first].push_back(std::move(sp));
            }
            for (size_t p = 0; p < outer.size(); ++p) {
                if (coeffAt(c.second, p) == 0 && steerCount[p] == 0 && !outer[p].unbounded && outer[p].hi > outer[p].lo) {
                    regRepeats[c.first] = 1;
                }
            }
        }
        return cands.size();
    }
    void closeRegs(size_t n, int ind) {
        for (size_t i = 0; i < n; ++i) {
            const Reg rg = regs.back();
            regs.pop_back();
            const int s = slotOf[rg.buf];
            const std::string dt = std::to_string(dtypeCode(km.buffers[rg.buf].dtype));
            line(ind, "mlk::storeOne<" + dt + ">(mb" + std::to_string(s) + ", " + rg.name + "f, " + rg.name + ");");
            ++memStores[rg.buf];
            ++regCloses[rg.buf];
        }
    }

    void children(const std::vector<uint32_t>& ch, std::vector<Range>& r, int ind, int level) {
        if (cx.failed) return;
        if (level > kMaxDepth || ++cx.visited > kMaxNodesVisited) {
            cx.fail(ErrorCode::UnsupportedCapability, "loop nest deeper or larger than the generic path takes");
            return;
        }
        for (size_t ci = 0; ci < ch.size() && !cx.failed; ++ci) {
            const uint32_t id = ch[ci];
            if (id >= km.nodes.size()) {
                cx.fail(ErrorCode::InvalidGraph, "walker: child id out of range");
                return;
            }
            const KernelNode& n = km.nodes[id];
            switch (n.op) {
                case KernelOp::Compute:
                    if (ci + 1 < ch.size() && ch[ci + 1] < km.nodes.size() && km.nodes[ch[ci + 1]].op == KernelOp::Store) {
                        pair(n, km.nodes[ch[ci + 1]], r, ind);
                        ++ci;
                    }
                    break;
                case KernelOp::Loop: loop(n, r, ind, level); break;
                case KernelOp::Guard: guard(n, r, ind, level); break;
                case KernelOp::Call: cx.fail(ErrorCode::UnsupportedCapability, "Call inside a loop nest"); return;
                default: break;  // Store alone, Load, Alloc, Copy, Barrier, Trace: no walker semantics
            }
        }
    }

    void loop(const KernelNode& n, std::vector<Range>& r, int ind, int level) {
        if (n.step != 1) {
            cx.fail(ErrorCode::UnsupportedCapability, "walker: non-unit loop step");
            return;
        }
        if (r.size() >= static_cast<size_t>(kMaxDepth)) {
            cx.fail(ErrorCode::UnsupportedCapability, "loop nest deeper than the generic path takes");
            return;
        }
        const LoopBounds lb = loopBounds(km, n);
        Range vr;
        bool dead = false, nonEmpty = false;
        if (!loopRange(cx, lb, r, vr, dead, nonEmpty) || dead) return;
        const size_t d = r.size();
        const std::string v = "v" + std::to_string(d);
        line(ind, "{");
        line(ind + 1, "const long long " + v + "b = " + affineCode(lb.begin, d) + ";");
        line(ind + 1, "const long long " + v + "e = " +
                          (lb.dynamicEnd ? std::string("a.elements - 1LL") : affineCode(lb.endInc, d)) + ";");
        // Register candidates of this loop's subtree.
        std::vector<Access> acc;
        r.push_back(vr);
        collect(cx, n.children, r, true, acc, level + 1);
        r.pop_back();
        if (cx.failed) return;
        const auto cands = regCandidates(acc, d, r);
        std::vector<size_t> steered;
        for (size_t p = 0; p < d; ++p) {
            if (coeffAt(lb.begin, p) != 0 || coeffAt(lb.endInc, p) != 0) {
                ++steerCount[p];
                steered.push_back(p);
            }
        }
        int bodyInd = ind + 1;
        if (!cands.empty()) {
            line(ind + 1, "if (" + v + "b <= " + v + "e) {");
            bodyInd = ind + 2;
        }
        const size_t opened = openRegs(cands, r, bodyInd);
        line(bodyInd, "for (long long " + v + " = " + v + "b; " + v + " <= " + v + "e; ++" + v + ") {");
        r.push_back(vr);
        // Per-iteration registers: addresses that move with this loop's
        // variable but not with the loops inside it.
        std::vector<Access> iter;
        collect(cx, n.children, r, true, iter, level + 1);
        if (cx.failed) return;
        const auto perIter = regCandidates(iter, d + 1, r);
        const size_t openedIter = openRegs(perIter, r, bodyInd + 1);
        children(n.children, r, bodyInd + 1, level + 1);
        closeRegs(openedIter, bodyInd + 1);
        r.pop_back();
        line(bodyInd, "}");
        closeRegs(opened, bodyInd);
        if (!cands.empty()) line(ind + 1, "}");
        line(ind, "}");
        for (const size_t p : steered) --steerCount[p];
    }

    void guard(const KernelNode& n, std::vector<Range>& r, int ind, int level) {
        if (n.guardCoeffs.empty()) return;  // the walker runs nothing under an empty guard
        std::vector<Range> rr = r;
        bool constTrue = false;
        if (!refineGuard(cx, n, rr, constTrue)) return;
        Affine g = trimmed(n.guardCoeffs, n.guardOffset, r.size());
        line(ind, constTrue ? "{" : "if (" + affineCode(g, r.size()) + " == 0LL) {");
        children(n.children, rr, ind + 1, level + 1);
        line(ind, "}");
    }
};

}  // namespace

Result<Step> planNestWith(const KernelModule& km, uint32_t root, bool allowSlabs, int maxChain) {
    Ctx cx{km, false, ErrorCode::UnsupportedCapability, std::string(), 0};
    Step st;
    st.kind = StepKind::Nest;
    st.what = "loop-nest";
    st.root = root;
    if (root >= km.nodes.size()) return err(ErrorCode::InvalidGraph, "walker: node id out of range");

    // The collapsed chain: parallel (marked or proven) unit-step loops with
    // static bounds, each but the last with a single loop child.
    std::vector<Range> r;
    std::vector<LoopBounds> chainB;
    std::vector<int64_t> trips;
    std::vector<bool> tripChecked;
    const KernelNode* body = nullptr;   // the last chain loop
    uint32_t cur = root;
    bool deadRoot = false;
    while (km.nodes[cur].op == KernelOp::Loop && chainB.size() < static_cast<size_t>(maxChain)) {
        const KernelNode& n = km.nodes[cur];
        if (n.step != 1) break;
        const LoopBounds lb = loopBounds(km, n);
        if (lb.dynamicEnd) break;
        Range vr;
        bool dead = false, nonEmpty = false;
        if (!loopRange(cx, lb, r, vr, dead, nonEmpty)) return err(cx.code, cx.why);
        if (vr.unbounded) break;
        if (dead) {
            deadRoot = true;
            break;
        }
        if (!n.parallel && !provablyParallel(cx, n, r, vr)) {
            if (cx.failed) return err(cx.code, cx.why);
            break;
        }
        // Padded trip count: max over the enclosing ranges of end - begin + 1.
        Affine diff;
        const size_t m = std::max(lb.begin.c.size(), lb.endInc.c.size());
        diff.c.assign(m, 0);
        for (size_t p = 0; p < m; ++p) diff.c[p] = coeffAt(lb.endInc, p) - coeffAt(lb.begin, p);
        diff.off = lb.endInc.off - lb.begin.off;
        int64_t dl = 0, dh = 0;
        bool du = false;
        if (!bound(diff, r, r.size(), dl, dh, du) || du) break;
        if (dh < 0) {
            deadRoot = true;
            break;
        }
        chainB.push_back(lb);
        trips.push_back(dh + 1);
        tripChecked.push_back(dl != dh);
        r.push_back(vr);
        body = &n;
        if (n.children.size() == 1 && n.children[0] < km.nodes.size() &&
            km.nodes[n.children[0]].op == KernelOp::Loop) {
            cur = n.children[0];
            continue;
        }
        break;
    }
    if (deadRoot) {
        st.kind = StepKind::Fail;  // no instance executes
        st.what = "empty";
        return st;
    }
    __int128 total = 1;
    for (const int64_t t : trips) {
        total *= t;
        if (total > kMaxInstances) {
            return err(ErrorCode::UnsupportedCapability, "collapsed iteration space above 2^40 instances");
        }
    }

    Emitter em(cx);
    const int64_t workgroups = std::min<int64_t>(std::max<int64_t>((static_cast<int64_t>(total) + 255) / 256, 1),
                                                 16384);   // the launch grid (driver gridFor)
    if (allowSlabs) em.slabs = planSlabs(km, root, workgroups);
    // The thread body: the last chain loop's children, or the root itself.
    const int ind = 2;
    std::string chainCodeText;
    const size_t chainLen = chainB.size();
    if (chainLen > 0) {
        chainCodeText += "        long long rem = g;\n";
        for (size_t l = chainLen; l-- > 0;) {
            const std::string ll = "l" + std::to_string(l);
            if (l == 0) {
                chainCodeText += "        const long long " + ll + " = rem;\n";
            } else {
                chainCodeText += "        const long long " + ll + " = rem % " + intLit(trips[l]) + ";\n";
                chainCodeText += "        rem /= " + intLit(trips[l]) + ";\n";
            }
        }
        for (size_t l = 0; l < chainLen; ++l) {
            const std::string v = "v" + std::to_string(l);
            chainCodeText += "        const long long " + v + " = " + affineCode(chainB[l].begin, l) + " + l" +
                             std::to_string(l) + ";\n";
            if (tripChecked[l]) {
                chainCodeText += "        if (" + v + " > " + affineCode(chainB[l].endInc, l) + ") continue;\n";
            }
        }
        em.chainLen = chainLen;
        // Chain loops whose bounds use an outer chain variable (a tile index
        // moving its point loop's window) steer it for the whole body.
        for (size_t l = 0; l < chainB.size(); ++l) {
            for (size_t p = 0; p < l; ++p) {
                if (coeffAt(chainB[l].begin, p) != 0 || coeffAt(chainB[l].endInc, p) != 0) ++em.steerCount[p];
            }
        }
        // Registers over the whole thread body.
        std::vector<Access> acc;
        collect(cx, body->children, r, true, acc, 1);
        if (cx.failed) return err(cx.code, cx.why);
        const auto cands = em.regCandidates(acc, chainLen, r);
        const size_t opened = em.openRegs(cands, r, ind);
        em.children(body->children, r, ind, 1);
        em.closeRegs(opened, ind);
    } else {
        const std::vector<uint32_t> self{root};
        em.children(self, r, ind, 1);
    }
    if (cx.failed) return err(cx.code, cx.why);
    for (const Slab& sl : em.slabs) em.slot(sl.buf);   // read by the emitted code, so already bound

    std::string src;
    src += "// generic loop nest: root node " + std::to_string(root) + ", " + std::to_string(chainLen) +
           " collapsed loop(s)\n";
    src += "// mlk-nest slots:";
    for (const uint32_t b : em.slots) src += " " + std::to_string(b);
    src += "\n// mlk-nest instances: " + std::to_string(static_cast<int64_t>(total)) + "\n";
    for (const Slab& sl : em.slabs) {
        src += "// mlk-nest slab: buffer " + std::to_string(sl.buf) + " elements [" + std::to_string(sl.lo) + ", " +
               std::to_string(sl.lo + sl.span) + ")\n";
    }
    src += deviceMathHeader();
    src += R"(
struct mlk_nest_args {
    void* p[16];
    long long n[16];
    int* status;
    long long elements;
};

// Threads per workgroup: 256 unless the launch form defines another.
#ifndef MLK_NEST_WG
#define MLK_NEST_WG 256
#endif

// The workgroup's threads share each slab's copy; a host harness that runs
// one thread at a time defines these to copy the whole slab per thread.
#ifndef MLK_SLAB_FIRST
#define MLK_SLAB_FIRST static_cast<long long>(threadIdx.x)
#define MLK_SLAB_STEP MLK_NEST_WG
#endif

template <int DT>
__device__ __forceinline__ double mlk_ld_chk(const void* p, long long f, long long n, int* st, bool& bad) {
    if (f < 0 || f >= n) {
        bad = true;
        *st = 6;
        return 0.0;
    }
    return mlk::loadOne<DT>(p, f);
}

extern "C" __global__ __launch_bounds__(MLK_NEST_WG) void mlk_nest(const mlk_nest_args a, const mlk_scalars sc,
                                                           long long total) {
    (void)sc;
)";
    for (size_t s = 0; s < em.slots.size(); ++s) {
        src += "    void* const mb" + std::to_string(s) + " = a.p[" + std::to_string(s) + "];\n";
    }
    for (size_t k = 0; k < em.slabs.size(); ++k) {
        const Slab& sl = em.slabs[k];
        const Dtype d = km.buffers[sl.buf].dtype;
        const std::string ty = d == Dtype::F32 ? "float" : (d == Dtype::F16 ? "_Float16" : "double");
        const std::string nm = "mlk_slab" + std::to_string(k);
        const std::string mb = "mb" + std::to_string(em.slot(sl.buf));
        src += "    __shared__ __attribute__((aligned(16))) " + ty + " " + nm + "[" + intLit(sl.span) + "];\n";
        src += "    for (long long i = MLK_SLAB_FIRST; i < " + intLit(sl.span) + "; i += MLK_SLAB_STEP) " + nm +
               "[i] = static_cast<const " + ty + "*>(" + mb + ")[" + intLit(sl.lo) + " + i];\n";
    }
    if (!em.slabs.empty()) src += "    __syncthreads();\n";
    src += "    const long long stride = static_cast<long long>(gridDim.x) * MLK_NEST_WG;\n";
    src += "    for (long long g = static_cast<long long>(blockIdx.x) * MLK_NEST_WG + threadIdx.x; g < total; "
           "g += stride) {\n";
    src += chainLen > 0 ? chainCodeText : "        (void)g;\n";
    src += em.code;
    src += "    }\n}\n";

    st.source = std::move(src);
    st.readHull = em.readHull;
    st.writeHull = em.writeHull;
    st.slabs = static_cast<int>(em.slabs.size());
    st.nestBufs = em.slots;
    st.threads = static_cast<int64_t>(total);
    st.collapsed = static_cast<int>(chainLen);
    st.checked = em.checked;
    st.transcendental = em.transcendental;
    for (const uint32_t b : em.slots) {
        const Dtype d = km.buffers[b].dtype;
        if (em.memStores[b] > 0) st.nestWrites.push_back(b);
        if (em.memReads[b] > 0 || em.regOpens[b] > 0) st.nestReads.push_back(b);
        if (d == Dtype::F16) st.touchesF16 = true;
        // A narrow buffer's value is rounded on every store; reading one back
        // (a memory read or += of a stored buffer, a register reopened on
        // one element by a repeating loop or by two sites whose element
        // hulls meet, or a register beside direct accesses) departs from the
        // walker, which holds f64 throughout.
        const bool regTrip = em.regSitesOverlap(b) || em.regRepeats[b] != 0 ||
                             (em.regOpens[b] > 0 && (em.memStores[b] > em.regCloses[b] || em.memReads[b] > 0));
        if (d != Dtype::F64 && ((em.memReads[b] > em.memAdds[b] && em.memStores[b] > 0) || em.memAdds[b] > 0 ||
                                regTrip)) {
            st.narrowRoundTrip = true;
        }
    }
    return st;
}

Result<Step> planNest(const KernelModule& km, uint32_t root) {
    // Schedule parameter "hip_slabs" = 0 keeps every buffer in global memory
    // (the reference's slabs are likewise an emitter option,
    // slab_plan.h:51-62); "hip_collapse_max" caps the collapsed loops.
    const bool slabsOn = km.param("hip_slabs", 1) != 0;
    const int maxChain = static_cast<int>(std::clamp<int64_t>(km.param("hip_collapse_max", kMaxChain), 0, kMaxChain));
    auto st = planNestWith(km, root, slabsOn, maxChain);
    if (!st.has_value() || st->kind != StepKind::Nest) return st;
    if (st->slabs > 0) {
        auto plain = planNestWith(km, root, false, maxChain);
        // Same slots: one binding serves both.
        if (plain.has_value() && plain->nestBufs == st->nestBufs) st->sourceNoSlabs = std::move(plain->source);
    }
    // Form 4: the innermost collapsed loop runs inside each thread. Declared
    // only where it and form 0 both hold the walker's values exactly (no
    // narrow round trip), so the two give the same bits.
    if (st->collapsed >= 2 && !st->narrowRoundTrip) {
        auto less = planNestWith(km, root, slabsOn, st->collapsed - 1);
        if (less.has_value() && less->kind == StepKind::Nest && less->nestBufs == st->nestBufs &&
            !less->narrowRoundTrip && less->collapsed == st->collapsed - 1) {
            st->sourceLessCollapse = std::move(less->source);
            st->threadsLessCollapse = less->threads;
            st->checkedLessCollapse = less->checked;
        }
    }
    return st;
}

std::vector<int> nestForms(const Step& st) {
    std::vector<int> v{0};
    if (!st.sourceNoSlabs.empty()) v.push_back(1);
    v.push_back(2);
    v.push_back(3);
    if (!st.sourceLessCollapse.empty()) v.push_back(4);
    return v;
}

unsigned nestFormThreads(int form) { return form == 2 ? 512u : (form == 3 ? 64u : 256u); }

std::string nestFormSource(const Step& st, int form) {
    switch (form) {
        case 0: return st.source;
        case 1: return st.sourceNoSlabs;
        case 2:
        case 3: return "#define MLK_NEST_WG " + std::to_string(nestFormThreads(form)) + "\n" + st.source;
        case 4: return st.sourceLessCollapse;
        default: return std::string();
    }
}

int64_t nestFormInstances(const Step& st, int form) { return form == 4 ? st.threadsLessCollapse : st.threads; }

bool nestFormChecked(const Step& st, int form) { return form == 4 ? st.checkedLessCollapse : st.checked; }

}  // namespace mlk::hip
