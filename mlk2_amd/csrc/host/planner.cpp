// Class recognition for the HIP backend.
//
// Tier-1 modules (no multi-dim feature) follow the reference executor's
// top-level loop (runtime/src/execution/kernel_buffers.cpp:921-1085): every
// Loop node runs its Compute children over [begin, end) paired with the
// first Store child; Call nodes run MatMul / Softmax / ReduceSum. Multi-dim
// modules follow the walker (:902-920): roots in id order, each recognized
// as one of
//   * a perfect loop nest ending in one Compute+Store pair (the poly.synth
//     broadcast elementwise nest, poly.synth.cpp:231-353)   -> elementwise
//   * the poly.synth GEMM nest (:58-147)                     -> gemm
//   * the poly.synth ReduceSum nest (:153-229)               -> row sum
//   * the poly.synth softmax nest (:363-523)                 -> softmax
//   * a Call node                                            -> as Tier 1
// and the three-root window batched-QK^T nest / scale+bias nest / softmax
// nest over one temp score matrix is fused into one score-softmax launch.
#include "planner.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>

#include "../device_abi.h"

namespace mlk::hip {

namespace {

using K = KernelOperand::Kind;

int64_t bufElems(const KernelBuffer& b) { return bufferElements(b, -1); }

/// min/max of offset + sum c_d * v_d over v_d in [0, e_d).
void affineRange(const StreamRef& s, int rank, const int64_t* ext, int64_t& lo, int64_t& hi) {
    lo = hi = s.offset;
    for (int d = 0; d < rank; ++d) {
        const int64_t span = s.coeff[d] * (ext[d] - 1);
        if (span < 0) lo += span; else hi += span;
    }
}

/// Sufficient injectivity test of an affine map over a box: sorted by
/// |coeff|, each coefficient exceeds the largest offset the smaller ones can
/// reach.
bool injective(const StreamRef& s, int rank, const int64_t* ext) {
    int64_t c[4];
    int64_t e[4];
    int n = 0;
    for (int d = 0; d < rank; ++d) {
        if (ext[d] <= 1) continue;
        const int64_t a = s.coeff[d] < 0 ? -s.coeff[d] : s.coeff[d];
        if (a == 0) return false;
        c[n] = a;
        e[n] = ext[d];
        ++n;
    }
    for (int i = 0; i < n; ++i) {
        for (int j = i + 1; j < n; ++j) {
            if (c[j] < c[i]) {
                std::swap(c[i], c[j]);
                std::swap(e[i], e[j]);
            }
        }
    }
    int64_t reach = 0;
    for (int i = 0; i < n; ++i) {
        if (c[i] <= reach) return false;
        reach += c[i] * (e[i] - 1);
    }
    return true;
}

bool sameMap(const StreamRef& a, const StreamRef& b, int rank) {
    if (a.buffer != b.buffer || a.offset != b.offset) return false;
    for (int d = 0; d < rank; ++d) {
        if (a.coeff[d] != b.coeff[d]) return false;
    }
    return true;
}

/// Significant bits of a stream's values: 24 (f32), 11 (f16), 99 for f64
/// and unbound ids (no exact-product claim).
int streamBits(const KernelModule& km, int64_t bid) {
    if (bid < 0 || static_cast<size_t>(bid) >= km.buffers.size()) return 99;
    const Dtype d = km.buffers[static_cast<size_t>(bid)].dtype;
    return d == Dtype::F32 ? 24 : (d == Dtype::F16 ? 11 : 99);
}

/// Adapts a stream-index lookup to chainCode's operand callback.
template <class StreamOf>
std::function<std::string(const KernelOperand&)> streamCode(StreamOf& streamOf) {
    return [&streamOf](const KernelOperand& o) -> std::string {
        const int s = streamOf(o);
        return s < 0 ? std::string() : "in[" + std::to_string(s) + "]";
    };
}

}  // namespace

std::string literal(double v) {
    if (std::isnan(v)) return "__builtin_nan(\"\")";
    if (std::isinf(v)) return v > 0 ? "__builtin_inf()" : "(-__builtin_inf())";
    char buf[64];
    std::snprintf(buf, sizeof(buf), "%a", v);
    return std::string("(") + buf + ")";
}

namespace {

/// Significant bits of an f64 constant whose products with f32/f16 values
/// stay normal and finite (|v| in [2^-200, 2^200], or zero); 99 otherwise.
int constBits(double v) {
    if (v == 0.0) return 0;
    if (!std::isfinite(v) || std::fabs(v) > 0x1p200 || std::fabs(v) < 0x1p-200) return 99;
    int e = 0;
    const double m = std::frexp(std::fabs(v), &e);
    uint64_t i = static_cast<uint64_t>(std::ldexp(m, 53));
    int bits = 53;
    while ((i & 1u) == 0) {
        i >>= 1;
        --bits;
    }
    return bits;
}

}  // namespace

/// Builds the f64 chain body; elemCode(o) returns the device expression of an
/// element operand (empty when it cannot be realized). The reference
/// evaluation (kernel_buffers.cpp:106-178): unary ops ignore b, Temp reads
/// earlier results, ScalarParam past the table reads 0.0.
///
/// A product used only by one sum, whose operands' significant bits
/// (elemBits: 24 for f32 streams, 11 for f16) add up to 53 or fewer, is exact
/// in f64; the sum is then written as one fused multiply-add, which rounds
/// once exactly as the reference's separate product and sum do.
Result<std::string> chainCode(const std::vector<KernelExpr>& exprs, bool poly7, bool f32Out,
                              const std::function<std::string(const KernelOperand&)>& elemCode,
                              const std::string& sink,
                              const std::function<int(const KernelOperand&)>& elemBits) {
    if (exprs.empty() || exprs.size() > 64) {
        return err(ErrorCode::UnsupportedCapability, "chain length outside 1..64");
    }
    // exp with f32 accuracy (mlk_exp_f32acc) where the result is rounded to
    // f32 and the exp's value reaches it only as a factor: every use of it,
    // and of each temp on the way, is an operand of Mul, Div or Neg, which
    // carry a relative error through unchanged. One such exp per chain, used
    // once, keeps the f32 result within 3 ULP of the reference's.
    const size_t last = exprs.size() - 1;
    std::vector<int> uses(exprs.size(), 0);
    std::vector<std::vector<size_t>> users(exprs.size());
    for (size_t j = 0; j < exprs.size(); ++j) {
        const KernelExpr& e = exprs[j];
        for (const KernelOperand* o : {&e.a, &e.b}) {
            if (o == &e.b && isUnaryMath(e.op)) continue;
            if (o->kind == K::Temp && o->index >= 0 && static_cast<size_t>(o->index) < j) {
                ++uses[static_cast<size_t>(o->index)];
                users[static_cast<size_t>(o->index)].push_back(j);
            }
        }
    }
    std::vector<char> factorPath(exprs.size(), 0);
    factorPath[last] = 1;
    for (size_t k = last; k-- > 0;) {
        bool ok = !users[k].empty();
        for (size_t j : users[k]) {
            const MathOp op = exprs[j].op;
            ok = ok && factorPath[j] && (op == MathOp::Mul || op == MathOp::Div || op == MathOp::Neg);
        }
        factorPath[k] = ok ? 1 : 0;
    }
    auto operandBits = [&](const KernelOperand& o) -> int {
        if (o.kind == K::Const) return constBits(o.constValue);
        if ((o.kind == K::ElemA || o.kind == K::ElemB || o.kind == K::ElemIdx) && elemBits) return elemBits(o);
        return 99;
    };
    std::vector<char> exactMul(exprs.size(), 0);
    for (size_t k = 0; k < exprs.size(); ++k) {
        const KernelExpr& e = exprs[k];
        exactMul[k] = e.op == MathOp::Mul && uses[k] == 1 && operandBits(e.a) + operandBits(e.b) <= 53;
    }
    auto exactTemp = [&](const KernelOperand& o, size_t self) {
        return o.kind == K::Temp && o.index >= 0 && static_cast<size_t>(o.index) < self &&
               exactMul[static_cast<size_t>(o.index)];
    };
    int fastExp = -1;
    if (f32Out) {
        for (size_t k = 0; k < exprs.size() && fastExp < 0; ++k) {
            if (exprs[k].op == MathOp::Exp && factorPath[k] && (k == last || uses[k] == 1)) {
                fastExp = static_cast<int>(k);
            }
        }
    }
    std::string body;
    auto operand = [&](const KernelOperand& o, size_t self, std::string& out) -> bool {
        switch (o.kind) {
            case K::Const: out = literal(o.constValue); return true;
            case K::ElemA:
            case K::ElemB:
            case K::ElemIdx:
                out = elemCode(o);
                return !out.empty();
            case K::ScalarParam:
                if (o.index < 0 || o.index >= MLKD_MAX_SCALARS) return false;
                out = "sc.v[" + std::to_string(o.index) + "]";
                return true;
            case K::Temp:
                if (o.index < 0 || static_cast<size_t>(o.index) >= self) return false;
                out = "t" + std::to_string(o.index);
                return true;
        }
        return false;
    };
    for (size_t k = 0; k < exprs.size(); ++k) {
        const KernelExpr& e = exprs[k];
        std::string a, b = "0.0";
        if (!operand(e.a, k, a)) {
            return err(ErrorCode::UnsupportedCapability,
                       "chain operand not realizable (forward temp, scalar index >= 8 or unbound stream)");
        }
        if (!isUnaryMath(e.op) && !operand(e.b, k, b)) {
            return err(ErrorCode::UnsupportedCapability,
                       "chain operand not realizable (forward temp, scalar index >= 8 or unbound stream)");
        }
        const std::string id = std::to_string(k);
        body += "    const double a" + id + " = " + a + ";\n";
        body += "    const double b" + id + " = " + b + ";\n";
        body += "    (void)b" + id + ";\n";
        const std::string A = "a" + id, B = "b" + id;
        std::string v;
        const bool isLast = k == last;
        // Fused forms of a sum with an exact product t = p*q (its line stays
        // and is dropped as dead code): t + X, X + t, t - X, X - t.
        const bool fuseA = (e.op == MathOp::Add || e.op == MathOp::Sub) && exactTemp(e.a, k);
        const bool fuseB = !fuseA && (e.op == MathOp::Add || e.op == MathOp::Sub) && exactTemp(e.b, k);
        const std::string P = fuseA ? "a" + std::to_string(e.a.index) : "a" + std::to_string(e.b.index);
        const std::string Q = fuseA ? "b" + std::to_string(e.a.index) : "b" + std::to_string(e.b.index);
        switch (e.op) {
            case MathOp::Add:
                if (fuseA) v = "__builtin_fma(" + P + ", " + Q + ", " + B + ")";
                else if (fuseB) v = "__builtin_fma(" + P + ", " + Q + ", " + A + ")";
                else v = A + " + " + B;
                break;
            case MathOp::Sub:
                if (fuseA) v = "__builtin_fma(" + P + ", " + Q + ", -" + B + ")";
                else if (fuseB) v = "__builtin_fma(-" + P + ", " + Q + ", " + A + ")";
                else v = A + " - " + B;
                break;
            case MathOp::Mul: v = A + " * " + B; break;
            case MathOp::Div: v = "(" + B + " != 0.0) ? " + A + " / " + B + " : 0.0"; break;
            case MathOp::Neg: v = "-" + A; break;
            case MathOp::Pow:
                v = "(" + A + " == 2.0 && " + B + " == 2.0) ? " + A + " * " + A + " : pow(" + A + ", " + B + ")";
                break;
            case MathOp::Exp:
                v = static_cast<int>(k) == fastExp ? "mlk_exp_f32acc(" + A + ", slow)" : "exp(" + A + ")";
                break;
            case MathOp::Log: v = "(" + A + " > 0.0) ? log(" + A + ") : 0.0"; break;
            case MathOp::Sin:
                v = poly7 ? ((isLast && f32Out) ? "mlk_p7_sin_f32out(" + A + ", slow)" : "mlk_p7_sin(" + A + ")")
                          : "sin(" + A + ")";
                break;
            case MathOp::Cos: v = "cos(" + A + ")"; break;
            case MathOp::Tan: v = "tan(" + A + ")"; break;
            case MathOp::Tanh: v = "tanh(" + A + ")"; break;
            case MathOp::Sqrt: v = "(" + A + " >= 0.0) ? sqrt(" + A + ") : 0.0"; break;
            case MathOp::Rsqrt: v = "(" + A + " > 0.0) ? 1.0 / sqrt(" + A + ") : 0.0"; break;
            case MathOp::Erf: v = "erf(" + A + ")"; break;
            case MathOp::Gelu:
                v = "0.5 * " + A + " * (1.0 + tanh(0.7978845608028654 * (" + A + " + 0.044715 * " + A +
                    " * " + A + " * " + A + ")))";
                break;
            default: v = "0.0"; break;
        }
        body += "    const double t" + id + " = " + v + ";\n";
    }
    body += "    " + sink + "t" + std::to_string(exprs.size() - 1) + ";\n";
    return body;
}

namespace {

struct NestInfo {
    int depth{0};
    int64_t begin[4]{0, 0, 0, 0};
    int64_t extent[4]{1, 1, 1, 1};
    const KernelNode* compute{nullptr};
    const KernelNode* store{nullptr};
};

/// Constant bounds of a loop (the walker's bound rules, :579-601, minus the
/// affine forms, which a perfect rectangular nest does not use).
bool constBounds(const KernelModule& km, const KernelNode& n, int64_t& b, int64_t& e) {
    if (n.step != 1 || !n.beginCoeffs.empty() || !n.endCoeffs.empty()) return false;
    b = n.begin;
    if (n.end == kDynamicBound) {
        if (n.endBuf == kInvalidId || n.endBuf >= km.buffers.size() || n.endDim < 0 ||
            n.endDim >= static_cast<int32_t>(km.buffers[n.endBuf].dims.size())) {
            return false;
        }
        e = km.buffers[n.endBuf].dims[static_cast<size_t>(n.endDim)];
    } else {
        e = n.end;
    }
    return true;
}

/// Perfect nest: Loop -> Loop -> ... -> Loop{Compute, Store}.
bool perfectNest(const KernelModule& km, uint32_t root, NestInfo& ni) {
    uint32_t cur = root;
    for (;;) {
        if (cur >= km.nodes.size() || ni.depth >= 4) return false;
        const KernelNode& n = km.nodes[cur];
        if (n.op != KernelOp::Loop) return false;
        int64_t b = 0, e = 0;
        if (!constBounds(km, n, b, e)) return false;
        ni.begin[ni.depth] = b;
        ni.extent[ni.depth] = e - b;
        ++ni.depth;
        if (n.children.size() == 1) {
            cur = n.children[0];
            continue;
        }
        if (n.children.size() != 2) return false;
        const uint32_t c0 = n.children[0], c1 = n.children[1];
        if (c0 >= km.nodes.size() || c1 >= km.nodes.size()) return false;
        if (km.nodes[c0].op != KernelOp::Compute || km.nodes[c1].op != KernelOp::Store) return false;
        ni.compute = &km.nodes[c0];
        ni.store = &km.nodes[c1];
        return true;
    }
}

/// Normalizes an ElemIdx (or store) map onto box-relative variables.
StreamRef mapRef(uint32_t buffer, const std::vector<int64_t>& coeffs, int64_t offset,
                 const NestInfo& ni) {
    StreamRef s;
    s.buffer = buffer;
    s.offset = offset;
    for (int d = 0; d < ni.depth && d < static_cast<int>(coeffs.size()); ++d) {
        s.coeff[d] = coeffs[static_cast<size_t>(d)];
        s.offset += coeffs[static_cast<size_t>(d)] * ni.begin[d];
    }
    return s;
}

Result<void> checkInBounds(const KernelModule& km, const StreamRef& s, int rank, const int64_t* ext,
                           const char* role) {
    if (s.buffer >= km.buffers.size()) return err(ErrorCode::InvalidGraph, std::string(role) + " buffer id out of range");
    const int64_t n = bufElems(km.buffers[s.buffer]);
    int64_t lo = 0, hi = 0;
    affineRange(s, rank, ext, lo, hi);
    if (n <= 0 || lo < 0 || hi >= n) {
        return err(ErrorCode::InvalidGraph,
                   std::string(role) + " reaches outside its buffer (" + std::to_string(lo) + ".." +
                       std::to_string(hi) + " of " + std::to_string(n) + " elements)");
    }
    return {};
}

/// Elementwise step over a perfect nest (poly.synth broadcast form, or any
/// rectangular nest with an injective output map).
Result<Step> elementwiseNest(const KernelModule& km, const NestInfo& ni) {
    Step st;
    st.kind = StepKind::Elementwise;
    st.what = "elementwise-nd";
    st.rank = ni.depth;
    for (int d = 0; d < ni.depth; ++d) st.extent[d] = ni.extent[d];
    for (int d = 0; d < ni.depth; ++d) {
        if (st.extent[d] <= 0) {
            st.kind = StepKind::Fail;  // empty loop: nothing executes
            st.what = "empty";
            return st;
        }
    }
    const KernelNode& cp = *ni.compute;
    const KernelNode& so = *ni.store;
    for (const KernelExpr& e : cp.exprs) {
        for (const KernelOperand* o : {&e.a, &e.b}) {
            if (o->kind == K::ElemA || o->kind == K::ElemB) {
                return err(ErrorCode::InvalidGraph, "walker: legacy element operand in a multi-dim compute");
            }
        }
    }
    if (so.bufferOut >= km.buffers.size()) return err(ErrorCode::InvalidArgument, "walker: output buffer not bound");
    st.out = mapRef(so.bufferOut, so.outIndexCoeffs, so.outIndexOffset, ni);
    st.accum = so.accum;
    {
        int64_t lo = 0, hi = 0;
        affineRange(st.out, st.rank, st.extent, lo, hi);
        if (lo < 0) {
            st.kind = StepKind::Fail;
            st.what = "negative-store";
            st.failCode = 1;
            return st;
        }
    }
    MLK_TRYV(checkInBounds(km, st.out, st.rank, st.extent, "store"));
    if (!injective(st.out, st.rank, st.extent)) {
        return err(ErrorCode::UnsupportedCapability,
                   "store map is not injective over the nest (a reduction, not an elementwise class)");
    }
    std::vector<StreamRef>& ins = st.inputs;
    bool bad = false;
    auto streamOf = [&](const KernelOperand& o) -> int {
        if (o.kind != K::ElemIdx || o.index < 0 || static_cast<size_t>(o.index) >= km.buffers.size()) {
            bad = true;
            return -1;
        }
        const StreamRef s = mapRef(static_cast<uint32_t>(o.index), o.idxCoeffs, o.idxOffset, ni);
        for (size_t i = 0; i < ins.size(); ++i) {
            if (sameMap(ins[i], s, st.rank)) return static_cast<int>(i);
        }
        if (ins.size() >= 4) {
            bad = true;
            return -1;
        }
        ins.push_back(s);
        return static_cast<int>(ins.size() - 1);
    };
    const Dtype od = km.buffers[so.bufferOut].dtype;
    // Split-precision sin only where its result is rounded to f32. An f16
    // output keeps the exact f64 form: its one rounding then gives the
    // reference's f16 value bit for bit, where a few f32 ULP of error would
    // move about one value in a thousand to the neighbouring f16.
    const bool f32Out = od == Dtype::F32 && so.accum == AccumMode::None;
    auto bits = [&km](const KernelOperand& o) {
        return o.kind == K::ElemIdx ? streamBits(km, o.index) : 99;
    };
    auto exact = chainCode(cp.exprs, cp.family == "poly7", false, streamCode(streamOf), "return ", bits);
    if (!exact.has_value()) return err(exact.error().code, exact.error().message);
    // The fast forms' exact pass re-reads its inputs after the vector stores.
    // A chain that reads the buffer it stores would re-read its own results,
    // so it runs the exact forms from the start.
    bool inPlace = false;
    for (const StreamRef& s : ins) inPlace = inPlace || s.buffer == so.bufferOut;
    auto body = inPlace ? exact
                        : chainCode(cp.exprs, cp.family == "poly7", f32Out, streamCode(streamOf), "return ", bits);
    if (!body.has_value()) return err(body.error().code, body.error().message);
    if (*exact != *body) st.chainExact = *exact;
    if (bad) return err(ErrorCode::UnsupportedCapability, "more than 4 distinct element streams");
    for (const StreamRef& s : ins) {
        MLK_TRYV(checkInBounds(km, s, st.rank, st.extent, "operand"));
        if (s.buffer == so.bufferOut && !sameMap(s, st.out, st.rank)) {
            return err(ErrorCode::UnsupportedCapability,
                       "operand reads the stored buffer at another element (loop-carried)");
        }
    }
    st.chainBody = *body;
    return st;
}

/// Tier-1 Loop: each Compute child with the first Store child
/// (kernel_buffers.cpp:921-1000, runElementwiseRange :342-402).
/// Buffer id the reference's 1-D executor reaches for `bid` (resolveInput /
/// resolveOutput in runtime/src/execution/kernel_buffers.cpp): its bindings
/// hold the input buffers, then the output buffers, each in id order, and it
/// indexes them by the id itself. kInvalidId where that index has no binding.
uint32_t resolve1d(const KernelModule& km, uint32_t bid, bool store) {
    if (bid == kInvalidId || bid >= km.buffers.size()) return kInvalidId;
    std::vector<uint32_t> ins, outs;
    for (uint32_t b = 0; b < km.buffers.size(); ++b) {
        if (km.buffers[b].isInput) ins.push_back(b);
        if (km.buffers[b].isOutput) outs.push_back(b);
    }
    const bool viaOutputs = store ? km.buffers[bid].isOutput : !km.buffers[bid].isInput;
    if (viaOutputs) {
        if (bid < ins.size()) return kInvalidId;
        const size_t o = bid - ins.size();
        return o < outs.size() ? outs[o] : kInvalidId;
    }
    return bid < ins.size() ? ins[bid] : kInvalidId;
}

/// The multi-dim walker reaches every non-temp buffer through the same
/// position lookup (kernel_buffers.cpp elemPtr :85-103, the store target in
/// execPair :730-737, the call executors :784-812 and their softmax /
/// reducesum twins), and temps by id. The multi-dim steps bind buffers by
/// id; for the tables the lowering emits (inputs, then outputs, then temps,
/// each in id order) the two agree. A module where a lookup lands on another
/// buffer than its id, or where an operand finds no binding (the walker
/// would read zeros), is declined. A store or call target that finds no
/// binding is the walker's InvalidArgument, raised here at plan time.
Result<void> walkerPositions(const KernelModule& km) {
    // One entry per lookup the walker makes: buffer id, store role, temps by
    // id, and the error an unbound lookup raises (nullptr: the walker reads
    // zeros instead).
    struct Lookup {
        uint32_t bid;
        bool store, tempById;
        const char* unbound;
    };
    std::vector<Lookup> looks;
    for (const KernelNode& n : km.nodes) {
        if (n.op == KernelOp::Store) {
            looks.push_back({n.bufferOut, true, true, "walker: output buffer not bound"});
        } else if (n.op == KernelOp::Call &&
                   (n.math == MathOp::MatMul || n.math == MathOp::Softmax || n.math == MathOp::ReduceSum)) {
            const char* msg = n.math == MathOp::MatMul    ? "matmul buffers not bound by the caller"
                              : n.math == MathOp::Softmax ? "softmax buffers not bound by the caller"
                                                          : "reducesum buffers not bound by the caller";
            looks.push_back({n.bufferA, false, false, msg});
            if (n.math == MathOp::MatMul) looks.push_back({n.bufferB, false, false, msg});
            looks.push_back({n.bufferOut, true, false, msg});
        } else if (n.op == KernelOp::Compute) {
            for (const KernelExpr& e : n.exprs) {
                for (const KernelOperand* o : {&e.a, &e.b}) {
                    if (o->kind == K::ElemIdx && o->index >= 0) {
                        looks.push_back({static_cast<uint32_t>(o->index), false, true, nullptr});
                    }
                }
            }
        }
    }
    auto resolved = [&km](const Lookup& l) {
        if (l.bid >= km.buffers.size()) return l.bid;  // range errors come from the step builders
        if (l.tempById && km.buffers[l.bid].isTemp) return l.bid;
        return resolve1d(km, l.bid, l.store);
    };
    // Errors before declines: an unbound target ends the walker's run
    // whatever the other roots would have read.
    for (const Lookup& l : looks) {
        if (l.unbound != nullptr && resolved(l) == kInvalidId) return err(ErrorCode::InvalidArgument, l.unbound);
    }
    for (const Lookup& l : looks) {
        if (resolved(l) != l.bid) {
            return err(ErrorCode::UnsupportedCapability,
                       "buffer '" + km.buffers[l.bid].name + "' resolves by position to another binding than its id");
        }
    }
    return {};
}

Result<std::vector<Step>> tier1Loop(const KernelModule& km, const KernelNode& loop) {
    std::vector<Step> out;
    const KernelNode* store = nullptr;
    for (const uint32_t sid : loop.children) {
        if (sid < km.nodes.size() && km.nodes[sid].op == KernelOp::Store) {
            store = &km.nodes[sid];
            break;
        }
    }
    for (const uint32_t cid : loop.children) {
        if (cid >= km.nodes.size()) return err(ErrorCode::InvalidGraph, "kernel child node out of range");
    }
    for (const uint32_t cid : loop.children) {
        const KernelNode& c = km.nodes[cid];
        if (c.op != KernelOp::Compute) continue;
        const KernelNode& so = store != nullptr ? *store : c;
        bool needsA = c.exprs.empty(), needsB = c.exprs.empty();
        for (const KernelExpr& e : c.exprs) {
            for (const KernelOperand* o : {&e.a, &e.b}) {
                needsA = needsA || o->kind == K::ElemA;
                needsB = needsB || o->kind == K::ElemB;
            }
        }
        // The 1-D path resolves buffer ids by position, as the reference's
        // executor does (kernel_buffers.cpp resolveInput / resolveOutput): an
        // input id indexes the inputs, any other operand id the outputs after
        // them; an output id indexes the outputs after the inputs, any other
        // store id the inputs. For modules laid out inputs first, outputs
        // after (lower.to_kernel_ir's), that is the id itself.
        const uint32_t bufA = resolve1d(km, c.bufferA, false);
        const uint32_t bufB = resolve1d(km, c.bufferB, false);
        const uint32_t bufOut = resolve1d(km, so.bufferOut, true);
        // Unresolved operands or output: the reference skips the pair.
        if (bufOut == kInvalidId || (needsA && bufA == kInvalidId) || (needsB && bufB == kInvalidId)) continue;
        Step st;
        st.kind = StepKind::Elementwise;
        st.what = "elementwise-1d";
        st.rank = 1;
        int64_t begin = loop.begin;
        int64_t end = loop.end;
        if (end == kDynamicBound) {
            st.dynamicExtent = true;
            st.dynBegin = begin;
        } else {
            if (end < begin) end = begin;
            st.extent[0] = end - begin;
        }
        std::vector<KernelExpr> exprs = c.exprs;
        if (exprs.empty()) {  // legacy single op over ElemA, ElemB
            KernelExpr e;
            e.op = c.math;
            e.a.kind = K::ElemA;
            e.b.kind = K::ElemB;
            exprs.push_back(e);
        }
        auto ref = [&](uint32_t bid) {
            StreamRef s;
            s.buffer = bid;
            s.offset = st.dynamicExtent ? 0 : begin;
            s.coeff[0] = 1;
            return s;
        };
        int slotA = -1, slotB = -1;
        auto streamOf = [&](const KernelOperand& o) -> int {
            if (o.kind == K::ElemA) {
                if (slotA < 0) {
                    st.inputs.push_back(ref(bufA));
                    slotA = static_cast<int>(st.inputs.size() - 1);
                }
                return slotA;
            }
            if (o.kind == K::ElemB) {
                if (slotB < 0) {
                    st.inputs.push_back(ref(bufB));
                    slotB = static_cast<int>(st.inputs.size() - 1);
                }
                return slotB;
            }
            return -1;  // ElemIdx is a multi-dim operand
        };
        const Dtype od = km.buffers[bufOut].dtype;
        // Split-precision sin for f32 outputs only, as in the n-D path.
        auto bits = [&](const KernelOperand& o) {
            return o.kind == K::ElemA ? streamBits(km, bufA == kInvalidId ? -1 : static_cast<int64_t>(bufA))
                                      : (o.kind == K::ElemB ? streamBits(km, bufB == kInvalidId ? -1 : static_cast<int64_t>(bufB)) : 99);
        };
        auto exact = chainCode(exprs, c.family == "poly7", false, streamCode(streamOf), "return ", bits);
        if (!exact.has_value()) return err(exact.error().code, exact.error().message);
        // In place: exact forms throughout, as in the n-D path (the fast
        // forms' exact pass would re-read stored results).
        bool inPlace = false;
        for (const StreamRef& s : st.inputs) inPlace = inPlace || s.buffer == bufOut;
        auto body = inPlace ? exact
                            : chainCode(exprs, c.family == "poly7", od == Dtype::F32, streamCode(streamOf), "return ", bits);
        if (!body.has_value()) return err(body.error().code, body.error().message);
        st.chainBody = *body;
        if (*exact != *body) st.chainExact = *exact;
        st.out = ref(bufOut);
        if (!st.dynamicExtent) {
            if (st.extent[0] == 0) continue;
            if (begin < 0) return err(ErrorCode::InvalidGraph, "1-D loop begins below element 0");
            for (const StreamRef& s : st.inputs) {
                MLK_TRYV(checkInBounds(km, s, 1, st.extent, "1-D operand"));
            }
            MLK_TRYV(checkInBounds(km, st.out, 1, st.extent, "1-D store"));
        }
        out.push_back(std::move(st));
    }
    return out;
}

Result<Step> callStep(const KernelModule& km, const KernelNode& top, bool walker) {
    Step st;
    if (!walker) {
        // The Tier-1 call executors take their data through the same
        // position-based lookup as the 1-D path (kernel_buffers.cpp
        // resolveInput / resolveOutput) and their shapes from the ids'
        // buffers. A lookup that finds no binding is the reference's
        // InvalidArgument; one that lands on another buffer than the id is
        // refused rather than run on mismatched shapes.
        const bool mm = top.math == MathOp::MatMul;
        const uint32_t ids[3] = {top.bufferA, mm ? top.bufferB : kInvalidId, top.bufferOut};
        for (int i = 0; i < 3; ++i) {
            if (ids[i] == kInvalidId || ids[i] >= km.buffers.size()) continue;   // checked below
            const uint32_t r = resolve1d(km, ids[i], i == 2);
            if (r == kInvalidId) return err(ErrorCode::InvalidArgument, "call buffers not bound by the caller");
            if (r != ids[i]) {
                return err(ErrorCode::UnsupportedCapability,
                           "call buffer resolves by position to another buffer than its id");
            }
        }
    }
    if (top.math == MathOp::MatMul) {
        if (top.bufferA >= km.buffers.size() || top.bufferB >= km.buffers.size() ||
            top.bufferOut >= km.buffers.size()) {
            return err(ErrorCode::InvalidGraph, "matmul buffer id out of range");
        }
        const auto& da = km.buffers[top.bufferA].dims;
        const auto& db = km.buffers[top.bufferB].dims;
        const auto& dc = km.buffers[top.bufferOut].dims;
        if (da.size() != 2 || db.size() != 2 || dc.size() != 2) {
            return err(ErrorCode::InvalidGraph, "matmul requires rank-2 buffer dims");
        }
        const int64_t m = da[0], k = da[1];
        const int64_t n = walker ? dc[1] : db[1];
        if (db[0] != k || dc[0] != m || dc[1] != n) return err(ErrorCode::InvalidGraph, "matmul operand shapes incompatible");
        if (walker && db[1] != n) {
            return err(ErrorCode::UnsupportedCapability, "matmul with B columns != C columns");
        }
        st.kind = StepKind::Gemm;
        st.what = "gemm-call";
        st.a = top.bufferA;
        st.b = top.bufferB;
        st.c = top.bufferOut;
        st.m = m;
        st.n = n;
        st.k = k;
        st.lda = k;
        st.ldb = n;
        st.ldc = n;
        st.accumulate = true;  // gemmRowBlock accumulates into C (:406-432)
        st.skipZeroA = true;   // ... and skips A[i,p] == 0 (:422)
        return st;
    }
    if (top.math == MathOp::Softmax || top.math == MathOp::ReduceSum) {
        const bool soft = top.math == MathOp::Softmax;
        if (top.bufferA >= km.buffers.size() || top.bufferOut >= km.buffers.size()) {
            return err(ErrorCode::InvalidGraph, soft ? "softmax buffer id out of range" : "reducesum buffer id out of range");
        }
        const auto& da = km.buffers[top.bufferA].dims;
        const auto& dy = km.buffers[top.bufferOut].dims;
        if (da.size() != 2 || dy.size() != (soft ? 2u : 1u)) {
            return err(ErrorCode::InvalidGraph, soft ? "softmax requires rank-2 operand and output"
                                                     : "reducesum requires rank-2 input over rank-1 output");
        }
        const int64_t m = da[0], k = da[1];
        if (dy[0] != m || (soft && dy[1] != k) || k <= 0 || m <= 0) {
            return err(ErrorCode::InvalidGraph, soft ? "softmax operand shapes incompatible" : "reducesum operand shapes incompatible");
        }
        st.kind = soft ? StepKind::Softmax : StepKind::RowSum;
        st.what = soft ? "softmax-call" : "reducesum-call";
        st.x = top.bufferA;
        st.y = top.bufferOut;
        st.rows = m;
        st.cols = k;
        return st;
    }
    return err(ErrorCode::UnsupportedCapability, "no executor for call target");
}

// ---------------------------------------------------------- patterns ----
const KernelNode* node(const KernelModule& km, uint32_t id) {
    return id < km.nodes.size() ? &km.nodes[id] : nullptr;
}

bool isLoop0(const KernelNode* n, int64_t& extent) {
    if (n == nullptr || n->op != KernelOp::Loop || n->step != 1 || n->begin != 0 ||
        !n->beginCoeffs.empty() || !n->endCoeffs.empty() || n->end <= 0) {
        return false;
    }
    extent = n->end;
    return true;
}

bool isConstStore(const KernelNode* c, double value) {
    if (c == nullptr || c->op != KernelOp::Compute || c->exprs.size() != 1) return false;
    const KernelExpr& e = c->exprs[0];
    if (e.op != MathOp::Add || e.a.kind != K::Const || e.b.kind != K::Const || e.b.constValue != 0.0) return false;
    if (std::isinf(value)) return std::isinf(e.a.constValue) && (e.a.constValue < 0) == (value < 0);
    return e.a.constValue == value;
}

bool elemIs(const KernelOperand& o, uint32_t buf, std::initializer_list<int64_t> coeffs) {
    if (o.kind != K::ElemIdx || o.index != static_cast<int64_t>(buf) || o.idxOffset != 0) return false;
    if (o.idxCoeffs.size() != coeffs.size()) return false;
    size_t i = 0;
    for (const int64_t c : coeffs) {
        if (o.idxCoeffs[i++] != c) return false;
    }
    return true;
}

bool storeIs(const KernelNode* s, uint32_t buf, std::initializer_list<int64_t> coeffs, AccumMode acc) {
    if (s == nullptr || s->op != KernelOp::Store || s->bufferOut != buf || s->outIndexOffset != 0 || s->accum != acc) {
        return false;
    }
    if (s->outIndexCoeffs.size() != coeffs.size()) return false;
    size_t i = 0;
    for (const int64_t c : coeffs) {
        if (s->outIndexCoeffs[i++] != c) return false;
    }
    return true;
}

bool isPassThrough(const KernelExpr& e, uint32_t buf, std::initializer_list<int64_t> coeffs) {
    // Sub(x, 0) is the exact passthrough of the softmax nest; Add(x, 0) the
    // GEMM operand load (which maps -0.0 to +0.0, immaterial to a product).
    return (e.op == MathOp::Sub || e.op == MathOp::Add) && e.b.kind == K::Const && e.b.constValue == 0.0 &&
           elemIs(e.a, buf, coeffs);
}

/// True when a node outside the subtrees of `own` reads or writes one of
/// `bufs` (an ElemIdx operand, a legacy Compute operand, a Store or Call
/// target). A fused class that keeps those buffers on chip must own every
/// access to them: the walker would hand any other access the values the
/// statements stored (kernel_buffers.cpp:902-920), where a fused launch never
/// materializes them.
bool touchedOutside(const KernelModule& km, std::initializer_list<uint32_t> own,
                    std::initializer_list<uint32_t> bufs) {
    std::vector<bool> inside(km.nodes.size(), false);
    std::vector<uint32_t> work(own.begin(), own.end());
    while (!work.empty()) {
        const uint32_t id = work.back();
        work.pop_back();
        if (id >= km.nodes.size() || inside[id]) continue;
        inside[id] = true;
        for (const uint32_t c : km.nodes[id].children) work.push_back(c);
    }
    auto hit = [&](int64_t b) {
        for (const uint32_t t : bufs) {
            if (b == static_cast<int64_t>(t)) return true;
        }
        return false;
    };
    for (uint32_t id = 0; id < km.nodes.size(); ++id) {
        if (inside[id]) continue;
        const KernelNode& n = km.nodes[id];
        if (n.op == KernelOp::Compute || n.op == KernelOp::Store || n.op == KernelOp::Call) {
            for (const uint32_t b : {n.bufferA, n.bufferB, n.bufferOut}) {
                if (b != kInvalidId && hit(b)) return true;
            }
        }
        for (const KernelExpr& e : n.exprs) {
            for (const KernelOperand* o : {&e.a, &e.b}) {
                if (o->kind == K::ElemIdx && hit(o->index)) return true;
            }
        }
    }
    return false;
}

/// poly.synth softmax nest (:363-523): m{ RM=-inf; k{RM max= x}; k{E=exp(x-RM)};
/// S=0; k{S += E}; k{Y = E/S} }.
bool matchSoftmaxNest(const KernelModule& km, uint32_t root, Step& st) {
    const KernelNode* ml = node(km, root);
    int64_t M = 0;
    if (!isLoop0(ml, M) || ml->children.size() != 8) return false;
    const auto& ch = ml->children;
    const KernelNode* c0 = node(km, ch[0]);
    const KernelNode* s0 = node(km, ch[1]);
    const KernelNode* lRM = node(km, ch[2]);
    const KernelNode* lE = node(km, ch[3]);
    const KernelNode* c3 = node(km, ch[4]);
    const KernelNode* s3 = node(km, ch[5]);
    const KernelNode* lS = node(km, ch[6]);
    const KernelNode* lD = node(km, ch[7]);
    if (s0 == nullptr || s3 == nullptr) return false;
    const uint32_t rm = s0->bufferOut, sm = s3->bufferOut;
    if (!isConstStore(c0, -INFINITY) || !storeIs(s0, rm, {1}, AccumMode::None)) return false;
    if (!isConstStore(c3, 0.0) || !storeIs(s3, sm, {1}, AccumMode::None)) return false;
    int64_t K1 = 0, K2 = 0, K3 = 0, K4 = 0;
    if (!isLoop0(lRM, K1) || !isLoop0(lE, K2) || !isLoop0(lS, K3) || !isLoop0(lD, K4)) return false;
    if (K1 != K2 || K1 != K3 || K1 != K4) return false;
    for (const KernelNode* l : {lRM, lE, lS, lD}) {
        if (l->children.size() != 2) return false;
    }
    const KernelNode* c1 = node(km, lRM->children[0]);
    const KernelNode* s1 = node(km, lRM->children[1]);
    const KernelNode* c2 = node(km, lE->children[0]);
    const KernelNode* s2 = node(km, lE->children[1]);
    const KernelNode* c4 = node(km, lS->children[0]);
    const KernelNode* s4 = node(km, lS->children[1]);
    const KernelNode* c5 = node(km, lD->children[0]);
    const KernelNode* s5 = node(km, lD->children[1]);
    for (const KernelNode* c : {c1, c2, c4, c5}) {
        if (c == nullptr || c->op != KernelOp::Compute) return false;
    }
    if (c1->exprs.size() != 1 || c2->exprs.size() != 2 || c4->exprs.size() != 1 || c5->exprs.size() != 1) return false;
    const KernelOperand& xo = c1->exprs[0].a;
    if (xo.kind != K::ElemIdx || xo.index < 0 || static_cast<size_t>(xo.index) >= km.buffers.size()) return false;
    const uint32_t x = static_cast<uint32_t>(xo.index);
    const int64_t K = K1;
    if (!isPassThrough(c1->exprs[0], x, {K, 1}) || c1->exprs[0].op != MathOp::Sub) return false;
    if (!storeIs(s1, rm, {1, 0}, AccumMode::Max)) return false;
    const KernelExpr& e20 = c2->exprs[0];
    const KernelExpr& e21 = c2->exprs[1];
    if (e20.op != MathOp::Sub || !elemIs(e20.a, x, {K, 1}) || !elemIs(e20.b, rm, {1, 0})) return false;
    if (e21.op != MathOp::Exp || e21.a.kind != K::Temp || e21.a.index != 0) return false;
    if (s2 == nullptr || s2->op != KernelOp::Store) return false;
    const uint32_t eb = s2->bufferOut;
    if (!storeIs(s2, eb, {K, 1}, AccumMode::None)) return false;
    if (!isPassThrough(c4->exprs[0], eb, {K, 1}) || c4->exprs[0].op != MathOp::Sub) return false;
    if (!storeIs(s4, sm, {1, 0}, AccumMode::Add)) return false;
    const KernelExpr& e5 = c5->exprs[0];
    if (e5.op != MathOp::Div || !elemIs(e5.a, eb, {K, 1}) || !elemIs(e5.b, sm, {1, 0})) return false;
    if (s5 == nullptr || s5->op != KernelOp::Store) return false;
    const uint32_t y = s5->bufferOut;
    if (!storeIs(s5, y, {K, 1}, AccumMode::None)) return false;
    // The three scratch buffers must be temps, sized as the statements
    // address them, that no other root touches; x and y must hold M*K
    // elements.
    for (const uint32_t t : {rm, eb, sm}) {
        if (t >= km.buffers.size() || !km.buffers[t].isTemp) return false;
    }
    if (bufElems(km.buffers[rm]) < M || bufElems(km.buffers[sm]) < M || bufElems(km.buffers[eb]) < M * K) return false;
    if (y >= km.buffers.size() || bufElems(km.buffers[x]) < M * K || bufElems(km.buffers[y]) < M * K) return false;
    if (x == rm || x == eb || x == sm || y == rm || y == eb || y == sm) return false;
    if (touchedOutside(km, {root}, {rm, eb, sm})) return false;
    st.kind = StepKind::Softmax;
    st.what = "softmax-nest";
    st.x = x;
    st.y = y;
    st.rows = M;
    st.cols = K;
    return true;
}

/// poly.synth ReduceSum nest (:153-229): i{ Y=0; k{ Y += A } }.
bool matchReduceSumNest(const KernelModule& km, uint32_t root, Step& st) {
    const KernelNode* il = node(km, root);
    int64_t M = 0, Kx = 0;
    if (!isLoop0(il, M) || il->children.size() != 3) return false;
    const KernelNode* c0 = node(km, il->children[0]);
    const KernelNode* s0 = node(km, il->children[1]);
    const KernelNode* kl = node(km, il->children[2]);
    if (s0 == nullptr || !isConstStore(c0, 0.0)) return false;
    const uint32_t y = s0->bufferOut;
    if (!storeIs(s0, y, {1}, AccumMode::None)) return false;
    if (!isLoop0(kl, Kx) || kl->children.size() != 2) return false;
    const KernelNode* c1 = node(km, kl->children[0]);
    const KernelNode* s1 = node(km, kl->children[1]);
    if (c1 == nullptr || c1->op != KernelOp::Compute || c1->exprs.size() != 1) return false;
    const KernelOperand& xo = c1->exprs[0].a;
    if (xo.kind != K::ElemIdx || xo.index < 0 || static_cast<size_t>(xo.index) >= km.buffers.size()) return false;
    const uint32_t x = static_cast<uint32_t>(xo.index);
    if (c1->exprs[0].op != MathOp::Add || !isPassThrough(c1->exprs[0], x, {Kx, 1})) return false;
    if (!storeIs(s1, y, {1, 0}, AccumMode::Add)) return false;
    if (x == y || bufElems(km.buffers[x]) < M * Kx || y >= km.buffers.size() || bufElems(km.buffers[y]) < M) return false;
    st.kind = StepKind::RowSum;
    st.what = "reducesum-nest";
    st.x = x;
    st.y = y;
    st.rows = M;
    st.cols = Kx;
    return true;
}

/// poly.synth GEMM nest (:58-147): i{ j{ C=0; k{ C += A[i,k]*B[k,j] } } }.
bool matchGemmNest(const KernelModule& km, uint32_t root, Step& st) {
    const KernelNode* il = node(km, root);
    int64_t M = 0, N = 0, Kx = 0;
    if (!isLoop0(il, M) || il->children.size() != 1) return false;
    const KernelNode* jl = node(km, il->children[0]);
    if (!isLoop0(jl, N) || jl->children.size() != 3) return false;
    const KernelNode* c0 = node(km, jl->children[0]);
    const KernelNode* s0 = node(km, jl->children[1]);
    const KernelNode* kl = node(km, jl->children[2]);
    if (s0 == nullptr || c0 == nullptr || c0->op != KernelOp::Compute || c0->exprs.size() != 1) return false;
    const KernelExpr& z = c0->exprs[0];
    if (z.op != MathOp::Add || z.a.kind != K::Const || z.a.constValue != 0.0 || z.b.kind != K::Const ||
        z.b.constValue != 0.0) {
        return false;
    }
    const uint32_t c = s0->bufferOut;
    if (!storeIs(s0, c, {N, 1}, AccumMode::None)) return false;
    if (!isLoop0(kl, Kx) || kl->children.size() != 2) return false;
    const KernelNode* c1 = node(km, kl->children[0]);
    const KernelNode* s1 = node(km, kl->children[1]);
    if (c1 == nullptr || c1->op != KernelOp::Compute || c1->exprs.size() != 3) return false;
    const KernelOperand& ao = c1->exprs[0].a;
    const KernelOperand& bo = c1->exprs[1].a;
    if (ao.kind != K::ElemIdx || bo.kind != K::ElemIdx || ao.index < 0 || bo.index < 0 ||
        static_cast<size_t>(ao.index) >= km.buffers.size() || static_cast<size_t>(bo.index) >= km.buffers.size()) {
        return false;
    }
    const uint32_t a = static_cast<uint32_t>(ao.index), b = static_cast<uint32_t>(bo.index);
    if (!isPassThrough(c1->exprs[0], a, {Kx, 0, 1}) || c1->exprs[0].op != MathOp::Add) return false;
    if (!isPassThrough(c1->exprs[1], b, {0, 1, N}) || c1->exprs[1].op != MathOp::Add) return false;
    const KernelExpr& mul = c1->exprs[2];
    if (mul.op != MathOp::Mul || mul.a.kind != K::Temp || mul.a.index != 0 || mul.b.kind != K::Temp || mul.b.index != 1) {
        return false;
    }
    if (!storeIs(s1, c, {N, 1, 0}, AccumMode::Add)) return false;
    if (c >= km.buffers.size() || c == a || c == b) return false;
    if (bufElems(km.buffers[a]) < M * Kx || bufElems(km.buffers[b]) < Kx * N || bufElems(km.buffers[c]) < M * N) return false;
    st.kind = StepKind::Gemm;
    st.what = "gemm-nest";
    st.a = a;
    st.b = b;
    st.c = c;
    st.m = M;
    st.n = N;
    st.k = Kx;
    st.lda = Kx;
    st.ldb = N;
    st.ldc = N;
    st.accumulate = false;  // S0 zeroes C first
    return true;
}

/// Batched score nest: b{ i{ j{ SC=0; k{ SC += Q[b,i,k]*K[b,j,k] } } } } over
/// a temp SC[batch*seq, seq]; then r{ j{ SC = Add(Div(SC, c), bias[j]) } };
/// then the softmax nest over SC rows into S. Fused into one launch.
bool matchScoreSoftmax(const KernelModule& km, const std::vector<uint32_t>& roots, size_t at, Step& st) {
    if (at + 2 >= roots.size()) return false;
    const KernelNode* bl = node(km, roots[at]);
    int64_t B = 0, S = 0, S2 = 0, D = 0;
    if (!isLoop0(bl, B) || bl->children.size() != 1) return false;
    const KernelNode* il = node(km, bl->children[0]);
    if (!isLoop0(il, S) || il->children.size() != 1) return false;
    const KernelNode* jl = node(km, il->children[0]);
    if (!isLoop0(jl, S2) || S2 != S || jl->children.size() != 3) return false;
    const KernelNode* c0 = node(km, jl->children[0]);
    const KernelNode* s0 = node(km, jl->children[1]);
    const KernelNode* kl = node(km, jl->children[2]);
    if (s0 == nullptr || c0 == nullptr || c0->op != KernelOp::Compute || c0->exprs.size() != 1) return false;
    const KernelExpr& z = c0->exprs[0];
    if (z.op != MathOp::Add || z.a.kind != K::Const || z.a.constValue != 0.0 || z.b.kind != K::Const ||
        z.b.constValue != 0.0) {
        return false;
    }
    const uint32_t sc = s0->bufferOut;
    if (!storeIs(s0, sc, {S * S, S, 1}, AccumMode::None)) return false;
    if (!isLoop0(kl, D) || kl->children.size() != 2) return false;
    const KernelNode* c1 = node(km, kl->children[0]);
    const KernelNode* s1 = node(km, kl->children[1]);
    if (c1 == nullptr || c1->op != KernelOp::Compute || c1->exprs.size() != 3) return false;
    const KernelOperand& qo = c1->exprs[0].a;
    const KernelOperand& ko = c1->exprs[1].a;
    if (qo.kind != K::ElemIdx || ko.kind != K::ElemIdx || qo.index < 0 || ko.index < 0 ||
        static_cast<size_t>(qo.index) >= km.buffers.size() || static_cast<size_t>(ko.index) >= km.buffers.size()) {
        return false;
    }
    const uint32_t q = static_cast<uint32_t>(qo.index), kb = static_cast<uint32_t>(ko.index);
    if (!isPassThrough(c1->exprs[0], q, {S * D, D, 0, 1}) || c1->exprs[0].op != MathOp::Add) return false;
    if (!isPassThrough(c1->exprs[1], kb, {S * D, 0, D, 1}) || c1->exprs[1].op != MathOp::Add) return false;
    const KernelExpr& mul = c1->exprs[2];
    if (mul.op != MathOp::Mul || mul.a.kind != K::Temp || mul.a.index != 0 || mul.b.kind != K::Temp || mul.b.index != 1) {
        return false;
    }
    if (!storeIs(s1, sc, {S * S, S, 1, 0}, AccumMode::Add)) return false;
    if (sc >= km.buffers.size() || !km.buffers[sc].isTemp) return false;
    // Root 2: r{ j{ SC = Add(Div(SC, c), bias[j]) } }.
    NestInfo ni;
    if (!perfectNest(km, roots[at + 1], ni) || ni.depth != 2 || ni.begin[0] != 0 || ni.begin[1] != 0 ||
        ni.extent[0] != B * S || ni.extent[1] != S) {
        return false;
    }
    const KernelNode& ec = *ni.compute;
    if (ec.exprs.size() != 2 || !storeIs(ni.store, sc, {S, 1}, AccumMode::None)) return false;
    const KernelExpr& dv = ec.exprs[0];
    const KernelExpr& ad = ec.exprs[1];
    if (dv.op != MathOp::Div || !elemIs(dv.a, sc, {S, 1}) || dv.b.kind != K::Const || dv.b.constValue == 0.0) return false;
    if (ad.op != MathOp::Add || ad.a.kind != K::Temp || ad.a.index != 0 || ad.b.kind != K::ElemIdx) return false;
    if (ad.b.index < 0 || static_cast<size_t>(ad.b.index) >= km.buffers.size()) return false;
    const uint32_t bias = static_cast<uint32_t>(ad.b.index);
    if (!elemIs(ad.b, bias, {0, 1})) return false;
    // Root 3: softmax over SC rows.
    Step soft;
    if (!matchSoftmaxNest(km, roots[at + 2], soft) || soft.x != sc || soft.rows != B * S || soft.cols != S) return false;
    // SC lives on chip only: no other root may read or write it.
    if (touchedOutside(km, {roots[at], roots[at + 1], roots[at + 2]}, {sc})) return false;
    if (bufElems(km.buffers[q]) < B * S * D || bufElems(km.buffers[kb]) < B * S * D ||
        bufElems(km.buffers[bias]) < S || bufElems(km.buffers[soft.y]) < B * S * S) {
        return false;
    }
    st.kind = StepKind::ScoreSoftmax;
    st.what = "score-softmax";
    st.q = q;
    st.kk = kb;
    st.bias = bias;
    st.s = soft.y;
    st.batch = B;
    st.seq = S;
    st.dim = D;
    st.div = dv.b.constValue;
    return true;
}

void markTemps(const KernelModule& km, const Step& st, std::vector<bool>& need) {
    auto mark = [&](uint32_t b) {
        if (b < km.buffers.size() && km.buffers[b].isTemp) need[b] = true;
    };
    switch (st.kind) {
        case StepKind::Elementwise:
            for (const StreamRef& s : st.inputs) mark(s.buffer);
            mark(st.out.buffer);
            break;
        case StepKind::Softmax:
        case StepKind::RowSum:
            mark(st.x);
            mark(st.y);
            break;
        case StepKind::Gemm:
            mark(st.a);
            mark(st.b);
            mark(st.c);
            break;
        case StepKind::ScoreSoftmax:
            mark(st.q);
            mark(st.kk);
            mark(st.bias);
            mark(st.s);
            break;
        case StepKind::Nest:
            for (const uint32_t b : st.nestBufs) mark(b);
            break;
        case StepKind::Fail:
            break;
    }
}

/// Buffers a step reads from and writes to device memory.
void stepIO(const Step& st, std::vector<uint32_t>& reads, std::vector<uint32_t>& writes) {
    reads.clear();
    writes.clear();
    switch (st.kind) {
        case StepKind::Elementwise:
            for (const StreamRef& s : st.inputs) reads.push_back(s.buffer);
            if (st.accum != AccumMode::None) reads.push_back(st.out.buffer);
            writes.push_back(st.out.buffer);
            break;
        case StepKind::Nest:
            reads = st.nestReads;
            writes = st.nestWrites;
            break;
        case StepKind::Softmax:
        case StepKind::RowSum:
            reads.push_back(st.x);
            writes.push_back(st.y);
            break;
        case StepKind::Gemm:
            reads.push_back(st.a);
            reads.push_back(st.b);
            if (st.accumulate) reads.push_back(st.c);
            writes.push_back(st.c);
            break;
        case StepKind::ScoreSoftmax:
            reads.push_back(st.q);
            reads.push_back(st.kk);
            reads.push_back(st.bias);
            writes.push_back(st.s);
            break;
        case StepKind::Fail: break;
    }
}

/// A step reads an f32/f16 buffer (not a temp: temps are held in f64) that
/// an earlier step wrote. The device rounds at that store; the reference
/// walker keeps f64 values in every buffer, so the later step sees other
/// bits (its result is still within an f32/f16 rounding's error).
bool crossStepNarrowRead(const KernelModule& km, const std::vector<Step>& steps, bool& f16) {
    using Hull = std::pair<int64_t, int64_t>;
    const Hull whole{INT64_MIN, INT64_MAX};
    std::vector<Hull> written(km.buffers.size(), Hull{INT64_MAX, INT64_MIN});
    std::vector<uint32_t> rd, wr;
    bool found = false;
    auto narrow = [&](uint32_t b) {
        return b < km.buffers.size() && !km.buffers[b].isTemp && km.buffers[b].dtype != Dtype::F64;
    };
    // The elements a stream map reaches over the step's box.
    auto streamHull = [&](const Step& st, const StreamRef& s) -> Hull {
        if (st.dynamicExtent) return whole;
        int64_t lo = s.offset, hi = s.offset;
        for (int d = 0; d < st.rank; ++d) {
            if (st.extent[d] <= 0) return Hull{INT64_MAX, INT64_MIN};
            const __int128 span = static_cast<__int128>(s.coeff[d]) * (st.extent[d] - 1);
            if (span > INT64_MAX / 4 || span < INT64_MIN / 4) return whole;
            (span < 0 ? lo : hi) += static_cast<int64_t>(span);
        }
        return Hull{lo, hi};
    };
    auto hullOf = [&](const Step& st, uint32_t b, bool write) -> Hull {
        const auto& v = write ? st.writeHull : st.readHull;
        if (st.kind == StepKind::Nest && b < v.size()) return v[b];
        if (st.kind == StepKind::Elementwise) {
            if (write || (st.accum != AccumMode::None && b == st.out.buffer)) {
                if (b == st.out.buffer) return streamHull(st, st.out);
            }
            Hull h{INT64_MAX, INT64_MIN};
            for (const StreamRef& s : st.inputs) {
                if (s.buffer != b) continue;
                const Hull x = streamHull(st, s);
                h.first = std::min(h.first, x.first);
                h.second = std::max(h.second, x.second);
            }
            return h;
        }
        return whole;
    };
    for (const Step& st : steps) {
        stepIO(st, rd, wr);
        for (const uint32_t b : rd) {
            if (!narrow(b)) continue;
            const Hull r = hullOf(st, b, false);
            if (r.first <= written[b].second && written[b].first <= r.second) {
                found = true;
                if (km.buffers[b].dtype == Dtype::F16) f16 = true;
            }
        }
        for (const uint32_t b : wr) {
            if (!narrow(b)) continue;
            const Hull w = hullOf(st, b, true);
            written[b].first = std::min(written[b].first, w.first);
            written[b].second = std::max(written[b].second, w.second);
        }
    }
    return found;
}

std::string policyFor(const KernelModule& km, const std::vector<Step>& steps) {
    bool transcend = false, gemm16 = false, gemm32 = false, soft = false, p7out = false, score = false;
    bool nestNarrow = false, nestF16 = false;
    for (const Step& st : steps) {
        switch (st.kind) {
            case StepKind::Nest:
                // f64 buffers and IEEE ops: bit-exact with the walker. A value
                // re-read from an f32/f16 buffer carries that buffer's rounding.
                if (st.transcendental) transcend = true;
                if (st.narrowRoundTrip) nestNarrow = true;
                if (st.touchesF16 && (st.narrowRoundTrip || st.transcendental)) nestF16 = true;
                break;
            case StepKind::Elementwise:
                if (st.chainBody.find("mlk_p7_sin_f32out") != std::string::npos) p7out = true;
                if (st.chainBody.find("mlk_exp_f32acc") != std::string::npos) transcend = true;
                for (const char* f : {"exp(", "log(", "sin(", "cos(", "tan(", "tanh(", "erf(", "pow("}) {
                    if (st.chainBody.find(std::string(" ") + f) != std::string::npos ||
                        st.chainBody.find(std::string("(") + f) != std::string::npos) {
                        transcend = true;
                    }
                }
                break;
            case StepKind::Softmax: soft = true; break;
            case StepKind::RowSum: soft = true; break;
            case StepKind::Gemm:
                if (km.buffers[st.a].dtype == Dtype::F16 || km.buffers[st.b].dtype == Dtype::F16) gemm16 = true;
                else gemm32 = true;
                break;
            case StepKind::ScoreSoftmax: score = true; break;
            case StepKind::Fail: break;
        }
    }
    bool crossF16 = false;
    const bool crossNarrow = crossStepNarrowRead(km, steps, crossF16);
    if (score || gemm16 || nestF16 || (crossNarrow && crossF16)) return "tol-rel1e-2-gfx950-v1";
    if (nestNarrow) return "tol-rel1e-6-gfx950-v1";
    if (gemm32) return "tol-rel1e-5sqrtk-gfx950-v1";
    if (soft || transcend) return "tol-rel1e-6-gfx950-v1";
    if (crossNarrow) return "tol-rel1e-6-gfx950-v1";
    if (p7out) return "tol-4ulp-f32-gfx950-v1";
    return "bitexact-rne-gfx950-v1";
}

}  // namespace

KernelModule deviceModule(const KernelModule& km) {
    KernelModule d = km;
    for (KernelBuffer& b : d.buffers) {
        if (b.isTemp && !b.isInput && !b.isOutput) b.dtype = Dtype::F64;
    }
    return d;
}

int64_t bufferElements(const KernelBuffer& b, int64_t dynamicElements) {
    if (!b.dims.empty()) {
        int64_t n = 1;
        for (const int64_t d : b.dims) {
            if (d < 0) return -1;
            n *= d;
        }
        return n;
    }
    if (b.elements >= 0) return b.elements;
    return dynamicElements;
}

Result<Plan> planModule(const KernelModule& input) {
    // Multi-dim forests are recognized in canonical form (tiled, split and
    // guarded bands folded back to their untiled shapes, canonical.cpp).
    // Two schedule parameters select the path for tests and variant search:
    // "hip_canonical" = 0 plans the module as written, "hip_generic" = 1 runs
    // every multi-dim root on the generic loop-nest kernel. ("hip_slabs" = 0,
    // read by planNest, turns that kernel's LDS slabs off.)
    const bool multiDim = isMultiDimModule(input);
    const bool canon = input.param("hip_canonical", 1) != 0;
    const bool genericOnly = input.param("hip_generic", 0) != 0;
    int rewrites = 0;
    const KernelModule km = multiDim && canon ? canonicalModule(input, &rewrites) : input;
    Plan plan;
    plan.canonicalized = rewrites != 0;
    plan.tempNeeded.assign(km.buffers.size(), false);
    if (km.nodes.empty()) return err(ErrorCode::InvalidGraph, "kernel module has no nodes");
    for (const KernelBuffer& b : km.buffers) {
        if (b.dtype == Dtype::Other && (b.isInput || b.isOutput || b.isTemp)) {
            return err(ErrorCode::UnsupportedCapability, "buffer dtype outside f16/f32/f64: " + b.name);
        }
    }
    plan.multiDim = multiDim;
    if (!plan.multiDim) {
        for (const KernelNode& top : km.nodes) {
            if (top.op == KernelOp::Loop) {
                auto steps = tier1Loop(km, top);
                if (!steps.has_value()) return err(steps.error().code, steps.error().message);
                for (Step& s : *steps) plan.steps.push_back(std::move(s));
            } else if (top.op == KernelOp::Call) {
                auto st = callStep(km, top, false);
                if (!st.has_value()) return err(st.error().code, st.error().message);
                plan.steps.push_back(std::move(*st));
            }
        }
    } else {
        MLK_TRYV(walkerPositions(input));
        const std::vector<uint32_t> roots = forestRoots(km);
        for (size_t i = 0; i < roots.size(); ++i) {
            const KernelNode& r = km.nodes[roots[i]];
            Step st;
            if (r.op == KernelOp::Call) {
                auto cs = callStep(km, r, true);
                if (!cs.has_value()) return err(cs.error().code, cs.error().message);
                plan.steps.push_back(std::move(*cs));
                continue;
            }
            if (r.op != KernelOp::Loop) {
                if (r.op == KernelOp::Guard && r.hasAffineGuard()) {
                    auto ns = planNest(km, roots[i]);
                    if (!ns.has_value()) return err(ns.error().code, ns.error().message);
                    plan.steps.push_back(std::move(*ns));
                }
                continue;  // Compute/Store/etc. at root carry no semantics for the walker
            }
            if (genericOnly) {
                auto ns = planNest(km, roots[i]);
                if (!ns.has_value()) return err(ns.error().code, ns.error().message);
                plan.steps.push_back(std::move(*ns));
                continue;
            }
            if (matchScoreSoftmax(km, roots, i, st)) {
                plan.steps.push_back(std::move(st));
                i += 2;
                continue;
            }
            if (matchSoftmaxNest(km, roots[i], st) || matchGemmNest(km, roots[i], st) ||
                matchReduceSumNest(km, roots[i], st)) {
                plan.steps.push_back(std::move(st));
                continue;
            }
            NestInfo ni;
            if (perfectNest(km, roots[i], ni)) {
                auto es = elementwiseNest(km, ni);
                if (es.has_value()) {
                    plan.steps.push_back(std::move(*es));
                    continue;
                }
                if (es.error().code != ErrorCode::UnsupportedCapability) return err(es.error().code, es.error().message);
            }
            // No hand-written class claims the root: the generic loop-nest kernel.
            auto ns = planNest(km, roots[i]);
            if (!ns.has_value()) return err(ns.error().code, ns.error().message);
            plan.steps.push_back(std::move(*ns));
        }
    }
    for (const Step& st : plan.steps) markTemps(km, st, plan.tempNeeded);
    for (size_t b = 0; b < km.buffers.size(); ++b) {
        if (!plan.tempNeeded[b]) continue;
        const int64_t n = bufElems(km.buffers[b]);
        if (n <= 0 || n > kTempElementsLimit) {
            return err(ErrorCode::InvalidGraph, "temp buffer element count out of range");
        }
    }
    std::string cls;
    for (const Step& st : plan.steps) {
        if (!cls.empty()) cls += "+";
        cls += st.what;
    }
    plan.className = cls.empty() ? "empty" : cls;
    plan.policy = policyFor(km, plan.steps);
    return plan;
}

}  // namespace mlk::hip
