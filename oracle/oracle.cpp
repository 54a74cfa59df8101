// CPU oracle for the KernelModule execution path — TEST INFRASTRUCTURE ONLY.
//
// This file restates, in plain C++17 over dense f64 buffers, what the
// reference CPU backend computes for a KernelModule:
//   executeKernelOnBuffers   runtime/src/execution/kernel_buffers.cpp:839-1106
//   ExprEvaluator            runtime/src/execution/kernel_buffers.cpp:55-179
//   decideThreads            runtime/src/execution/kernel_buffers.cpp:183-199
//   execReduceSumCall        runtime/src/execution/kernel_buffers.cpp:237-277
//   execSoftmaxCall          runtime/src/execution/kernel_buffers.cpp:290-340
//   runElementwiseRange      runtime/src/execution/kernel_buffers.cpp:342-402
//   gemmRowBlock             runtime/src/execution/kernel_buffers.cpp:406-432
//   MultiDimWalker           runtime/src/execution/kernel_buffers.cpp:453-835
//   families::polySin        compiler/include/mlk/support/math_families.h:22-90
// It is the checker the HIP backend is compared against. Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
// product library never links or calls it.
//
// Input format: the "mlk-kernel" JSON a KernelModule serializes to
// (compiler/src/support/kernel_ir.cpp:97-254), with two extensions the
// product parser shares: Call nodes carry "math" (the reference writer
// omits it), and the non-standard tokens Infinity/-Infinity/NaN carry exact
// non-finite constants (the reference writer clamps them,
// compiler/src/core/json.cpp:300-312). The parser here is independent of the
// product's parser on purpose.
//
// Pinning (each function is checked by tests/test_oracle.py):
//   poly7 sin   bit-exact vs the reference's own math_families.h compiled
//               from /root/reference (oracle/_ref), known answer
//               sin(x^2+3x)|x=2 (examples/scalar/README.md:9), <=2 ULP vs libm
//               on [-pi, pi] (README.md:34);
//   GEMM        bit-exact vs exact rational sums on the reference fixtures
//               (tests/unit/unit_poly.cpp:2024-2056, :680-682);
//   softmax     hand-computed stable form (unit_poly.cpp:3584-3607), K=1 -> 1,
//               NaN and +/-0 rows (unit_poly.cpp:3820-3835), Tier-1 Call vs
//               Tier-2 synthesized nest bit-exact;
//   broadcast   brute-force index identity y[i,j] = f(x[i,j], b[j]);
//   reducesum   exact sums of dyadic rationals;
//   walker      Tier-2 GEMM nest vs Call(MatMul) bit-exact, guards/affine
//               bounds vs brute-force enumeration.
// exp/log/tanh/erf come from the host libm (glibc): their bit patterns are
// not pinned by any reference fixture ("parity unpinned" for those ops; the
// GPU comparisons use tolerances that absorb <=1 ULP f64 libm variation).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

namespace oracle {

// ---------------------------------------------------------------- JSON ----
struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind{Null};
    bool b{false};
    double num{0.0};
    bool isInt{false};
    int64_t i{0};
    std::string s;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;

    const JVal* get(const char* key) const {
        if (kind != Obj) return nullptr;
        for (const auto& kv : obj) {
            if (kv.first == key) return &kv.second;
        }
        return nullptr;
    }
    int64_t asInt(int64_t fb = 0) const {
        if (kind != Num) return fb;
        return isInt ? i : static_cast<int64_t>(num);
    }
    double asNum(double fb = 0.0) const {
        if (kind != Num) return fb;
        return isInt ? static_cast<double>(i) : num;
    }
};

struct JParser {
    const char* p;
    const char* end;
    bool ok{true};

    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\t' || *p == '\r')) ++p;
    }
    bool lit(const char* t) {
        const size_t n = std::strlen(t);
        if (static_cast<size_t>(end - p) >= n && std::strncmp(p, t, n) == 0) {
            p += n;
            return true;
        }
        return false;
    }
    JVal value(int depth) {
        JVal v;
        if (depth > 64) { ok = false; return v; }
        ws();
        if (p >= end) { ok = false; return v; }
        const char c = *p;
        if (c == '{') {
            ++p;
            v.kind = JVal::Obj;
            ws();
            if (p < end && *p == '}') { ++p; return v; }
            while (ok) {
                ws();
                JVal k = value(depth + 1);
                if (k.kind != JVal::Str) { ok = false; break; }
                ws();
                if (p >= end || *p != ':') { ok = false; break; }
                ++p;
                JVal x = value(depth + 1);
                v.obj.emplace_back(k.s, std::move(x));
                ws();
                if (p < end && *p == ',') { ++p; continue; }
                if (p < end && *p == '}') { ++p; break; }
                ok = false;
            }
            return v;
        }
        if (c == '[') {
            ++p;
            v.kind = JVal::Arr;
            ws();
            if (p < end && *p == ']') { ++p; return v; }
            while (ok) {
                v.arr.push_back(value(depth + 1));
                ws();
                if (p < end && *p == ',') { ++p; continue; }
                if (p < end && *p == ']') { ++p; break; }
                ok = false;
            }
            return v;
        }
        if (c == '"') {
            ++p;
            v.kind = JVal::Str;
            while (p < end && *p != '"') {
                if (*p == '\\' && p + 1 < end) {
                    ++p;
                    switch (*p) {
                        case 'n': v.s.push_back('\n'); break;
                        case 't': v.s.push_back('\t'); break;
                        case 'u': p += 4; v.s.push_back('?'); break;
                        default: v.s.push_back(*p); break;
                    }
                    ++p;
                    continue;
                }
                v.s.push_back(*p++);
            }
            if (p >= end) { ok = false; return v; }
            ++p;
            return v;
        }
        if (lit("true")) { v.kind = JVal::Bool; v.b = true; return v; }
        if (lit("false")) { v.kind = JVal::Bool; v.b = false; return v; }
        if (lit("null")) { v.kind = JVal::Null; return v; }
        if (lit("NaN")) { v.kind = JVal::Num; v.num = NAN; return v; }
        if (lit("Infinity")) { v.kind = JVal::Num; v.num = INFINITY; return v; }
        if (lit("-Infinity")) { v.kind = JVal::Num; v.num = -INFINITY; return v; }
        // number
        const char* s = p;
        bool isFloat = false;
        if (p < end && (*p == '-' || *p == '+')) ++p;
        while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' ||
                           *p == 'E' || *p == '-' || *p == '+')) {
            if (*p == '.' || *p == 'e' || *p == 'E') isFloat = true;
            ++p;
        }
        if (p == s) { ok = false; return v; }
        std::string tok(s, p);
        v.kind = JVal::Num;
        if (isFloat) {
            v.num = std::strtod(tok.c_str(), nullptr);
        } else {
            v.isInt = true;
            v.i = std::strtoll(tok.c_str(), nullptr, 10);
            v.num = static_cast<double>(v.i);
        }
        return v;
    }
};

// ----------------------------------------------------------- Kernel IR ----
// Restatement of compiler/include/mlk/support/kernel_ir.h:22-224.
constexpr uint32_t kInvalidId = 0xFFFFFFFFu;
constexpr int64_t kDynamic = -1;                      // constants.h:92
constexpr int64_t kTempElementsLimit = int64_t{1} << 24;  // constants.h:99
constexpr int64_t kMaxThreads = 4;                    // constants.h:138
constexpr int64_t kParallelChunk = 16384;             // constants.h:142
constexpr int64_t kTileM = 64, kTileN = 64, kTileK = 32;  // constants.h:84-86
constexpr size_t kMaxTempSlots = 64;                  // kernel_buffers.cpp:35

enum class Op { Loop, Compute, Load, Store, Alloc, Copy, Barrier, Trace, Guard, Call, Bad };
enum class Math {
    Add, Sub, Mul, Div, Neg, Pow, Exp, Log, Sin, Cos, Tan, Tanh, Sqrt, Rsqrt,
    Erf, Gelu, MatMul, ReduceSum, Softmax, Other
};
enum class Kind { Const, ElemA, ElemB, Scalar, Temp, ElemIdx };
enum class Accum { None, Add, Max };

// Error codes follow compiler/include/mlk/core/result.h:23-41.
enum Err : int {
    kOk = 0, kInvalidArgument = 1, kInvalidGraph = 2, kUnsupported = 4,
    kResourceExhausted = 15,
};

struct Operand {
    Kind kind{Kind::Const};
    int64_t index{0};
    double value{0.0};
    std::vector<int64_t> coeffs;
    int64_t offset{0};
};
struct Expr {
    Math op{Math::Add};
    Operand a, b;
};
struct Node {
    Op op{Op::Loop};
    Math math{Math::Add};
    int64_t begin{0}, end{kDynamic}, step{1};
    std::vector<int64_t> beginCoeffs, endCoeffs;
    int64_t beginOffset{0}, endOffset{0};
    uint32_t endBuf{kInvalidId};
    int32_t endDim{-1};
    uint32_t bufA{kInvalidId}, bufB{kInvalidId}, bufOut{kInvalidId};
    std::vector<int64_t> outCoeffs;
    int64_t outOffset{0};
    Accum accum{Accum::None};
    bool parallel{false};
    std::vector<int64_t> guardCoeffs;
    int64_t guardOffset{0};
    bool poly7{false};
    std::vector<Expr> exprs;
    std::vector<uint32_t> children;
};
struct Buffer {
    bool isInput{false}, isOutput{false}, isTemp{false};
    int64_t elements{kDynamic};
    std::vector<int64_t> dims;
};
struct Module {
    std::vector<Buffer> buffers;
    std::vector<Node> nodes;
    bool hasThreads{false};
    int64_t threads{0};
    bool hasTile[3]{false, false, false};
    int64_t tile[3]{kTileM, kTileN, kTileK};
};

Math mathFromName(const std::string& s) {
    static const struct { const char* n; Math m; } kTab[] = {
        {"add", Math::Add}, {"sub", Math::Sub}, {"mul", Math::Mul},
        {"div", Math::Div}, {"neg", Math::Neg}, {"pow", Math::Pow},
        {"exp", Math::Exp}, {"log", Math::Log}, {"sin", Math::Sin},
        {"cos", Math::Cos}, {"tan", Math::Tan}, {"tanh", Math::Tanh},
        {"sqrt", Math::Sqrt}, {"rsqrt", Math::Rsqrt}, {"erf", Math::Erf},
        {"gelu", Math::Gelu}, {"matmul", Math::MatMul},
        {"reduce_sum", Math::ReduceSum}, {"softmax", Math::Softmax}};
    for (const auto& e : kTab) {
        if (s == e.n) return e.m;
    }
    return Math::Other;
}

Op opFromName(const std::string& s) {
    static const struct { const char* n; Op o; } kTab[] = {
        {"loop", Op::Loop}, {"compute", Op::Compute}, {"load", Op::Load},
        {"store", Op::Store}, {"alloc", Op::Alloc}, {"copy", Op::Copy},
        {"barrier", Op::Barrier}, {"trace", Op::Trace}, {"guard", Op::Guard},
        {"call", Op::Call}};
    for (const auto& e : kTab) {
        if (s == e.n) return e.o;
    }
    return Op::Bad;
}

std::vector<int64_t> intList(const JVal* v) {
    std::vector<int64_t> out;
    if (v == nullptr || v->kind != JVal::Arr) return out;
    for (const auto& x : v->arr) out.push_back(x.asInt());
    return out;
}

bool parseOperand(const JVal* j, Operand& o) {
    if (j == nullptr) return true;  // default Const 0.0
    const JVal* k = j->get("kind");
    if (k == nullptr || k->kind != JVal::Str) return false;
    if (k->s == "const") {
        o.kind = Kind::Const;
        const JVal* v = j->get("value");
        // The reference writer serializes NaN as null (json.cpp:301-303).
        o.value = (v == nullptr || v->kind == JVal::Null) ? (v ? NAN : 0.0) : v->asNum();
    } else if (k->s == "elem_a") {
        o.kind = Kind::ElemA;
    } else if (k->s == "elem_b") {
        o.kind = Kind::ElemB;
    } else if (k->s == "scalar_param") {
        o.kind = Kind::Scalar;
        o.index = j->get("index") ? j->get("index")->asInt() : 0;
    } else if (k->s == "temp") {
        o.kind = Kind::Temp;
        o.index = j->get("index") ? j->get("index")->asInt() : 0;
    } else if (k->s == "elem_idx") {
        o.kind = Kind::ElemIdx;
        o.index = j->get("buffer") ? j->get("buffer")->asInt() : -1;
        o.coeffs = intList(j->get("coeffs"));
        o.offset = j->get("offset") ? j->get("offset")->asInt() : 0;
    } else {
        return false;
    }
    return true;
}

bool parseModule(const char* text, size_t len, Module& m, std::string& why) {
    JParser ps{text, text + len};
    JVal doc = ps.value(0);
    if (!ps.ok || doc.kind != JVal::Obj) { why = "json parse error"; return false; }
    const JVal* fmt = doc.get("format");
    if (fmt == nullptr || fmt->s != "mlk-kernel") { why = "not an mlk-kernel document"; return false; }
    const JVal* bufs = doc.get("buffers");
    const JVal* nodes = doc.get("nodes");
    if (bufs == nullptr || nodes == nullptr || bufs->kind != JVal::Arr || nodes->kind != JVal::Arr) {
        why = "missing buffers/nodes";
        return false;
    }
    for (const auto& jb : bufs->arr) {
        Buffer b;
        b.isInput = jb.get("input") && jb.get("input")->b;
        b.isOutput = jb.get("output") && jb.get("output")->b;
        b.isTemp = jb.get("temp") && jb.get("temp")->b;
        b.elements = jb.get("elements") ? jb.get("elements")->asInt() : kDynamic;
        b.dims = intList(jb.get("dims"));
        m.buffers.push_back(b);
    }
    for (const auto& jn : nodes->arr) {
        Node n;
        const JVal* op = jn.get("op");
        n.op = op ? opFromName(op->s) : Op::Bad;
        if (n.op == Op::Bad) { why = "unknown node op"; return false; }
        if (const JVal* mth = jn.get("math")) n.math = mathFromName(mth->s);
        if (const JVal* fam = jn.get("family")) n.poly7 = fam->s == "poly7";
        if (const JVal* v = jn.get("begin")) n.begin = v->asInt();
        if (const JVal* v = jn.get("end")) n.end = v->asInt();
        if (const JVal* v = jn.get("step")) n.step = v->asInt();
        if (const JVal* v = jn.get("end_buf")) n.endBuf = static_cast<uint32_t>(v->asInt());
        if (const JVal* v = jn.get("end_dim")) n.endDim = static_cast<int32_t>(v->asInt());
        n.beginCoeffs = intList(jn.get("begin_coeffs"));
        n.endCoeffs = intList(jn.get("end_coeffs"));
        if (const JVal* v = jn.get("begin_offset")) n.beginOffset = v->asInt();
        if (const JVal* v = jn.get("end_offset")) n.endOffset = v->asInt();
        n.outCoeffs = intList(jn.get("out_index_coeffs"));
        if (const JVal* v = jn.get("out_index_offset")) n.outOffset = v->asInt();
        if (const JVal* v = jn.get("accumulate")) {
            if (v->b) {
                n.accum = Accum::Add;
                const JVal* mode = jn.get("accum_mode");
                if (mode != nullptr && mode->s == "max") n.accum = Accum::Max;
            }
        }
        if (const JVal* v = jn.get("parallel")) n.parallel = v->b;
        n.guardCoeffs = intList(jn.get("guard_coeffs"));
        if (const JVal* v = jn.get("guard_offset")) n.guardOffset = v->asInt();
        if (const JVal* v = jn.get("a")) n.bufA = static_cast<uint32_t>(v->asInt());
        if (const JVal* v = jn.get("b")) n.bufB = static_cast<uint32_t>(v->asInt());
        if (const JVal* v = jn.get("out")) n.bufOut = static_cast<uint32_t>(v->asInt());
        if (const JVal* xs = jn.get("exprs")) {
            for (const auto& je : xs->arr) {
                Expr e;
                const JVal* eop = je.get("op");
                e.op = eop ? mathFromName(eop->s) : Math::Other;
                if (!parseOperand(je.get("a"), e.a) || !parseOperand(je.get("b"), e.b)) {
                    why = "bad operand";
                    return false;
                }
                n.exprs.push_back(e);
            }
        }
        for (int64_t c : intList(jn.get("children"))) n.children.push_back(static_cast<uint32_t>(c));
        m.nodes.push_back(std::move(n));
    }
    if (const JVal* sched = doc.get("schedule")) {
        if (const JVal* t = sched->get("threads")) { m.hasThreads = true; m.threads = t->asInt(); }
        const char* keys[3] = {"tile_m", "tile_n", "tile_k"};
        for (int q = 0; q < 3; ++q) {
            if (const JVal* t = sched->get(keys[q])) { m.hasTile[q] = true; m.tile[q] = t->asInt(); }
        }
    }
    return true;
}

// --------------------------------------------------------- poly7 sin -----
// math_families.h:22-90, operation for operation (no contraction: this
// translation unit is compiled with -ffp-contract=off).
constexpr double kPiHalf = 1.57079632679489661923;
constexpr double kPio2Hi = 1.5707963267948965580e+00;
constexpr double kPio2Lo = 6.1232339957367660359e-17;
constexpr double kS[6] = {1.58962301576546568060e-10, -2.50507477628578072866e-8,
                          2.75573136213857245213e-6, -1.98412698295895385996e-4,
                          8.33333333332211858878e-3, -1.66666666666666307295e-1};
constexpr double kC[6] = {-1.13585365213876817300e-11, 2.08757530072652689750e-9,
                          -2.75573142103085808917e-7, 2.48015872890001867312e-5,
                          -1.38888888888783992457e-3, 4.16666666666666435770e-2};

double sinReduced(double x) {
    const double r2 = x * x;
    double p = kS[0];
    for (int i = 1; i < 6; ++i) p = p * r2 + kS[i];
    return x + x * r2 * p;
}
double cosReduced(double x) {
    const double r2 = x * x;
    double p = kC[0];
    for (int i = 1; i < 6; ++i) p = p * r2 + kC[i];
    return 1.0 - r2 * 0.5 + r2 * r2 * p;
}
double polySin(double x) {
    const double n = std::floor(x / kPiHalf + 0.5);
    const double r = (x - n * kPio2Hi) - n * kPio2Lo;
    int q = static_cast<int>(std::fmod(n, 4.0));
    q = q < 0 ? q + 4 : q;
    switch (q) {
        case 0: return sinReduced(r);
        case 1: return cosReduced(r);
        case 2: return -sinReduced(r);
        default: return -cosReduced(r);
    }
}

// ---------------------------------------------------------- executor -----
struct Bindings {
    std::vector<double*> inputs;   // io.inputs
    std::vector<double*> outputs;  // io.outputs
    std::vector<double> scalars;
    int64_t elements{0};
    std::vector<double*> temps;    // bufferId-indexed
    int64_t hwThreads{1};
};

struct Status {
    int code{kOk};
    std::string msg;
    bool ok() const { return code == kOk; }
};
Status fail(int code, const char* msg) { return Status{code, msg}; }

bool isUnary(Math op) {
    return op == Math::Neg || op == Math::Exp || op == Math::Log || op == Math::Sin ||
           op == Math::Cos || op == Math::Tan || op == Math::Tanh || op == Math::Sqrt ||
           op == Math::Rsqrt || op == Math::Erf || op == Math::Gelu;
}

double apply(Math op, double a, double b, bool poly7) {
    switch (op) {
        case Math::Add: return a + b;
        case Math::Sub: return a - b;
        case Math::Mul: return a * b;
        case Math::Div: return b != 0.0 ? a / b : 0.0;
        case Math::Neg: return -a;
        case Math::Pow: return a == 2.0 && b == 2.0 ? a * a : std::pow(a, b);
        case Math::Exp: return std::exp(a);
        case Math::Log: return a > 0.0 ? std::log(a) : 0.0;
        case Math::Sin: return poly7 ? polySin(a) : std::sin(a);
        case Math::Cos: return std::cos(a);
        case Math::Tan: return std::tan(a);
        case Math::Tanh: return std::tanh(a);
        case Math::Sqrt: return a >= 0.0 ? std::sqrt(a) : 0.0;
        case Math::Rsqrt: return a > 0.0 ? 1.0 / std::sqrt(a) : 0.0;
        case Math::Erf: return std::erf(a);
        case Math::Gelu:
            return 0.5 * a * (1.0 + std::tanh(0.7978845608028654 * (a + 0.044715 * a * a * a)));
        default: return 0.0;
    }
}

const double* resolveInput(const Module& m, const Bindings& io, uint32_t bid) {
    if (bid == kInvalidId || bid >= m.buffers.size()) return nullptr;
    if (m.buffers[bid].isInput) return bid < io.inputs.size() ? io.inputs[bid] : nullptr;
    const uint32_t o = bid - static_cast<uint32_t>(io.inputs.size());
    return o < io.outputs.size() ? io.outputs[o] : nullptr;
}
double* resolveOutput(const Module& m, const Bindings& io, uint32_t bid) {
    if (bid == kInvalidId || bid >= m.buffers.size()) return nullptr;
    if (m.buffers[bid].isOutput) {
        const uint32_t o = bid - static_cast<uint32_t>(io.inputs.size());
        return o < io.outputs.size() ? io.outputs[o] : nullptr;
    }
    return bid < io.inputs.size() ? io.inputs[bid] : nullptr;
}

struct Evaluator {
    const std::vector<Expr>& exprs;
    const double* elemA;
    const double* elemB;
    const std::vector<double>& scalars;
    bool poly7;
    const std::vector<int64_t>* vars{nullptr};
    const Module* mod{nullptr};
    const Bindings* io{nullptr};
    double temps[kMaxTempSlots] = {};

    int64_t flat(const Operand& o) const {
        int64_t f = o.offset;
        if (vars != nullptr) {
            const size_t n = std::min(o.coeffs.size(), vars->size());
            for (size_t p = 0; p < n; ++p) f += o.coeffs[p] * (*vars)[p];
        }
        return f;
    }
    const double* elemPtr(const Operand& o) const {
        if (mod == nullptr || io == nullptr) return nullptr;
        if (o.index < 0 || static_cast<size_t>(o.index) >= mod->buffers.size()) return nullptr;
        const uint32_t bid = static_cast<uint32_t>(o.index);
        const double* base = nullptr;
        if (mod->buffers[bid].isTemp) {
            base = bid < io->temps.size() ? io->temps[bid] : nullptr;
        } else if (mod->buffers[bid].isInput) {
            base = bid < io->inputs.size() ? io->inputs[bid] : nullptr;
        } else {
            const uint32_t oi = bid - static_cast<uint32_t>(io->inputs.size());
            base = oi < io->outputs.size() ? io->outputs[oi] : nullptr;
        }
        return base != nullptr ? base + flat(o) : nullptr;
    }
    double evalOne(const Operand& o, int64_t i) const {
        switch (o.kind) {
            case Kind::Const: return o.value;
            case Kind::ElemA: return elemA[i];
            case Kind::ElemB: return elemB != nullptr ? elemB[i] : 0.0;
            case Kind::Scalar: {
                const size_t idx = static_cast<size_t>(o.index);
                return idx < scalars.size() ? scalars[idx] : 0.0;
            }
            case Kind::Temp: {
                const size_t idx = static_cast<size_t>(o.index);
                return idx < kMaxTempSlots ? temps[idx] : 0.0;
            }
            case Kind::ElemIdx: {
                const double* p = elemPtr(o);
                return p != nullptr ? *p : 0.0;
            }
        }
        return 0.0;
    }
    double run(int64_t i) {
        for (size_t k = 0; k < exprs.size() && k < kMaxTempSlots; ++k) {
            const Expr& e = exprs[k];
            const double a = evalOne(e.a, i);
            const double b = isUnary(e.op) ? 0.0 : evalOne(e.b, i);
            temps[k] = apply(e.op, a, b, poly7);
        }
        const size_t last = exprs.size() - 1;
        return last < kMaxTempSlots ? temps[last] : 0.0;
    }
};

int64_t decideThreads(const Module& m, const Bindings& io, int64_t elements) {
    int64_t threads = io.hwThreads > 0 ? io.hwThreads : 1;
    if (threads > kMaxThreads) threads = kMaxThreads;
    if (m.hasThreads && m.threads >= 1) threads = m.threads;
    if (elements < kParallelChunk) threads = 1;
    return threads;
}

Status reduceSumCall(const Module& m, const Bindings& io, const Node& top) {
    if (top.bufA >= m.buffers.size() || top.bufOut >= m.buffers.size())
        return fail(kInvalidGraph, "reducesum buffer id out of range");
    const Buffer& ba = m.buffers[top.bufA];
    const Buffer& by = m.buffers[top.bufOut];
    if (ba.dims.size() != 2 || by.dims.size() != 1)
        return fail(kInvalidGraph, "reducesum requires rank-2 input over rank-1 output");
    const double* a = resolveInput(m, io, top.bufA);
    double* y = resolveOutput(m, io, top.bufOut);
    if (a == nullptr || y == nullptr) return fail(kInvalidArgument, "reducesum buffers not bound by the caller");
    const int64_t rows = ba.dims[0], k = ba.dims[1];
    if (by.dims[0] != rows || k <= 0 || rows <= 0)
        return fail(kInvalidGraph, "reducesum operand shapes incompatible");
    for (int64_t i = 0; i < rows; ++i) {
        double acc = 0.0;
        for (int64_t p = 0; p < k; ++p) acc += a[i * k + p];
        y[i] = acc;
    }
    return {};
}

Status softmaxCall(const Module& m, const Bindings& io, const Node& top) {
    if (top.bufA >= m.buffers.size() || top.bufOut >= m.buffers.size())
        return fail(kInvalidGraph, "softmax buffer id out of range");
    const Buffer& ba = m.buffers[top.bufA];
    const Buffer& by = m.buffers[top.bufOut];
    if (ba.dims.size() != 2 || by.dims.size() != 2)
        return fail(kInvalidGraph, "softmax requires rank-2 operand and output");
    const double* a = resolveInput(m, io, top.bufA);
    double* y = resolveOutput(m, io, top.bufOut);
    if (a == nullptr || y == nullptr) return fail(kInvalidArgument, "softmax buffers not bound by the caller");
    const int64_t rows = ba.dims[0], k = ba.dims[1];
    if (by.dims[0] != rows || by.dims[1] != k || k <= 0 || rows <= 0)
        return fail(kInvalidGraph, "softmax operand shapes incompatible");
    for (int64_t i = 0; i < rows; ++i) {
        const double* row = a + i * k;
        double* yrow = y + i * k;
        double r = -INFINITY;
        for (int64_t p = 0; p < k; ++p) r = (row[p] > r) ? row[p] : r;
        for (int64_t p = 0; p < k; ++p) yrow[p] = std::exp(row[p] - r);
        double s = 0.0;
        for (int64_t p = 0; p < k; ++p) s += yrow[p];
        for (int64_t p = 0; p < k; ++p) yrow[p] = s != 0.0 ? yrow[p] / s : 0.0;
    }
    return {};
}

void elementwiseRange(const Node& compute, const Node& store, const Module& m,
                      const Bindings& io, int64_t begin, int64_t end) {
    bool needsA = compute.exprs.empty();
    bool needsB = compute.exprs.empty();
    for (const Expr& e : compute.exprs) {
        if (e.a.kind == Kind::ElemA || e.b.kind == Kind::ElemA) needsA = true;
        if (e.a.kind == Kind::ElemB || e.b.kind == Kind::ElemB) needsB = true;
    }
    const double* inA = needsA ? resolveInput(m, io, compute.bufA) : nullptr;
    const double* inB = needsB ? resolveInput(m, io, compute.bufB) : nullptr;
    double* out = resolveOutput(m, io, store.bufOut);
    if (out == nullptr || (needsA && inA == nullptr) || (needsB && inB == nullptr)) return;
    if (!compute.exprs.empty()) {
        Evaluator ev{compute.exprs, inA, inB, io.scalars, compute.poly7};
        for (int64_t i = begin; i < end; ++i) out[i] = ev.run(i);
        return;
    }
    static const std::vector<Expr> kNone;
    Evaluator ev{kNone, inA, inB, io.scalars, compute.poly7};
    Operand a, b;
    a.kind = Kind::ElemA;
    b.kind = Kind::ElemB;
    for (int64_t i = begin; i < end; ++i) {
        out[i] = apply(compute.math, ev.evalOne(a, i), ev.evalOne(b, i), compute.poly7);
    }
}

void gemmRowBlock(const double* a, const double* b, double* c, int64_t n, int64_t k,
                  int64_t tileM, int64_t tileN, int64_t tileK, int64_t rowBegin, int64_t rowEnd) {
    for (int64_t ii = rowBegin; ii < rowEnd; ii += tileM) {
        const int64_t iEnd = std::min(ii + tileM, rowEnd);
        for (int64_t jj = 0; jj < n; jj += tileN) {
            const int64_t jEnd = std::min(jj + tileN, n);
            for (int64_t kk = 0; kk < k; kk += tileK) {
                const int64_t kEnd = std::min(kk + tileK, k);
                for (int64_t i = ii; i < iEnd; ++i) {
                    const double* aRow = a + i * k;
                    double* cRow = c + i * n;
                    for (int64_t p = kk; p < kEnd; ++p) {
                        const double aik = aRow[p];
                        if (aik == 0.0) continue;
                        const double* bRow = b + p * n;
                        for (int64_t j = jj; j < jEnd; ++j) cRow[j] += aik * bRow[j];
                    }
                }
            }
        }
    }
}

Status gemmCall(const Module& m, const Bindings& io, const Node& top, bool threaded) {
    if (top.bufA >= m.buffers.size() || top.bufB >= m.buffers.size() || top.bufOut >= m.buffers.size())
        return fail(kInvalidGraph, "matmul buffer id out of range");
    const Buffer& ba = m.buffers[top.bufA];
    const Buffer& bb = m.buffers[top.bufB];
    const Buffer& bc = m.buffers[top.bufOut];
    if (ba.dims.size() != 2 || bb.dims.size() != 2 || bc.dims.size() != 2)
        return fail(kInvalidGraph, "matmul requires rank-2 buffer dims");
    const int64_t rows = ba.dims[0], k = ba.dims[1];
    // The walker form takes N from C (kernel_buffers.cpp:359), the 1-D
    // top level from B (:1030); both must agree with the shape check.
    const int64_t n = threaded ? bb.dims[1] : bc.dims[1];
    if (bb.dims[0] != k || bc.dims[0] != rows || bc.dims[1] != n)
        return fail(kInvalidGraph, "matmul operand shapes incompatible");
    const double* a = resolveInput(m, io, top.bufA);
    const double* b = resolveInput(m, io, top.bufB);
    double* c = resolveOutput(m, io, top.bufOut);
    if (a == nullptr || b == nullptr || c == nullptr)
        return fail(kInvalidArgument, "matmul buffers not bound by the caller");
    const int64_t tm = m.tile[0], tn = m.tile[1], tk = m.tile[2];
    const int64_t threads = threaded ? decideThreads(m, io, rows * n) : 1;
    if (threads <= 1) {
        gemmRowBlock(a, b, c, n, k, tm, tn, tk, 0, rows);
        return {};
    }
    std::vector<std::thread> pool;
    const int64_t per = (rows + threads - 1) / threads;
    for (int64_t t = 0; t < threads; ++t) {
        const int64_t b0 = t * per, b1 = std::min(b0 + per, rows);
        if (b0 >= b1) break;
        pool.emplace_back([=]() { gemmRowBlock(a, b, c, n, k, tm, tn, tk, b0, b1); });
    }
    for (auto& th : pool) th.join();
    return {};
}

struct Walker {
    const Module& m;
    const Bindings& io;
    std::vector<int64_t> vars;

    bool subtreeSafe(uint32_t id) const {
        if (id >= m.nodes.size()) return false;
        const Node& n = m.nodes[id];
        if (n.op != Op::Loop && n.op != Op::Compute && n.op != Op::Store && n.op != Op::Guard) return false;
        for (uint32_t c : n.children) {
            if (!subtreeSafe(c)) return false;
        }
        return true;
    }
    bool bodySafe(const Node& loop) const {
        for (uint32_t c : loop.children) {
            if (!subtreeSafe(c)) return false;
        }
        return true;
    }
    Status childList(const std::vector<uint32_t>& children) {
        for (size_t ci = 0; ci < children.size(); ++ci) {
            const uint32_t cid = children[ci];
            if (cid >= m.nodes.size()) return fail(kInvalidGraph, "walker: child id out of range");
            if (m.nodes[cid].op == Op::Compute) {
                const Node* store = nullptr;
                if (ci + 1 < children.size() && children[ci + 1] < m.nodes.size() &&
                    m.nodes[children[ci + 1]].op == Op::Store) {
                    store = &m.nodes[children[ci + 1]];
                }
                Status s = exec(cid, store);
                if (!s.ok()) return s;
                if (store != nullptr) ++ci;
                continue;
            }
            Status s = exec(cid, nullptr);
            if (!s.ok()) return s;
        }
        return {};
    }
    Status loopRange(const Node& n, int64_t b, int64_t e) {
        for (int64_t v = b; v <= e; ++v) {
            vars.push_back(v);
            Status s = childList(n.children);
            if (!s.ok()) return s;
            vars.pop_back();
        }
        return {};
    }
    Status exec(uint32_t id, const Node* pairedStore) {
        if (id >= m.nodes.size()) return fail(kInvalidGraph, "walker: node id out of range");
        const Node& n = m.nodes[id];
        switch (n.op) {
            case Op::Loop: {
                if (n.step != 1) return fail(kUnsupported, "walker: non-unit loop step");
                int64_t begin = n.begin;
                int64_t endInc = n.end - 1;
                if (!n.beginCoeffs.empty()) {
                    begin = n.beginOffset;
                    for (size_t p = 0; p < n.beginCoeffs.size() && p < vars.size(); ++p)
                        begin += n.beginCoeffs[p] * vars[p];
                }
                if (!n.endCoeffs.empty()) {
                    endInc = n.endOffset;
                    for (size_t p = 0; p < n.endCoeffs.size() && p < vars.size(); ++p)
                        endInc += n.endCoeffs[p] * vars[p];
                } else if (n.end == kDynamic && n.endBuf != kInvalidId && n.endDim >= 0 &&
                           n.endBuf < m.buffers.size() &&
                           n.endDim < static_cast<int32_t>(m.buffers[n.endBuf].dims.size())) {
                    endInc = m.buffers[n.endBuf].dims[n.endDim] - 1;
                } else if (n.end == kDynamic) {
                    endInc = io.elements - 1;
                }
                if (endInc < begin) return {};
                if (n.parallel && bodySafe(n)) {
                    const int64_t threads = decideThreads(m, io, endInc - begin + 1);
                    if (threads > 1) {
                        std::vector<Status> slots(static_cast<size_t>(threads));
                        std::vector<std::thread> pool;
                        const int64_t total = endInc - begin + 1;
                        const int64_t chunk = (total + threads - 1) / threads;
                        for (int64_t t = 0; t < threads; ++t) {
                            const int64_t b = begin + t * chunk;
                            const int64_t e = std::min(b + chunk - 1, endInc);
                            if (b > endInc) break;
                            const std::vector<int64_t> outer = vars;
                            Status* slot = &slots[static_cast<size_t>(t)];
                            pool.emplace_back([this, &n, b, e, outer, slot]() {
                                Walker child{m, io, outer};
                                *slot = child.loopRange(n, b, e);
                            });
                        }
                        for (auto& th : pool) th.join();
                        for (const Status& s : slots) {
                            if (!s.ok()) return s;
                        }
                        return {};
                    }
                }
                return loopRange(n, begin, endInc);
            }
            case Op::Compute:
                if (pairedStore == nullptr) return {};
                return pair(n, *pairedStore);
            case Op::Guard: {
                if (n.guardCoeffs.empty()) return {};
                int64_t acc = n.guardOffset;
                for (size_t p = 0; p < n.guardCoeffs.size(); ++p) {
                    const int64_t c = n.guardCoeffs[p];
                    if (c == 0) continue;
                    if (p >= vars.size()) return fail(kInvalidGraph, "walker: guard references an unbound loop var");
                    int64_t term = 0;
                    if (__builtin_mul_overflow(c, vars[p], &term) || __builtin_add_overflow(acc, term, &acc))
                        return fail(kResourceExhausted, "walker: guard form overflow");
                }
                if (acc != 0) return {};
                return childList(n.children);
            }
            case Op::Call:
                if (n.math == Math::ReduceSum) return reduceSumCall(m, io, n);
                if (n.math == Math::Softmax) return softmaxCall(m, io, n);
                if (n.math != Math::MatMul) return fail(kUnsupported, "no executor for call target");
                return gemmCall(m, io, n, false);
            default:
                return {};
        }
    }
    Status pair(const Node& compute, const Node& store) {
        for (const Expr& e : compute.exprs) {
            for (const Operand* o : {&e.a, &e.b}) {
                if (o->kind == Kind::ElemA || o->kind == Kind::ElemB)
                    return fail(kInvalidGraph, "walker: legacy element operand in a multi-dim compute");
            }
        }
        double* outP = nullptr;
        if (store.bufOut < m.buffers.size() && m.buffers[store.bufOut].isTemp) {
            outP = store.bufOut < io.temps.size() ? io.temps[store.bufOut] : nullptr;
        } else {
            outP = resolveOutput(m, io, store.bufOut);
        }
        if (outP == nullptr) return fail(kInvalidArgument, "walker: output buffer not bound");
        Evaluator ev{compute.exprs, nullptr, nullptr, io.scalars, compute.poly7, &vars, &m, &io};
        Operand target;
        target.kind = Kind::ElemIdx;
        target.index = static_cast<int64_t>(store.bufOut);
        target.coeffs = store.outCoeffs;
        target.offset = store.outOffset;
        const int64_t flat = ev.flat(target);
        if (flat < 0) return fail(kInvalidGraph, "walker: negative store address");
        const double value = ev.run(0);
        double& slot = outP[flat];
        if (store.accum == Accum::Add) {
            slot += value;
        } else if (store.accum == Accum::Max) {
            slot = (value > slot) ? value : slot;
        } else {
            slot = value;
        }
        return {};
    }
};

bool isMultiDim(const Module& m) {
    for (const Node& n : m.nodes) {
        if (n.accum != Accum::None || !n.beginCoeffs.empty() || !n.endCoeffs.empty() ||
            (n.end == kDynamic && n.endBuf != kInvalidId))
            return true;
        if (!n.outCoeffs.empty() || (n.op == Op::Guard && !n.guardCoeffs.empty())) return true;
        for (const Expr& e : n.exprs) {
            if (e.a.kind == Kind::ElemIdx || e.b.kind == Kind::ElemIdx) return true;
        }
    }
    return false;
}

Status execute(const Module& m, Bindings& io) {
    if (m.nodes.empty()) return fail(kInvalidGraph, "kernel module has no nodes");
    std::vector<std::vector<double>> tempStorage;
    tempStorage.reserve(m.buffers.size());
    for (uint32_t bid = 0; bid < m.buffers.size(); ++bid) {
        const Buffer& b = m.buffers[bid];
        if (!b.isTemp) continue;
        int64_t n = b.elements;
        if (!b.dims.empty()) {
            n = 1;
            for (int64_t d : b.dims) {
                if (d <= 0 || n > kTempElementsLimit / d)
                    return fail(kInvalidGraph, "temp buffer element count out of range");
                n *= d;
            }
        }
        if (n <= 0 || n > kTempElementsLimit) return fail(kInvalidGraph, "temp buffer element count out of range");
        if (io.temps.size() < m.buffers.size()) io.temps.resize(m.buffers.size(), nullptr);
        tempStorage.emplace_back(static_cast<size_t>(n), 0.0);
        io.temps[bid] = tempStorage.back().data();
    }
    if (isMultiDim(m)) {
        Walker w{m, io, {}};
        for (uint32_t i = 0; i < m.nodes.size(); ++i) {
            bool referenced = false;
            for (const Node& n : m.nodes) {
                for (uint32_t c : n.children) referenced = referenced || c == i;
            }
            if (referenced) continue;
            Status s = w.exec(i, nullptr);
            if (!s.ok()) return s;
        }
        return {};
    }
    for (const Node& top : m.nodes) {
        if (top.op == Op::Loop) {
            int64_t begin = top.begin, end = top.end;
            if (end == kDynamic) end = io.elements;
            if (end < begin) end = begin;
            const int64_t threads = decideThreads(m, io, end - begin);
            auto body = [&](int64_t b, int64_t e) {
                for (uint32_t cid : top.children) {
                    if (cid >= m.nodes.size()) return;
                    const Node& c = m.nodes[cid];
                    if (c.op != Op::Compute) continue;
                    const Node* store = nullptr;
                    for (uint32_t sid : top.children) {
                        if (sid < m.nodes.size() && m.nodes[sid].op == Op::Store) {
                            store = &m.nodes[sid];
                            break;
                        }
                    }
                    elementwiseRange(c, store != nullptr ? *store : c, m, io, b, e);
                }
            };
            if (threads <= 1 || top.children.empty()) {
                for (uint32_t cid : top.children) {
                    if (cid >= m.nodes.size()) return fail(kInvalidGraph, "kernel child node out of range");
                }
                body(begin, end);
            } else {
                std::vector<std::thread> pool;
                const int64_t total = end - begin;
                const int64_t chunk = (total + threads - 1) / threads;
                for (int64_t t = 0; t < threads; ++t) {
                    const int64_t b = begin + t * chunk;
                    const int64_t e = std::min(b + chunk, end);
                    if (b >= e) break;
                    pool.emplace_back([&body, b, e]() { body(b, e); });
                }
                for (auto& th : pool) th.join();
            }
        } else if (top.op == Op::Call) {
            Status s;
            if (top.math == Math::ReduceSum) {
                s = reduceSumCall(m, io, top);
            } else if (top.math == Math::Softmax) {
                s = softmaxCall(m, io, top);
            } else if (top.math == Math::MatMul) {
                s = gemmCall(m, io, top, true);
            } else {
                s = fail(kUnsupported, "no executor for call target");
            }
            if (!s.ok()) return s;
        }
    }
    return {};
}

}  // namespace oracle

// --------------------------------------------------------------- C ABI ----
extern "C" {

/// Runs a KernelModule (mlk-kernel JSON) over caller-owned f64 buffers with
/// the reference binding rules (inputs / outputs arrays, scalars, dynamic
/// element count). `hw_threads` stands in for std::thread::
/// hardware_concurrency() (capped at 4 unless the module's "threads" param
/// overrides it). Returns the reference ErrorCode value (0 = ok) and writes
/// the message into `msg`.
int oracle_execute(const char* json, size_t len, double* const* inputs, int n_inputs,
                   double* const* outputs, int n_outputs, const double* scalars,
                   int n_scalars, int64_t elements, int hw_threads, char* msg,
                   size_t msg_cap) {
    oracle::Module m;
    std::string why;
    if (!oracle::parseModule(json, len, m, why)) {
        if (msg != nullptr && msg_cap > 0) std::snprintf(msg, msg_cap, "%s", why.c_str());
        return oracle::kInvalidArgument;
    }
    oracle::Bindings io;
    for (int i = 0; i < n_inputs; ++i) io.inputs.push_back(inputs[i]);
    for (int i = 0; i < n_outputs; ++i) io.outputs.push_back(outputs[i]);
    for (int i = 0; i < n_scalars; ++i) io.scalars.push_back(scalars[i]);
    io.elements = elements;
    io.hwThreads = hw_threads;
    oracle::Status s = oracle::execute(m, io);
    if (msg != nullptr && msg_cap > 0) std::snprintf(msg, msg_cap, "%s", s.msg.c_str());
    return s.code;
}

double oracle_poly_sin(double x) { return oracle::polySin(x); }

void oracle_poly_sin_many(const double* x, double* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle::polySin(x[i]);
}

/// Blocked GEMM row block exactly as gemmRowBlock (C += A*B).
void oracle_gemm_blocked(const double* a, const double* b, double* c, int64_t m, int64_t n,
                         int64_t k, int64_t tile_m, int64_t tile_n, int64_t tile_k) {
    oracle::gemmRowBlock(a, b, c, n, k, tile_m, tile_n, tile_k, 0, m);
}

}  // extern "C"
