// Reader for the "mlk-kernel" document and small Kernel IR utilities.
#include "kernel_ir.h"

#include <cmath>
#include <cstdlib>
#include <cstring>

namespace mlk::hip {

namespace {

// A compact JSON value tree: arrays/objects hold indices into one pool.
struct JNode {
    enum Type : uint8_t { Null, True, False, Number, String, Array, Object } type{Null};
    double number{0.0};
    int64_t integer{0};
    bool isInteger{false};
    std::string text;                      // String payload or object key
    std::vector<uint32_t> items;           // Array elements / Object members
};

class JsonReader {
public:
    JsonReader(const char* s, size_t n) : s_(s), n_(n) {}

    bool parse(uint32_t& root) {
        skip();
        if (!value(root, 0)) return false;
        skip();
        return pos_ == n_;
    }
    const JNode& at(uint32_t i) const { return pool_[i]; }
    const std::string& why() const { return why_; }

    /// Member `key` of object `obj`, or kInvalidId.
    uint32_t member(uint32_t obj, const char* key) const {
        if (obj == kInvalidId || pool_[obj].type != JNode::Object) return kInvalidId;
        for (const uint32_t m : pool_[obj].items) {
            if (pool_[m].text == key) return pool_[m].items.empty() ? kInvalidId : pool_[m].items[0];
        }
        return kInvalidId;
    }

private:
    const char* s_;
    size_t n_;
    size_t pos_{0};
    std::vector<JNode> pool_;
    std::string why_;

    void skip() {
        while (pos_ < n_ && (s_[pos_] == ' ' || s_[pos_] == '\t' || s_[pos_] == '\n' || s_[pos_] == '\r')) ++pos_;
    }
    bool fail(const char* m) {
        why_ = std::string(m) + " at byte " + std::to_string(pos_);
        return false;
    }
    bool word(const char* w) {
        const size_t k = std::strlen(w);
        if (n_ - pos_ >= k && std::memcmp(s_ + pos_, w, k) == 0) {
            pos_ += k;
            return true;
        }
        return false;
    }
    uint32_t make(JNode::Type t) {
        pool_.emplace_back();
        pool_.back().type = t;
        return static_cast<uint32_t>(pool_.size() - 1);
    }
    bool str(std::string& out) {
        if (pos_ >= n_ || s_[pos_] != '"') return fail("expected string");
        ++pos_;
        while (pos_ < n_ && s_[pos_] != '"') {
            char c = s_[pos_++];
            if (c == '\\') {
                if (pos_ >= n_) return fail("bad escape");
                const char e = s_[pos_++];
                if (e == 'u') {
                    if (n_ - pos_ < 4) return fail("bad unicode escape");
                    pos_ += 4;
                    c = '?';
                } else {
                    c = e == 'n' ? '\n' : e == 't' ? '\t' : e == 'r' ? '\r' : e;
                }
            }
            out.push_back(c);
        }
        if (pos_ >= n_) return fail("unterminated string");
        ++pos_;
        return true;
    }
    bool value(uint32_t& out, int depth) {
        if (depth > 64) return fail("nesting too deep");
        skip();
        if (pos_ >= n_) return fail("unexpected end");
        const char c = s_[pos_];
        if (c == '{') {
            ++pos_;
            out = make(JNode::Object);
            skip();
            if (pos_ < n_ && s_[pos_] == '}') {
                ++pos_;
                return true;
            }
            for (;;) {
                skip();
                std::string key;
                if (!str(key)) return false;
                skip();
                if (pos_ >= n_ || s_[pos_] != ':') return fail("expected ':'");
                ++pos_;
                uint32_t v = 0;
                if (!value(v, depth + 1)) return false;
                const uint32_t m = make(JNode::Null);
                pool_[m].text = std::move(key);
                pool_[m].items.push_back(v);
                pool_[out].items.push_back(m);
                skip();
                if (pos_ < n_ && s_[pos_] == ',') {
                    ++pos_;
                    continue;
                }
                if (pos_ < n_ && s_[pos_] == '}') {
                    ++pos_;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            ++pos_;
            out = make(JNode::Array);
            skip();
            if (pos_ < n_ && s_[pos_] == ']') {
                ++pos_;
                return true;
            }
            for (;;) {
                uint32_t v = 0;
                if (!value(v, depth + 1)) return false;
                pool_[out].items.push_back(v);
                skip();
                if (pos_ < n_ && s_[pos_] == ',') {
                    ++pos_;
                    continue;
                }
                if (pos_ < n_ && s_[pos_] == ']') {
                    ++pos_;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            out = make(JNode::String);
            std::string t;
            if (!str(t)) return false;
            pool_[out].text = std::move(t);
            return true;
        }
        if (word("true")) { out = make(JNode::True); return true; }
        if (word("false")) { out = make(JNode::False); return true; }
        if (word("null")) { out = make(JNode::Null); return true; }
        if (word("NaN")) { out = make(JNode::Number); pool_[out].number = NAN; return true; }
        if (word("Infinity")) { out = make(JNode::Number); pool_[out].number = INFINITY; return true; }
        if (word("-Infinity")) { out = make(JNode::Number); pool_[out].number = -INFINITY; return true; }
        const size_t start = pos_;
        bool frac = false;
        while (pos_ < n_) {
            const char d = s_[pos_];
            if ((d >= '0' && d <= '9') || d == '-' || d == '+') {
                ++pos_;
            } else if (d == '.' || d == 'e' || d == 'E') {
                frac = true;
                ++pos_;
            } else {
                break;
            }
        }
        if (pos_ == start) return fail("unexpected character");
        const std::string tok(s_ + start, pos_ - start);
        out = make(JNode::Number);
        char* endp = nullptr;
        if (frac) {
            pool_[out].number = std::strtod(tok.c_str(), &endp);
        } else {
            pool_[out].isInteger = true;
            pool_[out].integer = std::strtoll(tok.c_str(), &endp, 10);
            pool_[out].number = static_cast<double>(pool_[out].integer);
        }
        if (endp == nullptr || *endp != '\0') return fail("malformed number");
        return true;
    }
};

MathOp mathFromName(const std::string& s) {
    static const struct {
        const char* name;
        MathOp op;
    } kNames[] = {{"add", MathOp::Add},   {"sub", MathOp::Sub},     {"mul", MathOp::Mul},
                  {"div", MathOp::Div},   {"neg", MathOp::Neg},     {"pow", MathOp::Pow},
                  {"exp", MathOp::Exp},   {"log", MathOp::Log},     {"sin", MathOp::Sin},
                  {"cos", MathOp::Cos},   {"tan", MathOp::Tan},     {"tanh", MathOp::Tanh},
                  {"sqrt", MathOp::Sqrt}, {"rsqrt", MathOp::Rsqrt}, {"erf", MathOp::Erf},
                  {"gelu", MathOp::Gelu}, {"matmul", MathOp::MatMul},
                  {"reduce_sum", MathOp::ReduceSum}, {"softmax", MathOp::Softmax}};
    for (const auto& e : kNames) {
        if (s == e.name) return e.op;
    }
    return MathOp::Other;
}

bool opFromName(const std::string& s, KernelOp& op) {
    static const struct {
        const char* name;
        KernelOp op;
    } kNames[] = {{"loop", KernelOp::Loop},       {"compute", KernelOp::Compute},
                  {"load", KernelOp::Load},       {"store", KernelOp::Store},
                  {"alloc", KernelOp::AllocBuffer}, {"copy", KernelOp::CopyBuffer},
                  {"barrier", KernelOp::Barrier}, {"trace", KernelOp::Trace},
                  {"guard", KernelOp::Guard},     {"call", KernelOp::Call}};
    for (const auto& e : kNames) {
        if (s == e.name) {
            op = e.op;
            return true;
        }
    }
    return false;
}

Dtype dtypeFromName(const std::string& s) {
    if (s == "f32") return Dtype::F32;
    if (s == "f16") return Dtype::F16;
    if (s == "f64") return Dtype::F64;
    return Dtype::Other;
}

struct Decoder {
    const JsonReader& r;

    int64_t integer(uint32_t v, int64_t fb) const {
        if (v == kInvalidId || r.at(v).type != JNode::Number) return fb;
        return r.at(v).isInteger ? r.at(v).integer : static_cast<int64_t>(r.at(v).number);
    }
    double number(uint32_t v, double fb) const {
        if (v == kInvalidId) return fb;
        if (r.at(v).type == JNode::Null) return NAN;  // the reference writes NaN as null
        if (r.at(v).type != JNode::Number) return fb;
        return r.at(v).number;
    }
    bool boolean(uint32_t v) const { return v != kInvalidId && r.at(v).type == JNode::True; }
    std::string text(uint32_t v) const {
        return (v == kInvalidId || r.at(v).type != JNode::String) ? std::string() : r.at(v).text;
    }
    std::vector<int64_t> ints(uint32_t v) const {
        std::vector<int64_t> out;
        if (v == kInvalidId || r.at(v).type != JNode::Array) return out;
        for (const uint32_t it : r.at(v).items) out.push_back(integer(it, 0));
        return out;
    }
    bool operand(uint32_t v, KernelOperand& o) const {
        if (v == kInvalidId) return true;  // absent: Const 0.0
        const std::string k = text(r.member(v, "kind"));
        using K = KernelOperand::Kind;
        if (k == "const") {
            o.kind = K::Const;
            o.constValue = number(r.member(v, "value"), 0.0);
            // KernelModule::toJson spells +-inf as +-1e308 (serializeDouble,
            // compiler/src/core/json.cpp:301-312); read that spelling back as
            // the infinity it stands for. A module that literally holds
            // +-1e308 is indistinguishable and is read as +-inf too.
            if (o.constValue == 1e308 || o.constValue == -1e308) {
                o.constValue = o.constValue > 0 ? INFINITY : -INFINITY;
            }
        } else if (k == "elem_a") {
            o.kind = K::ElemA;
        } else if (k == "elem_b") {
            o.kind = K::ElemB;
        } else if (k == "scalar_param") {
            o.kind = K::ScalarParam;
            o.index = integer(r.member(v, "index"), 0);
        } else if (k == "temp") {
            o.kind = K::Temp;
            o.index = integer(r.member(v, "index"), 0);
        } else if (k == "elem_idx") {
            o.kind = K::ElemIdx;
            o.index = integer(r.member(v, "buffer"), -1);
            o.idxCoeffs = ints(r.member(v, "coeffs"));
            o.idxOffset = integer(r.member(v, "offset"), 0);
        } else {
            return false;
        }
        return true;
    }
};

}  // namespace

Result<KernelModule> parseKernelModule(const char* text, size_t len) {
    JsonReader rd(text, len);
    uint32_t root = 0;
    if (!rd.parse(root)) return err(ErrorCode::ParseError, "mlk-kernel: " + rd.why());
    Decoder d{rd};
    if (d.text(rd.member(root, "format")) != "mlk-kernel") {
        return err(ErrorCode::ParseError, "mlk-kernel: missing format tag");
    }
    KernelModule km;
    km.name = d.text(rd.member(root, "name"));
    const uint32_t bufs = rd.member(root, "buffers");
    const uint32_t nodes = rd.member(root, "nodes");
    if (bufs == kInvalidId || nodes == kInvalidId || rd.at(bufs).type != JNode::Array ||
        rd.at(nodes).type != JNode::Array) {
        return err(ErrorCode::ParseError, "mlk-kernel: buffers/nodes arrays required");
    }
    for (const uint32_t b : rd.at(bufs).items) {
        KernelBuffer kb;
        kb.name = d.text(rd.member(b, "name"));
        const std::string dt = d.text(rd.member(b, "dtype"));
        kb.dtype = dt.empty() ? Dtype::F32 : dtypeFromName(dt);
        kb.isInput = d.boolean(rd.member(b, "input"));
        kb.isOutput = d.boolean(rd.member(b, "output"));
        kb.isTemp = d.boolean(rd.member(b, "temp"));
        kb.elements = d.integer(rd.member(b, "elements"), kDynamicBound);
        kb.dims = d.ints(rd.member(b, "dims"));
        km.buffers.push_back(std::move(kb));
    }
    std::vector<uint32_t> callMath;  // Call nodes written without "math"
    for (const uint32_t n : rd.at(nodes).items) {
        KernelNode kn;
        if (!opFromName(d.text(rd.member(n, "op")), kn.op)) {
            return err(ErrorCode::ParseError, "mlk-kernel: unknown node op");
        }
        const uint32_t mth = rd.member(n, "math");
        if (mth != kInvalidId) kn.math = mathFromName(d.text(mth));
        const bool mathAbsent = mth == kInvalidId;
        kn.family = d.text(rd.member(n, "family"));
        kn.var = d.text(rd.member(n, "var"));
        kn.begin = d.integer(rd.member(n, "begin"), 0);
        kn.end = d.integer(rd.member(n, "end"), kDynamicBound);
        kn.step = d.integer(rd.member(n, "step"), 1);
        const uint32_t eb = rd.member(n, "end_buf");
        if (eb != kInvalidId) kn.endBuf = static_cast<uint32_t>(d.integer(eb, -1));
        kn.endDim = static_cast<int32_t>(d.integer(rd.member(n, "end_dim"), -1));
        kn.beginCoeffs = d.ints(rd.member(n, "begin_coeffs"));
        kn.beginOffset = d.integer(rd.member(n, "begin_offset"), 0);
        kn.endCoeffs = d.ints(rd.member(n, "end_coeffs"));
        kn.endOffset = d.integer(rd.member(n, "end_offset"), 0);
        kn.outIndexCoeffs = d.ints(rd.member(n, "out_index_coeffs"));
        kn.outIndexOffset = d.integer(rd.member(n, "out_index_offset"), 0);
        if (d.boolean(rd.member(n, "accumulate"))) {
            kn.accum = d.text(rd.member(n, "accum_mode")) == "max" ? AccumMode::Max : AccumMode::Add;
        }
        kn.parallel = d.boolean(rd.member(n, "parallel"));
        kn.vectorHint = d.boolean(rd.member(n, "vector_hint"));
        kn.guardCoeffs = d.ints(rd.member(n, "guard_coeffs"));
        kn.guardOffset = d.integer(rd.member(n, "guard_offset"), 0);
        const uint32_t a = rd.member(n, "a");
        const uint32_t b = rd.member(n, "b");
        const uint32_t o = rd.member(n, "out");
        if (a != kInvalidId) kn.bufferA = static_cast<uint32_t>(d.integer(a, -1));
        if (b != kInvalidId) kn.bufferB = static_cast<uint32_t>(d.integer(b, -1));
        if (o != kInvalidId) kn.bufferOut = static_cast<uint32_t>(d.integer(o, -1));
        const uint32_t xs = rd.member(n, "exprs");
        if (xs != kInvalidId && rd.at(xs).type == JNode::Array) {
            for (const uint32_t x : rd.at(xs).items) {
                KernelExpr e;
                e.op = mathFromName(d.text(rd.member(x, "op")));
                if (!d.operand(rd.member(x, "a"), e.a) || !d.operand(rd.member(x, "b"), e.b)) {
                    return err(ErrorCode::ParseError, "mlk-kernel: unknown operand kind");
                }
                kn.exprs.push_back(std::move(e));
            }
        }
        for (const int64_t c : d.ints(rd.member(n, "children"))) {
            kn.children.push_back(static_cast<uint32_t>(c));
        }
        if (kn.op == KernelOp::Call && mathAbsent) callMath.push_back(static_cast<uint32_t>(km.nodes.size()));
        km.nodes.push_back(std::move(kn));
    }
    // KernelModule::toJson writes "math" on Compute nodes only
    // (compiler/src/support/kernel_ir.cpp:130-135), so a Call's target comes
    // from its operands, as the reference builds them (tools/mlk-poly/
    // poly_bench.cpp:121-158, lower.to_kernel_ir.cpp:114-144): a bound B is
    // MatMul; otherwise a rank-1 output is ReduceSum (rank-2 in, rank-1 out)
    // and any other output Softmax (rank-2 in and out).
    for (const uint32_t id : callMath) {
        KernelNode& c = km.nodes[id];
        if (c.bufferB != kInvalidId) {
            c.math = MathOp::MatMul;
        } else if (c.bufferOut < km.buffers.size() && km.buffers[c.bufferOut].dims.size() == 1) {
            c.math = MathOp::ReduceSum;
        } else {
            c.math = MathOp::Softmax;
        }
    }
    const uint32_t sched = rd.member(root, "schedule");
    if (sched != kInvalidId && rd.at(sched).type == JNode::Object) {
        for (const uint32_t m : rd.at(sched).items) {
            km.schedule.emplace_back(rd.at(m).text, d.integer(rd.at(m).items[0], 0));
        }
    }
    return km;
}

bool isMultiDimModule(const KernelModule& km) {
    using K = KernelOperand::Kind;
    for (const KernelNode& n : km.nodes) {
        if (n.accum != AccumMode::None || !n.beginCoeffs.empty() || !n.endCoeffs.empty() ||
            (n.end == kDynamicBound && n.endBuf != kInvalidId) || n.hasAffineStore() ||
            (n.op == KernelOp::Guard && n.hasAffineGuard())) {
            return true;
        }
        for (const KernelExpr& e : n.exprs) {
            if (e.a.kind == K::ElemIdx || e.b.kind == K::ElemIdx) return true;
        }
    }
    return false;
}

std::vector<uint32_t> forestRoots(const KernelModule& km) {
    std::vector<bool> referenced(km.nodes.size(), false);
    for (const KernelNode& n : km.nodes) {
        for (const uint32_t c : n.children) {
            if (c < referenced.size()) referenced[c] = true;
        }
    }
    std::vector<uint32_t> roots;
    for (uint32_t i = 0; i < km.nodes.size(); ++i) {
        if (!referenced[i]) roots.push_back(i);
    }
    return roots;
}

int dtypeBytes(Dtype d) {
    switch (d) {
        case Dtype::F32: return 4;
        case Dtype::F16: return 2;
        case Dtype::F64: return 8;
        case Dtype::Other: return 0;
    }
    return 0;
}

const char* mathOpName(MathOp op) {
    static const char* kNames[] = {"add", "sub", "mul", "div", "neg", "pow", "exp", "log",
                                   "sin", "cos", "tan", "tanh", "sqrt", "rsqrt", "erf", "gelu",
                                   "matmul", "reduce_sum", "softmax", "?"};
    return kNames[static_cast<int>(op)];
}

bool isUnaryMath(MathOp op) {
    switch (op) {
        case MathOp::Neg: case MathOp::Exp: case MathOp::Log: case MathOp::Sin:
        case MathOp::Cos: case MathOp::Tan: case MathOp::Tanh: case MathOp::Sqrt:
        case MathOp::Rsqrt: case MathOp::Erf: case MathOp::Gelu:
            return true;
        default:
            return false;
    }
}

namespace {
uint64_t mix(uint64_t h, uint64_t v) {
    h ^= v + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2);
    return h;
}
uint64_t mixStr(uint64_t h, const std::string& s) {
    for (const char c : s) h = mix(h, static_cast<unsigned char>(c));
    return mix(h, s.size());
}
uint64_t mixVec(uint64_t h, const std::vector<int64_t>& v) {
    for (const int64_t x : v) h = mix(h, static_cast<uint64_t>(x));
    return mix(h, v.size());
}
uint64_t mixOperand(uint64_t h, const KernelOperand& o) {
    h = mix(h, static_cast<uint64_t>(o.kind));
    h = mix(h, static_cast<uint64_t>(o.index));
    uint64_t bits = 0;
    std::memcpy(&bits, &o.constValue, sizeof(bits));
    h = mix(h, o.kind == KernelOperand::Kind::Const ? bits : 0);
    h = mixVec(h, o.idxCoeffs);
    return mix(h, static_cast<uint64_t>(o.idxOffset));
}
}  // namespace

uint64_t moduleHash(const KernelModule& km) {
    uint64_t h = 0x6D6C6B2D6B65726EULL;
    for (const KernelBuffer& b : km.buffers) {
        h = mix(h, static_cast<uint64_t>(b.dtype));
        h = mix(h, (b.isInput ? 1u : 0u) | (b.isOutput ? 2u : 0u) | (b.isTemp ? 4u : 0u));
        h = mix(h, static_cast<uint64_t>(b.elements));
        h = mixVec(h, b.dims);
    }
    for (const KernelNode& n : km.nodes) {
        h = mix(h, static_cast<uint64_t>(n.op));
        h = mix(h, static_cast<uint64_t>(n.math));
        h = mix(h, static_cast<uint64_t>(n.begin));
        h = mix(h, static_cast<uint64_t>(n.end));
        h = mix(h, static_cast<uint64_t>(n.step));
        h = mixVec(h, n.beginCoeffs);
        h = mix(h, static_cast<uint64_t>(n.beginOffset));
        h = mixVec(h, n.endCoeffs);
        h = mix(h, static_cast<uint64_t>(n.endOffset));
        h = mix(h, n.endBuf);
        h = mix(h, static_cast<uint64_t>(n.endDim));
        h = mix(h, n.bufferA);
        h = mix(h, n.bufferB);
        h = mix(h, n.bufferOut);
        h = mixVec(h, n.outIndexCoeffs);
        h = mix(h, static_cast<uint64_t>(n.outIndexOffset));
        h = mix(h, static_cast<uint64_t>(n.accum));
        h = mixVec(h, n.guardCoeffs);
        h = mix(h, static_cast<uint64_t>(n.guardOffset));
        h = mixStr(h, n.family);
        for (const KernelExpr& e : n.exprs) {
            h = mix(h, static_cast<uint64_t>(e.op));
            h = mixOperand(h, e.a);
            h = mixOperand(h, e.b);
        }
        for (const uint32_t c : n.children) h = mix(h, c);
        h = mix(h, n.children.size());
    }
    for (const auto& kv : km.schedule) {
        h = mixStr(h, kv.first);
        h = mix(h, static_cast<uint64_t>(kv.second));
    }
    return h;
}

}  // namespace mlk::hip
