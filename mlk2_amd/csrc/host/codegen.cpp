// Instantiates the hand-written elementwise kernel template
// (device/elementwise_template.hip) for one planned step: a prelude of
// compile-time constants (box extents, stream dtypes and affine maps, output
// map, accumulate mode) and the chain body, followed by the template text.
#include <cstdio>
#include <string>

#include "planner.h"

namespace mlk::hip {

namespace {
#include "device_math.inc"           // kDeviceMathHeader (generated at build)
#include "elementwise_template.inc"  // kElementwiseTemplate (generated at build)

int dtypeCode(Dtype d) { return d == Dtype::F32 ? 0 : (d == Dtype::F16 ? 1 : 2); }

std::string list(const int64_t* v, int n) {
    std::string s = "{";
    for (int i = 0; i < n; ++i) {
        if (i) s += ", ";
        s += std::to_string(v[i]) + "LL";
    }
    return s + "}";
}
}  // namespace

/// mlk_elementwise_ followed by 12 hex digits of the FNV-1a hash of the
/// instance source.
std::string elementwiseKernelName(const std::string& source) {
    uint64_t h = 0xCBF29CE484222325ull;  // FNV-1a
    for (const char c : source) {
        h ^= static_cast<unsigned char>(c);
        h *= 0x100000001B3ull;
    }
    char buf[48];
    std::snprintf(buf, sizeof(buf), "mlk_elementwise_%012llx", static_cast<unsigned long long>(h >> 16));
    return buf;
}

std::string elementwiseSource(const KernelModule& km, const Step& st, std::string* kernelName) {
    const int nin = st.inputs.empty() ? 1 : static_cast<int>(st.inputs.size());
    std::string p;
    p += "#define MLK_GENERATED 1\n";
    p += "#define MLK_NIN " + std::to_string(nin) + "\n";
    p += "constexpr long long kHostSegment = " + std::to_string(kElementwiseSegment) + ";\n";
    p += "constexpr int kRank = " + std::to_string(st.rank) + ";\n";
    p += "constexpr bool kDynamicExtent = " + std::string(st.dynamicExtent ? "true" : "false") + ";\n";
    int64_t ext[4] = {st.extent[0], st.extent[1], st.extent[2], st.extent[3]};
    p += "constexpr long long kExt[4] = " + list(ext, 4) + ";\n";
    std::string dts = "{", offs = "{", cs = "{";
    for (int i = 0; i < nin; ++i) {
        const bool real = i < static_cast<int>(st.inputs.size());
        const StreamRef s = real ? st.inputs[static_cast<size_t>(i)] : StreamRef{};
        if (i) {
            dts += ", ";
            offs += ", ";
            cs += ", ";
        }
        dts += std::to_string(real ? dtypeCode(km.buffers[s.buffer].dtype) : 0);
        offs += std::to_string(s.offset) + "LL";
        int64_t c[4] = {s.coeff[0], s.coeff[1], s.coeff[2], s.coeff[3]};
        if (!real) c[st.rank - 1] = 0;
        cs += list(c, 4);
    }
    p += "constexpr int kInDt[MLK_NIN] = " + dts + "};\n";
    p += "constexpr long long kInOff[MLK_NIN] = " + offs + "};\n";
    p += "constexpr long long kInC[MLK_NIN][4] = " + cs + "};\n";
    p += "constexpr int kOutDt = " + std::to_string(dtypeCode(km.buffers[st.out.buffer].dtype)) + ";\n";
    p += "constexpr long long kOutOff = " + std::to_string(st.out.offset) + "LL;\n";
    int64_t oc[4] = {st.out.coeff[0], st.out.coeff[1], st.out.coeff[2], st.out.coeff[3]};
    p += "constexpr long long kOutC[4] = " + list(oc, 4) + ";\n";
    p += "constexpr int kAccum = " +
         std::to_string(st.accum == AccumMode::Add ? 1 : (st.accum == AccumMode::Max ? 2 : 0)) + ";\n";
    // One statement per line of a body, joined with line continuations.
    auto macro = [](const std::string& name, const std::string& body) {
        std::string joined = "#define " + name + " \\\n";
        size_t start = 0;
        while (start < body.size()) {
            size_t nl = body.find('\n', start);
            if (nl == std::string::npos) nl = body.size();
            joined += body.substr(start, nl - start) + " \\\n";
            start = nl + 1;
        }
        return joined + "\n";
    };
    p += macro("MLK_CHAIN_BODY", st.chainBody);
    if (!st.chainExact.empty()) p += macro("MLK_CHAIN_EXACT", st.chainExact);
    const std::string text = p + kDeviceMathHeader + kElementwiseTemplate;
    const std::string name = elementwiseKernelName(text);
    if (kernelName != nullptr) *kernelName = name;
    return "#define MLK_KERNEL_NAME " + name + "\n" + text;
}

const char* deviceMathHeader() { return kDeviceMathHeader; }

}  // namespace mlk::hip
