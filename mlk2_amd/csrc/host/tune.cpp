// Variant search for a built artifact: the gfx950 counterpart of fastkernel's
// native path (fastkernel/src/fast_kernel.cpp:797-887). Each step whose
// hand-written kernel has more than one launch form for its shape gets every
// form timed on the caller's device-resident buffers; a form is certified
// when its outputs match the default form's within half of the artifact's
// tolerance policy (bit for bit under an exact policy) -- the reference's
// identity gate (fast_kernel.cpp:1251-1261) restated for tolerance policies;
// the fastest certified form is kept. The choice is stored under a
// fingerprint binding the module hash, the declared target, the hipRTC
// version, the policy and the device (fast_kernel.cpp:727-763), in
// <cache_dir>/fk-<fingerprint>.json, which a later build with the same cache
// directory applies without searching again.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "driver.h"
#include "../device/runtime_abi.h"
#include "../../../include/mlk_hip.h"

namespace mlk::hip {

namespace {

constexpr uint32_t kCacheFormatVersion = 1;

uint64_t fnv(uint64_t h, const void* p, size_t n) {
    const unsigned char* b = static_cast<const unsigned char*>(p);
    for (size_t i = 0; i < n; ++i) {
        h ^= b[i];
        h *= 0x100000001B3ull;
    }
    return h;
}

uint64_t fnvStr(uint64_t h, const std::string& s) {
    const uint64_t n = s.size();
    h = fnv(h, &n, sizeof(n));
    return fnv(h, s.data(), s.size());
}

bool readText(const std::string& path, std::string& out) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (f == nullptr) return false;
    char buf[4096];
    size_t n = 0;
    while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) out.append(buf, n);
    std::fclose(f);
    return true;
}

bool writeTextAtomic(const std::string& path, const std::string& text) {
    const std::string tmp = path + ".tmp";
    FILE* f = std::fopen(tmp.c_str(), "wb");
    if (f == nullptr) return false;
    const bool ok = std::fwrite(text.data(), 1, text.size(), f) == text.size();
    std::fclose(f);
    if (!ok || std::rename(tmp.c_str(), path.c_str()) != 0) {
        std::remove(tmp.c_str());
        return false;
    }
    return true;
}

std::string num(double v) {
    char b[64];
    std::snprintf(b, sizeof(b), "%.6g", v);
    return b;
}

const char* kindName(StepKind k) {
    switch (k) {
        case StepKind::Elementwise: return "elementwise";
        case StepKind::Softmax: return "softmax";
        case StepKind::Gemm: return "gemm";
        case StepKind::RowSum: return "rowsum";
        case StepKind::ScoreSoftmax: return "score-softmax";
        case StepKind::Nest: return "loop-nest";
        case StepKind::Fail: return "empty";
    }
    return "?";
}

/// Largest reduction length of the plan's GEMM steps (tol-rel1e-5sqrtk).
int64_t maxK(const Plan& plan) {
    int64_t k = 1;
    for (const Step& st : plan.steps) {
        if (st.kind == StepKind::Gemm) k = std::max(k, st.k);
    }
    return k;
}

/// Certification threshold of a policy: half its tolerance (negative: bits).
double threshold(const std::string& policy, int64_t k) {
    if (policy.rfind("bitexact", 0) == 0) return -1.0;
    if (policy.rfind("tol-4ulp", 0) == 0) return -4.0;   // f32 ULP distance
    if (policy.rfind("tol-rel1e-6", 0) == 0) return 0.5e-6;
    if (policy.rfind("tol-rel1e-5sqrtk", 0) == 0) return 0.5e-5 * std::sqrt(static_cast<double>(k));
    if (policy.rfind("tol-rel1e-2", 0) == 0) return 0.5e-2;
    return -1.0;
}

int64_t orderedF32(float f) {
    int32_t i;
    std::memcpy(&i, &f, sizeof(i));
    return i < 0 ? -static_cast<int64_t>(i & 0x7FFFFFFF) : static_cast<int64_t>(i);
}

/// Compares candidate outputs with the reference ones under `thr`; returns
/// whether they pass and the worst measure (relative error or ULPs).
bool compare(const std::vector<std::vector<double>>& ref, const std::vector<std::vector<double>>& got,
             double thr, double& worst) {
    worst = 0.0;
    bool ok = true;
    for (size_t b = 0; b < ref.size(); ++b) {
        for (size_t i = 0; i < ref[b].size(); ++i) {
            const double r = ref[b][i], g = got[b][i];
            if (std::isnan(r) || std::isnan(g)) {
                if (std::isnan(r) != std::isnan(g)) {
                    ok = false;
                    worst = INFINITY;
                }
                continue;
            }
            if (thr == -1.0) {
                uint64_t rb, gb;
                std::memcpy(&rb, &r, 8);
                std::memcpy(&gb, &g, 8);
                if (rb != gb) {
                    ok = false;
                    worst = std::max(worst, std::fabs(g - r));
                }
            } else if (thr < 0.0) {
                const double u = static_cast<double>(std::llabs(orderedF32(static_cast<float>(g)) -
                                                                orderedF32(static_cast<float>(r))));
                worst = std::max(worst, u);
                if (u > -thr) ok = false;
            } else {
                const double e = std::fabs(g - r) / std::max(std::fabs(r), 1.0);
                worst = std::max(worst, e);
                if (!(e <= thr)) ok = false;
            }
        }
    }
    return ok;
}

/// Elements of a buffer from its dims, else its element count; unknown for
/// a dynamic extent without dims (fast_kernel.cpp:211-226).
int64_t bufferElements(const KernelBuffer& b, bool& known) {
    if (!b.dims.empty()) {
        int64_t prod = 1;
        for (const int64_t d : b.dims) {
            if (d < 0 || (d > 0 && prod > (int64_t{1} << 40) / d)) {
                known = false;
                return 0;
            }
            prod *= d;
        }
        return prod;
    }
    if (b.elements >= 0 && b.elements < kDynamicBound) return b.elements;
    known = false;
    return 0;
}

/// The reference's operation walk (fast_kernel.cpp:228-317): a Compute node
/// adds one op per expression plus one per accumulate store, a Call node
/// its class model (MatMul 2MKN, ReduceSum one per element of A, Softmax 5
/// per element), anything else leaves the count unknown. Like the
/// reference, the walk is started from every node and recurses into
/// children, so a nested node is counted once per path to it.
void walkOps(const KernelModule& km, const KernelNode& node, EssentialWork& w, int depth) {
    if (depth > 64) {
        w.opsKnown = false;
        return;
    }
    constexpr int64_t kCap = int64_t{1} << 40;
    if (node.op == KernelOp::Compute && w.opsKnown) {
        const int64_t add = static_cast<int64_t>(node.exprs.size()) + (node.accum != AccumMode::None ? 1 : 0);
        if (add > kCap - w.minOps) {
            w.opsKnown = false;
        } else {
            w.minOps += add;
        }
    } else if (node.op == KernelOp::Call && w.opsKnown) {
        bool known = true;
        if (node.bufferA >= km.buffers.size()) {
            w.opsKnown = false;
        } else {
            const int64_t aElems = bufferElements(km.buffers[node.bufferA], known);
            if (!known) {
                w.opsKnown = false;
            } else if (node.math == MathOp::MatMul) {
                const KernelBuffer* ba = &km.buffers[node.bufferA];
                const KernelBuffer* bb = node.bufferB < km.buffers.size() ? &km.buffers[node.bufferB] : nullptr;
                if (bb == nullptr || ba->dims.size() < 2 || bb->dims.size() < 2 || ba->dims[0] <= 0 ||
                    ba->dims[1] <= 0 || bb->dims.back() <= 0) {
                    w.opsKnown = false;
                } else {
                    const int64_t mk = ba->dims[0] * ba->dims[1];
                    if (mk > kCap - w.minOps) {
                        w.opsKnown = false;
                    } else {
                        w.minOps += 2 * mk * bb->dims.back();
                    }
                }
            } else if (node.math == MathOp::ReduceSum) {
                if (aElems > kCap - w.minOps) {
                    w.opsKnown = false;
                } else {
                    w.minOps += aElems;
                }
            } else if (node.math == MathOp::Softmax) {
                if (aElems > (kCap - w.minOps) / 5) {
                    w.opsKnown = false;
                } else {
                    w.minOps += 5 * aElems;
                }
            } else {
                w.opsKnown = false;
            }
        }
    }
    for (const uint32_t c : node.children) {
        if (c >= km.nodes.size()) {
            w.opsKnown = false;
            return;
        }
        walkOps(km, km.nodes[c], w, depth + 1);
    }
}

}  // namespace

EssentialWork essentialWork(const KernelModule& km) {
    EssentialWork w;
    // Bytes: every non-temp input or output buffer moved once, at its own
    // element size (the reference counts 8 bytes for every element).
    for (const KernelBuffer& b : km.buffers) {
        if (b.isTemp || (!b.isInput && !b.isOutput)) continue;
        bool known = true;
        const int64_t elems = bufferElements(b, known);
        if (!known || elems > (int64_t{1} << 40)) {
            w.bytesKnown = false;
            break;
        }
        w.minBytes += elems * dtypeBytes(b.dtype);
    }
    for (const KernelNode& n : km.nodes) {
        walkOps(km, n, w, 0);
        if (!w.opsKnown) break;
    }
    return w;
}

double peakOpsPerSec(const KernelModule& km, const Plan& plan) {
    // MI355X datasheet (dense): f16 MFMA 2.5 PFLOP/s, f32 157.3 TFLOP/s,
    // f64 78.6 TFLOP/s. A plan with an f16 GEMM is priced at the f16 rate,
    // one touching only f64 buffers at the f64 rate, anything else at f32.
    bool allF64 = true;
    for (const KernelBuffer& b : km.buffers) {
        if (!b.isTemp && b.dtype != Dtype::F64) allF64 = false;
    }
    for (const Step& st : plan.steps) {
        if ((st.kind == StepKind::Gemm && st.a != kInvalidId && km.buffers[st.a].dtype == Dtype::F16) ||
            st.kind == StepKind::ScoreSoftmax) {
            return 2.5e15;
        }
    }
    return allF64 ? 78.6e12 : 157.3e12;
}

const MeasuredEnvironment& measuredEnvironment() {
    static std::once_flag once;
    static MeasuredEnvironment env;
    std::call_once(once, [] {
        double bw = 0.0, f16 = 0.0;
        if (mlkd_probe_environment(&bw, &f16, nullptr) == 0 && bw > 0.0 && f16 > 0.0) {
            env.ok = true;
            env.bytesPerSec = bw;
            env.f16FlopsPerSec = f16;
        }
    });
    return env;
}

double rooflineLowerSec(const EssentialWork& w, double bytesPerSec, double opsPerSec) {
    if (!w.bytesKnown || !w.opsKnown || bytesPerSec <= 0.0 || opsPerSec <= 0.0) return 0.0;
    return std::max(static_cast<double>(w.minBytes) / bytesPerSec, static_cast<double>(w.minOps) / opsPerSec);
}

std::string launchCoverage(const KernelModule& km, const Step& st, int64_t elements) {
    // Each launcher's decomposition restated: instances of the step, the
    // workgroups that carry them, and whether their union is the domain
    // exactly once. Grid-stride forms cover any instance count; tiled forms
    // cover when the tile divides the extent (the launcher checks the same
    // divisibility and falls back to the bounds-checked general kernel).
    int64_t instances = 0, workgroups = 0, perGroup = 0;
    bool covered = true;
    const char* form = "";
    switch (st.kind) {
        case StepKind::Elementwise: {
            const int64_t w = st.dynamicExtent ? elements - st.dynBegin : st.extent[st.rank - 1];
            int64_t rows = 1;
            for (int d = 0; d + 1 < st.rank; ++d) rows *= st.extent[d];
            instances = rows * std::max<int64_t>(w, 0);
            const int64_t segs =
                rows * ((std::max<int64_t>(w, 0) + kElementwiseSegment - 1) / kElementwiseSegment);
            workgroups = std::min<int64_t>(std::max<int64_t>((segs * 64 + 255) / 256, 1), 16384);
            perGroup = 4 * kElementwiseSegment;
            form = "grid-stride 512-element segments, one per wave";
            break;
        }
        case StepKind::Nest: {
            const int nf = st.variant >= 0 ? st.variant : 0;
            const int64_t wg = nestFormThreads(nf);
            instances = nestFormInstances(st, nf);
            workgroups = std::min<int64_t>(std::max<int64_t>((st.threads + wg - 1) / wg, 1), 16384);
            perGroup = wg;
            form = "grid-stride over the collapsed parallel loops";
            break;
        }
        case StepKind::Softmax: {
            // f32 rows of at most 8192 (cols % 4 == 0) run the wave path:
            // form 5 (the default) two rows per wave, form 1 a fixed grid of
            // 2048 waves, the other forms a row per wave, at most 8192
            // workgroups; anything else a workgroup per row.
            instances = st.rows;
            auto dt = [&](uint32_t b) { return km.buffers[b].dtype; };
            const bool wave = dt(st.x) == Dtype::F32 && dt(st.y) == Dtype::F32 && st.cols % 4 == 0 && st.cols <= 8192;
            const int v = st.variant >= 0 ? st.variant : 5;
            if (!wave) {
                workgroups = std::min<int64_t>(std::max<int64_t>(st.rows, 1), 65536);
                perGroup = 1;
                form = "a workgroup per row, grid-stride";
            } else if (v == 5) {
                workgroups = std::min<int64_t>(std::max<int64_t>(((st.rows + 1) / 2 + 3) / 4, 1), 8192);
                perGroup = 8;
                form = "two adjacent rows per wave, grid-stride";
            } else if (v == 1) {
                workgroups = (std::min<int64_t>(std::max<int64_t>(st.rows, 1), 2048) + 3) / 4;
                perGroup = 4;
                form = "rows pipelined over a fixed grid of waves";
            } else {
                workgroups = std::min<int64_t>(std::max<int64_t>((st.rows + 3) / 4, 1), 8192);
                perGroup = 4;
                form = "a row per wave, grid-stride";
            }
            break;
        }
        case StepKind::RowSum:
            instances = st.rows;
            workgroups = std::min<int64_t>(std::max<int64_t>((st.rows + 3) / 4, 1), 16384);
            perGroup = 4;
            form = "a row per wave, grid-stride";
            break;
        case StepKind::Gemm: {
            // f16 x f16 -> f32 with M, N % 256 and K % 64 runs the MFMA forms
            // on 256 x 256 tiles (forms 5 and 6: 128 x 256); f32 with M, N % 64
            // and K % 32 the 64 x 64 MFMA tiles; anything else the
            // bounds-checked 64 x 64 general kernel.
            instances = st.m * st.n;
            auto dt = [&](uint32_t b) { return km.buffers[b].dtype; };
            const bool f16 = dt(st.a) == Dtype::F16 && dt(st.b) == Dtype::F16 && dt(st.c) == Dtype::F32 &&
                             st.m % 256 == 0 && st.n % 256 == 0 && st.k % 64 == 0 && st.k > 0;
            const bool f32 = dt(st.a) == Dtype::F32 && dt(st.b) == Dtype::F32 && dt(st.c) == Dtype::F32 &&
                             st.m % 64 == 0 && st.n % 64 == 0 && st.k % 32 == 0 && st.k > 0;
            const bool half = f16 && (st.variant == 5 || st.variant == 6);
            const int64_t tm = f16 ? (half ? 128 : 256) : 64, tn = f16 ? 256 : 64;
            workgroups = ((st.m + tm - 1) / tm) * ((st.n + tn - 1) / tn);
            perGroup = tm * tn;
            covered = workgroups * perGroup >= instances;
            form = f16 ? (half ? "128 x 256 output tiles, two workgroups per CU" : "256 x 256 output tiles")
                       : f32 ? "64 x 64 output tiles" : "64 x 64 output tiles, bounds-checked";
            break;
        }
        case StepKind::ScoreSoftmax: {
            // Output scores; the two-pass form (dim 128, seq % 256 == 0)
            // gives each workgroup of a pass 128 rows x half the keys. A
            // sequence off the 256-row blocks runs it on copies padded to
            // seq' (a multiple of 256).
            instances = st.batch * st.seq * st.seq;
            const int64_t sp = (st.seq + 255) / 256 * 256;
            const bool padded = st.seq % 256 != 0;
            const bool twoPass = st.dim == 128 && sp <= 8192 && st.variant != 1;
            workgroups = twoPass ? st.batch * (sp / 128) * 2 : st.batch * ((st.seq + 63) / 64) * ((st.seq + 127) / 128);
            perGroup = twoPass ? 64 * sp : 64 * 128;
            covered = workgroups * perGroup >= instances;
            form = !twoPass ? "64 x 128 score tiles, then row softmax"
                   : padded ? "128-row blocks x key halves, per pass, over zero-padded Q and K"
                            : "128-row blocks x key halves, per pass";
            break;
        }
        case StepKind::Fail:
            covered = false;
            break;
    }
    return "{\"form\":\"" + std::string(form) + "\",\"instances\":" + std::to_string(instances) +
           ",\"workgroups\":" + std::to_string(workgroups) + ",\"per_workgroup\":" + std::to_string(perGroup) +
           ",\"covered\":" + (covered ? "true" : "false") + "}";
}

std::vector<int> variantSpace(const KernelModule& km, const Step& st) {
    auto dt = [&](uint32_t b) { return km.buffers[b].dtype; };
    switch (st.kind) {
        case StepKind::Softmax:
            if (dt(st.x) == Dtype::F32 && dt(st.y) == Dtype::F32 && st.cols % 4 == 0 && st.cols <= 8192) {
                return {5, 0, 2, 3, 4, 1};
            }
            return {};
        case StepKind::Gemm:
            if (dt(st.a) == Dtype::F16 && dt(st.b) == Dtype::F16 && dt(st.c) == Dtype::F32 && st.m % 256 == 0 &&
                st.n % 256 == 0 && st.k % 64 == 0 && st.k > 0) {
                return {8, 7, 0, 1, 2, 3, 5, 6};
            }
            // f32: 0, both tiles direct to a 4-deep LDS ring (K % 64); 1,
            // register-staged with A transposed.
            if (dt(st.a) == Dtype::F32 && dt(st.b) == Dtype::F32 && dt(st.c) == Dtype::F32 && st.m % 64 == 0 &&
                st.n % 64 == 0 && st.k % 64 == 0 && st.k > 0) {
                return {0, 1};
            }
            return {};
        case StepKind::ScoreSoftmax:
            // 0: two-pass query-stationary (the default); 1: scores, then the
            // softmax kernel over S.
            if (dt(st.q) == Dtype::F16 && dt(st.kk) == Dtype::F16 && dt(st.bias) == Dtype::F32 &&
                dt(st.s) == Dtype::F32 && st.dim == 128 && st.seq % 256 == 0 && st.seq <= 8192) {
                return {0, 1};
            }
            return {};
        case StepKind::Nest:
            // 0: with the step's LDS slabs; 1: the same kernel without them
            // (where it has slabs); 2, 3: form 0 at 512 and 64 threads per
            // workgroup; 4: one fewer collapsed loop.
            return nestForms(st);
        default: return {};
    }
}

std::string artifactFingerprint(const KernelModule& km, const Plan& plan, const std::string& arch) {
    uint64_t h = 0xCBF29CE484222325ull;
    h = fnv(h, &kCacheFormatVersion, sizeof(kCacheFormatVersion));
    const uint64_t mh = moduleHash(km);
    h = fnv(h, &mh, sizeof(mh));
    h = fnvStr(h, arch);
    h = fnvStr(h, plan.policy);
    int major = 0, minor = 0;
    mlkd_jit_version(&major, &minor);
    h = fnv(h, &major, sizeof(major));
    h = fnv(h, &minor, sizeof(minor));
    int cus = 0, maxBlock = 0;
    int64_t maxGrid = 0, mem = 0;
    mlkd_rt_device_info(0, &cus, &maxGrid, &maxBlock, &mem);
    h = fnv(h, &cus, sizeof(cus));
    h = fnv(h, &mem, sizeof(mem));
    char hex[24];
    std::snprintf(hex, sizeof(hex), "%016llx", static_cast<unsigned long long>(h));
    return hex;
}

std::string cachePath(const std::string& dir, const std::string& fingerprint) {
    if (dir.empty()) return std::string();
    return dir + (dir.back() == '/' ? "" : "/") + "fk-" + fingerprint + ".json";
}

bool applyCachedVariants(const std::string& dir, const std::string& fingerprint, const KernelModule& km,
                         Plan& plan) {
    const std::string path = cachePath(dir, fingerprint);
    std::string text;
    if (path.empty() || !readText(path, text)) return false;
    if (text.find("\"fingerprint\":\"" + fingerprint + "\"") == std::string::npos) return false;
    const size_t at = text.find("\"variants\":[");
    if (at == std::string::npos) return false;
    std::vector<int> v;
    const char* p = text.c_str() + at + 12;
    while (*p != '\0' && *p != ']') {
        char* end = nullptr;
        const long x = std::strtol(p, &end, 10);
        if (end == p) return false;
        v.push_back(static_cast<int>(x));
        p = end;
        while (*p == ',' || *p == ' ') ++p;
    }
    if (v.size() != plan.steps.size()) return false;
    for (size_t i = 0; i < v.size(); ++i) {
        if (v[i] == -1) continue;
        const std::vector<int> space = variantSpace(km, plan.steps[i]);
        if (std::find(space.begin(), space.end(), v[i]) == space.end()) return false;
    }
    for (size_t i = 0; i < v.size(); ++i) plan.steps[i].variant = v[i];
    return true;
}

int HipLoadedKernel::setStepVariant(int step, int variant, std::string& why) {
    if (step < 0 || static_cast<size_t>(step) >= plan_.steps.size()) {
        why = "step out of range";
        return MLKHIP_BAD_BINDING;
    }
    if (variant != -1) {
        const std::vector<int> space = variantSpace(km_, plan_.steps[static_cast<size_t>(step)]);
        if (std::find(space.begin(), space.end(), variant) == space.end()) {
            why = "variant " + std::to_string(variant) + " is not in the step's variant space";
            return MLKHIP_BAD_BINDING;
        }
    }
    const Step& st = plan_.steps[static_cast<size_t>(step)];
    if (st.kind == StepKind::Nest && variant >= 1 && variant <= 4) {
        // Compiled now, so the allocation-free entry finds it loaded.
        void* fn = nullptr;
        if (const int rc = ensureNestForm(static_cast<size_t>(step), variant, fn, why); rc != MLKHIP_OK) return rc;
    }
    plan_.steps[static_cast<size_t>(step)].variant = variant;
    return MLKHIP_OK;
}

int HipLoadedKernel::autotune(const DeviceBinding* binds, int n, const double* scalars, int64_t nScalars,
                              int64_t elements, int reps, const std::string& cacheDir, std::string& report,
                              std::string& why) {
    if (n != static_cast<int>(bindables_.size())) {
        why = "expected " + std::to_string(bindables_.size()) + " bindings, got " + std::to_string(n);
        return MLKHIP_BAD_BINDING;
    }
    if (reps < 1) reps = 1;
    // Buffers the artifact writes, snapshotted so every trial starts from the
    // caller's contents and the caller gets them back unchanged.
    std::vector<bool> written(km_.buffers.size(), false);
    for (const Step& st : plan_.steps) {
        for (const uint32_t b : {st.out.buffer, st.y, st.c, st.s}) {
            if (b != kInvalidId && b < written.size()) written[b] = true;
        }
        for (const uint32_t b : st.nestWrites) written[b] = true;
    }
    struct Saved {
        int bind;
        size_t bytes;
        void* copy;
    };
    std::vector<Saved> saved;
    auto release = [&]() {
        for (Saved& s : saved) mlkd_rt_free(s.copy);
        saved.clear();
    };
    for (int i = 0; i < n; ++i) {
        const uint32_t b = bindables_[static_cast<size_t>(i)];
        const KernelBuffer& kb = km_.buffers[b];
        if (kb.isTemp || !(written[b] || kb.isOutput) || binds[i].ptr == nullptr || binds[i].elements <= 0) continue;
        const size_t bytes = static_cast<size_t>(binds[i].elements) * dtypeBytes(kb.dtype);
        void* c = nullptr;
        if (mlkd_rt_malloc(&c, bytes) != 0 || mlkd_rt_d2d(c, binds[i].ptr, bytes, nullptr) != 0) {
            if (c != nullptr) mlkd_rt_free(c);
            release();
            why = "autotune snapshot allocation failed";
            return MLKHIP_RUNTIME;
        }
        saved.push_back(Saved{i, bytes, c});
    }
    auto restore = [&]() -> bool {
        for (const Saved& s : saved) {
            if (mlkd_rt_d2d(binds[s.bind].ptr, s.copy, s.bytes, nullptr) != 0) return false;
        }
        return mlkd_rt_sync(nullptr) == 0;
    };
    auto outputs = [&](std::vector<std::vector<double>>& out) -> bool {
        out.clear();
        for (const Saved& s : saved) {
            const KernelBuffer& kb = km_.buffers[bindables_[static_cast<size_t>(s.bind)]];
            const int64_t cnt = binds[s.bind].elements;
            std::vector<unsigned char> raw(s.bytes);
            if (mlkd_rt_d2h(raw.data(), binds[s.bind].ptr, s.bytes, nullptr) != 0 || mlkd_rt_sync(nullptr) != 0) {
                return false;
            }
            std::vector<double> v(static_cast<size_t>(cnt));
            for (int64_t e = 0; e < cnt; ++e) {
                if (kb.dtype == Dtype::F64) {
                    std::memcpy(&v[static_cast<size_t>(e)], raw.data() + e * 8, 8);
                } else if (kb.dtype == Dtype::F32) {
                    float f;
                    std::memcpy(&f, raw.data() + e * 4, 4);
                    v[static_cast<size_t>(e)] = f;
                } else {
                    _Float16 h;
                    std::memcpy(&h, raw.data() + e * 2, 2);
                    v[static_cast<size_t>(e)] = static_cast<double>(h);
                }
            }
            out.push_back(std::move(v));
        }
        return true;
    };
    auto runOnce = [&](std::string& w) -> int {
        const int rc = runDevice(binds, n, scalars, nScalars, elements, nullptr, w);
        if (rc != MLKHIP_OK) return rc;
        return mlkd_rt_sync(nullptr) == 0 ? MLKHIP_OK : MLKHIP_LAUNCH;
    };
    // Benchmark certificate: median, min and max of `reps` launches timed
    // one by one after kWarmup untimed ones (fast_kernel.cpp:697-719).
    constexpr int kWarmup = 2;
    struct Bench {
        double median{0}, lo{0}, hi{0};
    };
    auto timeRuns = [&](Bench& out) -> int {
        std::string w;
        for (int r = 0; r < kWarmup; ++r) {
            if (runDevice(binds, n, scalars, nScalars, elements, nullptr, w) != MLKHIP_OK) return MLKHIP_LAUNCH;
        }
        void* e0 = nullptr;
        void* e1 = nullptr;
        if (mlkd_rt_event_create(&e0) != 0 || mlkd_rt_event_create(&e1) != 0) {
            if (e0 != nullptr) mlkd_rt_event_destroy(e0);
            return MLKHIP_LAUNCH;
        }
        std::vector<double> t;
        int rc = MLKHIP_OK;
        for (int r = 0; r < reps && rc == MLKHIP_OK; ++r) {
            float ms = 0.0f;
            if (mlkd_rt_event_record(e0, nullptr) != 0) rc = MLKHIP_LAUNCH;
            if (rc == MLKHIP_OK) rc = runDevice(binds, n, scalars, nScalars, elements, nullptr, w);
            if (rc == MLKHIP_OK &&
                (mlkd_rt_event_record(e1, nullptr) != 0 || mlkd_rt_event_elapsed_ms(e0, e1, &ms) != 0)) {
                rc = MLKHIP_LAUNCH;
            }
            t.push_back(1e-3 * ms);
        }
        mlkd_rt_event_destroy(e0);
        mlkd_rt_event_destroy(e1);
        if (rc != MLKHIP_OK) return rc;
        std::sort(t.begin(), t.end());
        const size_t m = t.size();
        out.median = m % 2 ? t[m / 2] : 0.5 * (t[m / 2 - 1] + t[m / 2]);
        out.lo = t.front();
        out.hi = t.back();
        return MLKHIP_OK;
    };

    const std::vector<int> chosenBefore = [&]() {
        std::vector<int> v;
        for (const Step& st : plan_.steps) v.push_back(st.variant);
        return v;
    }();
    // Reference: every step in its default form.
    for (Step& st : plan_.steps) st.variant = -1;
    std::vector<std::vector<double>> ref;
    int rc = restore() ? runOnce(why) : MLKHIP_RUNTIME;
    if (rc == MLKHIP_OK && !outputs(ref)) rc = MLKHIP_RUNTIME;
    if (rc != MLKHIP_OK) {
        for (size_t i = 0; i < plan_.steps.size(); ++i) plan_.steps[i].variant = chosenBefore[i];
        restore();
        release();
        if (why.empty()) why = "autotune reference run failed";
        return rc;
    }
    const double thr = threshold(plan_.policy, maxK(plan_));
    // Each step is searched with every other step in its default form, so a
    // candidate's deviation is its own; the chosen combination is certified
    // once more as a whole below.
    std::vector<int> chosen(plan_.steps.size(), -1);
    std::string steps;
    int searched = 0;
    for (size_t si = 0; si < plan_.steps.size(); ++si) {
        const std::vector<int> space = variantSpace(km_, plan_.steps[si]);
        if (space.size() < 2) continue;
        ++searched;
        std::string cands;
        double bestSec = INFINITY;
        for (const int v : space) {
            plan_.steps[si].variant = v;
            std::string w;
            double worst = 0.0;
            Bench bench;
            bool admissible = false;
            bool identity = false;
            const char* reason = "";
            std::string detail;
            std::vector<std::vector<double>> got;
            if (!restore()) {
                reason = "build-failed";
                detail = "could not restore the written buffers";
            } else if (runOnce(w) != MLKHIP_OK) {
                reason = "build-failed";
                detail = "run failed: " + w;
            } else if (!outputs(got)) {
                reason = "build-failed";
                detail = "read-back failed";
            } else if (!(identity = compare(ref, got, thr, worst))) {
                reason = "identity-mismatch";
                detail = "outside half of the policy's tolerance";
            } else if (timeRuns(bench) != MLKHIP_OK) {
                reason = "build-failed";
                detail = "timing failed";
            } else {
                admissible = true;
                if (bench.median < bestSec) {
                    bestSec = bench.median;
                    chosen[si] = v;
                }
            }
            if (!cands.empty()) cands += ",";
            cands += "{\"variant\":" + std::to_string(v) + ",\"admissible\":" + (admissible ? "true" : "false");
            if (*reason != '\0') cands += ",\"rejected\":{\"reason\":\"" + std::string(reason) + "\",\"detail\":\"" + detail + "\"}";
            cands += ",\"certificate\":{\"identity\":{\"certified\":" + std::string(identity ? "true" : "false") +
                     ",\"max_dev\":" + num(std::isinf(worst) ? 1e300 : worst) + "},\"runtime\":{\"upper_bound_sec\":" +
                     num(bench.median) + ",\"min_sec\":" + num(bench.lo) + ",\"max_sec\":" + num(bench.hi) +
                     ",\"reps\":" + std::to_string(admissible ? reps : 0) + ",\"warmup\":" +
                     std::to_string(admissible ? kWarmup : 0) + "}}}";
        }
        // The launch certificate is that of the chosen form.
        plan_.steps[si].variant = chosen[si];
        const std::string launch = launchCoverage(km_, plan_.steps[si], elements);
        plan_.steps[si].variant = -1;
        if (!steps.empty()) steps += ",";
        steps += "{\"step\":" + std::to_string(si) + ",\"class\":\"" + plan_.steps[si].what + "\",\"kernel\":\"" +
                 kindName(plan_.steps[si].kind) + "\",\"chosen\":" + std::to_string(chosen[si]) +
                 ",\"launch\":" + launch + ",\"candidates\":[" + cands + "]}";
    }
    for (size_t i = 0; i < plan_.steps.size(); ++i) plan_.steps[i].variant = chosen[i];
    bool combined = true;
    if (searched > 1) {
        std::string w;
        std::vector<std::vector<double>> got;
        double worst = 0.0;
        combined = restore() && runOnce(w) == MLKHIP_OK && outputs(got) && compare(ref, got, thr, worst);
        if (!combined) {
            for (Step& st : plan_.steps) st.variant = -1;
        }
    }
    // The whole artifact with the chosen forms, against the roofline lower
    // bound of its essential work (FastKernelReport's winner gap,
    // fast_kernel.h:327-346).
    Bench whole;
    const bool timedWhole = restore() && timeRuns(whole) == MLKHIP_OK;
    const EssentialWork work = essentialWork(km_);
    const double peak = peakOpsPerSec(km_, plan_);
    const double lower = rooflineLowerSec(work, 8.0e12, peak);
    // The same bound at the probed rates (other dtypes scaled from the
    // measured f16 rate by the datasheet ratio).
    const MeasuredEnvironment& menv = measuredEnvironment();
    const double lowerMeasured =
        menv.ok ? rooflineLowerSec(work, menv.bytesPerSec, peak * menv.f16FlopsPerSec / 2.5e15) : 0.0;
    const bool restored = restore();
    release();
    std::string variants;
    for (size_t i = 0; i < plan_.steps.size(); ++i) {
        if (i) variants += ",";
        variants += std::to_string(plan_.steps[i].variant);
    }
    std::string cacheFile;
    const std::string path = cachePath(cacheDir, fingerprint_);
    if (!path.empty()) {
        const std::string doc = "{\"format\":\"mlk-hip-fastkernel\",\"version\":" + std::to_string(kCacheFormatVersion) +
                                ",\"fingerprint\":\"" + fingerprint_ + "\",\"policy\":\"" + plan_.policy +
                                "\",\"variants\":[" + variants + "]}\n";
        if (writeTextAtomic(path, doc)) cacheFile = path;
    }
    report = "{\"fingerprint\":\"" + fingerprint_ + "\",\"policy\":\"" + plan_.policy + "\",\"threshold\":" +
             num(thr) + ",\"reps\":" + std::to_string(reps) + ",\"warmup\":" + std::to_string(kWarmup) +
             ",\"combined_certified\":" + (combined ? "true" : "false") + ",\"variants\":[" + variants +
             "],\"cache\":{\"file\":\"" + cacheFile + "\",\"hits\":" + (fromCache_ ? "1" : "0") +
             ",\"misses\":" + (fromCache_ ? "0" : "1") + "},\"work\":{\"min_bytes\":" +
             std::to_string(work.minBytes) + ",\"min_ops\":" + std::to_string(work.minOps) + ",\"bytes_known\":" +
             (work.bytesKnown ? "true" : "false") + ",\"ops_known\":" + (work.opsKnown ? "true" : "false") +
             "},\"environment\":{\"declared_bytes_per_sec\":8e+12,\"declared_ops_per_sec\":" + num(peak) +
             ",\"measured_bytes_per_sec\":" + num(menv.ok ? menv.bytesPerSec : 0.0) +
             ",\"measured_f16_flops_per_sec\":" + num(menv.ok ? menv.f16FlopsPerSec : 0.0) +
             "},\"roofline_lower_sec\":" + num(lower) + ",\"roofline_lower_sec_measured\":" + num(lowerMeasured) +
             ",\"winner_sec\":" + num(timedWhole ? whole.median : 0.0) +
             ",\"winner_gap_over_lower\":" + num(timedWhole && lower > 0.0 ? whole.median / lower - 1.0 : 0.0) +
             ",\"steps\":[" + steps + "]}";
    if (!restored) {
        why = "could not restore the caller's buffers after the search";
        return MLKHIP_RUNTIME;
    }
    return MLKHIP_OK;
}

}  // namespace mlk::hip
