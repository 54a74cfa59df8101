// In-process compilation of kernel-template instances with hipRTC, with a
// process-lifetime module table and an optional on-disk code-object cache
// (<cache_dir>/<fingerprint>.hsaco). The fingerprint covers the source text,
// the kernel name, the declared target and the hipRTC version, so a cached
// object is never reused for another target or toolchain. Loaded modules are
// never unloaded (the same lifetime rule as the reference's dlopen'd
// artifacts, backends/cpu/include/mlk/backend/backend_driver.h:110-116).
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "runtime_abi.h"

namespace {

struct Entry {
    hipModule_t module{nullptr};
    hipFunction_t fn{nullptr};
};

std::mutex& tableLock() {
    static std::mutex m;
    return m;
}

std::unordered_map<uint64_t, Entry>& table() {
    static std::unordered_map<uint64_t, Entry> t;
    return t;
}

uint64_t fnv1a(uint64_t h, const void* data, size_t n) {
    const unsigned char* p = static_cast<const unsigned char*>(data);
    for (size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 0x100000001B3ull;
    }
    return h;
}

void setLog(char* log, size_t cap, const std::string& s) {
    if (log == nullptr || cap == 0) return;
    const size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
    memcpy(log, s.data(), n);
    log[n] = '\0';
}

bool readFile(const std::string& path, std::vector<char>& out) {
    FILE* f = fopen(path.c_str(), "rb");
    if (f == nullptr) return false;
    fseek(f, 0, SEEK_END);
    const long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    if (n <= 0) {
        fclose(f);
        return false;
    }
    out.resize(static_cast<size_t>(n));
    const size_t got = fread(out.data(), 1, out.size(), f);
    fclose(f);
    return got == out.size();
}

void writeFileAtomic(const std::string& path, const std::vector<char>& data) {
    const std::string tmp = path + ".tmp" + std::to_string(reinterpret_cast<uintptr_t>(&data));
    FILE* f = fopen(tmp.c_str(), "wb");
    if (f == nullptr) return;
    const size_t put = fwrite(data.data(), 1, data.size(), f);
    fclose(f);
    if (put == data.size()) {
        rename(tmp.c_str(), path.c_str());
    } else {
        remove(tmp.c_str());
    }
}

/// hipRTC options of every instance: the declared target, -O3, C++17, no
/// floating-point contraction (f64 chains round like the reference's x86-64
/// build) and no packed FP32 instructions, as for the precompiled kernels.
struct JitOptions {
    std::string arch;
    const char* v[8];
    int n{0};
    explicit JitOptions(const char* target) : arch(std::string("--offload-arch=") + target) {
        v[n++] = arch.c_str();
        v[n++] = "-O3";
        v[n++] = "-std=c++17";
        v[n++] = "-ffp-contract=off";
        v[n++] = "-Xclang";
        v[n++] = "-target-feature";
        v[n++] = "-Xclang";
        v[n++] = "-packed-fp32-ops";
    }
};

}  // namespace

extern "C" {

/// The hipRTC option list (for inspection by tests): writes the options
/// separated by single spaces into `buf`; returns their count.
int mlkd_jit_options(const char* arch, char* buf, size_t cap) {
    const JitOptions o(arch != nullptr ? arch : "gfx950");
    std::string s;
    for (int i = 0; i < o.n; ++i) {
        if (i) s += ' ';
        s += o.v[i];
    }
    setLog(buf, cap, s);
    return o.n;
}

/// hipRTC's version (part of the variant-cache fingerprint).
int mlkd_jit_version(int* major, int* minor) {
    return hiprtcVersion(major, minor) == HIPRTC_SUCCESS ? 0 : MLKD_RT_LAUNCH;
}

/// Compiles (or fetches) `name` from `src` for `arch`. Returns 0 and the
/// function handle, or MLKD_RT_LAUNCH with the compiler log.
int mlkd_jit_build(const char* src, size_t len, const char* name, const char* arch,
                   const char* cache_dir, void** fn_out, uint64_t* fingerprint_out, char* log,
                   size_t cap) {
    *fn_out = nullptr;
    int major = 0, minor = 0;
    hiprtcVersion(&major, &minor);
    JitOptions jo(arch);
    const char** opts = jo.v;
    const int nopts = jo.n;
    uint64_t h = 0xCBF29CE484222325ull;
    h = fnv1a(h, src, len);
    h = fnv1a(h, name, strlen(name));
    for (int i = 0; i < nopts; ++i) h = fnv1a(h, opts[i], strlen(opts[i]));
    h = fnv1a(h, &major, sizeof(major));
    h = fnv1a(h, &minor, sizeof(minor));
    if (fingerprint_out != nullptr) *fingerprint_out = h;

    std::lock_guard<std::mutex> g(tableLock());
    auto it = table().find(h);
    if (it != table().end()) {
        *fn_out = it->second.fn;
        return 0;
    }
    std::vector<char> code;
    std::string cachePath;
    if (cache_dir != nullptr && cache_dir[0] != '\0') {
        char hex[32];
        snprintf(hex, sizeof(hex), "%016llx", static_cast<unsigned long long>(h));
        cachePath = std::string(cache_dir) + "/" + hex + ".hsaco";
        if (!readFile(cachePath, code)) code.clear();
    }
    if (code.empty()) {
        hiprtcProgram prog;
        std::string text(src, len);
        if (hiprtcCreateProgram(&prog, text.c_str(), "mlk_instance.hip", 0, nullptr, nullptr) !=
            HIPRTC_SUCCESS) {
            setLog(log, cap, "hiprtcCreateProgram failed");
            return MLKD_RT_LAUNCH;
        }
        const hiprtcResult rc = hiprtcCompileProgram(prog, nopts, opts);
        size_t logSize = 0;
        hiprtcGetProgramLogSize(prog, &logSize);
        std::string clog(logSize + 1, '\0');
        if (logSize > 0) hiprtcGetProgramLog(prog, &clog[0]);
        if (rc != HIPRTC_SUCCESS) {
            setLog(log, cap, std::string("hipRTC compile failed: ") + clog);
            hiprtcDestroyProgram(&prog);
            return MLKD_RT_LAUNCH;
        }
        size_t codeSize = 0;
        hiprtcGetCodeSize(prog, &codeSize);
        code.resize(codeSize);
        hiprtcGetCode(prog, code.data());
        hiprtcDestroyProgram(&prog);
        if (!cachePath.empty()) writeFileAtomic(cachePath, code);
    }
    Entry e;
    if (hipModuleLoadData(&e.module, code.data()) != hipSuccess) {
        setLog(log, cap, "hipModuleLoadData failed (code object not loadable on this device)");
        return MLKD_RT_NO_DEVICE;
    }
    if (hipModuleGetFunction(&e.fn, e.module, name) != hipSuccess) {
        setLog(log, cap, std::string("kernel symbol not found: ") + name);
        return MLKD_RT_LAUNCH;
    }
    table()[h] = e;
    *fn_out = e.fn;
    return 0;
}

/// Compiles `src` to a code object without loading it (build-time check on
/// hosts without a device). Returns the code-object size in bytes or -1.
long long mlkd_jit_compile_only(const char* src, size_t len, const char* arch, char* log,
                                size_t cap) {
    JitOptions jo(arch);
    hiprtcProgram prog;
    std::string text(src, len);
    if (hiprtcCreateProgram(&prog, text.c_str(), "mlk_instance.hip", 0, nullptr, nullptr) !=
        HIPRTC_SUCCESS) {
        setLog(log, cap, "hiprtcCreateProgram failed");
        return -1;
    }
    const hiprtcResult rc = hiprtcCompileProgram(prog, jo.n, jo.v);
    size_t logSize = 0;
    hiprtcGetProgramLogSize(prog, &logSize);
    std::string clog(logSize + 1, '\0');
    if (logSize > 0) hiprtcGetProgramLog(prog, &clog[0]);
    setLog(log, cap, clog);
    size_t codeSize = 0;
    if (rc == HIPRTC_SUCCESS) hiprtcGetCodeSize(prog, &codeSize);
    hiprtcDestroyProgram(&prog);
    return rc == HIPRTC_SUCCESS ? static_cast<long long>(codeSize) : -1;
}

/// Launches a template instance whose signature is
/// (const void*, const void*, const void*, const void*, void*, scalars,
/// long long dynamic_extent).
int mlkd_jit_launch_elementwise(void* fn, unsigned grid, const void* const* in, void* out,
                                const mlkd_scalars* scalars, long long dyn_extent, void* stream) {
    const void* p0 = in[0];
    const void* p1 = in[1];
    const void* p2 = in[2];
    const void* p3 = in[3];
    mlkd_scalars sc = *scalars;
    long long dyn = dyn_extent;
    void* args[] = {&p0, &p1, &p2, &p3, &out, &sc, &dyn};
    const hipError_t e = hipModuleLaunchKernel(static_cast<hipFunction_t>(fn), grid, 1, 1, 256,
                                               1, 1, 0, static_cast<hipStream_t>(stream), args,
                                               nullptr);
    return e == hipSuccess ? 0 : MLKD_RT_LAUNCH;
}

/// Launches a generic loop-nest instance, `block` threads per workgroup (the
/// instance's MLK_NEST_WG).
int mlkd_jit_launch_nest(void* fn, unsigned grid, unsigned block, const mlkd_nest_args* args,
                         const mlkd_scalars* scalars, long long total, void* stream) {
    if (block == 0 || block > 1024) return MLKD_RT_LAUNCH;
    mlkd_nest_args a = *args;
    mlkd_scalars sc = *scalars;
    long long t = total;
    void* kargs[] = {&a, &sc, &t};
    const hipError_t e = hipModuleLaunchKernel(static_cast<hipFunction_t>(fn), grid, 1, 1, block, 1, 1, 0,
                                               static_cast<hipStream_t>(stream), kargs, nullptr);
    return e == hipSuccess ? 0 : MLKD_RT_LAUNCH;
}

}  // extern "C"
