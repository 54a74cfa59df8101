// Per-module artifact emitter: the file-backed form of the reference's GPU
// artifact (backends/cpu/src/backend_driver.cpp:637-760 builds it, :427
// dlsym's `mlk_kernel`, :932-1042 calls it through an exactly typed
// pointer). The emitted libmlk_kernel.so exports `mlk_kernel` in the form
// the reference's LoadedKernel::run binds (docs/kernel_abi.md:25-40,
// backend_driver.h:15-46):
//   multi-dim modules: int mlk_kernel(<T0> p0, const int64_t* p0_dims, ...,
//                                     const double* mlk_scalars, int64_t mlk_n_scalars)
//   legacy 1-D modules: void mlk_kernel(<T0> p0, ..., int64_t n,
//                                       const double* mlk_scalars, int64_t mlk_n_scalars)
// with <Ti> = double* for buffers that are stored to, outputs or temps and
// const double* otherwise, one entry per bindable buffer in table order. The
// legacy form's status, which its void return cannot carry, is readable
// through mlk_kernel_status(). Each call forwards to this library's host
// f64 entry (mlkhip_kernel / mlkhip_kernel_1d): per-call device allocation,
// RNE conversion to the module's dtypes, launch, copy back, synchronously,
// as the reference's artifact does. Temp slots are materialized by the
// artifact; the pointers the driver passes there are ignored
// (backend_driver.cpp:853-865 passes dummies). The module document and the
// declared target are embedded; the first call builds the artifact
// (mlkhip_build) once per process.
#include <dlfcn.h>
#include <fcntl.h>
#include <spawn.h>
#include <sys/stat.h>
#include <sys/wait.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "driver.h"
#include "../../../include/mlk_hip.h"

extern char** environ;

namespace mlk::hip {

namespace {

/// Buffers some Store or Call node writes (their artifact pointer is mutable).
std::vector<bool> storedBuffers(const KernelModule& km) {
    std::vector<bool> w(km.buffers.size(), false);
    for (const KernelNode& n : km.nodes) {
        if ((n.op == KernelOp::Store || n.op == KernelOp::Call) && n.bufferOut < km.buffers.size()) {
            w[n.bufferOut] = true;
        }
    }
    return w;
}

std::string hexBytes(const std::string& s) {
    std::string out;
    char buf[8];
    for (size_t i = 0; i < s.size(); ++i) {
        std::snprintf(buf, sizeof(buf), "0x%02x,", static_cast<unsigned char>(s[i]));
        out += buf;
        if (i % 24 == 23) out += "\n    ";
    }
    return out;
}

bool validIdent(const std::string& s) {
    for (const char c : s) {
        const bool ok = (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || (c >= '0' && c <= '9') || c == '_';
        if (!ok) return false;
    }
    return !s.empty();
}

}  // namespace

Result<std::string> artifactSource(const std::string& moduleJson, const KernelModule& km, const Plan& plan,
                                   const std::string& arch) {
    if (!validArch(arch)) return err(ErrorCode::InvalidArgument, "invalid HIP target '" + arch + "'");
    const std::vector<bool> stored = storedBuffers(km);
    std::vector<uint32_t> bind;
    for (uint32_t b = 0; b < km.buffers.size(); ++b) {
        const KernelBuffer& kb = km.buffers[b];
        if (kb.isInput || kb.isOutput || kb.isTemp) bind.push_back(b);
    }
    if (bind.empty()) return err(ErrorCode::InvalidGraph, "module has no bindable buffer");
    const bool multi = plan.multiDim;
    std::string s;
    s += "// libmlk_kernel.so source written by mlkhip_emit_artifact: module \"";
    for (const char c : km.name) s += (c == '\n' || c == '\r') ? ' ' : c;
    s += "\", class " + plan.className + ", policy " + plan.policy + ", target " + arch + ".\n";
    s += "// " + std::string(multi ? "Multi-dim" : "Legacy 1-D") +
         " artifact ABI (docs/kernel_abi.md:25-40); forwards to libmlk_hip.so.\n";
    s += "#include <cstddef>\n#include <cstdint>\n#include <mutex>\n\n";
    s += "extern \"C\" {\n";
    s += "typedef struct mlkhip_artifact mlkhip_artifact;\n";
    s += "int mlkhip_build(const char*, size_t, const char*, const char*, mlkhip_artifact**);\n";
    s += "int mlkhip_kernel(const mlkhip_artifact*, double* const*, const int64_t* const*, int, const double*, "
         "int64_t, int64_t);\n";
    s += "int mlkhip_kernel_1d(const mlkhip_artifact*, double* const*, int, int64_t, const double*, int64_t);\n";
    s += "}\n\nnamespace {\n";
    s += "const unsigned char kModule[] = {\n    " + hexBytes(moduleJson) + "};\n";
    s += "const char kArch[] = \"" + arch + "\";\n";
    s += "std::once_flag gOnce;\nmlkhip_artifact* gArtifact = nullptr;\nint gBuildStatus = 0;\n";
    s += "thread_local int tStatus = 0;\n\n";
    s += "const mlkhip_artifact* artifact(int& status) {\n";
    s += "    std::call_once(gOnce, [] {\n";
    s += "        gBuildStatus = mlkhip_build(reinterpret_cast<const char*>(kModule), sizeof(kModule), kArch, nullptr,\n";
    s += "                                    &gArtifact);\n";
    s += "    });\n";
    s += "    status = gBuildStatus;\n";
    s += "    return gBuildStatus == 0 ? gArtifact : nullptr;\n";
    s += "}\n}  // namespace\n\n";
    s += "extern \"C\" int mlk_kernel_status(void) { return tStatus; }\n\n";
    std::string params, ptrs, dims;
    for (size_t i = 0; i < bind.size(); ++i) {
        const uint32_t b = bind[i];
        const KernelBuffer& kb = km.buffers[b];
        const bool mut = kb.isOutput || kb.isTemp || stored[b];
        const std::string p = "p" + std::to_string(i);
        const std::string label = validIdent(kb.name) ? " /* " + kb.name + " */" : "";
        params += std::string(i ? ", " : "") + (mut ? "double* " : "const double* ") + p + label;
        if (multi) params += ", const int64_t* " + p + "_dims";
        ptrs += std::string(i ? ", " : "") +
                (kb.isTemp ? std::string("nullptr") : (mut ? p : "const_cast<double*>(" + p + ")"));
        dims += std::string(i ? ", " : "") + p + (multi ? "_dims" : "");
    }
    const std::string n = std::to_string(bind.size());
    if (multi) {
        s += "extern \"C\" int mlk_kernel(" + params + ", const double* mlk_scalars, int64_t mlk_n_scalars) {\n";
        s += "    int status = 0;\n";
        s += "    const mlkhip_artifact* a = artifact(status);\n";
        s += "    if (a == nullptr) return tStatus = status;\n";
        s += "    double* const ptrs[" + n + "] = {" + ptrs + "};\n";
        s += "    const int64_t* const dims[" + n + "] = {" + dims + "};\n";
        s += "    return tStatus = mlkhip_kernel(a, ptrs, dims, " + n + ", mlk_scalars, mlk_n_scalars, 0);\n";
        s += "}\n";
    } else {
        s += "extern \"C\" void mlk_kernel(" + params +
             ", int64_t n, const double* mlk_scalars, int64_t mlk_n_scalars) {\n";
        s += "    int status = 0;\n";
        s += "    const mlkhip_artifact* a = artifact(status);\n";
        s += "    if (a == nullptr) {\n        tStatus = status;\n        return;\n    }\n";
        s += "    double* const ptrs[" + n + "] = {" + ptrs + "};\n";
        s += "    tStatus = mlkhip_kernel_1d(a, ptrs, " + n + ", n, mlk_scalars, mlk_n_scalars);\n";
        s += "}\n";
    }
    return s;
}

namespace {

/// Directory holding this library (libmlk_hip.so), for the artifact's link
/// line and run path.
std::string libraryDir() {
    Dl_info info;
    if (dladdr(reinterpret_cast<const void*>(&mlkhip_emit_artifact), &info) == 0 || info.dli_fname == nullptr) {
        return std::string();
    }
    std::string p = info.dli_fname;
    const size_t slash = p.rfind('/');
    return slash == std::string::npos ? std::string(".") : p.substr(0, slash);
}

bool writeText(const std::string& path, const std::string& text) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (f == nullptr) return false;
    const size_t put = std::fwrite(text.data(), 1, text.size(), f);
    const bool ok = std::fclose(f) == 0 && put == text.size();
    return ok;
}

/// Runs argv[0] (PATH lookup, no shell) as a child process with stdout and
/// stderr sent to `log`; returns its exit status or -1.
int runChild(const std::vector<std::string>& args, const std::string& log) {
    std::vector<char*> argv;
    for (const std::string& a : args) argv.push_back(const_cast<char*>(a.c_str()));
    argv.push_back(nullptr);
    posix_spawn_file_actions_t fa;
    posix_spawn_file_actions_init(&fa);
    posix_spawn_file_actions_addopen(&fa, 1, log.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0644);
    posix_spawn_file_actions_adddup2(&fa, 1, 2);
    pid_t pid = 0;
    const int rc = posix_spawnp(&pid, argv[0], &fa, nullptr, argv.data(), environ);
    posix_spawn_file_actions_destroy(&fa);
    if (rc != 0) return -1;
    int st = 0;
    if (waitpid(pid, &st, 0) != pid) return -1;
    return WIFEXITED(st) ? WEXITSTATUS(st) : -1;
}

std::string tail(const std::string& path) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (f == nullptr) return std::string();
    std::string s;
    char buf[4096];
    size_t got = 0;
    while ((got = std::fread(buf, 1, sizeof(buf), f)) > 0) s.append(buf, got);
    std::fclose(f);
    return s.size() > 2000 ? s.substr(s.size() - 2000) : s;
}

}  // namespace

Result<std::string> emitArtifact(const std::string& moduleJson, const std::string& arch, const std::string& compiler,
                                 const std::string& dir) {
    auto km = parseKernelModule(moduleJson.data(), moduleJson.size());
    if (!km.has_value()) return err(km.error().code, km.error().message);
    auto plan = planModule(deviceModule(*km));
    if (!plan.has_value()) return err(plan.error().code, plan.error().message);
    auto src = artifactSource(moduleJson, *km, *plan, arch);
    if (!src.has_value()) return err(src.error().code, src.error().message);
    if (dir.empty()) return err(ErrorCode::InvalidArgument, "artifact directory not given");
    ::mkdir(dir.c_str(), 0755);  // an existing directory is fine
    const std::string cpp = dir + "/mlk_kernel.cpp";
    const std::string so = dir + "/libmlk_kernel.so";
    const std::string log = dir + "/build.log";
    if (!writeText(cpp, *src)) return err(ErrorCode::InvalidArgument, "cannot write " + cpp);
    const std::string libdir = libraryDir();
    if (libdir.empty()) return err(ErrorCode::UnsupportedCapability, "cannot locate libmlk_hip.so");
    const std::vector<std::string> args = {compiler.empty() ? std::string("c++") : compiler,
                                           "-std=c++17", "-O2", "-shared", "-fPIC", "-o", so, cpp,
                                           "-L" + libdir, "-lmlk_hip", "-Wl,-rpath," + libdir};
    const int rc = runChild(args, log);
    if (rc != 0) {
        return err(ErrorCode::UnsupportedCapability,
                   "artifact compile failed (status " + std::to_string(rc) + "): " + tail(log));
    }
    return so;
}

}  // namespace mlk::hip

extern "C" int mlkhip_emit_artifact(const char* module_json, size_t len, const char* arch, const char* compiler,
                                    const char* dir, char* path_out, size_t cap) {
    if (module_json == nullptr || arch == nullptr || dir == nullptr) {
        return mlk::hip::setLastError(MLKHIP_REFUSED, "null argument");
    }
    auto so = mlk::hip::emitArtifact(std::string(module_json, len), arch, compiler != nullptr ? compiler : "",
                                     dir);
    if (!so.has_value()) return mlk::hip::setLastError(MLKHIP_REFUSED, so.error().message);
    if (path_out != nullptr && cap > 0) {
        const size_t n = so->size() < cap - 1 ? so->size() : cap - 1;
        std::memcpy(path_out, so->data(), n);
        path_out[n] = '\0';
    }
    return MLKHIP_OK;
}
