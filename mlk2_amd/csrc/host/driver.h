// C++ driver of the HIP backend: the gfx950 counterpart of the reference's
// GPU artifact driver (backends/cpu/include/mlk/backend/backend_driver.h:
// 91-228). Building an artifact plans the module onto the hand-written
// kernels and loads every template instance it needs; running it binds
// buffers exactly as LoadedKernel::run does (table order, temps owned by the
// artifact, zero-initialized per run).
#pragma once

#include <cstdint>
#include <memory>
#include <array>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../device_abi.h"
#include "planner.h"

namespace mlk::hip {

/// Driver knobs (GpuBackendDriverConfig, backend_driver.h:91-105). The
/// target is declared and validated, never probed or defaulted.
struct HipBackendDriverConfig {
    std::string arch;       // e.g. "gfx950"
    std::string cacheDir;   // code-object cache; empty = in-process only
};

/// gfx followed by 3 or 4 hex digits (gfx950, gfx90a, gfx1100).
bool validArch(const std::string& arch);

struct DeviceBinding {
    void* ptr{nullptr};
    int64_t elements{0};
    int32_t dtype{0};
};

/// Device memory a run takes all of its scratch from instead of allocating:
/// the allocation-free entry's file-scope array on the current device.
struct ScratchArena {
    char* base{nullptr};
    size_t bytes{0};
};

class HipLoadedKernel {
public:
    ~HipLoadedKernel();  // frees the artifact-owned scratch of every stream

    const KernelModule& module() const { return km_; }
    const Plan& plan() const { return plan_; }
    const std::vector<uint32_t>& bindables() const { return bindables_; }

    /// Device-resident run on `stream`; returns an ABI status code and sets
    /// `why` on failure. With `arena`, every scratch buffer (temps and
    /// launcher scratch) is carved out of it and nothing is allocated; steps
    /// that need a host read-back are refused (checked loop nests).
    int runDevice(const DeviceBinding* binds, int n, const double* scalars, int64_t nScalars,
                  int64_t elements, void* stream, std::string& why, const ScratchArena* arena = nullptr) const;

    /// Host f64 run (the mlk_kernel artifact ABI): converts, uploads, runs,
    /// downloads, synchronously.
    int runHost(double* const* ptrs, int n, const double* scalars, int64_t nScalars,
                int64_t elements, std::string& why) const;

    /// Fingerprint of the variant cache entry (module hash, target, hipRTC
    /// version, policy, device) and whether the build applied a cached entry.
    const std::string& fingerprint() const { return fingerprint_; }
    bool variantsFromCache() const { return fromCache_; }

    /// Pins step `step` to launch form `variant` (-1: the kernel's default);
    /// refuses a form outside the step's variant space.
    int setStepVariant(int step, int variant, std::string& why);

    /// The kernel symbol step `si` launches (its hipRTC instance, or the
    /// precompiled kernel its launcher picks for the step's shape, dtypes
    /// and pinned form); the text lives as long as the artifact.
    const char* stepKernelName(size_t si) const;

    /// Waits for `stream`, then frees the scratch set runs on it allocated.
    int releaseStreamScratch(void* stream, std::string& why);

    /// Times every launch form of every step that has more than one on the
    /// caller's device buffers, certifies each against the default form's
    /// outputs, keeps the fastest certified form per step and, when
    /// `cacheDir` is not empty, stores the choice under the fingerprint. The
    /// written buffers are snapshotted first and restored before returning.
    /// `report` receives a JSON document of every candidate.
    int autotune(const DeviceBinding* binds, int n, const double* scalars, int64_t nScalars,
                 int64_t elements, int reps, const std::string& cacheDir, std::string& report,
                 std::string& why);

private:
    friend Result<std::unique_ptr<HipLoadedKernel>> buildHipKernelArtifact(
        const KernelModule& km, const HipBackendDriverConfig& config);
    KernelModule km_;
    Plan plan_;
    std::string arch_;
    std::string cacheDir_;
    std::string fingerprint_;
    bool fromCache_{false};
    std::vector<uint32_t> bindables_;   // buffer ids in table order
    std::vector<int> bindIndex_;        // buffer id -> bindable index or -1
    // Artifact-owned device scratch of the runs on one stream: temps (zeroed
    // on every run like the reference's fresh temp storage), the status word
    // of loop-nest steps with run-time bounds checks, and per-step scratch a
    // launcher asks for (score-softmax row statistics). Allocated on first
    // use and kept until the artifact or the stream's set is released
    // (releaseStreamScratch). Each stream gets its own set, so runs on
    // different streams never share device memory; runs on one stream are
    // ordered by it.
    struct RunScratch {
        std::vector<void*> temp;
        std::vector<int64_t> tempElems;
        void* status{nullptr};
        std::vector<void*> step;
        std::vector<int64_t> stepBytes;
    };
    RunScratch& scratchFor(void* stream) const;  // caller holds scratchLock_
    static void freeScratch(RunScratch& rs);
    /// Offsets of a run's scratch in `arena`; refuses what does not fit or
    /// needs a host read-back.
    int arenaLayout(const DeviceBinding* binds, int64_t elements, const ScratchArena& arena,
                    std::vector<size_t>& tempOff, std::vector<size_t>& stepOff, std::vector<size_t>& padOff,
                    std::string& why) const;
    void fillScoreParams(const Step& st, const std::vector<void*>& ptr, mlkd_score_softmax& p) const;
    void fillGemmParams(const Step& st, const std::vector<void*>& ptr, mlkd_gemm& p) const;
    void fillSoftmaxParams(const Step& st, const std::vector<void*>& ptr, mlkd_softmax& p) const;
    mutable std::set<std::string> kernelNames_;  // under scratchLock_
    /// Loop-nest launch form `form` (1-4) of step `si`, compiled on first
    /// use under scratchLock_.
    int ensureNestForm(size_t si, int form, void*& fn, std::string& why) const;
    mutable std::mutex scratchLock_;
    mutable std::vector<std::pair<void*, std::unique_ptr<RunScratch>>> scratchByStream_;
    // Page-locked staging of the host-buffer run (runHost), at most 64 MiB,
    // used as two halves: each buffer is converted into one half while the
    // other half's chunk is in flight over PCIe. Allocated on the first
    // host-buffer run and kept until the artifact is released.
    // Host-buffer runs of one artifact hold hostLock_ for the whole call, so
    // they run one at a time.
    mutable std::mutex hostLock_;
    mutable void* hostStage_{nullptr};
    mutable size_t hostStageBytes_{0};
    mutable void* hostEvent_[2]{nullptr, nullptr};   // one per staging half
    // Loop-nest launch forms 1-4 (no LDS slabs; 512 and 64 threads per
    // workgroup; one fewer collapsed loop), each compiled on first use; form
    // 0 is the step's own.
    mutable std::vector<std::array<void*, 5>> nestFormFn_;
};

/// Essential work of a module (the reference's EssentialWork,
/// fastkernel/include/mlk/fastkernel/fast_kernel.h:100-117): bytes of every
/// non-temp input and output moved once, at the buffer's own element size;
/// operations by the reference's walk (fast_kernel.cpp:228-317).
struct EssentialWork {
    int64_t minBytes{0};
    int64_t minOps{0};
    bool bytesKnown{true};
    bool opsKnown{true};
};
EssentialWork essentialWork(const KernelModule& km);

/// max(bytes / bandwidth, ops / throughput), or 0 when either count is
/// unknown (fast_kernel.cpp:372-384).
double rooflineLowerSec(const EssentialWork& w, double bytesPerSec, double opsPerSec);

/// The MI355X datasheet rate a plan's operations are priced at.
double peakOpsPerSec(const KernelModule& km, const Plan& plan);

/// JSON launch-coverage certificate of one step (the GPU counterpart of
/// certifyLaunchCoverage, fast_kernel.cpp:386-497).
std::string launchCoverage(const KernelModule& km, const Step& st, int64_t elements);

/// The device's measured HBM bandwidth and f16 MFMA rate (the environment
/// model of fast_kernel.h:66-84), probed once per process on first use.
struct MeasuredEnvironment {
    bool ok{false};
    double bytesPerSec{0.0};
    double f16FlopsPerSec{0.0};
};
const MeasuredEnvironment& measuredEnvironment();

/// Launch forms a step's hand-written kernel offers for its shape (empty
/// when there is only the default); the first entry is the default form.
std::vector<int> variantSpace(const KernelModule& km, const Step& st);

/// Variant-cache fingerprint of a planned module on device 0.
std::string artifactFingerprint(const KernelModule& km, const Plan& plan, const std::string& arch);

/// Applies <dir>/fk-<fingerprint>.json to the plan's steps when the file
/// exists, names the same fingerprint and lists a form of each step's
/// variant space; returns whether it applied.
bool applyCachedVariants(const std::string& dir, const std::string& fingerprint, const KernelModule& km,
                         Plan& plan);

/// C++ source of the per-module artifact libmlk_kernel.so (artifact.cpp):
/// `mlk_kernel` in the module's ABI form, forwarding to this library.
Result<std::string> artifactSource(const std::string& moduleJson, const KernelModule& km, const Plan& plan,
                                   const std::string& arch);

/// Writes <dir>/mlk_kernel.cpp and compiles it out of process with
/// `compiler` (empty: c++) into <dir>/libmlk_kernel.so; returns its path.
Result<std::string> emitArtifact(const std::string& moduleJson, const std::string& arch, const std::string& compiler,
                                 const std::string& dir);

/// Records `message` as this thread's mlkhip_last_error and returns `code`.
int setLastError(int code, const std::string& message);

/// Plans, instantiates and loads (buildGpuKernelArtifact analogue).
Result<std::unique_ptr<HipLoadedKernel>> buildHipKernelArtifact(const KernelModule& km,
                                                                const HipBackendDriverConfig& config);

}  // namespace mlk::hip
