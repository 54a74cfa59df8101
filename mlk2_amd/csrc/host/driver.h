// C++ driver of the HIP backend: the gfx950 counterpart of the reference's
// GPU artifact driver (backends/cpu/include/mlk/backend/backend_driver.h:
// 91-228). Building an artifact plans the module onto the hand-written
// kernels and loads every template instance it needs; running it binds
// buffers exactly as LoadedKernel::run does (table order, temps owned by the
// artifact, zero-initialized per run).
#pragma once

#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

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

class HipLoadedKernel {
public:
    ~HipLoadedKernel();  // frees the artifact-owned scratch (temps, status word)

    const KernelModule& module() const { return km_; }
    const Plan& plan() const { return plan_; }
    const std::vector<uint32_t>& bindables() const { return bindables_; }

    /// Device-resident run on `stream`; returns an ABI status code and sets
    /// `why` on failure.
    int runDevice(const DeviceBinding* binds, int n, const double* scalars, int64_t nScalars,
                  int64_t elements, void* stream, std::string& why) const;

    /// Host f64 run (the mlk_kernel artifact ABI): converts, uploads, runs,
    /// downloads, synchronously.
    int runHost(double* const* ptrs, int n, const double* scalars, int64_t nScalars,
                int64_t elements, std::string& why) const;

private:
    friend Result<std::unique_ptr<HipLoadedKernel>> buildHipKernelArtifact(
        const KernelModule& km, const HipBackendDriverConfig& config);
    KernelModule km_;
    Plan plan_;
    std::string arch_;
    std::vector<uint32_t> bindables_;   // buffer ids in table order
    std::vector<int> bindIndex_;        // buffer id -> bindable index or -1
    // Artifact-owned temp scratch (allocated on first use, kept; zeroed on
    // every run like the reference's fresh temp storage).
    mutable std::mutex scratchLock_;
    mutable std::vector<void*> scratch_;
    mutable std::vector<int64_t> scratchElems_;
    // Status word of loop-nest steps with run-time bounds checks.
    mutable void* status_{nullptr};
    // Per-step device scratch a launcher asks for (score-softmax row
    // statistics), allocated on first use and kept.
    mutable std::vector<void*> stepScratch_;
    mutable std::vector<int64_t> stepScratchBytes_;
};

/// Plans, instantiates and loads (buildGpuKernelArtifact analogue).
Result<std::unique_ptr<HipLoadedKernel>> buildHipKernelArtifact(const KernelModule& km,
                                                                const HipBackendDriverConfig& config);

}  // namespace mlk::hip
