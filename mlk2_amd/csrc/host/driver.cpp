// HIP backend driver and the C ABI of include/mlk_hip.h.
#include "driver.h"

#include <pthread.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <new>
#include <unordered_map>

#include "../device/runtime_abi.h"
#include "../../../include/mlk_hip.h"

namespace mlk::hip {

namespace {

int dtypeCode(Dtype d) { return d == Dtype::F32 ? MLKD_F32 : (d == Dtype::F16 ? MLKD_F16 : MLKD_F64); }

unsigned gridFor(int64_t threads, int64_t perGroup = 256) {
    int64_t blocks = (threads + perGroup - 1) / perGroup;
    // Grid-stride beyond 64 workgroups of 4 waves per CU on 256 CUs.
    if (blocks > 16384) blocks = 16384;
    if (blocks < 1) blocks = 1;
    return static_cast<unsigned>(blocks);
}

/// f64 -> f16 bits with one rounding (round to nearest even), including
/// subnormals, overflow to inf and NaN.
uint16_t toHalfBits(double d) {
    const _Float16 h = static_cast<_Float16>(d);
    uint16_t bits = 0;
    std::memcpy(&bits, &h, sizeof(bits));
    return bits;
}

double fromHalfBits(uint16_t bits) {
    _Float16 h;
    std::memcpy(&h, &bits, sizeof(h));
    return static_cast<double>(h);
}

struct RangeJob {
    const void* fn;
    void (*call)(const void*, int64_t, int64_t);
    int64_t begin, end;
};

void* rangeThread(void* p) {
    const RangeJob* j = static_cast<const RangeJob*>(p);
    j->call(j->fn, j->begin, j->end);
    return nullptr;
}

/// Runs fn(begin, end) over [0, n) split across up to 16 host threads, each
/// taking at least 2^18 elements; below 2^20 elements, or for a thread that
/// cannot be started, the calling thread runs the range itself. The host
/// ABI's dtype conversions are element-wise, so the split changes no result.
template <typename F>
void parallelRange(int64_t n, const F& fn) {
    constexpr int kMaxThreads = 16;
    const long cpus = sysconf(_SC_NPROCESSORS_ONLN);
    int64_t t = std::min<int64_t>({kMaxThreads, cpus > 0 ? cpus : 1, n >> 18});
    if (n < (int64_t{1} << 20) || t < 2) {
        fn(int64_t{0}, n);
        return;
    }
    RangeJob jobs[kMaxThreads];
    pthread_t threads[kMaxThreads];
    bool started[kMaxThreads] = {};
    for (int64_t i = 0; i < t; ++i) {
        jobs[i] = {&fn, [](const void* f, int64_t b, int64_t e) { (*static_cast<const F*>(f))(b, e); }, n * i / t,
                   n * (i + 1) / t};
    }
    for (int64_t i = 1; i < t; ++i) started[i] = pthread_create(&threads[i], nullptr, rangeThread, &jobs[i]) == 0;
    fn(jobs[0].begin, jobs[0].end);
    for (int64_t i = 1; i < t; ++i) {
        if (started[i]) {
            pthread_join(threads[i], nullptr);
        } else {
            fn(jobs[i].begin, jobs[i].end);
        }
    }
}

/// The caller's f64 values [0, cnt) as `dt` elements at `out` (one rounding
/// to nearest even for f32 and f16).
void narrowTo(void* out, const double* src, int64_t cnt, Dtype dt) {
    if (dt == Dtype::F64) {
        double* o = static_cast<double*>(out);
        parallelRange(cnt, [&](int64_t b, int64_t e) {
            std::memcpy(o + b, src + b, static_cast<size_t>(e - b) * sizeof(double));
        });
    } else if (dt == Dtype::F32) {
        float* o = static_cast<float*>(out);
        parallelRange(cnt, [&](int64_t b, int64_t e) {
            for (int64_t x = b; x < e; ++x) o[x] = static_cast<float>(src[x]);
        });
    } else {
        uint16_t* o = static_cast<uint16_t*>(out);
        parallelRange(cnt, [&](int64_t b, int64_t e) {
            for (int64_t x = b; x < e; ++x) o[x] = toHalfBits(src[x]);
        });
    }
}

/// `dt` elements [0, cnt) at `in`, widened exactly into the caller's f64s.
void widenFrom(double* dst, const void* in, int64_t cnt, Dtype dt) {
    if (dt == Dtype::F64) {
        const double* s = static_cast<const double*>(in);
        parallelRange(cnt, [&](int64_t b, int64_t e) {
            std::memcpy(dst + b, s + b, static_cast<size_t>(e - b) * sizeof(double));
        });
    } else if (dt == Dtype::F32) {
        const float* s = static_cast<const float*>(in);
        parallelRange(cnt, [&](int64_t b, int64_t e) {
            for (int64_t x = b; x < e; ++x) dst[x] = static_cast<double>(s[x]);
        });
    } else {
        const uint16_t* s = static_cast<const uint16_t*>(in);
        parallelRange(cnt, [&](int64_t b, int64_t e) {
            for (int64_t x = b; x < e; ++x) dst[x] = fromHalfBits(s[x]);
        });
    }
}

constexpr size_t kHostStageBytes = size_t{64} << 20;

}  // namespace

bool validArch(const std::string& arch) {
    if (arch.size() < 6 || arch.size() > 7 || arch.compare(0, 3, "gfx") != 0) return false;
    for (size_t i = 3; i < arch.size(); ++i) {
        const char c = arch[i];
        const bool hex = (c >= '0' && c <= '9') || (c >= 'a' && c <= 'f');
        if (!hex) return false;
    }
    return true;
}

Result<std::unique_ptr<HipLoadedKernel>> buildHipKernelArtifact(const KernelModule& km,
                                                                const HipBackendDriverConfig& config) {
    if (!validArch(config.arch)) {
        return err(ErrorCode::InvalidArgument, "invalid HIP target '" + config.arch + "' (want gfx<hex>)");
    }
    std::unique_ptr<HipLoadedKernel> k(new HipLoadedKernel());
    k->km_ = deviceModule(km);
    auto plan = planModule(k->km_);
    if (!plan.has_value()) return err(plan.error().code, plan.error().message);
    k->plan_ = std::move(*plan);
    k->arch_ = config.arch;
    k->cacheDir_ = config.cacheDir;
    k->bindIndex_.assign(km.buffers.size(), -1);
    for (uint32_t b = 0; b < km.buffers.size(); ++b) {
        const KernelBuffer& kb = km.buffers[b];
        if (kb.isInput || kb.isOutput || kb.isTemp) {
            k->bindIndex_[b] = static_cast<int>(k->bindables_.size());
            k->bindables_.push_back(b);
        }
    }
    for (const Step& st : k->plan_.steps) {
        const uint32_t ids[] = {st.out.buffer, st.x, st.y, st.a, st.b, st.c, st.q, st.kk, st.bias, st.s};
        for (const uint32_t id : ids) {
            if (id != kInvalidId && (id >= km.buffers.size() || k->bindIndex_[id] < 0)) {
                return err(ErrorCode::InvalidGraph, "step references a buffer that is not bindable");
            }
        }
        for (const StreamRef& s : st.inputs) {
            if (s.buffer >= km.buffers.size() || k->bindIndex_[s.buffer] < 0) {
                return err(ErrorCode::InvalidGraph, "operand buffer is not bindable");
            }
        }
        for (const uint32_t b : st.nestBufs) {
            if (b >= km.buffers.size() || k->bindIndex_[b] < 0) {
                return err(ErrorCode::InvalidGraph, "loop-nest buffer is not bindable");
            }
        }
    }
    const int devices = mlkd_rt_device_count();
    if (devices <= 0) return err(ErrorCode::UnsupportedCapability, "no HIP device visible");
    char devArch[128] = {0};
    if (mlkd_rt_device_arch(0, devArch, sizeof(devArch)) != 0 ||
        std::strncmp(devArch, config.arch.c_str(), config.arch.size()) != 0) {
        return err(ErrorCode::UnsupportedCapability,
                   "declared target " + config.arch + " does not match device " + devArch);
    }
    for (Step& st : k->plan_.steps) {
        if (st.kind != StepKind::Elementwise && st.kind != StepKind::Nest) continue;
        const bool nest = st.kind == StepKind::Nest;
        if (nest) {
            st.kernelName = "mlk_nest";
        } else {
            st.source = elementwiseSource(k->km_, st, &st.kernelName);
        }
        char log[4096] = {0};
        void* fn = nullptr;
        uint64_t fp = 0;
        const int rc = mlkd_jit_build(st.source.data(), st.source.size(), st.kernelName.c_str(),
                                      config.arch.c_str(), config.cacheDir.c_str(), &fn, &fp, log,
                                      sizeof(log));
        if (rc != 0) {
            return err(ErrorCode::UnsupportedCapability,
                       std::string(nest ? "loop-nest instance: " : "template instance: ") + log);
        }
        st.fn = fn;
    }
    k->fingerprint_ = artifactFingerprint(k->km_, k->plan_, config.arch);
    k->fromCache_ = applyCachedVariants(config.cacheDir, k->fingerprint_, k->km_, k->plan_);
    k->nestFormFn_.assign(k->plan_.steps.size(), std::array<void*, 5>{});
    for (size_t si = 0; si < k->plan_.steps.size(); ++si) {
        const Step& st = k->plan_.steps[si];
        if (st.kind != StepKind::Nest || st.variant < 1 || st.variant > 4) continue;
        void* fn = nullptr;
        std::string why;
        if (k->ensureNestForm(si, st.variant, fn, why) != MLKHIP_OK) {
            return err(ErrorCode::UnsupportedCapability, "cached loop-nest launch form: " + why);
        }
    }
    return k;
}

void HipLoadedKernel::freeScratch(RunScratch& rs) {
    for (void* p : rs.temp) {
        if (p != nullptr) mlkd_rt_free(p);
    }
    if (rs.status != nullptr) mlkd_rt_free(rs.status);
    for (void* p : rs.step) {
        if (p != nullptr) mlkd_rt_free(p);
    }
}

HipLoadedKernel::~HipLoadedKernel() {
    for (auto& [stream, rs] : scratchByStream_) {
        (void)stream;
        freeScratch(*rs);
    }
    mlkd_rt_event_destroy(hostEvent_[0]);
    mlkd_rt_event_destroy(hostEvent_[1]);
    mlkd_rt_host_free(hostStage_);
}

int HipLoadedKernel::releaseStreamScratch(void* stream, std::string& why) {
    std::lock_guard<std::mutex> g(scratchLock_);
    for (size_t i = 0; i < scratchByStream_.size(); ++i) {
        if (scratchByStream_[i].first != stream) continue;
        if (mlkd_rt_sync(stream) != 0) {
            why = "stream wait failed";
            return MLKHIP_LAUNCH;
        }
        freeScratch(*scratchByStream_[i].second);
        scratchByStream_.erase(scratchByStream_.begin() + static_cast<std::ptrdiff_t>(i));
        return MLKHIP_OK;
    }
    return MLKHIP_OK;
}

HipLoadedKernel::RunScratch& HipLoadedKernel::scratchFor(void* stream) const {
    for (auto& [s, rs] : scratchByStream_) {
        if (s == stream) return *rs;
    }
    std::unique_ptr<RunScratch> rs(new RunScratch());
    rs->temp.assign(km_.buffers.size(), nullptr);
    rs->tempElems.assign(km_.buffers.size(), 0);
    rs->step.assign(plan_.steps.size(), nullptr);
    rs->stepBytes.assign(plan_.steps.size(), 0);
    scratchByStream_.emplace_back(stream, std::move(rs));
    return *scratchByStream_.back().second;
}

namespace {
size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }
}  // namespace

void HipLoadedKernel::fillScoreParams(const Step& st, const std::vector<void*>& ptr, mlkd_score_softmax& p) const {
    p.variant = st.variant;
    p.q = ptr[st.q];
    p.k = ptr[st.kk];
    p.bias = ptr[st.bias];
    p.s = ptr[st.s];
    p.qk_dtype = dtypeCode(km_.buffers[st.q].dtype);
    p.bias_dtype = dtypeCode(km_.buffers[st.bias].dtype);
    p.s_dtype = dtypeCode(km_.buffers[st.s].dtype);
    p.batch = st.batch;
    p.seq = st.seq;
    p.dim = st.dim;
    p.div = st.div;
    p.scratch = nullptr;
    p.scratch_bytes = 0;
    p.work = nullptr;
    p.work_bytes = 0;
}

int HipLoadedKernel::ensureNestForm(size_t si, int form, void*& fn, std::string& why) const {
    std::lock_guard<std::mutex> g(scratchLock_);
    if (nestFormFn_[si][form] == nullptr) {
        const std::string src = nestFormSource(plan_.steps[si], form);
        if (src.empty()) {
            why = "loop-nest launch form " + std::to_string(form) + " is not declared for this step";
            return MLKHIP_REFUSED;
        }
        char log[4096] = {0};
        uint64_t fp = 0;
        if (mlkd_jit_build(src.data(), src.size(), "mlk_nest", arch_.c_str(), cacheDir_.c_str(),
                           &nestFormFn_[si][form], &fp, log, sizeof(log)) != 0) {
            nestFormFn_[si][form] = nullptr;
            why = "loop-nest launch form " + std::to_string(form) + ": " + log;
            return MLKHIP_RUNTIME;
        }
    }
    fn = nestFormFn_[si][form];
    return MLKHIP_OK;
}

void HipLoadedKernel::fillSoftmaxParams(const Step& st, const std::vector<void*>& ptr, mlkd_softmax& p) const {
    p.variant = st.variant;
    p.pad = 0;
    p.x = ptr[st.x];
    p.y = ptr[st.y];
    p.x_dtype = dtypeCode(km_.buffers[st.x].dtype);
    p.y_dtype = dtypeCode(km_.buffers[st.y].dtype);
    p.rows = st.rows;
    p.cols = st.cols;
    p.x_row_stride = st.cols;
    p.y_row_stride = st.kind == StepKind::Softmax ? st.cols : 1;
}

const char* HipLoadedKernel::stepKernelName(size_t si) const {
    const Step& st = plan_.steps[si];
    std::string name = st.kernelName;
    if (name.empty()) {
        // What the launcher picks for this step's shape, dtypes and pinned
        // form, on device buffers as the runtime allocates them (256-byte
        // aligned) with the scratch the driver gives it.
        std::vector<void*> ptr(km_.buffers.size(), reinterpret_cast<void*>(uintptr_t{1} << 12));
        if (st.kind == StepKind::Softmax) {
            mlkd_softmax p;
            fillSoftmaxParams(st, ptr, p);
            name = mlkd_softmax_kernel_name(&p);
        } else if (st.kind == StepKind::RowSum) {
            name = "rowSumWave";
        } else if (st.kind == StepKind::Gemm) {
            mlkd_gemm p;
            fillGemmParams(st, ptr, p);
            if (const int64_t need = mlkd_gemm_pad_bytes(&p); need > 0) {
                p.work = ptr[0];   // runDevice gives such a step its padding workspace
                p.work_bytes = need;
            }
            name = mlkd_gemm_kernel_name(&p);
        } else if (st.kind == StepKind::ScoreSoftmax) {
            mlkd_score_softmax p;
            fillScoreParams(st, ptr, p);
            if (const int64_t need = mlkd_score_scratch_bytes(&p); need > 0) {
                p.scratch = ptr[0];
                p.scratch_bytes = need;
            }
            if (const int64_t need = mlkd_score_pad_bytes(&p); need > 0) {
                p.work = ptr[0];   // runDevice gives such a step its padding workspace
                p.work_bytes = need;
            }
            name = mlkd_score_kernel_names(&p);
        }
    }
    std::lock_guard<std::mutex> g(scratchLock_);
    return kernelNames_.insert(name).first->c_str();
}

void HipLoadedKernel::fillGemmParams(const Step& st, const std::vector<void*>& ptr, mlkd_gemm& p) const {
    p.variant = st.variant;
    p.skip_zero_a = st.skipZeroA && st.k > 0 ? 1 : 0;
    p.a = ptr[st.a];
    p.b = ptr[st.b];
    p.c = ptr[st.c];
    p.a_dtype = dtypeCode(km_.buffers[st.a].dtype);
    p.b_dtype = dtypeCode(km_.buffers[st.b].dtype);
    p.c_dtype = dtypeCode(km_.buffers[st.c].dtype);
    p.accumulate = st.accumulate ? 1 : 0;
    p.m = st.m;
    p.n = st.n;
    p.k = st.k;
    p.lda = st.lda;
    p.ldb = st.ldb;
    p.ldc = st.ldc;
    p.pad_ = 0;
    p.work = nullptr;
    p.work_bytes = 0;
}

int HipLoadedKernel::arenaLayout(const DeviceBinding* binds, int64_t elements, const ScratchArena& arena,
                                 std::vector<size_t>& tempOff, std::vector<size_t>& stepOff,
                                 std::vector<size_t>& padOff, std::string& why) const {
    size_t used = 0;
    tempOff.assign(km_.buffers.size(), 0);
    stepOff.assign(plan_.steps.size(), 0);
    for (size_t i = 0; i < bindables_.size(); ++i) {
        const uint32_t b = bindables_[i];
        const KernelBuffer& kb = km_.buffers[b];
        if (!kb.isTemp || binds[i].ptr != nullptr || !plan_.tempNeeded[b]) continue;
        tempOff[b] = used;
        used += align256(static_cast<size_t>(bufferElements(kb, elements)) * dtypeBytes(kb.dtype));
    }
    std::vector<void*> ptr(km_.buffers.size(), nullptr);
    for (size_t i = 0; i < bindables_.size(); ++i) ptr[bindables_[i]] = binds[i].ptr;
    for (size_t si = 0; si < plan_.steps.size(); ++si) {
        const Step& st = plan_.steps[si];
        if (st.kind == StepKind::Nest &&
            nestFormChecked(st, st.variant >= 1 && st.variant <= 4 ? st.variant : 0)) {
            why = "step " + std::to_string(si) + " (loop nest) reports run-time bounds checks through a host "
                  "read-back, which the allocation-free entry does not do";
            return MLKHIP_REFUSED;
        }
        if (st.kind == StepKind::Nest && st.variant >= 1 && st.variant <= 4) {
            // Pinned forms are compiled when they are pinned (at build from
            // the variant cache, or by setStepVariant); this is a guard.
            std::lock_guard<std::mutex> g(scratchLock_);
            if (nestFormFn_[si][st.variant] == nullptr) {
                why = "step " + std::to_string(si) + " pins loop-nest launch form " + std::to_string(st.variant) +
                      ", which is not loaded";
                return MLKHIP_REFUSED;
            }
        }
        int64_t need = 0;
        if (st.kind == StepKind::ScoreSoftmax) {
            mlkd_score_softmax p;
            fillScoreParams(st, ptr, p);
            need = mlkd_score_scratch_bytes(&p);
        }
        if (need > 0) {
            stepOff[si] = used;
            used += align256(static_cast<size_t>(need));
        }
    }
    if (used > arena.bytes) {
        why = "the run needs " + std::to_string(used) + " bytes of device scratch; the allocation-free entry holds " +
              std::to_string(arena.bytes);
        return MLKHIP_REFUSED;
    }
    // Padding workspaces (GEMM shapes off the MFMA tiles, score-softmax
    // lengths off the two-pass blocks) take the room that is left, in step
    // order; a step whose workspace does not fit runs on the general kernels.
    padOff.assign(plan_.steps.size(), SIZE_MAX);
    for (size_t si = 0; si < plan_.steps.size(); ++si) {
        const Step& st = plan_.steps[si];
        int64_t pad = 0;
        if (st.kind == StepKind::Gemm) {
            mlkd_gemm p;
            fillGemmParams(st, ptr, p);
            pad = mlkd_gemm_pad_bytes(&p);
        } else if (st.kind == StepKind::ScoreSoftmax) {
            mlkd_score_softmax p;
            fillScoreParams(st, ptr, p);
            pad = mlkd_score_pad_bytes(&p);
        }
        if (pad > 0 && align256(static_cast<size_t>(pad)) <= arena.bytes - used) {
            padOff[si] = used;
            used += align256(static_cast<size_t>(pad));
        }
    }
    return MLKHIP_OK;
}

int HipLoadedKernel::runDevice(const DeviceBinding* binds, int n, const double* scalars,
                               int64_t nScalars, int64_t elements, void* stream,
                               std::string& why, const ScratchArena* arena) const {
    if (n != static_cast<int>(bindables_.size())) {
        why = "expected " + std::to_string(bindables_.size()) + " bindings, got " + std::to_string(n);
        return MLKHIP_BAD_BINDING;
    }
    // Scratch comes from the caller's arena (the allocation-free entry), laid
    // out before anything is launched, or from this stream's own allocations.
    std::vector<size_t> tempOff, stepOff, padOff;
    if (arena != nullptr) {
        if (const int rc = arenaLayout(binds, elements, *arena, tempOff, stepOff, padOff, why); rc != MLKHIP_OK) {
            return rc;
        }
    }
    RunScratch* rs = nullptr;
    if (arena == nullptr) {
        std::lock_guard<std::mutex> g(scratchLock_);
        rs = &scratchFor(stream);
    }
    auto statusWord = [&]() -> void* {
        std::lock_guard<std::mutex> g(scratchLock_);
        if (rs->status == nullptr && mlkd_rt_malloc(&rs->status, 256) != 0) rs->status = nullptr;
        return rs->status;
    };
    std::vector<void*> ptr(km_.buffers.size(), nullptr);
    for (int i = 0; i < n; ++i) {
        const uint32_t b = bindables_[static_cast<size_t>(i)];
        const KernelBuffer& kb = km_.buffers[b];
        const int64_t need = bufferElements(kb, elements);
        if (kb.isTemp && binds[i].ptr == nullptr) {
            if (!plan_.tempNeeded[b]) continue;
            if (arena != nullptr) {
                ptr[b] = arena->base + tempOff[b];
            } else {
                std::lock_guard<std::mutex> g(scratchLock_);
                if (rs->temp[b] == nullptr || rs->tempElems[b] < need) {
                    if (rs->temp[b] != nullptr) mlkd_rt_free(rs->temp[b]);
                    rs->temp[b] = nullptr;
                    if (mlkd_rt_malloc(&rs->temp[b], static_cast<size_t>(need) * dtypeBytes(kb.dtype) + 16) != 0) {
                        rs->temp[b] = nullptr;
                        why = "temp scratch allocation failed";
                        return MLKHIP_RUNTIME;
                    }
                    rs->tempElems[b] = need;
                }
                ptr[b] = rs->temp[b];
            }
        } else {
            if (binds[i].dtype != dtypeCode(kb.dtype)) {
                why = "binding " + std::to_string(i) + " (" + kb.name + ") has the wrong dtype";
                return MLKHIP_BAD_BINDING;
            }
            if (need < 0 || binds[i].elements < need || (binds[i].ptr == nullptr && need > 0)) {
                why = "binding " + std::to_string(i) + " (" + kb.name + ") holds " +
                      std::to_string(binds[i].elements) + " elements, module needs " + std::to_string(need);
                return MLKHIP_BAD_BINDING;
            }
            ptr[b] = binds[i].ptr;
        }
        if (kb.isTemp && plan_.tempNeeded[b]) {
            // Fresh zeroed scratch per run (kernel_buffers.cpp:852-878).
            const size_t bytes = static_cast<size_t>(need) * dtypeBytes(kb.dtype);
            const size_t padded = (bytes + 3) & ~static_cast<size_t>(3);
            if (mlkd_rt_fill32(ptr[b], 0u, padded, stream) != 0) {
                why = "temp zero-fill failed";
                return MLKHIP_LAUNCH;
            }
        }
    }
    mlkd_scalars sc;
    for (int i = 0; i < MLKD_MAX_SCALARS; ++i) sc.v[i] = (scalars != nullptr && i < nScalars) ? scalars[i] : 0.0;
    for (size_t si = 0; si < plan_.steps.size(); ++si) {
        const Step& st = plan_.steps[si];
        int rc = 0;
        switch (st.kind) {
            case StepKind::Fail:
                if (st.failCode != 0) {
                    why = "negative store address";
                    return st.failCode;
                }
                break;
            case StepKind::Elementwise: {
                int64_t ext0 = st.extent[0];
                if (st.dynamicExtent) {
                    ext0 = elements - st.dynBegin;
                    if (ext0 <= 0) break;
                    for (const StreamRef& s : st.inputs) {
                        const int64_t have = binds[bindIndex_[s.buffer]].elements;
                        if (st.dynBegin < 0 || have < elements) {
                            why = "dynamic 1-D loop reaches past an operand buffer";
                            return MLKHIP_BAD_BINDING;
                        }
                    }
                    if (binds[bindIndex_[st.out.buffer]].elements < elements) {
                        why = "dynamic 1-D loop reaches past the output buffer";
                        return MLKHIP_BAD_BINDING;
                    }
                }
                const void* in[4] = {nullptr, nullptr, nullptr, nullptr};
                for (size_t i = 0; i < st.inputs.size(); ++i) {
                    in[i] = ptr[st.inputs[i].buffer];
                    if (st.dynamicExtent) {
                        in[i] = static_cast<const char*>(in[i]) +
                                st.dynBegin * dtypeBytes(km_.buffers[st.inputs[i].buffer].dtype);
                    }
                }
                void* out = ptr[st.out.buffer];
                if (st.dynamicExtent) {
                    out = static_cast<char*>(out) + st.dynBegin * dtypeBytes(km_.buffers[st.out.buffer].dtype);
                }
                int64_t rows = 1;
                for (int d = 0; d < st.rank - 1; ++d) rows *= st.extent[d];
                const int64_t w = st.rank == 1 ? ext0 : st.extent[st.rank - 1];
                // One wave per row segment (the template's kSeg).
                const int64_t threads =
                    rows * ((w + kElementwiseSegment - 1) / kElementwiseSegment) * 64;
                rc = mlkd_jit_launch_elementwise(st.fn, gridFor(threads), in, out, &sc, ext0, stream);
                break;
            }
            case StepKind::Softmax:
            case StepKind::RowSum: {
                mlkd_softmax p;
                fillSoftmaxParams(st, ptr, p);
                rc = st.kind == StepKind::Softmax ? mlkd_launch_softmax(&p, stream) : mlkd_launch_rowsum(&p, stream);
                break;
            }
            case StepKind::Gemm: {
                mlkd_gemm p;
                fillGemmParams(st, ptr, p);
                // The skip-zero-A decision (0 * inf and 0 * NaN are the only
                // products whose skip changes C beyond the sign of a zero
                // sum) is taken inside the MFMA kernel, per wave: one launch,
                // no host read-back.
                // A shape the MFMA forms do not tile runs on zero-padded
                // copies in a per-stream workspace, or, for the
                // allocation-free entry, in the arena when they fit there
                // (else on the general kernel).
                const int64_t need = mlkd_gemm_pad_bytes(&p);
                if (need > 0 && arena != nullptr && padOff[si] != SIZE_MAX) {
                    p.work = arena->base + padOff[si];
                    p.work_bytes = need;
                } else if (need > 0 && arena == nullptr) {
                    std::lock_guard<std::mutex> g(scratchLock_);
                    if (rs->step[si] == nullptr || rs->stepBytes[si] < need) {
                        if (rs->step[si] != nullptr) mlkd_rt_free(rs->step[si]);
                        rs->step[si] = nullptr;
                        rs->stepBytes[si] = 0;
                        if (mlkd_rt_malloc(&rs->step[si], static_cast<size_t>(need)) != 0) rs->step[si] = nullptr;
                        else rs->stepBytes[si] = need;
                    }
                    // Without the workspace the general kernel runs the step.
                    p.work = rs->step[si];
                    p.work_bytes = rs->stepBytes[si];
                }
                rc = mlkd_launch_gemm(&p, stream);
                break;
            }
            case StepKind::Nest: {
                mlkd_nest_args na;
                std::memset(&na, 0, sizeof(na));
                for (size_t sl = 0; sl < st.nestBufs.size(); ++sl) {
                    const uint32_t b = st.nestBufs[sl];
                    na.p[sl] = ptr[b];
                    const int bi = bindIndex_[b];
                    na.n[sl] = km_.buffers[b].isTemp && binds[bi].ptr == nullptr
                                   ? bufferElements(km_.buffers[b], elements)
                                   : binds[bi].elements;
                }
                na.elements = elements;
                const int form = st.variant >= 1 && st.variant <= 4 ? st.variant : 0;
                const bool checked = nestFormChecked(st, form);
                const int64_t instances = nestFormInstances(st, form);
                void* status = nullptr;
                if (checked) {
                    status = statusWord();
                    if (status == nullptr) {
                        why = "status word allocation failed";
                        return MLKHIP_RUNTIME;
                    }
                    if (mlkd_rt_fill32(status, 0u, 4, stream) != 0) {
                        why = "status word clear failed";
                        return MLKHIP_LAUNCH;
                    }
                    na.status = static_cast<int*>(status);
                }
                void* fn = st.fn;
                const unsigned wg = nestFormThreads(form);
                if (form != 0) {
                    if (const int frc = ensureNestForm(si, form, fn, why); frc != MLKHIP_OK) return frc;
                }
                rc = mlkd_jit_launch_nest(fn, gridFor(instances, wg), wg, &na, &sc, instances, stream);
                if (rc == 0 && checked) {
                    int code = 0;
                    if (mlkd_rt_d2h(&code, status, sizeof(code), stream) != 0 || mlkd_rt_sync(stream) != 0) {
                        why = "status word read-back failed";
                        return MLKHIP_LAUNCH;
                    }
                    if (code != 0) {
                        why = code == MLKHIP_NEG_STORE ? "walker: negative store address"
                                                       : "loop nest reaches outside a bound buffer";
                        return code;
                    }
                }
                break;
            }
            case StepKind::ScoreSoftmax: {
                if (km_.buffers[st.kk].dtype != km_.buffers[st.q].dtype) {
                    why = "score-softmax needs Q and K of one dtype";
                    return MLKHIP_REFUSED;
                }
                mlkd_score_softmax p;
                fillScoreParams(st, ptr, p);
                if (const int64_t need = mlkd_score_scratch_bytes(&p); need > 0 && arena != nullptr) {
                    p.scratch = arena->base + stepOff[si];
                    p.scratch_bytes = need;
                } else if (need > 0) {
                    std::lock_guard<std::mutex> g(scratchLock_);
                    if (rs->step[si] == nullptr || rs->stepBytes[si] < need) {
                        if (rs->step[si] != nullptr) mlkd_rt_free(rs->step[si]);
                        rs->step[si] = nullptr;
                        if (mlkd_rt_malloc(&rs->step[si], static_cast<size_t>(need)) != 0) {
                            rs->step[si] = nullptr;
                            why = "score-softmax scratch allocation failed";
                            return MLKHIP_RUNTIME;
                        }
                        rs->stepBytes[si] = need;
                    }
                    p.scratch = rs->step[si];
                    p.scratch_bytes = rs->stepBytes[si];
                } else if (const int64_t pad = mlkd_score_pad_bytes(&p); pad > 0 && arena != nullptr) {
                    if (padOff[si] != SIZE_MAX) {
                        p.work = arena->base + padOff[si];
                        p.work_bytes = pad;
                    }
                } else if (pad > 0) {
                    // A sequence length off the two-pass blocks runs on
                    // zero-padded copies, as for GEMM shapes off the MFMA
                    // tiles; without the workspace the general kernels run.
                    std::lock_guard<std::mutex> g(scratchLock_);
                    if (rs->step[si] == nullptr || rs->stepBytes[si] < pad) {
                        if (rs->step[si] != nullptr) mlkd_rt_free(rs->step[si]);
                        rs->step[si] = nullptr;
                        rs->stepBytes[si] = 0;
                        if (mlkd_rt_malloc(&rs->step[si], static_cast<size_t>(pad)) != 0) rs->step[si] = nullptr;
                        else rs->stepBytes[si] = pad;
                    }
                    p.work = rs->step[si];
                    p.work_bytes = rs->stepBytes[si];
                }
                rc = mlkd_launch_score_softmax(&p, stream);
                break;
            }
        }
        if (rc != 0) {
            why = std::string("launch failed: ") + mlkd_rt_last_error();
            return rc;
        }
    }
    return MLKHIP_OK;
}

int HipLoadedKernel::runHost(double* const* ptrs, int n, const double* scalars, int64_t nScalars,
                             int64_t elements, std::string& why) const {
    if (n != static_cast<int>(bindables_.size())) {
        why = "expected " + std::to_string(bindables_.size()) + " bindables, got " + std::to_string(n);
        return MLKHIP_BAD_BINDING;
    }
    // Host-buffer runs of this artifact share its page-locked staging.
    std::lock_guard<std::mutex> hostGuard(hostLock_);
    size_t maxBytes = 0;
    for (const uint32_t b : bindables_) {
        const KernelBuffer& kb = km_.buffers[b];
        const int64_t cnt = bufferElements(kb, elements);
        if (!kb.isTemp && cnt > 0) maxBytes = std::max(maxBytes, static_cast<size_t>(cnt) * dtypeBytes(kb.dtype));
    }
    // Two halves, each holding the largest buffer seen (rounded up to 256
    // bytes, so a half always holds an element), up to 32 MiB each; without
    // page-locked memory the copies go through an ordinary heap buffer.
    const size_t twoHalves = 2 * ((maxBytes + 255) & ~size_t{255});
    if (const size_t want = std::min(twoHalves, kHostStageBytes); want > hostStageBytes_) {
        void* p = nullptr;
        if (mlkd_rt_host_alloc(&p, want) == 0) {
            mlkd_rt_host_free(hostStage_);
            hostStage_ = p;
            hostStageBytes_ = want;
        }
    }
    if (hostStage_ != nullptr && hostEvent_[0] == nullptr) {
        if (mlkd_rt_event_create(&hostEvent_[0]) != 0 || mlkd_rt_event_create(&hostEvent_[1]) != 0) {
            mlkd_rt_event_destroy(hostEvent_[0]);
            hostEvent_[0] = hostEvent_[1] = nullptr;
        }
    }
    // Two halves of the staging: chunk i goes through half i % 2, and an
    // event recorded after its copy tells when that half is free again.
    const bool piped = hostStage_ != nullptr && hostEvent_[0] != nullptr;
    const size_t half = hostStageBytes_ / 2;
    auto halfPtr = [&](int64_t i) { return static_cast<unsigned char*>(hostStage_) + (i & 1) * half; };
    // Caller's f64s -> `dt` on the device, chunk by chunk through the
    // staging; converting chunk i overlaps the copy of chunk i - 1.
    auto copyIn = [&](void* d, const double* src, int64_t cnt, Dtype dt) -> bool {
        const size_t es = dtypeBytes(dt);
        if (!piped) {
            std::unique_ptr<unsigned char[]> heap(new (std::nothrow) unsigned char[static_cast<size_t>(cnt) * es]);
            if (!heap) return false;
            narrowTo(heap.get(), src, cnt, dt);
            return mlkd_rt_h2d(d, heap.get(), static_cast<size_t>(cnt) * es, nullptr) == 0 &&
                   mlkd_rt_sync(nullptr) == 0;
        }
        const int64_t per = static_cast<int64_t>(half / es);
        int64_t i = 0;
        for (int64_t c0 = 0; c0 < cnt; c0 += per, ++i) {
            const int64_t m = std::min(per, cnt - c0);
            if (i >= 2 && mlkd_rt_event_sync(hostEvent_[i & 1]) != 0) return false;   // chunk i - 2 sent
            narrowTo(halfPtr(i), src + c0, m, dt);
            if (mlkd_rt_h2d(static_cast<char*>(d) + c0 * static_cast<int64_t>(es), halfPtr(i),
                            static_cast<size_t>(m) * es, nullptr) != 0 ||
                mlkd_rt_event_record(hostEvent_[i & 1], nullptr) != 0) {
                return false;
            }
        }
        return mlkd_rt_sync(nullptr) == 0;
    };
    // Device `dt` values -> the caller's f64s: chunk i + 1 is in flight
    // while chunk i is widened.
    auto copyOut = [&](double* dst, const void* d, int64_t cnt, Dtype dt) -> bool {
        const size_t es = dtypeBytes(dt);
        if (!piped) {
            std::unique_ptr<unsigned char[]> heap(new (std::nothrow) unsigned char[static_cast<size_t>(cnt) * es]);
            if (!heap) return false;
            if (mlkd_rt_d2h(heap.get(), d, static_cast<size_t>(cnt) * es, nullptr) != 0 || mlkd_rt_sync(nullptr) != 0) {
                return false;
            }
            widenFrom(dst, heap.get(), cnt, dt);
            return true;
        }
        const int64_t per = static_cast<int64_t>(half / es);
        const int64_t chunks = (cnt + per - 1) / per;
        auto fetch = [&](int64_t i) {
            const int64_t c0 = i * per, m = std::min(per, cnt - c0);
            return mlkd_rt_d2h(halfPtr(i), static_cast<const char*>(d) + c0 * static_cast<int64_t>(es),
                               static_cast<size_t>(m) * es, nullptr) == 0 &&
                   mlkd_rt_event_record(hostEvent_[i & 1], nullptr) == 0;
        };
        if (chunks > 0 && !fetch(0)) return false;
        for (int64_t i = 0; i < chunks; ++i) {
            // Half (i + 1) % 2 last held chunk i - 1, widened in the previous pass.
            if (i + 1 < chunks && !fetch(i + 1)) return false;
            if (mlkd_rt_event_sync(hostEvent_[i & 1]) != 0) return false;
            const int64_t c0 = i * per;
            widenFrom(dst + c0, halfPtr(i), std::min(per, cnt - c0), dt);
        }
        return true;
    };
    // Buffers written by some step are copied back (outputs, and any input
    // a Store targets, as the reference writes through the caller's array).
    std::vector<bool> written(km_.buffers.size(), false);
    for (const Step& st : plan_.steps) {
        const uint32_t w[] = {st.out.buffer, st.y, st.c, st.s};
        for (const uint32_t b : w) {
            if (b != kInvalidId && b < written.size()) written[b] = true;
        }
        for (const uint32_t b : st.nestWrites) {
            if (b < written.size()) written[b] = true;
        }
    }
    std::vector<DeviceBinding> binds(bindables_.size());
    std::vector<void*> owned;
    auto cleanup = [&]() {
        for (void* p : owned) mlkd_rt_free(p);
    };
    int rc = MLKHIP_OK;
    for (size_t i = 0; i < bindables_.size(); ++i) {
        const KernelBuffer& kb = km_.buffers[bindables_[i]];
        binds[i].dtype = dtypeCode(kb.dtype);
        if (kb.isTemp) continue;  // the artifact materializes temps
        const int64_t cnt = bufferElements(kb, elements);
        if (cnt < 0) {
            why = "buffer " + kb.name + " has no size";
            cleanup();
            return MLKHIP_BAD_BINDING;
        }
        binds[i].elements = cnt;
        if (cnt == 0) continue;
        if (ptrs[i] == nullptr) {
            why = "buffer " + kb.name + " not bound";
            cleanup();
            return MLKHIP_BAD_BINDING;
        }
        const size_t bytes = static_cast<size_t>(cnt) * dtypeBytes(kb.dtype);
        void* d = nullptr;
        if (mlkd_rt_malloc(&d, bytes) != 0) {
            why = "device allocation failed";
            cleanup();
            return MLKHIP_RUNTIME;
        }
        owned.push_back(d);
        binds[i].ptr = d;
        if (!copyIn(d, ptrs[i], cnt, kb.dtype)) {
            why = "host-to-device copy failed";
            cleanup();
            return MLKHIP_RUNTIME;
        }
    }
    rc = runDevice(binds.data(), static_cast<int>(binds.size()), scalars, nScalars, elements, nullptr, why);
    if (rc == MLKHIP_OK && mlkd_rt_sync(nullptr) != 0) {
        why = "device synchronization failed";
        rc = MLKHIP_LAUNCH;
    }
    if (rc == MLKHIP_OK) {
        for (size_t i = 0; i < bindables_.size(); ++i) {
            const uint32_t b = bindables_[i];
            const KernelBuffer& kb = km_.buffers[b];
            if (kb.isTemp || !written[b] || binds[i].elements == 0) continue;
            const int64_t cnt = binds[i].elements;
            if (!copyOut(ptrs[i], binds[i].ptr, cnt, kb.dtype)) {
                why = "device-to-host copy failed";
                rc = MLKHIP_RUNTIME;
                break;
            }
        }
    }
    cleanup();
    return rc;
}

}  // namespace mlk::hip

// ------------------------------------------------------------------ C ABI --
using mlk::hip::HipLoadedKernel;

struct mlkhip_artifact {
    std::unique_ptr<HipLoadedKernel> k;
};

namespace {
thread_local std::string gLastError;

int setError(int code, const std::string& m) {
    gLastError = m;
    return code;
}

int mapBuildError(mlk::ErrorCode c) {
    return c == mlk::ErrorCode::UnsupportedCapability || c == mlk::ErrorCode::InvalidGraph ||
                   c == mlk::ErrorCode::ParseError || c == mlk::ErrorCode::InvalidArgument
               ? MLKHIP_REFUSED
               : MLKHIP_RUNTIME;
}

void copyOut(char* dst, size_t cap, const std::string& s) {
    if (dst == nullptr || cap == 0) return;
    const size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
    std::memcpy(dst, s.data(), n);
    dst[n] = '\0';
}
}  // namespace

int mlk::hip::setLastError(int code, const std::string& message) { return setError(code, message); }

extern "C" {

const char* mlkhip_last_error(void) { return gLastError.c_str(); }

int mlkhip_valid_arch(const char* arch) { return arch != nullptr && mlk::hip::validArch(arch) ? 1 : 0; }

int mlkhip_device_available(const char* arch) {
    if (mlkd_rt_device_count() <= 0) return 0;
    char dev[128] = {0};
    if (mlkd_rt_device_arch(0, dev, sizeof(dev)) != 0) return 0;
    if (arch == nullptr || arch[0] == '\0') return 1;
    return std::strncmp(dev, arch, std::strlen(arch)) == 0 ? 1 : 0;
}

int mlkhip_build(const char* module_json, size_t len, const char* arch, const char* cache_dir,
                 mlkhip_artifact** out) {
    if (out == nullptr || module_json == nullptr) return setError(MLKHIP_REFUSED, "null argument");
    *out = nullptr;
    auto km = mlk::hip::parseKernelModule(module_json, len);
    if (!km.has_value()) return setError(MLKHIP_REFUSED, km.error().message);
    mlk::hip::HipBackendDriverConfig cfg;
    cfg.arch = arch != nullptr ? arch : "";
    cfg.cacheDir = cache_dir != nullptr ? cache_dir : "";
    auto k = mlk::hip::buildHipKernelArtifact(*km, cfg);
    if (!k.has_value()) {
        const bool noDevice = k.error().message.find("no HIP device") != std::string::npos;
        return setError(noDevice ? MLKHIP_NO_DEVICE : mapBuildError(k.error().code), k.error().message);
    }
    *out = new mlkhip_artifact{std::move(*k)};
    return MLKHIP_OK;
}

int mlkhip_plan(const char* module_json, size_t len, char* class_name, size_t class_cap, char* policy,
                size_t policy_cap, int* n_steps) {
    auto km = mlk::hip::parseKernelModule(module_json, len);
    if (!km.has_value()) return setError(MLKHIP_REFUSED, km.error().message);
    auto plan = mlk::hip::planModule(mlk::hip::deviceModule(*km));
    if (!plan.has_value()) return setError(MLKHIP_REFUSED, plan.error().message);
    copyOut(class_name, class_cap, plan->className);
    copyOut(policy, policy_cap, plan->policy);
    if (n_steps != nullptr) *n_steps = static_cast<int>(plan->steps.size());
    return MLKHIP_OK;
}

long long mlkhip_compile_check(const char* module_json, size_t len, int step, const char* arch,
                               char* source, size_t source_cap) {
    auto km = mlk::hip::parseKernelModule(module_json, len);
    if (!km.has_value()) return setError(-1, km.error().message);
    const mlk::hip::KernelModule dm = mlk::hip::deviceModule(*km);
    auto plan = mlk::hip::planModule(dm);
    if (!plan.has_value()) return setError(-1, plan.error().message);
    if (step < 0 || static_cast<size_t>(step) >= plan->steps.size()) return setError(-1, "step out of range");
    const mlk::hip::Step& st = plan->steps[static_cast<size_t>(step)];
    if (st.kind != mlk::hip::StepKind::Elementwise && st.kind != mlk::hip::StepKind::Nest) return 0;
    const std::string src = st.kind == mlk::hip::StepKind::Nest ? st.source : mlk::hip::elementwiseSource(dm, st);
    copyOut(source, source_cap, src);
    if (arch == nullptr || !mlk::hip::validArch(arch)) return setError(-1, "invalid arch");
    char log[4096] = {0};
    const long long n = mlkd_jit_compile_only(src.data(), src.size(), arch, log, sizeof(log));
    if (n < 0) return setError(-1, log);
    return n;
}

int mlkhip_jit_options(const char* arch, char* buf, size_t cap) { return mlkd_jit_options(arch, buf, cap); }

void mlkhip_release(mlkhip_artifact* a) { delete a; }

int mlkhip_release_stream_scratch(mlkhip_artifact* a, void* stream) {
    if (a == nullptr) return setError(MLKHIP_BAD_BINDING, "null artifact");
    std::string why;
    const int rc = a->k->releaseStreamScratch(stream, why);
    return rc == MLKHIP_OK ? rc : setError(rc, why);
}

int mlkhip_is_multidim(const mlkhip_artifact* a) { return a != nullptr && a->k->plan().multiDim ? 1 : 0; }

const char* mlkhip_class_name(const mlkhip_artifact* a) { return a != nullptr ? a->k->plan().className.c_str() : ""; }

const char* mlkhip_policy(const mlkhip_artifact* a) { return a != nullptr ? a->k->plan().policy.c_str() : ""; }

int mlkhip_num_bindables(const mlkhip_artifact* a) {
    return a != nullptr ? static_cast<int>(a->k->bindables().size()) : 0;
}

int mlkhip_bindable_info(const mlkhip_artifact* a, int i, int32_t* dtype, int64_t* elements, int* is_input,
                         int* is_output, int* is_temp) {
    if (a == nullptr || i < 0 || static_cast<size_t>(i) >= a->k->bindables().size()) return MLKHIP_BAD_BINDING;
    const mlk::hip::KernelBuffer& b = a->k->module().buffers[a->k->bindables()[static_cast<size_t>(i)]];
    if (dtype) *dtype = b.dtype == mlk::hip::Dtype::F32 ? MLKHIP_F32 : (b.dtype == mlk::hip::Dtype::F16 ? MLKHIP_F16 : MLKHIP_F64);
    if (elements) *elements = mlk::hip::bufferElements(b, -1);
    if (is_input) *is_input = b.isInput ? 1 : 0;
    if (is_output) *is_output = b.isOutput ? 1 : 0;
    if (is_temp) *is_temp = b.isTemp ? 1 : 0;
    return MLKHIP_OK;
}

int mlkhip_kernel(const mlkhip_artifact* a, double* const* ptrs, const int64_t* const* dims, int n_bindables,
                  const double* scalars, int64_t n_scalars, int64_t elements) {
    (void)dims;  // logical dims come from the module, as in the reference (the executor trusts the binder)
    if (a == nullptr) return setError(MLKHIP_BAD_BINDING, "null artifact");
    std::string why;
    const int rc = a->k->runHost(ptrs, n_bindables, scalars, n_scalars, elements, why);
    if (rc != MLKHIP_OK) setError(rc, why);
    return rc;
}

int mlkhip_kernel_1d(const mlkhip_artifact* a, double* const* ptrs, int n_ptrs, int64_t n, const double* scalars,
                     int64_t n_scalars) {
    if (a == nullptr) return setError(MLKHIP_BAD_BINDING, "null artifact");
    std::string why;
    const int rc = a->k->runHost(ptrs, n_ptrs, scalars, n_scalars, n, why);
    if (rc != MLKHIP_OK) setError(rc, why);
    return rc;
}

int mlkhip_run_device(const mlkhip_artifact* a, const mlkhip_binding* binds, int n_binds, const double* scalars,
                      int64_t n_scalars, int64_t elements, void* stream) {
    if (a == nullptr) return setError(MLKHIP_BAD_BINDING, "null artifact");
    std::vector<mlk::hip::DeviceBinding> b(static_cast<size_t>(n_binds > 0 ? n_binds : 0));
    for (int i = 0; i < n_binds; ++i) {
        b[static_cast<size_t>(i)].ptr = binds[i].ptr;
        b[static_cast<size_t>(i)].elements = binds[i].elements;
        b[static_cast<size_t>(i)].dtype = binds[i].dtype;
    }
    std::string why;
    const int rc = a->k->runDevice(b.data(), n_binds, scalars, n_scalars, elements, stream, why);
    if (rc != MLKHIP_OK) setError(rc, why);
    return rc;
}

int mlkhip_run_device_noalloc(const mlkhip_artifact* a, const mlkhip_binding* binds, int n_binds,
                              const double* scalars, int64_t n_scalars, int64_t elements, void* stream) {
    if (a == nullptr) return setError(MLKHIP_BAD_BINDING, "null artifact");
    mlk::hip::ScratchArena arena;
    void* base = nullptr;
    if (const int rc = mlkd_rt_noalloc_scratch(&base, &arena.bytes); rc != 0) {
        return setError(rc, "allocation-free scratch is not available on the current device");
    }
    arena.base = static_cast<char*>(base);
    std::vector<mlk::hip::DeviceBinding> b(static_cast<size_t>(n_binds > 0 ? n_binds : 0));
    for (int i = 0; i < n_binds; ++i) {
        b[static_cast<size_t>(i)].ptr = binds[i].ptr;
        b[static_cast<size_t>(i)].elements = binds[i].elements;
        b[static_cast<size_t>(i)].dtype = binds[i].dtype;
    }
    std::string why;
    const int rc = a->k->runDevice(b.data(), n_binds, scalars, n_scalars, elements, stream, why, &arena);
    if (rc != MLKHIP_OK) setError(rc, why);
    return rc;
}

size_t mlkhip_noalloc_scratch_bytes(void) {
    void* base = nullptr;
    size_t bytes = 0;
    return mlkd_rt_noalloc_scratch(&base, &bytes) == 0 ? bytes : 0;
}

int mlkhip_time_device(const mlkhip_artifact* a, const mlkhip_binding* binds, int n_binds, const double* scalars,
                       int64_t n_scalars, int64_t elements, void* stream, int warmup, int reps, float* ms_out) {
    for (int w = 0; w < warmup; ++w) {
        const int rc = mlkhip_run_device(a, binds, n_binds, scalars, n_scalars, elements, stream);
        if (rc != MLKHIP_OK) return rc;
    }
    void* e0 = nullptr;
    void* e1 = nullptr;
    if (mlkd_rt_event_create(&e0) != 0 || mlkd_rt_event_create(&e1) != 0) return setError(MLKHIP_LAUNCH, "event create");
    int rc = MLKHIP_OK;
    for (int r = 0; r < reps && rc == MLKHIP_OK; ++r) {
        mlkd_rt_event_record(e0, stream);
        rc = mlkhip_run_device(a, binds, n_binds, scalars, n_scalars, elements, stream);
        mlkd_rt_event_record(e1, stream);
        float ms = 0.0f;
        if (rc == MLKHIP_OK && mlkd_rt_event_elapsed_ms(e0, e1, &ms) != 0) rc = setError(MLKHIP_LAUNCH, "event timing");
        if (ms_out != nullptr) ms_out[r] = ms;
    }
    mlkd_rt_event_destroy(e0);
    mlkd_rt_event_destroy(e1);
    return rc;
}

int mlkhip_time_device_span(const mlkhip_artifact* a, const mlkhip_binding* binds, int n_binds,
                            const double* scalars, int64_t n_scalars, int64_t elements, void* stream,
                            int warmup, int reps, float* avg_ms) {
    for (int w = 0; w < warmup; ++w) {
        const int rc = mlkhip_run_device(a, binds, n_binds, scalars, n_scalars, elements, stream);
        if (rc != MLKHIP_OK) return rc;
    }
    void* e0 = nullptr;
    void* e1 = nullptr;
    if (mlkd_rt_event_create(&e0) != 0 || mlkd_rt_event_create(&e1) != 0) return setError(MLKHIP_LAUNCH, "event create");
    int rc = mlkd_rt_event_record(e0, stream) == 0 ? MLKHIP_OK : MLKHIP_LAUNCH;
    for (int r = 0; r < reps && rc == MLKHIP_OK; ++r) {
        rc = mlkhip_run_device(a, binds, n_binds, scalars, n_scalars, elements, stream);
    }
    float ms = 0.0f;
    if (rc == MLKHIP_OK && (mlkd_rt_event_record(e1, stream) != 0 || mlkd_rt_event_elapsed_ms(e0, e1, &ms) != 0)) {
        rc = setError(MLKHIP_LAUNCH, "event timing");
    }
    if (avg_ms != nullptr) *avg_ms = reps > 0 ? ms / static_cast<float>(reps) : 0.0f;
    mlkd_rt_event_destroy(e0);
    mlkd_rt_event_destroy(e1);
    return rc;
}

int mlkhip_num_steps(const mlkhip_artifact* a) {
    return a != nullptr ? static_cast<int>(a->k->plan().steps.size()) : 0;
}

namespace {
int listVariants(const mlk::hip::KernelModule& km, const mlk::hip::Plan& plan, int step, int* out, int cap) {
    if (step < 0 || static_cast<size_t>(step) >= plan.steps.size()) return setError(-1, "step out of range");
    const std::vector<int> v = mlk::hip::variantSpace(km, plan.steps[static_cast<size_t>(step)]);
    for (size_t i = 0; i < v.size() && static_cast<int>(i) < cap; ++i) {
        if (out != nullptr) out[i] = v[i];
    }
    return static_cast<int>(v.size());
}
}  // namespace

int mlkhip_step_variants(const mlkhip_artifact* a, int step, int* out, int cap) {
    if (a == nullptr) return setError(-1, "null artifact");
    return listVariants(a->k->module(), a->k->plan(), step, out, cap);
}

int mlkhip_plan_variants(const char* module_json, size_t len, int step, int* out, int cap) {
    auto km = mlk::hip::parseKernelModule(module_json, len);
    if (!km.has_value()) return setError(-1, km.error().message);
    const mlk::hip::KernelModule dm = mlk::hip::deviceModule(*km);
    auto plan = mlk::hip::planModule(dm);
    if (!plan.has_value()) return setError(-1, plan.error().message);
    return listVariants(dm, *plan, step, out, cap);
}

const char* mlkhip_step_kernel_name(const mlkhip_artifact* a, int step) {
    if (a == nullptr || step < 0 || static_cast<size_t>(step) >= a->k->plan().steps.size()) return "";
    return a->k->stepKernelName(static_cast<size_t>(step));
}

int mlkhip_step_variant(const mlkhip_artifact* a, int step) {
    if (a == nullptr || step < 0 || static_cast<size_t>(step) >= a->k->plan().steps.size()) return -2;
    return a->k->plan().steps[static_cast<size_t>(step)].variant;
}

int mlkhip_set_step_variant(mlkhip_artifact* a, int step, int variant) {
    if (a == nullptr) return setError(MLKHIP_BAD_BINDING, "null artifact");
    std::string why;
    const int rc = a->k->setStepVariant(step, variant, why);
    return rc == MLKHIP_OK ? rc : setError(rc, why);
}

const char* mlkhip_fingerprint(const mlkhip_artifact* a) {
    return a != nullptr ? a->k->fingerprint().c_str() : "";
}

int mlkhip_variants_from_cache(const mlkhip_artifact* a) {
    return a != nullptr && a->k->variantsFromCache() ? 1 : 0;
}

int mlkhip_autotune(mlkhip_artifact* a, const mlkhip_binding* binds, int n_binds, const double* scalars,
                    int64_t n_scalars, int64_t elements, int reps, const char* cache_dir, char* report,
                    size_t report_cap) {
    if (a == nullptr) return setError(MLKHIP_BAD_BINDING, "null artifact");
    std::vector<mlk::hip::DeviceBinding> b(static_cast<size_t>(n_binds > 0 ? n_binds : 0));
    for (int i = 0; i < n_binds; ++i) {
        b[static_cast<size_t>(i)].ptr = binds[i].ptr;
        b[static_cast<size_t>(i)].elements = binds[i].elements;
        b[static_cast<size_t>(i)].dtype = binds[i].dtype;
    }
    std::string why, rep;
    const int rc = a->k->autotune(b.data(), n_binds, scalars, n_scalars, elements, reps,
                                  cache_dir != nullptr ? cache_dir : "", rep, why);
    copyOut(report, report_cap, rep);
    return rc == MLKHIP_OK ? rc : setError(rc, why);
}

}  // extern "C"

namespace {
/// Artifacts built by the execute entries, keyed by target and module text:
/// an ExecutionEngine hook calls per graph run and must not rebuild.
struct ExecCache {
    std::mutex lock;
    std::unordered_map<std::string, std::unique_ptr<mlk::hip::HipLoadedKernel>> map;
};

ExecCache& execCache() {
    static ExecCache c;
    return c;
}

int cachedArtifact(const char* module_json, size_t len, const char* arch, mlk::hip::HipLoadedKernel** out) {
    if (module_json == nullptr || arch == nullptr) return setError(MLKHIP_REFUSED, "null argument");
    std::string key = std::string(arch) + '\n';
    key.append(module_json, len);
    ExecCache& c = execCache();
    std::lock_guard<std::mutex> g(c.lock);
    auto it = c.map.find(key);
    if (it == c.map.end()) {
        auto km = mlk::hip::parseKernelModule(module_json, len);
        if (!km.has_value()) return setError(MLKHIP_REFUSED, km.error().message);
        mlk::hip::HipBackendDriverConfig cfg;
        cfg.arch = arch;
        auto k = mlk::hip::buildHipKernelArtifact(*km, cfg);
        if (!k.has_value()) {
            const bool noDevice = k.error().message.find("no HIP device") != std::string::npos;
            return setError(noDevice ? MLKHIP_NO_DEVICE : mapBuildError(k.error().code), k.error().message);
        }
        it = c.map.emplace(std::move(key), std::move(*k)).first;
    }
    *out = it->second.get();
    return MLKHIP_OK;
}
}  // namespace

extern "C" {

int mlkhip_execute_kernel_on_buffers(const char* module_json, size_t len, const char* arch, double* const* inputs,
                                     int n_inputs, double* const* outputs, int n_outputs, const double* scalars,
                                     int64_t n_scalars, int64_t elements) {
    mlk::hip::HipLoadedKernel* k = nullptr;
    if (const int rc = cachedArtifact(module_json, len, arch, &k); rc != MLKHIP_OK) return rc;
    // The reference resolves a buffer id through the table layout (inputs
    // first, then outputs): an input id indexes `inputs`, an output id
    // indexes `outputs` after the input count (kernel_buffers.cpp:200-230).
    // Temps are the artifact's own scratch.
    const mlk::hip::KernelModule& km = k->module();
    std::vector<double*> ptrs;
    for (const uint32_t b : k->bindables()) {
        const mlk::hip::KernelBuffer& kb = km.buffers[b];
        double* p = nullptr;
        if (kb.isTemp) {
            p = nullptr;
        } else if (kb.isInput) {
            if (static_cast<int>(b) >= n_inputs || inputs == nullptr) {
                return setError(MLKHIP_BAD_BINDING, "input buffer " + std::to_string(b) + " is not bound");
            }
            p = inputs[b];
        } else {
            const int o = static_cast<int>(b) - n_inputs;
            if (o < 0 || o >= n_outputs || outputs == nullptr) {
                return setError(MLKHIP_BAD_BINDING, "output buffer " + std::to_string(b) + " is not bound");
            }
            p = outputs[o];
        }
        if (!kb.isTemp && p == nullptr) {
            return setError(MLKHIP_BAD_BINDING, "buffer " + std::to_string(b) + " is bound to NULL");
        }
        ptrs.push_back(p);
    }
    std::string why;
    const int rc = k->runHost(ptrs.data(), static_cast<int>(ptrs.size()), scalars, n_scalars, elements, why);
    return rc == MLKHIP_OK ? rc : setError(rc, why);
}

int mlkhip_execute_kernel(const char* module_json, size_t len, const char* arch, const double* input_scalars,
                          int n_inputs, double* output_scalars, int n_outputs) {
    mlk::hip::HipLoadedKernel* k = nullptr;
    if (const int rc = cachedArtifact(module_json, len, arch, &k); rc != MLKHIP_OK) return rc;
    const mlk::hip::KernelModule& km = k->module();
    std::vector<std::vector<double>> slots;
    for (const mlk::hip::KernelBuffer& kb : km.buffers) {
        if (kb.isInput) {
            return setError(MLKHIP_REFUSED, "tensor kernel requires buffer bindings, not scalar inputs");
        }
        if (kb.isOutput) slots.emplace_back(static_cast<size_t>(kb.elements > 0 ? kb.elements : 1), 0.0);
    }
    if (slots.empty()) return setError(MLKHIP_REFUSED, "kernel module has no output buffer");
    if (n_outputs != static_cast<int>(slots.size()) || output_scalars == nullptr) {
        return setError(MLKHIP_BAD_BINDING, "expected " + std::to_string(slots.size()) + " output slots");
    }
    std::vector<double*> outs;
    for (auto& sl : slots) outs.push_back(sl.data());
    const int rc = mlkhip_execute_kernel_on_buffers(module_json, len, arch, nullptr, 0, outs.data(),
                                                    static_cast<int>(outs.size()), input_scalars, n_inputs, 1);
    if (rc != MLKHIP_OK) return rc;
    for (size_t i = 0; i < slots.size(); ++i) output_scalars[i] = slots[i][0];
    return MLKHIP_OK;
}

int mlkhip_execute_cache_size(void) {
    ExecCache& c = execCache();
    std::lock_guard<std::mutex> g(c.lock);
    return static_cast<int>(c.map.size());
}

void mlkhip_execute_cache_clear(void) {
    ExecCache& c = execCache();
    std::lock_guard<std::mutex> g(c.lock);
    c.map.clear();
}

int mlkhip_essential_work(const char* module_json, size_t len, double bytes_per_sec, double ops_per_sec,
                          int64_t* min_bytes, int64_t* min_ops, int* bytes_known, int* ops_known,
                          double* roofline_lower_sec) {
    if (module_json == nullptr) return setError(MLKHIP_REFUSED, "null argument");
    auto km = mlk::hip::parseKernelModule(module_json, len);
    if (!km.has_value()) return setError(MLKHIP_REFUSED, km.error().message);
    const mlk::hip::EssentialWork w = mlk::hip::essentialWork(*km);
    double tput = ops_per_sec;
    if (tput <= 0.0) {
        auto plan = mlk::hip::planModule(mlk::hip::deviceModule(*km));
        if (!plan.has_value()) return setError(MLKHIP_REFUSED, plan.error().message);
        tput = mlk::hip::peakOpsPerSec(*km, *plan);
    }
    const double bw = bytes_per_sec > 0.0 ? bytes_per_sec : 8.0e12;
    if (min_bytes != nullptr) *min_bytes = w.minBytes;
    if (min_ops != nullptr) *min_ops = w.minOps;
    if (bytes_known != nullptr) *bytes_known = w.bytesKnown ? 1 : 0;
    if (ops_known != nullptr) *ops_known = w.opsKnown ? 1 : 0;
    if (roofline_lower_sec != nullptr) *roofline_lower_sec = mlk::hip::rooflineLowerSec(w, bw, tput);
    return MLKHIP_OK;
}

int mlkhip_measure_environment(double* bytes_per_sec, double* f16_flops_per_sec) {
    if (bytes_per_sec == nullptr || f16_flops_per_sec == nullptr) return setError(MLKHIP_BAD_BINDING, "null argument");
    if (mlkd_rt_device_count() <= 0) return setError(MLKHIP_NO_DEVICE, "no HIP device visible");
    const mlk::hip::MeasuredEnvironment& env = mlk::hip::measuredEnvironment();
    if (!env.ok) return setError(MLKHIP_LAUNCH, "environment probe failed");
    *bytes_per_sec = env.bytesPerSec;
    *f16_flops_per_sec = env.f16FlopsPerSec;
    return MLKHIP_OK;
}

int mlkhip_malloc(void** p, size_t bytes) { return mlkd_rt_malloc(p, bytes); }
int mlkhip_free(void* p) { return mlkd_rt_free(p); }
int mlkhip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    const int rc = mlkd_rt_h2d(dst, src, bytes, nullptr);
    return rc != 0 ? rc : mlkd_rt_sync(nullptr);
}
int mlkhip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    const int rc = mlkd_rt_d2h(dst, src, bytes, nullptr);
    return rc != 0 ? rc : mlkd_rt_sync(nullptr);
}
int mlkhip_fill32(void* p, uint32_t value, size_t bytes) {
    const int rc = mlkd_rt_fill32(p, value, bytes, nullptr);
    return rc != 0 ? rc : mlkd_rt_sync(nullptr);
}
int mlkhip_synchronize(void) { return mlkd_rt_device_sync(); }
int mlkhip_stream_create(void** s) { return mlkd_rt_stream_create(s); }
int mlkhip_stream_destroy(void* s) { return mlkd_rt_stream_destroy(s); }

}  // extern "C"
