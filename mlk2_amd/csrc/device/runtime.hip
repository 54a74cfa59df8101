// Thin C ABI over the HIP runtime. The C++ host planner/driver calls HIP only
// through these functions (no HIP headers in host code). Status codes follow
// the artifact ABI of docs/kernel_abi.md:25-40: 0 ok, 2 runtime alloc/copy,
// 3 launch/sync, 4 no device.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <string.h>

#include <mutex>

#include "runtime_abi.h"

namespace {

/// Device scratch of the allocation-free entry (mlkhip_run_device_noalloc):
/// one file-scope array that each GPU the library runs on holds until the
/// process ends. Host code never uses the name as an address: it takes the
/// address hipGetSymbolAddress reports for the current device.
constexpr size_t kNoAllocScratchBytes = size_t{32} << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex gScratchLock;
void* gScratchPtr[kMaxDevices] = {};

int mapErr(hipError_t e, int code) { return e == hipSuccess ? 0 : code; }

__global__ void fillKernel(uint32_t* p, uint32_t v, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        p[i] = v;
    }
}

}  // namespace

extern "C" {

int mlkd_rt_noalloc_scratch(void** ptr, size_t* bytes) {
    *ptr = nullptr;
    *bytes = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MLKD_RT_NO_DEVICE;
    std::lock_guard<std::mutex> g(gScratchLock);
    if (gScratchPtr[dev] == nullptr) {
        // Once per device, with that device current: this device's copy of
        // the array.
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return MLKD_RT_LAUNCH;
        gScratchPtr[dev] = p;
    }
    *ptr = gScratchPtr[dev];
    *bytes = kNoAllocScratchBytes;
    return 0;
}

int mlkd_rt_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int mlkd_rt_device_arch(int dev, char* buf, size_t cap) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return MLKD_RT_NO_DEVICE;
    if (buf != nullptr && cap > 0) {
        strncpy(buf, prop.gcnArchName, cap - 1);
        buf[cap - 1] = '\0';
    }
    return 0;
}

int mlkd_rt_device_info(int dev, int* cu_count, int64_t* max_grid_x, int* max_block,
                        int64_t* global_mem) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return MLKD_RT_NO_DEVICE;
    if (cu_count) *cu_count = prop.multiProcessorCount;
    if (max_grid_x) *max_grid_x = prop.maxGridSize[0];
    if (max_block) *max_block = prop.maxThreadsPerBlock;
    if (global_mem) *global_mem = (int64_t)prop.totalGlobalMem;
    return 0;
}

int mlkd_rt_malloc(void** p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) bytes = 256;
    return mapErr(hipMalloc(p, bytes), MLKD_RT_ALLOC);
}

int mlkd_rt_free(void* p) {
    if (p == nullptr) return 0;
    return mapErr(hipFree(p), MLKD_RT_ALLOC);
}

int mlkd_rt_host_alloc(void** p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) bytes = 256;
    return mapErr(hipHostMalloc(p, bytes, hipHostMallocDefault), MLKD_RT_ALLOC);
}

int mlkd_rt_host_free(void* p) {
    if (p == nullptr) return 0;
    return mapErr(hipHostFree(p), MLKD_RT_ALLOC);
}

int mlkd_rt_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return 0;
    return mapErr(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice,
                                 static_cast<hipStream_t>(stream)),
                  MLKD_RT_ALLOC);
}

int mlkd_rt_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return 0;
    return mapErr(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost,
                                 static_cast<hipStream_t>(stream)),
                  MLKD_RT_ALLOC);
}

int mlkd_rt_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return 0;
    return mapErr(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice,
                                 static_cast<hipStream_t>(stream)),
                  MLKD_RT_ALLOC);
}

/// Fills `bytes` (a multiple of 4) with a 32-bit pattern using a kernel, so
/// that the call is safe inside stream capture (no memset nodes).
int mlkd_rt_fill32(void* p, uint32_t value, size_t bytes, void* stream) {
    if (bytes == 0) return 0;
    if ((bytes & 3u) != 0) return MLKD_RT_LAUNCH;
    const int64_t n = static_cast<int64_t>(bytes / 4);
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fillKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<uint32_t*>(p), value, n);
    return mapErr(hipGetLastError(), MLKD_RT_LAUNCH);
}

int mlkd_rt_sync(void* stream) {
    return mapErr(hipStreamSynchronize(static_cast<hipStream_t>(stream)), MLKD_RT_LAUNCH);
}

int mlkd_rt_device_sync(void) { return mapErr(hipDeviceSynchronize(), MLKD_RT_LAUNCH); }

int mlkd_rt_stream_create(void** s) {
    hipStream_t st = nullptr;
    const int rc = mapErr(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), MLKD_RT_LAUNCH);
    *s = st;
    return rc;
}

int mlkd_rt_stream_destroy(void* s) {
    if (s == nullptr) return 0;
    return mapErr(hipStreamDestroy(static_cast<hipStream_t>(s)), MLKD_RT_LAUNCH);
}

int mlkd_rt_event_create(void** e) {
    hipEvent_t ev = nullptr;
    const int rc = mapErr(hipEventCreate(&ev), MLKD_RT_LAUNCH);
    *e = ev;
    return rc;
}

int mlkd_rt_event_destroy(void* e) {
    if (e == nullptr) return 0;
    return mapErr(hipEventDestroy(static_cast<hipEvent_t>(e)), MLKD_RT_LAUNCH);
}

int mlkd_rt_event_record(void* e, void* stream) {
    return mapErr(hipEventRecord(static_cast<hipEvent_t>(e), static_cast<hipStream_t>(stream)),
                  MLKD_RT_LAUNCH);
}

int mlkd_rt_event_sync(void* e) {
    return mapErr(hipEventSynchronize(static_cast<hipEvent_t>(e)), MLKD_RT_LAUNCH);
}

int mlkd_rt_event_elapsed_ms(void* start, void* stop, float* ms) {
    if (hipEventSynchronize(static_cast<hipEvent_t>(stop)) != hipSuccess) return MLKD_RT_LAUNCH;
    return mapErr(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                      static_cast<hipEvent_t>(stop)),
                  MLKD_RT_LAUNCH);
}

const char* mlkd_rt_last_error(void) { return hipGetErrorString(hipGetLastError()); }

}  // extern "C"
