// Environment probe of the device: the measured counterpart of the
// reference's measureEnvironment (fastkernel/src/fast_kernel.cpp:319-335),
// which probes CPU bandwidth and scalar throughput. Here: HBM bandwidth from
// a streaming copy of irregular data (4 workgroups per CU, grid-stride,
// 16-byte nontemporal stores: the fastest copy shape measured on gfx950),
// and v_mfma_f32_32x32x16_f16 throughput from independent register-only
// MFMAs. Both are timed with HIP events on the given stream.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "runtime_abi.h"

namespace {

typedef float f32x4p __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8p __attribute__((ext_vector_type(8)));
typedef float f32x16p __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void probeCopy(const f32x4p* __restrict__ x, f32x4p* __restrict__ y, int64_t n4) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n4; i += stride) {
        __builtin_nontemporal_store(x[i], y + i);
    }
}

__global__ __launch_bounds__(256) void probeFill(f32x4p* __restrict__ x, int64_t n4) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n4; i += stride) {
        uint32_t h = static_cast<uint32_t>(i) * 2654435761u;
        f32x4p v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            h ^= h >> 13;
            h *= 0x5bd1e995u;
            v[e] = static_cast<float>(h >> 8) * (1.0f / 16777216.0f) - 0.5f;
        }
        x[i] = v;
    }
}

/// Each wave issues `iters` rounds of 16 independent MFMAs on register
/// operands; the sum goes to memory so nothing is eliminated.
__global__ __launch_bounds__(256) void probeMfma(float* __restrict__ out, int iters, float seed) {
    f16x8p a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = static_cast<_Float16>(seed * static_cast<float>((threadIdx.x + e) % 7));
        b[e] = static_cast<_Float16>(seed * static_cast<float>((threadIdx.x * 3 + e) % 5));
    }
    f32x16p acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[i], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[i][r];
    }
    out[static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x] = s;
}

}  // namespace

extern "C" int mlkd_probe_environment(double* bytes_per_sec, double* f16_flops_per_sec, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
        return MLKD_RT_LAUNCH;
    }
    constexpr int64_t kBytes = int64_t{1} << 28;   // 256 MiB each way: far beyond every cache
    void* x = nullptr;
    void* y = nullptr;
    float* out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = MLKD_RT_LAUNCH;
    const unsigned mfmaBlocks = static_cast<unsigned>(cus);   // one wave per SIMD
    constexpr int kIters = 2000;
    do {
        if (hipMalloc(&x, kBytes) != hipSuccess || hipMalloc(&y, kBytes) != hipSuccess ||
            hipMalloc(&out, static_cast<size_t>(mfmaBlocks) * 256 * sizeof(float)) != hipSuccess ||
            hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
            break;
        }
        const int64_t n4 = kBytes / 16;
        const unsigned copyBlocks = static_cast<unsigned>(cus) * 4;
        // Irregular contents: the memory system moves all-zero data faster
        // than real data, which would overstate the bandwidth.
        hipLaunchKernelGGL(probeFill, dim3(copyBlocks), dim3(256), 0, st, static_cast<f32x4p*>(x), n4);
        hipLaunchKernelGGL(probeCopy, dim3(copyBlocks), dim3(256), 0, st, static_cast<const f32x4p*>(x),
                           static_cast<f32x4p*>(y), n4);   // warm-up
        if (hipGetLastError() != hipSuccess) break;
        constexpr int kReps = 5;
        if (hipEventRecord(e0, st) != hipSuccess) break;
        for (int r = 0; r < kReps; ++r) {
            hipLaunchKernelGGL(probeCopy, dim3(copyBlocks), dim3(256), 0, st, static_cast<const f32x4p*>(x),
                               static_cast<f32x4p*>(y), n4);
        }
        if (hipGetLastError() != hipSuccess || hipEventRecord(e1, st) != hipSuccess) break;
        float ms = 0.0f;
        if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess || ms <= 0.0f) break;
        const double bytesPerSec = 2.0 * static_cast<double>(kBytes) * kReps / (1e-3 * ms);
        hipLaunchKernelGGL(probeMfma, dim3(mfmaBlocks), dim3(256), 0, st, out, 10, 0.01f);
        if (hipGetLastError() != hipSuccess || hipEventRecord(e0, st) != hipSuccess) break;
        hipLaunchKernelGGL(probeMfma, dim3(mfmaBlocks), dim3(256), 0, st, out, kIters, 0.01f);
        if (hipGetLastError() != hipSuccess || hipEventRecord(e1, st) != hipSuccess) break;
        if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess || ms <= 0.0f) break;
        const double flops = static_cast<double>(mfmaBlocks) * 4 * kIters * 16 * (2.0 * 32 * 32 * 16);
        *bytes_per_sec = bytesPerSec;
        *f16_flops_per_sec = flops / (1e-3 * ms);
        rc = 0;
    } while (false);
    // Best-effort release: a failure here leaves nothing further to undo.
    if (e0 != nullptr) (void)hipEventDestroy(e0);
    if (e1 != nullptr) (void)hipEventDestroy(e1);
    if (out != nullptr) (void)hipFree(out);
    if (y != nullptr) (void)hipFree(y);
    if (x != nullptr) (void)hipFree(x);
    return rc;
}
