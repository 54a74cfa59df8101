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

/// Operands for the rate probe: hashed per lane into [-1, 1) when RANDOM
/// (the GEMM benches' data), else all ones. The chip draws more power on
/// random operands, so the two rates bracket what a real GEMM can reach.
template <bool RANDOM>
__device__ __forceinline__ f16x8p probeOperand(uint32_t& h) {
    f16x8p v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        if (RANDOM) {
            h ^= h >> 13;
            h *= 0x5bd1e995u;
            h ^= h >> 15;
            v[e] = static_cast<_Float16>(static_cast<float>(h >> 8) * (1.0f / 8388608.0f) - 1.0f);
        } else {
            v[e] = static_cast<_Float16>(1.0f);
        }
    }
    return v;
}

typedef float f32x4q __attribute__((ext_vector_type(4)));

/// Register-only MFMA loop: every wave owns TM x TN independent accumulator
/// tiles and issues them back to back `iters` times. SHAPE 0:
/// v_mfma_f32_16x16x32_f16 (TM x TN = 8 x 8 at one wave per SIMD, 8 x 4 at
/// two); SHAPE 1: v_mfma_f32_32x32x16_f16 (4 x 4, or 4 x 2). At one wave per
/// SIMD the accumulators fill 256 registers, at two 128, as in the GEMM forms.
template <int SHAPE, bool RANDOM, int WPS>
__global__ __launch_bounds__(256 * WPS) void probeMfmaRate(float* __restrict__ out, int iters) {
    constexpr int TM = SHAPE == 0 ? 8 : 4;
    constexpr int TN = (SHAPE == 0 ? 8 : 4) / WPS;
    uint32_t h = (blockIdx.x * 256u * WPS + threadIdx.x) * 2654435761u + 1u;
    f16x8p a[TM], b[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) a[i] = probeOperand<RANDOM>(h);
#pragma unroll
    for (int j = 0; j < TN; ++j) b[j] = probeOperand<RANDOM>(h);
    float s = 0.0f;
    if constexpr (SHAPE == 0) {
        f32x4q acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = f32x4q{0.0f, 0.0f, 0.0f, 0.0f};
        }
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int i = 0; i < TM; ++i) {
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j) s += acc[i][j][0] + acc[i][j][1] + acc[i][j][2] + acc[i][j][3];
        }
    } else {
        f32x16p acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
            }
        }
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int i = 0; i < TM; ++i) {
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
#pragma unroll
                for (int r = 0; r < 16; ++r) s += acc[i][j][r];
            }
        }
    }
    out[static_cast<int64_t>(blockIdx.x) * 256 * WPS + threadIdx.x] = s;
}

template <int SHAPE, bool RANDOM, int WPS>
void launchRate(unsigned blocks, hipStream_t st, float* out, int iters) {
    hipLaunchKernelGGL((probeMfmaRate<SHAPE, RANDOM, WPS>), dim3(blocks), dim3(256 * WPS), 0, st, out, iters);
}

}  // namespace

/// Sustained f16 MFMA rate of register-only loops (no memory traffic inside
/// the loop): shape 0 = 16x16x32, 1 = 32x32x16; `random` selects hashed
/// operands over all-ones; `waves_per_simd` 1 or 2. One workgroup per CU.
/// Launches back to back for about `settle_ms` first, so the rate is the
/// chip's settled one under its power limit, then times `reps` launches.
extern "C" int mlkd_probe_mfma_rate(int shape, int random, int waves_per_simd, double settle_ms, int reps,
                                    double* flops_per_sec, void* stream) {
    if ((shape != 0 && shape != 1) || (waves_per_simd != 1 && waves_per_simd != 2) || reps < 1 ||
        flops_per_sec == nullptr) {
        return MLKD_RT_LAUNCH;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
        return MLKD_RT_LAUNCH;
    }
    const unsigned blocks = static_cast<unsigned>(cus);
    float* out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = MLKD_RT_LAUNCH;
    auto launch = [&](int iters) {
        const int k = shape * 4 + (random ? 2 : 0) + (waves_per_simd - 1);
        switch (k) {
            case 0: launchRate<0, false, 1>(blocks, st, out, iters); break;
            case 1: launchRate<0, false, 2>(blocks, st, out, iters); break;
            case 2: launchRate<0, true, 1>(blocks, st, out, iters); break;
            case 3: launchRate<0, true, 2>(blocks, st, out, iters); break;
            case 4: launchRate<1, false, 1>(blocks, st, out, iters); break;
            case 5: launchRate<1, false, 2>(blocks, st, out, iters); break;
            case 6: launchRate<1, true, 1>(blocks, st, out, iters); break;
            default: launchRate<1, true, 2>(blocks, st, out, iters); break;
        }
    };
    // Per SIMD and iteration: 64 tiles of 16x16x32 (2^20 flop) or 16 of
    // 32x32x16 (2^19 flop).
    const double flopsPerIter = static_cast<double>(blocks) * 4 * (shape == 0 ? 1048576.0 : 524288.0);
    constexpr int kIters = 4000;
    do {
        if (hipMalloc(&out, static_cast<size_t>(blocks) * 512 * sizeof(float)) != hipSuccess ||
            hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
            break;
        }
        launch(16);
        if (hipGetLastError() != hipSuccess || hipEventRecord(e0, st) != hipSuccess) break;
        launch(kIters);
        if (hipGetLastError() != hipSuccess || hipEventRecord(e1, st) != hipSuccess) break;
        float ms = 0.0f;
        if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess || ms <= 0.0f) break;
        const int settle = static_cast<int>(settle_ms / ms) + 1;
        bool ok = true;
        for (int r = 0; r < settle && ok; ++r) {
            launch(kIters);
            ok = hipGetLastError() == hipSuccess;
        }
        if (!ok || hipEventRecord(e0, st) != hipSuccess) break;
        for (int r = 0; r < reps && ok; ++r) {
            launch(kIters);
            ok = hipGetLastError() == hipSuccess;
        }
        if (!ok || hipEventRecord(e1, st) != hipSuccess) break;
        if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess || ms <= 0.0f) break;
        *flops_per_sec = flopsPerIter * kIters * reps / (1e-3 * ms);
        rc = 0;
    } while (false);
    if (e0 != nullptr) (void)hipEventDestroy(e0);
    if (e1 != nullptr) (void)hipEventDestroy(e1);
    if (out != nullptr) (void)hipFree(out);
    return rc;
}

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
