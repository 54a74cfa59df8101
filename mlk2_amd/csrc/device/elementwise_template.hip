// Fused elementwise kernel template: the Loop{Compute; Store} class of
// runtime/src/execution/kernel_buffers.cpp:342-402 (1-D) and of the
// poly.synth broadcast nests (compiler/src/passes/poly/poly.synth.cpp:231-353).
//
// The host planner instantiates this template for one KernelModule by
// prepending a prelude that fixes, at compile time, the box extents, every
// stream's dtype and affine coefficients, the output map and accumulate mode,
// and `mlk_chain`, the module's expression chain as straight-line f64 code
// (the reference executor evaluates every chain in f64). The instance is
// compiled in-process with hipRTC for the declared gfx950 target and cached.
// Without a prelude the file compiles standalone with a sample instance (the
// C1 chain), which is how the build checks it.
//
// Mapping: a wave owns a segment of 64*kPer consecutive elements of one
// innermost row of the box; lane l holds the 4-element groups at columns
// seg*64*kPer + g*256 + 4*l (g < kPer/4), so each vector load or store of the
// wave covers one contiguous 256-element span (1 KiB of f32). A stream with
// innermost coefficient 1 is read with one vector access per group when
// aligned (16 B for f32/f64 pairs, 8 B for f16), coefficient 0 is one
// broadcast load per lane, any other coefficient is a gather. The output is
// written the same way. Index arithmetic divides by compile-time extents.
// Compiled with -ffp-contract=off: f64 mul/add round separately, as on the
// reference's x86-64 build; the only fused multiply-adds are the explicit
// ones of the f32 residual polynomial in mlk_p7_sin_f32out.
#ifndef MLK_DEVICE_MATH_H
#include "mlk_device_math.h"
#endif

// Each instance's kernel symbol is mlk_elementwise_<hash of its source>, so
// profiles tell instances apart; the standalone build keeps the plain name.
#ifndef MLK_KERNEL_NAME
#define MLK_KERNEL_NAME mlk_elementwise
#endif

#ifndef MLK_GENERATED
#define MLK_NIN 1
constexpr int kRank = 1;
constexpr bool kDynamicExtent = false;
constexpr long long kExt[4] = {1 << 24, 1, 1, 1};
constexpr int kInDt[MLK_NIN] = {0};
constexpr long long kInOff[MLK_NIN] = {0};
constexpr long long kInC[MLK_NIN][4] = {{1, 0, 0, 0}};
constexpr int kOutDt = 0;
constexpr long long kOutOff = 0;
constexpr long long kOutC[4] = {1, 0, 0, 0};
constexpr int kAccum = 0;
#define MLK_CHAIN_BODY                      \
    const double t0 = in[0] * in[0];        \
    const double t1 = 3.0 * in[0];          \
    const double t2 = t0 + t1;              \
    const double t3 = mlk_p7_sin_f32out(t2); \
    return t3;
#endif

typedef float mlk_f32x4 __attribute__((ext_vector_type(4)));
typedef double mlk_f64x2 __attribute__((ext_vector_type(2)));
typedef _Float16 mlk_f16x4 __attribute__((ext_vector_type(4)));

namespace mlk {

constexpr int kThreads = 256;
constexpr int kPer = 16;

}  // namespace mlk

__device__ __forceinline__ double mlk_chain(const double* in, const mlk_scalars& sc) {
    (void)in;
    (void)sc;
    MLK_CHAIN_BODY
}

namespace mlk {

template <int DT>
constexpr int kBytes = DT == 0 ? 4 : (DT == 1 ? 2 : 8);

/// Alignment (bytes) a 4-element group needs for its vector access.
template <int DT>
constexpr unsigned long long kGroupAlign = DT == 1 ? 8ull : 16ull;

constexpr int kGroups = kPer / 4;  // 4-element groups per lane
constexpr int kSeg = 64 * kPer;    // elements per wave segment of a row

/// Four consecutive elements at flat index i (group-aligned).
template <int DT>
__device__ __forceinline__ void loadGroup(const void* p, long long i, double* v) {
    if constexpr (DT == 0) {
        const mlk_f32x4 f = *reinterpret_cast<const mlk_f32x4*>(static_cast<const float*>(p) + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = static_cast<double>(f[e]);
    } else if constexpr (DT == 1) {
        const mlk_f16x4 h = *reinterpret_cast<const mlk_f16x4*>(static_cast<const _Float16*>(p) + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = static_cast<double>(static_cast<float>(h[e]));
    } else {
        const mlk_f64x2* q = reinterpret_cast<const mlk_f64x2*>(static_cast<const double*>(p) + i);
        const mlk_f64x2 a = q[0];
        const mlk_f64x2 b = q[1];
        v[0] = a[0];
        v[1] = a[1];
        v[2] = b[0];
        v[3] = b[1];
    }
}

template <int DT>
__device__ __forceinline__ void storeGroup(void* p, long long i, const double* v) {
    if constexpr (DT == 0) {
        mlk_f32x4 f;
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = static_cast<float>(v[e]);
        __builtin_nontemporal_store(f, reinterpret_cast<mlk_f32x4*>(static_cast<float*>(p) + i));
    } else if constexpr (DT == 1) {
        mlk_f16x4 h;
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = toHalf(v[e]);
        __builtin_nontemporal_store(h, reinterpret_cast<mlk_f16x4*>(static_cast<_Float16*>(p) + i));
    } else {
        mlk_f64x2* q = reinterpret_cast<mlk_f64x2*>(static_cast<double*>(p) + i);
        mlk_f64x2 a, b;
        a[0] = v[0];
        a[1] = v[1];
        b[0] = v[2];
        b[1] = v[3];
        __builtin_nontemporal_store(a, q);
        __builtin_nontemporal_store(b, q + 1);
    }
}

constexpr long long outerRows() {
    long long r = 1;
    for (int d = 0; d < kRank - 1; ++d) r *= kExt[d];
    return r;
}

/// Element g*4+e of a lane sits at column lane0 + g*256 + e, lane0 =
/// seg*kSeg + 4*lane: each vector instruction of a wave covers one
/// contiguous 64x4-element span.
template <int K>
__device__ __forceinline__ void loadStream(const void* p, const long long (&var)[4], long long lane0,
                                           bool full, long long W, double (&v)[kPer]) {
    constexpr int DT = kInDt[K];
    long long base = kInOff[K];
#pragma unroll
    for (int d = 0; d < kRank - 1; ++d) base += kInC[K][d] * var[d];
    constexpr long long ci = kInC[K][kRank - 1];
    if constexpr (ci == 0) {
        const double x = loadOne<DT>(p, base);
#pragma unroll
        for (int e = 0; e < kPer; ++e) v[e] = x;
    } else {
        const bool vec = ci == 1 && full &&
                         ((reinterpret_cast<unsigned long long>(p) + (base + lane0) * kBytes<DT>) &
                          (kGroupAlign<DT> - 1)) == 0;
        if (vec) {
#pragma unroll
            for (int g = 0; g < kGroups; ++g) loadGroup<DT>(p, base + lane0 + g * 256, &v[4 * g]);
        } else {
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const long long col = lane0 + g * 256 + e;
                    v[4 * g + e] = col < W ? loadOne<DT>(p, base + ci * col) : 0.0;
                }
            }
        }
    }
}

template <int K>
__device__ __forceinline__ void loadAll(const void* const (&ptr)[4], const long long (&var)[4],
                                        long long lane0, bool full, long long W,
                                        double (&in)[MLK_NIN][kPer]) {
    if constexpr (K < MLK_NIN) {
        loadStream<K>(ptr[K], var, lane0, full, W, in[K]);
        loadAll<K + 1>(ptr, var, lane0, full, W, in);
    }
}

}  // namespace mlk

extern "C" __global__ __launch_bounds__(256) void MLK_KERNEL_NAME(const void* p0, const void* p1,
                                                                  const void* p2, const void* p3,
                                                                  void* out, const mlk_scalars sc,
                                                                  long long dynExtent) {
    using namespace mlk;
    // The 1-D dynamic form (loop end = the run's element count) takes its
    // extent at launch; every other extent is a compile-time constant.
    const long long W = kDynamicExtent ? dynExtent : kExt[kRank - 1];
    const long long segsPerRow = (W + kSeg - 1) / kSeg;
    constexpr long long rows = outerRows();
    const long long total = rows * segsPerRow;
    const void* const ptr[4] = {p0, p1, p2, p3};
    const int lane = threadIdx.x & 63;
    const long long waves = static_cast<long long>(gridDim.x) * (kThreads / 64);
    for (long long w = static_cast<long long>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
         w < total; w += waves) {
        const long long row = w / segsPerRow;
        const long long seg = w - row * segsPerRow;
        const long long lane0 = seg * kSeg + 4 * lane;
        const bool full = (seg + 1) * kSeg <= W;
        long long var[4] = {0, 0, 0, 0};
        {
            long long rem = row;
#pragma unroll
            for (int d = kRank - 2; d >= 0; --d) {
                var[d] = rem % kExt[d];
                rem /= kExt[d];
            }
        }
        double in[MLK_NIN][kPer];
        loadAll<0>(ptr, var, lane0, full, W, in);
        double res[kPer];
#pragma unroll
        for (int e = 0; e < kPer; ++e) {
            double x[MLK_NIN];
#pragma unroll
            for (int k = 0; k < MLK_NIN; ++k) x[k] = in[k][e];
            res[e] = mlk_chain(x, sc);
        }
        long long obase = kOutOff;
#pragma unroll
        for (int d = 0; d < kRank - 1; ++d) obase += kOutC[d] * var[d];
        constexpr long long oc = kOutC[kRank - 1];
        if constexpr (kAccum != 0) {
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const long long col = lane0 + g * 256 + e;
                    if (col < W) {
                        const long long at = obase + oc * col;
                        const double old = loadOne<kOutDt>(out, at);
                        const double r = res[4 * g + e];
                        storeOne<kOutDt>(out, at, kAccum == 1 ? old + r : ((r > old) ? r : old));
                    }
                }
            }
        } else {
            const bool vec = oc == 1 && full &&
                             ((reinterpret_cast<unsigned long long>(out) + (obase + lane0) * kBytes<kOutDt>) &
                              (kGroupAlign<kOutDt> - 1)) == 0;
            if (vec) {
#pragma unroll
                for (int g = 0; g < kGroups; ++g) storeGroup<kOutDt>(out, obase + lane0 + g * 256, &res[4 * g]);
            } else {
#pragma unroll
                for (int g = 0; g < kGroups; ++g) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const long long col = lane0 + g * 256 + e;
                        if (col < W) storeOne<kOutDt>(out, obase + oc * col, res[4 * g + e]);
                    }
                }
            }
        }
    }
}
