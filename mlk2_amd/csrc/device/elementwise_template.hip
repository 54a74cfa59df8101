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
// broadcast load per lane, any other coefficient is a gather. Loaded values
// stay in their buffer's dtype until the chain reads them (an f32 stream
// holds one register per element, not two). The output is written the same
// way. Index arithmetic divides by compile-time extents. One segment per
// wave: the grid covers the box once.
//
// A chain may use forms that decline some arguments (mlk_p7_sin_f32out,
// mlk_exp_f32acc add the lane to the wave mask `slow`). A wave with a declined element in any lane then
// recomputes its whole segment, after the vector stores, with
// MLK_CHAIN_EXACT (the chain in the reference's f64 forms): each lane
// re-reads its inputs element by element and stores each result over the
// fast one (same lane, same address: program order). The exact pass is one
// rolled loop, out of the unrolled hot path.
//
// Compiled with -ffp-contract=off: f64 mul/add round separately, as on the
// reference's x86-64 build. The fused multiply-adds are explicit: the f32
// residual polynomial of mlk_p7_sin_f32out, and chain sums of a product whose
// operands make it exact in f64 (one rounding either way).
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
#define MLK_CHAIN_BODY                             \
    const double t1 = 3.0 * in[0];                 \
    const double t2 = __builtin_fma(in[0], in[0], t1); \
    const double t3 = mlk_p7_sin_f32out(t2, slow); \
    return t3;
#define MLK_CHAIN_EXACT                            \
    const double t0 = in[0] * in[0];               \
    const double t1 = 3.0 * in[0];                 \
    const double t2 = t0 + t1;                     \
    const double t3 = mlk_p7_sin(t2);              \
    return t3;
#endif

typedef float mlk_f32x4 __attribute__((ext_vector_type(4)));
typedef double mlk_f64x2 __attribute__((ext_vector_type(2)));
typedef _Float16 mlk_f16x4 __attribute__((ext_vector_type(4)));

namespace mlk {

constexpr int kThreads = 256;
constexpr int kPer = 8;

}  // namespace mlk

__device__ __forceinline__ double mlk_chain(const double* in, const mlk_scalars& sc, unsigned long long& slow) {
    (void)in;
    (void)sc;
    (void)slow;
    MLK_CHAIN_BODY
}

#ifdef MLK_CHAIN_EXACT
__device__ __forceinline__ double mlk_chain_exact(const double* in, const mlk_scalars& sc) {
    (void)in;
    (void)sc;
    MLK_CHAIN_EXACT
}
#endif

namespace mlk {

template <int DT>
constexpr int kBytes = DT == 0 ? 4 : (DT == 1 ? 2 : 8);

/// Alignment (bytes) a 4-element group needs for its vector access.
template <int DT>
constexpr unsigned long long kGroupAlign = DT == 1 ? 8ull : 16ull;

constexpr int kGroups = kPer / 4;  // 4-element groups per lane
constexpr int kSeg = 64 * kPer;    // elements per wave segment of a row
#ifdef MLK_GENERATED
static_assert(kSeg == kHostSegment, "the host sizes the grid by this segment");
#endif

template <int DT>
struct RawOf {
    using T = double;
};
template <>
struct RawOf<0> {
    using T = float;
};
template <>
struct RawOf<1> {
    using T = _Float16;
};

/// One lane's loaded elements of streams K.. in their buffers' dtypes.
template <int K, bool End = (K >= MLK_NIN)>
struct Frame {
    typename RawOf<kInDt[K]>::T v[kPer];
    Frame<K + 1> next;
};
template <int K>
struct Frame<K, true> {};

template <int K, int J>
__device__ __forceinline__ auto& streamOf(Frame<J>& f) {
    if constexpr (K == J) return f.v;
    else return streamOf<K, J + 1>(f.next);
}

/// Four consecutive elements at flat index i (group-aligned).
template <int DT>
__device__ __forceinline__ void loadGroup(const void* p, long long i, typename RawOf<DT>::T* v) {
    if constexpr (DT == 0) {
        const mlk_f32x4 f = *reinterpret_cast<const mlk_f32x4*>(static_cast<const float*>(p) + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = f[e];
    } else if constexpr (DT == 1) {
        const mlk_f16x4 h = *reinterpret_cast<const mlk_f16x4*>(static_cast<const _Float16*>(p) + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = h[e];
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
__device__ __forceinline__ typename RawOf<DT>::T loadRaw(const void* p, long long i) {
    return static_cast<const typename RawOf<DT>::T*>(p)[i];
}

/// f64 -> the buffer dtype (f32 RNE; f16 with one rounding; f64 as is).
template <int DT>
__device__ __forceinline__ typename RawOf<DT>::T narrow(double v) {
    if constexpr (DT == 0) return static_cast<float>(v);
    else if constexpr (DT == 1) return toHalf(v);
    else return v;
}

template <int DT>
__device__ __forceinline__ void storeGroup(void* p, long long i, const typename RawOf<DT>::T* v) {
    if constexpr (DT == 0) {
        mlk_f32x4 f;
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = v[e];
        __builtin_nontemporal_store(f, reinterpret_cast<mlk_f32x4*>(static_cast<float*>(p) + i));
    } else if constexpr (DT == 1) {
        mlk_f16x4 h;
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = v[e];
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

template <int K>
__device__ __forceinline__ long long streamBase(const long long (&var)[4]) {
    long long base = kInOff[K];
#pragma unroll
    for (int d = 0; d < kRank - 1; ++d) base += kInC[K][d] * var[d];
    return base;
}

/// Element g*4+e of a lane sits at column lane0 + g*256 + e, lane0 =
/// seg*kSeg + 4*lane: each vector instruction of a wave covers one
/// contiguous 64x4-element span.
template <int K>
__device__ __forceinline__ void loadStream(const void* p, const long long (&var)[4], long long lane0,
                                           bool full, long long W, typename RawOf<kInDt[K]>::T (&v)[kPer]) {
    constexpr int DT = kInDt[K];
    using T = typename RawOf<DT>::T;
    const long long base = streamBase<K>(var);
    constexpr long long ci = kInC[K][kRank - 1];
    if constexpr (ci == 0) {
        const T x = loadRaw<DT>(p, base);
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
                    v[4 * g + e] = col < W ? loadRaw<DT>(p, base + ci * col) : T(0);
                }
            }
        }
    }
}

template <int K>
__device__ __forceinline__ void loadAll(const void* const (&ptr)[4], const long long (&var)[4], long long lane0,
                                        bool full, long long W, Frame<0>& fr) {
    if constexpr (K < MLK_NIN) {
        loadStream<K>(ptr[K], var, lane0, full, W, streamOf<K, 0>(fr));
        loadAll<K + 1>(ptr, var, lane0, full, W, fr);
    }
}

/// Element e of every stream, widened to f64 (exact for all three dtypes).
template <int K>
__device__ __forceinline__ void widen(Frame<0>& fr, int e, double (&x)[MLK_NIN]) {
    if constexpr (K < MLK_NIN) {
        if constexpr (kInDt[K] == 2) x[K] = streamOf<K, 0>(fr)[e];
        else x[K] = static_cast<double>(static_cast<float>(streamOf<K, 0>(fr)[e]));
        widen<K + 1>(fr, e, x);
    }
}

#ifdef MLK_CHAIN_EXACT
/// Element `col` of every stream, re-read one by one (the exact pass).
template <int K>
__device__ __forceinline__ void reloadElem(const void* const (&ptr)[4], const long long (&var)[4], long long col,
                                           double (&x)[MLK_NIN]) {
    if constexpr (K < MLK_NIN) {
        x[K] = loadOne<kInDt[K]>(ptr[K], streamBase<K>(var) + kInC[K][kRank - 1] * col);
        reloadElem<K + 1>(ptr, var, col, x);
    }
}
#endif

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
        Frame<0> fr;
        loadAll<0>(ptr, var, lane0, full, W, fr);
        long long obase = kOutOff;
#pragma unroll
        for (int d = 0; d < kRank - 1; ++d) obase += kOutC[d] * var[d];
        constexpr long long oc = kOutC[kRank - 1];
        const bool vecOut = oc == 1 && full &&
                            ((reinterpret_cast<unsigned long long>(out) + (obase + lane0) * kBytes<kOutDt>) &
                             (kGroupAlign<kOutDt> - 1)) == 0;
        // Plain stores take each result in the output dtype as soon as it is
        // computed (the empty asm statements pin that point, so the compiler
        // cannot defer the tail of every element's chain to the stores and
        // hold all their intermediates at once), and each 4-element group is
        // stored as soon as it is complete, so writes start while the rest of
        // the segment computes. Accumulating stores keep f64 and go last.
        typename RawOf<kOutDt>::T res[kPer];
        double acc[kPer];
        unsigned long long slowWave = 0;  // lanes with a declined element
#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
#pragma unroll
            for (int e = 4 * g; e < 4 * g + 4; ++e) {
                double x[MLK_NIN];
                widen<0>(fr, e, x);
                const double v = mlk_chain(x, sc, slowWave);
                if constexpr (kAccum == 0) {
                    res[e] = narrow<kOutDt>(v);
                    asm volatile("" : "+v"(res[e]));
                } else {
                    acc[e] = v;
                }
#ifdef MLK_CHAIN_EXACT
                asm volatile("" : "+s"(slowWave));
#endif
            }
            if constexpr (kAccum == 0) {
                if (vecOut) {
                    storeGroup<kOutDt>(out, obase + lane0 + g * 256, &res[4 * g]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const long long col = lane0 + g * 256 + e;
                        if (col < W) {
                            static_cast<typename RawOf<kOutDt>::T*>(out)[obase + oc * col] = res[4 * g + e];
                        }
                    }
                }
            }
        }
        if constexpr (kAccum != 0) {
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const long long col = lane0 + g * 256 + e;
                    if (col < W) {
                        const long long at = obase + oc * col;
                        const double old = loadOne<kOutDt>(out, at);
                        const double r = acc[4 * g + e];
                        storeOne<kOutDt>(out, at, kAccum == 1 ? old + r : ((r > old) ? r : old));
                    }
                }
            }
        }
#ifdef MLK_CHAIN_EXACT
        static_assert(kAccum == 0, "fast chain forms are planned for plain stores only");
        if (slowWave != 0) {  // wave-uniform: every lane redoes its segment exactly
#pragma unroll 1
            for (int e = 0; e < kPer; ++e) {
                const long long col = lane0 + (e >> 2) * 256 + (e & 3);
                if (col < W) {
                    double x[MLK_NIN];
                    reloadElem<0>(ptr, var, col, x);
                    storeOne<kOutDt>(out, obase + oc * col, mlk_chain_exact(x, sc));
                }
            }
        }
#endif
    }
}
