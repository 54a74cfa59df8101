// Device math shared by every hipRTC instance (the elementwise template and
// the generic loop-nest kernels): the poly7 sine of
// compiler/include/mlk/support/math_families.h:22-90 in its exact f64 form
// and its split-precision form, the scalar-parameter block, and one-element
// loads and stores of the three buffer dtypes with the rounding the artifact
// ABI promises (f64 -> f32 RNE, f64 -> f16 with a single rounding). The
// static kernels' f64 paths (general softmax, general GEMM, unfused score)
// include it for that f16 store. Instances are compiled with
// -ffp-contract=off.
#ifndef MLK_DEVICE_MATH_H
#define MLK_DEVICE_MATH_H

#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#endif

namespace mlk {

// math_families.h:22-65: Cody-Waite split of pi/2 and the residual polynomials.
constexpr double kPiHalf = 1.57079632679489661923;
constexpr double kTwoOverPi = 0.63661977236758134308;
constexpr double kPio2Hi = 1.5707963267948965580e+00;
constexpr double kPio2Lo = 6.1232339957367660359e-17;
constexpr double kS[6] = {1.58962301576546568060e-10, -2.50507477628578072866e-8,
                          2.75573136213857245213e-6, -1.98412698295895385996e-4,
                          8.33333333332211858878e-3, -1.66666666666666307295e-1};
constexpr double kC[6] = {-1.13585365213876817300e-11, 2.08757530072652689750e-9,
                          -2.75573142103085808917e-7, 2.48015872890001867312e-5,
                          -1.38888888888783992457e-3, 4.16666666666666435770e-2};

__device__ __forceinline__ int quadrantOf(double n) {
    if (__builtin_fabs(n) < 4503599627370496.0) {  // |n| < 2^52: exact in int64
        return static_cast<int>(static_cast<long long>(n) & 3LL);
    }
    int q = static_cast<int>(fmod(n, 4.0));
    return q < 0 ? q + 4 : q;
}

}  // namespace mlk

/// poly7 sin, operation for operation as math_families.h:81-90 (f64).
__device__ __forceinline__ double mlk_p7_sin(double x) {
    using namespace mlk;
    const double n = floor(x / kPiHalf + 0.5);
    const double r = (x - n * kPio2Hi) - n * kPio2Lo;
    const int q = quadrantOf(n);
    const double r2 = r * r;
    double v;
    if (q & 1) {
        double p = kC[0];
        for (int i = 1; i < 6; ++i) p = p * r2 + kC[i];
        v = 1.0 - r2 * 0.5 + r2 * r2 * p;
    } else {
        double p = kS[0];
        for (int i = 1; i < 6; ++i) p = p * r2 + kS[i];
        v = r + r * r2 * p;
    }
    return (q & 2) ? -v : v;
}

/// poly7 sin for a value rounded to f32 right after (the planner uses it
/// only when sin is the chain's last op and the output is f32). The
/// reduction r = (x - n*hi) - n*lo stays in f64; the residual polynomials run
/// in f32 on r rounded to f32 (|r| <= pi/4: ~1 f32 ULP, plus r's own 0.5 ULP
/// relative rounding). n = floor(x*2/pi + 0.5) can differ from the
/// reference's floor(x/(pi/2) + 0.5) only within an ULP of an odd multiple of
/// pi/4, where both reductions are valid and agree to polynomial accuracy.
__device__ __forceinline__ double mlk_p7_sin_f32out(double x) {
    using namespace mlk;
    const double n = floor(x * kTwoOverPi + 0.5);
    const double r = (x - n * kPio2Hi) - n * kPio2Lo;
    const int q = quadrantOf(n);
    const float rf = static_cast<float>(r);
    const float r2 = rf * rf;
    float ps = static_cast<float>(kS[0]);
    float pc = static_cast<float>(kC[0]);
#pragma unroll
    for (int i = 1; i < 6; ++i) {
        ps = __builtin_fmaf(ps, r2, static_cast<float>(kS[i]));
        pc = __builtin_fmaf(pc, r2, static_cast<float>(kC[i]));
    }
    const float s = __builtin_fmaf(rf * r2, ps, rf);
    const float c = __builtin_fmaf(r2 * r2, pc, __builtin_fmaf(-0.5f, r2, 1.0f));
    float v = (q & 1) ? c : s;
    v = (q & 2) ? -v : v;
    return r == r ? static_cast<double>(v) : r;  // NaN/inf arguments give NaN
}

struct mlk_scalars {
    double v[8];
};

namespace mlk {

// dtype codes: 0 f32, 1 f16, 2 f64 (mlkd_dtype).
template <int DT>
__device__ __forceinline__ double loadOne(const void* p, long long i) {
    if constexpr (DT == 0) return static_cast<double>(static_cast<const float*>(p)[i]);
    else if constexpr (DT == 1)
        return static_cast<double>(static_cast<float>(static_cast<const _Float16*>(p)[i]));
    else return static_cast<const double*>(p)[i];
}

/// f64 -> f16 with one rounding: round-to-odd into f32 (truncate, set the last
/// bit when inexact), then RNE to f16.
__device__ __forceinline__ _Float16 toHalf(double d) {
    float t = __double2float_rz(d);
    if (static_cast<double>(t) != d && t == t) t = __uint_as_float(__float_as_uint(t) | 1u);
    return static_cast<_Float16>(t);
}

template <int DT>
__device__ __forceinline__ void storeOne(void* p, long long i, double v) {
    if constexpr (DT == 0) static_cast<float*>(p)[i] = static_cast<float>(v);
    else if constexpr (DT == 1) static_cast<_Float16*>(p)[i] = toHalf(v);
    else static_cast<double*>(p)[i] = v;
}


}  // namespace mlk

#endif  // MLK_DEVICE_MATH_H
