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

/// fmod(n, 4) taken into [0, 4) for the integral n of the reduction
/// (math_families.h:71-72): n - 4 * floor(n / 4). Every step is exact for any
/// finite n (the scalings are by powers of two, and the difference is an
/// integer in [0, 3], or 0 once ulp(n) >= 8), so it gives the reference's
/// quadrant with four f64 operations and no fmod.
__device__ __forceinline__ int quadrantOf(double n) {
    const double f = floor(n * 0.25);
    return static_cast<int>(n - 4.0 * f);
}

// Residual polynomials for results rounded to f32, on |r| <= pi/4:
// sin r ~ r + r^3 (s0 + s1 r^2 + s2 r^4), cos r ~ 1 - r^2/2 + r^4 (c0 + c1 r^2
// + c2 r^4). Fitted by iteratively reweighted least squares on 2e5 points
// (converging to the minimax): relative error 3.9e-9 (sine) and 1.2e-10
// (cosine) before the coefficients' rounding to f32.
constexpr float kSinF32[3] = {-0x1.555546p-3f, 0x1.11073cp-7f, -0x1.994446p-13f};
constexpr float kCosF32[3] = {0x1.55554ap-5f, -0x1.6c0c34p-10f, 0x1.99ebf6p-16f};

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

#ifndef MLK_HOST_SHIM
/// The hardware f32 exp2 (v_exp_f32, 1 ULP on the finite range).
__device__ __forceinline__ float mlk_hw_exp2f(float x) { return __builtin_amdgcn_exp2f(x); }
/// Bitwise select: bits of a where m is set, of b elsewhere (v_bitop3_b32,
/// truth table 0xCA).
__device__ __forceinline__ unsigned mlk_bitsel(unsigned m, unsigned a, unsigned b) {
    return __builtin_amdgcn_bitop3_b32(m, a, b, 0xCA);
}
/// The wave's lanes where a >= b or either is NaN (one compare into a
/// scalar lane mask; LLVM's FCMP_UGE).
__device__ __forceinline__ unsigned long long mlk_lanes_uge(double a, double b) {
    return __builtin_amdgcn_fcmp(a, b, 11);
}
#endif

/// poly7 sin for a value rounded to f32 right after (the planner uses it
/// only when sin is the chain's last op, the output is f32 and stores are
/// plain).
///
/// The reduction is the reference's r = (x - n*hi) - n*lo in f64, with n =
/// floor(y), y = x*(2/pi) + 0.5 in one fused operation where the reference
/// divides by pi/2. For |y| < 2^20 that y is within 5 ULP (< 2^-30) of the
/// reference's, so the two n differ only where x is that close to an odd
/// multiple of pi/4; there both reductions are valid (|r| ~ pi/4, each
/// exact to 2^-32) and give the same value to 1e-9 relative. Elsewhere n,
/// r and the quadrant are the reference's bits, so r near a zero of the sine
/// is the reference's r. For |y| >= 2^20, NaN and infinities the function
/// adds the lane to the wave mask `slow` and the caller recomputes the
/// element with mlk_p7_sin. The degree-7 sine and degree-8 cosine residual
/// polynomials (kSinF32, kCosF32) run in f32 on r rounded to f32: within 2
/// f32 ULP of the f64 form rounded to f32 (CPU sweeps of 3.2e7 arguments,
/// and of 3e6 within 4 ULP of multiples of pi/4, find no larger). The exact
/// form is not inlined here, so the caller's unrolled hot loop carries no
/// f64 division or full polynomial.
__device__ __forceinline__ float mlk_p7_sin_f32out(double x, unsigned long long& slow) {
    using namespace mlk;
    const double y = __builtin_fma(x, kTwoOverPi, 0.5);
    const double n = floor(y);
    const double r = (x - n * kPio2Hi) - n * kPio2Lo;
    slow |= mlk_lanes_uge(__builtin_fabs(y), 0x1p20);
    const int q = static_cast<int>(n);  // |n| <= 2^20 wherever the result is used
    const float rf = static_cast<float>(r);
    const float r2 = rf * rf;
    const float ps = __builtin_fmaf(__builtin_fmaf(kSinF32[2], r2, kSinF32[1]), r2, kSinF32[0]);
    const float pc = __builtin_fmaf(__builtin_fmaf(kCosF32[2], r2, kCosF32[1]), r2, kCosF32[0]);
    const float s = __builtin_fmaf(rf * r2, ps, rf);
    const float c = __builtin_fmaf(r2, __builtin_fmaf(r2, pc, -0.5f), 1.0f);  // 1 - r2/2 + r2^2 pc
    // Odd quadrants take the cosine (an all-ones mask from bit 0 selects it
    // bitwise), quadrants 2 and 3 flip the sign (bit 1 moved to bit 31).
    const unsigned odd = static_cast<unsigned>(static_cast<int>(static_cast<unsigned>(q) << 31) >> 31);
    const unsigned v = mlk_bitsel(odd, __float_as_uint(c), __float_as_uint(s));
    return __uint_as_float(v ^ ((static_cast<unsigned>(q) << 30) & 0x80000000u));
}


/// exp for a chain whose result reaches an f32 output only through products
/// and quotients (which carry a relative error through unchanged):
/// exp(u) = 2^k * 2^f with t = u*log2(e) in f64, k = rint(t), f = t - k
/// (exact, |f| <= 1/2) and 2^f from the hardware's f32 exp2 on f rounded to
/// f32 (1 f32 ULP, plus 2e-8 from the rounding of f): about 1.4e-7 relative,
/// so the f32 result is within 2 ULP of the reference's f64 exp rounded to
/// f32. |t| >= 1000 (near overflow and underflow), NaN and infinities add
/// the lane to the wave mask `slow`: the caller recomputes that element with
/// the f64 exp.
__device__ __forceinline__ double mlk_exp_f32acc(double u, unsigned long long& slow) {
    const double t = u * 1.4426950408889634074;
    slow |= mlk_lanes_uge(__builtin_fabs(t), 1000.0);
    const double k = __builtin_rint(t);
    const float e = mlk_hw_exp2f(static_cast<float>(t - k));
    return __builtin_ldexp(static_cast<double>(e), static_cast<int>(k));
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
