// Host stand-ins for the HIP names a generated loop-nest kernel uses, so the
// kernel text compiles as plain C++ for the CPU (under AddressSanitizer) and
// its grid can be run one thread at a time. Test infrastructure only.
#pragma once
#include <math.h>
#include <stdint.h>
#include <string.h>

#define __HIPCC_RTC__ 1
#define __device__
#define __host__
#define __global__
#define __forceinline__ inline
#define __launch_bounds__(...)
// LDS slabs: one static copy stands for the workgroup's, and each thread the
// harness runs copies the whole slab before reading it.
#define __shared__ static
#define MLK_SLAB_FIRST 0LL
#define MLK_SLAB_STEP 1LL
inline void __syncthreads() {}

struct mlk_dim3 {
    unsigned x, y, z;
};
extern mlk_dim3 blockIdx, threadIdx, gridDim, blockDim;

/// The hardware f32 exp2 (v_exp_f32, 1 ULP) stands as libm's exp2f.
#define MLK_HOST_SHIM 1
inline float mlk_hw_exp2f(float x) { return exp2f(x); }
inline unsigned mlk_bitsel(unsigned m, unsigned a, unsigned b) { return (a & m) | (b & ~m); }
/// One thread at a time: lane masks of a wave of one.
inline unsigned long long mlk_lanes_uge(double a, double b) { return !(a < b) ? 1ull : 0ull; }

inline float __uint_as_float(unsigned u) {
    float f;
    memcpy(&f, &u, sizeof(f));
    return f;
}
inline unsigned __float_as_uint(float f) {
    unsigned u;
    memcpy(&u, &f, sizeof(u));
    return u;
}
/// f64 -> f32 rounded toward zero.
inline float __double2float_rz(double d) {
    float f = static_cast<float>(d);
    if (f != f) return f;
    if (isinf(f) && !isinf(d)) return nextafterf(f, 0.0f);
    if ((d >= 0 && static_cast<double>(f) > d) || (d <= 0 && static_cast<double>(f) < d)) f = nextafterf(f, 0.0f);
    return f;
}
