// Correctly rounded square roots for the exact paths.
//
// v_sqrt_f32 is accurate to 1 ulp only (hipcc lowers __fsqrt_rn to it), and
// the expansion hipcc emits for double sqrt is not documented as correctly
// rounded either, so both take an estimate s and pick among its neighbours
// with Tuckerman's rounding test: the residuals x - s_dn*s and x - s_up*s,
// whose signs an FMA gives exactly, tell which of s_dn, s, s_up is sqrt(x)
// rounded to nearest.  Tiny inputs (subnormal or close to it, where the
// residuals could underflow) are scaled by an even power of two first, which
// changes neither the rounding nor the result beyond the exact rescale.
#pragma once
#include <hip/hip_runtime.h>

namespace aq_math {

__device__ inline float sqrt_rn(float x) {
    if (!(x > 0.0f) || !(x < INFINITY)) return __builtin_amdgcn_sqrtf(x);   // 0, -0, <0, Inf, NaN
    float scale = 1.0f;
    if (x < 0x1p-100f) {
        x *= 0x1p100f;
        scale = 0x1p-50f;
    }
    const float s = __builtin_amdgcn_sqrtf(x);
    const float sd = __int_as_float(__float_as_int(s) - 1);
    const float su = __int_as_float(__float_as_int(s) + 1);
    const float rd = __fmaf_rn(-sd, s, x);
    const float ru = __fmaf_rn(-su, s, x);
    float out = s;
    if (rd <= 0.0f) out = sd;
    if (ru > 0.0f) out = su;
    return out * scale;
}

__device__ inline double sqrt_rn(double x) {
    if (!(x > 0.0) || !(x < INFINITY)) return __builtin_sqrt(x);
    double scale = 1.0;
    if (x < 0x1p-900) {
        x *= 0x1p256;
        scale = 0x1p-128;
    }
    const double s = __builtin_sqrt(x);
    const double sd = __longlong_as_double(__double_as_longlong(s) - 1);
    const double su = __longlong_as_double(__double_as_longlong(s) + 1);
    const double rd = __fma_rn(-sd, s, x);
    const double ru = __fma_rn(-su, s, x);
    double out = s;
    if (rd <= 0.0) out = sd;
    if (ru > 0.0) out = su;
    return out * scale;
}

}  // namespace aq_math
