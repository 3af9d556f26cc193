// fp64.hpp — short correctly rounded fp64 division and square root for operands
// in known, moderate ranges (the Jacobi rotation's scalar chain).
//
// For a / b and sqrt(x) the compiler emits a refinement of the hardware
// reciprocal (v_rcp_f64) or reciprocal square root (v_rsq_f64) wrapped in range
// handling: v_div_scale / v_div_fmas / v_div_fixup for division, and a 2^256
// pre-scale of tiny inputs plus a class check for 0 and inf for sqrt. The helpers
// below keep the refinement and drop the wrapping, so on operands that never need
// it they return the same bits as IEEE `/` and `sqrt` in fewer dependent steps:
//   * div_rn(a, b): two Newton-Raphson steps r <- r + r (1 - b r) on the
//     reciprocal, then q = a r corrected once by the exact residual a - b q
//     (Markstein's correctly rounded quotient). Needs b and a / b normal and far
//     from overflow, which holds for |b| in [2^-900, 2^900] and |a| < 2^900.
//   * sqrt_ge1(x): Goldschmidt's coupled iteration g -> sqrt(x), h -> 1/(2 sqrt x)
//     from y = rsq(x), then two residual corrections g += (x - g^2) h. Needs
//     1 <= x < 2^900, where no pre-scale applies.
//   * rcp_sqrt_ge1(x): 1 / sqrt(x) with both roundings, from the same iteration.
// slime_probe_fp64_core (probe.hip) checks both against `/` and `sqrt` bit for
// bit over the rotation's operand ranges on the device.
#pragma once

#include <hip/hip_runtime.h>

namespace slime {

__device__ __forceinline__ double div_rn(double a, double b) {
    double r = __builtin_amdgcn_rcp(b);
    r = __builtin_fma(r, __builtin_fma(-b, r, 1.0), r);
    r = __builtin_fma(r, __builtin_fma(-b, r, 1.0), r);
    const double q = a * r;
    return __builtin_fma(__builtin_fma(-b, q, a), r, q);
}

__device__ __forceinline__ double sqrt_ge1(double x) {
    const double y = __builtin_amdgcn_rsq(x);
    double g = x * y, h = 0.5 * y;
    const double e = __builtin_fma(-h, g, 0.5);
    g = __builtin_fma(g, e, g);
    h = __builtin_fma(h, e, h);
    g = __builtin_fma(__builtin_fma(-g, g, x), h, g);
    return __builtin_fma(__builtin_fma(-g, g, x), h, g);
}

// rcp_sqrt_ge1(x) = 1 / sqrt(x) with both IEEE roundings (the bits of `1.0 / sqrt(x)`),
// 1 <= x < 2^900: sqrt_ge1's g, then the reciprocal of g from 2 h (h approximates
// 1 / (2 sqrt x) to ~2^-44 after the coupled step) by one Newton-Raphson step and
// the same correction as div_rn with a = 1. This replaces the v_rcp_f64 and one of
// the two refinement steps that div_rn(1, sqrt_ge1(x)) takes.
__device__ __forceinline__ double rcp_sqrt_ge1(double x) {
    const double y = __builtin_amdgcn_rsq(x);
    double g = x * y, h = 0.5 * y;
    const double e = __builtin_fma(-h, g, 0.5);
    g = __builtin_fma(g, e, g);
    h = __builtin_fma(h, e, h);
    g = __builtin_fma(__builtin_fma(-g, g, x), h, g);
    g = __builtin_fma(__builtin_fma(-g, g, x), h, g);
    double r = 2.0 * h;
    r = __builtin_fma(r, __builtin_fma(-g, r, 1.0), r);
    return __builtin_fma(__builtin_fma(-g, r, 1.0), r, r);
}

// The rotation of the cyclic Jacobi solve for the 2x2 block [[app, apq], [apq, aqq]],
// |apq| > 0: tau = (aqq - app) / (2 apq), t = sign(tau) / (|tau| + sqrt(1 + tau^2))
// (t = +1 at tau = +-0), c = 1 / sqrt(1 + t^2), s = t c. |t| <= 1, so the second
// square root sees x in [1, 2]. With the fast helpers (kFast) every precondition
// holds when |2 apq| >= 2^-900 and |tau| < 2^440 (then 1 + tau^2 < 2^900): for a
// Gram of fp32 values summed over at most 2^40 cells, |a_ij| < 2^297, and the
// solve rotates only for |apq| > 1e-6, so |tau| < 2^317.
template <bool kFast>
__device__ __forceinline__ void jacobi_rotation(double app, double aqq, double apq, double& c, double& s) {
    if constexpr (kFast) {
        const double tau = div_rn(aqq - app, 2.0 * apq);
        const double u = div_rn(1.0, fabs(tau) + sqrt_ge1(1.0 + tau * tau));
        const double t = tau < 0.0 ? -u : u;
        c = rcp_sqrt_ge1(1.0 + t * t);
        s = t * c;
    } else {
        const double tau = (aqq - app) / (2.0 * apq);
        const double u = 1.0 / (fabs(tau) + sqrt(1.0 + tau * tau));
        const double t = tau < 0.0 ? -u : u;
        c = 1.0 / sqrt(1.0 + t * t);
        s = t * c;
    }
}

}  // namespace slime
