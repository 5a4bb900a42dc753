// fp32 vector / quaternion helpers for the step kernel.
//
// Semantics follow the reference's MSL helpers (src/shaders/all_shaders.metal:76-100):
// operations evaluate left to right, dot(a,b) = a.x*b.x + a.y*b.y + a.z*b.z,
// length = sqrt(dot), quat_normalize divides each component by the length. The library is
// compiled with -ffp-contract=off and correctly rounded division and square root, so each
// expression rounds exactly as written.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace za {

struct f3 { float x, y, z; };
struct q4 { float x, y, z, w; };

__device__ __forceinline__ f3 mk3(float x, float y, float z) { return {x, y, z}; }
__device__ __forceinline__ q4 mk4(float x, float y, float z, float w) { return {x, y, z, w}; }
__device__ __forceinline__ f3 add(f3 a, f3 b) { return {a.x + b.x, a.y + b.y, a.z + b.z}; }
__device__ __forceinline__ f3 sub(f3 a, f3 b) { return {a.x - b.x, a.y - b.y, a.z - b.z}; }
__device__ __forceinline__ f3 mul(f3 a, f3 b) { return {a.x * b.x, a.y * b.y, a.z * b.z}; }
__device__ __forceinline__ f3 scale(f3 a, float s) { return {a.x * s, a.y * s, a.z * s}; }
__device__ __forceinline__ f3 sscale(float s, f3 a) { return {s * a.x, s * a.y, s * a.z}; }
// Several fp32 quotients with one divisor, through one fp64 reciprocal. y = 1 / b is the
// v_rcp_f64 estimate r0 refined by the cubic correction r0 (1 + e + e^2), e = 1 - b r0 (three
// dependent fp64 FMAs; the relative error becomes about e^3 plus one rounding). Over every
// finite nonzero fp32 b, |1 - b r0| <= 2^-24.39 and |1 - b y| <= 2^-53 (measured exhaustively
// on gfx950: zeno_amd_selfcheck_reciprocal_error), so q = fp64(a * y) is within ~2^-52 of a / b.
//
// Why fp32(q) is the correctly rounded a / b. Write a = A 2^ea, b = B 2^eb (A, B < 2^24
// integers) and let m = M 2^em be a rounding boundary of the fp32 grid (a midpoint of two
// neighbours, M odd). If a / b != m, then a - m b is a nonzero multiple of 2^min(ea, em+eb),
// which puts a / b at least 2^-50 (relative to m) away from m; q, within 2^-52, lies on the
// same side of every boundary, and its rounding is that of a / b. A quotient exactly at a
// boundary (a = m b) needs A = M B 2^j: for a normal quotient M has 25 bits, more than A holds,
// so this cannot happen; for a subnormal quotient the boundaries are the odd multiples of
// 2^-150 and small M make exact ties possible (a = 147 2^-149, b = 98), where q, off the tie
// by its error, would round to either side; to_f32_tie_even settles them. Overflowing quotients
// land beyond the fp32 range of q and convert to infinity. A zero or infinite divisor keeps the
// raw reciprocal (+-inf, +-0, exact), so a * y gives the IEEE quotient (+-inf, +-0 or NaN); a
// NaN divisor gives NaN.
__device__ __forceinline__ double rcp64(float b) {
    const double d = (double)b;
    const double r0 = __builtin_amdgcn_rcp(d);
    const double e = __builtin_fma(-d, r0, 1.0);
    const double r = __builtin_fma(r0, __builtin_fma(e, e, e), r0);
    return (__builtin_isfinite(b) && b != 0.0f) ? r : r0;
}
// fp32(q) for q = fp64(a * y). |q| is first rounded to a multiple of 2^-176 by adding and
// subtracting C = 1.5 2^-124 (both exact-rounding fp64 operations; -fno-fast-math keeps them):
// for |q| < 2^-125 the sum lies in [2^-124, 2^-123), where the spacing is 2^-176, and the
// subtraction is exact; for |q| >= 2^-71 both operations give q back unchanged; in between
// they move q by at most 2^-52 relative. A subnormal tie sits within 2^-177.4 of its midpoint,
// an odd multiple of 2^-150, and lands on it exactly; every other subnormal quotient is at
// least 2^-174 from a midpoint and keeps its side. The fp32 conversion then rounds a tie to
// even, as IEEE division does. The sign is copied back so that -0 stays -0.
__device__ __forceinline__ float to_f32_tie_even(double q) {
    constexpr double C = 0x1.8p-124;
    return (float)__builtin_copysign((__builtin_fabs(q) + C) - C, q);
}
__device__ __forceinline__ f3 divs(f3 a, float s) {
    const double y = rcp64(s);
    return {to_f32_tie_even((double)a.x * y), to_f32_tie_even((double)a.y * y), to_f32_tie_even((double)a.z * y)};
}
// q / l for the four components, through one reciprocal (see divs).
__device__ __forceinline__ q4 qdivs(q4 q, float l) {
    const double y = rcp64(l);
    return {to_f32_tie_even((double)q.x * y), to_f32_tie_even((double)q.y * y),
            to_f32_tie_even((double)q.z * y), to_f32_tie_even((double)q.w * y)};
}
__device__ __forceinline__ f3 neg(f3 a) { return {-a.x, -a.y, -a.z}; }
__device__ __forceinline__ float dot(f3 a, f3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
__device__ __forceinline__ float len(f3 a) { return __builtin_sqrtf(dot(a, a)); }
// Square root for a value that is compared against a threshold of at least 2^-47 before the
// root is used: v_sqrt_f32 followed by the one-ulp correction of a correctly rounded fp32
// square root (the residuals x - s' s for s' one ulp below and above s decide between the three
// candidates), without the scaling of inputs below 2^-96 and the final select for 0 and
// infinity. For x >= 2^-96 the operations are those of the correctly rounded root; +-0, +inf,
// NaN and negative x come out as the correctly rounded root does (the failing compares keep
// s); for 0 < x < 2^-96 the result is below 2^-47 and fails every such threshold.
__device__ __forceinline__ float sqrt_gate(float x) {
    const float s = __builtin_amdgcn_sqrtf(x);
    const float sd = __int_as_float(__float_as_int(s) - 1), su = __int_as_float(__float_as_int(s) + 1);
    const float t = __builtin_fmaf(-sd, s, x) <= 0.0f ? sd : s;
    return __builtin_fmaf(-su, s, x) > 0.0f ? su : t;
}
__device__ __forceinline__ float len_gate(f3 a) { return sqrt_gate(dot(a, a)); }
__device__ __forceinline__ f3 cross(f3 a, f3 b) {
    return {a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}
__device__ __forceinline__ f3 xyz(float4 v) { return {v.x, v.y, v.z}; }
__device__ __forceinline__ f3 xyz(q4 v) { return {v.x, v.y, v.z}; }
__device__ __forceinline__ q4 toq(float4 v) { return {v.x, v.y, v.z, v.w}; }
__device__ __forceinline__ float4 tof4(q4 v) { return make_float4(v.x, v.y, v.z, v.w); }
__device__ __forceinline__ float4 tof4(f3 v, float w) { return make_float4(v.x, v.y, v.z, w); }

__device__ __forceinline__ q4 qadd(q4 a, q4 b) { return {a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w}; }
__device__ __forceinline__ q4 qsub(q4 a, q4 b) { return {a.x - b.x, a.y - b.y, a.z - b.z, a.w - b.w}; }
__device__ __forceinline__ q4 qscale(q4 a, float s) { return {a.x * s, a.y * s, a.z * s, a.w * s}; }
__device__ __forceinline__ q4 qneg(q4 a) { return {-a.x, -a.y, -a.z, -a.w}; }
__device__ __forceinline__ q4 qconj(q4 q) { return {-q.x, -q.y, -q.z, q.w}; }
// Hamilton product, xyzw storage.
__device__ __forceinline__ q4 qmul(q4 a, q4 b) {
    return {a.w * b.x + a.x * b.w + a.y * b.z - a.z * b.y,
            a.w * b.y - a.x * b.z + a.y * b.w + a.z * b.x,
            a.w * b.z + a.x * b.y - a.y * b.x + a.z * b.w,
            a.w * b.w - a.x * b.x - a.y * b.y - a.z * b.z};
}
// v + 2 (w (q x v) + q x (q x v))
__device__ __forceinline__ f3 qrot(f3 v, q4 q) {
    f3 qv = {q.x, q.y, q.z};
    f3 uv = cross(qv, v);
    f3 uuv = cross(qv, uv);
    return {v.x + 2.0f * (q.w * uv.x + uuv.x), v.y + 2.0f * (q.w * uv.y + uuv.y),
            v.z + 2.0f * (q.w * uv.z + uuv.z)};
}
__device__ __forceinline__ float qlen(q4 q) { return __builtin_sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w); }
__device__ __forceinline__ q4 qnormalize(q4 q) {
    const float l = qlen(q);
    if (!(l > 1e-8f)) return q4{0.0f, 0.0f, 0.0f, 1.0f};
    return qdivs(q, l);
}
// qnormalize with the quotients evaluated before the length test and the identity selected
// after it (same results; sqrt_gate is exact wherever the test l > 1e-8 passes).
__device__ __forceinline__ q4 qnormalize_sel(q4 q) {
    const float l = sqrt_gate(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w);
    const q4 r = qdivs(q, l);
    return l > 1e-8f ? r : q4{0.0f, 0.0f, 0.0f, 1.0f};
}
// Quaternion step q + s * ((d, 0) (x) q) used by every XPBD rotation update.
__device__ __forceinline__ q4 qdelta(f3 d, q4 q) { return qscale(qmul(mk4(d.x, d.y, d.z, 0.0f), q), 0.5f); }
__device__ __forceinline__ float clampf(float x, float lo, float hi) { return fminf(fmaxf(x, lo), hi); }

// atan2 / asin after S. Moshier's Cephes single-precision routines (atanf.c, asinf.c):
// reduction at tan(3pi/8) and tan(pi/8) with a degree-9 odd polynomial for atan; the 0.5
// split with sqrt reduction and a degree-11 odd polynomial for asin. Max error 3 ulp. The
// CPU oracle evaluates the same operations (oracle/zeno_oracle.c).
constexpr float kPi = 3.14159265358979323846f;
constexpr float kPiO2 = 1.57079632679489661923f;
constexpr float kPiO4 = 0.78539816339744830962f;

// atan2 without branches: every case of the branching form (NaN, x == 0, y == 0,
// infinities, the three reduction ranges of atan) is evaluated and selected, so lanes do
// not diverge. The reduction range selects the operands of its single division: -1 / q
// above tan(3pi/8), (q - 1) / (q + 1) above tan(pi/8); each result equals the branching
// form's bit for bit.
__device__ __forceinline__ float z_atan2f(float y, float x) {
    const float ax = __builtin_fabsf(x), ay = __builtin_fabsf(y);
    const float q = ay / ax;
    const bool big = q > 2.414213562373095f, mid = q > 0.4142135623730950f;
    const float num = big ? -1.0f : q - 1.0f;
    const float den = big ? q : q + 1.0f;
    const float t = mid ? num / den : q;
    const float y0 = big ? kPiO2 : (mid ? kPiO4 : 0.0f);
    const float z = t * t;
    const float p = (((8.05374449538e-2f * z - 1.38776856032e-1f) * z + 1.99777106478e-1f) * z - 3.33329491539e-1f) * z * t + t;
    const float at = y0 + p;
    float r = x > 0.0f ? at : kPi - at;
    const bool ix = __builtin_isinf(ax), iy = __builtin_isinf(ay);
    r = ix ? (iy ? (x > 0.0f ? kPiO4 : 3.0f * kPiO4) : (x > 0.0f ? 0.0f : kPi)) : (iy ? kPiO2 : r);
    float res = y < 0.0f ? -r : r;
    const float on_axis = __builtin_signbit(x) ? (__builtin_signbit(y) ? -kPi : kPi) : y;  // y == 0 (and x == 0, y == 0)
    const float x_zero = y > 0.0f ? kPiO2 : (y < 0.0f ? -kPiO2 : on_axis);
    res = y == 0.0f ? on_axis : res;
    res = x == 0.0f ? x_zero : res;
    return (__builtin_isnan(x) || __builtin_isnan(y)) ? x + y : res;
}

__device__ __forceinline__ float z_asinf(float x) {
    if (__builtin_isnan(x)) return x;
    float a = __builtin_fabsf(x);
    if (a > 1.0f) return __builtin_nanf("");
    float z, t;
    bool flag = a > 0.5f;
    if (flag) { z = 0.5f * (1.0f - a); t = __builtin_sqrtf(z); }
    else { t = a; z = a * a; }
    float p = ((((4.2163199048e-2f * z + 2.4181311049e-2f) * z + 4.5470025998e-2f) * z + 7.4953002686e-2f) * z + 1.6666752422e-1f) * z * t + t;
    if (flag) p = kPiO2 - (p + p);
    return x < 0.0f ? -p : p;
}

}  // namespace za
