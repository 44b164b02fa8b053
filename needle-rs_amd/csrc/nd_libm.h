// Single-precision exp and log with a fixed, documented algorithm, usable in
// host and device code alike, so that the device forward rounds exactly as
// the reference's CPU path does.
//
// The reference calls libm 0.2 (`libm::expf`, `libm::logf`,
// crates/needle-core/src/math.rs:3-16), whose expf and logf follow the
// FreeBSD msun e_expf.c / e_logf.c algorithms by way of musl:
//   expf: reduce x = k ln2 + r (ln2 split hi/lo, k from x/ln2 + 1/2
//         truncated), then exp(r) = 1 + r + r c/(2 - c) with the degree-2
//         remez polynomial c = r - r^2 (P1 + r^2 P2), scaled by 2^k;
//   logf: x = 2^k (1 + f), f in [sqrt(2)/2 - 1, sqrt(2) - 1], s = f/(2 + f),
//         log(1 + f) = f - hfsq + s (hfsq + R(s^2)) with a degree-4 even
//         polynomial R (Lg1..Lg4), plus k ln2 (hi/lo).
// Built without FP contraction, every operation below rounds as written.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define ND_LIBM_FN __host__ __device__ inline
#else
#define ND_LIBM_FN static inline
#endif

ND_LIBM_FN uint32_t nd_f2u(float f)
{
    union {
        float f;
        uint32_t u;
    } v;
    v.f = f;
    return v.u;
}

ND_LIBM_FN float nd_u2f(uint32_t u)
{
    union {
        float f;
        uint32_t u;
    } v;
    v.u = u;
    return v.f;
}

// x * 2^n with the over/underflow steps of scalbnf.
ND_LIBM_FN float nd_scalbnf(float x, int n)
{
    const float x1p127 = nd_u2f(0x7f000000u);
    const float x1p_126 = nd_u2f(0x00800000u);
    const float x1p24 = nd_u2f(0x4b800000u);
    if (n > 127) {
        x *= x1p127;
        n -= 127;
        if (n > 127) {
            x *= x1p127;
            n -= 127;
            if (n > 127) n = 127;
        }
    } else if (n < -126) {
        x *= x1p_126 * x1p24;
        n += 126 - 24;
        if (n < -126) {
            x *= x1p_126 * x1p24;
            n += 126 - 24;
            if (n < -126) n = -126;
        }
    }
    return x * nd_u2f((uint32_t)(0x7f + n) << 23);
}

ND_LIBM_FN float nd_expf(float x)
{
    const float half[2] = {0.5f, -0.5f};
    const float ln2_hi = 6.9314575195e-01f;  // 0x3f317200
    const float ln2_lo = 1.4286067653e-06f;  // 0x35bfbe8e
    const float inv_ln2 = 1.4426950216e+00f; // 0x3fb8aa3b
    const float p1 = 1.6666625440e-1f;
    const float p2 = -2.7667332906e-3f;
    uint32_t hx = nd_f2u(x);
    const int sign = (int)(hx >> 31);
    hx &= 0x7fffffffu;
    if (hx >= 0x42aeac50u) {       // |x| >= 87.33655 or NaN
        if (hx > 0x7f800000u) return x;  // NaN
        if (hx >= 0x42b17218u && !sign) return x * nd_u2f(0x7f000000u);  // overflow
        if (sign && hx >= 0x42cff1b5u) return 0.0f;  // x <= -103.972084: underflow
    }
    int k;
    float hi, lo;
    if (hx > 0x3eb17218u) {        // |x| > ln2 / 2
        if (hx > 0x3f851592u)      // |x| > 1.5 ln2
            k = (int)(inv_ln2 * x + half[sign]);
        else
            k = 1 - sign - sign;
        const float kf = (float)k;
        hi = x - kf * ln2_hi;
        lo = kf * ln2_lo;
        x = hi - lo;
    } else if (hx > 0x39000000u) { // |x| > 2^-14
        k = 0;
        hi = x;
        lo = 0.0f;
    } else {
        return 1.0f + x;
    }
    const float xx = x * x;
    const float c = x - xx * (p1 + xx * p2);
    const float y = 1.0f + (x * c / (2.0f - c) - lo + hi);
    return k == 0 ? y : nd_scalbnf(y, k);
}

ND_LIBM_FN float nd_logf(float x)
{
    const float ln2_hi = 6.9313812256e-01f;  // 0x3f317180
    const float ln2_lo = 9.0580006145e-06f;  // 0x3717f7d1
    const float lg1 = 0.66666662693f;
    const float lg2 = 0.40000972152f;
    const float lg3 = 0.28498786688f;
    const float lg4 = 0.24279078841f;
    uint32_t ix = nd_f2u(x);
    int k = 0;
    if (ix < 0x00800000u || (ix >> 31)) {  // x < 2^-126, or negative
        if ((ix << 1) == 0) return -1.0f / (x * x);  // log(+-0) = -inf
        if (ix >> 31) return (x - x) / 0.0f;          // log(negative) = NaN
        k -= 25;                                      // subnormal: scale up
        x *= nd_u2f(0x4c000000u);
        ix = nd_f2u(x);
    } else if (ix >= 0x7f800000u) {
        return x;
    } else if (ix == 0x3f800000u) {
        return 0.0f;
    }
    ix += 0x3f800000u - 0x3f3504f3u;
    k += (int)(ix >> 23) - 0x7f;
    ix = (ix & 0x007fffffu) + 0x3f3504f3u;
    x = nd_u2f(ix);
    const float f = x - 1.0f;
    const float s = f / (2.0f + f);
    const float z = s * s;
    const float w = z * z;
    const float t1 = w * (lg2 + w * lg4);
    const float t2 = z * (lg1 + w * lg3);
    const float r = t2 + t1;
    const float hfsq = 0.5f * f * f;
    const float dk = (float)k;
    return s * (hfsq + r) + dk * ln2_lo - hfsq + f + dk * ln2_hi;
}

ND_LIBM_FN float nd_sigmoidf(float x) { return 1.0f / (1.0f + nd_expf(-x)); }
