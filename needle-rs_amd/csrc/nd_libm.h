// Single-precision exp, log, pow, sin and cos with a fixed, documented
// algorithm, usable in host and device code alike, so that the device
// forward rounds exactly as the reference's CPU path does.
//
// The reference calls libm 0.2.16 (`libm::expf`, `libm::logf`,
// `libm::powf`, `libm::sinf`, `libm::cosf`, crates/needle-core/src/math.rs:3-46),
// whose single-precision functions follow the FreeBSD msun algorithms by way
// of musl (e_expf.c, e_logf.c, e_powf.c, s_sinf.c, s_cosf.c, k_sinf.c,
// k_cosf.c, e_rem_pio2f.c, k_rem_pio2.c):
//   expf: reduce x = k ln2 + r (ln2 split hi/lo, k from x/ln2 + 1/2
//         truncated), then exp(r) = 1 + r + r c/(2 - c) with the degree-2
//         remez polynomial c = r - r^2 (P1 + r^2 P2), scaled by 2^k;
//   logf: x = 2^k (1 + f), f in [sqrt(2)/2 - 1, sqrt(2) - 1], s = f/(2 + f),
//         log(1 + f) = f - hfsq + s (hfsq + R(s^2)) with a degree-4 even
//         polynomial R (Lg1..Lg4), plus k ln2 (hi/lo);
//   powf: log2|x| = n + log2(1.5^k (1 + s)/(1 - s)) from a degree-6 series
//         in s^2 carried as a high/low pair with 12-bit high parts, times y
//         split the same way, then 2^(n + r) with r reduced to [-1/2, 1/2]
//         and a degree-5 expansion of r (e^r + 1)/(e^r - 1) (P1..P5);
//   sinf, cosf: |x| <= 9 pi/4 reduced by the nearest multiple of pi/2 in
//         double; beyond, x - n pi/2 with a 25 + 53 bit pi/2 while
//         |x| < 2^28 pi/2, and Payne-Hanek over 24-bit chunks of 2/pi above;
//         the reduced argument goes through degree-4 double polynomials for
//         sin (S1..S4) and cos (C0..C3), rounded once to float.
// Built without FP contraction, every operation below rounds as written.
#pragma once

#include <math.h>
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

// e_expf.c as one straight line: every path's result is computed and the
// input's class selects it, so lanes of a wave whose inputs take different
// msun paths do not serialise.  The arithmetic of each path is msun's: the
// specials (NaN, overflow, underflow) return what msun returns; with k = 0
// the reduction computes hi = x - 0 = x and lo = +0, the values msun's
// middle path sets; |x| <= 2^-14 gives 1 + x.  The main path runs on 0 in
// place of a special input, so every conversion in it stays in range.
ND_LIBM_FN float nd_expf(float x)
{
    const float ln2_hi = 6.9314575195e-01f;  // 0x3f317200
    const float ln2_lo = 1.4286067653e-06f;  // 0x35bfbe8e
    const float inv_ln2 = 1.4426950216e+00f; // 0x3fb8aa3b
    const float p1 = 1.6666625440e-1f;
    const float p2 = -2.7667332906e-3f;
    const uint32_t bx = nd_f2u(x);
    const int sign = (int)(bx >> 31);
    const uint32_t ax = bx & 0x7fffffffu;
    const int nan = ax > 0x7f800000u;
    const int over = !sign && ax >= 0x42b17218u;  // x >= 88.7228 (and +inf)
    const int under = sign && ax >= 0x42cff1b5u;  // x <= -103.972084 (and -inf)
    const int special = nan | over | under;
    const float xs = special ? 0.0f : x;
    const uint32_t hx = special ? 0u : ax;
    // k: round(x / ln2) past 1.5 ln2 (the +-1/2 a select, not a table in
    // memory), +-1 past ln2 / 2, else 0
    const int kr = (int)(inv_ln2 * xs + (sign ? -0.5f : 0.5f));
    const int k = hx > 0x3eb17218u ? (hx > 0x3f851592u ? kr : 1 - sign - sign) : 0;
    const float kf = (float)k;
    const float hi = xs - kf * ln2_hi;
    const float lo = kf * ln2_lo;
    const float xr = hi - lo;
    const float xx = xr * xr;
    const float c = xr - xx * (p1 + xx * p2);
    const float y = 1.0f + (xr * c / (2.0f - c) - lo + hi);
    // scalbnf(y, k) for the k this range gives (-150..128): one over- or
    // underflow step at most, then the power of two
    const float ys = k > 127 ? y * nd_u2f(0x7f000000u)
                             : (k < -126 ? y * (nd_u2f(0x00800000u) * nd_u2f(0x4b800000u)) : y);
    const int ks = k > 127 ? k - 127 : (k < -126 ? k + 126 - 24 : k);
    float r = k == 0 ? y : ys * nd_u2f((uint32_t)(0x7f + ks) << 23);
    r = hx > 0x39000000u ? r : 1.0f + xs;  // |x| <= 2^-14
    r = under ? 0.0f : r;
    r = over ? x * nd_u2f(0x7f000000u) : r;
    return nan ? x : r;
}

// e_logf.c as one straight line: subnormals are scaled up by 2^25 (k -25)
// before the main path, which runs on 1 in place of zero, negative,
// infinite or NaN input; the input's class selects msun's result: -inf for
// +-0, a NaN for a negative input ((x - x) times infinity, the invalid
// operation msun's (x - x) / 0 is), x for +inf and NaN, an exact 0 for 1.
ND_LIBM_FN float nd_logf(float x)
{
    const float ln2_hi = 6.9313812256e-01f;  // 0x3f317180
    const float ln2_lo = 9.0580006145e-06f;  // 0x3717f7d1
    const float lg1 = 0.66666662693f;
    const float lg2 = 0.40000972152f;
    const float lg3 = 0.28498786688f;
    const float lg4 = 0.24279078841f;
    const uint32_t bx = nd_f2u(x);
    const int zero = (bx << 1) == 0;
    const int neg = (bx >> 31) && !zero;
    const int upper = !(bx >> 31) && bx >= 0x7f800000u;  // +inf, NaN
    const int sub = bx < 0x00800000u && !zero;
    const int one = bx == 0x3f800000u;
    const float xs = (zero | neg | upper) ? 1.0f : (sub ? x * nd_u2f(0x4c000000u) : x);
    uint32_t ix = nd_f2u(xs);
    int k = sub ? -25 : 0;
    ix += 0x3f800000u - 0x3f3504f3u;
    k += (int)(ix >> 23) - 0x7f;
    ix = (ix & 0x007fffffu) + 0x3f3504f3u;
    const float xm = nd_u2f(ix);
    const float f = xm - 1.0f;
    const float s = f / (2.0f + f);
    const float z = s * s;
    const float w = z * z;
    const float t1 = w * (lg2 + w * lg4);
    const float t2 = z * (lg1 + w * lg3);
    const float r = t2 + t1;
    const float hfsq = 0.5f * f * f;
    const float dk = (float)k;
    float v = s * (hfsq + r) + dk * ln2_lo - hfsq + f + dk * ln2_hi;
    v = one ? 0.0f : v;
    v = upper ? x : v;
    v = neg ? (x - x) * nd_u2f(0x7f800000u) : v;
    return zero ? nd_u2f(0xff800000u) : v;
}

ND_LIBM_FN float nd_sigmoidf(float x) { return 1.0f / (1.0f + nd_expf(-x)); }

// ---- powf (e_powf.c) ---------------------------------------------------------

ND_LIBM_FN float nd_powf(float x, float y)
{
    const float bp1 = 1.5f, dp_h1 = 5.84960938e-01f, dp_l1 = 1.56322085e-06f;  // 0x3f15c000, 0x35d1cfdc
    const float two24 = 16777216.0f;
    const float huge = 1.0e30f, tiny = 1.0e-30f;
    // (3/2) (log(x) - 2s - 2/3 s^3) series
    const float L1 = 6.0000002384e-01f, L2 = 4.2857143283e-01f, L3 = 3.3333334327e-01f;
    const float L4 = 2.7272811532e-01f, L5 = 2.3066075146e-01f, L6 = 2.0697501302e-01f;
    const float P1 = 1.6666667163e-01f, P2 = -2.7777778450e-03f, P3 = 6.6137559770e-05f;
    const float P4 = -1.6533901999e-06f, P5 = 4.1381369442e-08f;
    const float lg2 = 6.9314718246e-01f, lg2_h = 6.93145752e-01f, lg2_l = 1.42860654e-06f;
    const float ovt = 4.2995665694e-08f;  // -(128 - log2(ovfl + .5 ulp))
    const float cp = 9.6179670095e-01f, cp_h = 9.6191406250e-01f, cp_l = -1.1736857402e-04f;
    const float ivln2 = 1.4426950216e+00f, ivln2_h = 1.4426879883e+00f,
                ivln2_l = 7.0526075433e-06f;

    const int32_t hx = (int32_t)nd_f2u(x), hy = (int32_t)nd_f2u(y);
    int32_t ix = hx & 0x7fffffff;
    const int32_t iy = hy & 0x7fffffff;

    if (iy == 0) return 1.0f;                  // x^0 = 1
    if (hx == 0x3f800000) return 1.0f;         // 1^y = 1, y NaN too
    if (ix > 0x7f800000 || iy > 0x7f800000) return x + y;  // NaN

    // yisint: 0 y not an integer, 1 odd, 2 even (only needed for x < 0)
    int32_t yisint = 0;
    if (hx < 0) {
        if (iy >= 0x4b800000) {
            yisint = 2;
        } else if (iy >= 0x3f800000) {
            const int32_t k = (iy >> 23) - 0x7f;
            const int32_t j = iy >> (23 - k);
            if ((j << (23 - k)) == iy) yisint = 2 - (j & 1);
        }
    }
    if (iy == 0x7f800000) {                    // y = +-inf
        if (ix == 0x3f800000) return 1.0f;     // (-1)^+-inf = 1
        if (ix > 0x3f800000) return hy >= 0 ? y : 0.0f;
        return hy >= 0 ? 0.0f : -y;
    }
    if (iy == 0x3f800000) return hy >= 0 ? x : 1.0f / x;  // y = +-1
    if (hy == 0x40000000) return x * x;        // y = 2
    if (hy == 0x3f000000 && hx >= 0) return sqrtf(x);  // y = 0.5, x >= +0

    float ax = fabsf(x);
    if (ix == 0x7f800000 || ix == 0 || ix == 0x3f800000) {  // x = +-0, +-inf, +-1
        float z = ax;
        if (hy < 0) z = 1.0f / z;
        if (hx < 0) {
            if (((ix - 0x3f800000) | yisint) == 0)
                z = (z - z) / (z - z);         // (-1)^non-integer = NaN
            else if (yisint == 1)
                z = -z;
        }
        return z;
    }

    float sn = 1.0f;                           // sign of the result
    if (hx < 0) {
        if (yisint == 0) return (x - x) / (x - x);  // (x < 0)^non-integer
        if (yisint == 1) sn = -1.0f;
    }

    float t1, t2;
    if (iy > 0x4d000000) {                     // |y| > 2^27
        if (ix < 0x3f7ffff8) return hy < 0 ? sn * huge * huge : sn * tiny * tiny;
        if (ix > 0x3f800007) return hy > 0 ? sn * huge * huge : sn * tiny * tiny;
        // |1 - x| <= 2^-20: log(x) by x - x^2/2 + x^3/3 - x^4/4
        const float t = ax - 1.0f;
        const float w = (t * t) * (0.5f - t * (3.33333343e-01f - t * 0.25f));
        const float u = ivln2_h * t;
        const float v = t * ivln2_l - w * ivln2;
        t1 = nd_u2f(nd_f2u(u + v) & 0xfffff000u);
        t2 = v - (t1 - u);
    } else {
        int32_t n = 0;
        if (ix < 0x00800000) {                 // subnormal x
            ax *= two24;
            n -= 24;
            ix = (int32_t)nd_f2u(ax);
        }
        n += (ix >> 23) - 0x7f;
        const int32_t j = ix & 0x007fffff;
        int k;
        ix = j | 0x3f800000;                   // |x| scaled into [1, 2)
        if (j <= 0x1cc471) {                   // |x| < sqrt(3/2)
            k = 0;
        } else if (j < 0x5db3d7) {             // |x| < sqrt(3)
            k = 1;
        } else {
            k = 0;
            n += 1;
            ix -= 0x00800000;
        }
        ax = nd_u2f((uint32_t)ix);
        // s = s_h + s_l = (x - 1)/(x + 1) or (x - 1.5)/(x + 1.5)
        const float bpk = k ? bp1 : 1.0f, dphk = k ? dp_h1 : 0.0f, dplk = k ? dp_l1 : 0.0f;
        float u = ax - bpk;
        float v = 1.0f / (ax + bpk);
        const float s = u * v;
        const float s_h = nd_u2f(nd_f2u(s) & 0xfffff000u);
        float t_h = nd_u2f((uint32_t)((((ix >> 1) & 0xfffff000) | 0x20000000) + 0x00400000 +
                                      (k << 21)));
        float t_l = ax - (t_h - bpk);
        const float s_l = v * ((u - s_h * t_h) - s_h * t_l);
        // log(ax)
        float s2 = s * s;
        float r = s2 * s2 * (L1 + s2 * (L2 + s2 * (L3 + s2 * (L4 + s2 * (L5 + s2 * L6)))));
        r += s_l * (s_h + s);
        s2 = s_h * s_h;
        t_h = nd_u2f(nd_f2u(3.0f + s2 + r) & 0xfffff000u);
        t_l = r - ((t_h - 3.0f) - s2);
        u = s_h * t_h;
        v = s_l * t_h + t_l * s;
        // 2/(3 log2) (s + ...)
        const float p_h = nd_u2f(nd_f2u(u + v) & 0xfffff000u);
        const float p_l = v - (p_h - u);
        const float z_h = cp_h * p_h;
        const float z_l = cp_l * p_h + p_l * cp + dplk;
        // log2(ax) = n + dp_h + z_h + z_l
        const float t = (float)n;
        t1 = nd_u2f(nd_f2u(((z_h + z_l) + dphk) + t) & 0xfffff000u);
        t2 = z_l - (((t1 - t) - dphk) - z_h);
    }

    // (y1 + y2)(t1 + t2)
    const float y1 = nd_u2f(nd_f2u(y) & 0xfffff000u);
    const float p_l = (y - y1) * t1 + y * t2;
    float p_h = y1 * t1;
    float z = p_l + p_h;
    int32_t j = (int32_t)nd_f2u(z);
    if (j > 0x43000000) {                      // z > 128
        return sn * huge * huge;
    } else if (j == 0x43000000) {              // z == 128
        if (p_l + ovt > z - p_h) return sn * huge * huge;
    } else if ((j & 0x7fffffff) > 0x43160000) {  // z < -150
        return sn * tiny * tiny;
    } else if ((uint32_t)j == 0xc3160000u) {   // z == -150
        if (p_l <= z - p_h) return sn * tiny * tiny;
    }
    // 2^(p_h + p_l)
    const int32_t i = j & 0x7fffffff;
    int32_t k = (i >> 23) - 0x7f;
    int32_t n = 0;
    if (i > 0x3f000000) {                      // |z| > 0.5: n = [z + 0.5]
        n = j + (0x00800000 >> (k + 1));
        k = ((n & 0x7fffffff) >> 23) - 0x7f;
        const float t = nd_u2f((uint32_t)(n & ~(0x007fffff >> k)));
        n = ((n & 0x007fffff) | 0x00800000) >> (23 - k);
        if (j < 0) n = -n;
        p_h -= t;
    }
    float t = nd_u2f(nd_f2u(p_l + p_h) & 0xffff8000u);
    const float u = t * lg2_h;
    const float v = (p_l - (t - p_h)) * lg2 + t * lg2_l;
    z = u + v;
    const float w = v - (z - u);
    t = z * z;
    t1 = z - t * (P1 + t * (P2 + t * (P3 + t * (P4 + t * P5))));
    const float r = (z * t1) / (t1 - 2.0f) - (w + z * w);
    z = 1.0f - (r - z);
    j = (int32_t)nd_f2u(z);
    j += (int32_t)((uint32_t)n << 23);
    if ((j >> 23) <= 0)
        z = nd_scalbnf(z, n);                  // subnormal result
    else
        z = nd_u2f((uint32_t)j);
    return sn * z;
}

// ---- sinf / cosf (s_sinf.c, s_cosf.c, k_sinf.c, k_cosf.c) ------------------

// sin(x) on |x| <= pi/4 in double: |sin(x)/x - s(x)| < 2^-37.5.
ND_LIBM_FN float nd_k_sinf(double x)
{
    const double S1 = -0x15555554cbac77.0p-55;  // -0.166666666416265235595
    const double S2 = 0x111110896efbb2.0p-59;   //  0.0083333293858894631756
    const double S3 = -0x1a00f9e2cae774.0p-65;  // -0.000198393348360966317347
    const double S4 = 0x16cd878c3b46a7.0p-71;   //  0.0000027183114939898219064
    const double z = x * x;
    const double w = z * z;
    const double r = S3 + z * S4;
    const double s = z * x;
    return (float)((x + s * (S1 + z * S2)) + s * w * r);
}

// cos(x) on |x| <= pi/4 in double: |cos(x) - c(x)| < 2^-34.1.
ND_LIBM_FN float nd_k_cosf(double x)
{
    const double C0 = -0x1ffffffd0c5e81.0p-54;  // -0.499999997251031003120
    const double C1 = 0x155553e1053a42.0p-57;   //  0.0416666233237390631894
    const double C2 = -0x16c087e80f1e27.0p-62;  // -0.00138867637746099294692
    const double C3 = 0x199342e0ee5069.0p-68;   //  0.0000243904487962774090654
    const double z = x * x;
    const double w = z * z;
    const double r = C2 + z * C3;
    return (float)(((1.0 + z * C0) + w * C1) + (w * z) * r);
}

// x * 2^n for the exponents the reduction below produces (no overflow or
// underflow there, so the product is exact, as scalbn's).
ND_LIBM_FN double nd_scalbn_exact(double x, int n)
{
    union {
        double d;
        uint64_t u;
    } v;
    v.u = (uint64_t)(0x3ff + n) << 52;
    return x * v.d;
}

// Payne-Hanek reduction of one 24-bit-chunk input (k_rem_pio2.c with
// nx = 1, prec = 0): returns n mod 8 and y ~ x - n pi/2, x = tx 2^e0.
ND_LIBM_FN int nd_rem_pio2_large(double tx, double *y, int e0)
{
    // 2/pi in 24-bit chunks, most significant first
    const int32_t ipio2[24] = {
        0xA2F983, 0x6E4E44, 0x1529FC, 0x2757D1, 0xF534DD, 0xC0DB62, 0x95993C, 0x439041,
        0xFE5163, 0xABDEBB, 0xC561B7, 0x246E3A, 0x424DD2, 0xE00649, 0x2EEA09, 0xD1921C,
        0xFE1DEB, 0x1CB129, 0xA73EE8, 0x8235F5, 0x2EBB44, 0x84E99C, 0x7026B4, 0x5F7E41};
    // pi/2 in 24-bit chunks
    const double pio2[8] = {
        1.57079625129699707031e+00, 7.54978941586159635335e-08, 5.39030252995776476554e-15,
        3.28200341580791294123e-22, 1.27065575308067607349e-29, 1.22933308981111328932e-36,
        2.73370053816464559624e-44, 2.16741683877804819444e-51};
    const double two24 = 16777216.0, twon24 = 5.9604644775390625e-08;
    const int jk = 3, jp = 3, jx = 0;
    double f[20], fq[20], q[20];
    int32_t iq[20];
    int jv = (e0 - 3) / 24;
    if (jv < 0) jv = 0;
    int q0 = e0 - 24 * (jv + 1);
    for (int i = 0, j = jv - jx; i <= jx + jk; ++i, ++j) f[i] = j < 0 ? 0.0 : (double)ipio2[j];
    for (int i = 0; i <= jk; ++i) q[i] = 0.0 + tx * f[jx + i];
    int jz = jk;
    double z, fw;
    int n, ih;
    for (;;) {
        // distill q[] into iq[], lowest chunk first
        z = q[jz];
        for (int i = 0, j = jz; j > 0; ++i, --j) {
            fw = (double)(int32_t)(twon24 * z);
            iq[i] = (int32_t)(z - two24 * fw);
            z = q[j - 1] + fw;
        }
        z = nd_scalbn_exact(z, q0);
        z -= 8.0 * floor(z * 0.125);
        n = (int32_t)z;
        z -= (double)n;
        ih = 0;
        if (q0 > 0) {
            const int32_t i = iq[jz - 1] >> (24 - q0);
            n += i;
            iq[jz - 1] -= i << (24 - q0);
            ih = iq[jz - 1] >> (23 - q0);
        } else if (q0 == 0) {
            ih = iq[jz - 1] >> 23;
        } else if (z >= 0.5) {
            ih = 2;
        }
        if (ih > 0) {                          // fraction > 0.5: take 1 - q
            n += 1;
            int carry = 0;
            for (int i = 0; i < jz; ++i) {
                const int32_t j = iq[i];
                if (carry == 0) {
                    if (j != 0) {
                        carry = 1;
                        iq[i] = 0x1000000 - j;
                    }
                } else {
                    iq[i] = 0xffffff - j;
                }
            }
            if (q0 == 1) iq[jz - 1] &= 0x7fffff;
            else if (q0 == 2) iq[jz - 1] &= 0x3fffff;
            if (ih == 2) {
                z = 1.0 - z;
                if (carry != 0) z -= nd_scalbn_exact(1.0, q0);
            }
        }
        if (z != 0.0) break;
        int32_t any = 0;
        for (int i = jz - 1; i >= jk; --i) any |= iq[i];
        if (any != 0) break;
        int k = 1;                             // more chunks of 2/pi are needed
        while (iq[jk - k] == 0) ++k;
        for (int i = jz + 1; i <= jz + k; ++i) {
            f[jx + i] = (double)ipio2[jv + i];
            q[i] = 0.0 + tx * f[jx + i];
        }
        jz += k;
    }
    if (z == 0.0) {                            // chop off zero chunks
        jz -= 1;
        q0 -= 24;
        while (iq[jz] == 0) {
            jz -= 1;
            q0 -= 24;
        }
    } else {                                   // split z into 24-bit chunks
        z = nd_scalbn_exact(z, -q0);
        if (z >= two24) {
            fw = (double)(int32_t)(twon24 * z);
            iq[jz] = (int32_t)(z - two24 * fw);
            jz += 1;
            q0 += 24;
            iq[jz] = (int32_t)fw;
        } else {
            iq[jz] = (int32_t)z;
        }
    }
    fw = nd_scalbn_exact(1.0, q0);
    for (int i = jz; i >= 0; --i) {
        q[i] = fw * (double)iq[i];
        fw *= twon24;
    }
    for (int i = jz; i >= 0; --i) {
        fw = 0.0;
        for (int k = 0; k <= jp && k <= jz - i; ++k) fw += pio2[k] * q[i + k];
        fq[jz - i] = fw;
    }
    fw = 0.0;
    for (int i = jz; i >= 0; --i) fw += fq[i];
    *y = ih == 0 ? fw : -fw;
    return n & 7;
}

// x - n pi/2 for |x| > pi/4 (e_rem_pio2f.c); returns n.
ND_LIBM_FN int nd_rem_pio2f(float x, double *y)
{
    const double toint = 1.5 / 2.220446049250313080847e-16;   // 1.5 / DBL_EPSILON
    const double invpio2 = 6.36619772367581382433e-01;        // 53 bits of 2/pi
    const double pio2_1 = 1.57079631090164184570e+00;         // first 25 bits of pi/2
    const double pio2_1t = 1.58932547735281966916e-08;        // pi/2 - pio2_1
    const uint32_t ux = nd_f2u(x);
    const uint32_t ix = ux & 0x7fffffffu;
    if (ix < 0x4dc90fdbu) {                    // |x| < 2^28 pi/2: 25 + 53 bit pi/2
        const double fn = ((double)x * invpio2 + toint) - toint;
        *y = (double)x - fn * pio2_1 - fn * pio2_1t;
        return (int32_t)fn;
    }
    if (ix >= 0x7f800000u) {                   // inf or NaN
        *y = (double)x - (double)x;
        return 0;
    }
    const int e0 = (int)(ix >> 23) - (0x7f + 23);  // |x| = tx 2^e0, tx in [2^23, 2^24)
    const double tx = (double)nd_u2f(ix - ((uint32_t)e0 << 23));
    double ty;
    const int n = nd_rem_pio2_large(tx, &ty, e0);
    if (ux >> 31) {
        *y = -ty;
        return -n;
    }
    *y = ty;
    return n;
}

ND_LIBM_FN float nd_sinf(float x)
{
    const double pio2_1 = 1.57079632679489655800e+00;  // 1 pi/2, 0x3FF921FB54442D18
    const double pio2_2 = 3.14159265358979311600e+00;  // 2 pi/2, 0x400921FB54442D18
    const double pio2_3 = 4.71238898038468967400e+00;  // 3 pi/2, 0x4012D97C7F3321D2
    const double pio2_4 = 6.28318530717958623200e+00;  // 4 pi/2, 0x401921FB54442D18
    const uint32_t ux = nd_f2u(x);
    const int neg = (int)(ux >> 31);
    const uint32_t ix = ux & 0x7fffffffu;
    const double xd = (double)x;
    if (ix <= 0x3f490fdau) {                   // |x| <= pi/4
        if (ix < 0x39800000u) return x;        // |x| < 2^-12
        return nd_k_sinf(xd);
    }
    if (ix <= 0x407b53d1u) {                   // |x| <= 5 pi/4
        if (ix <= 0x4016cbe3u)                 // |x| <= 3 pi/4
            return neg ? -nd_k_cosf(xd + pio2_1) : nd_k_cosf(xd - pio2_1);
        return nd_k_sinf(neg ? -(xd + pio2_2) : -(xd - pio2_2));
    }
    if (ix <= 0x40e231d5u) {                   // |x| <= 9 pi/4
        if (ix <= 0x40afeddfu)                 // |x| <= 7 pi/4
            return neg ? nd_k_cosf(xd + pio2_3) : -nd_k_cosf(xd - pio2_3);
        return nd_k_sinf(neg ? xd + pio2_4 : xd - pio2_4);
    }
    if (ix >= 0x7f800000u) return x - x;       // inf or NaN
    double y;
    const int n = nd_rem_pio2f(x, &y);
    switch (n & 3) {
    case 0: return nd_k_sinf(y);
    case 1: return nd_k_cosf(y);
    case 2: return nd_k_sinf(-y);
    default: return -nd_k_cosf(y);
    }
}

ND_LIBM_FN float nd_cosf(float x)
{
    const double pio2_1 = 1.57079632679489655800e+00;  // 1 pi/2
    const double pio2_2 = 3.14159265358979311600e+00;  // 2 pi/2
    const double pio2_3 = 4.71238898038468967400e+00;  // 3 pi/2
    const double pio2_4 = 6.28318530717958623200e+00;  // 4 pi/2
    const uint32_t ux = nd_f2u(x);
    const int neg = (int)(ux >> 31);
    const uint32_t ix = ux & 0x7fffffffu;
    const double xd = (double)x;
    if (ix <= 0x3f490fdau) {                   // |x| <= pi/4
        if (ix < 0x39800000u) return 1.0f;     // |x| < 2^-12
        return nd_k_cosf(xd);
    }
    if (ix <= 0x407b53d1u) {                   // |x| <= 5 pi/4
        if (ix > 0x4016cbe3u)                  // |x| > 3 pi/4
            return -nd_k_cosf(neg ? xd + pio2_2 : xd - pio2_2);
        return neg ? nd_k_sinf(xd + pio2_1) : nd_k_sinf(pio2_1 - xd);
    }
    if (ix <= 0x40e231d5u) {                   // |x| <= 9 pi/4
        if (ix > 0x40afeddfu)                  // |x| > 7 pi/4
            return nd_k_cosf(neg ? xd + pio2_4 : xd - pio2_4);
        return neg ? nd_k_sinf(-xd - pio2_3) : nd_k_sinf(xd - pio2_3);
    }
    if (ix >= 0x7f800000u) return x - x;       // inf or NaN
    double y;
    const int n = nd_rem_pio2f(x, &y);
    switch (n & 3) {
    case 0: return nd_k_cosf(y);
    case 1: return nd_k_sinf(-y);
    case 2: return -nd_k_cosf(y);
    default: return nd_k_sinf(y);
    }
}
