/*
 * needle_oracle.c -- CPU restatement of needle-rs's Needle-3 hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the CPU
 * baseline bench.py times.  The shipped library never links or calls it.
 *
 * Float order follows the Rust source exactly; build with
 * -ffp-contract=off (rustc never fuses a*b+c) and without -ffast-math.
 * Citations are file:line in the needle-rs checkout.  The pinning status of
 * each function is listed in needle_oracle.h.
 */
#include "needle_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================== */
/* math.rs                                                                  */
/* ======================================================================== */

/* math.rs:53-68: exact binary16 -> f32, subnormals, Inf and NaN payloads. */
float or_f16_to_f32(uint16_t bits)
{
    uint32_t sign = ((uint32_t)(bits >> 15)) << 31;
    uint32_t exp = (bits >> 10) & 0x1F;
    uint32_t mant = bits & 0x3FF;
    uint32_t out;
    float f;
    if (exp == 0) {
        float val = (float)mant / (float)(1u << 24);
        return sign ? -val : val;
    }
    if (exp == 31)
        out = sign | 0x7F800000u | (mant << 13);
    else
        out = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    memcpy(&f, &out, 4);
    return f;
}

/*
 * math.rs:3-11 route exp and ln through libm 0.2.16 (Cargo.lock:267-269),
 * whose expf/logf are the FreeBSD msun algorithms (e_expf.c, e_logf.c, as
 * carried by musl).  Restated here from those published sources; glibc's
 * expf/logf are a different (table-driven) algorithm and can differ in the
 * last bit, which an int8 KV cache can amplify into a flipped code.
 */
static uint32_t bits_of(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float float_of(uint32_t u)
{
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* scalbnf: y * 2^n, with the two-step scaling near the exponent limits. */
static float scale_pow2(float y, int n)
{
    if (n > 127) {
        y *= float_of(0x7f000000u);
        n -= 127;
        if (n > 127) {
            y *= float_of(0x7f000000u);
            n -= 127;
            if (n > 127)
                n = 127;
        }
    } else if (n < -126) {
        y *= float_of(0x00800000u) * float_of(0x4b800000u);
        n += 102;
        if (n < -126) {
            y *= float_of(0x00800000u) * float_of(0x4b800000u);
            n += 102;
            if (n < -126)
                n = -126;
        }
    }
    return y * float_of((uint32_t)(127 + n) << 23);
}

float or_expf(float x)
{
    /* ln2 split so that k*LN2_HI is exact; |r| <= ln2/2 after reduction. */
    const float LN2_HI = float_of(0x3f317200u), LN2_LO = float_of(0x35bfbe8eu);
    const float INV_LN2 = float_of(0x3fb8aa3bu);
    /* remez coefficients of r*(e^r+1)/(e^r-1) on [-ln2/2, ln2/2] */
    const float P1 = float_of(0x3e2aaa8fu), P2 = float_of(0xbb355215u);
    uint32_t ax = bits_of(x);
    int neg = (int)(ax >> 31);
    ax &= 0x7fffffffu;
    if (ax >= 0x42aeac50u) {          /* |x| >= 87.33655 */
        if (ax > 0x7f800000u)
            return x;                 /* NaN */
        if (!neg && ax >= 0x42b17218u)
            return x * float_of(0x7f000000u); /* overflow to +inf */
        if (neg && ax >= 0x42cff1b5u)
            return 0.0f;              /* below -103.972084: underflow */
    }
    int k;
    float hi, lo;
    if (ax > 0x3eb17218u) {           /* |x| > ln2/2 */
        if (ax > 0x3f851592u)         /* |x| > 1.5 ln2 */
            k = (int)(INV_LN2 * x + (neg ? -0.5f : 0.5f));
        else
            k = neg ? -1 : 1;
        hi = x - (float)k * LN2_HI;
        lo = (float)k * LN2_LO;
        x = hi - lo;
    } else if (ax > 0x39000000u) {    /* |x| > 2^-14 */
        k = 0;
        hi = x;
        lo = 0.0f;
    } else {
        return 1.0f + x;
    }
    float xx = x * x;
    float c = x - xx * (P1 + xx * P2);
    float y = 1.0f + (x * c / (2.0f - c) - lo + hi);
    return k ? scale_pow2(y, k) : y;
}

float or_logf(float x)
{
    const float LN2_HI = float_of(0x3f317180u), LN2_LO = float_of(0x3717f7d1u);
    /* |(log(1+s)-log(1-s))/s - Lg(s)| < 2^-34.24 */
    const float LG1 = float_of(0x3f2aaaaau), LG2 = float_of(0x3eccce13u);
    const float LG3 = float_of(0x3e91e9eeu), LG4 = float_of(0x3e789e26u);
    uint32_t ix = bits_of(x);
    int k = 0;
    if (ix < 0x00800000u || (ix >> 31)) {
        if ((ix << 1) == 0)
            return -1.0f / (x * x);   /* log(+-0) = -inf */
        if (ix >> 31)
            return (x - x) / 0.0f;    /* log(x < 0) = NaN */
        k = -25;                      /* subnormal: scale by 2^25 */
        x *= float_of(0x4c000000u);
        ix = bits_of(x);
    } else if (ix >= 0x7f800000u) {
        return x;
    } else if (ix == 0x3f800000u) {
        return 0.0f;
    }
    /* x = 2^k (1 + f) with 1 + f in [sqrt(2)/2, sqrt(2)) */
    ix += 0x3f800000u - 0x3f3504f3u;
    k += (int)(ix >> 23) - 0x7f;
    ix = (ix & 0x007fffffu) + 0x3f3504f3u;
    float f = float_of(ix) - 1.0f;
    float s = f / (2.0f + f);
    float z = s * s;
    float w = z * z;
    float t1 = w * (LG2 + w * LG4);
    float t2 = z * (LG1 + w * LG3);
    float r = t2 + t1;
    float hfsq = 0.5f * f * f;
    float dk = (float)k;
    return s * (hfsq + r) + dk * LN2_LO - hfsq + f + dk * LN2_HI;
}

/*
 * math.rs:13-36 route sin, cos and powf through libm 0.2.16 as well; the
 * RoPE table (model.rs:378-413) is their only caller on the path.  Their
 * single-precision versions are msun's e_powf.c, s_sinf.c / s_cosf.c with
 * the k_sinf.c / k_cosf.c kernels and the e_rem_pio2f.c / k_rem_pio2.c
 * reductions, restated here from those published sources.
 */
static double double_of(uint64_t u)
{
    double d;
    memcpy(&d, &u, 8);
    return d;
}

/* k_sinf.c: sin on [-pi/4, pi/4], |sin(x)/x - s(x)| < 2^-37.5 */
static float kern_sin(double x)
{
    const double S1 = double_of(0xBFC5555554CBAC77ull), S2 = double_of(0x3F811110896EFBB2ull);
    const double S3 = double_of(0xBF2A00F9E2CAE774ull), S4 = double_of(0x3EC6CD878C3B46A7ull);
    double z = x * x, w = z * z, r = S3 + z * S4, s = z * x;
    return (float)((x + s * (S1 + z * S2)) + s * w * r);
}

/* k_cosf.c: cos on [-pi/4, pi/4], |cos(x) - c(x)| < 2^-34.1 */
static float kern_cos(double x)
{
    const double C0 = double_of(0xBFDFFFFFFD0C5E81ull), C1 = double_of(0x3FA55553E1053A42ull);
    const double C2 = double_of(0xBF56C087E80F1E27ull), C3 = double_of(0x3EF99342E0EE5069ull);
    double z = x * x, w = z * z, r = C2 + z * C3;
    return (float)(((1.0 + z * C0) + w * C1) + (w * z) * r);
}

/* k_rem_pio2.c for one input chunk (nx = 1) at prec 0 (jk = jp = 3):
 * x = t * 2^e0 with t an integer below 2^24; returns n mod 8, *y the
 * remainder x - n*pi/2. */
static int rem_pio2_big(double t, int e0, double *y)
{
    /* 2/pi, 24 bits per entry */
    static const int32_t TWO_OVER_PI[24] = {
        0xA2F983, 0x6E4E44, 0x1529FC, 0x2757D1, 0xF534DD, 0xC0DB62,
        0x95993C, 0x439041, 0xFE5163, 0xABDEBB, 0xC561B7, 0x246E3A,
        0x424DD2, 0xE00649, 0x2EEA09, 0xD1921C, 0xFE1DEB, 0x1CB129,
        0xA73EE8, 0x8235F5, 0x2EBB44, 0x84E99C, 0x7026B4, 0x5F7E41};
    /* pi/2, 24 bits per entry */
    static const uint64_t PIO2_BITS[8] = {
        0x3FF921FB40000000ull, 0x3E74442D00000000ull, 0x3CF8469880000000ull,
        0x3B78CC5160000000ull, 0x39F01B8380000000ull, 0x387A252040000000ull,
        0x36E3822280000000ull, 0x3569F31D00000000ull};
    const double T24 = 16777216.0, TM24 = 1.0 / 16777216.0;
    const int JK = 3;
    double f[20], q[20], fq[20], z, w;
    int32_t iq[20];
    int jv = (e0 - 3) / 24, q0, jz, n, ih, i, j, k;
    if (jv < 0)
        jv = 0;
    q0 = e0 - 24 * (jv + 1);
    for (i = 0; i <= JK; i++) {
        j = jv + i;
        f[i] = j < 0 ? 0.0 : (double)TWO_OVER_PI[j];
        q[i] = 0.0 + t * f[i];
    }
    jz = JK;
recompute:
    z = q[jz];
    for (i = 0, j = jz; j > 0; i++, j--) {
        w = (double)(int32_t)(TM24 * z);
        iq[i] = (int32_t)(z - T24 * w);
        z = q[j - 1] + w;
    }
    z = ldexp(z, q0);
    z -= 8.0 * floor(z * 0.125);
    n = (int32_t)z;
    z -= (double)n;
    ih = 0;
    if (q0 > 0) {
        i = iq[jz - 1] >> (24 - q0);
        n += i;
        iq[jz - 1] -= i << (24 - q0);
        ih = iq[jz - 1] >> (23 - q0);
    } else if (q0 == 0) {
        ih = iq[jz - 1] >> 23;
    } else if (z >= 0.5) {
        ih = 2;
    }
    if (ih > 0) {
        int carry = 0;
        n += 1;
        for (i = 0; i < jz; i++) {
            j = iq[i];
            if (carry == 0) {
                if (j != 0) {
                    carry = 1;
                    iq[i] = 0x1000000 - j;
                }
            } else {
                iq[i] = 0xffffff - j;
            }
        }
        if (q0 == 1)
            iq[jz - 1] &= 0x7fffff;
        if (q0 == 2)
            iq[jz - 1] &= 0x3fffff;
        if (ih == 2) {
            z = 1.0 - z;
            if (carry)
                z -= ldexp(1.0, q0);
        }
    }
    if (z == 0.0) {
        j = 0;
        for (i = jz - 1; i >= JK; i--)
            j |= iq[i];
        if (j == 0) {
            for (k = 1; iq[JK - k] == 0; k++)
                ;
            for (i = jz + 1; i <= jz + k; i++) {
                f[i] = (double)TWO_OVER_PI[jv + i];
                q[i] = 0.0 + t * f[i];
            }
            jz += k;
            goto recompute;
        }
    }
    if (z == 0.0) {
        jz--;
        q0 -= 24;
        while (iq[jz] == 0) {
            jz--;
            q0 -= 24;
        }
    } else {
        z = ldexp(z, -q0);
        if (z >= T24) {
            w = (double)(int32_t)(TM24 * z);
            iq[jz] = (int32_t)(z - T24 * w);
            jz++;
            q0 += 24;
            iq[jz] = (int32_t)w;
        } else {
            iq[jz] = (int32_t)z;
        }
    }
    w = ldexp(1.0, q0);
    for (i = jz; i >= 0; i--) {
        q[i] = w * (double)iq[i];
        w *= TM24;
    }
    for (i = jz; i >= 0; i--) {
        w = 0.0;
        for (k = 0; k <= JK && k <= jz - i; k++)
            w += double_of(PIO2_BITS[k]) * q[i + k];
        fq[jz - i] = w;
    }
    w = 0.0;
    for (i = jz; i >= 0; i--)
        w += fq[i];
    *y = ih == 0 ? w : -w;
    return n & 7;
}

/* e_rem_pio2f.c: n and x - n*pi/2 in double. */
static int rem_pio2f(float x, double *y)
{
    const double TOINT = double_of(0x4338000000000000ull);   /* 1.5 * 2^52 */
    const double INV_PIO2 = double_of(0x3FE45F306DC9C883ull);
    const double PIO2_1 = double_of(0x3FF921FB50000000ull);  /* 25 bits */
    const double PIO2_1T = double_of(0x3E5110B4611A6263ull); /* the rest */
    uint32_t u = bits_of(x), ax = u & 0x7fffffffu;
    if (ax < 0x4dc90fdbu) {
        double fn = (double)x * INV_PIO2 + TOINT;
        fn = fn - TOINT;
        *y = (double)x - fn * PIO2_1 - fn * PIO2_1T;
        return (int)fn;
    }
    if (ax >= 0x7f800000u) {
        *y = (double)x - (double)x;
        return 0;
    }
    int e0 = (int)(ax >> 23) - 150;
    double r;
    int n = rem_pio2_big((double)float_of(ax - ((uint32_t)e0 << 23)), e0, &r);
    if (u >> 31) {
        *y = -r;
        return -n;
    }
    *y = r;
    return n;
}

/* s_sinf.c */
float or_sinf(float x)
{
    const double P1 = double_of(0x3FF921FB54442D18ull), P2 = double_of(0x400921FB54442D18ull);
    const double P3 = double_of(0x4012D97C7F3321D2ull), P4 = double_of(0x401921FB54442D18ull);
    uint32_t u = bits_of(x), ax = u & 0x7fffffffu;
    int neg = (int)(u >> 31);
    double d = (double)x, y;
    if (ax <= 0x3f490fdau)
        return ax < 0x39800000u ? x : kern_sin(d);
    if (ax <= 0x407b53d1u) {
        if (ax <= 0x4016cbe3u)
            return neg ? -kern_cos(d + P1) : kern_cos(d - P1);
        return kern_sin(neg ? -(d + P2) : -(d - P2));
    }
    if (ax <= 0x40e231d5u) {
        if (ax <= 0x40afeddfu)
            return neg ? kern_cos(d + P3) : -kern_cos(d - P3);
        return kern_sin(neg ? d + P4 : d - P4);
    }
    if (ax >= 0x7f800000u)
        return x - x;
    int n = rem_pio2f(x, &y) & 3;
    if (n == 0)
        return kern_sin(y);
    if (n == 1)
        return kern_cos(y);
    if (n == 2)
        return kern_sin(-y);
    return -kern_cos(y);
}

/* s_cosf.c */
float or_cosf(float x)
{
    const double P1 = double_of(0x3FF921FB54442D18ull), P2 = double_of(0x400921FB54442D18ull);
    const double P3 = double_of(0x4012D97C7F3321D2ull), P4 = double_of(0x401921FB54442D18ull);
    uint32_t u = bits_of(x), ax = u & 0x7fffffffu;
    int neg = (int)(u >> 31);
    double d = (double)x, y;
    if (ax <= 0x3f490fdau)
        return ax < 0x39800000u ? 1.0f : kern_cos(d);
    if (ax <= 0x407b53d1u) {
        if (ax > 0x4016cbe3u)
            return -kern_cos(neg ? d + P2 : d - P2);
        return neg ? kern_sin(d + P1) : kern_sin(P1 - d);
    }
    if (ax <= 0x40e231d5u) {
        if (ax > 0x40afeddfu)
            return kern_cos(neg ? d + P4 : d - P4);
        return neg ? kern_sin(-d - P3) : kern_sin(d - P3);
    }
    if (ax >= 0x7f800000u)
        return x - x;
    int n = rem_pio2f(x, &y) & 3;
    if (n == 0)
        return kern_cos(y);
    if (n == 1)
        return kern_sin(-y);
    if (n == 2)
        return -kern_cos(y);
    return kern_sin(y);
}

/* Keep the high 20 bits of a float (the 12-bit-mantissa split). */
static float hi20(float v) { return float_of(bits_of(v) & 0xfffff000u); }

/* e_powf.c */
float or_powf(float x, float y)
{
    const float BP[2] = {1.0f, 1.5f};
    const float DP_H[2] = {0.0f, float_of(0x3f15c000u)};
    const float DP_L[2] = {0.0f, float_of(0x35d1cfdcu)};
    const float L1 = float_of(0x3f19999au), L2 = float_of(0x3edb6db7u);
    const float L3 = float_of(0x3eaaaaabu), L4 = float_of(0x3e8ba305u);
    const float L5 = float_of(0x3e6c3255u), L6 = float_of(0x3e53f142u);
    const float P1 = float_of(0x3e2aaaabu), P2 = float_of(0xbb360b61u);
    const float P3 = float_of(0x388ab355u), P4 = float_of(0xb5ddea0eu);
    const float P5 = float_of(0x3331bb4cu);
    const float LG2 = float_of(0x3f317218u), LG2_H = float_of(0x3f317200u);
    const float LG2_L = float_of(0x35bfbe8cu);
    const float OVT = float_of(0x3338aa3cu);
    const float CP = float_of(0x3f76384fu), CP_H = float_of(0x3f764000u);
    const float CP_L = float_of(0xb8f623c6u);
    const float IVLN2 = float_of(0x3fb8aa3bu), IVLN2_H = float_of(0x3fb8aa00u);
    const float IVLN2_L = float_of(0x36eca570u);
    const float BIG = float_of(0x7149f2cau), SMALL = float_of(0x0da24260u); /* 1e30, 1e-30 */
    int32_t hx = (int32_t)bits_of(x), hy = (int32_t)bits_of(y);
    int32_t ix = hx & 0x7fffffff, iy = hy & 0x7fffffff;
    int32_t yisint = 0, n, j, k, i;
    float ax, sn, t1, t2, z, p_h, p_l, t, u, v, w, r;

    if (iy == 0 || hx == 0x3f800000)
        return 1.0f;
    if (ix > 0x7f800000 || iy > 0x7f800000)
        return x + y;
    if (hx < 0) {
        if (iy >= 0x4b800000) {
            yisint = 2;
        } else if (iy >= 0x3f800000) {
            k = (iy >> 23) - 127;
            j = iy >> (23 - k);
            if ((j << (23 - k)) == iy)
                yisint = 2 - (j & 1);
        }
    }
    if (iy == 0x7f800000) {
        if (ix == 0x3f800000)
            return 1.0f;
        if (ix > 0x3f800000)
            return hy >= 0 ? y : 0.0f;
        return hy >= 0 ? 0.0f : -y;
    }
    if (iy == 0x3f800000)
        return hy >= 0 ? x : 1.0f / x;
    if (hy == 0x40000000)
        return x * x;
    if (hy == 0x3f000000 && hx >= 0)
        return sqrtf(x);
    ax = fabsf(x);
    if (ix == 0x7f800000 || ix == 0 || ix == 0x3f800000) {
        z = hy < 0 ? 1.0f / ax : ax;
        if (hx < 0) {
            if (((ix - 0x3f800000) | yisint) == 0)
                z = (z - z) / (z - z);
            else if (yisint == 1)
                z = -z;
        }
        return z;
    }
    sn = 1.0f;
    if (hx < 0) {
        if (yisint == 0)
            return (x - x) / (x - x);
        if (yisint == 1)
            sn = -1.0f;
    }
    if (iy > 0x4d000000) {
        /* |y| > 2^27: overflow or underflow unless |1 - x| <= 2^-20 */
        if (ix < 0x3f7ffff8)
            return hy < 0 ? sn * BIG * BIG : sn * SMALL * SMALL;
        if (ix > 0x3f800007)
            return hy > 0 ? sn * BIG * BIG : sn * SMALL * SMALL;
        t = ax - 1.0f;
        w = (t * t) * (0.5f - t * (float_of(0x3eaaaaabu) - t * 0.25f));
        u = IVLN2_H * t;
        v = t * IVLN2_L - w * IVLN2;
        t1 = hi20(u + v);
        t2 = v - (t1 - u);
    } else {
        float s, s_h, s_l, s2, t_h, t_l, z_h, z_l;
        n = 0;
        if (ix < 0x00800000) {
            ax *= float_of(0x4b800000u);
            n -= 24;
            ix = (int32_t)bits_of(ax);
        }
        n += (ix >> 23) - 127;
        j = ix & 0x007fffff;
        ix = j | 0x3f800000;
        if (j <= 0x1cc471) {
            k = 0;
        } else if (j < 0x5db3d7) {
            k = 1;
        } else {
            k = 0;
            n += 1;
            ix -= 0x00800000;
        }
        ax = float_of((uint32_t)ix);
        u = ax - BP[k];
        v = 1.0f / (ax + BP[k]);
        s = u * v;
        s_h = hi20(s);
        t_h = float_of((uint32_t)((((ix >> 1) & 0xfffff000) | 0x20000000) + 0x00400000 + (k << 21)));
        t_l = ax - (t_h - BP[k]);
        s_l = v * ((u - s_h * t_h) - s_h * t_l);
        s2 = s * s;
        r = s2 * s2 * (L1 + s2 * (L2 + s2 * (L3 + s2 * (L4 + s2 * (L5 + s2 * L6)))));
        r += s_l * (s_h + s);
        s2 = s_h * s_h;
        t_h = hi20(3.0f + s2 + r);
        t_l = r - ((t_h - 3.0f) - s2);
        u = s_h * t_h;
        v = s_l * t_h + t_l * s;
        p_h = hi20(u + v);
        p_l = v - (p_h - u);
        z_h = CP_H * p_h;
        z_l = CP_L * p_h + p_l * CP + DP_L[k];
        t = (float)n;
        t1 = hi20(((z_h + z_l) + DP_H[k]) + t);
        t2 = z_l - (((t1 - t) - DP_H[k]) - z_h);
    }
    {
        float y1 = hi20(y);
        p_l = (y - y1) * t1 + y * t2;
        p_h = y1 * t1;
    }
    z = p_l + p_h;
    j = (int32_t)bits_of(z);
    if (j > 0x43000000)
        return sn * BIG * BIG;
    if (j == 0x43000000) {
        if (p_l + OVT > z - p_h)
            return sn * BIG * BIG;
    } else if ((j & 0x7fffffff) > 0x43160000) {
        return sn * SMALL * SMALL;
    } else if (bits_of(z) == 0xc3160000u) {
        if (p_l <= z - p_h)
            return sn * SMALL * SMALL;
    }
    i = j & 0x7fffffff;
    k = (i >> 23) - 127;
    n = 0;
    if (i > 0x3f000000) {
        n = j + (0x00800000 >> (k + 1));
        k = ((n & 0x7fffffff) >> 23) - 127;
        t = float_of((uint32_t)(n & ~(0x007fffff >> k)));
        n = ((n & 0x007fffff) | 0x00800000) >> (23 - k);
        if (j < 0)
            n = -n;
        p_h -= t;
    }
    t = float_of(bits_of(p_l + p_h) & 0xffff8000u);
    u = t * LG2_H;
    v = (p_l - (t - p_h)) * LG2 + t * LG2_L;
    z = u + v;
    w = v - (z - u);
    t = z * z;
    t1 = z - t * (P1 + t * (P2 + t * (P3 + t * (P4 + t * P5))));
    r = (z * t1) / (t1 - 2.0f) - (w + z * w);
    z = 1.0f - (r - z);
    j = (int32_t)(bits_of(z) + ((uint32_t)n << 23));
    if ((j >> 23) <= 0)
        z = scale_pow2(z, n);
    else
        z = float_of((uint32_t)j);
    return sn * z;
}

void or_sinf_n(const float *x, size_t n, float *y)
{
    for (size_t i = 0; i < n; i++)
        y[i] = or_sinf(x[i]);
}

void or_cosf_n(const float *x, size_t n, float *y)
{
    for (size_t i = 0; i < n; i++)
        y[i] = or_cosf(x[i]);
}

void or_powf_n(const float *x, const float *e, size_t n, float *y)
{
    for (size_t i = 0; i < n; i++)
        y[i] = or_powf(x[i], e[i]);
}

void or_expf_n(const float *x, size_t n, float *y)
{
    for (size_t i = 0; i < n; i++)
        y[i] = or_expf(x[i]);
}

void or_logf_n(const float *x, size_t n, float *y)
{
    for (size_t i = 0; i < n; i++)
        y[i] = or_logf(x[i]);
}

/* ======================================================================== */
/* hadamard.rs                                                              */
/* ======================================================================== */

/* hadamard.rs:24-42: in-place unnormalised Sylvester butterfly. */
void or_fwht(float *x, size_t n)
{
    size_t h = 1;
    while (h < n) {
        for (size_t i = 0; i < n; i += h << 1) {
            for (size_t j = i; j < i + h; j++) {
                float a = x[j];
                float b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
        }
        h <<= 1;
    }
}

/* hadamard.rs:48-55: butterfly, then multiply by 1/sqrt(n). */
void or_fwht_normalized(float *x, size_t n)
{
    or_fwht(x, n);
    float inv = 1.0f / sqrtf((float)n);
    for (size_t i = 0; i < n; i++)
        x[i] *= inv;
}

/* ======================================================================== */
/* cq.rs -- Format A                                                        */
/* ======================================================================== */

#define ACC_LANES 8 /* cq.rs:830 */

/* cq.rs:107-114 */
size_t or_packed_row_bytes(size_t in_padded, uint8_t bits)
{
    size_t eff = bits == OR_TERNARY_RECORD_BITS ? 2 : bits;
    return in_padded * eff / 8;
}

/* cq.rs:914-925: LSB-first field of `bits` at bit offset `bit`. */
uint32_t or_read_bits(const uint8_t *row, size_t bit, size_t bits, uint32_t mask)
{
    size_t byte = bit / 8;
    size_t shift = bit % 8;
    uint32_t lo = row[byte];
    uint32_t hi = (shift + bits > 8) ? row[byte + 1] : 0;
    return ((lo | (hi << 8)) >> shift) & mask;
}

/* cq.rs:948-958: ternary crumb -> trit index. */
static size_t ternary_index(uint32_t code)
{
    switch (code) {
    case 3: return 0;
    case 0: return 1;
    case 1: return 2;
    default: return 1;
    }
}

/* cq.rs:932-964 */
size_t or_build_lut(uint8_t bits, const float *levels, float *lut)
{
    int ternary = bits == OR_TERNARY_RECORD_BITS;
    size_t width = ternary ? 2 : bits;
    size_t per_byte;
    if (width == 2)
        per_byte = 4;
    else if (width == 4)
        per_byte = 2;
    else
        return 0;
    if (!lut)
        return per_byte;
    uint32_t mask = (1u << width) - 1;
    for (size_t byte = 0; byte < 256; byte++) {
        for (size_t k = 0; k < per_byte; k++) {
            uint32_t code = ((uint32_t)byte >> (k * width)) & mask;
            size_t idx = ternary ? ternary_index(code) : code;
            lut[byte * per_byte + k] = levels[idx];
        }
    }
    return per_byte;
}

static int is_pow2(size_t v) { return v && !(v & (v - 1)); }

/* cq.rs:181-238 (with codebook_slice, cq.rs:93-103). */
int or_cq_from_blob(const uint8_t *blob, size_t blob_len, size_t out_feat,
                    size_t in_feat, size_t group, uint8_t bits,
                    const float *codebook, size_t codebook_len, or_cq **out)
{
    float levels[16];
    size_t n_levels;
    *out = NULL;
    if (out_feat == 0 || in_feat == 0)
        return OR_CQ_EMPTY_SHAPE;
    if (group == 0 || group % 8 != 0 || !is_pow2(group) || group > OR_MAX_GROUP)
        return OR_CQ_BAD_GROUP;
    if (bits == OR_TERNARY_RECORD_BITS) {
        float s = 1.2240064f / sqrtf((float)group);
        levels[0] = -s;
        levels[1] = 0.0f;
        levels[2] = s;
        n_levels = 3;
    } else {
        if (codebook_len != OR_CODEBOOK_LEN)
            return OR_CQ_BAD_CODEBOOK_LEN;
        size_t off;
        switch (bits) {
        case 2: off = 0; n_levels = 4; break;
        case 3: off = 4; n_levels = 8; break;
        case 4: off = 12; n_levels = 16; break;
        default: return OR_CQ_UNSUPPORTED_BITS;
        }
        memcpy(levels, codebook + off, n_levels * sizeof(float));
    }
    size_t in_padded = (in_feat + group - 1) / group * group;
    size_t num_groups = in_padded / group;
    size_t row_bytes = or_packed_row_bytes(in_padded, bits);
    size_t n_packed = out_feat * row_bytes;
    size_t n_norm_bytes = out_feat * num_groups * 2;
    if (blob_len < n_packed + n_norm_bytes)
        return OR_CQ_SHORT_BLOB;

    or_cq *w = calloc(1, sizeof(*w));
    w->packed = malloc(n_packed ? n_packed : 1);
    memcpy(w->packed, blob, n_packed);
    w->norms = malloc(out_feat * num_groups * sizeof(float));
    for (size_t i = 0; i < out_feat * num_groups; i++) {
        const uint8_t *c = blob + n_packed + 2 * i;
        w->norms[i] = or_f16_to_f32((uint16_t)(c[0] | (c[1] << 8)));
    }
    w->per_byte = or_build_lut(bits, levels, NULL);
    if (w->per_byte) {
        w->lut = malloc(256 * w->per_byte * sizeof(float));
        or_build_lut(bits, levels, w->lut);
    }
    w->row_bytes = row_bytes;
    w->num_groups = num_groups;
    w->out_feat = out_feat;
    w->in_feat = in_feat;
    w->in_padded = in_padded;
    w->group = group;
    w->bits = bits;
    memcpy(w->levels, levels, sizeof(levels));
    w->n_levels = n_levels;
    *out = w;
    return OR_CQ_OK;
}

void or_cq_free(or_cq *w)
{
    if (!w)
        return;
    free(w->packed);
    free(w->norms);
    free(w->lut);
    free(w);
}

/* cq.rs:264-274: copy, zero the padded tail, normalised FWHT per group. */
void or_cq_prepare_input(const or_cq *w, const float *x, float *xh)
{
    memcpy(xh, x, w->in_feat * sizeof(float));
    for (size_t i = w->in_feat; i < w->in_padded; i++)
        xh[i] = 0.0f;
    for (size_t g = 0; g < w->num_groups; g++)
        or_fwht_normalized(xh + g * w->group, w->group);
}

/* The eight accumulator lanes as one vector: `lanes += v * xs` is eight
 * independent IEEE multiplies and then eight adds (no contraction), lane k's
 * arithmetic exactly that of `lanes[k] += vals[k] * xs[k]`. */
typedef float or_lanes8 __attribute__((vector_size(ACC_LANES * sizeof(float))));
typedef float or_lanes4 __attribute__((vector_size(4 * sizeof(float))));

/* cq.rs:838-873: eight-lane packed dot of one group, lanes summed 0..7.
 * Always inlined and called with a literal P (4 or 2), as the reference's
 * `dot_group::<P>` is a const generic, so the loops unroll and the lane
 * update runs as vector multiplies and then vector adds (no FMA): lane k's
 * arithmetic is exactly `lanes[k] += vals[k] * xs[k]`.  For P = 4 the eight
 * lanes are two 4-wide halves (one byte's LUT entry each); for P = 2 the
 * four entries of 2 are copied into one 8-wide vector. */
static inline __attribute__((always_inline)) float
dot_group(const size_t P, const float *lut, const uint8_t *gbytes, size_t nbytes,
          const float *gx)
{
    const size_t per_iter = ACC_LANES / P;
    or_lanes4 lo = {0}, hi = {0};
    or_lanes8 lanes = {0};
    size_t full = nbytes - nbytes % per_iter;
    size_t bi = 0;
    while (bi < full) {
        const float *xp = gx + bi * P;
        if (P == 4) {
            or_lanes4 a, b, xa, xb;
            memcpy(&a, lut + (size_t)gbytes[bi] * 4, sizeof a);
            memcpy(&b, lut + (size_t)gbytes[bi + 1] * 4, sizeof b);
            memcpy(&xa, xp, sizeof xa);
            memcpy(&xb, xp + 4, sizeof xb);
            lo += a * xa;
            hi += b * xb;
        } else {
            float vals[ACC_LANES];
            for (size_t t = 0; t < per_iter; t++)
                memcpy(vals + t * P, lut + (size_t)gbytes[bi + t] * P, P * sizeof(float));
            or_lanes8 v, xs;
            memcpy(&v, vals, sizeof v);
            memcpy(&xs, xp, sizeof xs);
            lanes += v * xs;
        }
        bi += per_iter;
    }
    float acc = 0.0f;
    if (P == 4) {
        for (size_t k = 0; k < 4; k++)
            acc += lo[k];
        for (size_t k = 0; k < 4; k++)
            acc += hi[k];
    } else {
        for (size_t k = 0; k < ACC_LANES; k++)
            acc += lanes[k];
    }
    for (size_t b = bi; b < nbytes; b++) {
        size_t base = (size_t)gbytes[b] * P;
        for (size_t k = 0; k < P; k++)
            acc += lut[base + k] * gx[b * P + k];
    }
    return acc;
}

/* ------------------------------------------------------------------------ */
/* Threads.  The reference splits a call across its rayon pool only past     */
/* fixed size rules (cq.rs:301-323, 446-472, 474-581; constants :815-823);   */
/* each row's (or batch row's) arithmetic is unchanged, so every split is    */
/* bit-identical to the serial loop.  OR_SPLIT_REFERENCE applies those rules */
/* (the CPU baseline); OR_SPLIT_ALL also splits every smaller row loop and    */
/* attention's heads, for a faster checker with the same bits.               */
/* ------------------------------------------------------------------------ */

#define MIN_PAR_ROWS 64   /* cq.rs:815 */
#define MIN_PAR_BATCH 8   /* cq.rs:819 */
#define PAR_MIN_MACS ((size_t)1 << 20) /* cq.rs:823 */

static int or_threads = 1;
static int or_split = OR_SPLIT_REFERENCE;

void or_set_threads(int threads, int split)
{
    or_threads = threads > 0 ? threads : 1;
    or_split = split;
}

int or_get_threads(void) { return or_threads; }

static size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

/* cq.rs:721-735: `matvec_lut_impl::<P>`, instantiated below for P = 4 and
 * P = 2 (matvec_lut::<4|2>, cq.rs:693-709). */
static inline __attribute__((always_inline)) void
matvec_rows_lut(const size_t P, const or_cq *w, const float *xh, size_t row_start,
                size_t rows, float *y)
{
    const size_t bpg = w->group / P;
    const float *lut = w->lut;
    for (size_t yi = 0; yi < rows; yi++) {
        size_t o = row_start + yi;
        const uint8_t *row = w->packed + o * w->row_bytes;
        const float *rn = w->norms + o * w->num_groups;
        float total = 0.0f;
        for (size_t g = 0; g < w->num_groups; g++)
            total += rn[g] * dot_group(P, lut, row + g * bpg, bpg, xh + g * w->group);
        y[yi] = total;
    }
}

static void matvec_rows_lut4(const or_cq *w, const float *xh, size_t row_start,
                             size_t rows, float *y)
{
    matvec_rows_lut(4, w, xh, row_start, rows, y);
}

static void matvec_rows_lut2(const or_cq *w, const float *xh, size_t row_start,
                             size_t rows, float *y)
{
    matvec_rows_lut(2, w, xh, row_start, rows, y);
}

/* cq.rs:738-757: bit-at-a-time path for 3-bit rows. */
static void matvec_rows_generic(const or_cq *w, const float *xh, size_t row_start,
                                size_t rows, float *y)
{
    size_t bits = w->bits;
    uint32_t mask = (1u << bits) - 1;
    for (size_t yi = 0; yi < rows; yi++) {
        size_t o = row_start + yi;
        const uint8_t *row = w->packed + o * w->row_bytes;
        const float *rn = w->norms + o * w->num_groups;
        float total = 0.0f;
        for (size_t g = 0; g < w->num_groups; g++) {
            const float *gx = xh + g * w->group;
            float acc = 0.0f;
            for (size_t k = 0; k < w->group; k++) {
                size_t bit = (g * w->group + k) * bits;
                uint32_t idx = or_read_bits(row, bit, bits, mask);
                acc += w->levels[idx] * gx[k];
            }
            total += rn[g] * acc;
        }
        y[yi] = total;
    }
}

/* cq.rs:713-735 dispatch on the packing (per_byte 4, 2, or 0 for 3-bit). */
static void matvec_rows_serial(const or_cq *w, const float *xh,
                               size_t row_start, size_t rows, float *y)
{
    if (w->per_byte == 4)
        matvec_rows_lut4(w, xh, row_start, rows, y);
    else if (w->per_byte == 2)
        matvec_rows_lut2(w, xh, row_start, rows, y);
    else
        matvec_rows_generic(w, xh, row_start, rows, y);
}

/* cq.rs:301-323: rows split into bands of max(ceil(rows/threads), 64) when
 * should_parallelise (rows >= 128 and rows*in_padded >= 2^20, :474-484). */
void or_cq_matvec_rows_prepared(const or_cq *w, const float *xh,
                                size_t row_start, size_t rows, float *y)
{
    int split;
    size_t chunk;
    if (or_split == OR_SPLIT_ALL) {
        split = rows >= 2 && rows * w->in_padded >= 4096;
        chunk = div_ceil(rows, (size_t)or_threads);
    } else {
        split = rows >= 2 * MIN_PAR_ROWS && rows * w->in_padded >= PAR_MIN_MACS;
        chunk = div_ceil(rows, (size_t)or_threads);
        if (chunk < MIN_PAR_ROWS)
            chunk = MIN_PAR_ROWS;
    }
    if (or_threads <= 1 || !split) {
        matvec_rows_serial(w, xh, row_start, rows, y);
        return;
    }
    long bands = (long)div_ceil(rows, chunk);
#pragma omp parallel for num_threads(or_threads) schedule(static, 1)
    for (long b = 0; b < bands; b++) {
        size_t r0 = (size_t)b * chunk;
        size_t n = rows - r0 < chunk ? rows - r0 : chunk;
        matvec_rows_serial(w, xh, row_start + r0, n, y + r0);
    }
}

/* cq.rs:283-287 */
void or_cq_matvec(const or_cq *w, const float *x, float *y)
{
    float *xh = malloc(w->in_padded * sizeof(float));
    or_cq_prepare_input(w, x, xh);
    or_cq_matvec_rows_prepared(w, xh, 0, w->out_feat, y);
    free(xh);
}

/* cq.rs:393-426: the crate's own single-accumulator reference. */
void or_cq_matvec_prepared_reference(const or_cq *w, const float *xh, float *y)
{
    size_t bits = w->bits == OR_TERNARY_RECORD_BITS ? 2 : w->bits;
    uint32_t mask = (1u << bits) - 1;
    for (size_t o = 0; o < w->out_feat; o++) {
        const uint8_t *row = w->packed + o * w->row_bytes;
        float total = 0.0f;
        for (size_t g = 0; g < w->num_groups; g++) {
            float norm = w->norms[o * w->num_groups + g];
            float acc = 0.0f;
            for (size_t k = 0; k < w->group; k++) {
                uint32_t code = or_read_bits(row, (g * w->group + k) * bits, bits, mask);
                size_t idx = w->bits == OR_TERNARY_RECORD_BITS ? ternary_index(code) : code;
                acc += w->levels[idx] * xh[g * w->group + k];
            }
            total += norm * acc;
        }
        y[o] = total;
    }
}

/* cq.rs:791-809: levels * norm for one group, before the rotation.  The
 * byte-LUT widths go through decode_group_lut with a literal P, so the
 * per-byte loop unrolls; the products are the same either way. */
static inline __attribute__((always_inline)) void
decode_group_lut(const size_t P, const float *lut, const uint8_t *gb, size_t bpg,
                 float norm, float *buf)
{
    for (size_t bi = 0; bi < bpg; bi++)
        for (size_t k = 0; k < P; k++)
            buf[bi * P + k] = lut[(size_t)gb[bi] * P + k] * norm;
}

static void decode_group(const or_cq *w, const uint8_t *row, size_t g,
                         float norm, float *buf)
{
    if (w->per_byte == 4) {
        size_t bpg = w->group / 4;
        decode_group_lut(4, w->lut, row + g * bpg, bpg, norm, buf);
    } else if (w->per_byte == 2) {
        size_t bpg = w->group / 2;
        decode_group_lut(2, w->lut, row + g * bpg, bpg, norm, buf);
    } else {
        size_t bits = w->bits;
        uint32_t mask = (1u << bits) - 1;
        for (size_t k = 0; k < w->group; k++) {
            uint32_t idx = or_read_bits(row, (g * w->group + k) * bits, bits, mask);
            buf[k] = w->levels[idx] * norm;
        }
    }
}

/* cq.rs:879-895 */
static float group_dot_lanes(const float *u, const float *x, size_t n)
{
    size_t chunks = n / ACC_LANES;
    or_lanes8 lanes = {0};
    for (size_t c = 0; c < chunks; c++) {
        or_lanes8 uu, xx;
        memcpy(&uu, u + c * ACC_LANES, sizeof uu);
        memcpy(&xx, x + c * ACC_LANES, sizeof xx);
        lanes += uu * xx;
    }
    float s = 0.0f;
    for (size_t k = 0; k < ACC_LANES; k++)
        s += lanes[k];
    for (size_t k = chunks * ACC_LANES; k < n; k++)
        s += u[k] * x[k];
    return s;
}

/* cq.rs:899-906 */
static float group_dot_serial(const float *u, const float *x, size_t n)
{
    float s = 0.0f;
    for (size_t k = 0; k < n; k++)
        s += u[k] * x[k];
    return s;
}

/* cq.rs:632-679: decode each group once (norm 1.0), dot with every batch
 * row in the matvec's lane order, acc[b] += norm * s; batch-major output
 * with row stride `ystride` (the caller's `rows`). */
static void matmul_rows_serial(const or_cq *w, const float *xh, size_t batch,
                               size_t row_start, size_t rows, float *y, size_t ystride)
{
    size_t stride = w->in_padded;
    float ug[OR_MAX_GROUP];
    float *acc = malloc((batch ? batch : 1) * sizeof(float));
    int lanewise = w->per_byte != 0;
    for (size_t r = 0; r < rows; r++) {
        size_t o = row_start + r;
        const uint8_t *row = w->packed + o * w->row_bytes;
        const float *rn = w->norms + o * w->num_groups;
        for (size_t b = 0; b < batch; b++)
            acc[b] = 0.0f;
        for (size_t g = 0; g < w->num_groups; g++) {
            decode_group(w, row, g, 1.0f, ug);
            size_t base = g * w->group;
            for (size_t b = 0; b < batch; b++) {
                const float *gx = xh + b * stride + base;
                float s = lanewise ? group_dot_lanes(ug, gx, w->group)
                                   : group_dot_serial(ug, gx, w->group);
                acc[b] += rn[g] * s;
            }
        }
        for (size_t b = 0; b < batch; b++)
            y[b * ystride + r] = acc[b];
    }
    free(acc);
}

/* cq.rs:446-472: past 2^20 multiply-adds, row bands of
 * max(ceil(rows/threads), 64) when rows >= 128 (:494-544), else batch bands
 * of max(ceil(batch/threads), 8) when batch >= 16 (:552-581). */
void or_cq_matmul_rows_prepared(const or_cq *w, const float *xh, size_t batch,
                                size_t row_start, size_t rows, float *y)
{
    size_t work = rows * batch * w->in_padded;
    int all = or_split == OR_SPLIT_ALL;
    int big = all ? work >= 4096 : work >= PAR_MIN_MACS;
    if (or_threads > 1 && big && rows >= (all ? 2 : 2 * MIN_PAR_ROWS)) {
        size_t chunk = div_ceil(rows, (size_t)or_threads);
        if (!all && chunk < MIN_PAR_ROWS)
            chunk = MIN_PAR_ROWS;
        long bands = (long)div_ceil(rows, chunk);
#pragma omp parallel for num_threads(or_threads) schedule(static, 1)
        for (long b = 0; b < bands; b++) {
            size_t r0 = (size_t)b * chunk;
            size_t n = rows - r0 < chunk ? rows - r0 : chunk;
            matmul_rows_serial(w, xh, batch, row_start + r0, n, y + r0, rows);
        }
        return;
    }
    if (or_threads > 1 && big && batch >= (all ? 2 : 2 * MIN_PAR_BATCH)) {
        size_t band = div_ceil(batch, (size_t)or_threads);
        if (!all && band < MIN_PAR_BATCH)
            band = MIN_PAR_BATCH;
        long bands = (long)div_ceil(batch, band);
#pragma omp parallel for num_threads(or_threads) schedule(static, 1)
        for (long b = 0; b < bands; b++) {
            size_t b0 = (size_t)b * band;
            size_t n = batch - b0 < band ? batch - b0 : band;
            matmul_rows_serial(w, xh + b0 * w->in_padded, n, row_start, rows, y + b0 * rows, rows);
        }
        return;
    }
    matmul_rows_serial(w, xh, batch, row_start, rows, y, rows);
}

/* cq.rs:763-779: u = levels * norm, FWHT per group, truncate to in_feat. */
void or_cq_dequantize_row(const or_cq *w, size_t o, float *out)
{
    const uint8_t *row = w->packed + o * w->row_bytes;
    const float *rn = w->norms + o * w->num_groups;
    float *buf = malloc(w->group * sizeof(float));
    for (size_t g = 0; g < w->num_groups; g++) {
        decode_group(w, row, g, rn[g], buf);
        or_fwht_normalized(buf, w->group);
        size_t base = g * w->group;
        for (size_t k = 0; k < w->group; k++)
            if (base + k < w->in_feat)
                out[base + k] = buf[k];
    }
    free(buf);
}

/* ======================================================================== */
/* Format B: y[o] = sum_k cb[o/64][W[o,k]] * x[k].  No reference function   */
/* exists; this is the closed form, summed in k order.                      */
/* ======================================================================== */

void or_cb8_gemv(const uint8_t *w, const float *cb, const float *x, float *y,
                 size_t out, size_t in)
{
    for (size_t o = 0; o < out; o++) {
        const float *c = cb + (o / 64) * 256;
        const uint8_t *row = w + o * in;
        float acc = 0.0f;
        for (size_t k = 0; k < in; k++)
            acc += c[row[k]] * x[k];
        y[o] = acc;
    }
}

/* The same rows split across OpenMP threads (each row's arithmetic is
 * unchanged, as the reference's rayon row bands are, cq.rs:314-323). */
void or_cb8_gemv_omp(const uint8_t *w, const float *cb, const float *x,
                     float *y, size_t out, size_t in)
{
    long n = (long)out;
#pragma omp parallel for schedule(static)
    for (long o = 0; o < n; o++) {
        const float *c = cb + ((size_t)o / 64) * 256;
        const uint8_t *row = w + (size_t)o * in;
        float acc = 0.0f;
        for (size_t k = 0; k < in; k++)
            acc += c[row[k]] * x[k];
        y[o] = acc;
    }
}

/* The closed-form GEMM with output rows split across threads in bands,
 * as the reference's matmul_rows_par splits its row bands (cq.rs:494-544);
 * each output keeps or_cb8_gemm's k-order sum, so the bits are the same. */
void or_cb8_gemm_omp(const float *x, const uint8_t *w, const float *cb, float *y,
                     size_t m, size_t out, size_t in, int threads)
{
    long n = (long)out;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (long o = 0; o < n; o++) {
        const float *c = cb + ((size_t)o / 64) * 256;
        const uint8_t *row = w + (size_t)o * in;
        for (size_t i = 0; i < m; i++) {
            const float *xi = x + i * in;
            float acc = 0.0f;
            for (size_t k = 0; k < in; k++)
                acc += c[row[k]] * xi[k];
            y[i * out + (size_t)o] = acc;
        }
    }
}

void or_cb8_gemv_f64(const uint8_t *w, const float *cb, const float *x,
                     double *y, size_t out, size_t in)
{
    for (size_t o = 0; o < out; o++) {
        const float *c = cb + (o / 64) * 256;
        double acc = 0.0;
        for (size_t k = 0; k < in; k++)
            acc += (double)c[w[o * in + k]] * (double)x[k];
        y[o] = acc;
    }
}

void or_cb8_gemm(const float *x, const uint8_t *w, const float *cb, float *y,
                 size_t m, size_t out, size_t in)
{
    for (size_t i = 0; i < m; i++)
        or_cb8_gemv(w, cb, x + i * in, y + i * out, out, in);
}

/* Format B through the reference's LUT-kernel shape, for the CPU baseline
 * (the format has no reference function; these are what its CPU path would
 * be).  GEMV: dot_group with one level per byte (cq.rs:838-873, P = 1):
 * eight accumulator lanes, element k into lane k % 8, lanes summed 0..7,
 * rows in bands over `threads` (cq.rs:314-323).  GEMM: matmul_rows_prepared's
 * order (cq.rs:632-679): each weight row decoded once through its codebook,
 * then dotted with every activation row by group_dot_lanes (cq.rs:879-895).
 * Both sum in a different order from or_cb8_gemv, so they agree with it to
 * float rounding, not bit for bit. */
static void cb8_row_lanes(const float *c, const uint8_t *row, const float *x, size_t in,
                          float *y)
{
    or_lanes8 lanes = {0};
    size_t full = in - in % ACC_LANES, k = 0;
    for (; k < full; k += ACC_LANES) {
        float vals[ACC_LANES];
        for (size_t t = 0; t < ACC_LANES; t++)
            vals[t] = c[row[k + t]];
        or_lanes8 v, xs;
        memcpy(&v, vals, sizeof v);
        memcpy(&xs, x + k, sizeof xs);
        lanes += v * xs;
    }
    float acc = 0.0f;
    for (size_t t = 0; t < ACC_LANES; t++)
        acc += lanes[t];
    for (; k < in; k++)
        acc += c[row[k]] * x[k];
    *y = acc;
}

void or_cb8_gemv_lanes(const uint8_t *w, const float *cb, const float *x, float *y,
                       size_t out, size_t in, int threads)
{
    long n = (long)out;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (long o = 0; o < n; o++)
        cb8_row_lanes(cb + ((size_t)o / 64) * 256, w + (size_t)o * in, x, in, y + o);
}

void or_cb8_gemm_lanes(const float *x, const uint8_t *w, const float *cb, float *y,
                       size_t m, size_t out, size_t in, int threads)
{
    long n = (long)out;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        float *u = malloc((in ? in : 1) * sizeof(float));
#pragma omp for schedule(static)
        for (long o = 0; o < n; o++) {
            const float *c = cb + ((size_t)o / 64) * 256;
            const uint8_t *row = w + (size_t)o * in;
            for (size_t k = 0; k < in; k++)
                u[k] = c[row[k]];
            for (size_t i = 0; i < m; i++)
                y[i * out + (size_t)o] = group_dot_lanes(u, x + i * in, in);
        }
        free(u);
    }
}

/* ======================================================================== */
/* v3/cache.rs                                                              */
/* ======================================================================== */

/* cache.rs:80-91 */
static void quant_scale(const float *x, size_t n, uint32_t bits, float *scale,
                        float *inv, float *qmax)
{
    *qmax = (float)((1u << (bits - 1)) - 1);
    float absmax = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float a = x[i] < 0.0f ? -x[i] : x[i];
        if (a > absmax)
            absmax = a;
    }
    *scale = absmax > 0.0f ? absmax / *qmax : 1.0f;
    *inv = 1.0f / *scale;
}

static float clampf(float v, float lo, float hi)
{
    return v < lo ? lo : (v > hi ? hi : v);
}

/* cache.rs:68-73; math::round is libm::roundf, half away from zero. */
void or_fake_quant_vec(float *x, size_t n, uint32_t bits)
{
    float scale, inv, qmax;
    quant_scale(x, n, bits, &scale, &inv, &qmax);
    for (size_t i = 0; i < n; i++)
        x[i] = clampf(roundf(x[i] * inv), -qmax - 1.0f, qmax) * scale;
}

/* cache.rs:98-104 */
float or_quant_into(const float *src, size_t n, int8_t *dst)
{
    float scale, inv, qmax;
    quant_scale(src, n, 8, &scale, &inv, &qmax);
    for (size_t i = 0; i < n; i++)
        dst[i] = (int8_t)clampf(roundf(src[i] * inv), -qmax - 1.0f, qmax);
    return scale;
}

/* cache.rs:113-122 */
void or_quantize_rows(const float *x, size_t rows, size_t head_dim,
                      int8_t *ints, float *scales)
{
    for (size_t r = 0; r < rows; r++)
        scales[r] = or_quant_into(x + r * head_dim, head_dim, ints + r * head_dim);
}

/* v3/model.rs:99-106 */
void or_quant_rows(float *x, size_t seq, size_t heads, size_t head_dim)
{
    for (size_t t = 0; t < seq; t++)
        for (size_t h = 0; h < heads; h++)
            or_fake_quant_vec(x + (t * heads + h) * head_dim, head_dim, 8);
}

/* cache.rs:177-238 (one layer): slots = hint.min(cap), cap = window or
 * max_seq_len. */
or_ring *or_ring_new(int int8, size_t num_kv_heads, size_t qk, size_t vd,
                     size_t hint, size_t window, size_t max_seq_len)
{
    or_ring *r = calloc(1, sizeof(*r));
    if (hint < 1)
        hint = 1;
    if (hint > max_seq_len)
        hint = max_seq_len;
    r->int8 = int8;
    r->num_kv_heads = num_kv_heads;
    r->qk_head_dim = qk;
    r->v_head_dim = vd;
    r->window = window;
    r->cap = window ? (window < max_seq_len ? window : max_seq_len) : max_seq_len;
    r->slots = hint < r->cap ? hint : r->cap;
    size_t kd = num_kv_heads * qk, vdim = num_kv_heads * vd;
    size_t heads = r->slots * num_kv_heads;
    if (int8) {
        r->kq = calloc(r->slots * kd, 1);
        r->vq = calloc(r->slots * vdim, 1);
        r->k_scale = malloc(heads * sizeof(float));
        r->v_scale = malloc(heads * sizeof(float));
        for (size_t i = 0; i < heads; i++)
            r->k_scale[i] = r->v_scale[i] = 1.0f;
    } else {
        r->k = calloc(r->slots * kd, sizeof(float));
        r->v = calloc(r->slots * vdim, sizeof(float));
    }
    return r;
}

void or_ring_free(or_ring *r)
{
    if (!r)
        return;
    free(r->k);
    free(r->v);
    free(r->kq);
    free(r->vq);
    free(r->k_scale);
    free(r->v_scale);
    free(r);
}

/* cache.rs:291-309: grow by doubling to the cap; new scales start at 1. */
static void ring_ensure(or_ring *r, size_t pos)
{
    if (pos < r->slots || r->slots >= r->cap)
        return;
    size_t want = r->slots * 2;
    if (want < pos + 1)
        want = pos + 1;
    if (want > r->cap)
        want = r->cap;
    size_t kd = r->num_kv_heads * r->qk_head_dim, vdim = r->num_kv_heads * r->v_head_dim;
    if (r->int8) {
        r->kq = realloc(r->kq, want * kd);
        memset(r->kq + r->slots * kd, 0, (want - r->slots) * kd);
        r->vq = realloc(r->vq, want * vdim);
        memset(r->vq + r->slots * vdim, 0, (want - r->slots) * vdim);
        r->k_scale = realloc(r->k_scale, want * r->num_kv_heads * sizeof(float));
        r->v_scale = realloc(r->v_scale, want * r->num_kv_heads * sizeof(float));
        for (size_t i = r->slots * r->num_kv_heads; i < want * r->num_kv_heads; i++)
            r->k_scale[i] = r->v_scale[i] = 1.0f;
    } else {
        r->k = realloc(r->k, want * kd * sizeof(float));
        memset(r->k + r->slots * kd, 0, (want - r->slots) * kd * sizeof(float));
        r->v = realloc(r->v, want * vdim * sizeof(float));
        memset(r->v + r->slots * vdim, 0, (want - r->slots) * vdim * sizeof(float));
    }
    r->slots = want;
}

/* cache.rs:346-379 */
void or_ring_write_kv(or_ring *r, size_t pos, const float *k, const float *v)
{
    ring_ensure(r, pos);
    size_t qk = r->qk_head_dim, vh = r->v_head_dim, H = r->num_kv_heads;
    size_t kd = H * qk, vdim = H * vh;
    size_t slot = pos % r->slots;
    if (!r->int8) {
        memcpy(r->k + slot * kd, k, kd * sizeof(float));
        memcpy(r->v + slot * vdim, v, vdim * sizeof(float));
        return;
    }
    size_t base = slot * H;
    for (size_t h = 0; h < H; h++) {
        r->k_scale[base + h] = or_quant_into(k + h * qk, qk, r->kq + slot * kd + h * qk);
        r->v_scale[base + h] = or_quant_into(v + h * vh, vh, r->vq + slot * vdim + h * vh);
    }
}

/* cache.rs:322-331 */
void or_ring_span(const or_ring *r, size_t pos, size_t *lo, size_t *hi)
{
    size_t l = 0;
    if (r->window && pos + 1 > r->window)
        l = pos + 1 - r->window;
    size_t clamp = pos + 1 > r->slots ? pos + 1 - r->slots : 0;
    *lo = l > clamp ? l : clamp;
    *hi = pos;
}

/* ======================================================================== */
/* v3/attention.rs                                                          */
/* ======================================================================== */

/* F32View::dot / Int8View::dot (attention.rs:171-177, 200-207). */
static float dot_f32(const float *q, const float *k, size_t n)
{
    float a = 0.0f;
    for (size_t i = 0; i < n; i++)
        a += q[i] * k[i];
    return a;
}

static float dot_i8(const float *q, const int8_t *k, size_t n, float scale)
{
    float a = 0.0f;
    for (size_t i = 0; i < n; i++)
        a += q[i] * (float)k[i];
    return a * scale;
}

/* attention.rs:327-377, generic over the view via two pointers. */
static void attend_step_impl(const float *q, const float *kf, const float *vf,
                             const int8_t *kq, const float *ks,
                             const int8_t *vq, const float *vs, size_t slots,
                             size_t lo, size_t hi, const or_attn_dims *d,
                             float *out)
{
    float scale = 1.0f / sqrtf((float)d->qk_head_dim);
    size_t repeat = d->num_heads / d->num_kv_heads;
    size_t span = hi - lo + 1;
    size_t QK = d->qk_head_dim, VD = d->v_head_dim, H = d->num_kv_heads;
    /* Heads are independent; the checker's split runs them on threads. */
    int par = or_threads > 1 && or_split == OR_SPLIT_ALL && span * d->num_heads >= 4096;
#pragma omp parallel for num_threads(or_threads) schedule(static, 1) if (par)
    for (long hh = 0; hh < (long)d->num_heads; hh++) {
        size_t h = (size_t)hh;
        float *scores = malloc(span * sizeof(float));
        size_t kvh = h / repeat;
        const float *qv = q + h * QK;
        float max = -INFINITY;
        for (size_t i = 0; i < span; i++) {
            size_t slot = (lo + i) % slots;
            size_t ko = (slot * H + kvh) * QK;
            float acc = kq ? dot_i8(qv, kq + ko, QK, ks[slot * H + kvh])
                           : dot_f32(qv, kf + ko, QK);
            scores[i] = acc * scale;
            if (scores[i] > max)
                max = scores[i];
        }
        float sum = 0.0f;
        for (size_t i = 0; i < span; i++) {
            scores[i] = or_expf(scores[i] - max);
            sum += scores[i];
        }
        float inv = 1.0f / sum;
        float *o = out + h * VD;
        for (size_t j = 0; j < VD; j++)
            o[j] = 0.0f;
        for (size_t i = 0; i < span; i++) {
            float w = scores[i] * inv;
            size_t slot = (lo + i) % slots;
            size_t vo = (slot * H + kvh) * VD;
            if (vq) {
                float ww = w * vs[slot * H + kvh];
                for (size_t j = 0; j < VD; j++)
                    o[j] += ww * (float)vq[vo + j];
            } else {
                for (size_t j = 0; j < VD; j++)
                    o[j] += w * vf[vo + j];
            }
        }
        free(scores);
    }
}

/* `count` independent sessions' attend_step over their own int8 caches
 * (session i's at k + i*slots*kvh*qk and likewise), sessions split across
 * threads as a server runs one V3Cache per session on its pool
 * (v3_engine.rs:547-560); each session's arithmetic is attend_step's. */
void or_attend_step_i8_sessions(size_t count, const float *q, const int8_t *k,
                                const float *k_scale, const int8_t *v,
                                const float *v_scale, size_t slots, size_t lo, size_t hi,
                                const or_attn_dims *d, float *out, int threads)
{
    size_t H = d->num_kv_heads, qn = d->num_heads * d->qk_head_dim;
    size_t on = d->num_heads * d->v_head_dim;
    int saved = or_threads;
    or_threads = 1; /* one session per thread; its heads stay serial */
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(dynamic, 1)
    for (long i = 0; i < (long)count; i++) {
        size_t s = (size_t)i;
        attend_step_impl(q + s * qn, NULL, NULL, k + s * slots * H * d->qk_head_dim,
                         k_scale + s * slots * H, v + s * slots * H * d->v_head_dim,
                         v_scale + s * slots * H, slots, lo, hi, d, out + s * on);
    }
    or_threads = saved;
}

void or_attend_step_f32(const float *q, const float *k, const float *v,
                        size_t slots, size_t lo, size_t hi,
                        const or_attn_dims *d, float *out)
{
    attend_step_impl(q, k, v, NULL, NULL, NULL, NULL, slots, lo, hi, d, out);
}

void or_attend_step_i8(const float *q, const int8_t *k, const float *k_scale,
                       const int8_t *v, const float *v_scale, size_t slots,
                       size_t lo, size_t hi, const or_attn_dims *d, float *out)
{
    attend_step_impl(q, NULL, NULL, k, k_scale, v, v_scale, slots, lo, hi, d, out);
}

/* attention.rs:241-287: every position t, window lo = t+1-w. */
static void attend_impl(const float *q, const float *kf, const float *vf,
                        const int8_t *kq, const float *ks, const int8_t *vq,
                        const float *vs, const or_attn_dims *d, size_t window,
                        float *out)
{
    float scale = 1.0f / sqrtf((float)d->qk_head_dim);
    size_t repeat = d->num_heads / d->num_kv_heads;
    size_t QK = d->qk_head_dim, VD = d->v_head_dim, H = d->num_kv_heads;
    float *scores = malloc((d->seq ? d->seq : 1) * sizeof(float));
    for (size_t t = 0; t < d->seq; t++) {
        size_t lo = (window && t + 1 > window) ? t + 1 - window : 0;
        for (size_t h = 0; h < d->num_heads; h++) {
            size_t kvh = h / repeat;
            const float *qv = q + (t * d->num_heads + h) * QK;
            float max = -INFINITY;
            for (size_t n = lo; n <= t; n++) {
                size_t ko = (n * H + kvh) * QK;
                float acc = kq ? dot_i8(qv, kq + ko, QK, ks[n * H + kvh])
                               : dot_f32(qv, kf + ko, QK);
                scores[n] = acc * scale;
                if (scores[n] > max)
                    max = scores[n];
            }
            float sum = 0.0f;
            for (size_t n = lo; n <= t; n++) {
                scores[n] = or_expf(scores[n] - max);
                sum += scores[n];
            }
            float inv = 1.0f / sum;
            float *o = out + (t * d->num_heads + h) * VD;
            for (size_t j = 0; j < VD; j++)
                o[j] = 0.0f;
            for (size_t n = lo; n <= t; n++) {
                float w = scores[n] * inv;
                size_t vo = (n * H + kvh) * VD;
                if (vq) {
                    float ww = w * vs[n * H + kvh];
                    for (size_t j = 0; j < VD; j++)
                        o[j] += ww * (float)vq[vo + j];
                } else {
                    for (size_t j = 0; j < VD; j++)
                        o[j] += w * vf[vo + j];
                }
            }
        }
    }
    free(scores);
}

void or_attend_f32(const float *q, const float *k, const float *v,
                   const or_attn_dims *d, size_t window, float *out)
{
    attend_impl(q, k, v, NULL, NULL, NULL, NULL, d, window, out);
}

void or_attend_i8(const float *q, const int8_t *k, const float *k_scale,
                  const int8_t *v, const float *v_scale,
                  const or_attn_dims *d, size_t window, float *out)
{
    attend_impl(q, NULL, NULL, k, k_scale, v, v_scale, d, window, out);
}

/* attend_step over a ring's own store (model.rs:295-307). */
void or_ring_attend_step(const or_ring *r, const float *q, size_t lo,
                         size_t hi, size_t num_heads, float *out)
{
    or_attn_dims d = {1, num_heads, r->num_kv_heads, r->qk_head_dim, r->v_head_dim};
    if (r->int8)
        or_attend_step_i8(q, r->kq, r->k_scale, r->vq, r->v_scale, r->slots, lo, hi, &d, out);
    else
        or_attend_step_f32(q, r->k, r->v, r->slots, lo, hi, &d, out);
}
