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

/* cq.rs:838-873: eight-lane packed dot of one group, lanes summed 0..7. */
static float dot_group(size_t P, const float *lut, const uint8_t *gbytes,
                       size_t nbytes, const float *gx)
{
    size_t per_iter = ACC_LANES / P;
    float lanes[ACC_LANES] = {0};
    size_t full = nbytes - nbytes % per_iter;
    size_t bi = 0;
    while (bi < full) {
        float vals[ACC_LANES];
        for (size_t t = 0; t < per_iter; t++) {
            size_t base = (size_t)gbytes[bi + t] * P;
            for (size_t k = 0; k < P; k++)
                vals[t * P + k] = lut[base + k];
        }
        const float *xs = gx + bi * P;
        for (size_t k = 0; k < ACC_LANES; k++)
            lanes[k] += vals[k] * xs[k];
        bi += per_iter;
    }
    float acc = 0.0f;
    for (size_t k = 0; k < ACC_LANES; k++)
        acc += lanes[k];
    for (size_t b = bi; b < nbytes; b++) {
        size_t base = (size_t)gbytes[b] * P;
        for (size_t k = 0; k < P; k++)
            acc += lut[base + k] * gx[b * P + k];
    }
    return acc;
}

/* cq.rs:721-735 (LUT widths) and cq.rs:738-757 (3-bit generic). */
void or_cq_matvec_rows_prepared(const or_cq *w, const float *xh,
                                size_t row_start, size_t rows, float *y)
{
    for (size_t yi = 0; yi < rows; yi++) {
        size_t o = row_start + yi;
        const uint8_t *row = w->packed + o * w->row_bytes;
        const float *rn = w->norms + o * w->num_groups;
        float total = 0.0f;
        if (w->per_byte) {
            size_t P = w->per_byte;
            size_t bpg = w->group / P;
            for (size_t g = 0; g < w->num_groups; g++)
                total += rn[g] * dot_group(P, w->lut, row + g * bpg, bpg,
                                           xh + g * w->group);
        } else {
            size_t bits = w->bits;
            uint32_t mask = (1u << bits) - 1;
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
        }
        y[yi] = total;
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

/* cq.rs:791-809: levels * norm for one group, before the rotation. */
static void decode_group(const or_cq *w, const uint8_t *row, size_t g,
                         float norm, float *buf)
{
    if (w->per_byte) {
        size_t p = w->per_byte;
        size_t bpg = w->group / p;
        const uint8_t *gb = row + g * bpg;
        for (size_t bi = 0; bi < bpg; bi++)
            for (size_t k = 0; k < p; k++)
                buf[bi * p + k] = w->lut[(size_t)gb[bi] * p + k] * norm;
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
    float lanes[ACC_LANES] = {0};
    for (size_t c = 0; c < chunks; c++)
        for (size_t k = 0; k < ACC_LANES; k++)
            lanes[k] += u[c * ACC_LANES + k] * x[c * ACC_LANES + k];
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
 * row in the matvec's lane order, acc[b] += norm * s; batch-major output. */
void or_cq_matmul_rows_prepared(const or_cq *w, const float *xh, size_t batch,
                                size_t row_start, size_t rows, float *y)
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
            y[b * rows + r] = acc[b];
    }
    free(acc);
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
    float *scores = malloc(span * sizeof(float));
    size_t QK = d->qk_head_dim, VD = d->v_head_dim, H = d->num_kv_heads;
    for (size_t h = 0; h < d->num_heads; h++) {
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
    }
    free(scores);
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
