/*
 * needle_oracle.h -- CPU restatement of needle-rs's Needle-3 hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP path is
 * compared against, and the CPU baseline bench.py times.  Nothing in the
 * shipped library (needle-rs_amd/) links, loads or calls it; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may.
 *
 * Every function restates the reference's arithmetic in the reference's own
 * float order (built with -ffp-contract=off, as rustc never contracts) and
 * cites the file:line it follows, relative to the needle-rs checkout.
 *
 * Pinning (what fixes each function independently of this restatement):
 *   or_f16_to_f32            known values of math.rs:77-93 + exhaustive
 *                            round trip (math.rs:96-107)                 PINNED
 *   or_fwht*                 dense Sylvester matrix, exact on integers
 *                            (hadamard.rs:102-120), involution (:147-158) PINNED
 *   or_read_bits/build_lut   brute force vs an independent bit packer
 *                            (cq.rs:989-1005 pack_lsb) over every width   PINNED
 *   or_cq_* (Format A)       dense reconstruction built the upstream way
 *                            (cq.rs:1028-1088), matvec == dense (1e-4),
 *                            matmul == matvec bit-exact (cq.rs:1270-1323),
 *                            row band == full (cq.rs:1209-1229), simple
 *                            reference agreement (cq.rs:1236-1268),
 *                            shipped blob sizes (cq.rs:1347-1363 and the
 *                            v3 directory records)                      PINNED
 *   or_cb8_* (Format B)      closed form; checked against an f64 brute
 *                            force (no reference function exists)       PINNED
 *   or_fake_quant_vec etc.   tests/v3_kv_quant_vectors.json (upstream
 *                            fake_quant), all-zero and half-step
 *                            invariants (v3_kv_quant_parity.rs:67-92)   PINNED
 *                            (exact .5 ties: roundf's half-away-from-zero
 *                            contract, tests/test_oracle_kv.py)
 *   or_ring_*                wrap/growth readback (cache.rs:578-636),
 *                            caps (:638-665), spans (:795-812), global
 *                            clamp (:699-730)                           PINNED
 *   or_attend_step/attend    ring-wrap KAT (attention.rs:399-431),
 *                            window-1 KAT (:433-456), hoisted-scale
 *                            reader vs dequantised buffer
 *                            (v3_kv_quant_parity.rs:102-218), f64
 *                            textbook softmax attention                 PINNED
 *                            (expf: libm's published algorithm restated,
 *                            within 1 ulp of the exactly rounded value and
 *                            equal to the device copy; tests/test_oracle_libm.py)
 */
#ifndef NEEDLE_ORACLE_H
#define NEEDLE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- math.rs ---------------------------------------------------------- */
float or_f16_to_f32(uint16_t bits);
/* libm 0.2.16 expf / logf (FreeBSD e_expf.c / e_logf.c), math.rs:3-11. */
float or_expf(float x);
float or_logf(float x);
void or_expf_n(const float *x, size_t n, float *y);
void or_logf_n(const float *x, size_t n, float *y);
/* libm 0.2.16 sinf / cosf / powf (msun s_sinf.c, s_cosf.c, k_sinf.c,
 * k_cosf.c, e_rem_pio2f.c, k_rem_pio2.c, e_powf.c), math.rs:13-36: the RoPE
 * table's functions (v3/model.rs:378-413). */
float or_sinf(float x);
float or_cosf(float x);
float or_powf(float x, float y);
void or_sinf_n(const float *x, size_t n, float *y);
void or_cosf_n(const float *x, size_t n, float *y);
void or_powf_n(const float *x, const float *e, size_t n, float *y);

/* ---- hadamard.rs ------------------------------------------------------ */
void or_fwht(float *x, size_t n);
void or_fwht_normalized(float *x, size_t n);

/* ---- cq.rs (Format A, Cactus-Quants) ---------------------------------- */
#define OR_TERNARY_RECORD_BITS 5
#define OR_CODEBOOK_LEN 28
#define OR_MAX_GROUP 1024

enum or_cq_error {
    OR_CQ_OK = 0,
    OR_CQ_UNSUPPORTED_BITS = 1,
    OR_CQ_BAD_GROUP = 2,
    OR_CQ_BAD_CODEBOOK_LEN = 3,
    OR_CQ_SHORT_BLOB = 4,
    OR_CQ_EMPTY_SHAPE = 5,
};

typedef struct or_cq {
    uint8_t *packed;   /* out_feat * row_bytes */
    float *norms;      /* out_feat * num_groups */
    float *lut;        /* 256 * per_byte, or NULL */
    size_t per_byte;
    size_t row_bytes;
    size_t num_groups;
    size_t out_feat;
    size_t in_feat;
    size_t in_padded;
    size_t group;
    uint8_t bits;
    float levels[16];
    size_t n_levels;
} or_cq;

size_t or_packed_row_bytes(size_t in_padded, uint8_t bits);
uint32_t or_read_bits(const uint8_t *row, size_t bit, size_t bits, uint32_t mask);
/* Fills lut (256*per_byte floats, caller-owned, may be NULL to query);
 * returns per_byte (0 for 3-bit). */
size_t or_build_lut(uint8_t bits, const float *levels, float *lut);

int or_cq_from_blob(const uint8_t *blob, size_t blob_len, size_t out_feat,
                    size_t in_feat, size_t group, uint8_t bits,
                    const float *codebook, size_t codebook_len, or_cq **out);
void or_cq_free(or_cq *w);
void or_cq_prepare_input(const or_cq *w, const float *x, float *xh);
void or_cq_matvec_rows_prepared(const or_cq *w, const float *xh,
                                size_t row_start, size_t rows, float *y);
void or_cq_matvec(const or_cq *w, const float *x, float *y);
void or_cq_matvec_prepared_reference(const or_cq *w, const float *xh, float *y);
void or_cq_matmul_rows_prepared(const or_cq *w, const float *xh, size_t batch,
                                size_t row_start, size_t rows, float *y);
void or_cq_dequantize_row(const or_cq *w, size_t o, float *out);

/* ---- Format B: uint8 codes, one 256-entry fp32 codebook per 64 rows --- */
void or_cb8_gemv(const uint8_t *w, const float *cb, const float *x, float *y,
                 size_t out, size_t in);
void or_cb8_gemv_f64(const uint8_t *w, const float *cb, const float *x,
                     double *y, size_t out, size_t in);
void or_cb8_gemm(const float *x, const uint8_t *w, const float *cb, float *y,
                 size_t m, size_t out, size_t in);
/* Threads for the reference's rayon splits (cq.rs:301-323, 446-581):
 * OR_SPLIT_REFERENCE applies its size rules (the CPU baseline);
 * OR_SPLIT_ALL splits every independent row loop and attention's heads too
 * (a faster checker, the same bits).  One thread (the default) is serial. */
#define OR_SPLIT_REFERENCE 0
#define OR_SPLIT_ALL 1
void or_set_threads(int threads, int split);
int or_get_threads(void);

void or_cb8_gemv_omp(const uint8_t *w, const float *cb, const float *x,
                     float *y, size_t out, size_t in);
void or_cb8_gemm_omp(const float *x, const uint8_t *w, const float *cb, float *y,
                     size_t m, size_t out, size_t in, int threads);
/* The CPU baseline's Format B kernels, in the reference's LUT-kernel order
 * (eight lanes; the GEMM decodes each row once): within float rounding of
 * the closed form above, rows in bands over `threads`. */
void or_cb8_gemv_lanes(const uint8_t *w, const float *cb, const float *x, float *y,
                       size_t out, size_t in, int threads);
void or_cb8_gemm_lanes(const float *x, const uint8_t *w, const float *cb, float *y,
                       size_t m, size_t out, size_t in, int threads);

/* ---- v3/cache.rs ------------------------------------------------------ */
void or_fake_quant_vec(float *x, size_t n, uint32_t bits);
float or_quant_into(const float *src, size_t n, int8_t *dst);
void or_quantize_rows(const float *x, size_t rows, size_t head_dim,
                      int8_t *ints, float *scales);
void or_quant_rows(float *x, size_t seq, size_t heads, size_t head_dim);

/* One layer of V3Cache, int8 or f32, reference (slot-major) layout. */
typedef struct or_ring {
    int int8;
    size_t num_kv_heads, qk_head_dim, v_head_dim;
    size_t slots, cap, window; /* window 0 = global */
    float *k, *v;              /* f32: slots * k_dim / v_dim */
    int8_t *kq, *vq;           /* int8 */
    float *k_scale, *v_scale;  /* slots * num_kv_heads */
} or_ring;

or_ring *or_ring_new(int int8, size_t num_kv_heads, size_t qk, size_t vd,
                     size_t hint, size_t window, size_t max_seq_len);
void or_ring_free(or_ring *r);
void or_ring_write_kv(or_ring *r, size_t pos, const float *k, const float *v);
void or_ring_span(const or_ring *r, size_t pos, size_t *lo, size_t *hi);

/* ---- v3/attention.rs ---------------------------------------------------- */
typedef struct or_attn_dims {
    size_t seq, num_heads, num_kv_heads, qk_head_dim, v_head_dim;
} or_attn_dims;

void or_attend_step_f32(const float *q, const float *k, const float *v,
                        size_t slots, size_t lo, size_t hi,
                        const or_attn_dims *d, float *out);
void or_attend_step_i8(const float *q, const int8_t *k, const float *k_scale,
                       const int8_t *v, const float *v_scale, size_t slots,
                       size_t lo, size_t hi, const or_attn_dims *d, float *out);
void or_attend_step_i8_sessions(size_t count, const float *q, const int8_t *k,
                                const float *k_scale, const int8_t *v,
                                const float *v_scale, size_t slots, size_t lo, size_t hi,
                                const or_attn_dims *d, float *out, int threads);
void or_attend_f32(const float *q, const float *k, const float *v,
                   const or_attn_dims *d, size_t window, float *out);
void or_attend_i8(const float *q, const int8_t *k, const float *k_scale,
                  const int8_t *v, const float *v_scale,
                  const or_attn_dims *d, size_t window, float *out);
void or_ring_attend_step(const or_ring *r, const float *q, size_t lo,
                         size_t hi, size_t num_heads, float *out);

#ifdef __cplusplus
}
#endif
#endif
