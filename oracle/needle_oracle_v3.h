/*
 * needle_oracle_v3.h -- the oracle's Needle-3 forward (decode step) around
 * the hot path.  TEST INFRASTRUCTURE ONLY.
 *
 * Pinning: the helpers below are pinned by closed forms and the reference's
 * own invariants (tests/test_oracle_v3.py): Kronecker apply vs a dense
 * np.kron product, Sinkhorn rows/columns summing to one, the Engram hash
 * KATs (engram.rs:139-172), conv step vs the sequence conv
 * (cache.rs:814-841), RoPE as a norm-preserving rotation that is the
 * identity at position 0, mix_down's gated-lane-sum KAT (mhc.rs:168-189),
 * scatter_up's mass conservation (mhc.rs:191-238).  The whole decode step
 * with an f32 KV cache agrees with the reference's numpy transcription of
 * the forward (tools/needle3_reference.py) on a seeded random-init container
 * to float rounding, greedy tokens identical (tests/test_forward_reference.py);
 * the int8 path adds the quantiser, pinned by its own fixture.  The oracle
 * is test infrastructure: the GPU engine's checker.
 */
#ifndef NEEDLE_ORACLE_V3_H
#define NEEDLE_ORACLE_V3_H

#include <stddef.h>
#include <stdint.h>

#include "needle_oracle.h"

#ifdef __cplusplus
extern "C" {
#endif

#define OR_V3_MAX_HIST 16

/* V3Config (v3/config.rs:45-77) with the Engram fields flattened. */
typedef struct or_v3_cfg {
    size_t vocab_size, out_vocab, d_model, num_heads, num_kv_heads, num_layers;
    size_t qk_head_dim, v_head_dim, max_seq_len, hada_n, mhc_lanes;
    float rope_theta;
    size_t sliding_window, n_global, global_layers[64], qkv_conv_taps;
    size_t n_orders, orders[8], e_heads, e_slots, e_sub_dim, n_sites, sites[64];
    size_t e_conv_taps, e_conv_dilation, e_seed_heads;
} or_v3_cfg;

enum { OR_REC_F32 = 1, OR_REC_CQ = 3 };

/* One container record: a CQ blob (kind 3, shape out x in, group, bits) or
 * an f32 array (kind 1; `in` carries the second dimension when 2-D). */
typedef struct or_v3_record {
    int kind;
    const uint8_t *data;
    size_t len, out, in, group, bits;
} or_v3_record;

typedef struct or_v3_mlp {
    float *d1, *d2, *b2, *d3, *d4, *w1a, *w1b, *w2a, *w2b, *w3a, *w3b, *cond_v, *cond_u;
    size_t cond_rank;
} or_v3_mlp;

typedef struct or_v3_layer {
    float *norm_in;
    or_cq *q_proj, *k_proj, *v_proj;
    float *q_taps, *k_taps, *v_taps, *q_norm, *k_norm;
    or_cq *gate_proj, *out_proj;
    float *post_norm, attn_gate, *pre_hada;
    or_v3_mlp mlp;
} or_v3_layer;

typedef struct or_v3_engram {
    or_cq *tables, *key_proj, *value_proj;
    float *taps;
} or_v3_engram;

typedef struct or_v3_model {
    or_v3_cfg cfg;
    float codebook[OR_CODEBOOK_LEN];
    or_cq *embedding;
    or_v3_layer *layers;
    float *a_pre, *a_post, *a_res, *b_pre, *b_post, *b_res;
    or_cq *phi_pre, *phi_post, *phi_res;
    uint32_t *p1, *p2;
    or_v3_engram *engrams;
    float *final_norm, embed_scale;
} or_v3_model;

typedef struct or_v3_cache {
    or_v3_cfg cfg;
    int int8;
    or_ring **rings;
    float **q_tail, **k_tail, **v_tail, **engram_tail;
    uint32_t tokens[OR_V3_MAX_HIST];
    size_t n_tokens, pos;
} or_v3_cache;

or_v3_model *or_v3_model_new(const or_v3_cfg *cfg, const float *codebook,
                             const or_v3_record *recs, size_t n);
void or_v3_model_free(or_v3_model *m);
or_v3_cache *or_v3_cache_new(const or_v3_cfg *cfg, size_t hint, int int8);
void or_v3_cache_free(or_v3_cache *c);
void or_v3_decode_step(const or_v3_model *m, or_v3_cache *cache, uint32_t token, float *out);
void or_v3_generate(const or_v3_model *m, or_v3_cache *cache, const uint32_t *prompt,
                    size_t n_prompt, size_t steps, uint32_t *out_tokens, float *out_margin);
uint32_t or_argmax(const float *x, size_t n);
void or_v3_decode_sessions(const or_v3_model *m, or_v3_cache **caches, const uint32_t *tokens,
                           size_t n, float *logits, int threads);
void or_v3_cache_fill_synthetic(or_v3_cache *k, size_t pos, uint64_t seed);

void or_sinkhorn(float *m, size_t n);
void or_hada_blocks(size_t n, size_t *ba, size_t *bb);
void or_kron_apply(const float *z, const float *a, const float *b, size_t ba, size_t bb,
                   float *out);
void or_hadamard_mlp(const float *x, size_t d_model, const or_v3_mlp *w, const uint32_t *p1,
                     const uint32_t *p2, size_t hada_n, float *out);
void or_engram_indices(const uint32_t *tokens, size_t seq, const size_t *orders,
                       size_t n_orders, size_t heads, uint32_t slots, size_t seed_heads,
                       uint32_t *out);
int or_ngram_valid(size_t p, size_t table, const size_t *orders, size_t heads);
void or_v3_rope_at(const or_v3_cfg *c, size_t pos, float *cs, float *sn);
/* The routines behind the RoPE table (process-wide; tests only):
 * OR_ROPE_LIBM, the reference's (the default); OR_ROPE_POWF_CR, theta^e
 * correctly rounded; OR_ROPE_GLIBC, the C library's powf/cosf/sinf. */
#define OR_ROPE_LIBM 0
#define OR_ROPE_POWF_CR 1
#define OR_ROPE_GLIBC 2
void or_v3_set_rope_variant(int variant);
void or_v3_apply_site(float *x, const float *k, const float *v, size_t d);
void or_v3_conv_step(float *tail, const float *taps, float *raw, size_t dim, size_t n_taps,
                     size_t pos);
void or_v3_engram_conv_step(float *tail, const float *taps, float *raw, size_t d, size_t n_taps,
                            size_t dil, size_t max_order, size_t pos);
void or_v3_norm_and_rope(float *buf, const float *scale, const float *cs, const float *sn,
                         size_t heads, size_t hd);
void or_v3_mix_down(const float *lanes, float *rows, float a_pre, const float *b_pre,
                    size_t layer, size_t n, size_t d, float *u);
void or_v3_scatter_up(float *lanes, float *post, float *res, const float *y, float a_post,
                      const float *b_post, float a_res, const float *b_res, size_t layer, size_t n,
                      size_t d);

#ifdef __cplusplus
}
#endif
#endif
