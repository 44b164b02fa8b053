/*
 * needle_oracle_v3.c -- CPU restatement of the Needle-3 forward (decode step)
 * around the hot path: the caller of the CQ projections and the int8 KV
 * cache.  TEST INFRASTRUCTURE ONLY (the checker for the GPU engine).
 *
 * Follows crates/needle-core/src/v3/model.rs:150-375 (decode_step) and the
 * helpers it calls, in the reference's float order (-ffp-contract=off):
 *   kernels.rs:22-85 (rms_unit_to, sinkhorn, logsumexp), norm.rs:23-30,
 *   ops.rs:40-43 (sigmoid), 111-114 (silu), v3/engram.rs:30-132,
 *   v3/mhc.rs:54-152, v3/kernels.rs:26-188, v3/attention.rs:85-150
 *   (causal conv, norm_and_rope), v3/cache.rs:401-482 (conv_step,
 *   engram_conv_step), v3/model.rs:378-394 (rope_at),
 *   needle-infer/src/v3_engine.rs:410-420 (argmax, first maximum wins).
 * Weights arrive as records in the canonical .cact order of
 * needle-infer/src/v3.rs:236-330 (V3Layout::derive).
 */
#include "needle_oracle.h"
#include "needle_oracle_v3.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define EPS 1e-6f
#define SINKHORN_ITERS 20

/* ---- shared primitives -------------------------------------------------- */

/* ops.rs:40-43 */
static float sigmoid(float x) { return 1.0f / (1.0f + or_expf(-x)); }
/* ops.rs:111-114 */
static float silu(float x) { return x * sigmoid(x); }

/* kernels.rs:33-41 */
static void rms_unit_to(const float *x, float *out, size_t n)
{
    float s = 0.0f;
    for (size_t i = 0; i < n; i++)
        s += x[i] * x[i];
    float mean_sq = s / (float)n;
    float inv = 1.0f / sqrtf(mean_sq + EPS);
    for (size_t i = 0; i < n; i++)
        out[i] = x[i] * inv;
}

/* norm.rs:23-30 */
static void zc_rms_norm_vec(float *x, const float *scale, size_t n)
{
    float s = 0.0f;
    for (size_t i = 0; i < n; i++)
        s += x[i] * x[i];
    float mean_sq = s / (float)n;
    float inv = 1.0f / sqrtf(mean_sq + EPS);
    for (size_t i = 0; i < n; i++)
        x[i] = (1.0f + scale[i]) * x[i] * inv;
}

/* kernels.rs:78-85 */
static float logsumexp(const float *x, size_t n)
{
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++)
        max = fmaxf(max, x[i]);
    if (!isfinite(max))
        return max;
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++)
        sum += or_expf(x[i] - max);
    return max + or_logf(sum);
}

/* kernels.rs:48-74 */
void or_sinkhorn(float *m, size_t n)
{
    for (int it = 0; it < SINKHORN_ITERS; it++) {
        for (size_t i = 0; i < n; i++) {
            float lse = logsumexp(m + i * n, n);
            for (size_t j = 0; j < n; j++)
                m[i * n + j] -= lse;
        }
        for (size_t j = 0; j < n; j++) {
            float max = -INFINITY;
            for (size_t i = 0; i < n; i++)
                max = fmaxf(max, m[i * n + j]);
            float sum = 0.0f;
            for (size_t i = 0; i < n; i++)
                sum += or_expf(m[i * n + j] - max);
            float lse = max + or_logf(sum);
            for (size_t i = 0; i < n; i++)
                m[i * n + j] -= lse;
        }
    }
    for (size_t i = 0; i < n * n; i++)
        m[i] = or_expf(m[i]);
}

/* v3/kernels.rs:26-34 */
void or_hada_blocks(size_t n, size_t *ba, size_t *bb)
{
    size_t bits = 0;
    while ((1ull << bits) < n)
        bits++; /* = bit_length(n - 1) for a power of two n > 1 */
    *ba = (size_t)1 << (bits / 2);
    *bb = n / *ba;
}

/* v3/kernels.rs:41-81: out[k,l] = sum_ij z[i,j] a[i,k] b[j,l]. */
void or_kron_apply(const float *z, const float *a, const float *b, size_t ba, size_t bb,
                   float *out)
{
    float *t = calloc(ba * bb, sizeof(float));
    for (size_t i = 0; i < ba; i++)
        for (size_t k = 0; k < ba; k++) {
            float aik = a[i * ba + k];
            if (aik == 0.0f)
                continue;
            for (size_t j = 0; j < bb; j++)
                t[k * bb + j] += z[i * bb + j] * aik;
        }
    for (size_t k = 0; k < ba; k++) {
        for (size_t l = 0; l < bb; l++)
            out[k * bb + l] = 0.0f;
        for (size_t j = 0; j < bb; j++) {
            float tkj = t[k * bb + j];
            if (tkj == 0.0f)
                continue;
            for (size_t l = 0; l < bb; l++)
                out[k * bb + l] += tkj * b[j * bb + l];
        }
    }
    free(t);
}

/* v3/kernels.rs:119-180 */
void or_hadamard_mlp(const float *x, size_t d_model, const or_v3_mlp *w, const uint32_t *p1,
                     const uint32_t *p2, size_t hada_n, float *out)
{
    size_t ba, bb;
    or_hada_blocks(hada_n, &ba, &bb);
    size_t r = w->cond_rank;
    float proj[64];
    for (size_t j = 0; j < r; j++) {
        float acc = 0.0f;
        for (size_t i = 0; i < d_model; i++)
            acc += x[i] * w->cond_v[i * r + j];
        proj[j] = acc;
    }
    float max = -INFINITY;
    for (size_t j = 0; j < r; j++)
        max = fmaxf(max, proj[j]);
    float sum = 0.0f;
    for (size_t j = 0; j < r; j++) {
        proj[j] = or_expf(proj[j] - max);
        sum += proj[j];
    }
    for (size_t j = 0; j < r; j++)
        proj[j] /= sum;
    float *cond = malloc(hada_n * sizeof(float));
    for (size_t c = 0; c < hada_n; c++)
        cond[c] = 1.0f;
    for (size_t j = 0; j < r; j++) {
        if (proj[j] == 0.0f)
            continue;
        for (size_t c = 0; c < hada_n; c++)
            cond[c] += proj[j] * w->cond_u[j * hada_n + c];
    }
    float *z = calloc(hada_n, sizeof(float));
    float *buf = calloc(hada_n, sizeof(float));
    memcpy(z, x, d_model * sizeof(float));
    for (size_t i = 0; i < hada_n; i++)
        z[i] *= w->d1[i];
    or_kron_apply(z, w->w1a, w->w1b, ba, bb, buf);
    for (size_t i = 0; i < hada_n; i++)
        z[i] = buf[p1[i]];
    for (size_t i = 0; i < hada_n; i++)
        z[i] = silu(w->d2[i] * cond[i] * z[i] + w->b2[i]);
    or_kron_apply(z, w->w2a, w->w2b, ba, bb, buf);
    for (size_t i = 0; i < hada_n; i++)
        z[i] = buf[p2[i]];
    for (size_t i = 0; i < hada_n; i++)
        z[i] *= w->d3[i];
    or_kron_apply(z, w->w3a, w->w3b, ba, bb, buf);
    for (size_t i = 0; i < d_model; i++)
        out[i] = buf[i] * w->d4[i];
    free(cond);
    free(z);
    free(buf);
}

/* ---- Engram (v3/engram.rs) ---------------------------------------------- */

#define ENGRAM_SEED 0x9E3779B9u
#define ENGRAM_PRIME 0x01000193u

/* v3/engram.rs:30-59; out is (seq, num_tables). */
void or_engram_indices(const uint32_t *tokens, size_t seq, const size_t *orders,
                       size_t n_orders, size_t heads, uint32_t slots, size_t seed_heads,
                       uint32_t *out)
{
    size_t stride = seed_heads == 0 ? heads : seed_heads;
    size_t num_tables = n_orders * heads;
    for (size_t oi = 0; oi < n_orders; oi++)
        for (size_t h = 0; h < heads; h++) {
            size_t table = oi * heads + h;
            uint32_t seed = ENGRAM_SEED * (uint32_t)(oi * stride + h + 1);
            for (size_t p = 0; p < seq; p++) {
                uint32_t acc = seed;
                for (size_t j = 0; j < orders[oi]; j++) {
                    uint32_t tok = j > p ? 0u : tokens[p - j];
                    acc = (acc ^ tok) * ENGRAM_PRIME;
                }
                acc ^= acc >> 15;
                out[p * num_tables + table] = acc % slots;
            }
        }
}

/* v3/engram.rs:64-67 */
int or_ngram_valid(size_t p, size_t table, const size_t *orders, size_t heads)
{
    return p + 1 >= orders[table / heads];
}

/* v3/engram.rs:111-132 */
void or_v3_apply_site(float *x, const float *k, const float *v, size_t d)
{
    float sx = 0.0f, sk = 0.0f;
    for (size_t i = 0; i < d; i++)
        sx += x[i] * x[i];
    float ux = 1.0f / sqrtf(sx / (float)d + 1e-6f);
    for (size_t i = 0; i < d; i++)
        sk += k[i] * k[i];
    float uk = 1.0f / sqrtf(sk / (float)d + 1e-6f);
    float dot = 0.0f;
    for (size_t i = 0; i < d; i++)
        dot += x[i] * k[i];
    float alpha = sigmoid(dot * ux * uk / sqrtf((float)d));
    for (size_t i = 0; i < d; i++)
        x[i] += alpha * v[i];
}

/* ---- model construction from canonical records --------------------------- */

static float *take_floats(const or_v3_record *r, size_t want)
{
    if (r->kind != OR_REC_F32 || r->len != want * 4)
        return NULL;
    float *p = malloc(want * sizeof(float));
    memcpy(p, r->data, want * sizeof(float));
    return p;
}

static or_cq *take_cq(const or_v3_record *r, const float *codebook, size_t out, size_t in)
{
    or_cq *w = NULL;
    if (r->kind != OR_REC_CQ || r->out != out || r->in != in)
        return NULL;
    if (or_cq_from_blob(r->data, r->len, r->out, r->in, r->group, (uint8_t)r->bits, codebook,
                        OR_CODEBOOK_LEN, &w) != OR_CQ_OK)
        return NULL;
    return w;
}

/* needle-infer/src/v3.rs:236-330 record order; v3.rs:395-482 field use. */
or_v3_model *or_v3_model_new(const or_v3_cfg *cfg, const float *codebook,
                             const or_v3_record *recs, size_t n)
{
    size_t i = 0;
    size_t d = cfg->d_model, L = cfg->num_layers, nl = cfg->mhc_lanes;
    size_t qd = cfg->num_heads * cfg->qk_head_dim, kd = cfg->num_kv_heads * cfg->qk_head_dim;
    size_t vd = cfg->num_kv_heads * cfg->v_head_dim, od = cfg->num_heads * cfg->v_head_dim;
    size_t T = cfg->qkv_conv_taps, hn = cfg->hada_n;
    or_v3_model *m = calloc(1, sizeof(*m));
    m->cfg = *cfg;
    memcpy(m->codebook, codebook, sizeof(m->codebook));
#define NEXT() (i < n ? &recs[i++] : NULL)
#define NEED(x)            \
    do {                   \
        if (!(x))          \
            goto fail;     \
    } while (0)
    const or_v3_record *r;
    NEED(r = NEXT());
    NEED(m->embedding = take_cq(r, codebook, cfg->vocab_size, d));
    m->layers = calloc(L, sizeof(or_v3_layer));
    for (size_t li = 0; li < L; li++) {
        or_v3_layer *l = &m->layers[li];
        NEED(r = NEXT()); NEED(l->norm_in = take_floats(r, d));
        NEED(r = NEXT()); NEED(l->q_proj = take_cq(r, codebook, qd, d));
        NEED(r = NEXT()); NEED(l->k_proj = take_cq(r, codebook, kd, d));
        NEED(r = NEXT()); NEED(l->v_proj = take_cq(r, codebook, vd, d));
        if (T > 0) {
            NEED(r = NEXT()); NEED(l->q_taps = take_floats(r, T * qd));
            NEED(r = NEXT()); NEED(l->k_taps = take_floats(r, T * kd));
            NEED(r = NEXT()); NEED(l->v_taps = take_floats(r, T * vd));
        }
        NEED(r = NEXT()); NEED(l->q_norm = take_floats(r, cfg->qk_head_dim));
        NEED(r = NEXT()); NEED(l->k_norm = take_floats(r, cfg->qk_head_dim));
        NEED(r = NEXT()); NEED(l->gate_proj = take_cq(r, codebook, od, d));
        NEED(r = NEXT()); NEED(l->out_proj = take_cq(r, codebook, d, od));
        NEED(r = NEXT()); NEED(l->post_norm = take_floats(r, d));
        NEED(r = NEXT());
        float *ag = take_floats(r, 1);
        NEED(ag);
        l->attn_gate = ag[0];
        free(ag);
        NEED(r = NEXT()); NEED(l->pre_hada = take_floats(r, d));
        or_v3_mlp *w = &l->mlp;
        size_t ba, bb;
        or_hada_blocks(hn, &ba, &bb);
        NEED(r = NEXT()); NEED(w->d1 = take_floats(r, hn));
        NEED(r = NEXT()); NEED(w->d2 = take_floats(r, hn));
        NEED(r = NEXT()); NEED(w->b2 = take_floats(r, hn));
        NEED(r = NEXT()); NEED(w->d3 = take_floats(r, hn));
        NEED(r = NEXT()); NEED(w->d4 = take_floats(r, hn));
        NEED(r = NEXT()); NEED(w->w1a = take_floats(r, ba * ba));
        NEED(r = NEXT()); NEED(w->w1b = take_floats(r, bb * bb));
        NEED(r = NEXT()); NEED(w->w2a = take_floats(r, ba * ba));
        NEED(r = NEXT()); NEED(w->w2b = take_floats(r, bb * bb));
        NEED(r = NEXT()); NEED(w->w3a = take_floats(r, ba * ba));
        NEED(r = NEXT()); NEED(w->w3b = take_floats(r, bb * bb));
        NEED(r = NEXT());
        w->cond_rank = r->in;
        NEED(w->cond_rank > 0 && w->cond_rank <= 64);
        NEED(w->cond_v = take_floats(r, d * w->cond_rank));
        NEED(r = NEXT()); NEED(w->cond_u = take_floats(r, w->cond_rank * hn));
    }
    NEED(r = NEXT()); NEED(m->a_pre = take_floats(r, L));
    NEED(r = NEXT()); NEED(m->a_post = take_floats(r, L));
    NEED(r = NEXT()); NEED(m->a_res = take_floats(r, L));
    NEED(r = NEXT()); NEED(m->b_pre = take_floats(r, L * nl));
    NEED(r = NEXT()); NEED(m->b_post = take_floats(r, L * nl));
    NEED(r = NEXT()); NEED(m->b_res = take_floats(r, L * nl * nl));
    NEED(r = NEXT()); NEED(m->phi_pre = take_cq(r, codebook, L * nl, nl * d));
    NEED(r = NEXT()); NEED(m->phi_post = take_cq(r, codebook, L * nl, nl * d));
    NEED(r = NEXT()); NEED(m->phi_res = take_cq(r, codebook, L * nl * nl, nl * d));
    for (int pi = 0; pi < 2; pi++) {
        NEED(r = NEXT());
        float *pf = take_floats(r, hn);
        NEED(pf);
        uint32_t *pp = malloc(hn * sizeof(uint32_t));
        for (size_t k = 0; k < hn; k++)
            pp[k] = (uint32_t)pf[k];
        free(pf);
        if (pi == 0) m->p1 = pp; else m->p2 = pp;
    }
    size_t nt = cfg->n_orders * cfg->e_heads;
    m->engrams = calloc(cfg->n_sites, sizeof(or_v3_engram));
    for (size_t s = 0; s < cfg->n_sites; s++) {
        or_v3_engram *e = &m->engrams[s];
        NEED(r = NEXT()); NEED(e->tables = take_cq(r, codebook, nt * cfg->e_slots, cfg->e_sub_dim));
        NEED(r = NEXT()); NEED(e->key_proj = take_cq(r, codebook, d, nt * cfg->e_sub_dim));
        NEED(r = NEXT()); NEED(e->value_proj = take_cq(r, codebook, d, nt * cfg->e_sub_dim));
        NEED(r = NEXT()); NEED(e->taps = take_floats(r, cfg->e_conv_taps * d));
    }
    NEED(r = NEXT()); NEED(m->final_norm = take_floats(r, d));
    m->embed_scale = sqrtf((float)d);
#undef NEXT
#undef NEED
    return m;
fail:
    or_v3_model_free(m);
    return NULL;
}

void or_v3_model_free(or_v3_model *m)
{
    if (!m)
        return;
    or_cq_free(m->embedding);
    if (m->layers) {
        for (size_t li = 0; li < m->cfg.num_layers; li++) {
            or_v3_layer *l = &m->layers[li];
            free(l->norm_in); or_cq_free(l->q_proj); or_cq_free(l->k_proj); or_cq_free(l->v_proj);
            free(l->q_taps); free(l->k_taps); free(l->v_taps); free(l->q_norm); free(l->k_norm);
            or_cq_free(l->gate_proj); or_cq_free(l->out_proj); free(l->post_norm); free(l->pre_hada);
            or_v3_mlp *w = &l->mlp;
            free(w->d1); free(w->d2); free(w->b2); free(w->d3); free(w->d4);
            free(w->w1a); free(w->w1b); free(w->w2a); free(w->w2b); free(w->w3a); free(w->w3b);
            free(w->cond_v); free(w->cond_u);
        }
        free(m->layers);
    }
    free(m->a_pre); free(m->a_post); free(m->a_res); free(m->b_pre); free(m->b_post);
    free(m->b_res);
    or_cq_free(m->phi_pre); or_cq_free(m->phi_post); or_cq_free(m->phi_res);
    free(m->p1); free(m->p2);
    if (m->engrams) {
        for (size_t s = 0; s < m->cfg.n_sites; s++) {
            or_cq_free(m->engrams[s].tables); or_cq_free(m->engrams[s].key_proj);
            or_cq_free(m->engrams[s].value_proj); free(m->engrams[s].taps);
        }
        free(m->engrams);
    }
    free(m->final_norm);
    free(m);
}

/* ---- V3Cache (v3/cache.rs) ----------------------------------------------- */

static size_t attention_span(const or_v3_cfg *c, size_t layer)
{
    for (size_t i = 0; i < c->n_global; i++)
        if (c->global_layers[i] == layer)
            return 0;
    return c->sliding_window;
}

static size_t max_order(const or_v3_cfg *c)
{
    size_t m = 1;
    for (size_t i = 0; i < c->n_orders; i++)
        if (c->orders[i] > m)
            m = c->orders[i];
    return m;
}

/* cache.rs:177-238 */
or_v3_cache *or_v3_cache_new(const or_v3_cfg *c, size_t hint, int int8)
{
    or_v3_cache *k = calloc(1, sizeof(*k));
    k->cfg = *c;
    k->int8 = int8;
    size_t qd = c->num_heads * c->qk_head_dim, kd = c->num_kv_heads * c->qk_head_dim;
    size_t vd = c->num_kv_heads * c->v_head_dim, tt = c->qkv_conv_taps ? c->qkv_conv_taps - 1 : 0;
    k->rings = calloc(c->num_layers, sizeof(or_ring *));
    k->q_tail = calloc(c->num_layers, sizeof(float *));
    k->k_tail = calloc(c->num_layers, sizeof(float *));
    k->v_tail = calloc(c->num_layers, sizeof(float *));
    for (size_t li = 0; li < c->num_layers; li++) {
        k->rings[li] = or_ring_new(int8, c->num_kv_heads, c->qk_head_dim, c->v_head_dim, hint,
                                   attention_span(c, li), c->max_seq_len);
        k->q_tail[li] = calloc(tt * qd + 1, sizeof(float));
        k->k_tail[li] = calloc(tt * kd + 1, sizeof(float));
        k->v_tail[li] = calloc(tt * vd + 1, sizeof(float));
    }
    size_t reach = (c->e_conv_taps ? c->e_conv_taps - 1 : 0) * c->e_conv_dilation;
    k->engram_tail = calloc(c->n_sites, sizeof(float *));
    for (size_t s = 0; s < c->n_sites; s++)
        k->engram_tail[s] = calloc(reach * c->d_model + 1, sizeof(float));
    return k;
}

void or_v3_cache_free(or_v3_cache *k)
{
    if (!k)
        return;
    for (size_t li = 0; li < k->cfg.num_layers; li++) {
        or_ring_free(k->rings[li]);
        free(k->q_tail[li]); free(k->k_tail[li]); free(k->v_tail[li]);
    }
    for (size_t s = 0; s < k->cfg.n_sites; s++)
        free(k->engram_tail[s]);
    free(k->rings); free(k->q_tail); free(k->k_tail); free(k->v_tail); free(k->engram_tail);
    free(k);
}

/* cache.rs:283-289 */
static void push_token(or_v3_cache *k, uint32_t tok)
{
    size_t keep = max_order(&k->cfg);
    if (keep > OR_V3_MAX_HIST)
        keep = OR_V3_MAX_HIST;
    if (k->n_tokens == keep) {
        memmove(k->tokens, k->tokens + 1, (keep - 1) * sizeof(uint32_t));
        k->n_tokens--;
    }
    k->tokens[k->n_tokens++] = tok;
}

/* cache.rs:401-438: conv over Q/K/V at position `pos` with the retained raw
 * tail ((n_taps - 1) x dim, oldest first). */
void or_v3_conv_step(float *tail, const float *taps, float *raw, size_t dim, size_t n_taps,
                     size_t pos)
{
    if (n_taps == 0)
        return;
    float *out = malloc(dim * sizeof(float));
    for (size_t c = 0; c < dim; c++) {
        float acc = taps[c] * raw[c];
        for (size_t j = 1; j < n_taps; j++) {
            if (j > pos)
                break;
            size_t slot = n_taps - 1 - j;
            acc += taps[j * dim + c] * tail[slot * dim + c];
        }
        out[c] = acc;
    }
    if (n_taps > 1) {
        memmove(tail, tail + dim, (n_taps - 2) * dim * sizeof(float));
        memcpy(tail + (n_taps - 2) * dim, raw, dim * sizeof(float));
    }
    memcpy(raw, out, dim * sizeof(float));
    free(out);
}

static void conv_step(or_v3_cache *k, float *tail, const float *taps, float *raw, size_t dim)
{
    or_v3_conv_step(tail, taps, raw, dim, k->cfg.qkv_conv_taps, k->pos);
}

/* cache.rs:445-482: the Engram value conv at position `pos`, retained tail of
 * (n_taps - 1) * dil rows. */
void or_v3_engram_conv_step(float *tail, const float *taps, float *raw, size_t d, size_t n_taps,
                            size_t dil, size_t mo, size_t pos)
{
    size_t reach = (n_taps - 1) * dil;
    float *out = malloc(d * sizeof(float));
    for (size_t ch = 0; ch < d; ch++) {
        float acc = 0.0f;
        for (size_t j = 0; j < n_taps; j++) {
            size_t back = j * dil;
            if (back > pos || pos < j * mo)
                continue;
            float val = j == 0 ? raw[ch] : tail[(reach - back) * d + ch];
            acc += taps[j * d + ch] * val;
        }
        out[ch] = acc;
    }
    if (reach > 0) {
        memmove(tail, tail + d, (reach - 1) * d * sizeof(float));
        memcpy(tail + (reach - 1) * d, raw, d * sizeof(float));
    }
    memcpy(raw, out, d * sizeof(float));
    free(out);
}

static void engram_conv_step(or_v3_cache *k, size_t site, const float *taps, float *raw)
{
    const or_v3_cfg *c = &k->cfg;
    or_v3_engram_conv_step(k->engram_tail[site], taps, raw, c->d_model, c->e_conv_taps,
                           c->e_conv_dilation, max_order(c), k->pos);
}

/* attention.rs:108-150 with seq = 1. */
void or_v3_norm_and_rope(float *buf, const float *scale, const float *cs, const float *sn,
                          size_t heads, size_t hd)
{
    size_t half = hd / 2;
    for (size_t h = 0; h < heads; h++) {
        float *x = buf + h * hd;
        float sq = 0.0f;
        for (size_t i = 0; i < hd; i++)
            sq += x[i] * x[i];
        float rms = sqrtf(sq / (float)hd + 1e-6f);
        for (size_t i = 0; i < hd; i++)
            x[i] = (1.0f + scale[i]) * x[i] / rms;
        for (size_t i = 0; i < half; i++) {
            float c = cs[i], s = sn[i];
            float x1 = x[i], x2 = x[half + i];
            x[i] = x1 * c - x2 * s;
            x[half + i] = x2 * c + x1 * s;
        }
    }
}

/* Which routines build the RoPE table.  OR_ROPE_LIBM (the default) is the
 * reference's: libm 0.2.16's powf, cosf and sinf (model.rs:376-394), restated
 * as or_powf / or_cosf / or_sinf.  The other two exist to measure how much the
 * greedy tokens depend on those routines' last bits: OR_ROPE_POWF_CR takes
 * the correctly rounded theta^e (from powl) wherever or_powf differs from it,
 * and OR_ROPE_GLIBC the C library's powf, cosf and sinf. */
static int rope_variant = OR_ROPE_LIBM;

void or_v3_set_rope_variant(int variant) { rope_variant = variant; }

static float rope_pow(float theta, float e)
{
    if (rope_variant == OR_ROPE_GLIBC)
        return powf(theta, e);
    if (rope_variant == OR_ROPE_POWF_CR)
        return (float)powl((long double)theta, (long double)e);
    return or_powf(theta, e);
}

/* model.rs:376-394 */
void or_v3_rope_at(const or_v3_cfg *c, size_t pos, float *cs, float *sn)
{
    size_t half = c->qk_head_dim / 2;
    int glibc = rope_variant == OR_ROPE_GLIBC;
    for (size_t i = 0; i < half; i++) {
        float freq = 1.0f / rope_pow(c->rope_theta, (float)(2 * i) / (float)c->qk_head_dim);
        float angle = (float)pos * freq;
        cs[i] = glibc ? cosf(angle) : or_cosf(angle);
        sn[i] = glibc ? sinf(angle) : or_sinf(angle);
    }
}

/* mhc.rs:59-74 */
static float pre_off(size_t layer, size_t lane, size_t lanes)
{
    return lane == layer % lanes ? 4.0f : -4.0f;
}
static float post_off(size_t layer, size_t lane, size_t lanes)
{
    return lane == layer % lanes ? 0.0f : -4.0f;
}

/* mhc.rs:79-102: rows (in: nx . phi_pre, out: the gates) and u, the gated
 * lane sum. */
void or_v3_mix_down(const float *lanes, float *rows, float a_pre, const float *b_pre,
                    size_t layer, size_t n, size_t d, float *u)
{
    for (size_t lane = 0; lane < n; lane++)
        rows[lane] = sigmoid(a_pre * rows[lane] + b_pre[lane] + pre_off(layer, lane, n));
    for (size_t c = 0; c < d; c++) {
        float acc = 0.0f;
        for (size_t lane = 0; lane < n; lane++)
            acc += rows[lane] * lanes[lane * d + c];
        u[c] = acc;
    }
}

/* mhc.rs:109-152: post (n) and res (n*n) in: nx . phi rows, out: the gates
 * applied; lanes (n x d) get the doubly-stochastic remix plus post * y. */
void or_v3_scatter_up(float *lanes, float *post, float *res, const float *y, float a_post,
                      const float *b_post, float a_res, const float *b_res, size_t layer, size_t n,
                      size_t d)
{
    for (size_t lane = 0; lane < n; lane++)
        post[lane] = 2.0f * sigmoid(a_post * post[lane] + b_post[lane] + post_off(layer, lane, n));
    for (size_t x = 0; x < n * n; x++)
        res[x] = a_res * res[x] + b_res[x];
    or_sinkhorn(res, n);
    float *scratch = malloc(n * d * sizeof(float));
    memcpy(scratch, lanes, n * d * sizeof(float));
    for (size_t i = 0; i < n; i++) {
        float hp = post[i];
        for (size_t c = 0; c < d; c++) {
            float acc = 0.0f;
            for (size_t j = 0; j < n; j++)
                acc += res[i * n + j] * scratch[j * d + c];
            lanes[i * d + c] = acc + hp * y[c];
        }
    }
    free(scratch);
}

/* model.rs:150-375: one decode position; logits (logit_rows) into `out`. */
void or_v3_decode_step(const or_v3_model *m, or_v3_cache *cache, uint32_t token, float *out)
{
    const or_v3_cfg *cfg = &m->cfg;
    size_t d = cfg->d_model, n = cfg->mhc_lanes, pos = cache->pos;
    size_t qd = cfg->num_heads * cfg->qk_head_dim, kd = cfg->num_kv_heads * cfg->qk_head_dim;
    size_t vd = cfg->num_kv_heads * cfg->v_head_dim, od = cfg->num_heads * cfg->v_head_dim;
    size_t rows = cfg->out_vocab ? cfg->out_vocab : cfg->vocab_size;

    push_token(cache, token);

    /* Engram for this position (model.rs:162-191). */
    size_t nt = cfg->n_orders * cfg->e_heads, sub = cfg->e_sub_dim, ns = cfg->n_sites;
    size_t here = cache->n_tokens - 1;
    uint32_t *idx = malloc(cache->n_tokens * nt * sizeof(uint32_t));
    or_engram_indices(cache->tokens, cache->n_tokens, cfg->orders, cfg->n_orders, cfg->e_heads,
                      (uint32_t)cfg->e_slots, cfg->e_seed_heads, idx);
    float *ek = calloc(ns * d, sizeof(float)), *ev = calloc(ns * d, sizeof(float));
    float *fetched = calloc(nt * sub, sizeof(float));
    for (size_t s = 0; s < ns; s++) {
        const or_v3_engram *site = &m->engrams[s];
        for (size_t t = 0; t < nt; t++) {
            float *dst = fetched + t * sub;
            if (or_ngram_valid(pos, t, cfg->orders, cfg->e_heads))
                or_cq_dequantize_row(site->tables, t * cfg->e_slots + idx[here * nt + t], dst);
            else
                memset(dst, 0, sub * sizeof(float));
        }
        or_cq_matvec(site->key_proj, fetched, ek + s * d);
        or_cq_matvec(site->value_proj, fetched, ev + s * d);
        engram_conv_step(cache, s, site->taps, ev + s * d);
    }
    free(idx);
    free(fetched);

    /* Lane stream (model.rs:194-203). */
    float *lanes = malloc(n * d * sizeof(float)), *emb = malloc(d * sizeof(float));
    size_t tok = token < cfg->vocab_size ? token : cfg->vocab_size - 1;
    or_cq_dequantize_row(m->embedding, tok, emb);
    for (size_t i = 0; i < d; i++)
        emb[i] *= m->embed_scale;
    for (size_t l = 0; l < n; l++)
        memcpy(lanes + l * d, emb, d * sizeof(float));

    size_t half = cfg->qk_head_dim / 2;
    float cs[128], sn[128];
    or_v3_rope_at(cfg, pos, cs, sn);
    (void)half;

    float *nx = malloc(n * d * sizeof(float)), *nx_prep = malloc(m->phi_pre->in_padded * sizeof(float));
    float hpre[16], hpost[16], hres[256];
    float *scratch = malloc(n * d * sizeof(float)), *u = malloc(d * sizeof(float));
    float *bx = malloc(d * sizeof(float)), *h = malloc(d * sizeof(float));
    float *q = malloc(qd * sizeof(float)), *k = malloc(kd * sizeof(float)), *v = malloc(vd * sizeof(float));
    float *attn = malloc(od * sizeof(float)), *gate = malloc(od * sizeof(float));
    float *proj = malloc(d * sizeof(float)), *mlp_out = malloc(d * sizeof(float)), *y = malloc(d * sizeof(float));

    for (size_t li = 0; li < cfg->num_layers; li++) {
        const or_v3_layer *L = &m->layers[li];
        /* mix down (mhc.rs:80-103) */
        rms_unit_to(lanes, nx, n * d);
        or_cq_prepare_input(m->phi_pre, nx, nx_prep);
        or_cq_matvec_rows_prepared(m->phi_pre, nx_prep, li * n, n, hpre);
        or_v3_mix_down(lanes, hpre, m->a_pre[li], m->b_pre + li * n, li, n, d, u);
        memcpy(bx, u, d * sizeof(float));
        for (size_t s = 0; s < ns; s++)
            if (cfg->sites[s] == li) {
                or_v3_apply_site(bx, ek + s * d, ev + s * d, d);
                break;
            }

        memcpy(h, bx, d * sizeof(float));
        zc_rms_norm_vec(h, L->norm_in, d);
        or_cq_matvec(L->q_proj, h, q);
        or_cq_matvec(L->k_proj, h, k);
        or_cq_matvec(L->v_proj, h, v);
        if (cfg->qkv_conv_taps > 0) {
            conv_step(cache, cache->q_tail[li], L->q_taps, q, qd);
            conv_step(cache, cache->k_tail[li], L->k_taps, k, kd);
            conv_step(cache, cache->v_tail[li], L->v_taps, v, vd);
        }
        or_v3_norm_and_rope(q, L->q_norm, cs, sn, cfg->num_heads, cfg->qk_head_dim);
        or_v3_norm_and_rope(k, L->k_norm, cs, sn, cfg->num_kv_heads, cfg->qk_head_dim);
        if (cache->int8)
            or_quant_rows(q, 1, cfg->num_heads, cfg->qk_head_dim);
        or_ring_write_kv(cache->rings[li], pos, k, v);
        size_t lo, hi;
        or_ring_span(cache->rings[li], pos, &lo, &hi);
        or_ring_attend_step(cache->rings[li], q, lo, hi, cfg->num_heads, attn);

        or_cq_matvec(L->gate_proj, h, gate);
        for (size_t i = 0; i < od; i++)
            attn[i] *= sigmoid(gate[i]);
        or_cq_matvec(L->out_proj, attn, proj);
        zc_rms_norm_vec(proj, L->post_norm, d);
        float agate = sigmoid(L->attn_gate);
        for (size_t i = 0; i < d; i++)
            bx[i] += agate * proj[i];

        memcpy(proj, bx, d * sizeof(float));
        zc_rms_norm_vec(proj, L->pre_hada, d);
        or_hadamard_mlp(proj, d, &L->mlp, m->p1, m->p2, cfg->hada_n, mlp_out);
        for (size_t i = 0; i < d; i++)
            bx[i] += mlp_out[i];
        for (size_t c = 0; c < d; c++)
            y[c] = bx[c] - u[c];

        /* scatter up (mhc.rs:111-152) */
        rms_unit_to(lanes, nx, n * d);
        or_cq_prepare_input(m->phi_post, nx, nx_prep);
        or_cq_matvec_rows_prepared(m->phi_post, nx_prep, li * n, n, hpost);
        or_cq_prepare_input(m->phi_res, nx, nx_prep);
        or_cq_matvec_rows_prepared(m->phi_res, nx_prep, li * n * n, n * n, hres);
        or_v3_scatter_up(lanes, hpost, hres, y, m->a_post[li], m->b_post + li * n, m->a_res[li],
                         m->b_res + li * n * n, li, n, d);
    }
    cache->pos++;

    float *x = malloc(d * sizeof(float));
    for (size_t c = 0; c < d; c++) {
        float acc = 0.0f;
        for (size_t lane = 0; lane < n; lane++)
            acc += lanes[lane * d + c];
        x[c] = acc / (float)n;
    }
    zc_rms_norm_vec(x, m->final_norm, d);
    float *full = malloc(cfg->vocab_size * sizeof(float));
    or_cq_matvec(m->embedding, x, full);
    memcpy(out, full, rows * sizeof(float));
    free(full); free(x);
    free(ek); free(ev); free(lanes); free(emb); free(nx); free(nx_prep); free(scratch); free(u);
    free(bx); free(h); free(q); free(k); free(v); free(attn); free(gate); free(proj);
    free(mlp_out); free(y);
}

/* One decode step for each of `n` sessions (V3Model::decode_step per
 * session, v3/model.rs:150-375), sessions split across `threads` as a
 * server runs one V3Cache per session on its pool (v3_engine.rs:547-560);
 * each session's step runs serially.  logits: [n][logit rows]. */
void or_v3_decode_sessions(const or_v3_model *m, or_v3_cache **caches, const uint32_t *tokens,
                           size_t n, float *logits, int threads)
{
    size_t rows = m->cfg.out_vocab ? m->cfg.out_vocab : m->cfg.vocab_size;
    int saved = or_get_threads();
    or_set_threads(1, OR_SPLIT_REFERENCE);
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(dynamic, 1)
    for (long i = 0; i < (long)n; i++)
        or_v3_decode_step(m, caches[i], tokens[i], logits + (size_t)i * rows);
    or_set_threads(saved, OR_SPLIT_REFERENCE);
}

static uint64_t splitmix64(uint64_t *s)
{
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* For timing only: put a fresh int8 cache, made with a hint of at least
 * `pos` + the steps to be timed (so its rings need not grow), at position
 * `pos` as if `pos` tokens had been decoded -- every slot's codes and
 * scales, the conv and Engram tails and the token history filled from a
 * seeded generator -- so that a decode step's work (spans, reads) is that
 * of a session at `pos` without prefilling it. */
void or_v3_cache_fill_synthetic(or_v3_cache *k, size_t pos, uint64_t seed)
{
    const or_v3_cfg *c = &k->cfg;
    uint64_t st = seed;
    for (size_t li = 0; li < c->num_layers; li++) {
        or_ring *r = k->rings[li];
        size_t kn = r->slots * r->num_kv_heads * r->qk_head_dim;
        size_t vn = r->slots * r->num_kv_heads * r->v_head_dim;
        for (size_t i = 0; i < kn; i++)
            r->kq[i] = (int8_t)((int)(splitmix64(&st) % 255) - 127);
        for (size_t i = 0; i < vn; i++)
            r->vq[i] = (int8_t)((int)(splitmix64(&st) % 255) - 127);
        for (size_t i = 0; i < r->slots * r->num_kv_heads; i++) {
            r->k_scale[i] = 0.01f + (float)(splitmix64(&st) % 1000) * 1e-5f;
            r->v_scale[i] = 0.01f + (float)(splitmix64(&st) % 1000) * 1e-5f;
        }
    }
    size_t qd = c->num_heads * c->qk_head_dim, kd = c->num_kv_heads * c->qk_head_dim;
    size_t vd = c->num_kv_heads * c->v_head_dim, tt = c->qkv_conv_taps ? c->qkv_conv_taps - 1 : 0;
    for (size_t li = 0; li < c->num_layers; li++) {
        for (size_t i = 0; i < tt * qd; i++)
            k->q_tail[li][i] = (float)(splitmix64(&st) % 2001) * 1e-3f - 1.0f;
        for (size_t i = 0; i < tt * kd; i++)
            k->k_tail[li][i] = (float)(splitmix64(&st) % 2001) * 1e-3f - 1.0f;
        for (size_t i = 0; i < tt * vd; i++)
            k->v_tail[li][i] = (float)(splitmix64(&st) % 2001) * 1e-3f - 1.0f;
    }
    size_t reach = (c->e_conv_taps ? c->e_conv_taps - 1 : 0) * c->e_conv_dilation;
    for (size_t s = 0; s < c->n_sites; s++)
        for (size_t i = 0; i < reach * c->d_model; i++)
            k->engram_tail[s][i] = (float)(splitmix64(&st) % 2001) * 1e-3f - 1.0f;
    size_t keep = max_order(c);
    if (keep > OR_V3_MAX_HIST)
        keep = OR_V3_MAX_HIST;
    k->n_tokens = pos < keep ? pos : keep;
    for (size_t i = 0; i < k->n_tokens; i++)
        k->tokens[i] = 3 + (uint32_t)(splitmix64(&st) % (c->vocab_size - 3));
    k->pos = pos;
}

/* v3_engine.rs:410-420: strict '>' so the first maximum wins. */
uint32_t or_argmax(const float *x, size_t n)
{
    size_t best = 0;
    float top = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (x[i] > top) {
            top = x[i];
            best = i;
        }
    return (uint32_t)best;
}

/* Prefill by stepping: the reference asserts its batched prefill is
 * bit-identical to stepping decode_step over the prompt
 * (needle-infer/tests/v3_kv_int8.rs:190-302, v3_forward_parity.rs:133-199),
 * so stepping is the oracle for both.  Greedy generation as in
 * v3_engine.rs:250-302 without stop tokens: `steps` tokens after the prompt. */
void or_v3_generate(const or_v3_model *m, or_v3_cache *cache, const uint32_t *prompt,
                    size_t n_prompt, size_t steps, uint32_t *out_tokens, float *out_margin)
{
    size_t rows = m->cfg.out_vocab ? m->cfg.out_vocab : m->cfg.vocab_size;
    float *logits = malloc(rows * sizeof(float));
    for (size_t i = 0; i < n_prompt; i++)
        or_v3_decode_step(m, cache, prompt[i], logits);
    for (size_t s = 0; s < steps; s++) {
        uint32_t next = or_argmax(logits, rows);
        if (out_margin) {
            float top2 = -INFINITY;
            for (size_t i = 0; i < rows; i++)
                if (i != next && logits[i] > top2)
                    top2 = logits[i];
            out_margin[s] = logits[next] - top2;
        }
        out_tokens[s] = next;
        if (s + 1 < steps)
            or_v3_decode_step(m, cache, next, logits);
    }
    free(logits);
}
