/*
 * needle_amd.h -- C ABI of the MI355X (gfx950) Needle-3 hot path.
 *
 * Plain pointers and sizes only.  Unless a parameter says "host", every
 * buffer pointer is a device pointer (hipMalloc'd, or nd_malloc'd) and
 * every call is asynchronous on the context's stream; nd_ctx_synchronize()
 * waits for it.  Each call returns ND_OK (0) or an error code, and keeps a
 * per-thread message for nd_last_error(), mirroring needle_last_error
 * (crates/needle-c/include/needle.h:487, crates/needle-c/src/lib.rs:27-39).
 *
 * Citations name the reference interface each entry point replaces, as
 * path:line in the needle-rs checkout.
 */
#ifndef NEEDLE_AMD_H
#define NEEDLE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ------------------------------------------------------------ */
enum nd_status {
    ND_OK = 0,
    ND_ERR_ARG = 1,      /* invalid argument (shape, NULL, range) */
    ND_ERR_HIP = 2,      /* a HIP runtime call failed */
    ND_ERR_NOMEM = 3,    /* device or host allocation failed */
    ND_ERR_BUSY = 4,     /* the context or batch is inside a call on another
                          * host thread (see "Threads" below) */
    /* CqWeight::from_blob errors, cq.rs:76-89 (CqError), same order */
    ND_ERR_CQ_UNSUPPORTED_BITS = 11,
    ND_ERR_CQ_BAD_GROUP = 12,
    ND_ERR_CQ_BAD_CODEBOOK_LEN = 13,
    ND_ERR_CQ_SHORT_BLOB = 14,
    ND_ERR_CQ_EMPTY_SHAPE = 15,
    /* .cact v3 container: CactError (needle-infer/src/cact.rs:58-108), a
     * header that contradicts itself (V3GeometryError, v3.rs:84-90) and a
     * directory that contradicts the header (V3LayoutError, v3.rs:180-190);
     * the message names the variant and its fields */
    ND_ERR_CACT = 20,
    ND_ERR_V3_GEOMETRY = 21,
    ND_ERR_V3_LAYOUT = 22
};

/* Last error message on this thread, or NULL.  Borrowed; valid until the
 * next nd_* call on this thread.  Replaces needle_last_error
 * (needle.h:487; lib.rs:27-39). */
const char *nd_last_error(void);

/* ---- threads ----------------------------------------------------------- */
/*
 * Which objects may be shared between host threads (the reference: V3Model
 * is Send + Sync and shared by every session, a V3Cache is per session,
 * needle-infer/src/v3_engine.rs:544-561; a C handle is used by one thread at
 * a time, docs/c-ffi.md:383-393):
 *   - nd_cq and nd_v3_model are read-only once created: any number of
 *     threads may use one at once, each through its own context on the
 *     model's device;
 *   - nd_ctx (a stream and a workspace) and nd_v3_batch (sessions' caches
 *     and step state, like V3Cache) are used by one thread at a time.  They
 *     may move between threads between calls.  A call on a context or batch
 *     that another thread is inside fails with ND_ERR_BUSY and changes
 *     nothing; a batch is stepped through one context at a time;
 *   - nd_last_error() is per thread.
 * Creating and freeing an object is not concurrent with its use.
 */

/* ---- context: one device, one stream ------------------------------------ */
typedef struct nd_ctx nd_ctx;

/* A context with a non-blocking stream it creates and owns.  No reference
 * counterpart: the reference is CPU-only. */
int nd_ctx_create(int device, nd_ctx **out);
/* A context that launches on the caller's hipStream_t `stream` (NULL: the
 * device's default stream), e.g. the stream a framework's tensors live on. */
int nd_ctx_create_on_stream(int device, void *stream, nd_ctx **out);
void nd_ctx_destroy(nd_ctx *ctx);
int nd_ctx_synchronize(nd_ctx *ctx);

/* Device memory helpers, so a C caller needs no HIP headers. */
int nd_malloc(nd_ctx *ctx, size_t bytes, void **out);
int nd_free(nd_ctx *ctx, void *ptr);
int nd_memcpy_htod(nd_ctx *ctx, void *dst, const void *host_src, size_t bytes);
int nd_memcpy_dtoh(nd_ctx *ctx, void *host_dst, const void *src, size_t bytes);

/* ---- Format B: uint8 codes, one 256-entry fp32 codebook per 64 rows ----- */
/*
 * y[o] = sum_k cb[o/64][w[o*in + k]] * x[k].
 * w: [out][in] uint8; cb: [ceil(out/64)][256] f32; x: [in]; y: [out].
 * in must be a multiple of 16.  The format has no reference function; its
 * nearest analogues are the byte-LUT matvec (cq.rs:838-873) and the simple
 * reference matvec (cq.rs:393-426).
 */
int nd_cb8_gemv(nd_ctx *ctx, const uint8_t *w, const float *cb,
                const float *x, float *y, size_t out, size_t in);

/* `count` independent GEMVs in one launch: problem i reads
 * w + i*w_stride, cb + i*cb_stride, x + i*x_stride and writes
 * y + i*y_stride (strides in elements). */
int nd_cb8_gemv_batched(nd_ctx *ctx, size_t count,
                        const uint8_t *w, size_t w_stride,
                        const float *cb, size_t cb_stride,
                        const float *x, size_t x_stride,
                        float *y, size_t y_stride, size_t out, size_t in);

/* Y[m][o] = sum_k X[m][k] * cb[o/64][w[o][k]], with X and the decoded
 * weights rounded to bf16 and products accumulated in fp32 on MFMA.
 * out must be a multiple of 64 and in a multiple of 32.  Batched analogue:
 * CqWeight::matmul_rows_prepared (cq.rs:446-472). */
int nd_cb8_gemm(nd_ctx *ctx, const float *x, const uint8_t *w,
                const float *cb, float *y, size_t m, size_t out, size_t in);

/* `count` independent GEMMs in one launch: problem i reads x + i*x_stride,
 * w + i*w_stride, cb + i*cb_stride and writes y + i*y_stride (strides in
 * elements), e.g. the several projections of one prefill chunk. */
int nd_cb8_gemm_batched(nd_ctx *ctx, size_t count, const float *x, size_t x_stride,
                        const uint8_t *w, size_t w_stride, const float *cb,
                        size_t cb_stride, float *y, size_t y_stride, size_t m,
                        size_t out, size_t in);

/* ---- Format A: Cactus-Quants weights (cq.rs) ----------------------------- */
typedef struct nd_cq nd_cq;

/* Parse a CQ blob (host memory: packed LSB-first codes then FP16 norms)
 * and upload it.  Replaces CqWeight::from_blob (cq.rs:181-238); the same
 * errors in the same order (ND_ERR_CQ_*).  `codebook` (host) is the
 * 28-float cb2|cb3|cb4 header block, ignored for ternary (bits == 5). */
int nd_cq_from_blob(nd_ctx *ctx, const uint8_t *blob, size_t blob_len,
                    size_t out_feat, size_t in_feat, size_t group,
                    uint8_t bits, const float *codebook, size_t codebook_len,
                    nd_cq **out);
void nd_cq_free(nd_cq *w);
/* Geometry: CqWeight::{out_feat, in_feat, in_padded, group, bits}. */
int nd_cq_shape(const nd_cq *w, size_t *out_feat, size_t *in_feat,
                size_t *in_padded, size_t *group, uint8_t *bits);

/* xh[b] = per-group normalised FWHT of zero-padded x[b], for `batch` rows.
 * x: [batch][in_feat], xh: [batch][in_padded].  Replaces
 * CqWeight::prepare_input (cq.rs:264-274) -> fwht_normalized
 * (hadamard.rs:48-55). */
int nd_cq_prepare_input(nd_ctx *ctx, const nd_cq *w, const float *x,
                        size_t batch, float *xh);

/* y[r] = W[row_start + r] . xh, r < rows.  Replaces
 * CqWeight::matvec_rows_prepared (cq.rs:301-307 -> 721-757, 838-873).
 * Within the reference's tolerance (1e-4 * max(|want|, 1)); 2-bit and
 * ternary weights in groups of 128 with at least 655,360 rows (the
 * environment variable NEEDLE_AMD_CQ_FP4_MIN_ROWS moves the bound) run on
 * the fp4 matrix cores, the rest on lookup-table kernels. */
int nd_cq_matvec_rows_prepared(nd_ctx *ctx, const nd_cq *w, const float *xh,
                               size_t row_start, size_t rows, float *y);

/* y[b*rows + r] = W[row_start + r] . xh[b], batch-major.  Replaces
 * CqWeight::matmul_rows_prepared (cq.rs:446-472 -> 632-679). */
int nd_cq_matmul_rows_prepared(nd_ctx *ctx, const nd_cq *w, const float *xh,
                               size_t batch, size_t row_start, size_t rows,
                               float *y);

/* As nd_cq_matvec_rows_prepared / nd_cq_matmul_rows_prepared, summing in
 * the reference's order (eight lane accumulators per 128-group, element e
 * into lane e % 8, lanes added 0..7, group totals added in group order), so
 * the outputs are bit-identical to CqWeight::matvec_rows_prepared
 * (cq.rs:721-757, 838-873) and matmul_rows_prepared (cq.rs:632-679,
 * 879-906).  The Needle-3 forward uses these. */
int nd_cq_matvec_rows_exact(nd_ctx *ctx, const nd_cq *w, const float *xh,
                            size_t row_start, size_t rows, float *y);
int nd_cq_matmul_rows_exact(nd_ctx *ctx, const nd_cq *w, const float *xh,
                            size_t batch, size_t row_start, size_t rows,
                            float *y);

/* y[r] = ((0 + x[r][0]) + x[r][1]) + ... + x[r][n-1] in fp32, each add
 * rounded as the reference's sequential f32 sums round: the sums of squares
 * of rms_unit and ZCRMSNorm (kernels.rs:22-24, norm.rs:25) and the softmax
 * sum of attend_step (v3/attention.rs:361-365).  x is [rows][n], 1 <= n <=
 * 4096.  Rows whose terms are all >= +0 and finite take an exact parallel
 * method with the same bits; other rows are summed as the plain chain. */
int nd_fold_rows(nd_ctx *ctx, const float *x, size_t rows, size_t n, float *y);

/* out[i] = dequantized row rows[i] (in_feat floats each); rows is a device
 * int32 array of n row indices, a negative index giving a row of zeros (a
 * masked Engram fetch, v3/model.rs:172-183).  Replaces
 * CqWeight::dequantize_row (cq.rs:763-779), gathered. */
int nd_cq_dequantize_rows(nd_ctx *ctx, const nd_cq *w, const int32_t *rows,
                          size_t n, float *out);

/* ---- int8 KV cache (v3/cache.rs, v3/attention.rs) -------------------------- */

/* fake_quant_vec(x[r], 8) for every row r of `dim` floats, in place.
 * Replaces fake_quant_vec (cache.rs:68-73) and quant_rows
 * (v3/model.rs:99-106). */
int nd_fake_quant(nd_ctx *ctx, float *x, size_t rows, size_t dim);

/* ints[r] = quant_into(x[r]); scales[r] its scale.  Replaces quantize_rows
 * (cache.rs:113-122).  Bit-exact. */
int nd_quantize_rows(nd_ctx *ctx, const float *x, size_t rows,
                     size_t head_dim, int8_t *ints, float *scales);

/*
 * Geometry of one int8 KV block: one layer of one session.  Device layout
 * (head-major, so one kv head's span is one contiguous byte run):
 *   k  int8 [num_kv_heads][cap][qk_head_dim]    at offset 0
 *   v  int8 [num_kv_heads][cap][v_head_dim]     at nd_kv_v_offset()
 *   ks f32  [num_kv_heads][cap]                 at nd_kv_ks_offset()
 *   vs f32  [num_kv_heads][cap]                 at nd_kv_vs_offset()
 * Logical position p lives at slot p % cap.  qk_head_dim and v_head_dim
 * must be multiples of 16 and at most 256; num_heads a multiple of
 * num_kv_heads with num_heads / num_kv_heads <= 8.
 */
typedef struct nd_kv_geom {
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t qk_head_dim;
    int32_t v_head_dim;
    int32_t cap;
} nd_kv_geom;

size_t nd_kv_block_bytes(const nd_kv_geom *g);
size_t nd_kv_v_offset(const nd_kv_geom *g);
size_t nd_kv_ks_offset(const nd_kv_geom *g);
size_t nd_kv_vs_offset(const nd_kv_geom *g);

/* For i < count: quantise k[i] ([num_kv_heads][qk] f32) and v[i] per kv
 * head and store them, with their scales, at slot pos[i] % cap of the block
 * at kv + i*kv_stride bytes (kv_stride 0: every row into one block, e.g. a
 * prompt).  pos: device int32[count].  Replaces V3Cache::write_kv
 * (cache.rs:346-379) -> quant_into (cache.rs:98-104); bit-exact.  The rows
 * of one call are written in parallel: two rows for one block must not map
 * to one slot (the reference's sequential writes would keep the later). */
int nd_kv_write(nd_ctx *ctx, const nd_kv_geom *g, void *kv, size_t kv_stride,
                size_t count, const int32_t *pos, const float *k,
                const float *v);

/*
 * For i < count: out[i] ([num_heads][v_head_dim]) = softmax attention of
 * q[i] ([num_heads][qk_head_dim]) over logical positions lo[i]..=hi[i] of
 * the block at kv + i*kv_stride bytes, GQA head h reading kv head
 * h / (num_heads / num_kv_heads), scores scaled by `scale`.  With
 * quant_query != 0, each query head is first fake-quantised to 8 bits
 * (quant_rows, v3/model.rs:289-293).  Requires hi[i] - lo[i] < cap.
 * Split-K over the span; partials live in a context workspace.
 * Replaces attend_step with KvStore::Int8 (attention.rs:300-377) -- and,
 * with kv_stride 0 and lo/hi per prompt row, attend (attention.rs:218-287).
 */
int nd_attend_step_i8(nd_ctx *ctx, const nd_kv_geom *g, const void *kv,
                      size_t kv_stride, size_t count, const int32_t *lo,
                      const int32_t *hi, const float *q, float scale,
                      int quant_query, float *out);

/*
 * nd_attend_step_i8 without any allocation, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No reference counterpart.
 * The same kernels and the same results, bit for bit; the split-K
 * partials live in a fixed 4 MiB device array per GPU (held until the
 * process ends) instead of the context workspace.  A call whose partials
 * need more -- count * num_heads * splits * (v_head_dim + 2) floats above
 * 1048576 -- fails with ND_ERR_ARG.  The span is split only while
 * count * num_kv_heads < 4 * CUs, so the partials stay below
 * 8 * CUs * (num_heads / num_kv_heads) * (v_head_dim + 2) floats: on a
 * 256-CU MI355X only 8 query heads per kv head can exceed the array.
 * Every call on a GPU shares that GPU's array: calls that overlap on one
 * GPU (two streams, or two threads) race.
 */
int nd_attend_step_i8_noalloc(nd_ctx *ctx, const nd_kv_geom *g, const void *kv,
                              size_t kv_stride, size_t count, const int32_t *lo,
                              const int32_t *hi, const float *q, float scale,
                              int quant_query, float *out);

/* As nd_attend_step_i8, bit-identical to attend_step over the int8 view
 * (attention.rs:327-377): each score is one dot chain over the head dim,
 * scaled by the key scale and then `scale`; the softmax sum and every
 * output column are single chains over the span in position order; exp is
 * libm's expf algorithm.  Also requires cap <= 12288 (one span's scores and
 * a 16 KB chunk of V rows sit in LDS).  The Needle-3 forward uses this. */
int nd_attend_step_i8_exact(nd_ctx *ctx, const nd_kv_geom *g, const void *kv,
                            size_t kv_stride, size_t count, const int32_t *lo,
                            const int32_t *hi, const float *q, float scale,
                            int quant_query, float *out);

/* ---- libm on the device (crates/needle-core/src/math.rs:3-46) ------------- */

/* y[i] = f(x[i]) for i < n (device buffers), f the device copy of the
 * reference's libm 0.2.16 wrapper that the device path uses: fn 0 expf
 * (math::exp), 1 logf (math::ln), 2 the sigmoid 1 / (1 + expf(-x))
 * (ops::sigmoid).  The same bits as the reference's functions for every
 * input (the msun algorithms, restated); used to check the device copies. */
int nd_libm_map(nd_ctx *ctx, int fn, const float *x, size_t n, float *y);

/* ---- f32 KV cache (KvPrecision::F32, v3/cache.rs:177-238, 355-362) ------- */

/*
 * An f32 KV block of the same geometry: the layer's keys and values stored
 * as written, head-major like the int8 block,
 *   k  f32 [num_kv_heads][cap][qk_head_dim]     at offset 0
 *   v  f32 [num_kv_heads][cap][v_head_dim]      at nd_kv_f32_v_offset()
 * each part 256-byte aligned.  Logical position p lives at slot p % cap.
 */
size_t nd_kv_f32_block_bytes(const nd_kv_geom *g);
size_t nd_kv_f32_v_offset(const nd_kv_geom *g);

/* For i < count: store k[i] ([num_kv_heads][qk] f32) and v[i] unchanged at
 * slot pos[i] % cap of the f32 block at kv + i*kv_stride bytes (kv_stride
 * 0: every row into one block).  pos: device int32[count].  Replaces
 * V3Cache::write_kv with KvPrecision::F32 (cache.rs:346-362).  As for
 * nd_kv_write, two rows of one call must not map to one slot of a block. */
int nd_kv_write_f32(nd_ctx *ctx, const nd_kv_geom *g, void *kv, size_t kv_stride,
                    size_t count, const int32_t *pos, const float *k,
                    const float *v);

/* As nd_attend_step_i8_exact over the f32 block: bit-identical to
 * attend_step over KvStore::F32 (F32View, attention.rs:166-189, 327-377):
 * each score is one dot chain q . k over the head dim, then times `scale`;
 * the weights are exp(s - max) * (1 / sum), each output column one chain
 * of w * v over the span.  The query is used as given (the reference
 * fake-quantises it for the int8 cache only, v3/model.rs:289-293).
 * Requires v_head_dim <= 128 and cap <= 8192. */
int nd_attend_step_f32_exact(nd_ctx *ctx, const nd_kv_geom *g, const void *kv,
                             size_t kv_stride, size_t count, const int32_t *lo,
                             const int32_t *hi, const float *q, float scale,
                             float *out);

/* ---- Needle-3 forward on the device (v3/model.rs, v3/cache.rs) ----------- */

/* V3Config (crates/needle-core/src/v3/config.rs:45-77), Engram flattened. */
typedef struct nd_v3_cfg {
    int32_t vocab_size, out_vocab, d_model, num_heads, num_kv_heads, num_layers;
    int32_t qk_head_dim, v_head_dim, max_seq_len, hada_n, mhc_lanes;
    float rope_theta;
    int32_t sliding_window, n_global, global_layers[64], qkv_conv_taps;
    int32_t n_orders, orders[8], e_heads, e_slots, e_sub_dim, n_sites, sites[64];
    int32_t e_conv_taps, e_conv_dilation, e_seed_heads;
} nd_v3_cfg;

enum { ND_REC_F32 = 1, ND_REC_CQ = 3 };

/* One container record (host memory): a Cactus-Quants blob (kind 3, shape
 * out x in, group, bits) or f32 data (kind 1; `in` is the second dimension
 * of a 2-D tensor, else 1). */
typedef struct nd_v3_record {
    int32_t kind;
    const void *data;
    size_t len, out, in, group, bits;
} nd_v3_record;

typedef struct nd_v3_model nd_v3_model;
typedef struct nd_v3_batch nd_v3_batch;

/* Upload a model from records in the canonical container order walked by
 * V3Layout::derive (crates/needle-infer/src/v3.rs:236-330) and bound as in
 * model_from_cact (v3.rs:395-482).  `codebook` (host) is the 28-float
 * cb2|cb3|cb4 header block.  ND_ERR_ARG names the first record that does not
 * fit the geometry. */
int nd_v3_model_create(nd_ctx *ctx, const nd_v3_cfg *cfg, const float *codebook,
                       size_t codebook_len, const nd_v3_record *recs, size_t n,
                       nd_v3_model **out);
void nd_v3_model_free(nd_v3_model *m);
/* Rows of the tied head scored per position (V3Config::logit_rows). */
size_t nd_v3_logit_rows(const nd_v3_model *m);

/* `sessions` decode sessions with int8 KV caches (V3Cache::with_precision
 * (.., KvPrecision::Int8), cache.rs:177-238) able to hold `max_len`
 * positions each; `hint` sizes the reference's logical ring growth. */
int nd_v3_batch_create(nd_ctx *ctx, const nd_v3_model *m, size_t sessions, size_t max_len,
                       size_t hint, nd_v3_batch **out);
/* As nd_v3_batch_create, for steps of up to `max_chunk` consecutive
 * positions per session (nd_v3_prefill): the per-row buffers hold
 * sessions * max_chunk rows and each local layer's ring max_chunk - 1 more
 * positions than its window, so that a step's own writes never reach a slot
 * one of its rows still attends over.  No reference counterpart: it sizes
 * the device state behind the reference's chunked prefill
 * (V3Model::prefill, v3/model.rs:512-523). */
int nd_v3_batch_create_chunked(nd_ctx *ctx, const nd_v3_model *m, size_t sessions,
                               size_t max_len, size_t hint, size_t max_chunk,
                               nd_v3_batch **out);
/* As nd_v3_batch_create_chunked with the sessions' KV precision chosen:
 * kv_int8 != 0 is KvPrecision::Int8 (the batch the other constructors
 * make), kv_int8 == 0 KvPrecision::F32 -- the default of needle_v3_run and
 * needle_v3_generate(kv_int8 = false) (crates/needle-c/src/v3.rs:219-250):
 * keys and values cached as f32 (nd_kv_write_f32) and read through the f32
 * view (nd_attend_step_f32_exact), the query not fake-quantised.  Steps
 * stay bit-identical to V3Model::decode_step / prefill with that cache. */
int nd_v3_batch_create_ex(nd_ctx *ctx, const nd_v3_model *m, size_t sessions,
                          size_t max_len, size_t hint, size_t max_chunk, int kv_int8,
                          nd_v3_batch **out);
void nd_v3_batch_free(nd_v3_batch *b);
/* Whether this batch's single-position steps (nd_v3_step) run as one
 * captured HIP graph -- off by default: the step's kernels are captured on
 * the second such step and replayed from then on, on a stream of the batch's
 * own ordered after and before the context's stream by events.  Off: every
 * step is enqueued kernel by kernel, which measures faster on ROCm 7.2
 * (1.85 against 2.03 ms per single-session step).  The results are identical
 * either way; a batch whose capture fails runs eagerly.  No reference
 * counterpart: it is a way of running the reference's decode_step loop. */
int nd_v3_batch_set_graphs(nd_v3_batch *b, int on);
/* Each session's next write position (V3Cache::pos). */
int nd_v3_positions(const nd_v3_batch *b, int32_t *pos);

/* One decode position for every session: tokens[i] (host) is fed to
 * session i, exactly as V3Model::decode_step (v3/model.rs:150-375) with an
 * int8 cache -- the logits are bit-identical to the reference's CPU order.
 * When `next` (host, per session) is given it receives the greedy argmax of
 * the logits, first maximum winning (needle-infer/src/v3_engine.rs:410-420),
 * and the call returns once it is known; otherwise the step is only queued
 * on the context's stream (a side stream of the batch carries the mHC
 * gates, joined by events).  When `logits` (device, [sessions][logit_rows])
 * is given the logits are copied there.  A prompt is prefilled by stepping
 * it: the reference's batched prefill is bit-identical to stepping
 * (needle-infer/tests/v3_kv_int8.rs:190-302).  Steps on one batch must not
 * be issued from two threads at once.  After an error the batch's state is
 * undefined; free it. */
int nd_v3_step(nd_ctx *ctx, const nd_v3_model *m, nd_v3_batch *b, const int32_t *tokens,
               int32_t *next, float *logits);

/* out[r] = the greedy token of row r of x ([count][n] fp32): the index of
 * its first maximum under a strict `>` scan from -inf, so a tie keeps the
 * lower index, NaN never wins and a row of -inf or NaN gives 0.  Replaces
 * the engine's argmax (needle-infer/src/v3_engine.rs:410-420); the same
 * kernel picks nd_v3_step's `next`. */
int nd_argmax_rows(nd_ctx *ctx, const float *x, size_t count, size_t n, int32_t *out);

/* `count` consecutive positions for every session in one pass over the
 * layers: tokens (host) is [sessions][count], session-major.  Replaces the
 * reference's chunked prefill (V3Model::prefill -> forward_impl_pooled,
 * v3/model.rs:512-523, 550-980), which is bit-identical to stepping
 * (needle-infer/tests/v3_kv_int8.rs:269-282): so is this -- the caches,
 * the conv tails and the logits of the last position equal `count`
 * nd_v3_step calls.  Every position's projections, attention and MLP run
 * as rows of one batch; the causal conv and the Engram conv read the step's
 * earlier rows.  `next` and `logits` as for nd_v3_step, for each session's
 * last position.  count <= the batch's max_chunk. */
int nd_v3_prefill(nd_ctx *ctx, const nd_v3_model *m, nd_v3_batch *b, const int32_t *tokens,
                  size_t count, int32_t *next, float *logits);

/* The greedy loop of V3Engine::generate_with (needle-infer/src/
 * v3_engine.rs:254-312, behind needle_v3_generate, needle-c/src/v3.rs:219-250)
 * with temperature 0 and no stop tokens, for every session at once:
 * `steps` single-position steps, the first feeding first[i] (host, [sessions];
 * e.g. the `next` of the prompt's last prefill pass), each later one the
 * greedy token of the step before.  tokens (host, [sessions][steps],
 * session-major) receives each step's greedy token: first[i] followed by
 * tokens[i][..] is the reference's out_tokens.  The choices stay on the
 * device between steps (the Engram hash of the retained ids runs there
 * too), so the device does not wait for the host between steps; the
 * tokens, caches and positions afterwards equal `steps` nd_v3_step calls
 * that feed back `next`, bit for bit.  Sessions do not stop early: a caller
 * with stop tokens truncates each row at its first one. */
int nd_v3_generate(nd_ctx *ctx, const nd_v3_model *m, nd_v3_batch *b, const int32_t *first,
                   size_t steps, int32_t *tokens);

/* nd_v3_generate for n (1..8) batches of one model at once, from one host
 * thread: batch i on context ctxs[i] (its own stream), from first[i], into
 * tokens[i].  Step k of every batch is enqueued before step k + 1 of any,
 * so the batches' launches interleave on their streams and run side by
 * side on the device (a batch's per-session kernels use one workgroup a
 * session; another batch's projections and attention fill the rest).
 * Each batch ends exactly as nd_v3_generate would leave it, bit for bit.
 * The contexts and the batches must be distinct; all are held for the
 * call.  No reference counterpart: the reference serves concurrent
 * sessions from its own threads (V3Engine per session, v3_engine.rs:544-561);
 * this is the one-thread form of that, for a server that groups its
 * sessions into a few batches.  The streams run side by side only on
 * hardware queues of their own: HIP gives a process GPU_MAX_HW_QUEUES
 * (default 4) of them, shared with every other stream, so n batches want
 * that at n + 1 or more (set before HIP starts). */
int nd_v3_generate_many(nd_ctx *const *ctxs, const nd_v3_model *m, nd_v3_batch *const *bs,
                        size_t n, const int32_t *const *first, size_t steps,
                        int32_t *const *tokens);

/* ---- the .cact v3 container (needle-infer/src/cact.rs, v3.rs) ----------- */

/* Reads a Needle-3 container held in host memory (`bytes`, `len`): the
 * 49-word header, the 28-float codebook, the 44-byte directory records,
 * then the nameless canon walked and shape-checked as V3Layout::derive and
 * validate do (v3.rs:236-330), with every float slot decoded (FP16 widened
 * exactly).  Fills `cfg` as config_from_geometry does (v3.rs:25-82) and
 * `canon_records` (optional) with the number of records up to final_norm;
 * the heads manifest, probe-head tensors and tokenizer that may follow are
 * not read.  Host only.  Replaces CactV3::from_bytes (cact.rs:994-1030) with
 * config_from_geometry and V3Layout::derive. */
int nd_v3_cact_config(const void *bytes, size_t len, nd_v3_cfg *cfg, size_t *canon_records);

/* As nd_v3_cact_config, then uploads the model: the CQ blobs go up as
 * stored (no repacking), the float tensors widened to f32.  Replaces
 * model_from_cact (v3.rs:438-482). */
int nd_v3_model_from_cact(nd_ctx *ctx, const void *bytes, size_t len, nd_v3_model **out);

/* Key/value cache bytes a session of `seq_len` positions needs under `cfg`:
 * per layer min(seq_len, sliding_window) positions (all of them on a global
 * layer), each a key and a value per kv head at f32, or with kv_int8 at one
 * byte plus one f32 scale per stored head vector.  0 (and ND_ERR_ARG in
 * nd_last_error) for a null cfg.  Host only; what needle_v3_kv_bytes
 * reports.  Replaces V3Config::kv_bytes_at
 * (crates/needle-core/src/v3/config.rs:143-179). */
size_t nd_v3_kv_bytes(const nd_v3_cfg *cfg, size_t seq_len, int kv_int8);

/* ---- ladder rungs: a shallower model sliced from the full container ------ */

/* The `depth` blocks a rung of a `num_layers`-block stack keeps, ascending,
 * into kept[0..depth): the first `depth` of the ladder order (both
 * endpoints, then the widest remaining gap split at its midpoint, leftmost
 * first).  ND_ERR_ARG ("depth is outside the ladder") unless
 * 2 <= depth <= num_layers.  Host only.  Replaces ladder_layer_indices
 * (crates/needle-core/src/v3/ladder.rs:67-74). */
int nd_v3_ladder(size_t num_layers, size_t depth, int32_t *kept);

/* As nd_v3_cact_config for the `depth`-block rung: the parent geometry is
 * read and checked, the ladder applied, every block's shapes checked and
 * the kept blocks' tensors decoded; `cfg` receives the rung's geometry (kept
 * blocks renumbered, global layers and Engram sites following their blocks)
 * and `kept` (optional, `depth` entries) the parent blocks kept.  depth ==
 * num_layers is the ordinary read.  Host only.  Replaces config_at_depth
 * (needle-infer/src/v3.rs:620-637) with model_from_cact_at_depth's checks
 * (v3.rs:656-664). */
int nd_v3_cact_config_at_depth(const void *bytes, size_t len, size_t depth, nd_v3_cfg *cfg,
                               int32_t *kept);

/* Uploads the `depth`-block rung of a full-depth container: the kept blocks
 * whole, the mHC scalars of the kept blocks, the phi lane rows of the kept
 * blocks (packed rows and FP16 norms copied unchanged: nothing is
 * re-quantised), the Engram sites on kept blocks, the rest as stored.
 * Replaces model_from_cact_at_depth (v3.rs:656-734) behind
 * V3Engine::load_with_depth and needle_v3_load_with_depth. */
int nd_v3_model_from_cact_at_depth(nd_ctx *ctx, const void *bytes, size_t len, size_t depth,
                                   nd_v3_model **out);

#ifdef __cplusplus
}
#endif
#endif /* NEEDLE_AMD_H */
