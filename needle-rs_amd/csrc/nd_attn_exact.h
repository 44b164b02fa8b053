// The reference-order decode attention over the int8 (or f32) KV view
// (attend_step, v3/attention.rs:300-377 and 166-216), device code shared by
// the attention entry points and the decode step's launch that forms the
// step's own q, k and v first.  Every float operation is the reference's,
// in its order.
#pragma once

#include "nd_fold.h"
#include "nd_kv_internal.h"
#include "nd_libm.h"
#include "nd_ref_order.h"

#include <hip/hip_runtime.h>

#include <type_traits>

namespace ndattn {

__device__ inline float i8_lane(uint32_t dw, int b) { return float(int32_t(dw << (24 - 8 * b)) >> 24); }

// Output column `lane` (0..63, all 64 lanes of the wave) of one head, with
// `gate` set: attn * sigmoid(gate) (v3/model.rs:309-312), then butterfly
// stages h = 1..32 of the normalised FWHT prepare_input applies to the
// out projection's 128-wide groups (hadamard.rs:24-42): with a 64-wide head
// each half of a group is one head, and those stages pair columns within
// it.  The last stage (h = 64, across the two heads) and the 1/sqrt(128)
// scale are left to the projection's activation load.
__device__ inline float gate_half_fwht(float v, const float *gate, int lane)
{
    if (!gate) return v;
    v = v * nd_sigmoidf(gate[lane]);
    return ndl::wave_fwht64(v);
}

// The same arithmetic, with the value pass split between roles.  Of the 256
// threads, CW consumer waves hold one output column per lane and run the
// column chains; the other 4 - CW producer waves stream V a chunk of
// positions ahead, form each product ((e * inv) * v_scale) * v into an LDS
// double buffer, and keep kPrefetch chunks of V loads in flight.  A chain
// then costs one add per position.  At most 128 VGPRs, so four workgroups fit
// a CU and a 64-session layer (768 workgroups) is resident at once.
// Blocks are numbered so that the heads sharing a kv head run on one XCD
// (workgroups are dealt to the 8 XCDs round-robin), where they share that
// XCD's L2 copy of the span.
constexpr int kAttn2Threads = 256;
constexpr int kProdBuf = 64 * 52;  // products per buffer: VD x (T + 4) <= 64 x 52, 128 x 20
constexpr int kPrefetch = 8;
constexpr int kAttn2MaxCap = 8192;  // scores 32 KB + two product buffers 26 KB
constexpr int kScoreBatch = 4;      // positions per thread whose K rows load together
// Spans of 1024..4096 positions sum by the parallel fold, its unrolled loop
// sized to the terms a thread holds (4, 9 or 16: the masked iterations past
// a thread's terms cost as much as real ones).  Measured against the chain
// (12 q / 2 kv heads, qk 48, vd 64, one launch): span 4096 53.6 -> 45.9 us
// a workgroup; span 2048 at 64 sessions 37.5 -> 35.9 us, at one session
// 24.6 -> 23.7; span 1024 at one session 15.3 -> 14.7, at 64 sessions no
// change.  Shorter spans keep the chain (at 384, 10.2 against 12.8 us for
// the fold at 16 a thread).
constexpr int kAttnFoldMin = 1024;
constexpr int kAttnFoldC = 16;
static_assert(sizeof(NdFoldLds<kAttn2Threads>) <= 2 * kProdBuf * sizeof(float),
              "the fold's LDS lives in the product buffers");

// The last position of a span whose K and V rows the launch itself formed
// (the decode step's conv, norm, RoPE and quantisation in the attention
// launch): its int8 rows and scales, in LDS.  The launch writes them to the
// ring slot too, but reads them only from here.
struct AttnNewRow {
    uint4 k[4];  // qk <= 64 codes
    uint4 v[4];  // vd <= 64 codes
    float ks, vs;
};

// LDS of one workgroup besides the dynamic part (scores, product buffers).
struct AttnLds {
    float qs[ndkv::kMaxDim];  // the query head, fake-quantised when asked
    float red[kAttn2Threads / 64];
    float total;
};

// One (q, key) score chain per position, QC = qk / 16 pieces of 16 codes
// (0: any qk, read piece by piece).  With QC set, a thread loads the K rows
// of kScoreBatch positions at once and runs their chains interleaved.
template <int QC, int NT, bool NEW>
__device__ __forceinline__ float attn_scores(const ndkv::Geom &g, const float *qs, const int8_t *kb,
                                             const float *ks, int base, int span, float scale,
                                             float *sc, const AttnNewRow *nr)
{
    static_assert(!NEW || QC > 0, "the launch's own row needs whole 16-code pieces");
    const int tid = threadIdx.x;
    float mx = -INFINITY;
    if constexpr (QC > 0) {
        // U positions t0, t0 + NT, ... (all inside the span) with their K
        // rows loaded together and their chains interleaved
        auto batch = [&](auto uc, int t0) {
            constexpr int U = decltype(uc)::value;
            uint4 kw[U][QC];
            float ksv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                int slot = base + t0 + u * NT;
                if (slot >= g.cap) slot -= g.cap;
                const uint4 *kr = reinterpret_cast<const uint4 *>(kb + size_t(slot) * (16 * QC));
#pragma unroll
                for (int c = 0; c < QC; ++c) kw[u][c] = kr[c];
                ksv[u] = ks[slot];
            }
            if constexpr (NEW) {
                // the span's last position: the launch's own row
                if (t0 + (U - 1) * NT >= span - 1) {
#pragma unroll
                    for (int u = 0; u < U; ++u)
                        if (t0 + u * NT == span - 1) {
#pragma unroll
                            for (int c = 0; c < QC; ++c) kw[u][c] = nr->k[c];
                            ksv[u] = nr->ks;
                        }
                }
            }
            float acc[U];
#pragma unroll
            for (int u = 0; u < U; ++u) acc[u] = 0.0f;
#pragma unroll
            for (int c = 0; c < QC; ++c) {
#pragma unroll
                for (int d = 0; d < 4; ++d) {
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const float qv = qs[c * 16 + d * 4 + b];
#pragma unroll
                        for (int u = 0; u < U; ++u) {
                            const uint32_t dw = d == 0 ? kw[u][c].x
                                              : d == 1 ? kw[u][c].y
                                              : d == 2 ? kw[u][c].z
                                                       : kw[u][c].w;
                            acc[u] += qv * i8_lane(dw, b);
                        }
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float s = acc[u] * ksv[u] * scale;
                sc[t0 + u * NT] = s;
                if (s > mx) mx = s;
            }
        };
        // whole batches, then this thread's last one to three positions in
        // batches of 2 and 1: a thread with one position more than another
        // does a fraction of a batch more, not a whole batch of mostly
        // unused chains (spans past a multiple of 4 * NT)
        int t0 = tid;
        for (; t0 + (kScoreBatch - 1) * NT < span; t0 += NT * kScoreBatch)
            batch(std::integral_constant<int, kScoreBatch>{}, t0);
        if (t0 + NT < span) {
            batch(std::integral_constant<int, 2>{}, t0);
            t0 += 2 * NT;
        }
        if (t0 < span) batch(std::integral_constant<int, 1>{}, t0);
    } else {
        for (int t = tid; t < span; t += NT) {
            int slot = base + t;
            if (slot >= g.cap) slot -= g.cap;
            const uint4 *kr = reinterpret_cast<const uint4 *>(kb + size_t(slot) * g.QK);
            float acc = 0.0f;
            for (int c = 0; c < g.QK / 16; ++c) {
                const uint4 w = kr[c];
                const uint32_t dws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int d = 0; d < 4; ++d)
#pragma unroll
                    for (int b = 0; b < 4; ++b) acc += qs[c * 16 + d * 4 + b] * i8_lane(dws[d], b);
            }
            const float s = acc * ks[slot] * scale;
            sc[t] = s;
            if (s > mx) mx = s;
        }
    }
    return mx;
}

// The same over the f32 view (F32View::dot, attention.rs:171-178): each
// score is its own qk-long chain of q[e] * k[e], then times 1/sqrt(qk); no
// key scale.  QC > 0: two positions' K rows load together and their chains
// run interleaved.
template <int QC, int NT>
__device__ __forceinline__ float attn_scores_f32(const ndkv::Geom &g, const float *qs,
                                                 const float *kb, int base, int span, float scale,
                                                 float *sc)
{
    constexpr int kB = QC >= 4 ? 1 : 2;  // K rows in registers: at most 96 floats
    const int tid = threadIdx.x;
    float mx = -INFINITY;
    if constexpr (QC > 0) {
        for (int t0 = tid; t0 < span; t0 += NT * kB) {
            float4 kw[kB][4 * QC];
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                const int t = t0 + u * NT;
                int slot = base + (t < span ? t : 0);
                if (slot >= g.cap) slot -= g.cap;
                const float4 *kr = reinterpret_cast<const float4 *>(kb + size_t(slot) * (16 * QC));
#pragma unroll
                for (int c = 0; c < 4 * QC; ++c) kw[u][c] = kr[c];
            }
            float acc[kB];
#pragma unroll
            for (int u = 0; u < kB; ++u) acc[u] = 0.0f;
#pragma unroll
            for (int c = 0; c < 4 * QC; ++c) {
#pragma unroll
                for (int u = 0; u < kB; ++u) {
                    acc[u] += qs[4 * c] * kw[u][c].x;
                    acc[u] += qs[4 * c + 1] * kw[u][c].y;
                    acc[u] += qs[4 * c + 2] * kw[u][c].z;
                    acc[u] += qs[4 * c + 3] * kw[u][c].w;
                }
            }
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                const int t = t0 + u * NT;
                if (t < span) {
                    const float s = acc[u] * scale;
                    sc[t] = s;
                    if (s > mx) mx = s;
                }
            }
        }
    } else {
        for (int t = tid; t < span; t += NT) {
            int slot = base + t;
            if (slot >= g.cap) slot -= g.cap;
            const float4 *kr = reinterpret_cast<const float4 *>(kb + size_t(slot) * g.QK);
            float acc = 0.0f;
            for (int c = 0; c < g.QK / 4; ++c) {
                const float4 w = kr[c];
                acc += qs[4 * c] * w.x;
                acc += qs[4 * c + 1] * w.y;
                acc += qs[4 * c + 2] * w.z;
                acc += qs[4 * c + 3] * w.w;
            }
            const float s = acc * scale;
            sc[t] = s;
            if (s > mx) mx = s;
        }
    }
    return mx;
}

// One value item of the producers: 16 columns of one position, int8 codes
// and the position's scale, or f32 values.
template <bool KF>
struct AttnVItem {
    uint4 v;
    float s;
};
template <>
struct AttnVItem<true> {
    float4 v[4];
};

// acc += v[0]; acc += v[1]; ... acc += v[n-1] in index order, v 16-byte
// aligned LDS with at least 32 readable floats past v[n-1].  Terms go in
// groups of 32, read into two register sets in turn, so that a group's
// reads are in flight while the group before it is added.
__device__ inline float lds_chain(float acc, const float *v, int n)
{
    const int G = (n + 31) / 32;
    if (G == 0) return acc;
    float4 a[8], b[8];
    auto rd = [&](float4 (&r)[8], int gi) {
        const float4 *v4 = reinterpret_cast<const float4 *>(v + gi * 32);
#pragma unroll
        for (int u = 0; u < 8; ++u) r[u] = v4[u];
    };
    auto add32 = [&](float s, const float4 (&r)[8], int m) {
        const float4 lo[4] = {r[0], r[1], r[2], r[3]};
        const float4 hi[4] = {r[4], r[5], r[6], r[7]};
        if (m >= 32) return nd_add16(nd_add16(s, lo), hi);
        s = nd_add_first(s, lo, m);
        return m > 16 ? nd_add_first(s, hi, m - 16) : s;
    };
    rd(a, 0);
    int gi = 0;
    for (; gi + 2 < G; gi += 2) {
        rd(b, gi + 1);
        acc = add32(acc, a, 32);
        rd(a, gi + 2);
        acc = add32(acc, b, 32);
    }
    if (gi + 1 < G) {
        rd(b, gi + 1);
        acc = add32(acc, a, 32);
        acc = add32(acc, b, n - (gi + 1) * 32);
    } else {
        acc = add32(acc, a, n - gi * 32);
    }
    return acc;
}

// The pass after the query head is in L.qs (written and synchronised):
// scores, softmax, the value pass and the epilogue of query head h of kv
// head kvh over the span [p0, p0 + span) of KV block blk (0 <= p0,
// 1 <= span <= cap); output column c goes to out_row[c], gated and half
// transformed when gate_row is set.  Every thread of the workgroup calls it.
// NEW: the span's last position is nr's row (int8 view, QC > 0).
// KF: the cache is the f32 view (F32View, attention.rs:166-189): f32 K/V
// rows at the f32 block's offsets, no scales, weights e * inv.
template <int CW, int QC, bool KF, bool NEW>
__device__ __forceinline__ void attn_exact2_run(const ndkv::Geom &g, const uint8_t *blk, int kvh,
                                                int p0, int span, float scale, float *sm,
                                                AttnLds &L, const AttnNewRow *nr, float *out_row,
                                                const float *gate_row)
{
    static_assert(!NEW || !KF, "the launch's own row is int8");
    constexpr int NT = kAttn2Threads;
    const int tid = threadIdx.x;
    float *sc = sm;                         // [span] scores, then exps
    float *prod = sm + ((g.cap + 3) & ~3);  // [2][kProdBuf] products
    const int base = p0 % g.cap;
    float mx;
    if constexpr (KF) {
        const float *kb = reinterpret_cast<const float *>(blk) + size_t(kvh) * g.cap * g.QK;
        mx = attn_scores_f32<QC, NT>(g, L.qs, kb, base, span, scale, sc);
    } else {
        const int8_t *kb = reinterpret_cast<const int8_t *>(blk) + size_t(kvh) * g.cap * g.QK;
        const float *ks = reinterpret_cast<const float *>(blk + g.ks_off) + size_t(kvh) * g.cap;
        mx = attn_scores<QC, NT, NEW>(g, L.qs, kb, ks, base, span, scale, sc, nr);
    }
    mx = ndkv::wave_max(mx);
    if ((tid & 63) == 0) L.red[tid >> 6] = mx;
    __syncthreads();
    mx = L.red[0];
    for (int w = 1; w < NT / 64; ++w) mx = L.red[w] > mx ? L.red[w] : mx;
    int te = tid;
    for (; te + 3 * NT < span; te += 4 * NT) {
        // four independent exps per thread in flight
        float e[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) e[u] = nd_expf(sc[te + u * NT] - mx);
#pragma unroll
        for (int u = 0; u < 4; ++u) sc[te + u * NT] = e[u];
    }
    // the thread's last one to three, one at a time
    for (; te < span; te += NT) sc[te] = nd_expf(sc[te] - mx);
    __syncthreads();

    // Products sit column-major, [VD][T + 4] per buffer: a consumer lane reads
    // four positions of its column per 16-byte read, and the 4-float pad puts
    // the columns of one read in different banks.  Producer item (pc, tl) of a
    // chunk is position tl, columns pc*16..+15; a wave's items are consecutive
    // positions of one column piece.
    constexpr int T = CW == 1 ? 48 : 16;  // positions per chunk: one item per producer
    constexpr int TS = T + 4;
    const int pieces = g.VD / 16;
    const int nch = (span + T - 1) / T;
    const bool producer = tid >= 64 * CW;
    const int pt = tid - 64 * CW;
    const int pc = pt / T, tl = pt - (pt / T) * T;
    const bool has_item = producer && pc < pieces;
    // chunks of V loads in flight: f32 items are four times the registers
    constexpr int PF = KF ? 2 : kPrefetch;
    AttnVItem<KF> vb[PF];
    // Every load is issued unconditionally (a position past the span reads
    // position 0 and is never used), so the compiler can count the loads in
    // flight and wait for the oldest one only.
    auto load = [&](int k, AttnVItem<KF> &it) {
        int t = k * T + tl;
        t = has_item && t < span ? t : 0;
        int slot = base + t;
        if (slot >= g.cap) slot -= g.cap;
        if constexpr (KF) {
            // V is the f32 block's last part: a thread without an item reads
            // piece 0, so no read passes the row
            const float4 *src = reinterpret_cast<const float4 *>(
                reinterpret_cast<const float *>(blk + g.v_off) +
                (size_t(kvh) * g.cap + slot) * g.VD + (has_item ? pc : 0) * 16);
#pragma unroll
            for (int u = 0; u < 4; ++u) it.v[u] = src[u];
        } else {
            const int8_t *vbase = reinterpret_cast<const int8_t *>(blk + g.v_off) + size_t(kvh) * g.cap * g.VD;
            const float *vs = reinterpret_cast<const float *>(blk + g.vs_off) + size_t(kvh) * g.cap;
            it.v = *reinterpret_cast<const uint4 *>(vbase + size_t(slot) * g.VD + pc * 16);
            it.s = vs[slot];
        }
    };
#pragma unroll
    for (int j = 0; j < PF; ++j) load(j, vb[j]);
    // The softmax sum, with the bits of one chain in position order.  The
    // exps are >= +0, so a span long enough to pay for it takes the exact
    // parallel fold, its LDS in the product buffers (first written after the
    // barrier below); a shorter or longer one is the chain itself.
    if (span >= kAttnFoldMin && span <= NT * kAttnFoldC) {
        NdFoldLds<NT> &fl = *reinterpret_cast<NdFoldLds<NT> *>(prod);
        const int cpt = (span + NT - 1) / NT;
        float s;
        if (cpt <= 4) s = nd_fold_nonneg<NT, 4>(sc, span, fl);
        else if (cpt <= 9) s = nd_fold_nonneg<NT, 9>(sc, span, fl);
        else s = nd_fold_nonneg<NT, kAttnFoldC>(sc, span, fl);
        if (tid == 0) L.total = s;
    } else if (tid == 0) {
        __builtin_amdgcn_s_setprio(2);
        const float s = lds_chain(0.0f, sc, span);
        L.total = s;
        __builtin_amdgcn_s_setprio(0);
    }
    __syncthreads();
    const float inv = 1.0f / L.total;
    float acc = 0.0f;
    // Step k: producers fill chunk k, consumers add chunk k - 1.  Each role
    // runs its own loop; the roles are whole waves and both pass the same
    // number of barriers (a multiple of PF, the last few empty).
    const int steps = (nch + 1 + PF - 1) / PF * PF;
    if (producer) {
        // this item's exp for the step after the current one, read ahead
        float e_next = sc[tl < span ? tl : 0];
        for (int k0 = 0; k0 < steps; k0 += PF) {
#pragma unroll
            for (int j = 0; j < PF; ++j) {
                const int k = k0 + j;
                const int t = k * T + tl;
                const float e = e_next;
                const int tn = t + T;
                e_next = sc[tn < span ? tn : 0];
                if (has_item && k < nch && t < span) {
                    AttnVItem<KF> it = vb[j];
                    if constexpr (NEW) {
                        // the span's last position: the launch's own row
                        if (k == nch - 1 && t == span - 1) {
                            it.v = nr->v[pc];
                            it.s = nr->vs;
                        }
                    }
                    float p[16];
                    if constexpr (KF) {
                        // F32View::accum: w = e * inv, then w * v
                        const float w = e * inv;
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            p[4 * u] = w * it.v[u].x;
                            p[4 * u + 1] = w * it.v[u].y;
                            p[4 * u + 2] = w * it.v[u].z;
                            p[4 * u + 3] = w * it.v[u].w;
                        }
                    } else {
                        // Int8View::accum: w = (e * inv) * v_scale, then w * code
                        const float w = e * inv * it.s;
                        const uint32_t dws[4] = {it.v.x, it.v.y, it.v.z, it.v.w};
#pragma unroll
                        for (int d = 0; d < 4; ++d)
#pragma unroll
                            for (int b = 0; b < 4; ++b) p[d * 4 + b] = w * i8_lane(dws[d], b);
                    }
                    float *dst = prod + (k & 1) * kProdBuf + (pc * 16) * TS + tl;
#pragma unroll
                    for (int u = 0; u < 16; ++u) dst[u * TS] = p[u];
                }
                load(k + PF, vb[j]);
                __syncthreads();
            }
        }
    } else {
        const float *col = prod + (tid < g.VD ? tid : 0) * TS;
        // whole chunks inside the loop, each group's adds waiting for that
        // group's reads only (the next group's are in flight); a ragged last
        // chunk after it, once no producer writes its buffer any more
        const int nfull = span / T;
        for (int k = 0; k < steps; ++k) {
            const int c = k - 1;
            if (c >= 0 && c < nfull && tid < g.VD) {
                __builtin_amdgcn_s_setprio(2);
                const float *buf = col + (c & 1) * kProdBuf;
                float4 a[4], b[4];
                nd_lds_read16(a, buf);
#pragma unroll
                for (int gi = 0; gi < T / 16; ++gi) {
                    if (gi % 2 == 0) {
                        if (gi + 1 < T / 16) nd_lds_read16(b, buf + (gi + 1) * 16);
                        acc = nd_add16(acc, a);
                    } else {
                        if (gi + 1 < T / 16) nd_lds_read16(a, buf + (gi + 1) * 16);
                        acc = nd_add16(acc, b);
                    }
                }
                __builtin_amdgcn_s_setprio(0);
            }
            __syncthreads();
        }
        if (nfull < nch && tid < g.VD) {
            const float *buf = col + (nfull & 1) * kProdBuf;
            const int rem = span - nfull * T;
            for (int gi = 0; gi * 16 < rem; ++gi) {
                float4 a[4];
                nd_lds_read16(a, buf + gi * 16);
                acc = nd_add_first(acc, a, rem - gi * 16);
            }
        }
    }
    if (tid < g.VD) out_row[tid] = gate_half_fwht(acc, gate_row, tid);
}

}  // namespace ndattn
