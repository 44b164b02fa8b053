// Reference-order kernels: the same result bits as the reference's CPU path.
//
// A float sum depends on its order, and in the Needle-3 forward a last-bit
// difference anywhere upstream of the int8 KV quantiser can move a value
// across a rounding boundary and flip a cached code.  The flip changes every
// later step, so token-identical greedy decoding needs the device to
// reproduce the reference's sums exactly.  These kernels keep every
// reference chain as one sequential chain in one thread and run the
// independent chains side by side; the file is built without FP
// contraction, so a*b+c rounds twice as rustc's code does.
//
//   cq_exact       CqWeight::matvec_rows_prepared / matmul_rows_prepared for
//                  the byte-aligned widths (cq.rs:721-735, 838-873, 632-679,
//                  879-906).  Eight lane accumulators per (row, group):
//                  element e of the group goes to lane e % 8, lanes summed
//                  0..7, then the row total adds norm[g] * group_sum over the
//                  groups in order.  One thread per (row, group): its codes
//                  are decoded once per 8 elements and dotted with up to 8
//                  activation rows held in LDS; the group sums meet in LDS
//                  and one thread per (row, batch row) chains them.
//   cq_exact_serial   any other width or group: one thread per output, the
//                  reference's loop verbatim (3-bit bit reader, 8-lane
//                  groups with a serial tail).
//   attn_exact     attend_step over the int8 view (attention.rs:327-377):
//                  per (query, head) a workgroup computes every score with
//                  its own 16..256-long dot chain, the maximum, exp, the
//                  softmax sum as one chain, and each output column as one
//                  chain over the span.
#include "nd_cq_internal.h"
#include "nd_internal.h"
#include "nd_kv_internal.h"
#include "nd_libm.h"

#include <cmath>

namespace {

constexpr int kThreads = 256;
constexpr int kMaxBt = 8;             // activation rows per workgroup
constexpr size_t kLdsBudget = 64 * 1024;
constexpr int kAttnMaxCap = 16384;    // scores of one span live in LDS
constexpr uint8_t kTernary = 5;

struct CqExact {
    const uint8_t *packed;
    const float *norms;
    const float *lv;
    const float *xh;
    float *y;
    size_t row_bytes;
    int in_padded, group, G, row_start, rows, batch, rpb, ternary;
};

// cq.rs:948-958
__device__ inline int ternary_index(int code) { return code == 3 ? 0 : (code == 1 ? 2 : 1); }

template <int P, int BT>
__global__ __launch_bounds__(kThreads) void cq_exact_kernel(CqExact a)
{
    constexpr int W = 8 / P;                // bits per code
    constexpr uint32_t MASK = (1u << W) - 1;
    constexpr int PER_DW = 32 / W;          // codes per dword (8 or 16)
    extern __shared__ __align__(16) float sm[];
    float *lvl = sm;                        // [16] code -> level
    float *xs = sm + 16;                    // [BT][in_padded]
    float *gs = xs + BT * a.in_padded;      // [BT][rpb * G] group sums
    const int tid = threadIdx.x;
    const int b0 = blockIdx.y * BT;
    const int nb = a.batch - b0 < BT ? a.batch - b0 : BT;
    if (tid < 16) lvl[tid] = a.lv[a.ternary ? ternary_index(tid) : tid];
    for (int bb = 0; bb < nb; ++bb) {
        const float *src = a.xh + size_t(b0 + bb) * a.in_padded;
        for (int e = tid; e < a.in_padded; e += kThreads) xs[bb * a.in_padded + e] = src[e];
    }
    __syncthreads();
    const int pairs = a.rpb * a.G;
    const int r0 = a.row_start + int(blockIdx.x) * a.rpb;
    const int row_end = a.row_start + a.rows;
    if (tid < pairs) {
        const int rl = tid / a.G, g = tid - rl * a.G;
        const int r = r0 + rl;
        if (r < row_end) {
            const uint32_t *cw = reinterpret_cast<const uint32_t *>(
                a.packed + size_t(r) * a.row_bytes + size_t(g) * (a.group / P));
            float lanes[BT][8];
#pragma unroll
            for (int bb = 0; bb < BT; ++bb)
#pragma unroll
                for (int k = 0; k < 8; ++k) lanes[bb][k] = 0.0f;
            const int iters = a.group / 8;
            const float *xg = xs + g * a.group;
            for (int i = 0; i < iters; ++i) {
                const uint32_t dw = cw[(i * 8) / PER_DW];
                const int sh = (i * 8 * W) & 31;
                float v[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) v[k] = lvl[(dw >> (sh + k * W)) & MASK];
#pragma unroll
                for (int bb = 0; bb < BT; ++bb) {
                    if (bb < nb) {
                        const float4 xa = *reinterpret_cast<const float4 *>(xg + bb * a.in_padded + i * 8);
                        const float4 xb = *reinterpret_cast<const float4 *>(xg + bb * a.in_padded + i * 8 + 4);
                        lanes[bb][0] += v[0] * xa.x;
                        lanes[bb][1] += v[1] * xa.y;
                        lanes[bb][2] += v[2] * xa.z;
                        lanes[bb][3] += v[3] * xa.w;
                        lanes[bb][4] += v[4] * xb.x;
                        lanes[bb][5] += v[5] * xb.y;
                        lanes[bb][6] += v[6] * xb.z;
                        lanes[bb][7] += v[7] * xb.w;
                    }
                }
            }
#pragma unroll
            for (int bb = 0; bb < BT; ++bb) {
                float acc = 0.0f;
#pragma unroll
                for (int k = 0; k < 8; ++k) acc += lanes[bb][k];
                if (bb < nb) gs[bb * pairs + tid] = acc;
            }
        }
    }
    __syncthreads();
    for (int o = tid; o < a.rpb * nb; o += kThreads) {
        const int bb = o / a.rpb, rl = o - bb * a.rpb;
        const int r = r0 + rl;
        if (r < row_end) {
            const float *rn = a.norms + size_t(r) * a.G;
            const float *gp = gs + bb * pairs + rl * a.G;
            float total = 0.0f;
            for (int g = 0; g < a.G; ++g) total += rn[g] * gp[g];
            a.y[size_t(b0 + bb) * a.rows + (r - a.row_start)] = total;
        }
    }
}

struct CqSerial {
    const uint8_t *packed;
    const float *norms;
    const float *lut;   // [256][per_byte], per_byte widths
    const float *lv;    // levels, 3-bit
    const float *xh;
    float *y;
    size_t row_bytes;
    int in_padded, group, G, row_start, rows, batch, per_byte, bits;
};

// cq.rs:914-925
__device__ inline uint32_t read_bits(const uint8_t *row, size_t bit, int bits, uint32_t mask)
{
    const size_t byte = bit / 8;
    const int shift = int(bit % 8);
    const uint32_t lo = row[byte];
    const uint32_t hi = shift + bits > 8 ? row[byte + 1] : 0u;
    return ((lo | (hi << 8)) >> shift) & mask;
}

__global__ __launch_bounds__(kThreads) void cq_exact_serial_kernel(CqSerial a)
{
    const size_t idx = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (idx >= size_t(a.batch) * a.rows) return;
    const int b = int(idx / a.rows), rl = int(idx % a.rows);
    const int r = a.row_start + rl;
    const uint8_t *row = a.packed + size_t(r) * a.row_bytes;
    const float *rn = a.norms + size_t(r) * a.G;
    const float *x = a.xh + size_t(b) * a.in_padded;
    float total = 0.0f;
    for (int g = 0; g < a.G; ++g) {
        const float *gx = x + size_t(g) * a.group;
        float acc = 0.0f;
        if (a.per_byte) {
            const int P = a.per_byte, bpg = a.group / P, per_iter = 8 / P;
            const uint8_t *gb = row + size_t(g) * bpg;
            const int full = bpg - bpg % per_iter;
            float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int bi = 0; bi < full; bi += per_iter) {
                float vals[8];
                for (int t = 0; t < per_iter; ++t)
                    for (int k = 0; k < P; ++k) vals[t * P + k] = a.lut[int(gb[bi + t]) * P + k];
                for (int k = 0; k < 8; ++k) lanes[k] += vals[k] * gx[bi * P + k];
            }
            for (int k = 0; k < 8; ++k) acc += lanes[k];
            for (int bi = full; bi < bpg; ++bi)
                for (int k = 0; k < P; ++k) acc += a.lut[int(gb[bi]) * P + k] * gx[bi * P + k];
        } else {
            const uint32_t mask = (1u << a.bits) - 1;
            for (int k = 0; k < a.group; ++k) {
                const uint32_t code =
                    read_bits(row, (size_t(g) * a.group + k) * size_t(a.bits), a.bits, mask);
                acc += a.lv[code] * gx[k];
            }
        }
        total += rn[g] * acc;
    }
    a.y[size_t(b) * a.rows + rl] = total;
}

template <int P, int BT>
void launch_exact(const CqExact &a, hipStream_t s)
{
    const unsigned gx = unsigned((a.rows + a.rpb - 1) / a.rpb);
    const unsigned gy = unsigned((a.batch + BT - 1) / BT);
    const size_t lds = 4 * (16 + size_t(BT) * a.in_padded + size_t(BT) * a.rpb * a.G);
    hipLaunchKernelGGL((cq_exact_kernel<P, BT>), dim3(gx, gy), dim3(kThreads), lds, s, a);
}

template <int P>
void launch_bt(const CqExact &a, int bt, hipStream_t s)
{
    switch (bt) {
    case 8: launch_exact<P, 8>(a, s); break;
    case 4: launch_exact<P, 4>(a, s); break;
    case 2: launch_exact<P, 2>(a, s); break;
    default: launch_exact<P, 1>(a, s); break;
    }
}

int cq_exact(nd_ctx *ctx, const nd_cq *w, const float *xh, size_t batch, size_t row_start,
             size_t rows, float *y, const char *what)
{
    if (int rc = nd::enter(ctx)) return rc;
    ND_REQUIRE(w && xh && y, "%s: null argument", what);
    if (rows == 0 || batch == 0) return ND_OK;
    ND_REQUIRE(row_start <= w->out_feat && rows <= w->out_feat - row_start,
               "%s: rows %zu..%zu outside %zu", what, row_start, row_start + rows, w->out_feat);
    ND_REQUIRE(w->out_feat < (1u << 30) && batch <= 65535u * kMaxBt && w->in_padded < (1u << 24),
               "%s: shape too large", what);
    const size_t G = w->num_groups;
    const int P = int(w->per_byte);
    const bool fast = (P == 2 || P == 4) && w->group % 8 == 0 && (w->group / P) % 4 == 0 && G <= kThreads &&
                      w->row_bytes % 4 == 0;
    if (fast) {
        const int rpb = int(kThreads / G);
        int bt = kMaxBt;
        while (bt > 1 && (size_t(bt) / 2 >= batch ||
                          4 * (16 + size_t(bt) * w->in_padded + size_t(bt) * rpb * G) > kLdsBudget))
            bt /= 2;
        if (4 * (16 + size_t(bt) * w->in_padded + size_t(bt) * rpb * G) <= kLdsBudget) {
            CqExact a{w->packed, w->norms, w->lv, xh, y, w->row_bytes, int(w->in_padded),
                      int(w->group), int(G), int(row_start), int(rows), int(batch), rpb,
                      int(w->bits == kTernary)};
            if (P == 4)
                launch_bt<4>(a, bt, ctx->stream);
            else
                launch_bt<2>(a, bt, ctx->stream);
            return nd::check_launch(what);
        }
    }
    const size_t total = batch * rows;
    ND_REQUIRE((total + kThreads - 1) / kThreads <= 0x7fffffffu, "%s: too many outputs", what);
    CqSerial a{w->packed, w->norms, w->lut, w->lv, xh, y, w->row_bytes, int(w->in_padded),
               int(w->group), int(G), int(row_start), int(rows), int(batch), P,
               int(w->bits == kTernary ? 2 : w->bits)};
    hipLaunchKernelGGL(cq_exact_serial_kernel, dim3(unsigned((total + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, ctx->stream, a);
    return nd::check_launch(what);
}

// ---------------------------------------------------------------------------
// attend_step over the int8 view, in the reference's order.
// ---------------------------------------------------------------------------
__device__ inline float i8_lane(uint32_t dw, int b) { return float(int32_t(dw << (24 - 8 * b)) >> 24); }

__global__ __launch_bounds__(kThreads) void attn_exact_kernel(ndkv::Geom g,
                                                             const uint8_t *__restrict__ kv,
                                                             size_t stride,
                                                             const int32_t *__restrict__ lo,
                                                             const int32_t *__restrict__ hi,
                                                             const float *__restrict__ q, float scale,
                                                             int quant_query, float *__restrict__ out)
{
    extern __shared__ __align__(16) float sc[];  // [span] scores, then weights
    __shared__ float qs[ndkv::kMaxDim];
    __shared__ float red[kThreads / 64];
    __shared__ float total;
    const int h = blockIdx.x, tid = threadIdx.x;
    const size_t i = blockIdx.y;
    const int kvh = h / (g.H / g.KVH);
    const uint8_t *blk = kv + i * stride;
    const int p0 = lo[i];
    const int span = hi[i] - p0 + 1;
    if (p0 < 0 || span < 1 || span > g.cap) {
        // outside the contract (0 <= lo <= hi < lo + cap): NaN, as nd_attend_step_i8
        for (int j = tid; j < g.VD; j += kThreads) out[(i * g.H + h) * size_t(g.VD) + j] = NAN;
        return;
    }
    const float *qv = q + (i * g.H + h) * size_t(g.QK);
    if (tid < 64) {
        // quant_rows (v3/model.rs:289-293): fake-quantised query head
        if (quant_query) {
            float s, inv;
            ndkv::quant_scale_wave(qv, g.QK, s, inv);
            for (int e = tid; e < g.QK; e += 64) qs[e] = ndkv::quant_code(qv[e], inv) * s;
        } else {
            for (int e = tid; e < g.QK; e += 64) qs[e] = qv[e];
        }
    }
    __syncthreads();
    const int8_t *kb = reinterpret_cast<const int8_t *>(blk) + size_t(kvh) * g.cap * g.QK;
    const float *ks = reinterpret_cast<const float *>(blk + g.ks_off) + size_t(kvh) * g.cap;
    const int base = p0 % g.cap;
    float mx = -INFINITY;
    for (int t = tid; t < span; t += kThreads) {
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
    mx = ndkv::wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0];
    for (int w = 1; w < kThreads / 64; ++w) mx = red[w] > mx ? red[w] : mx;
    for (int t = tid; t < span; t += kThreads) sc[t] = nd_expf(sc[t] - mx);
    __syncthreads();
    if (tid == 0) {
        float s = 0.0f;
        int t = 0;
        for (; t + 4 <= span; t += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(sc + t);
            s += v.x;
            s += v.y;
            s += v.z;
            s += v.w;
        }
        for (; t < span; ++t) s += sc[t];
        total = s;
    }
    __syncthreads();
    const float inv = 1.0f / total;
    const float *vs = reinterpret_cast<const float *>(blk + g.vs_off) + size_t(kvh) * g.cap;
    for (int t = tid; t < span; t += kThreads) {
        int slot = base + t;
        if (slot >= g.cap) slot -= g.cap;
        sc[t] = sc[t] * inv * vs[slot];
    }
    __syncthreads();
    const int8_t *vb = reinterpret_cast<const int8_t *>(blk + g.v_off) + size_t(kvh) * g.cap * g.VD;
    float *o = out + (i * g.H + h) * size_t(g.VD);
    for (int j = tid; j < g.VD; j += kThreads) {
        float acc = 0.0f;
        int slot = base;
        for (int t = 0; t < span; ++t) {
            acc += sc[t] * float(vb[size_t(slot) * g.VD + j]);
            if (++slot == g.cap) slot = 0;
        }
        o[j] = acc;
    }
}

}  // namespace

extern "C" {

int nd_cq_matvec_rows_exact(nd_ctx *ctx, const nd_cq *w, const float *xh, size_t row_start,
                            size_t rows, float *y)
{
    return cq_exact(ctx, w, xh, 1, row_start, rows, y, "cq_matvec_exact");
}

int nd_cq_matmul_rows_exact(nd_ctx *ctx, const nd_cq *w, const float *xh, size_t batch,
                            size_t row_start, size_t rows, float *y)
{
    return cq_exact(ctx, w, xh, batch, row_start, rows, y, "cq_matmul_exact");
}

int nd_attend_step_i8_exact(nd_ctx *ctx, const nd_kv_geom *g, const void *kv, size_t kv_stride,
                            size_t count, const int32_t *lo, const int32_t *hi, const float *q,
                            float scale, int quant_query, float *out)
{
    if (int rc = nd::enter(ctx)) return rc;
    if (int rc = ndkv::check_geom(g)) return rc;
    if (count == 0) return ND_OK;
    ND_REQUIRE(kv && lo && hi && q && out, "null buffer");
    ND_REQUIRE(count <= 65535, "count %zu above 65535", count);
    ND_REQUIRE(g->cap <= kAttnMaxCap, "cap %d above %d for the reference-order attention", g->cap,
               kAttnMaxCap);
    ND_REQUIRE((reinterpret_cast<uintptr_t>(kv) & 255) == 0 && kv_stride % 256 == 0,
               "kv blocks must be 256-byte aligned");
    dim3 grid(unsigned(g->num_heads), unsigned(count));
    hipLaunchKernelGGL(attn_exact_kernel, grid, dim3(kThreads), size_t(g->cap) * 4, ctx->stream,
                       ndkv::make_geom(g), static_cast<const uint8_t *>(kv), kv_stride, lo, hi, q,
                       scale, quant_query, out);
    return nd::check_launch("attn_exact");
}

}  // extern "C"
