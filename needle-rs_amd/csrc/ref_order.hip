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
//                  are decoded a byte at a time through the reference's byte
//                  LUT (one LDS read per byte) and dotted with up to 8
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
#include "nd_fold.h"
#include "nd_internal.h"
#include "nd_kv_internal.h"
#include "nd_libm.h"
#include "nd_ref_order.h"
#include "nd_attn_exact.h"

#include <cmath>

namespace {

constexpr int kThreads = 256;
constexpr int kMaxBt = 8;             // activation rows per workgroup
constexpr size_t kLdsBudget = 64 * 1024;
constexpr int kVChunk = 16384;        // bytes of V rows staged per pass
constexpr int kAttnMaxCap = 12288;    // one span's scores + a V chunk fit 64 KB of LDS
constexpr uint8_t kTernary = 5;

struct CqExact {
    const uint8_t *packed;
    const float *norms;
    const float *lv;
    const float *xh;
    float *y;
    size_t row_bytes;
    int in_padded, group, G, row_start, rows, batch, rpb, ternary;
    // 0: xh is prepared.  Otherwise xh holds each 128-group with butterfly
    // stages h = 1..32 done; the load finishes the transform: stage h = 64
    // and the scale by half_inv (1/sqrt(128)), as fwht_normalized would.
    float half_inv;
};

// Up to kMaxSet weights with the same input, width and group in one launch:
// blocks [tile0[k], tile0[k + 1]) work on weight k.
constexpr int kMaxSet = 12;
struct CqExactSet {
    CqExact w[kMaxSet];
    int tile0[kMaxSet + 1];
    int n;
};

// cq.rs:948-958
__device__ inline int ternary_index(int code) { return code == 3 ? 0 : (code == 1 ? 2 : 1); }

// GR: the group size when it is 128 (codes preloaded into registers), or 0
// for any other multiple of 8 (codes read as the loop needs them).
template <int P, int BT, int GR>
__global__ __launch_bounds__(kThreads) void cq_exact_kernel(CqExactSet set)
{
    int wk = set.n - 1;
    while (wk > 0 && int(blockIdx.x) < set.tile0[wk]) --wk;
    const CqExact &a = set.w[wk];
    const int tile = int(blockIdx.x) - set.tile0[wk];
    constexpr int W = 8 / P;                // bits per code
    constexpr uint32_t MASK = (1u << W) - 1;
    constexpr int PER_DW = 32 / W;          // codes per dword (8 or 16)
    constexpr int NDW = GR ? GR / PER_DW : 1;
    extern __shared__ __align__(16) float sm[];
    // activations in LDS with each group padded by 4 floats, so that the
    // groups a wave reads at once fall in different banks
    const int gstride = a.group + 4, xstride = a.G * gstride;
    float *lut = sm;                        // [256][P] byte -> its P levels (build_lut)
    float *ns = sm + 256 * P;               // [kThreads] this block's norms
    float *xs = ns + kThreads;              // [BT][G][group + 4]
    float *gs = xs + BT * xstride;          // [BT][rpb * G] group sums
    const int tid = threadIdx.x;
    const int b0 = blockIdx.y * BT;
    const int nb = a.batch - b0 < BT ? a.batch - b0 : BT;
    const int pairs = a.rpb * a.G;
    const int r0 = a.row_start + tile * a.rpb;
    const int row_end = a.row_start + a.rows;
    const int nrows = row_end - r0 < a.rpb ? row_end - r0 : a.rpb;
    // the byte LUT of cq.rs:932-964: slot k of byte b is the level of code k
    // (bits k*W of b), so one read decodes a byte
#pragma unroll
    for (int k = 0; k < P; ++k) {
        const int c = int((uint32_t(tid) >> (k * W)) & MASK);
        lut[tid * P + k] = a.lv[a.ternary ? ternary_index(c) : c];
    }
    if (tid < nrows * a.G) ns[tid] = a.norms[size_t(r0) * a.G + tid];
    for (int bb = 0; bb < nb; ++bb) {
        const float4 *src = reinterpret_cast<const float4 *>(a.xh + size_t(b0 + bb) * a.in_padded);
        for (int e = tid; e < a.in_padded / 4; e += kThreads) {
            const int g = (4 * e) / a.group, k = 4 * e - g * a.group;
            float4 v = src[e];
            if (a.half_inv != 0.0f) {
                // the last butterfly stage: lower half a + b, upper half a - b
                const float4 o = src[e + (k < 64 ? 16 : -16)];
                const float s = a.half_inv;
                v = k < 64 ? make_float4((v.x + o.x) * s, (v.y + o.y) * s, (v.z + o.z) * s, (v.w + o.w) * s)
                           : make_float4((o.x - v.x) * s, (o.y - v.y) * s, (o.z - v.z) * s, (o.w - v.w) * s);
            }
            *reinterpret_cast<float4 *>(xs + bb * xstride + g * gstride + k) = v;
        }
    }
    // this thread's (row, group) and its codes
    const int rl = tid / a.G, g = tid - rl * a.G;
    const int r = r0 + rl;
    const bool active = tid < pairs && rl < nrows;
    const uint32_t *cw = reinterpret_cast<const uint32_t *>(
        a.packed + size_t(active ? r : a.row_start) * a.row_bytes + size_t(g) * (a.group / P));
    uint32_t code[NDW];
    if (GR && active) {
#pragma unroll
        for (int k = 0; k < NDW; k += 4) {
            const uint4 c4 = *reinterpret_cast<const uint4 *>(cw + k);
            code[k] = c4.x;
            code[k + 1] = c4.y;
            code[k + 2] = c4.z;
            code[k + 3] = c4.w;
        }
    }
    __syncthreads();
    if (active) {
        float lanes[BT][8];
#pragma unroll
        for (int bb = 0; bb < BT; ++bb)
#pragma unroll
            for (int k = 0; k < 8; ++k) lanes[bb][k] = 0.0f;
        const float *xg = xs + g * gstride;
        // iteration i: elements 8i..8i+7 of the group, element 8i+k into lane k
        auto step = [&](int i, uint32_t dw) {
            const int sh = (i * 8 * W) & 31;
            float v[8];
            if (P == 4) {  // 2 bits: elements 8i..8i+7 are two bytes
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const float4 l4 = *reinterpret_cast<const float4 *>(lut + ((dw >> (sh + 8 * q)) & 0xffu) * 4);
                    v[4 * q] = l4.x;
                    v[4 * q + 1] = l4.y;
                    v[4 * q + 2] = l4.z;
                    v[4 * q + 3] = l4.w;
                }
            } else {  // 4 bits: four bytes
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float2 l2 = *reinterpret_cast<const float2 *>(lut + ((dw >> (sh + 8 * q)) & 0xffu) * 2);
                    v[2 * q] = l2.x;
                    v[2 * q + 1] = l2.y;
                }
            }
#pragma unroll
            for (int bb = 0; bb < BT; ++bb) {
                if (bb < nb) {
                    const float4 xa = *reinterpret_cast<const float4 *>(xg + bb * xstride + i * 8);
                    const float4 xb = *reinterpret_cast<const float4 *>(xg + bb * xstride + i * 8 + 4);
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
        };
        if constexpr (GR != 0) {
#pragma unroll
            for (int i = 0; i < GR / 8; ++i) step(i, code[(i * 8) / PER_DW]);
        } else {
            for (int i = 0; i < a.group / 8; ++i) step(i, cw[(i * 8) / PER_DW]);
        }
#pragma unroll
        for (int bb = 0; bb < BT; ++bb) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) acc += lanes[bb][k];
            if (bb < nb) gs[bb * pairs + tid] = acc;
        }
    }
    __syncthreads();
    for (int o = tid; o < nrows * nb; o += kThreads) {
        const int bb = o / nrows, rr = o - bb * nrows;
        const float *rn = ns + rr * a.G;
        const float *gp = gs + bb * pairs + rr * a.G;
        float total = 0.0f;
        for (int gg = 0; gg < a.G; ++gg) total += rn[gg] * gp[gg];
        a.y[size_t(b0 + bb) * a.rows + (r0 + rr - a.row_start)] = total;
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

size_t exact_lds(int bt, int per_byte, size_t in_padded, size_t group, size_t pairs)
{
    const size_t padded = in_padded / group * (group + 4);
    return 4 * (256 * size_t(per_byte) + size_t(kThreads) + size_t(bt) * padded + size_t(bt) * pairs);
}

template <int P, int BT>
void launch_exact(const CqExactSet &set, hipStream_t s)
{
    const CqExact &a = set.w[0];
    const unsigned gy = unsigned((a.batch + BT - 1) / BT);
    const size_t lds = exact_lds(BT, P, a.in_padded, a.group, size_t(a.rpb) * a.G);
    const dim3 grid(unsigned(set.tile0[set.n]), gy);
    if (a.group == 128)
        hipLaunchKernelGGL((cq_exact_kernel<P, BT, 128>), grid, dim3(kThreads), lds, s, set);
    else
        hipLaunchKernelGGL((cq_exact_kernel<P, BT, 0>), grid, dim3(kThreads), lds, s, set);
}

template <int P>
void launch_bt(const CqExactSet &set, int bt, hipStream_t s)
{
    switch (bt) {
    case 8: launch_exact<P, 8>(set, s); break;
    case 4: launch_exact<P, 4>(set, s); break;
    case 2: launch_exact<P, 2>(set, s); break;
    default: launch_exact<P, 1>(set, s); break;
    }
}

int cq_serial(hipStream_t stream, const nd_cq *w, const float *xh, size_t batch,
              size_t row_start, size_t rows, float *y, const char *what)
{
    const size_t total = batch * rows;
    ND_REQUIRE((total + kThreads - 1) / kThreads <= 0x7fffffffu, "%s: too many outputs", what);
    CqSerial a{w->packed, w->norms, w->lut, w->lv, xh, y, w->row_bytes, int(w->in_padded),
               int(w->group), int(w->num_groups), int(row_start), int(rows), int(batch),
               int(w->per_byte), int(w->bits == kTernary ? 2 : w->bits)};
    hipLaunchKernelGGL(cq_exact_serial_kernel, dim3(unsigned((total + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, stream, a);
    return nd::check_launch(what);
}

}  // namespace

// n weights sharing the input xh ([batch][in_padded]); y[k] gets
// rows[k] rows of weight k from row_start[k], batch-major.
int nd_cq_exact_set(nd_ctx *ctx, hipStream_t stream, int n, const nd_cq *const *w, const float *xh,
                    size_t batch, const size_t *row_start, const size_t *rows, float *const *y,
                    const char *what, float half_inv)
{
    ND_REQUIRE(n >= 1 && n <= kMaxSet, "%s: %d weights in one set", what, n);
    const float *xhs[kMaxSet];
    for (int k = 0; k < n; ++k) xhs[k] = xh;
    return nd_cq_exact_multi(ctx, stream, n, w, xhs, batch, row_start, rows, y, what, half_inv);
}

int nd_cq_exact_multi(nd_ctx *ctx, hipStream_t stream, int n, const nd_cq *const *w,
                      const float *const *xhs, size_t batch, const size_t *row_start,
                      const size_t *rows, float *const *y, const char *what, float half_inv)
{
    ND_ENTER(ctx);
    ND_REQUIRE(n >= 1 && n <= kMaxSet && w && xhs && row_start && rows && y, "%s: bad arguments",
               what);
    if (batch == 0) return ND_OK;
    const nd_cq *w0 = w[0];
    bool same = true, aligned = true;
    for (int k = 0; k < n; ++k) {
        ND_REQUIRE(w[k] && y[k] && xhs[k], "%s: null weight, input or output", what);
        aligned = aligned && (reinterpret_cast<uintptr_t>(xhs[k]) & 15) == 0;
        ND_REQUIRE(row_start[k] <= w[k]->out_feat && rows[k] <= w[k]->out_feat - row_start[k],
                   "%s: rows %zu..%zu outside %zu", what, row_start[k], row_start[k] + rows[k],
                   w[k]->out_feat);
        ND_REQUIRE(w[k]->out_feat < (1u << 30) && w[k]->in_padded < (1u << 24),
                   "%s: shape too large", what);
        same = same && w[k]->per_byte == w0->per_byte && w[k]->group == w0->group &&
               w[k]->in_padded == w0->in_padded && w[k]->bits == w0->bits;
    }
    ND_REQUIRE(batch <= 65535u * kMaxBt, "%s: batch too large", what);
    const size_t G = w0->num_groups;
    const int P = int(w0->per_byte);
    const bool fast = same && (P == 2 || P == 4) && w0->group % 8 == 0 && (w0->group / P) % 4 == 0 &&
                      G <= kThreads && w0->row_bytes % 4 == 0 && aligned;
    if (fast) {
        const int rpb = int(kThreads / G);
        const size_t pairs = size_t(rpb) * G;
        size_t tiles = 0;
        for (int k = 0; k < n; ++k) tiles += (rows[k] + rpb - 1) / rpb;
        // fewest activation rows per workgroup that still leave two
        // workgroups per CU, so a large batch fills the GPU
        const size_t want = 2 * size_t(ctx->num_cus > 0 ? ctx->num_cus : 256);
        int bt = kMaxBt;
        while (bt > 1 &&
               (size_t(bt) / 2 >= batch || exact_lds(bt, P, w0->in_padded, w0->group, pairs) > kLdsBudget ||
                tiles * ((batch + bt - 1) / bt) < want))
            bt /= 2;
        ND_REQUIRE(half_inv == 0.0f || w0->group == 128,
                   "%s: a half-transformed input needs 128-wide groups", what);
        if (exact_lds(bt, P, w0->in_padded, w0->group, pairs) <= kLdsBudget) {
            CqExactSet set{};
            set.n = 0;
            int tiles = 0;
            for (int k = 0; k < n; ++k) {
                if (rows[k] == 0) continue;
                set.w[set.n] = CqExact{w[k]->packed, w[k]->norms, w[k]->lv, xhs[k], y[k], w[k]->row_bytes,
                                       int(w[k]->in_padded), int(w[k]->group), int(G),
                                       int(row_start[k]), int(rows[k]), int(batch), rpb,
                                       int(w[k]->bits == kTernary), half_inv};
                set.tile0[set.n++] = tiles;
                tiles += int((rows[k] + rpb - 1) / rpb);
            }
            if (set.n == 0) return ND_OK;
            set.tile0[set.n] = tiles;
            if (P == 4)
                launch_bt<4>(set, bt, stream);
            else
                launch_bt<2>(set, bt, stream);
            return nd::check_launch(what);
        }
    }
    ND_REQUIRE(half_inv == 0.0f, "%s: a half-transformed input needs the 128-group kernel", what);
    for (int k = 0; k < n; ++k)
        if (rows[k])
            if (int rc = cq_serial(stream, w[k], xhs[k], batch, row_start[k], rows[k], y[k], what))
                return rc;
    return ND_OK;
}

namespace {

using namespace ndattn;

// ---------------------------------------------------------------------------
// attend_step over the int8 view, in the reference's order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void attn_exact_kernel(ndkv::Geom g,
                                                             const uint8_t *__restrict__ kv,
                                                             size_t stride, int rows_per_block,
                                                             const int32_t *__restrict__ lo,
                                                             const int32_t *__restrict__ hi,
                                                             const float *__restrict__ q, float scale,
                                                             int quant_query, float *__restrict__ out,
                                                             const float *__restrict__ gate)
{
    extern __shared__ __align__(16) float sc[];  // [span] scores, then weights
    __shared__ float qs[ndkv::kMaxDim];
    __shared__ float red[kThreads / 64];
    __shared__ float total;
    const int h = blockIdx.x, tid = threadIdx.x;
    const size_t i = blockIdx.y;
    const int kvh = h / (g.H / g.KVH);
    const uint8_t *blk = kv + (i / size_t(rows_per_block)) * stride;
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
        // the softmax sum: one chain in position order
        float s = 0.0f;
        int t = 0;
        for (; t + 16 <= span; t += 16) {
            const float4 a = *reinterpret_cast<const float4 *>(sc + t);
            const float4 b = *reinterpret_cast<const float4 *>(sc + t + 4);
            const float4 c = *reinterpret_cast<const float4 *>(sc + t + 8);
            const float4 d = *reinterpret_cast<const float4 *>(sc + t + 12);
            s += a.x; s += a.y; s += a.z; s += a.w;
            s += b.x; s += b.y; s += b.z; s += b.w;
            s += c.x; s += c.y; s += c.z; s += c.w;
            s += d.x; s += d.y; s += d.z; s += d.w;
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
    // Output column j: one chain over the span in position order.  V rows
    // are staged through LDS a chunk at a time so the chain reads LDS.
    int8_t *vl = reinterpret_cast<int8_t *>(sc + ((g.cap + 3) & ~3));
    const int8_t *vb = reinterpret_cast<const int8_t *>(blk + g.v_off) + size_t(kvh) * g.cap * g.VD;
    const int pieces = g.VD / 16;        // 16-byte pieces per V row
    const int chunk = kVChunk / g.VD;    // positions per pass
    float acc = 0.0f;
    for (int c0 = 0; c0 < span; c0 += chunk) {
        const int cn = span - c0 < chunk ? span - c0 : chunk;
        __syncthreads();  // weights written / previous chunk consumed
        for (int e = tid; e < cn * pieces; e += kThreads) {
            const int t = e / pieces, pc = e - t * pieces;
            int slot = base + c0 + t;
            if (slot >= g.cap) slot -= g.cap;
            reinterpret_cast<uint4 *>(vl)[e] =
                *reinterpret_cast<const uint4 *>(vb + size_t(slot) * g.VD + pc * 16);
        }
        __syncthreads();
        if (tid < g.VD) {
            const float *w = sc + c0;  // c0 is a multiple of the chunk: 16-byte aligned
            const int8_t *col = vl + tid;
            int t = 0;
            for (; t + 16 <= cn; t += 16) {
                const float4 w0 = *reinterpret_cast<const float4 *>(w + t);
                const float4 w1 = *reinterpret_cast<const float4 *>(w + t + 4);
                const float4 w2 = *reinterpret_cast<const float4 *>(w + t + 8);
                const float4 w3 = *reinterpret_cast<const float4 *>(w + t + 12);
                const float ws[16] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w,
                                      w2.x, w2.y, w2.z, w2.w, w3.x, w3.y, w3.z, w3.w};
                float p[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) p[u] = ws[u] * float(col[(t + u) * g.VD]);
#pragma unroll
                for (int u = 0; u < 16; ++u) acc += p[u];
            }
            for (; t < cn; ++t) acc += w[t] * float(col[t * g.VD]);
        }
    }
    if (tid < g.VD)
        out[(i * g.H + h) * size_t(g.VD) + tid] =
            gate_half_fwht(acc, gate ? gate + (i * g.H + h) * size_t(g.VD) : nullptr, tid);
}

// One workgroup per (query row, query head): the query head into LDS
// (fake-quantised on request, quant_rows, v3/model.rs:289-293), then the
// shared pass.  Blocks are numbered as described above.
template <int CW, int QC, bool KF>
__global__ __launch_bounds__(kAttn2Threads, 4) void attn_exact2_kernel(
    ndkv::Geom g, const uint8_t *__restrict__ kv, size_t stride, const int32_t *__restrict__ lo,
    const int32_t *__restrict__ hi, const float *__restrict__ q, float scale, int quant_query,
    float *__restrict__ out, int groups, int rows_per_block, const float *__restrict__ gate)
{
    extern __shared__ __align__(16) float sm[];
    __shared__ AttnLds L;
    const int tid = threadIdx.x;
    const int R = g.H / g.KVH;
    const int xcd = int(blockIdx.x) & 7, slot8 = int(blockIdx.x) >> 3;
    const int grp = (slot8 / R) * 8 + xcd;
    if (grp >= groups) return;  // padding block: the whole block leaves
    const int i = grp / g.KVH, kvh = grp - (grp / g.KVH) * g.KVH;
    const int h = kvh * R + slot8 % R;
    const uint8_t *blk = kv + size_t(i / rows_per_block) * stride;
    const int p0 = lo[i];
    const int span = hi[i] - p0 + 1;
    float *orow = out + (size_t(i) * g.H + h) * g.VD;
    if (p0 < 0 || span < 1 || span > g.cap) {
        for (int j = tid; j < g.VD; j += kAttn2Threads) orow[j] = NAN;
        return;
    }
    const float *qv = q + (size_t(i) * g.H + h) * g.QK;
    if (tid < 64) {
        if (quant_query) {
            float s, inv;
            ndkv::quant_scale_wave(qv, g.QK, s, inv);
            for (int e = tid; e < g.QK; e += 64) L.qs[e] = ndkv::quant_code(qv[e], inv) * s;
        } else {
            for (int e = tid; e < g.QK; e += 64) L.qs[e] = qv[e];
        }
    }
    __syncthreads();
    attn_exact2_run<CW, QC, KF, false>(g, blk, kvh, p0, span, scale, sm, L, nullptr, orow,
                                       gate ? gate + (size_t(i) * g.H + h) * g.VD : nullptr);
}

// ---------------------------------------------------------------------------
// Row sums in the reference's order: ((0 + x[0]) + x[1]) + ... per row, one
// workgroup a row, the row staged in LDS.  Rows of terms >= +0 (sums of
// squares, softmax sums) take the exact parallel fold of nd_fold.h; any
// other row the plain chain, which the fold itself falls back to.
// ---------------------------------------------------------------------------
constexpr int kFoldRowMax = 4096;
constexpr int kFoldThreads = 256;

__global__ __launch_bounds__(kFoldThreads) void fold_rows_kernel(const float *__restrict__ x, int n,
                                                                  float *__restrict__ y)
{
    __shared__ __align__(16) float buf[kFoldRowMax];
    __shared__ NdFoldLds<kFoldThreads> fl;
    const float *row = x + size_t(blockIdx.x) * n;
    for (int i = threadIdx.x; i < n; i += kFoldThreads) buf[i] = row[i];
    __syncthreads();
    const float f = nd_fold_nonneg<kFoldThreads, kFoldRowMax / kFoldThreads>(buf, n, fl);
    if (threadIdx.x == 0) y[blockIdx.x] = f;
}

}  // namespace

extern "C" {

int nd_fold_rows(nd_ctx *ctx, const float *x, size_t rows, size_t n, float *y)
{
    ND_ENTER(ctx);
    ND_REQUIRE(n >= 1 && n <= size_t(kFoldRowMax), "fold_rows: n %zu outside 1..%d", n, kFoldRowMax);
    if (rows == 0) return ND_OK;
    ND_REQUIRE(x && y, "fold_rows: null buffer");
    ND_REQUIRE(rows <= 0x7fffffffu, "fold_rows: %zu rows", rows);
    hipLaunchKernelGGL(fold_rows_kernel, dim3(unsigned(rows)), dim3(kFoldThreads), 0, ctx->stream, x,
                       int(n), y);
    return nd::check_launch("fold_rows");
}

int nd_cq_matvec_rows_exact(nd_ctx *ctx, const nd_cq *w, const float *xh, size_t row_start,
                            size_t rows, float *y)
{
    return nd_cq_exact_set(ctx, ctx ? ctx->stream : nullptr, 1, &w, xh, 1, &row_start, &rows, &y,
                           "cq_matvec_exact");
}

int nd_cq_matmul_rows_exact(nd_ctx *ctx, const nd_cq *w, const float *xh, size_t batch,
                            size_t row_start, size_t rows, float *y)
{
    return nd_cq_exact_set(ctx, ctx ? ctx->stream : nullptr, 1, &w, xh, batch, &row_start, &rows, &y,
                           "cq_matmul_exact");
}

int nd_attend_step_i8_exact(nd_ctx *ctx, const nd_kv_geom *g, const void *kv, size_t kv_stride,
                            size_t count, const int32_t *lo, const int32_t *hi, const float *q,
                            float scale, int quant_query, float *out)
{
    return nd_attend_exact_rows(ctx, g, kv, kv_stride, count, 1, lo, hi, q, scale, quant_query, out,
                                nullptr);
}

int nd_attend_step_f32_exact(nd_ctx *ctx, const nd_kv_geom *g, const void *kv, size_t kv_stride,
                             size_t count, const int32_t *lo, const int32_t *hi, const float *q,
                             float scale, float *out)
{
    return nd_attend_exact_rows(ctx, g, kv, kv_stride, count, 1, lo, hi, q, scale, 0, out, nullptr,
                                1);
}

}  // extern "C"

int nd_attend_exact_rows(nd_ctx *ctx, const nd_kv_geom *g, const void *kv, size_t kv_stride,
                         size_t count, int rows_per_block, const int32_t *lo, const int32_t *hi,
                         const float *q, float scale, int quant_query, float *out,
                         const float *gate, int kv_f32)
{
    ND_ENTER(ctx);
    ND_REQUIRE(rows_per_block >= 1, "rows_per_block %d", rows_per_block);
    ND_REQUIRE(!gate || g->v_head_dim == 64, "the gated epilogue needs v_head_dim 64, not %d",
               g->v_head_dim);
    if (int rc = ndkv::check_geom(g)) return rc;
    ND_REQUIRE(!kv_f32 || !quant_query, "the f32 view takes the query as it is");
    ND_REQUIRE(!kv_f32 || (g->v_head_dim <= 128 && g->cap <= kAttn2MaxCap),
               "the f32 view needs v_head_dim <= 128 and cap <= %d (v %d, cap %d)", kAttn2MaxCap,
               g->v_head_dim, g->cap);
    if (count == 0) return ND_OK;
    ND_REQUIRE(kv && lo && hi && q && out, "null buffer");
    ND_REQUIRE(count <= 65535, "count %zu above 65535", count);
    ND_REQUIRE(g->cap <= kAttnMaxCap, "cap %d above %d for the reference-order attention", g->cap,
               kAttnMaxCap);
    ND_REQUIRE((reinterpret_cast<uintptr_t>(kv) & 255) == 0 && kv_stride % 256 == 0,
               "kv blocks must be 256-byte aligned");
    if (g->v_head_dim <= 128 && g->cap <= kAttn2MaxCap) {
        const int R = g->num_heads / g->num_kv_heads;
        const size_t groups = count * size_t(g->num_kv_heads);
        const size_t blocks = 8 * size_t(R) * ((groups + 7) / 8);
        ND_REQUIRE(blocks <= 0x7fffffffu, "count %zu too large", count);
        const size_t lds = size_t((g->cap + 3) & ~3) * 4 + 2 * kProdBuf * sizeof(float);
        const int cw = g->v_head_dim <= 64 ? 1 : 2;
        const int qc = g->qk_head_dim <= 64 ? g->qk_head_dim / 16 : 0;
        ndkv::Geom kg = ndkv::make_geom(g);
        if (kv_f32) kg.v_off = nd_kv_f32_v_offset(g);
#define ND_ATTN2(CW, QC)                                                                          \
    if (kv_f32)                                                                                   \
        hipLaunchKernelGGL((attn_exact2_kernel<CW, QC, true>), dim3(unsigned(blocks)),            \
                           dim3(kAttn2Threads), lds, ctx->stream, kg,                             \
                           static_cast<const uint8_t *>(kv), kv_stride, lo, hi, q, scale, 0, out, \
                           int(groups), rows_per_block, gate);                                    \
    else                                                                                          \
        hipLaunchKernelGGL((attn_exact2_kernel<CW, QC, false>), dim3(unsigned(blocks)),           \
                           dim3(kAttn2Threads), lds, ctx->stream, kg,                             \
                           static_cast<const uint8_t *>(kv), kv_stride, lo, hi, q, scale,         \
                           quant_query, out, int(groups), rows_per_block, gate)
#define ND_ATTN2_QC(CW)                    \
    switch (qc) {                          \
    case 1: ND_ATTN2(CW, 1); break;        \
    case 2: ND_ATTN2(CW, 2); break;        \
    case 3: ND_ATTN2(CW, 3); break;        \
    case 4: ND_ATTN2(CW, 4); break;        \
    default: ND_ATTN2(CW, 0); break;       \
    }
        if (cw == 1) {
            ND_ATTN2_QC(1)
        } else {
            ND_ATTN2_QC(2)
        }
#undef ND_ATTN2_QC
#undef ND_ATTN2
        return nd::check_launch("attn_exact2");
    }
    dim3 grid(unsigned(g->num_heads), unsigned(count));
    const size_t lds = size_t((g->cap + 3) & ~3) * 4 + kVChunk;
    hipLaunchKernelGGL(attn_exact_kernel, grid, dim3(kThreads), lds, ctx->stream,
                       ndkv::make_geom(g), static_cast<const uint8_t *>(kv), kv_stride,
                       rows_per_block, lo, hi, q, scale, quant_query, out, gate);
    return nd::check_launch("attn_exact");
}
