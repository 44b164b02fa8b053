// int8 KV cache: quantise-on-append and decode attention that reads the int8
// cache directly (crates/needle-core/src/v3/cache.rs, v3/attention.rs).
//
// Quantisation is bit-exact with quant_scale/quant_into (cache.rs:80-104):
// absmax (order-free), scale = absmax / 127 with an IEEE divide,
// inv = 1 / scale, q = clamp(roundf(x * inv), -128, 127), roundf being
// round-half-away-from-zero as libm::roundf.  One wave per head vector.
//
// Attention (attend_step over Int8View, attention.rs:300-377) is split-K:
// a workgroup owns (query, kv head, span chunk) and every query head of its
// GQA group, so a kv head's int8 rows are read once for all of them.
//   scores  16-byte K vectors, NQ = qk/16 lanes per position, the lane's
//           16-wide slice of each query head in registers; lane partials are
//           summed per position through LDS, then * k_scale * scale.
//   softmax chunk max, e = exp(s - m), l = sum e.
//   values  4 columns per lane (one int8 dword per position), all query
//           heads accumulated in registers, reduced over position groups.
// Chunks merge in a second kernel with the usual (m, l, o) rescaling.
#include "nd_internal.h"

#include <cmath>

namespace {

constexpr int kThreads = 256;
constexpr int kMaxRep = 8;
constexpr int kMaxDim = 256;

__device__ inline float wave_max(float v)
{
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ inline float wave_sum(float v)
{
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// absmax of a head vector read by one wave; returns (scale, inv) exactly as
// quant_scale (cache.rs:80-91).
__device__ inline void quant_scale_wave(const float *x, int n, float &scale, float &inv)
{
    const int lane = threadIdx.x & 63;
    float a = 0.0f;
    for (int i = lane; i < n; i += 64) {
        const float v = x[i];
        const float av = v < 0.0f ? -v : v;
        if (av > a) a = av;
    }
    const float absmax = wave_max(a);
    scale = absmax > 0.0f ? absmax / 127.0f : 1.0f;
    inv = 1.0f / scale;
}

__device__ inline float quant_code(float x, float inv)
{
    const float r = roundf(x * inv);
    return r < -128.0f ? -128.0f : (r > 127.0f ? 127.0f : r);
}

// fake_quant_vec over rows (cache.rs:68-73); one wave per row.
__global__ __launch_bounds__(kThreads) void fake_quant_kernel(float *__restrict__ x, size_t rows,
                                                             int dim)
{
    const size_t r = size_t(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
    if (r >= rows) return;
    float *v = x + r * dim;
    float scale, inv;
    quant_scale_wave(v, dim, scale, inv);
    for (int i = threadIdx.x & 63; i < dim; i += 64) v[i] = quant_code(v[i], inv) * scale;
}

// quantize_rows (cache.rs:113-122); one wave per row.
__global__ __launch_bounds__(kThreads) void quantize_rows_kernel(const float *__restrict__ x,
                                                                size_t rows, int dim,
                                                                int8_t *__restrict__ q,
                                                                float *__restrict__ scales)
{
    const size_t r = size_t(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float *v = x + r * dim;
    float scale, inv;
    quant_scale_wave(v, dim, scale, inv);
    for (int i = threadIdx.x & 63; i < dim; i += 64) q[r * dim + i] = int8_t(quant_code(v[i], inv));
    if ((threadIdx.x & 63) == 0) scales[r] = scale;
}

struct Geom {
    int H, KVH, QK, VD, cap;
    size_t v_off, ks_off, vs_off;
};

// write_kv (cache.rs:346-379): wave w of block (i, h) quantises K (w=0) or
// V (w=1) of kv head h for row i into slot pos[i] % cap.
__global__ __launch_bounds__(128) void kv_write_kernel(Geom g, uint8_t *__restrict__ kv,
                                                      size_t kv_stride,
                                                      const int32_t *__restrict__ pos,
                                                      const float *__restrict__ k,
                                                      const float *__restrict__ v)
{
    const size_t i = blockIdx.x;
    const int h = blockIdx.y;
    const int which = threadIdx.x >> 6;
    const int p = pos[i];
    if (p < 0) return;
    const int slot = p % g.cap;
    uint8_t *blk = kv + i * kv_stride;
    const int dim = which ? g.VD : g.QK;
    const float *src = which ? v + i * size_t(g.KVH) * g.VD + size_t(h) * g.VD
                             : k + i * size_t(g.KVH) * g.QK + size_t(h) * g.QK;
    int8_t *dst = reinterpret_cast<int8_t *>(blk + (which ? g.v_off : 0)) +
                  (size_t(h) * g.cap + slot) * dim;
    float *sc = reinterpret_cast<float *>(blk + (which ? g.vs_off : g.ks_off)) + size_t(h) * g.cap + slot;
    float scale, inv;
    quant_scale_wave(src, dim, scale, inv);
    for (int e = threadIdx.x & 63; e < dim; e += 64) dst[e] = int8_t(quant_code(src[e], inv));
    if ((threadIdx.x & 63) == 0) *sc = scale;
}

// ---------------------------------------------------------------------------
// Split-K decode attention.
// ---------------------------------------------------------------------------
template <int REP, int NQ, int NV4>
__global__ __launch_bounds__(kThreads) void attn_i8_kernel(
    Geom g, const uint8_t *__restrict__ kv, size_t kv_stride, const int32_t *__restrict__ lo_a,
    const int32_t *__restrict__ hi_a, const float *__restrict__ q, float scale, int quant_query,
    int chunk, int nchunks, float *__restrict__ out, float *__restrict__ part_o,
    float *__restrict__ part_ml)
{
    // NQ = qk/16 lanes per position for K; NV4 = vd/4 lanes per position for V.
    constexpr int kTPK = kThreads / NQ;   // positions per K pass
    constexpr int kTPV = kThreads / NV4;  // positions per V pass (position groups)
    extern __shared__ float smem[];
    float *qs = smem;                          // [REP][QK]
    float *sp = qs + REP * kMaxDim;            // [REP][chunk][NQ] partial dots
    float *ss = sp + REP * chunk * NQ;         // [chunk][REP] scores, then weights
    float *red = ss + chunk * REP;             // reductions: [REP][kThreads/64] + stats
    float *vred = red + 2 * REP * (kThreads / 64) + 2 * REP;  // [4 waves][16 lanes][REP*4]

    const size_t qi = blockIdx.z;
    const int kvh = blockIdx.y;
    const int c = blockIdx.x;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int QK = NQ * 16, VD = NV4 * 4;

    const int lo = lo_a[qi], hi = hi_a[qi];
    const int span = hi - lo + 1;
    const bool bad = lo < 0 || span < 1 || span > g.cap || span > chunk * nchunks;
    const int p0 = c * chunk;
    const int n = bad ? 0 : max(0, min(chunk, span - p0));

    const uint8_t *blk = kv + qi * kv_stride;
    const int8_t *kb = reinterpret_cast<const int8_t *>(blk) + size_t(kvh) * g.cap * QK;
    const int8_t *vb = reinterpret_cast<const int8_t *>(blk + g.v_off) + size_t(kvh) * g.cap * VD;
    const float *ksb = reinterpret_cast<const float *>(blk + g.ks_off) + size_t(kvh) * g.cap;
    const float *vsb = reinterpret_cast<const float *>(blk + g.vs_off) + size_t(kvh) * g.cap;

    // Query heads kvh*REP .. +REP, optionally fake-quantised per head.
    const float *qg = q + qi * size_t(g.H) * QK + size_t(kvh) * REP * QK;
    for (int e = t; e < REP * QK; e += kThreads) qs[(e / QK) * kMaxDim + e % QK] = qg[e];
    __syncthreads();
    if (quant_query) {
        for (int r = wave; r < REP; r += kThreads / 64) {
            float sc, inv;
            quant_scale_wave(qs + r * kMaxDim, QK, sc, inv);
            for (int e = lane; e < QK; e += 64) qs[r * kMaxDim + e] = quant_code(qs[r * kMaxDim + e], inv) * sc;
        }
        __syncthreads();
    }

    // ---- scores ----
    const int sub = t % NQ;
    const bool kact = t < kTPK * NQ;
    float qr[REP][16];
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
        for (int e = 0; e < 16; ++e) qr[r][e] = qs[r * kMaxDim + sub * 16 + e];
    for (int pl = t / NQ; kact && pl < n; pl += kTPK) {
        const int slot = (lo + p0 + pl) % g.cap;
        const uint4 kvv = *reinterpret_cast<const uint4 *>(kb + size_t(slot) * QK + sub * 16);
        const uint32_t dw[4] = {kvv.x, kvv.y, kvv.z, kvv.w};
        float kf[16];
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                kf[4 * d + b] = float(int32_t(dw[d] << (24 - 8 * b)) >> 24);
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; e += 2) {
                a0 += qr[r][e] * kf[e];
                a1 += qr[r][e + 1] * kf[e + 1];
            }
            sp[(r * chunk + pl) * NQ + sub] = a0 + a1;
        }
    }
    __syncthreads();
    float mloc[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r) mloc[r] = -INFINITY;
    for (int pl = t; pl < n; pl += kThreads) {
        const int slot = (lo + p0 + pl) % g.cap;
        const float ks = ksb[slot];
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            float a = 0.0f;
#pragma unroll
            for (int s2 = 0; s2 < NQ; ++s2) a += sp[(r * chunk + pl) * NQ + s2];
            const float s = (a * ks) * scale;
            ss[pl * REP + r] = s;
            mloc[r] = fmaxf(mloc[r], s);
        }
    }
    // block max per head
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        const float m = wave_max(mloc[r]);
        if (lane == 0) red[r * (kThreads / 64) + wave] = m;
    }
    __syncthreads();
    float mx[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        float m = -INFINITY;
#pragma unroll
        for (int w2 = 0; w2 < kThreads / 64; ++w2) m = fmaxf(m, red[r * (kThreads / 64) + w2]);
        mx[r] = m;
    }
    __syncthreads();
    // e = exp(s - m); weights w = e * v_scale for the value pass; l = sum e.
    float lloc[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r) lloc[r] = 0.0f;
    for (int pl = t; pl < n; pl += kThreads) {
        const int slot = (lo + p0 + pl) % g.cap;
        const float vs = vsb[slot];
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            const float e = expf(ss[pl * REP + r] - mx[r]);
            lloc[r] += e;
            ss[pl * REP + r] = e * vs;
        }
    }
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        const float l = wave_sum(lloc[r]);
        if (lane == 0) red[r * (kThreads / 64) + wave] = l;
    }
    __syncthreads();

    // ---- values: lane owns columns 4*(t % NV4) .. +4 ----
    const int vsub = t % NV4;
    float acc[REP][4];
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[r][e] = 0.0f;
    for (int pl = t / NV4; pl < n; pl += kTPV) {
        const int slot = (lo + p0 + pl) % g.cap;
        const uint32_t dw = *reinterpret_cast<const uint32_t *>(vb + size_t(slot) * VD + vsub * 4);
        float vf[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) vf[b] = float(int32_t(dw << (24 - 8 * b)) >> 24);
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            const float wgt = ss[pl * REP + r];
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[r][e] += wgt * vf[e];
        }
    }
    // Reduce over position groups: lanes sharing vsub within a wave, then
    // across waves through LDS.
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            for (int off = NV4; off < 64; off <<= 1) acc[r][e] += __shfl_xor(acc[r][e], off, 64);
    if (lane < NV4) {
#pragma unroll
        for (int r = 0; r < REP; ++r)
#pragma unroll
            for (int e = 0; e < 4; ++e) vred[(wave * NV4 + lane) * REP * 4 + r * 4 + e] = acc[r][e];
    }
    __syncthreads();

    // ---- write this chunk ----
    for (int o = t; o < REP * VD; o += kThreads) {
        const int r = o / VD, col = o % VD;
        const int ls = col / 4, e = col % 4;
        float s = 0.0f;
        for (int w2 = 0; w2 < kThreads / 64; ++w2) s += vred[(w2 * NV4 + ls) * REP * 4 + r * 4 + e];
        float l = 0.0f;
        for (int w2 = 0; w2 < kThreads / 64; ++w2) l += red[r * (kThreads / 64) + w2];
        const int head = kvh * REP + r;
        if (nchunks == 1) {
            out[qi * size_t(g.H) * VD + size_t(head) * VD + col] = bad ? NAN : s / l;
        } else {
            part_o[((qi * g.H + head) * size_t(nchunks) + c) * VD + col] = s;
            if (col == 0) {
                float *ml = part_ml + ((qi * g.H + head) * size_t(nchunks) + c) * 2;
                ml[0] = bad ? NAN : (n > 0 ? mx[r] : -INFINITY);
                ml[1] = l;
            }
        }
    }
}

// Merge chunk partials: out = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M).
__global__ __launch_bounds__(kThreads) void attn_combine_kernel(Geom g, int nchunks,
                                                               const float *__restrict__ part_o,
                                                               const float *__restrict__ part_ml,
                                                               float *__restrict__ out)
{
    const size_t qi = blockIdx.y;
    const int head = blockIdx.x;
    const size_t base = (qi * g.H + head) * size_t(nchunks);
    float M = -INFINITY;
    for (int c = 0; c < nchunks; ++c) M = fmaxf(M, part_ml[(base + c) * 2]);
    for (int col = threadIdx.x; col < g.VD; col += blockDim.x) {
        float O = 0.0f, L = 0.0f;
        for (int c = 0; c < nchunks; ++c) {
            const float m = part_ml[(base + c) * 2];
            if (m == -INFINITY) continue;
            const float f = expf(m - M);
            O += part_o[(base + c) * g.VD + col] * f;
            L += part_ml[(base + c) * 2 + 1] * f;
        }
        out[qi * size_t(g.H) * g.VD + size_t(head) * g.VD + col] = O / L;
    }
}

Geom make_geom(const nd_kv_geom *k)
{
    Geom g;
    g.H = k->num_heads;
    g.KVH = k->num_kv_heads;
    g.QK = k->qk_head_dim;
    g.VD = k->v_head_dim;
    g.cap = k->cap;
    g.v_off = nd_kv_v_offset(k);
    g.ks_off = nd_kv_ks_offset(k);
    g.vs_off = nd_kv_vs_offset(k);
    return g;
}

int check_geom(const nd_kv_geom *g)
{
    ND_REQUIRE(g, "null geometry");
    ND_REQUIRE(g->num_kv_heads > 0 && g->num_heads > 0 && g->num_heads % g->num_kv_heads == 0,
               "num_heads %d must be a positive multiple of num_kv_heads %d", g->num_heads,
               g->num_kv_heads);
    ND_REQUIRE(g->num_heads / g->num_kv_heads <= kMaxRep, "kv repeat %d above %d",
               g->num_heads / g->num_kv_heads, kMaxRep);
    ND_REQUIRE(g->qk_head_dim > 0 && g->qk_head_dim % 16 == 0 && g->qk_head_dim <= kMaxDim,
               "qk_head_dim %d must be a multiple of 16 in 16..%d", g->qk_head_dim, kMaxDim);
    ND_REQUIRE(g->v_head_dim > 0 && g->v_head_dim % 16 == 0 && g->v_head_dim <= kMaxDim,
               "v_head_dim %d must be a multiple of 16 in 16..%d", g->v_head_dim, kMaxDim);
    ND_REQUIRE(g->cap > 0 && g->cap <= (1 << 24), "cap %d out of range", g->cap);
    return ND_OK;
}

size_t attn_smem_bytes(int rep, int nq, int chunk)
{
    return sizeof(float) * (size_t(rep) * kMaxDim + size_t(rep) * chunk * nq + size_t(chunk) * rep +
                            2 * rep * (kThreads / 64) + 2 * rep + 4 * 16 * rep * 4);
}

template <int REP, int NQ, int NV4>
void launch_attn(dim3 grid, size_t smem, hipStream_t s, Geom g, const uint8_t *kv, size_t stride,
                 const int32_t *lo, const int32_t *hi, const float *q, float scale, int qq,
                 int chunk, int nchunks, float *out, float *po, float *pml)
{
    hipLaunchKernelGGL((attn_i8_kernel<REP, NQ, NV4>), grid, dim3(kThreads), smem, s, g, kv, stride,
                       lo, hi, q, scale, qq, chunk, nchunks, out, po, pml);
}

using AttnFn = void (*)(dim3, size_t, hipStream_t, Geom, const uint8_t *, size_t, const int32_t *,
                        const int32_t *, const float *, float, int, int, int, float *, float *,
                        float *);

// Instantiated shapes: the v3 geometry (12/2 heads, qk 48, v 64) and the
// MHA cache (qk = v = 64), plus every repeat 1..8 at qk 48/64, v 64.
template <int REP>
AttnFn pick_nq(int nq, int nv4)
{
    if (nv4 != 16) return nullptr;
    switch (nq) {
    case 3: return launch_attn<REP, 3, 16>;
    case 4: return launch_attn<REP, 4, 16>;
    default: return nullptr;
    }
}

AttnFn pick_attn(int rep, int nq, int nv4)
{
    switch (rep) {
    case 1: return pick_nq<1>(nq, nv4);
    case 2: return pick_nq<2>(nq, nv4);
    case 3: return pick_nq<3>(nq, nv4);
    case 4: return pick_nq<4>(nq, nv4);
    case 6: return pick_nq<6>(nq, nv4);
    case 8: return pick_nq<8>(nq, nv4);
    default: return nullptr;
    }
}

}  // namespace

extern "C" {

size_t nd_kv_v_offset(const nd_kv_geom *g)
{
    return nd::align_up(size_t(g->num_kv_heads) * g->cap * g->qk_head_dim, 256);
}

size_t nd_kv_ks_offset(const nd_kv_geom *g)
{
    return nd_kv_v_offset(g) + nd::align_up(size_t(g->num_kv_heads) * g->cap * g->v_head_dim, 256);
}

size_t nd_kv_vs_offset(const nd_kv_geom *g)
{
    return nd_kv_ks_offset(g) + nd::align_up(size_t(g->num_kv_heads) * g->cap * 4, 256);
}

size_t nd_kv_block_bytes(const nd_kv_geom *g)
{
    return nd_kv_vs_offset(g) + nd::align_up(size_t(g->num_kv_heads) * g->cap * 4, 256);
}

int nd_fake_quant(nd_ctx *ctx, float *x, size_t rows, size_t dim)
{
    if (int rc = nd::enter(ctx)) return rc;
    if (rows == 0) return ND_OK;
    ND_REQUIRE(x && dim > 0 && dim <= (1u << 20), "bad arguments");
    const size_t blocks = (rows + 3) / 4;
    ND_REQUIRE(blocks <= 0x7fffffff, "too many rows");
    hipLaunchKernelGGL(fake_quant_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0, ctx->stream, x,
                       rows, int(dim));
    return nd::check_launch("fake_quant");
}

int nd_quantize_rows(nd_ctx *ctx, const float *x, size_t rows, size_t head_dim, int8_t *ints,
                     float *scales)
{
    if (int rc = nd::enter(ctx)) return rc;
    if (rows == 0) return ND_OK;
    ND_REQUIRE(x && ints && scales && head_dim > 0 && head_dim <= (1u << 20), "bad arguments");
    const size_t blocks = (rows + 3) / 4;
    ND_REQUIRE(blocks <= 0x7fffffff, "too many rows");
    hipLaunchKernelGGL(quantize_rows_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0, ctx->stream,
                       x, rows, int(head_dim), ints, scales);
    return nd::check_launch("quantize_rows");
}

int nd_kv_write(nd_ctx *ctx, const nd_kv_geom *g, void *kv, size_t kv_stride, size_t count,
                const int32_t *pos, const float *k, const float *v)
{
    if (int rc = nd::enter(ctx)) return rc;
    if (int rc = check_geom(g)) return rc;
    if (count == 0) return ND_OK;
    ND_REQUIRE(kv && pos && k && v, "null buffer");
    ND_REQUIRE(count <= 0x7fffffff, "count too large");
    dim3 grid(unsigned(count), unsigned(g->num_kv_heads));
    hipLaunchKernelGGL(kv_write_kernel, grid, dim3(128), 0, ctx->stream, make_geom(g),
                       static_cast<uint8_t *>(kv), kv_stride, pos, k, v);
    return nd::check_launch("kv_write");
}

int nd_attend_step_i8(nd_ctx *ctx, const nd_kv_geom *g, const void *kv, size_t kv_stride,
                      size_t count, const int32_t *lo, const int32_t *hi, const float *q,
                      float scale, int quant_query, float *out)
{
    if (int rc = nd::enter(ctx)) return rc;
    if (int rc = check_geom(g)) return rc;
    if (count == 0) return ND_OK;
    ND_REQUIRE(kv && lo && hi && q && out, "null buffer");
    ND_REQUIRE(count <= 65535, "count %zu above 65535", count);
    ND_REQUIRE((reinterpret_cast<uintptr_t>(kv) & 255) == 0 && kv_stride % 256 == 0,
               "kv blocks must be 256-byte aligned");
    const int rep = g->num_heads / g->num_kv_heads;
    const int nq = g->qk_head_dim / 16, nv4 = g->v_head_dim / 4;
    AttnFn fn = pick_attn(rep, nq, nv4);
    ND_REQUIRE(fn, "no attention kernel for repeat %d, qk %d, v %d", rep, g->qk_head_dim,
               g->v_head_dim);
    // Chunk: the largest that keeps the partial buffer within 32 KB and still
    // gives the launch a few thousand workgroups.
    const int span = g->cap;
    int chunk = 512;
    while (chunk > 64 && size_t(rep) * chunk * nq > 8192) chunk /= 2;
    while (chunk > 64 && count * size_t(g->num_kv_heads) * ((span + chunk - 1) / chunk) < 2048)
        chunk /= 2;
    const int nchunks = (span + chunk - 1) / chunk;
    ND_REQUIRE(nchunks <= 65535, "span too long");
    float *po = nullptr, *pml = nullptr;
    if (nchunks > 1) {
        void *wsp = nullptr;
        const size_t n_o = count * size_t(g->num_heads) * nchunks * g->v_head_dim;
        const size_t n_ml = count * size_t(g->num_heads) * nchunks * 2;
        if (int rc = nd::workspace(ctx, (n_o + n_ml) * sizeof(float), &wsp)) return rc;
        po = static_cast<float *>(wsp);
        pml = po + n_o;
    }
    const size_t smem = attn_smem_bytes(rep, nq, chunk);
    dim3 grid(unsigned(nchunks), unsigned(g->num_kv_heads), unsigned(count));
    fn(grid, smem, ctx->stream, make_geom(g), static_cast<const uint8_t *>(kv), kv_stride, lo, hi, q,
       scale, quant_query, chunk, nchunks, out, po, pml);
    if (int rc = nd::check_launch("attn_i8")) return rc;
    if (nchunks > 1) {
        hipLaunchKernelGGL(attn_combine_kernel, dim3(unsigned(g->num_heads), unsigned(count)),
                           dim3(64), 0, ctx->stream, make_geom(g), nchunks, po, pml, out);
        return nd::check_launch("attn_combine");
    }
    return ND_OK;
}

}  // extern "C"
