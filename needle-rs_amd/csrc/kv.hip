// int8 KV cache: quantise-on-append and decode attention that reads the int8
// cache directly (crates/needle-core/src/v3/cache.rs, v3/attention.rs).
//
// Quantisation is bit-exact with quant_scale/quant_into (cache.rs:80-104):
// absmax (order-free), scale = absmax / 127 with an IEEE divide,
// inv = 1 / scale, q = clamp(roundf(x * inv), -128, 127), roundf being
// round-half-away-from-zero as libm::roundf.  One wave per head vector.
//
// Attention (attend_step over Int8View, attention.rs:300-377) reads the int8
// cache directly: a workgroup owns (query, kv head) -- every query head of
// the GQA group, so a kv head's int8 rows are read once for all of them --
// and walks its span in chunks with an online softmax (flash decoding).  The
// span is split across workgroups, with a merge pass, only when there are
// too few (query, kv head) pairs to fill the GPU (batch-1 decode).
#include "nd_internal.h"
#include "nd_kv_internal.h"

#include <cmath>
#include <mutex>

// Split-K partials of nd_attend_step_i8_noalloc: one fixed device array per
// GPU (every device the library runs on holds its copy until the process
// ends).  Host code never passes `scratch` itself to a kernel: its name is a
// host-side stand-in, and the device address comes from hipGetSymbolAddress
// once per device (nd::noalloc_setup, called when a context is created; if
// it fails there, the context is still created and this entry point reports
// the missing address).
static constexpr size_t kNoAllocScratchFloats = size_t(1) << 20;  // 4 MiB
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch[kMaxDevices] = {};
}  // namespace

namespace nd {

int noalloc_setup(int device)
{
    if (device < 0 || device >= kMaxDevices)
        return fail(ND_ERR_ARG, "device %d beyond the %d the no-allocation scratch covers", device,
                    kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[device]) return ND_OK;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(ND_ERR_HIP, "hipGetSymbolAddress(scratch) gave a null address");
    g_scratch[device] = static_cast<float *>(p);
    return ND_OK;
}

}  // namespace nd

namespace {

using namespace ndkv;

constexpr int kThreads = 256;

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

// write_kv with KvPrecision::F32 (cache.rs:359-362): block (i, h) copies kv
// head h's K and V of row i into slot pos[i] % cap of the f32 block.
__global__ __launch_bounds__(64) void kv_write_f32_kernel(Geom g, uint8_t *__restrict__ kv,
                                                          size_t kv_stride,
                                                          const int32_t *__restrict__ pos,
                                                          const float *__restrict__ k,
                                                          const float *__restrict__ v)
{
    const size_t i = blockIdx.x;
    const int h = blockIdx.y;
    const int p = pos[i];
    if (p < 0) return;
    const int slot = p % g.cap;
    uint8_t *blk = kv + i * kv_stride;
    const float *ks = k + (i * size_t(g.KVH) + h) * g.QK;
    const float *vs = v + (i * size_t(g.KVH) + h) * g.VD;
    float *kd = reinterpret_cast<float *>(blk) + (size_t(h) * g.cap + slot) * g.QK;
    float *vd = reinterpret_cast<float *>(blk + g.v_off) + (size_t(h) * g.cap + slot) * g.VD;
    for (int e = threadIdx.x; e < g.QK; e += 64) kd[e] = ks[e];
    for (int e = threadIdx.x; e < g.VD; e += 64) vd[e] = vs[e];
}

// ---------------------------------------------------------------------------
// Decode attention over the int8 ring, flash-decoding style.
//
// Block = (query i, kv head g, split s).  It walks its share of the span in
// chunks of CH positions with an online softmax (running max m, running sum
// l, accumulator rescaled by exp(m_old - m_new)), so one block can cover a
// whole span and no merge is needed when sessions x kv heads fill the GPU.
// Register pipeline: a chunk's K and V are already in registers when it
// starts; the next chunk's K loads are issued as soon as the scores are
// done, and its V loads as soon as the value pass is done.
//   K: KL = qk/16 lanes per position, one 16-byte int8 vector each, the
//      lane's 16-wide slice of every query head of the group in registers.
//   V: VL = vd/VW lanes per position, VW bytes each (16 for up to two query
//      heads per kv head, else 8), REP x VW accumulators per lane.
// Scores, weights and block reductions go through LDS.
template <int REP, int QK, int VD, int VW>
struct AttnShape {
    static constexpr int KL = QK / 16;
    static constexpr int KPP = kThreads / KL;                 // positions per K pass
    static constexpr int VL = VD / VW;
    static constexpr int VPP = kThreads / VL;                 // positions per V pass
    // positions per chunk: 256 keeps the registers at 119 (four waves a
    // SIMD) and two chunks of a 512-long span in flight; 512 took 157
    // (three), and at 12 heads x 64 measured 5.37 / 5.96 / 5.96 TB/s at ctx
    // 512 / 2048 / 8192 against 5.69 / 6.32 / 6.34 with 256 (192: 5.10 /
    // 5.83 / 5.91; 384: 4.43 / 5.47 / 5.73)
    static constexpr int CH = 256;
    static constexpr int KP = (CH + KPP - 1) / KPP;           // K passes per chunk
    // One query head a kv head, KL a power of two (qk 16 .. 256) and one
    // pass per lane of a position: the KL partial dots meet through DPP in
    // registers, no LDS and no barrier.  qk 48 (three lanes a position)
    // sums them in LDS, and so do grouped heads (their REP dots a pass held
    // across the passes took 6-55 more VGPRs than the LDS sums)
    static constexpr bool kLaneSums =
        REP == 1 && (KL & (KL - 1)) == 0 && KL <= 16 && KP == KL && KPP * KL == kThreads;
    static constexpr int VP = CH / VPP;                       // V passes per chunk
};

template <int VW>
struct VVec;
template <>
struct VVec<16> {
    typedef uint32_t T __attribute__((ext_vector_type(4)));
};
template <>
struct VVec<8> {
    typedef uint32_t T __attribute__((ext_vector_type(2)));
};

__device__ inline float i8_at(uint32_t dw, int b) { return float(int32_t(dw << (24 - 8 * b)) >> 24); }

template <int REP, int QK, int VD, int VW>
__global__ __launch_bounds__(kThreads) void attn_i8_kernel(
    Geom g, const uint8_t *__restrict__ kv, size_t kv_stride, const int32_t *__restrict__ lo_a,
    const int32_t *__restrict__ hi_a, const float *__restrict__ q, float scale, int quant_query,
    int splits, float *__restrict__ out, float *__restrict__ part_o, float *__restrict__ part_ml)
{
    using S = AttnShape<REP, QK, VD, VW>;
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    using VT = typename VVec<VW>::T;
    constexpr int CH = S::CH, NW = kThreads / 64;
    __shared__ float qs[REP][QK];
    __shared__ float sp[REP][CH * S::KL];  // lane partial dots
    __shared__ float wsh[REP][CH];         // scores, then weights
    __shared__ float red[REP][NW];
    __shared__ float vred[NW][REP][VD];

    const size_t qi = blockIdx.z;
    const int kvh = blockIdx.y;
    const int split = blockIdx.x;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;

    const int lo = lo_a[qi], hi = hi_a[qi];
    const int span = hi - lo + 1;
    const bool bad = lo < 0 || span < 1 || span > g.cap;
    const int nch = bad ? 0 : (span + CH - 1) / CH;
    const int c_begin = int((long long)nch * split / splits);
    const int c_end = int((long long)nch * (split + 1) / splits);

    const uint8_t *blk = kv + qi * kv_stride;
    const int8_t *kb = reinterpret_cast<const int8_t *>(blk) + size_t(kvh) * g.cap * QK;
    const int8_t *vb = reinterpret_cast<const int8_t *>(blk + g.v_off) + size_t(kvh) * g.cap * VD;
    const float *ksb = reinterpret_cast<const float *>(blk + g.ks_off) + size_t(kvh) * g.cap;
    const float *vsb = reinterpret_cast<const float *>(blk + g.vs_off) + size_t(kvh) * g.cap;

    // Query heads kvh*REP .. +REP (fake-quantised per head on request).
    const float *qg = q + qi * size_t(g.H) * QK + size_t(kvh) * REP * QK;
    for (int e = t; e < REP * QK; e += kThreads) qs[e / QK][e % QK] = qg[e];
    __syncthreads();
    if (quant_query) {
        for (int r = wave; r < REP; r += NW) {
            float sc, inv;
            quant_scale_wave(qs[r], QK, sc, inv);
            for (int e = lane; e < QK; e += 64) qs[r][e] = quant_code(qs[r][e], inv) * sc;
        }
        __syncthreads();
    }
    const int ksub = t % S::KL;
    const int kpos = t / S::KL;  // position within a K pass
    const bool kact = t < S::KPP * S::KL;
    float qr[REP][16];
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
        for (int e = 0; e < 16; ++e) qr[r][e] = qs[r][ksub * 16 + e];
    const int vsub = t % S::VL;
    const int vpos = t / S::VL;

    u4 kr[S::KP];
    VT vr[S::VP];
    auto load_k = [&](int c) {
#pragma unroll
        for (int p = 0; p < S::KP; ++p) {
            const int pl = p * S::KPP + kpos;
            const int pc = min(c * CH + pl, span - 1);  // clamp: read a valid slot
            const int slot = (lo + pc) % g.cap;
            kr[p] = __builtin_nontemporal_load(reinterpret_cast<const u4 *>(kb + size_t(slot) * QK) + ksub);
        }
    };
    auto load_v = [&](int c) {
#pragma unroll
        for (int p = 0; p < S::VP; ++p) {
            const int pc = min(c * CH + p * S::VPP + vpos, span - 1);
            const int slot = (lo + pc) % g.cap;
            vr[p] = __builtin_nontemporal_load(reinterpret_cast<const VT *>(vb + size_t(slot) * VD) + vsub);
        }
    };
    if (c_begin < c_end) {
        load_k(c_begin);
        load_v(c_begin);
    }

    float m_run[REP], l_loc[REP], acc[REP][VW];
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        m_run[r] = -INFINITY;
        l_loc[r] = 0.0f;
#pragma unroll
        for (int e = 0; e < VW; ++e) acc[r][e] = 0.0f;
    }

    for (int c = c_begin; c < c_end; ++c) {
        const int n = min(CH, span - c * CH);
        float cmax[REP];
#pragma unroll
        for (int r = 0; r < REP; ++r) cmax[r] = -INFINITY;
        // the position this lane scores, its score and V scale (lane sums)
        const int own = ksub * S::KPP + kpos;
        float own_sc[REP], own_vs = 0.0f;
        if constexpr (S::kLaneSums) {
            // ---- scores: lane partial dots summed across the position's KL
            // lanes by DPP; lane ksub keeps pass ksub's position, and its
            // K and V scales are requested before the dots ----
            const int oslot = (lo + c * CH + min(own, n - 1)) % g.cap;
            const float ks = ksb[oslot];
            own_vs = vsb[oslot];
            float dot[REP];
#pragma unroll
            for (int r = 0; r < REP; ++r) dot[r] = 0.0f;
#pragma unroll
            for (int p = 0; p < S::KP; ++p) {
                const uint32_t dw[4] = {kr[p].x, kr[p].y, kr[p].z, kr[p].w};
                float kf[16];
#pragma unroll
                for (int d = 0; d < 4; ++d)
#pragma unroll
                    for (int b = 0; b < 4; ++b) kf[4 * d + b] = i8_at(dw[d], b);
#pragma unroll
                for (int r = 0; r < REP; ++r) {
                    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
                    for (int e = 0; e < 16; e += 2) {
                        a0 += qr[r][e] * kf[e];
                        a1 += qr[r][e + 1] * kf[e + 1];
                    }
                    const float v = ndl::group_sum<S::KL>(a0 + a1);
                    dot[r] = ksub == p ? v : dot[r];
                }
            }
            if (c + 1 < c_end) load_k(c + 1);  // lands during softmax and values
#pragma unroll
            for (int r = 0; r < REP; ++r) {
                own_sc[r] = (dot[r] * ks) * scale;
                if (own < n) cmax[r] = own_sc[r];
            }
        } else {
        // ---- scores: lane partial dots ----
#pragma unroll
        for (int p = 0; p < S::KP; ++p) {
            const int pl = p * S::KPP + kpos;
            if (kact && pl < CH) {
                const uint32_t dw[4] = {kr[p].x, kr[p].y, kr[p].z, kr[p].w};
                float kf[16];
#pragma unroll
                for (int d = 0; d < 4; ++d)
#pragma unroll
                    for (int b = 0; b < 4; ++b) kf[4 * d + b] = i8_at(dw[d], b);
#pragma unroll
                for (int r = 0; r < REP; ++r) {
                    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
                    for (int e = 0; e < 16; e += 2) {
                        a0 += qr[r][e] * kf[e];
                        a1 += qr[r][e + 1] * kf[e + 1];
                    }
                    sp[r][pl * S::KL + ksub] = a0 + a1;
                }
            }
        }
        if (c + 1 < c_end) load_k(c + 1);  // lands during softmax and values
        __syncthreads();
        // ---- per-position score, chunk max ----
        for (int pl = t; pl < n; pl += kThreads) {
            const int slot = (lo + c * CH + pl) % g.cap;
            const float ks = ksb[slot];
#pragma unroll
            for (int r = 0; r < REP; ++r) {
                float a = 0.0f;
#pragma unroll
                for (int s2 = 0; s2 < S::KL; ++s2) a += sp[r][pl * S::KL + s2];
                const float sc = (a * ks) * scale;
                wsh[r][pl] = sc;
                cmax[r] = fmaxf(cmax[r], sc);
            }
        }
        }
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            const float m = wave_max(cmax[r]);
            if (lane == 0) red[r][wave] = m;
        }
        __syncthreads();
        float alpha[REP], mnew[REP];
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            float m = m_run[r];
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) m = fmaxf(m, red[r][w2]);
            mnew[r] = m;
            alpha[r] = expf(m_run[r] - m);  // exp(-inf) = 0 on the first chunk
            m_run[r] = m;
            l_loc[r] *= alpha[r];
        }
        // ---- weights e * v_scale; running sum ----
        if constexpr (S::kLaneSums) {
            if (own < n) {
#pragma unroll
                for (int r = 0; r < REP; ++r) {
                    const float e = expf(own_sc[r] - mnew[r]);
                    l_loc[r] = l_loc[r] + e;
                    wsh[r][own] = e * own_vs;
                }
            }
        } else {
            for (int pl = t; pl < n; pl += kThreads) {
                const int slot = (lo + c * CH + pl) % g.cap;
                const float vs = vsb[slot];
#pragma unroll
                for (int r = 0; r < REP; ++r) {
                    const float e = expf(wsh[r][pl] - mnew[r]);
                    l_loc[r] = l_loc[r] + e;
                    wsh[r][pl] = e * vs;
                }
            }
        }
        __syncthreads();
        // ---- values ----
#pragma unroll
        for (int r = 0; r < REP; ++r)
#pragma unroll
            for (int e = 0; e < VW; ++e) acc[r][e] *= alpha[r];
#pragma unroll
        for (int p = 0; p < S::VP; ++p) {
            const int pl = p * S::VPP + vpos;
            if (pl < n) {
                float vf[VW];
#pragma unroll
                for (int d = 0; d < VW / 4; ++d)
#pragma unroll
                    for (int b = 0; b < 4; ++b) vf[4 * d + b] = i8_at(vr[p][d], b);
#pragma unroll
                for (int r = 0; r < REP; ++r) {
                    const float wgt = wsh[r][pl];
#pragma unroll
                    for (int e = 0; e < VW; ++e) acc[r][e] += wgt * vf[e];
                }
            }
        }
        if (c + 1 < c_end) load_v(c + 1);  // lands during the next scores
        __syncthreads();
    }

    // ---- reduce over the lanes sharing a V column slice ----
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
        for (int e = 0; e < VW; ++e)
            acc[r][e] = ndl::wave_sum_from<S::VL>(acc[r][e]);
    if (lane < S::VL) {
#pragma unroll
        for (int r = 0; r < REP; ++r)
#pragma unroll
            for (int e = 0; e < VW; ++e) vred[wave][r][lane * VW + e] = acc[r][e];
    }
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        const float l = wave_sum(l_loc[r]);
        if (lane == 0) red[r][wave] = l;
    }
    __syncthreads();
    for (int o = t; o < REP * VD; o += kThreads) {
        const int r = o / VD, col = o % VD;
        float s = 0.0f, l = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < NW; ++w2) {
            s += vred[w2][r][col];
            l += red[r][w2];
        }
        const int head = kvh * REP + r;
        if (splits == 1) {
            out[qi * size_t(g.H) * VD + size_t(head) * VD + col] = bad ? NAN : s / l;
        } else {
            part_o[((qi * g.H + head) * size_t(splits) + split) * VD + col] = s;
            if (col == 0) {
                float *ml = part_ml + ((qi * g.H + head) * size_t(splits) + split) * 2;
                ml[0] = bad ? NAN : (c_begin < c_end ? m_run[r] : -INFINITY);
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



template <int REP, int QK>
void launch_attn(dim3 grid, hipStream_t s, Geom g, const uint8_t *kv, size_t stride,
                 const int32_t *lo, const int32_t *hi, const float *q, float scale, int qq,
                 int splits, float *out, float *po, float *pml)
{
    constexpr int VW = REP <= 2 ? 16 : 8;
    hipLaunchKernelGGL((attn_i8_kernel<REP, QK, 64, VW>), grid, dim3(kThreads), 0, s, g, kv, stride,
                       lo, hi, q, scale, qq, splits, out, po, pml);
}

using AttnFn = void (*)(dim3, hipStream_t, Geom, const uint8_t *, size_t, const int32_t *,
                        const int32_t *, const float *, float, int, int, float *, float *, float *);

// Instantiated: qk 48 (the shipped v3 geometry) and 64 (the MHA cache), v 64,
// query heads per kv head 1, 2, 3, 4, 6, 8.
template <int REP>
AttnFn pick_qk(int qk, int vd)
{
    if (vd != 64) return nullptr;
    switch (qk) {
    case 48: return launch_attn<REP, 48>;
    case 64: return launch_attn<REP, 64>;
    default: return nullptr;
    }
}

AttnFn pick_attn(int rep, int qk, int vd)
{
    switch (rep) {
    case 1: return pick_qk<1>(qk, vd);
    case 2: return pick_qk<2>(qk, vd);
    case 3: return pick_qk<3>(qk, vd);
    case 4: return pick_qk<4>(qk, vd);
    case 6: return pick_qk<6>(qk, vd);
    case 8: return pick_qk<8>(qk, vd);
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

size_t nd_kv_f32_v_offset(const nd_kv_geom *g)
{
    return nd::align_up(size_t(g->num_kv_heads) * g->cap * g->qk_head_dim * 4, 256);
}

size_t nd_kv_f32_block_bytes(const nd_kv_geom *g)
{
    return nd_kv_f32_v_offset(g) + nd::align_up(size_t(g->num_kv_heads) * g->cap * g->v_head_dim * 4, 256);
}

int nd_kv_write_f32(nd_ctx *ctx, const nd_kv_geom *g, void *kv, size_t kv_stride, size_t count,
                    const int32_t *pos, const float *k, const float *v)
{
    ND_ENTER(ctx);
    if (int rc = check_geom(g)) return rc;
    if (count == 0) return ND_OK;
    ND_REQUIRE(kv && pos && k && v, "null buffer");
    ND_REQUIRE(count <= 0x7fffffff, "count too large");
    Geom kg = make_geom(g);
    kg.v_off = nd_kv_f32_v_offset(g);
    dim3 grid(unsigned(count), unsigned(g->num_kv_heads));
    hipLaunchKernelGGL(kv_write_f32_kernel, grid, dim3(64), 0, ctx->stream, kg,
                       static_cast<uint8_t *>(kv), kv_stride, pos, k, v);
    return nd::check_launch("kv_write_f32");
}

int nd_fake_quant(nd_ctx *ctx, float *x, size_t rows, size_t dim)
{
    ND_ENTER(ctx);
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
    ND_ENTER(ctx);
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
    ND_ENTER(ctx);
    if (int rc = check_geom(g)) return rc;
    if (count == 0) return ND_OK;
    ND_REQUIRE(kv && pos && k && v, "null buffer");
    ND_REQUIRE(count <= 0x7fffffff, "count too large");
    dim3 grid(unsigned(count), unsigned(g->num_kv_heads));
    hipLaunchKernelGGL(kv_write_kernel, grid, dim3(128), 0, ctx->stream, make_geom(g),
                       static_cast<uint8_t *>(kv), kv_stride, pos, k, v);
    return nd::check_launch("kv_write");
}

}  // extern "C"

namespace {

// nd_attend_step_i8 with its split-K partials either in the context's
// growable workspace (fixed == nullptr) or in `fixed`, `fixed_floats` long.
int attend_i8(nd_ctx *ctx, const nd_kv_geom *g, const void *kv, size_t kv_stride, size_t count,
              const int32_t *lo, const int32_t *hi, const float *q, float scale, int quant_query,
              float *out, float *fixed, size_t fixed_floats)
{
    ND_ENTER(ctx);
    if (int rc = check_geom(g)) return rc;
    if (count == 0) return ND_OK;
    ND_REQUIRE(kv && lo && hi && q && out, "null buffer");
    ND_REQUIRE(count <= 65535, "count %zu above 65535", count);
    ND_REQUIRE((reinterpret_cast<uintptr_t>(kv) & 255) == 0 && kv_stride % 256 == 0,
               "kv blocks must be 256-byte aligned");
    const int rep = g->num_heads / g->num_kv_heads;
    AttnFn fn = pick_attn(rep, g->qk_head_dim, g->v_head_dim);
    ND_REQUIRE(fn, "no attention kernel for repeat %d, qk %d, v %d", rep, g->qk_head_dim,
               g->v_head_dim);
    // Split each span across blocks only when (query, kv head) pairs cannot
    // give every CU a few blocks; the split partials merge in a second pass.
    const size_t pairs = count * size_t(g->num_kv_heads);
    const size_t want = size_t(ctx->num_cus > 0 ? ctx->num_cus : 256) * 4;
    // a split covers at least 512 positions (256 with more than two query
    // heads a kv head): with one query head, splits of one 256-position
    // chunk measured slower at one session (ctx 512: 13.1 against 10.6 us,
    // ctx 8192: 20.4 against 14.9), the merge costing more than they save
    const size_t span_min = rep <= 2 ? 512 : 256;
    const size_t max_splits = (size_t(g->cap) + span_min - 1) / span_min;
    size_t splits = pairs >= want ? 1 : (want + pairs - 1) / pairs;
    if (splits > max_splits) splits = max_splits;
    if (splits > 65535) splits = 65535;
    float *po = nullptr, *pml = nullptr;
    if (splits > 1) {
        void *wsp = nullptr;
        const size_t n_o = count * size_t(g->num_heads) * splits * g->v_head_dim;
        const size_t n_ml = count * size_t(g->num_heads) * splits * 2;
        if (fixed) {
            ND_REQUIRE(n_o + n_ml <= fixed_floats,
                       "split-K partials need %zu floats (%zu queries x %d heads x %zu splits x "
                       "(%d + 2)); the no-allocation scratch holds %zu",
                       n_o + n_ml, count, g->num_heads, splits, g->v_head_dim, fixed_floats);
            wsp = fixed;
        } else if (int rc = nd::workspace(ctx, (n_o + n_ml) * sizeof(float), &wsp)) {
            return rc;
        }
        po = static_cast<float *>(wsp);
        pml = po + n_o;
    }
    dim3 grid(unsigned(splits), unsigned(g->num_kv_heads), unsigned(count));
    fn(grid, ctx->stream, make_geom(g), static_cast<const uint8_t *>(kv), kv_stride, lo, hi, q,
       scale, quant_query, int(splits), out, po, pml);
    if (int rc = nd::check_launch("attn_i8")) return rc;
    if (splits > 1) {
        hipLaunchKernelGGL(attn_combine_kernel, dim3(unsigned(g->num_heads), unsigned(count)),
                           dim3(64), 0, ctx->stream, make_geom(g), int(splits), po, pml, out);
        return nd::check_launch("attn_combine");
    }
    return ND_OK;
}

}  // namespace

extern "C" {

int nd_attend_step_i8(nd_ctx *ctx, const nd_kv_geom *g, const void *kv, size_t kv_stride,
                      size_t count, const int32_t *lo, const int32_t *hi, const float *q,
                      float scale, int quant_query, float *out)
{
    return attend_i8(ctx, g, kv, kv_stride, count, lo, hi, q, scale, quant_query, out, nullptr, 0);
}

int nd_attend_step_i8_noalloc(nd_ctx *ctx, const nd_kv_geom *g, const void *kv, size_t kv_stride,
                              size_t count, const int32_t *lo, const int32_t *hi, const float *q,
                              float scale, int quant_query, float *out)
{
    if (!ctx) return nd::fail(ND_ERR_ARG, "null context");
    float *p = ctx->device >= 0 && ctx->device < kMaxDevices ? g_scratch[ctx->device] : nullptr;
    if (!p) return nd::fail(ND_ERR_HIP, "no-allocation scratch of device %d was not set up",
                            ctx->device);
    // Every partial the merge reads is written by the same call first, so
    // the array's previous contents never matter and nothing is cleared.
    return attend_i8(ctx, g, kv, kv_stride, count, lo, hi, q, scale, quant_query, out, p,
                     kNoAllocScratchFloats);
}

}  // extern "C"
