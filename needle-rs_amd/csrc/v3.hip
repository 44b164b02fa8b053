// Needle-3 forward on the device: the caller of the codebook projections and
// the int8 KV cache (crates/needle-core/src/v3/model.rs:150-375,
// decode_step), batched over sessions.
//
// The forward reproduces the reference's result bits.  Every projection is
// the reference-order Cactus-Quants matvec/matmul and the attention the
// reference-order attend_step (ref_order.hip); the int8 KV append is
// kv.hip's bit-exact quantiser.  The per-position glue is a handful of fused
// kernels, one workgroup per session:
//   mhc_in     mHC gate + mix down, Engram gate, ZCRMSNorm   (mhc.rs:80-103,
//              engram.rs:111-132, norm.rs:23-30)
//   qkv_post   causal conv step over q/k/v with the retained tails, then
//              ZCRMSNorm + RoPE on q and k                    (cache.rs:401-438,
//              attention.rs:108-150)
//   gate       attn *= sigmoid(gate)                          (model.rs:309-312)
//   post_attn  post-norm, gated residual, pre-MLP norm        (model.rs:313-321)
//   hada_mlp   HadamardMLP: low-rank conditioning, three Kronecker stages of
//              32x32 factors, permutations, silu; residual and block delta
//              (v3/kernels.rs:119-180)
//   mhc_out    post/res gates, 4x4 Sinkhorn, lane scatter    (mhc.rs:111-152)
//   engram     dilated value conv step with its tail         (cache.rs:445-482)
//   final      lane mean + final norm; argmax (first maximum wins)
// This file is built without FP contraction, so elementwise arithmetic
// rounds as rustc's (which never fuses a*b+c); every reduction the reference
// folds sequentially (norms, the Engram gate, the conditioning projection,
// lane sums) is one sequential chain on one thread, in the reference's
// index order; exp and log are libm's algorithms (nd_libm.h).
#include "nd_cq_internal.h"
#include "nd_fold.h"
#include "nd_internal.h"
#include "nd_kv_internal.h"
#include "nd_libm.h"
#include "nd_ref_order.h"
#include "nd_attn_exact.h"

#include <cmath>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

namespace {

constexpr int kT = 256;

__device__ inline float sigmoidf_(float x) { return nd_sigmoidf(x); }

// ((0 + p[0]) + p[1]) + ... + p[n-1]: a sequential fold, as the reference's
// loops and iterator sums, run by one thread over values already in LDS.
// Products are formed in parallel beforehand; a product rounds the same
// whether it is formed here or inside the fold.
// A workgroup barrier that orders LDS only: it does not wait for the
// global loads in flight (__syncthreads does), whose registers the compiler
// waits for at their first use.
__device__ inline void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Orders one wave's LDS writes before its own later LDS reads of other
// lanes' values (a wave's LDS operations execute in order; this keeps the
// compiler from moving them across).
__device__ inline void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

__device__ inline float chain_sum(const float *p, int n)
{
    __builtin_amdgcn_s_setprio(2);
    float s = 0.0f;
    if ((reinterpret_cast<uintptr_t>(p) & 15) == 0) {
        s = nd_lds_fold(0.0f, p, n);
    } else {
        for (int i = 0; i < n; ++i) s += p[i];
    }
    __builtin_amdgcn_s_setprio(0);
    return s;
}

// CqWeight::prepare_input's normalised FWHT (hadamard.rs:24-55) over the
// n / group groups of buf (LDS), in place: the butterfly pairs of a stage
// are disjoint, so evaluating them in parallel gives the sequential loop's
// bits; then x * (1 / sqrtf(group)).  Every thread of the block calls it,
// after buf is written and synchronised.
__device__ inline void fwht_groups_lds(float *buf, int n, int group, float inv)
{
    const int half = group / 2, pairs = n / 2;
    for (int h = 1; h < group; h <<= 1) {
        for (int e = threadIdx.x; e < pairs; e += blockDim.x) {
            const int g = e / half, i = e - g * half;
            const int jj = g * group + (i / h) * (2 * h) + (i % h);
            const float a = buf[jj], c = buf[jj + h];
            buf[jj] = a + c;
            buf[jj + h] = a - c;
        }
        __syncthreads();
    }
    for (int e = threadIdx.x; e < n; e += blockDim.x) buf[e] *= inv;
    __syncthreads();
}

// The same transform for one 128-wide group held by one wave: element e
// sits in lane e % 64, slot e / 64.  Stage h pairs lanes l and l ^ h (h <
// 64) or the two slots (h = 64); the lane with bit h clear forms a + b, the
// other a - b, exactly the butterfly's two results.  No block barrier.
__device__ inline void fwht128_wave(float &x0, float &x1, float inv)
{
    x0 = ndl::wave_fwht64(x0);
    x1 = ndl::wave_fwht64(x1);
    const float a = x0, b = x1;
    x0 = (a + b) * inv;
    x1 = (a - b) * inv;
}

// Butterfly stage H of fwht128_wave on NG groups' register pairs.
template <int H, int NG>
__device__ inline void fwht_stage_n(float (&x0)[NG], float (&x1)[NG])
{
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        x0[q] = ndl::wave_butterfly<H>(x0[q]);
        x1[q] = ndl::wave_butterfly<H>(x1[q]);
    }
}

// fwht128_wave over NG groups at once (one pair of registers per group),
// each stage applied to every group before the next, so the lane moves of
// different groups overlap; the same operations as fwht128_wave per group.
template <int NG>
__device__ inline void fwht128_wave_n(float (&x0)[NG], float (&x1)[NG], float inv)
{
    fwht_stage_n<1>(x0, x1);
    fwht_stage_n<2>(x0, x1);
    fwht_stage_n<4>(x0, x1);
    fwht_stage_n<8>(x0, x1);
    fwht_stage_n<16>(x0, x1);
    fwht_stage_n<32>(x0, x1);
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        const float a = x0[q], b = x1[q];
        x0[q] = (a + b) * inv;
        x1[q] = (a - b) * inv;
    }
}

// prepare_input of `buf` (LDS, pp.in_padded floats, written and synchronised)
// into `out` (global, and back into buf when `keep`): one wave per 128-group
// when the group is 128, else the block-wide butterfly.  Every thread of the
// block calls it; it ends synchronised.
__device__ inline void prepare_lds(float *buf, float *out, int in_padded, int group, float inv,
                                   bool keep)
{
    if (group == 128) {
        const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
        for (int g = wave; g < in_padded / 128; g += nw) {
            float x0 = buf[g * 128 + lane], x1 = buf[g * 128 + 64 + lane];
            fwht128_wave(x0, x1, inv);
            out[g * 128 + lane] = x0;
            out[g * 128 + 64 + lane] = x1;
            if (keep) {
                buf[g * 128 + lane] = x0;
                buf[g * 128 + 64 + lane] = x1;
            }
        }
        __syncthreads();
        return;
    }
    fwht_groups_lds(buf, in_padded, group, inv);
    for (int e = threadIdx.x; e < in_padded; e += blockDim.x) out[e] = buf[e];
    __syncthreads();
}

// Geometry of a prepared input: in_padded floats in groups of `group`.
struct Prep {
    int in_padded, group;
    float inv;  // 1 / sqrtf(group)
};

// ---- embedding broadcast: lanes[b][l][c] = emb[b][c] * scale ---------------
__global__ void k_embed(const float *__restrict__ emb, float *__restrict__ lanes, float scale,
                        int n, int d)
{
    const size_t b = blockIdx.y;
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < d; c += gridDim.x * blockDim.x) {
        const float e = emb[b * d + c] * scale;
        for (int l = 0; l < n; ++l) lanes[(b * n + l) * d + c] = e;
    }
}

// mhc.rs:111-152, scatter up: lanes[i] = sum_j H_res[i][j] lanes[j] +
// H_post[i] y, for one channel c (j ascending), into `ln` (LDS) and the
// global lanes.
__device__ inline void scatter_up(float *lg, float *ln, const float *gp, const float *gr,
                                  const float *y, int n, int d)
{
    for (int c = threadIdx.x; c < d; c += blockDim.x) {
        float old[16];
        for (int j = 0; j < n; ++j) old[j] = lg[size_t(j) * d + c];
        const float yc = y[c];
        for (int i = 0; i < n; ++i) {
            float acc = 0.0f;
            for (int j = 0; j < n; ++j) acc += gr[i * n + j] * old[j];
            const float v = acc + gp[i] * yc;
            lg[size_t(i) * d + c] = v;
            ln[i * d + c] = v;
        }
    }
}

// ---- Engram value conv step (cache.rs:445-482), every site at once ----------
// (blockIdx.z: the site; its values at ev + z * site_stride)
constexpr int kMaxSitesLaunch = 8;
struct EngramConv {
    float *ev;
    size_t site_stride;
    const float *taps[kMaxSitesLaunch];
    float *tail[kMaxSitesLaunch];
};

__global__ void k_engram_conv(EngramConv a, const int32_t *__restrict__ pos, int taps_n, int dil,
                              int max_order, int reach, int d)
{
    const size_t b = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= d) return;
    float *__restrict__ ev = a.ev + blockIdx.z * a.site_stride;
    const float *__restrict__ taps = a.taps[blockIdx.z];
    const int p = pos[b];
    float *tb = a.tail[blockIdx.z] + b * size_t(reach) * d;
    const float raw = ev[b * d + c];
    float acc = 0.0f;
    for (int j = 0; j < taps_n; ++j) {
        const int back = j * dil;
        if (back > p || p < j * max_order) continue;
        const float val = j == 0 ? raw : tb[size_t(reach - back) * d + c];
        acc += taps[j * d + c] * val;
    }
    for (int r = 0; r + 1 < reach; ++r) tb[size_t(r) * d + c] = tb[size_t(r + 1) * d + c];
    if (reach > 0) tb[size_t(reach - 1) * d + c] = raw;
    ev[b * d + c] = acc;
}

// k_engram_conv for a step of C consecutive positions per session: the raw
// values of the step's rows in `raw` ([R][d], unchanged), the conv into
// `out`, the tails as they stood before the step (updated after by
// k_tails).
__global__ void k_engram_conv_rows(const float *__restrict__ raw, float *__restrict__ out,
                                   const float *__restrict__ taps, const float *__restrict__ tail,
                                   const int32_t *__restrict__ pos, int taps_n, int dil,
                                   int max_order, int reach, int d, int C)
{
    const size_t b = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= d) return;
    const size_t sess = b / C;
    const int r = int(b % C);
    const int p = pos[b];
    const float *tb = tail + sess * size_t(reach) * d;
    float acc = 0.0f;
    for (int j = 0; j < taps_n; ++j) {
        const int back = j * dil;
        if (back > p || p < j * max_order) continue;
        const float val = back <= r ? raw[(b - back) * d + c] : tb[size_t(reach - (back - r)) * d + c];
        acc += taps[j * d + c] * val;
    }
    out[b * d + c] = acc;
}

// ---- Engram fetch, every site at once (engram.rs:67-104, model.rs:162-191):
// one wave per (site, row, table) takes the hashed table row through
// dequantize_row (cq.rs:763-779: level * norm, then the normalised FWHT of
// its one 128-wide group) and then through the key projection's
// prepare_input (hadamard.rs:24-55: the FWHT of that same group of the
// concatenated input), into the site's prepared key input.  A masked row
// (an n-gram with too little history) is zeros throughout.
struct EngramFetch {
    const uint8_t *packed[kMaxSitesLaunch];
    const float *norms[kMaxSitesLaunch];
    const float *lv[kMaxSitesLaunch];
    float *fh[kMaxSitesLaunch];  // [B][nt * 128] per site
    const int32_t *rows;         // [B][nt] table rows, -1 masked
    int out_feat, row_bytes, w, ternary, count, sites;  // count = B * nt
    float inv_t, inv_k;
};

__device__ inline uint32_t fetch_code(const uint8_t *row, int k, int w, int row_bytes)
{
    const int bit = k * w, byte = bit >> 3, shift = bit & 7;
    const uint32_t lo = row[byte];
    const uint32_t hi = (shift + w > 8 && byte + 1 < row_bytes) ? row[byte + 1] : 0u;
    return ((lo | (hi << 8)) >> shift) & ((1u << w) - 1u);
}

__global__ __launch_bounds__(256) void k_engram_fetch(EngramFetch a)
{
    const int wave = int(blockIdx.x) * 4 + int(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (wave >= a.sites * a.count) return;  // the whole wave leaves
    const int s = wave / a.count, i = wave - s * a.count;
    int o = a.rows[i];
    float x0 = 0.0f, x1 = 0.0f;
    if (o >= 0) {
        o = o >= a.out_feat ? a.out_feat - 1 : o;
        const uint8_t *row = a.packed[s] + size_t(o) * a.row_bytes;
        const float norm = a.norms[s][o];
        const uint32_t c0 = fetch_code(row, lane, a.w, a.row_bytes);
        const uint32_t c1 = fetch_code(row, 64 + lane, a.w, a.row_bytes);
        const float *lv = a.lv[s];
        x0 = lv[a.ternary ? (c0 == 3 ? 0 : (c0 == 1 ? 2 : 1)) : int(c0)] * norm;
        x1 = lv[a.ternary ? (c1 == 3 ? 0 : (c1 == 1 ? 2 : 1)) : int(c1)] * norm;
        fwht128_wave(x0, x1, a.inv_t);
        fwht128_wave(x0, x1, a.inv_k);
    }
    float *dst = a.fh[s] + size_t(i) * 128;
    dst[lane] = x0;
    dst[64 + lane] = x1;
}

// ---- layer input: the previous layer's scatter up, then this layer's mix
// down (mhc.rs:80-103): rms_unit of the lanes, prepare_input, the phi_pre
// rows, the gated lane sum, the Engram gate and ZCRMSNorm, prepared for the
// q/k/v/gate projections.  One workgroup per session.
constexpr int kMaxLanesD = 4096;  // mhc_lanes * d_model
constexpr int kFoldC256 = 12;     // terms a thread of the parallel rms fold at 256 threads (4 lanes x 768)
constexpr int kMaxPhiPairs = 768; // (phi rows of a layer) * (phi input groups)
// k_layer_in's workgroup: one per session, so at most a few dozen run at
// once; 8 waves give its parallel phases (the lane update, the phi dots,
// the prepares) two waves per SIMD and half the work per thread, the
// sequential chains being unchanged (16 waves spilled registers)
constexpr int kLayerInThreads = 512;
constexpr int kPadGroup = 132;    // a 128-group's stride in LDS, padded

struct LayerIn {
    float *lanes;             // [B][n][d]
    const float *y;           // [B][d]     previous layer's block delta   (update)
    const float *gp, *gr;     // [B][n], [B][n*n] previous layer's gates (update)
    int update;
    float *nxh;               // [B][pnx.in_padded] prepared rms_unit(lanes)
    Prep pnx;
    const uint8_t *phi_packed;  // phi_pre
    const float *phi_norms, *phi_lv;
    size_t phi_row_bytes;
    int phi_G, phi_row0, phi_ternary;
    const float *b_pre;       // [n] this layer's slice
    float a_pre;
    int layer, n, d;
    // with `gates`, this layer's phi_post and phi_res rows too (the raw
    // scatter-up gates, into graw [B][n + n*n]): same width, group and input
    int gates;
    const uint8_t *post_packed, *res_packed;
    const float *post_norms, *res_norms, *post_lv, *res_lv;
    size_t post_row_bytes, res_row_bytes;
    int post_row0, res_row0, post_ternary, res_ternary;
    float *graw;
    const float *ek, *ev;     // [B][d] this layer's Engram site, or null
    const float *norm_in;     // [d]
    float *u, *bx;            // [B][d]
    float *hh;                // [B][ph.in_padded]
    Prep ph;
};

template <int PP, int NTH>
__global__ __launch_bounds__(NTH) void k_layer_in(LayerIn a)
{
    constexpr int kCh = 1024 / NTH;  // model-dim channels per thread
    // phi (row, group) pairs a thread holds codes for; terms a thread of the
    // parallel rms fold
    constexpr int kPhiPerThread = (kMaxPhiPairs + NTH - 1) / NTH;
    constexpr int kFoldC = NTH >= 512 ? kMaxLanesD / NTH : kFoldC256;
    __shared__ __align__(16) float ln[kMaxLanesD], nb[kMaxLanesD];
    __shared__ __align__(16) float us[1024], bxs[1024], pa[1024], pb[1024], pc[1024];
    __shared__ float gs[kMaxPhiPairs], pn[kMaxPhiPairs], lvl[48], hp[16], gpp[16], grr[256], tot[4];
    __shared__ NdFoldLds<NTH> fl;
    const size_t b = blockIdx.x;
    const int tid = threadIdx.x, n = a.n, d = a.d, nd = n * d;
    // phi rows: phi_pre's n, then (gates) phi_post's n and phi_res's n * n
    const int G = a.phi_G, prows = a.gates ? 2 * n + n * n : n, pairs = prows * G;
    float *lg = a.lanes + b * size_t(nd);
    const float *ek = a.ek ? a.ek + b * d : nullptr;
    // the previous layer's lanes and block delta for this thread's channels
    constexpr int kUpLanes = 4;
    const bool up_regs = a.update && n <= kUpLanes;
    // every lane loads (indices clamped, values past the ends unused), so
    // no lane waits inside a branch of its own before the rest are issued
    float old[kCh][kUpLanes], yv[kCh], gpv = 0.0f, grv = 0.0f;
    if (a.update) {
        gpv = a.gp[b * n + (tid < n ? tid : 0)];
        grv = a.gr[b * n * n + (tid < n * n ? tid : 0)];
    }
#pragma unroll
    for (int k = 0; k < kCh; ++k) {
        const int c = tid + k * NTH, cc = c < d ? c : 0;
        yv[k] = up_regs ? a.y[b * d + cc] : 0.0f;
#pragma unroll
        for (int j = 0; j < kUpLanes; ++j) old[k][j] = up_regs && j < n ? lg[size_t(j) * d + cc] : 0.0f;
    }
    if (a.update) {
        if (tid < n) gpp[tid] = gpv;
        if (tid < n * n) grr[tid] = grv;
        lds_barrier();
        if (up_regs) {
            // mhc.rs:140-151 from the preloaded values
#pragma unroll
            for (int k = 0; k < kCh; ++k) {
                const int c = tid + k * NTH;
                if (c >= d) continue;
#pragma unroll
                for (int i = 0; i < kUpLanes; ++i) {
                    if (i >= n) break;
                    float acc = 0.0f;
#pragma unroll
                    for (int j = 0; j < kUpLanes; ++j)
                        if (j < n) acc += grr[i * n + j] * old[k][j];
                    const float v = acc + gpp[i] * yv[k];
                    lg[size_t(i) * d + c] = v;
                    ln[i * d + c] = v;
                }
            }
        } else {
            scatter_up(lg, ln, gpp, grr, a.y + b * d, n, d);
        }
    } else {
        for (int e = tid; e < nd; e += NTH) ln[e] = lg[e];
    }
    lds_barrier();
    // rms_unit (kernels.rs:33-41): products, then one chain
    for (int e = tid; e < nd; e += NTH) nb[e] = ln[e] * ln[e];
    lds_barrier();
    // operands needed after the chain, issued before lane 0 of wave 0 starts
    // folding: this thread's phi_pre group codes and norm, its channels'
    // norm_in / Engram key and value, the phi levels; values bound for LDS
    // are stored after the fold, so no wave waits on them first
    // pair t = (row t / G, group t % G); row r of phi_pre, phi_post or phi_res
    auto phi_row = [&](int r, const float *&norms, int &wsel) -> const uint8_t * {
        if (r < n) {
            norms = a.phi_norms + size_t(a.phi_row0 + r) * G;
            wsel = 0;
            return a.phi_packed + size_t(a.phi_row0 + r) * a.phi_row_bytes;
        }
        if (r < 2 * n) {
            norms = a.post_norms + size_t(a.post_row0 + r - n) * G;
            wsel = 1;
            return a.post_packed + size_t(a.post_row0 + r - n) * a.post_row_bytes;
        }
        norms = a.res_norms + size_t(a.res_row0 + r - 2 * n) * G;
        wsel = 2;
        return a.res_packed + size_t(a.res_row0 + r - 2 * n) * a.res_row_bytes;
    };
    CqGroupCodes<PP> codes[kPhiPerThread];
    float pnv[kPhiPerThread];
    int wsel[kPhiPerThread];
    // pairs past the first NTH (at most NTH / 4 of them): four threads a
    // pair, each two of its eight lane chains, so that no thread holds two
    // whole dots (the phase would last two dots for one wave)
    const int extra = pairs - NTH;
    const bool quarters = kPhiPerThread == 2 && extra > 0 && extra <= NTH / 4;
#pragma unroll
    for (int k = 0; k < kPhiPerThread; ++k) {
        const int t = k == 1 && quarters ? NTH + (tid >> 2) : tid + k * NTH;
        const bool has = t < pairs;
        const int r = has ? t / G : 0, g = has ? t - (t / G) * G : 0;
        const float *nr;
        const uint8_t *row = phi_row(r, nr, wsel[k]);
        if (k == 0 || has) cq_group_codes128<PP>(row + size_t(g) * (128 / PP), codes[k]);
        pnv[k] = has ? nr[g] : 0.0f;
    }
    float nin[kCh], ekv[kCh], evv[kCh];
#pragma unroll
    for (int k = 0; k < kCh; ++k) {
        const int c = tid + k * NTH, cc = c < d ? c : 0;
        nin[k] = a.norm_in[cc];
        ekv[k] = ek ? ek[cc] : 0.0f;
        evv[k] = ek ? a.ev[b * d + cc] : 0.0f;
    }
    const float bpre = a.b_pre[tid < n ? tid : 0];
    float lvv = 0.0f;
    if (tid < 48) {
        const int k = tid & 15, w = tid >> 4;
        const float *lv = w == 0 ? a.phi_lv : (w == 1 ? a.post_lv : a.res_lv);
        const int tern = w == 0 ? a.phi_ternary : (w == 1 ? a.post_ternary : a.res_ternary);
        if (w == 0 || a.gates) lvv = lv[tern ? (k == 3 ? 0 : (k == 1 ? 2 : 1)) : k];
    }
    // the rms sum of squares: the workgroup folds it in parallel with the
    // chain's bits (nd_fold.h) when it fits kFoldC terms a thread
    if (nd >= kNdFoldMinN && nd <= NTH * kFoldC) {
        const float f = nd_fold_nonneg<NTH, kFoldC>(nb, nd, fl);
        if (tid == 0) tot[0] = f;
    } else if (tid == 0) {
        tot[0] = chain_sum(nb, nd);
    }
#pragma unroll
    for (int k = 0; k < kPhiPerThread; ++k) {
        if (k == 1 && quarters) {
            if ((tid & 3) == 0 && NTH + (tid >> 2) < pairs) pn[NTH + (tid >> 2)] = pnv[k];
        } else if (tid + k * NTH < pairs) {
            pn[tid + k * NTH] = pnv[k];
        }
    }
    if (tid < 48) lvl[tid] = lvv;
    lds_barrier();
    {
        // prepare_input of rms_unit(lanes): one wave per 128-group straight
        // from the lanes; the result goes to global nxh and, each group
        // padded by 4 floats (so a wave's reads of different groups fall in
        // different banks), to nb for the phi_pre dots
        const float inv = 1.0f / sqrtf(tot[0] / float(nd) + 1e-6f);
        const int wave = tid >> 6, lane = tid & 63;
        float *xo = a.nxh + b * a.pnx.in_padded;
        // three groups a wave at a time, their lane moves overlapped
        constexpr int NG = 3;
        for (int g0 = wave; g0 < G; g0 += NG * (NTH / 64)) {
            float x0[NG], x1[NG];
#pragma unroll
            for (int q = 0; q < NG; ++q) {
                const int e0 = (g0 + q * (NTH / 64)) * 128 + lane, e1 = e0 + 64;
                x0[q] = e0 < nd ? ln[e0] * inv : 0.0f;
                x1[q] = e1 < nd ? ln[e1] * inv : 0.0f;
            }
            fwht128_wave_n<NG>(x0, x1, a.pnx.inv);
#pragma unroll
            for (int q = 0; q < NG; ++q) {
                const int g = g0 + q * (NTH / 64);
                if (g >= G) break;
                xo[g * 128 + lane] = x0[q];
                xo[g * 128 + 64 + lane] = x1[q];
                nb[g * kPadGroup + lane] = x0[q];
                nb[g * kPadGroup + 64 + lane] = x1[q];
            }
        }
    }
    lds_barrier();
    // this layer's phi rows (matvec_rows_prepared, reference order)
#pragma unroll
    for (int k = 0; k < kPhiPerThread; ++k) {
        if (k == 1 && quarters) {
            const int t = NTH + (tid >> 2), q = tid & 3;
            if (t < pairs) {
                float l0, l1;
                cq_group_quarter128<PP>(codes[k], lvl + 16 * wsel[k], nb + (t % G) * kPadGroup, q, l0, l1);
                // the pair's eight lane chains summed 0..7, as
                // cq_group_dot128 ends, from the quad's registers
                float acc = 0.0f;
                acc += ndl::quad_lane<0>(l0);
                acc += ndl::quad_lane<0>(l1);
                acc += ndl::quad_lane<1>(l0);
                acc += ndl::quad_lane<1>(l1);
                acc += ndl::quad_lane<2>(l0);
                acc += ndl::quad_lane<2>(l1);
                acc += ndl::quad_lane<3>(l0);
                acc += ndl::quad_lane<3>(l1);
                if (q == 0) gs[t] = acc;
            }
            continue;
        }
        const int t = tid + k * NTH;
        if (t < pairs) gs[t] = cq_group_dot128<PP>(codes[k], lvl + 16 * wsel[k], nb + (t % G) * kPadGroup);
    }
    lds_barrier();
    if (tid < prows) {
        float total = 0.0f;
        for (int g = 0; g < G; ++g) total += pn[tid * G + g] * gs[tid * G + g];
        if (tid < n) {
            const float off = tid == a.layer % n ? 4.0f : -4.0f;
            hp[tid] = sigmoidf_(a.a_pre * total + bpre + off);
        } else {
            a.graw[b * (prows - n) + (tid - n)] = total;  // nx . phi_post, nx . phi_res
        }
    }
    lds_barrier();
    // gated lane sum, Engram gate (engram.rs:111-132), ZCRMSNorm (norm.rs:23-30)
#pragma unroll
    for (int k = 0; k < kCh; ++k) {
        const int c = tid + k * NTH;
        if (c >= d) continue;
        float acc = 0.0f;
        for (int l = 0; l < n; ++l) acc += hp[l] * ln[l * d + c];
        us[c] = acc;
        a.u[b * d + c] = acc;
        if (ek) {
            pa[c] = acc * acc;
            pb[c] = ekv[k] * ekv[k];
            pc[c] = acc * ekv[k];
        }
    }
    lds_barrier();
    if (ek) {
        // three sequential sums, side by side on lanes 0-2
        if (tid < 3) tot[1 + tid] = chain_sum(tid == 0 ? pa : (tid == 1 ? pb : pc), d);
        lds_barrier();
        const float ux = 1.0f / sqrtf(tot[1] / float(d) + 1e-6f);
        const float uk = 1.0f / sqrtf(tot[2] / float(d) + 1e-6f);
        const float alpha = sigmoidf_(tot[3] * ux * uk / sqrtf(float(d)));
#pragma unroll
        for (int k = 0; k < kCh; ++k) {
            const int c = tid + k * NTH;
            if (c >= d) continue;
            const float v = us[c] + alpha * evv[k];
            bxs[c] = v;
            pa[c] = v * v;
        }
    } else {
        for (int c = tid; c < d; c += NTH) {
            bxs[c] = us[c];
            pa[c] = us[c] * us[c];
        }
    }
    lds_barrier();
    if (tid == 0) tot[0] = chain_sum(pa, d);
    lds_barrier();
    const float inv = 1.0f / sqrtf(tot[0] / float(d) + 1e-6f);
#pragma unroll
    for (int k = 0; k < kCh; ++k) {
        const int c = tid + k * NTH;
        if (c < d) {
            a.bx[b * d + c] = bxs[c];
            pa[c] = (1.0f + nin[k]) * bxs[c] * inv;
        }
    }
    for (int c = d + tid; c < a.ph.in_padded; c += NTH) pa[c] = 0.0f;
    lds_barrier();
    prepare_lds(pa, a.hh + b * a.ph.in_padded, a.ph.in_padded, a.ph.group, a.ph.inv, false);
}

// ---- the scatter-up gates of a layer (mhc.rs:111-152), on the side stream:
// H_post = 2 sigmoid(a_post . raw + b_post + off), H_res = Sinkhorn(a_res .
// raw + b_res).  They depend only on the layer's input lanes.
struct MhcGates {
    const float *hpost_raw;    // [B][n]
    const float *hres_raw;     // [B][n*n]
    const float *b_post;       // [n]
    const float *b_res;        // [n*n]
    float a_post, a_res;
    int layer, n;
    float *gp, *gr;            // [B][n], [B][n*n]
};

__device__ inline float lse_row(const float *x, int n)
{
    float mx = -INFINITY;
    for (int i = 0; i < n; ++i) mx = fmaxf(mx, x[i]);
    if (!(mx == mx) || mx == INFINITY || mx == -INFINITY) return mx;
    float s = 0.0f;
    for (int i = 0; i < n; ++i) s += nd_expf(x[i] - mx);
    return mx + nd_logf(s);
}

// kernels.rs:48-74 on an n x n matrix (n * n <= 64) held one entry per lane
// of one wave: every row (then column) logsumexp is the reference's loop --
// max, sequential sum of exps, max + log.  Each lane exponentiates its own
// entry; the lanes of a row (column) then fold the row's exps in index
// order from shuffles, all rows at once (any n; the decode step's split
// gate phases use the DPP form below for n = 4).
__device__ inline float sinkhorn_wave(float m, int n)
{
    const int lane = threadIdx.x & 63;
    const int i = lane / n, j = lane - (lane / n) * n;
    const int rb = i * n;  // first lane of this row
    for (int it = 0; it < 20; ++it) {
        {
            float mx = -INFINITY;
            for (int k = 0; k < n; ++k) mx = fmaxf(mx, __shfl(m, rb + k, 64));
            const float e = nd_expf(m - mx);
            float s = 0.0f;
            for (int k = 0; k < n; ++k) s += __shfl(e, rb + k, 64);
            const bool finite = mx == mx && mx != INFINITY && mx != -INFINITY;
            m -= finite ? mx + nd_logf(s) : mx;
        }
        {
            float mx = -INFINITY;
            for (int k = 0; k < n; ++k) mx = fmaxf(mx, __shfl(m, k * n + j, 64));
            const float e = nd_expf(m - mx);
            float s = 0.0f;
            for (int k = 0; k < n; ++k) s += __shfl(e, k * n + j, 64);
            m -= mx + nd_logf(s);
        }
    }
    return nd_expf(m);
}

// One iteration of sinkhorn_wave (rows, then columns).
__device__ inline float sinkhorn_iter_wave(float m, int n)
{
    const int lane = threadIdx.x & 63;
    const int i = lane / n, j = lane - (lane / n) * n;
    const int rb = i * n;
    {
        float mx = -INFINITY;
        for (int k = 0; k < n; ++k) mx = fmaxf(mx, __shfl(m, rb + k, 64));
        const float e = nd_expf(m - mx);
        float s = 0.0f;
        for (int k = 0; k < n; ++k) s += __shfl(e, rb + k, 64);
        const bool finite = mx == mx && mx != INFINITY && mx != -INFINITY;
        m -= finite ? mx + nd_logf(s) : mx;
    }
    {
        float mx = -INFINITY;
        for (int k = 0; k < n; ++k) mx = fmaxf(mx, __shfl(m, k * n + j, 64));
        const float e = nd_expf(m - mx);
        float s = 0.0f;
        for (int k = 0; k < n; ++k) s += __shfl(e, k * n + j, 64);
        m -= mx + nd_logf(s);
    }
    return m;
}

__global__ __launch_bounds__(64) void k_mhc_gates(MhcGates a)
{
    __shared__ float hr[256];
    const size_t b = blockIdx.x;
    const int n = a.n, tid = threadIdx.x;
    if (tid < n) {
        const float off = tid == a.layer % n ? 0.0f : -4.0f;
        a.gp[b * n + tid] = 2.0f * sigmoidf_(a.a_post * a.hpost_raw[b * n + tid] + a.b_post[tid] + off);
    }
    if (n * n <= 64) {
        const bool on = tid < n * n;
        float m = on ? a.a_res * a.hres_raw[b * n * n + tid] + a.b_res[tid] : 0.0f;
        m = sinkhorn_wave(m, n);
        if (on) a.gr[b * n * n + tid] = m;
        return;
    }
    if (tid == 0) {
        for (int x = 0; x < n * n; ++x) hr[x] = a.a_res * a.hres_raw[b * n * n + x] + a.b_res[x];
        for (int it = 0; it < 20; ++it) {
            for (int i = 0; i < n; ++i) {
                const float lse = lse_row(hr + i * n, n);
                for (int j = 0; j < n; ++j) hr[i * n + j] -= lse;
            }
            for (int j = 0; j < n; ++j) {
                float mx = -INFINITY;
                for (int i = 0; i < n; ++i) mx = fmaxf(mx, hr[i * n + j]);
                float s = 0.0f;
                for (int i = 0; i < n; ++i) s += nd_expf(hr[i * n + j] - mx);
                const float lse = mx + nd_logf(s);
                for (int i = 0; i < n; ++i) hr[i * n + j] -= lse;
            }
        }
        for (int x = 0; x < n * n; ++x) a.gr[b * n * n + x] = nd_expf(hr[x]);
    }
}

// The same Sinkhorn for n = 4 without a trip through LDS: lane 4i + j of
// lanes 0..15 holds m[i][j], so a row is a quad and its entries reach every
// lane of the quad by DPP quad broadcasts (in index order, as the loops
// read them).  The column pass runs as a row pass of the transpose, which
// DPP row shifts build: lane 4a + b takes lane 4b + a, 3(b - a) lanes away.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                  0xf, 0xf, false));
}

constexpr int quad_bcast(int k) { return k | (k << 2) | (k << 4) | (k << 6); }

// m minus the logsumexp of its quad's four entries (kernels.rs:76-85 for a
// row; with `row` false the column pass's form, which has no finite check)
__device__ __forceinline__ float lse_quad(float m, bool row)
{
    float mx = -INFINITY;
    mx = fmaxf(mx, dpp_f<quad_bcast(0)>(m));
    mx = fmaxf(mx, dpp_f<quad_bcast(1)>(m));
    mx = fmaxf(mx, dpp_f<quad_bcast(2)>(m));
    mx = fmaxf(mx, dpp_f<quad_bcast(3)>(m));
    const float e = nd_expf(m - mx);
    float s = 0.0f;
    s += dpp_f<quad_bcast(0)>(e);
    s += dpp_f<quad_bcast(1)>(e);
    s += dpp_f<quad_bcast(2)>(e);
    s += dpp_f<quad_bcast(3)>(e);
    const bool finite = mx == mx && mx != INFINITY && mx != -INFINITY;
    return m - (row && !finite ? mx : mx + nd_logf(s));
}

// lane 4a + b <- lane 4b + a within each 16-lane row (row_shl:n reads lane
// l + n, row_shr:n lane l - n)
__device__ __forceinline__ float transpose4x4(float m)
{
    const int l = threadIdx.x & 15, d = (l & 3) - (l >> 2);
    const float u3 = dpp_f<0x103>(m), u6 = dpp_f<0x106>(m), u9 = dpp_f<0x109>(m);
    const float d3 = dpp_f<0x113>(m), d6 = dpp_f<0x116>(m), d9 = dpp_f<0x119>(m);
    return d == 0 ? m : d == 1 ? u3 : d == 2 ? u6 : d == 3 ? u9 : d == -1 ? d3 : d == -2 ? d6 : d9;
}

// ---- the scatter-up gates inside the layer's own launches.  k_layer_in
// leaves the raw gates nx . phi_post and nx . phi_res in graw (its phi
// rows); phase 0, a second workgroup per row of k_qkv_kv's launch, forms
// H_post (mhc.rs:126-128) and runs the first `split` Sinkhorn iterations of
// H_res (mhc.rs:129-138, kernels.rs:46-74); phase 1, a second workgroup per
// row of k_post_hada's, runs the rest and the final exp.  The 16 Sinkhorn
// values pass between the phases through `state`.  So the gates need no
// stream of their own and lengthen no launch of the layer's chain.
constexpr int kSinkhornIters = 20;   // SINKHORN_ITERS (kernels.rs)
// iterations in phase 0: about 1.1 us each; 4 fit k_qkv_kv's time (3 to 5
// measured alike at 64 sessions, 6 slower) and the other 16 k_post_hada's.
// In the attention launch (k_attn_step), 6: 64 sessions 1.931 / 1.909 /
// 1.912 / 1.911 / 1.914 ms a step at 4 / 6 / 8 / 10 / 12, one session 1.245
// / 1.225 / 1.226 / 1.246 / 1.296 ms a token
constexpr int kGateSplit = 4;
constexpr int kGateSplitAttn = 6;
struct MhcIn {
    int on;                     // this launch runs a gate phase
    const float *graw;          // [B][n + n*n] from k_layer_in
    int n, layer, split;
    const float *b_post, *b_res;  // this layer's slices
    float a_post, a_res;
    float *gp, *gr;             // [B][n], [B][n*n]
    float *state;               // [B][64]: lane values of the Sinkhorn wave between phases
};

__device__ inline float sinkhorn_iters(float m, int n, int it0, int it1)
{
    for (int it = it0; it < it1; ++it) {
        if (n == 4) {
            m = lse_quad(m, true);
            m = transpose4x4(lse_quad(transpose4x4(m), false));
        } else {
            m = sinkhorn_iter_wave(m, n);
        }
    }
    return m;
}

// Phase 0: one wave's work (the block's other waves leave).
__device__ void mhc_gates_phase0(const MhcIn &a, size_t b)
{
    const int tid = threadIdx.x, n = a.n, rows = n + n * n;
    if (tid >= 64) return;
    const float *raw = a.graw + b * rows;
    if (tid < n) {
        const float off = tid == a.layer % n ? 0.0f : -4.0f;
        a.gp[b * n + tid] = 2.0f * sigmoidf_(a.a_post * raw[tid] + a.b_post[tid] + off);
    }
    float m = tid < n * n ? a.a_res * raw[n + tid] + a.b_res[tid] : 0.0f;
    a.state[b * 64 + tid] = sinkhorn_iters(m, n, 0, a.split);
}

// Phase 1: one wave's work (the block's other waves leave).
__device__ void mhc_gates_phase1(const MhcIn &a, size_t b)
{
    const int tid = threadIdx.x, n = a.n;
    if (tid >= 64) return;
    float m = a.state[b * 64 + tid];
    m = nd_expf(sinkhorn_iters(m, n, a.split, kSinkhornIters));
    if (tid < n * n) a.gr[b * n * n + tid] = m;
}

// ---- after the projections: causal conv step over q/k/v with the retained
// tails (cache.rs:401-438), ZCRMSNorm + RoPE on q and k
// (attention.rs:108-150), q to global, and k and v quantised straight into
// the session's int8 KV block at slot pos % cap (write_kv, cache.rs:346-379).
struct QkvKv {
    float *q;                               // [R][qd] in: projection, out: normed + roped
    const float *k, *v;                     // [R][kd], [R][vd] projections
    float *qt, *kt, *vt;                    // tails [B][taps-1][dim]
    const float *q_taps, *k_taps, *v_taps;  // [taps][dim]
    const float *q_norm, *k_norm;           // [hd]
    const float *rope;                      // [max_seq_len][2][hd/2]: cos then sin
    const int32_t *pos;                     // [R]
    int qd, kd, vd, taps, H, KVH, hd, VD;
    uint8_t *kv;                            // session s's block at kv + s * kv_stride
    size_t kv_stride, v_off, ks_off, vs_off;
    int cap;
    // Several consecutive positions per session (prefill): row r of the C
    // rows of a session is position pos[r]; earlier positions of the step
    // are read from the projection rows before it, older ones from the
    // tails, which this kernel does not change; the normed q goes to q_out.
    int C;
    float *q_out;
};

// cache.rs:401-438 for one channel: the conv output, with the tail shifted
// and the raw value retained.
__device__ inline float conv_one(float raw, float *tail, const float *taps, int dim, int c, int T,
                                 int p)
{
    float acc = taps[c] * raw;
    for (int j = 1; j < T; ++j) {
        if (j > p) break;
        acc += taps[j * dim + c] * tail[size_t(T - 1 - j) * dim + c];
    }
    for (int r = 0; r + 2 < T; ++r) tail[size_t(r) * dim + c] = tail[size_t(r + 1) * dim + c];
    if (T > 1) tail[size_t(T - 2) * dim + c] = raw;
    return acc;
}

// conv_one for row r (position p) of a step holding C consecutive positions
// of one session: the value j positions back comes from row r - j of `rows`
// (row stride `dim`) while it is in this step, else from the tail as it
// stood before the step (tail[T - 2] the position just before the step).
__device__ inline float conv_rows(const float *rows, const float *tail, const float *taps, int dim,
                                  int c, int T, int p, int r)
{
    float acc = taps[c] * rows[size_t(r) * dim + c];
    for (int j = 1; j < T; ++j) {
        if (j > p) break;
        const float prev = j <= r ? rows[size_t(r - j) * dim + c]
                                  : tail[size_t(T - 1 - (j - r)) * dim + c];
        acc += taps[j * dim + c] * prev;
    }
    return acc;
}

// After a step of C positions: each session's tail of the last `keep`
// values of `rows` (row stride `dim`, the session's C rows consecutive),
// older entries shifted in from the previous tail when C < keep.
__global__ void k_tails(const float *__restrict__ rows, float *__restrict__ tail, int keep, int C,
                        int dim)
{
    const size_t s = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= dim || keep <= 0) return;
    float *tb = tail + s * size_t(keep) * dim;
    const float *rb = rows + s * size_t(C) * dim;
    float old[16];
    for (int k = 0; k < keep && k < 16; ++k) old[k] = tb[size_t(k) * dim + c];
    for (int k = 0; k < keep && k < 16; ++k) {
        const int from_row = C - keep + k;  // row of the step, or an older position
        tb[size_t(k) * dim + c] = from_row >= 0 ? rb[size_t(from_row) * dim + c] : old[k + C];
    }
}

constexpr int kMaxQkDims = 2048;  // (num_heads + num_kv_heads) * qk_head_dim
// k_qkv_kv's workgroup, one per row: its conv, rope and quantise phases are
// element-wise over ~800 channels
constexpr int kQkvThreads = 512;
constexpr int kMaxVDims = 1024;   // num_kv_heads * v_head_dim

// KF: the session's cache is f32 (write_kv with KvPrecision::F32,
// cache.rs:359-362): k and v are stored as they are.
// With mhc.on (single positions), a second workgroup per row runs phase 0
// of the layer's scatter-up gates in the same launch.
template <bool CHUNK, bool KF, int NTH>
__global__ __launch_bounds__(NTH) void k_qkv_kv(QkvKv a, MhcIn mhc)
{
    __shared__ __align__(16) float qk[kMaxQkDims], sq[kMaxQkDims], vl[kMaxVDims];
    __shared__ float rms[64];
    if (blockIdx.y == 1) {
        mhc_gates_phase0(mhc, blockIdx.x);
        return;
    }
    const size_t b = blockIdx.x;
    const size_t sess = CHUNK ? b / a.C : b;
    const int r = CHUNK ? int(b % a.C) : 0;
    const int p = a.pos[b], T = a.taps, hd = a.hd, half = hd / 2;
    const int nq = a.qd + a.kd, heads = a.H + a.KVH;
    // One position a session with at most kTapRegs taps: every operand of
    // the thread's channels (projection, taps, tail) is loaded before the
    // first is used, then the conv runs from registers.  The loop below
    // waits for each tap's load in turn.
    constexpr int kChRegs = (kMaxQkDims + kMaxVDims + NTH - 1) / NTH, kTapRegs = 4;
    const int nc = nq + a.vd;
    // the RoPE operands of the thread's (head, pair) items, loaded up front
    // too (heads * hd <= kMaxQkDims)
    constexpr int kRopeRegs = (kMaxQkDims / 2 + NTH - 1) / NTH;
    const int ne = heads * half;
    const float *cs = a.rope + size_t(p) * 2 * half, *sn = cs + half;
    float rn1[kRopeRegs], rn2[kRopeRegs], rc[kRopeRegs], rs[kRopeRegs];
#pragma unroll
    for (int k = 0; k < kRopeRegs; ++k) {
        if (k * NTH >= ne) break;
        const int e0 = threadIdx.x + k * NTH, e = e0 < ne ? e0 : 0;
        const int hh = e / half, i = e - hh * half;
        const float *sc = hh < a.H ? a.q_norm : a.k_norm;
        rn1[k] = sc[i];
        rn2[k] = sc[half + i];
        rc[k] = cs[i];
        rs[k] = sn[i];
    }
    if (!CHUNK && T <= kTapRegs) {
        // this session's rows and tails (per-lane offsets below stay 32-bit)
        const size_t tr = size_t(T > 1 ? T - 1 : 0);
        const float *rq = a.q + b * a.qd, *rk = a.k + b * a.kd, *rv = a.v + b * a.vd;
        float *tq = a.qt + b * tr * a.qd, *tk = a.kt + b * tr * a.kd, *tw = a.vt + b * tr * a.vd;
        float raw[kChRegs], tp[kChRegs][kTapRegs], tv[kChRegs][kTapRegs];
#pragma unroll
        for (int k = 0; k < kChRegs; ++k) {
            if (k * NTH >= nc) break;
            const int c0 = threadIdx.x + k * NTH, c = c0 < nc ? c0 : 0;
            const int seg = c < a.qd ? 0 : (c < nq ? 1 : 2);
            const int dim = seg == 0 ? a.qd : (seg == 1 ? a.kd : a.vd);
            const int cl = seg == 0 ? c : (seg == 1 ? c - a.qd : c - nq);
            const float *src = seg == 0 ? rq : (seg == 1 ? rk : rv);
            const float *taps = seg == 0 ? a.q_taps : (seg == 1 ? a.k_taps : a.v_taps);
            const float *tail = seg == 0 ? tq : (seg == 1 ? tk : tw);
            raw[k] = src[cl];
#pragma unroll
            for (int j = 0; j < kTapRegs; ++j) {
                tp[k][j] = j < T ? taps[j * dim + cl] : 0.0f;
                // the value j positions back: tail row T - 1 - j
                tv[k][j] = j >= 1 && j < T ? tail[(T - 1 - j) * dim + cl] : 0.0f;
            }
        }
#pragma unroll
        for (int k = 0; k < kChRegs; ++k) {
            if (k * NTH >= nc) break;
            const int c = threadIdx.x + k * NTH;
            if (c >= nc) break;
            const int seg = c < a.qd ? 0 : (c < nq ? 1 : 2);
            const int dim = seg == 0 ? a.qd : (seg == 1 ? a.kd : a.vd);
            const int cl = seg == 0 ? c : (seg == 1 ? c - a.qd : c - nq);
            float v = raw[k];
            if (T > 0) {
                // conv_one's order: tap 0, then each tap back while j <= p
                float acc = tp[k][0] * v;
#pragma unroll
                for (int j = 1; j < kTapRegs; ++j)
                    if (j < T && j <= p) acc += tp[k][j] * tv[k][j];
                float *tail = seg == 0 ? tq : (seg == 1 ? tk : tw);
                // the tail shifts one position: row r takes row r + 1's value,
                // the value j = T - 2 - r positions back
#pragma unroll
                for (int j = 1; j + 1 < kTapRegs; ++j)
                    if (j + 2 <= T) tail[(T - 2 - j) * dim + cl] = tv[k][j];
                if (T > 1) tail[(T - 2) * dim + cl] = v;
                v = acc;
            }
            if (seg == 2) {
                vl[cl] = v;
            } else {
                qk[c] = v;
                sq[c] = v * v;
            }
        }
    }
    for (int c = threadIdx.x; c < nc && (CHUNK || T > kTapRegs); c += NTH) {
        if (c < a.qd) {
            float v = a.q[b * a.qd + c];
            if (T > 0) {
                const float *tl = a.qt + sess * size_t(T - 1) * a.qd;
                v = CHUNK ? conv_rows(a.q + (b - r) * a.qd, tl, a.q_taps, a.qd, c, T, p, r)
                          : conv_one(v, a.qt + b * size_t(T - 1) * a.qd, a.q_taps, a.qd, c, T, p);
            }
            qk[c] = v;
            sq[c] = v * v;
        } else if (c < nq) {
            float v = a.k[b * a.kd + c - a.qd];
            if (T > 0) {
                const float *tl = a.kt + sess * size_t(T - 1) * a.kd;
                v = CHUNK ? conv_rows(a.k + (b - r) * a.kd, tl, a.k_taps, a.kd, c - a.qd, T, p, r)
                          : conv_one(v, a.kt + b * size_t(T - 1) * a.kd, a.k_taps, a.kd, c - a.qd,
                                     T, p);
            }
            qk[c] = v;
            sq[c] = v * v;
        } else {
            float v = a.v[b * a.vd + c - nq];
            if (T > 0) {
                const float *tl = a.vt + sess * size_t(T - 1) * a.vd;
                v = CHUNK ? conv_rows(a.v + (b - r) * a.vd, tl, a.v_taps, a.vd, c - nq, T, p, r)
                          : conv_one(v, a.vt + b * size_t(T - 1) * a.vd, a.v_taps, a.vd, c - nq,
                                     T, p);
            }
            vl[c - nq] = v;
        }
    }
    lds_barrier();
    // one sequential sum of squares per head, the heads side by side
    if (threadIdx.x < heads)
        rms[threadIdx.x] = sqrtf(chain_sum(sq + threadIdx.x * hd, hd) / float(hd) + 1e-6f);
    lds_barrier();
#pragma unroll
    for (int k = 0; k < kRopeRegs; ++k) {
        const int e = threadIdx.x + k * NTH;
        if (e >= ne) break;
        const int hh = e / half, i = e - hh * half;
        const float *x = qk + hh * hd;
        const float r = rms[hh];
        const float x1 = (1.0f + rn1[k]) * x[i] / r;
        const float x2 = (1.0f + rn2[k]) * x[half + i] / r;
        const float c = rc[k], s = rs[k];
        const float o1 = x1 * c - x2 * s, o2 = x2 * c + x1 * s;
        if (hh < a.H) {
            float *o = (CHUNK ? a.q_out : a.q) + b * a.qd + hh * hd;
            o[i] = o1;
            o[half + i] = o2;
        } else {
            sq[hh * hd + i] = o1;  // the roped k, reusing the squares' space
            sq[hh * hd + half + i] = o2;
        }
    }
    lds_barrier();
    // quantise (cache.rs:80-104): one wave per kv head vector, K then V
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    uint8_t *blk = a.kv + sess * a.kv_stride;
    const int slot = p % a.cap;
    if constexpr (KF) {
        for (int vec = wave; vec < 2 * a.KVH; vec += NTH / 64) {
            const bool isv = vec >= a.KVH;
            const int h = isv ? vec - a.KVH : vec;
            const int dim = isv ? a.VD : hd;
            const float *src = isv ? vl + h * a.VD : sq + (a.H + h) * hd;
            float *dst = reinterpret_cast<float *>(blk + (isv ? a.v_off : 0)) + (size_t(h) * a.cap + slot) * dim;
            for (int e = lane; e < dim; e += 64) dst[e] = src[e];
        }
        return;
    }
    for (int vec = wave; vec < 2 * a.KVH; vec += NTH / 64) {
        const bool isv = vec >= a.KVH;
        const int h = isv ? vec - a.KVH : vec;
        const int dim = isv ? a.VD : hd;
        const float *src = isv ? vl + h * a.VD : sq + (a.H + h) * hd;
        int8_t *dst = reinterpret_cast<int8_t *>(blk + (isv ? a.v_off : 0)) + (size_t(h) * a.cap + slot) * dim;
        float *scl = reinterpret_cast<float *>(blk + (isv ? a.vs_off : a.ks_off)) + size_t(h) * a.cap + slot;
        float scale, inv;
        ndkv::quant_scale_wave(src, dim, scale, inv);
        for (int e = lane; e < dim; e += 64) dst[e] = int8_t(ndkv::quant_code(src[e], inv));
        if (lane == 0) *scl = scale;
    }
}

// ---- a decode step's attention launch with the q/k/v step folded in.
// Workgroup (session i, kv head kvh, query head h) of the exact attention
// first forms what k_qkv_kv would have left for it, with k_qkv_kv's
// arithmetic: the causal conv of its query head and of its kv head's k and
// v over the retained tails (cache.rs:401-438), ZCRMSNorm + RoPE on q and k
// (attention.rs:108-150), k and v quantised (cache.rs:80-104) and q
// fake-quantised (quant_rows, model.rs:289-293).  The kv head's first
// workgroup writes k and v to the ring slot; every workgroup reads the
// step's own row from LDS (the slot is not read back in the launch).  The
// tails shift afterwards, in k_post_hada.  With mhc.on, B more workgroups
// after the attention's run the scatter-up gates' phase 0.
struct AttnStep {
    QkvKv a;             // projections, taps, tails, norms, RoPE table, KV blocks
    ndkv::Geom g;
    const int32_t *lo, *hi;
    float scale;
    float *out;          // [B][H * 64] gated, half-transformed attention
    const float *gate;   // [B][H * 64]
    int groups;          // B * KVH
    int attn_blocks;     // 8 * R * ceil(groups / 8)
};

template <int QC>
__global__ __launch_bounds__(ndattn::kAttn2Threads, 4) void k_attn_step(AttnStep s, MhcIn mhc)
{
    using namespace ndattn;
    extern __shared__ __align__(16) float sm[];
    __shared__ AttnLds L;
    __shared__ AttnNewRow nr;
    __shared__ __align__(16) float xs[3][64], sqs[2][64];
    if (int(blockIdx.x) >= s.attn_blocks) {
        mhc_gates_phase0(mhc, blockIdx.x - s.attn_blocks);
        return;
    }
    const QkvKv &a = s.a;
    const ndkv::Geom &g = s.g;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int R = g.H / g.KVH;
    const int xcd = int(blockIdx.x) & 7, slot8 = int(blockIdx.x) >> 3;
    const int grp = (slot8 / R) * 8 + xcd;
    if (grp >= s.groups) return;  // padding block: the whole block leaves
    const int i = grp / g.KVH, kvh = grp - (grp / g.KVH) * g.KVH;
    const int h = kvh * R + slot8 % R;
    const int hd = a.hd, half = hd / 2, T = a.taps, p = a.pos[i];
    const int p0 = s.lo[i], hi = s.hi[i];
    // wave 0: the query head's channels, wave 1 the kv head's k, wave 2 its
    // v; lane = channel (lanes past the head read channel 0, unused).  Each
    // wave's part is its own: it syncs with itself only, then all meet once.
    const int seg = wave < 3 ? wave : 0;
    const int dim = seg == 0 ? a.qd : (seg == 1 ? a.kd : a.vd);
    const int width = seg == 2 ? a.VD : hd;
    const int c = (seg == 0 ? h * hd : (seg == 1 ? kvh * hd : kvh * a.VD)) + (lane < width ? lane : 0);
    const float *src = seg == 0 ? a.q : (seg == 1 ? a.k : a.v);
    const float *taps = seg == 0 ? a.q_taps : (seg == 1 ? a.k_taps : a.v_taps);
    const float *tail = seg == 0 ? a.qt : (seg == 1 ? a.kt : a.vt);
    const size_t tr = size_t(T > 1 ? T - 1 : 0);
    // every operand before the first use
    const float raw = src[size_t(i) * dim + c];
    float tp[4], tv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        tp[j] = j < T ? taps[j * dim + c] : 0.0f;
        tv[j] = j >= 1 && j < T ? tail[(size_t(i) * tr + (T - 1 - j)) * dim + c] : 0.0f;
    }
    const int li = lane < half ? lane : 0;
    const float *nrm = seg == 0 ? a.q_norm : a.k_norm;
    const float rn1 = nrm[li], rn2 = nrm[half + li];
    const float *cs = a.rope + size_t(p) * 2 * half;
    const float rc = cs[li], rsn = cs[half + li];
    uint8_t *blk = a.kv + size_t(i) * a.kv_stride;
    if (wave < 3) {
        // conv_one's order: tap 0, then each tap back while j <= p
        float v = raw;
        if (T > 0) {
            float acc = tp[0] * v;
#pragma unroll
            for (int j = 1; j < 4; ++j)
                if (j < T && j <= p) acc += tp[j] * tv[j];
            v = acc;
        }
        float *x = xs[seg];
        if (lane < width) {
            x[lane] = v;
            if (seg < 2) sqs[seg][lane] = v * v;
        }
        wave_lds_sync();
        if (seg < 2) {
            // ZCRMSNorm: the head's sequential sum of squares, then RoPE
            float r = 0.0f;
            if (lane == 0) r = sqrtf(chain_sum(sqs[seg], hd) / float(hd) + 1e-6f);
            r = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 0));
            if (lane < half) {
                const float x1 = (1.0f + rn1) * x[lane] / r;
                const float x2 = (1.0f + rn2) * x[half + lane] / r;
                x[lane] = x1 * rc - x2 * rsn;
                x[half + lane] = x2 * rc + x1 * rsn;
            }
            wave_lds_sync();
        }
        // quantise: the query (fake), k and v into LDS and, by the kv
        // head's first workgroup, into the ring slot
        const int slot = p % g.cap;
        const bool writer = slot8 % R == 0;
        float scl, inv;
        ndkv::quant_scale_wave(x, width, scl, inv);
        if (seg == 0) {
            for (int e = lane; e < hd; e += 64) L.qs[e] = ndkv::quant_code(x[e], inv) * scl;
        } else {
            int8_t *mine = reinterpret_cast<int8_t *>(seg == 1 ? nr.k : nr.v);
            int8_t *dst = reinterpret_cast<int8_t *>(blk + (seg == 2 ? g.v_off : 0)) +
                          (size_t(kvh) * g.cap + slot) * width;
            for (int e = lane; e < width; e += 64) {
                const int8_t code = int8_t(ndkv::quant_code(x[e], inv));
                mine[e] = code;
                if (writer) dst[e] = code;
            }
            if (lane == 0) {
                if (seg == 1) nr.ks = scl; else nr.vs = scl;
                if (writer)
                    *(reinterpret_cast<float *>(blk + (seg == 2 ? g.vs_off : g.ks_off)) +
                      size_t(kvh) * g.cap + slot) = scl;
            }
        }
    }
    __syncthreads();
    const int span = hi - p0 + 1;
    float *orow = s.out + (size_t(i) * g.H + h) * g.VD;
    // the span must end at the step's own position
    if (p0 < 0 || span < 1 || span > g.cap || hi != p) {
        for (int j = tid; j < g.VD; j += kAttn2Threads) orow[j] = NAN;
        return;
    }
    attn_exact2_run<1, QC, false, true>(g, blk, kvh, p0, span, s.scale, sm, L, &nr, orow,
                                        s.gate + (size_t(i) * g.H + h) * g.VD);
}

// attn *= sigmoid(gate) (model.rs:309-312), then prepare_input for out_proj.
constexpr int kMaxGatePad = 2048;

__global__ __launch_bounds__(kT) void k_gate_prep(const float *__restrict__ attn,
                                                 const float *__restrict__ gate,
                                                 float *__restrict__ ah, int od, Prep pp)
{
    __shared__ __align__(16) float buf[kMaxGatePad];
    const size_t b = blockIdx.x;
    for (int c = threadIdx.x; c < pp.in_padded; c += kT)
        buf[c] = c < od ? attn[b * od + c] * sigmoidf_(gate[b * od + c]) : 0.0f;
    __syncthreads();
    prepare_lds(buf, ah + b * pp.in_padded, pp.in_padded, pp.group, pp.inv, false);
}

// ---- post-norm, gated residual, pre-MLP norm (model.rs:313-321), then the
// HadamardMLP (v3/kernels.rs:119-180, hada_n = 1024 = 32 x 32), the
// residual and the block delta y = bx - u.  One 1024-thread workgroup per
// session; with the gates on (mhc.on), a second one per session computes
// the layer's scatter-up gates.
struct HadaArgs {
    const float *proj;  // [B][d] out_proj output
    const float *post_norm, *pre_hada;  // [d]
    float agate;
    const float *u;   // [B][d]
    float *bx, *y;    // [B][d]
    const float *d1, *d2, *b2, *d3, *d4;  // [1024]
    const float *w1a, *w1b, *w2a, *w2b, *w3a, *w3b;  // [32*32], stored transposed
    const float *cond_v;  // [d][rank]
    const float *cond_u;  // [rank][1024]
    const int32_t *p1, *p2perm;  // [1024]
    int d, rank;
    // Decode steps whose attention launch ran the q/k/v conv (k_attn_step):
    // the conv tails of q, k and v shift here, one channel of the q|k|v
    // concatenation per thread (at most 1024 channels, taps <= 4); the raw
    // projections are still in their buffers.  shift_taps <= 1: nothing to do.
    int shift_taps = 0;
    const float *sraw[3] = {};  // [B][dim] raw q, k, v
    float *stail[3] = {};       // [B][taps - 1][dim]
    int sdim[3] = {};
};

// out[k][l] = sum_j (sum_i z[i][l] a[i][k]) b[j][l], i and j ascending, each
// product rounded before its add and zero factors skipped, as kron_apply
// (v3/kernels.rs:41-81) does.  Thread (k, l) = (tid / 32, tid % 32) of 1024.
// z, a and b are held transposed at a padded row stride (zT[l*kKS + i] =
// z[i][l], aT[k*kKS + i] = a[i][k], bT[l*kKS + j] = b[j][l]) and t at the same
// stride, so every operand is read four terms at a time as a float4, from
// distinct banks; out is 32x32 row-major.  A pass whose skipping factor holds
// no zero at all (`a_zero` false for a; for t, found at the barrier between
// the passes) adds every product, which is the same sum.
constexpr int kKS = 36;

__device__ inline int kron_t(int e) { return (e & 31) * kKS + (e >> 5); }  // z[e / 32][e % 32]

__device__ inline void kron32(const float *zT, const float *aT, const float *bT, float *t, float *out,
                              bool a_zero)
{
    const int tid = threadIdx.x;
    const int k = tid >> 5, l = tid & 31;
    float acc = 0.0f;
#pragma unroll
    for (int i0 = 0; i0 < 32; i0 += 4) {
        const float4 av = *reinterpret_cast<const float4 *>(aT + k * kKS + i0);
        const float4 zv = *reinterpret_cast<const float4 *>(zT + l * kKS + i0);
        const float a4[4] = {av.x, av.y, av.z, av.w}, z4[4] = {zv.x, zv.y, zv.z, zv.w};
        if (a_zero) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float p = z4[u] * a4[u];
                acc = a4[u] == 0.0f ? acc : acc + p;
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) acc += z4[u] * a4[u];
        }
    }
    t[k * kKS + l] = acc;
    const bool t_zero = __syncthreads_or(acc == 0.0f);
    float o = 0.0f;
#pragma unroll
    for (int j0 = 0; j0 < 32; j0 += 4) {
        const float4 tv = *reinterpret_cast<const float4 *>(t + k * kKS + j0);
        const float4 bv = *reinterpret_cast<const float4 *>(bT + l * kKS + j0);
        const float t4[4] = {tv.x, tv.y, tv.z, tv.w}, b4[4] = {bv.x, bv.y, bv.z, bv.w};
        if (t_zero) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float p = t4[u] * b4[u];
                o = t4[u] == 0.0f ? o : o + p;
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) o += t4[u] * b4[u];
        }
    }
    out[k * 32 + l] = o;
    __syncthreads();
}

constexpr int kMaxCondRegs = 8;     // cond_v / cond_u values a thread preloads
constexpr int kCondProd = 6144;     // conditioning products held in LDS at once


__global__ __launch_bounds__(1024) void k_post_hada(HadaArgs a, MhcIn mhc)
{
    __shared__ __align__(16) float z[32 * kKS], buf[1024], t[32 * kKS], fa[32 * kKS], fb[32 * kKS], cond[1024];
    __shared__ __align__(16) float nbs[1024], prod[kCondProd];
    __shared__ float proj[64], tot[2];
    __shared__ unsigned zf;  // bit k: the a factor of Kronecker pass k holds a zero
    if (blockIdx.y == 1) {
        mhc_gates_phase1(mhc, blockIdx.x);
        return;
    }
    const size_t b = blockIdx.x;
    const int tid = threadIdx.x, d = a.d, r = a.rank;
    // what the first chain and the step after it need, up front
    // loads from a clamped channel (the values of threads past d are never
    // used): a load under a condition becomes a branch whose first use waits
    // for it at once
    const bool ch = tid < d;
    const int cc = ch ? tid : 0;
    const float pv = a.proj[b * d + cc];
    const float bxv = a.bx[b * d + cc];
    const float post_n = a.post_norm[cc];
    // post-norm of the projection, gated residual, pre-MLP norm: two chains
    buf[tid] = pv * pv;
    if (tid == 0) zf = 0;
    lds_barrier();
    if (tid == 0) tot[0] = chain_sum(buf, d);
    // every other operand, issued while lane 0 of wave 0 folds (its own
    // after the chain; nothing waits for them before the Kronecker passes)
    const float uv = a.u[b * d + cc];
    const float pre_n = a.pre_hada[cc];
    const float d1 = a.d1[tid], d2 = a.d2[tid], b2 = a.b2[tid], d3 = a.d3[tid], d4 = a.d4[tid];
    const float w1a = a.w1a[tid], w1b = a.w1b[tid], w2a = a.w2a[tid], w2b = a.w2b[tid];
    const float w3a = a.w3a[tid], w3b = a.w3b[tid];
    const int p1 = a.p1[tid], p2 = a.p2perm[tid];
    const bool regs = r <= kMaxCondRegs && r * d <= kCondProd;
    float cv[kMaxCondRegs], cu[kMaxCondRegs];
#pragma unroll
    for (int j = 0; j < kMaxCondRegs; ++j) {
        const bool on = regs && j < r;
        const float v = a.cond_v[on ? cc * r + j : 0], u = a.cond_u[on ? j * 1024 + tid : 0];
        cv[j] = on ? v : 0.0f;
        cu[j] = on ? u : 0.0f;
    }
    // the conv tails' shift: this thread's channel, its raw value and the
    // tail rows that move up, loaded now and stored after the norms
    const int nsh = a.shift_taps > 1 ? a.sdim[0] + a.sdim[1] + a.sdim[2] : 0;
    float shv[3] = {0.0f, 0.0f, 0.0f};
    float *shp = nullptr;
    int shd = 1;
    if (nsh > 0) {
        const int c = tid < nsh ? tid : 0;
        const int sg = c < a.sdim[0] ? 0 : (c < a.sdim[0] + a.sdim[1] ? 1 : 2);
        const int cl = sg == 0 ? c : (sg == 1 ? c - a.sdim[0] : c - a.sdim[0] - a.sdim[1]);
        shd = sg == 0 ? a.sdim[0] : (sg == 1 ? a.sdim[1] : a.sdim[2]);
        const float *rw = sg == 0 ? a.sraw[0] : (sg == 1 ? a.sraw[1] : a.sraw[2]);
        float *tl = sg == 0 ? a.stail[0] : (sg == 1 ? a.stail[1] : a.stail[2]);
        shp = tl + b * size_t(a.shift_taps - 1) * shd + cl;
        shv[0] = rw[b * shd + cl];
#pragma unroll
        for (int j = 1; j < 3; ++j) shv[j] = j + 1 < a.shift_taps ? shp[size_t(j) * shd] : 0.0f;
    }
    lds_barrier();
    if (ch) {
        const float inv = 1.0f / sqrtf(tot[0] / float(d) + 1e-6f);
        const float pn = (1.0f + post_n) * pv * inv;
        const float nb = bxv + a.agate * pn;
        nbs[tid] = nb;
        z[tid] = nb * nb;
    }
    lds_barrier();
    if (tid == 0) tot[1] = chain_sum(z, d);
    // tail row r takes row r + 1, the last row the raw value (conv_one)
    if (nsh > 0 && tid < nsh) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
            if (r + 2 < a.shift_taps) shp[size_t(r) * shd] = shv[r + 1];
        shp[size_t(a.shift_taps - 2) * shd] = shv[0];
    }
    lds_barrier();
    const float xv = ch ? (1.0f + pre_n) * nbs[tid] * (1.0f / sqrtf(tot[1] / float(d) + 1e-6f)) : 0.0f;
    // cond = 1 + softmax(x . cond_v) . cond_u.  Projection j is one chain
    // over the model dim, the r chains side by side on lanes 0..r-1 of wave
    // 0, over products formed in parallel (prod[j][i], contiguous per j).
    if (regs) {
        if (ch)
#pragma unroll
            for (int j = 0; j < kMaxCondRegs; ++j)
                if (j < r) prod[j * d + tid] = xv * cv[j];
        lds_barrier();
        if (tid < r) proj[tid] = chain_sum(prod + tid * d, d);
    } else {
        // wide rank: products a chunk of rows at a time
        buf[tid] = xv;
        lds_barrier();
        const int chn = kCondProd / r;
        float acc = 0.0f;
        for (int i0 = 0; i0 < d; i0 += chn) {
            const int ni = d - i0 < chn ? d - i0 : chn;
            for (int e = tid; e < ni * r; e += 1024) {
                const int ii = e / r, j = e - ii * r;
                prod[j * chn + ii] = buf[i0 + ii] * a.cond_v[(i0 + ii) * r + j];
            }
            lds_barrier();
            if (tid < r)
                for (int ii = 0; ii < ni; ++ii) acc += prod[tid * chn + ii];
            lds_barrier();
        }
        if (tid < r) proj[tid] = acc;
    }
    lds_barrier();
    if (tid < 64) {
        // softmax over the r projections: the max is order-free, each exp
        // on its own lane, the sum one chain in j order (every lane folds it)
        const float pj = tid < r ? proj[tid] : -INFINITY;
        float mx = pj;
        mx = ndl::wave_max64(mx);
        const float e = tid < r ? nd_expf(pj - mx) : 0.0f;
        float sum = 0.0f;
        for (int j = 0; j < r; ++j) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j));
        if (tid < r) proj[tid] = e / sum;
    }
    lds_barrier();
    {
        float c = 1.0f;
        if (regs) {
#pragma unroll
            for (int j = 0; j < kMaxCondRegs; ++j)
                if (j < r && proj[j] != 0.0f) c += proj[j] * cu[j];
        } else {
            for (int j = 0; j < r; ++j)
                if (proj[j] != 0.0f) c += proj[j] * a.cond_u[j * 1024 + tid];
        }
        cond[tid] = c;
    }
    {
        const unsigned zb = unsigned(w1a == 0.0f) | unsigned(w2a == 0.0f) << 1 | unsigned(w3a == 0.0f) << 2;
        if (zb) atomicOr(&zf, zb);
    }
    z[kron_t(tid)] = xv * d1;
    fa[(tid >> 5) * kKS + (tid & 31)] = w1a;  // w1a is stored transposed
    fb[(tid >> 5) * kKS + (tid & 31)] = w1b;  // w1b is stored transposed
    lds_barrier();
    kron32(z, fa, fb, t, buf, zf & 1u);
    z[kron_t(tid)] = buf[p1];
    fa[(tid >> 5) * kKS + (tid & 31)] = w2a;  // w2a is stored transposed
    fb[(tid >> 5) * kKS + (tid & 31)] = w2b;  // w2b is stored transposed
    lds_barrier();
    {
        const float zz = d2 * cond[tid] * z[kron_t(tid)] + b2;
        z[kron_t(tid)] = zz * sigmoidf_(zz);
    }
    lds_barrier();
    kron32(z, fa, fb, t, buf, zf & 2u);
    z[kron_t(tid)] = buf[p2] * d3;
    fa[(tid >> 5) * kKS + (tid & 31)] = w3a;  // w3a is stored transposed
    fb[(tid >> 5) * kKS + (tid & 31)] = w3b;  // w3b is stored transposed
    lds_barrier();
    kron32(z, fa, fb, t, buf, zf & 4u);
    if (ch) {
        const float o = buf[tid] * d4;
        const float nb = nbs[tid] + o;
        a.bx[b * d + tid] = nb;
        a.y[b * d + tid] = nb - uv;
    }
}

// ---- the last layer's scatter up, lane mean, final norm (model.rs:360-368),
// prepared for the tied LM head.
__global__ __launch_bounds__(kT) void k_final(float *__restrict__ lanes, const float *__restrict__ y,
                                             const float *__restrict__ gp, const float *__restrict__ gr,
                                             const float *__restrict__ final_norm,
                                             float *__restrict__ xh, int n, int d, Prep pp, int rstride)
{
    __shared__ __align__(16) float ln[kMaxLanesD], ms[1024], sq[1024];
    __shared__ float gpp[16], grr[256], tot;
    const size_t b = blockIdx.x;                       // output row: one per session
    const size_t rw = b * rstride + (rstride - 1);     // the session's last position
    if (threadIdx.x < n) gpp[threadIdx.x] = gp[rw * n + threadIdx.x];
    if (threadIdx.x < n * n) grr[threadIdx.x] = gr[rw * n * n + threadIdx.x];
    __syncthreads();
    scatter_up(lanes + rw * size_t(n) * d, ln, gpp, grr, y + rw * d, n, d);
    __syncthreads();
    for (int c = threadIdx.x; c < d; c += kT) {
        float acc = 0.0f;
        for (int l = 0; l < n; ++l) acc += ln[l * d + c];
        const float m = acc / float(n);
        ms[c] = m;
        sq[c] = m * m;
    }
    __syncthreads();
    if (threadIdx.x == 0) tot = chain_sum(sq, d);
    __syncthreads();
    const float inv = 1.0f / sqrtf(tot / float(d) + 1e-6f);
    for (int c = threadIdx.x; c < pp.in_padded; c += kT)
        sq[c] = c < d ? (1.0f + final_norm[c]) * ms[c] * inv : 0.0f;
    __syncthreads();
    prepare_lds(sq, xh + b * pp.in_padded, pp.in_padded, pp.group, pp.inv, false);
}

// ---- the device copies of the reference's libm wrappers (math.rs:3-46), one
// value a thread: expf, logf, and the sigmoid built on expf (ops.rs)
__global__ __launch_bounds__(256) void k_libm_map(int fn, const float *__restrict__ x, size_t n,
                                                  float *__restrict__ y)
{
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    y[i] = fn == 0 ? nd_expf(v) : (fn == 1 ? nd_logf(v) : nd_sigmoidf(v));
}

// ---- greedy argmax, first maximum wins (v3_engine.rs:410-420) -----------------
// Greedy token: the first index of the largest logit (v3_engine.rs:410-420:
// a strict `>` scan, so NaN never wins and a tie keeps the lower index).
// Each thread scans its indices in increasing order with all its loads in
// flight first; the partial (value, index) pairs then combine by "larger
// value, or equal value and lower index", which is the scan's own order.
__device__ inline void argmax_take(float &best, int &bi, float v, int i)
{
    if (v > best || (v == best && i < bi)) {
        best = v;
        bi = i;
    }
}

__global__ __launch_bounds__(kT) void k_argmax(const float *__restrict__ logits, int rows,
                                              int32_t *__restrict__ next, int32_t *__restrict__ also)
{
    __shared__ float sv[kT / 64];
    __shared__ int si[kT / 64];
    const size_t b = blockIdx.x;
    const float *row = logits + b * rows;
    float best = -INFINITY;
    int bi = 0;
    if ((rows & 3) == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0) {
        constexpr int U = 8;
        const float4 *r4 = reinterpret_cast<const float4 *>(row);
        const int n4 = rows / 4;
        for (int base = threadIdx.x; base < n4; base += kT * U) {
            float4 q[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i4 = base + u * kT;
                q[u] = r4[i4 < n4 ? i4 : n4 - 1];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i4 = base + u * kT;
                if (i4 < n4) {
                    if (q[u].x > best) { best = q[u].x; bi = 4 * i4; }
                    if (q[u].y > best) { best = q[u].y; bi = 4 * i4 + 1; }
                    if (q[u].z > best) { best = q[u].z; bi = 4 * i4 + 2; }
                    if (q[u].w > best) { best = q[u].w; bi = 4 * i4 + 3; }
                }
            }
        }
    } else {
        for (int i = threadIdx.x; i < rows; i += kT) {
            const float v = row[i];
            if (v > best) {
                best = v;
                bi = i;
            }
        }
    }
    argmax_take(best, bi, ndl::wave_xor<32>(best), ndl::wave_xor_int<32>(bi));
    argmax_take(best, bi, ndl::wave_xor<16>(best), ndl::wave_xor_int<16>(bi));
    argmax_take(best, bi, ndl::wave_xor<8>(best), ndl::wave_xor_int<8>(bi));
    argmax_take(best, bi, ndl::wave_xor<4>(best), ndl::wave_xor_int<4>(bi));
    argmax_take(best, bi, ndl::wave_xor<2>(best), ndl::wave_xor_int<2>(bi));
    argmax_take(best, bi, ndl::wave_xor<1>(best), ndl::wave_xor_int<1>(bi));
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[w] = best;
        si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < kT / 64; ++k) argmax_take(best, bi, sv[k], si[k]);
        next[b] = bi;
        if (also) also[b] = bi;
    }
}

// ---- a step's tokens from the device (nd_v3_generate): each session's
// token is the previous step's greedy choice.  Per session: the clamped id
// for the embedding row (model.rs:196-200), the token pushed into the
// retained history (cache.rs:283-289; kept right-aligned, the newest at
// mo - 1, so that at position pos the history holds min(pos + 1, mo) ids),
// and the Engram table rows hashed from it (engram.rs:30-67), -1 where an
// order reaches before position 0.
constexpr int kMaxOrders = 8;
struct StepTokens {
    const int32_t *src;  // [S]
    const int32_t *pos;  // [S]
    int32_t *tok;        // [S]
    int32_t *hist;       // [S][mo]
    int32_t *rows;       // [S][n_orders * e_heads]
    int S, mo, vocab, n_orders, e_heads, stride, e_slots;
    int orders[kMaxOrders];
};

__global__ void k_step_tokens(StepTokens a)
{
    const int row = int(blockIdx.x * blockDim.x + threadIdx.x);
    if (row >= a.S) return;
    const uint32_t tok = uint32_t(a.src[row]);
    int32_t *h = a.hist + size_t(row) * a.mo;
    for (int j = 0; j + 1 < a.mo; ++j) h[j] = h[j + 1];
    h[a.mo - 1] = int32_t(tok);
    a.tok[row] = int32_t(tok < uint32_t(a.vocab) ? tok : uint32_t(a.vocab - 1));
    const int pos = a.pos[row];
    const int here = (pos + 1 < a.mo ? pos + 1 : a.mo) - 1;
    const int nt = a.n_orders * a.e_heads;
    for (int oi = 0; oi < a.n_orders; ++oi)
        for (int hh = 0; hh < a.e_heads; ++hh) {
            const int table = oi * a.e_heads + hh;
            uint32_t acc = 0x9E3779B9u * uint32_t(oi * a.stride + hh + 1);
            for (int j = 0; j < a.orders[oi]; ++j) {
                const uint32_t t2 = j > here ? 0u : uint32_t(h[a.mo - 1 - j]);
                acc = (acc ^ t2) * 0x01000193u;
            }
            acc ^= acc >> 15;
            const uint32_t slot = acc % uint32_t(a.e_slots);
            const bool valid = pos + 1 >= a.orders[oi];
            a.rows[size_t(row) * nt + table] =
                valid ? int32_t(uint32_t(table) * uint32_t(a.e_slots) + slot) : -1;
        }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------

struct Layer {
    float *norm_in = nullptr;
    nd_cq *q = nullptr, *k = nullptr, *v = nullptr, *gate = nullptr, *out = nullptr;
    float *q_taps = nullptr, *k_taps = nullptr, *v_taps = nullptr, *q_norm = nullptr,
          *k_norm = nullptr;
    float *post_norm = nullptr, attn_gate = 0.0f, *pre_hada = nullptr;
    float *d1 = nullptr, *d2 = nullptr, *b2 = nullptr, *d3 = nullptr, *d4 = nullptr;
    float *w1a = nullptr, *w1b = nullptr, *w2a = nullptr, *w2b = nullptr, *w3a = nullptr,
          *w3b = nullptr, *cond_v = nullptr, *cond_u = nullptr;
    int cond_rank = 0;
};

struct Site {
    nd_cq *tables = nullptr, *key = nullptr, *value = nullptr;
    float *taps = nullptr;
};

bool is_global(const nd_v3_cfg &c, int li)
{
    for (int i = 0; i < c.n_global; ++i)
        if (c.global_layers[i] == li) return true;
    return false;
}

int site_of(const nd_v3_cfg &c, int li)
{
    for (int s = 0; s < c.n_sites; ++s)
        if (c.sites[s] == li) return s;
    return -1;
}

int max_order(const nd_v3_cfg &c)
{
    int m = 1;
    for (int i = 0; i < c.n_orders; ++i) m = c.orders[i] > m ? c.orders[i] : m;
    return m;
}

}  // namespace

struct nd_v3_model {
    nd_v3_cfg cfg{};
    int device = 0;
    nd_cq *embedding = nullptr;
    std::vector<Layer> layers;
    std::vector<float> a_pre, a_post, a_res;  // host copies, per layer
    std::vector<std::vector<float>> staged;  // host data of in-flight uploads
    float *b_pre = nullptr, *b_post = nullptr, *b_res = nullptr;
    nd_cq *phi_pre = nullptr, *phi_post = nullptr, *phi_res = nullptr;
    int32_t *p1 = nullptr, *p2 = nullptr;
    std::vector<Site> sites;
    float *final_norm = nullptr;
    float embed_scale = 1.0f;
    // RoPE frequencies 1 / theta^(2j / qk), libm's powf (model.rs:378-386)
    std::vector<float> rope_freq;
    // [max_seq_len][qk]: cos then sin of pos * freq[j], libm's cosf/sinf
    // (model.rs:387-394), for every position a session can reach
    float *rope_tab = nullptr;
    // prepared-input geometry of the projections each fused kernel feeds
    Prep pre_nx{}, pre_h{}, pre_attn{}, pre_x{};
    std::vector<void *> mem;  // every device float/int buffer
    std::vector<nd_cq *> cqs;

    ~nd_v3_model()
    {
        (void)hipSetDevice(device);
        for (void *p : mem) (void)hipFree(p);
        for (nd_cq *w : cqs) nd_cq_free(w);
    }
};

struct SessionHost {
    int pos = 0;
    std::vector<uint32_t> hist;
    std::vector<int> slots;  // the reference's logical ring size per layer
};

struct nd_v3_batch {
    int device = 0;
    int B = 0, max_len = 0;
    // positions one step may take per session (prefill), and the rows the
    // per-row buffers hold: B * chunk
    int chunk = 1, R = 0;
    // KvPrecision::F32: f32 KV blocks, the query not fake-quantised
    bool kv_f32 = false;
    std::vector<SessionHost> s;
    std::vector<uint8_t *> kv;        // per layer: B blocks
    std::vector<size_t> kv_stride;    // per layer
    std::vector<nd_kv_geom> geom;     // per layer
    std::vector<int> cap;             // per layer
    std::vector<float *> qt, kt, vt;  // per layer conv tails [B][taps-1][dim]
    std::vector<float *> et;          // per site Engram tails [B][reach][d]
    // activations
    // (nxh, hh, ah, xh: prepared inputs of the projections, in_padded wide)
    float *lanes = nullptr, *nxh = nullptr, *u = nullptr, *bx = nullptr, *hh = nullptr,
          *q = nullptr, *k = nullptr, *v = nullptr, *gate = nullptr, *attn = nullptr,
          *ah = nullptr, *proj = nullptr, *p2 = nullptr, *y = nullptr, *hpre = nullptr,
          *hpost = nullptr, *hres = nullptr, *emb = nullptr, *fetched = nullptr, *fh = nullptr,
          *ek = nullptr, *ev = nullptr, *xh = nullptr, *logits = nullptr;
    float *gp = nullptr, *gr = nullptr;  // scatter-up gates of the latest layer
    float *gstate = nullptr;             // [R][64] Sinkhorn state between the gate phases
    float *graw = nullptr;               // [R][n + n*n] raw gates from k_layer_in
    // several positions per step: the normed q ([R][qd]) and the Engram
    // conv ([sites][R][d]) go here, the projections' rows stay as they are
    float *qn = nullptr, *evc = nullptr;
    size_t fh_width = 0;  // floats per row of a site's prepared key input
    int32_t *next = nullptr;
    // nd_v3_generate: each session's retained token ids on the device
    // ([B][mo], right-aligned), and the steps' greedy tokens ([steps][B],
    // grown on demand, owned here)
    int32_t *hist_dev = nullptr;
    int32_t *gen_out = nullptr;
    size_t gen_cap = 0;
    std::vector<int32_t> gen_init;  // the loop's first tokens and ids, read by its uploads
    // The scatter-up gates of a layer depend only on its input lanes: they
    // run on `side` while the layer's attention and MLP run on the caller's
    // stream; ev_in[l % 2] marks a layer's input ready, ev_gates[l % 2] its
    // gates.
    hipStream_t side = nullptr;
    hipEvent_t ev_in[2] = {}, ev_gates[2] = {};
    // Per-step inputs, uploaded from pinned host memory in one copy.  The
    // copy is asynchronous, so a host buffer is reused only once the copy
    // that read it has completed: a ring of kStages buffers, each with the
    // event recorded after its copy, lets the host run that many steps ahead.
    static constexpr int kStages = 4;
    void *step_dev = nullptr;
    void *stage_host[kStages] = {};
    hipEvent_t stage_done[kStages] = {};
    bool stage_pending[kStages] = {};
    int stage_next = 0;
    size_t step_bytes = 0;
    int32_t *next_host = nullptr;
    std::vector<void *> mem;
    // the host thread inside a call on this batch (one at a time)
    nd::Owner owner;
    // With `graphs` (off unless asked for), one decode position per session
    // replays a captured graph of the step's kernels on `gstream`: captured on
    // the second such step (the first, eager, has sized everything the
    // kernels touch), launched as one unit after; g_in / g_out order it after
    // and before the caller's stream.  On ROCm 7.2 the replay of this
    // two-branch graph of ~200 kernels is slower than enqueueing them.
    bool graphs = false;
    int eager_steps = 0;
    hipGraphExec_t graph_exec = nullptr;
    hipStream_t gstream = nullptr;
    hipEvent_t g_in = nullptr, g_out = nullptr;

    ~nd_v3_batch()
    {
        (void)hipSetDevice(device);
        if (graph_exec) {
            (void)hipDeviceSynchronize();
            (void)hipGraphExecDestroy(graph_exec);
        }
        if (side) (void)hipStreamSynchronize(side);
        for (int i = 0; i < kStages; ++i)
            if (stage_pending[i]) (void)hipEventSynchronize(stage_done[i]);
        if (gen_out) (void)hipFree(gen_out);
        for (void *p : mem) (void)hipFree(p);  // hipFree waits for the device's work
        for (int i = 0; i < kStages; ++i) {
            if (stage_host[i]) (void)hipHostFree(stage_host[i]);
            if (stage_done[i]) (void)hipEventDestroy(stage_done[i]);
        }
        if (next_host) (void)hipHostFree(next_host);
        for (int i = 0; i < 2; ++i) {
            if (ev_in[i]) (void)hipEventDestroy(ev_in[i]);
            if (ev_gates[i]) (void)hipEventDestroy(ev_gates[i]);
        }
        if (side) (void)hipStreamDestroy(side);
        if (g_in) (void)hipEventDestroy(g_in);
        if (g_out) (void)hipEventDestroy(g_out);
        if (gstream) (void)hipStreamDestroy(gstream);
    }
};

namespace {

template <typename T>
int dalloc(std::vector<void *> &mem, T **p, size_t count)
{
    void *q = nullptr;
    hipError_t e = hipMalloc(&q, count * sizeof(T) + 16);
    if (e != hipSuccess) return nd::hip_fail(e, "hipMalloc");
    mem.push_back(q);
    *p = static_cast<T *>(q);
    return ND_OK;
}

int upload_floats(nd_ctx *ctx, nd_v3_model *m, const nd_v3_record &r, size_t want, float **out,
                  const char *what, size_t idx)
{
    if (r.kind != ND_REC_F32 || r.len != want * 4)
        return nd::fail(ND_ERR_ARG, "record %zu (%s): want %zu f32, got kind %d with %zu bytes", idx,
                        what, want, int(r.kind), r.len);
    if (int rc = dalloc(m->mem, out, want)) return rc;
    ND_HIP(hipMemcpyAsync(*out, r.data, want * 4, hipMemcpyHostToDevice, ctx->stream));
    return ND_OK;
}

// A 32x32 f32 record uploaded transposed (the factors of the HadamardMLP's
// Kronecker passes, read column-wise); the host copy lives as long as the model.
int upload_transposed32(nd_ctx *ctx, nd_v3_model *m, const nd_v3_record &r, float **out,
                        const char *what, size_t idx)
{
    if (r.kind != ND_REC_F32 || r.len != 1024 * 4)
        return nd::fail(ND_ERR_ARG, "record %zu (%s): want 1024 f32, got kind %d with %zu bytes", idx,
                        what, int(r.kind), r.len);
    const float *src = static_cast<const float *>(r.data);
    m->staged.emplace_back(1024);
    std::vector<float> &tr = m->staged.back();
    for (int i = 0; i < 32; ++i)
        for (int k = 0; k < 32; ++k) tr[size_t(k) * 32 + i] = src[i * 32 + k];
    if (int rc = dalloc(m->mem, out, 1024)) return rc;
    ND_HIP(hipMemcpyAsync(*out, tr.data(), 1024 * 4, hipMemcpyHostToDevice, ctx->stream));
    return ND_OK;
}

int take_cq(nd_ctx *ctx, nd_v3_model *m, const nd_v3_record &r, const float *cb, size_t out,
            size_t in, nd_cq **w, const char *what, size_t idx)
{
    if (r.kind != ND_REC_CQ || r.out != out || r.in != in)
        return nd::fail(ND_ERR_ARG, "record %zu (%s): want a %zux%zu CQ tensor, got kind %d %zux%zu",
                        idx, what, out, in, int(r.kind), r.out, r.in);
    if (int rc = nd_cq_from_blob(ctx, static_cast<const uint8_t *>(r.data), r.len, r.out, r.in,
                                 r.group, uint8_t(r.bits), cb, 28, w))
        return rc;
    m->cqs.push_back(*w);
    return ND_OK;
}

// Projections over `B` prepared rows in the reference's summation order,
// batch-major output; weights that share the input go in one launch.
int project(nd_ctx *ctx, const nd_cq *w, const float *xh, int B, size_t row_start, size_t rows,
            float *y)
{
    return nd_cq_exact_set(ctx, ctx->stream, 1, &w, xh, size_t(B), &row_start, &rows, &y,
                           "v3 projection");
}

Prep prep_of(const nd_cq *w)
{
    return Prep{int(w->in_padded), int(w->group), w->inv_sqrt_group};
}

}  // namespace

extern "C" {

int nd_v3_model_create(nd_ctx *ctx, const nd_v3_cfg *cfg, const float *codebook,
                       size_t codebook_len, const nd_v3_record *recs, size_t n, nd_v3_model **out)
{
    ND_ENTER(ctx);
    ND_REQUIRE(cfg && recs && out && codebook, "null argument");
    ND_REQUIRE(codebook_len == 28, "codebook must be 28 floats (got %zu)", codebook_len);
    *out = nullptr;
    const nd_v3_cfg &c = *cfg;
    ND_REQUIRE(c.hada_n == 1024, "hada_n %d: the device HadamardMLP is built for 1024 (32x32)",
               c.hada_n);
    ND_REQUIRE(c.mhc_lanes >= 1 && c.mhc_lanes <= 16, "mhc_lanes %d out of range", c.mhc_lanes);
    ND_REQUIRE(c.d_model > 0 && c.d_model <= 1024, "d_model %d out of range", c.d_model);
    ND_REQUIRE(c.num_layers > 0 && c.n_sites >= 0 && c.n_sites <= 64 && c.n_global <= 64 &&
                   c.n_orders >= 1 && c.n_orders <= 8,
               "bad layer/site counts");
    ND_REQUIRE(c.qk_head_dim % 2 == 0 && c.qk_head_dim <= 128, "qk_head_dim %d", c.qk_head_dim);
    ND_REQUIRE(c.num_heads >= 1 && c.num_kv_heads >= 1 && c.num_heads + c.num_kv_heads <= 64 &&
                   (c.num_heads + c.num_kv_heads) * c.qk_head_dim <= kMaxQkDims,
               "%d query + %d kv heads of %d: the q/k post-processing holds at most 64 heads "
               "and %d values", c.num_heads, c.num_kv_heads, c.qk_head_dim, kMaxQkDims);
    nd_v3_model *m = new (std::nothrow) nd_v3_model;
    if (!m) return nd::fail(ND_ERR_NOMEM, "host allocation failed");
    m->cfg = c;
    for (int j = 0; j < c.qk_head_dim / 2; ++j)
        m->rope_freq.push_back(1.0f / nd_powf(c.rope_theta, float(2 * j) / float(c.qk_head_dim)));
    m->device = ctx->device;
    {
        const int half = c.qk_head_dim / 2;
        m->staged.emplace_back(size_t(c.max_seq_len) * c.qk_head_dim);
        std::vector<float> &tab = m->staged.back();
        for (int pos = 0; pos < c.max_seq_len; ++pos)
            for (int j = 0; j < half; ++j) {
                const float angle = float(pos) * m->rope_freq[j];
                tab[size_t(pos) * c.qk_head_dim + j] = nd_cosf(angle);
                tab[size_t(pos) * c.qk_head_dim + half + j] = nd_sinf(angle);
            }
        int rc0 = dalloc(m->mem, &m->rope_tab, tab.size());
        if (rc0) {
            delete m;
            return rc0;
        }
        hipError_t e = hipMemcpyAsync(m->rope_tab, tab.data(), tab.size() * 4, hipMemcpyHostToDevice,
                                      ctx->stream);
        if (e != hipSuccess) {
            delete m;
            return nd::hip_fail(e, "hipMemcpyAsync (RoPE table)");
        }
    }
    const size_t d = c.d_model, L = c.num_layers, nl = c.mhc_lanes;
    const size_t qd = size_t(c.num_heads) * c.qk_head_dim, kd = size_t(c.num_kv_heads) * c.qk_head_dim;
    const size_t vd = size_t(c.num_kv_heads) * c.v_head_dim, od = size_t(c.num_heads) * c.v_head_dim;
    const size_t T = c.qkv_conv_taps, hn = c.hada_n;
    size_t i = 0;
    int rc = ND_OK;
    auto next = [&](const char *what) -> const nd_v3_record * {
        if (i >= n) {
            rc = nd::fail(ND_ERR_ARG, "records end before %s (record %zu)", what, i);
            return nullptr;
        }
        return &recs[i++];
    };
#define REC(name) \
    const nd_v3_record *r_##name = next(#name); \
    if (!r_##name) goto fail;
#define F32(dst, name, count)                                                          \
    {                                                                                  \
        REC(name);                                                                     \
        if ((rc = upload_floats(ctx, m, *r_##name, (count), &(dst), #name, i - 1))) goto fail; \
    }
#define CQ(dst, name, o, in_)                                                              \
    {                                                                                      \
        REC(name);                                                                         \
        if ((rc = take_cq(ctx, m, *r_##name, codebook, (o), (in_), &(dst), #name, i - 1))) goto fail; \
    }
    {
        CQ(m->embedding, embedding, size_t(c.vocab_size), d);
        m->layers.resize(L);
        for (size_t li = 0; li < L; ++li) {
            Layer &l = m->layers[li];
            F32(l.norm_in, norm_in, d);
            CQ(l.q, q_proj, qd, d);
            CQ(l.k, k_proj, kd, d);
            CQ(l.v, v_proj, vd, d);
            if (T > 0) {
                F32(l.q_taps, q_taps, T * qd);
                F32(l.k_taps, k_taps, T * kd);
                F32(l.v_taps, v_taps, T * vd);
            }
            F32(l.q_norm, q_norm, size_t(c.qk_head_dim));
            F32(l.k_norm, k_norm, size_t(c.qk_head_dim));
            CQ(l.gate, gate_proj, od, d);
            CQ(l.out, out_proj, d, od);
            F32(l.post_norm, post_norm, d);
            {
                REC(attn_gate);
                if (r_attn_gate->kind != ND_REC_F32 || r_attn_gate->len != 4) {
                    rc = nd::fail(ND_ERR_ARG, "record %zu (attn_gate): want 1 f32", i - 1);
                    goto fail;
                }
                std::memcpy(&l.attn_gate, r_attn_gate->data, 4);
            }
            F32(l.pre_hada, pre_hada, d);
            F32(l.d1, d1, hn);
            F32(l.d2, d2, hn);
            F32(l.b2, b2, hn);
            F32(l.d3, d3, hn);
            F32(l.d4, d4, hn);
            {
                REC(w1a);
                if ((rc = upload_transposed32(ctx, m, *r_w1a, &l.w1a, "w1a", i - 1))) goto fail;
            }
            {
                REC(w1b);
                if ((rc = upload_transposed32(ctx, m, *r_w1b, &l.w1b, "w1b", i - 1))) goto fail;
            }
            {
                REC(w2a);
                if ((rc = upload_transposed32(ctx, m, *r_w2a, &l.w2a, "w2a", i - 1))) goto fail;
            }
            {
                REC(w2b);
                if ((rc = upload_transposed32(ctx, m, *r_w2b, &l.w2b, "w2b", i - 1))) goto fail;
            }
            {
                REC(w3a);
                if ((rc = upload_transposed32(ctx, m, *r_w3a, &l.w3a, "w3a", i - 1))) goto fail;
            }
            {
                REC(w3b);
                if ((rc = upload_transposed32(ctx, m, *r_w3b, &l.w3b, "w3b", i - 1))) goto fail;
            }
            {
                if (i >= n) {
                    rc = nd::fail(ND_ERR_ARG, "records end before cond_v");
                    goto fail;
                }
                l.cond_rank = int(recs[i].in);
                if (l.cond_rank < 1 || l.cond_rank > 64) {
                    rc = nd::fail(ND_ERR_ARG, "record %zu (cond_v): rank %d out of 1..64", i, l.cond_rank);
                    goto fail;
                }
            }
            F32(l.cond_v, cond_v, d * l.cond_rank);
            F32(l.cond_u, cond_u, size_t(l.cond_rank) * hn);
        }
        for (const char *nm : {"a_pre", "a_post", "a_res"}) {
            REC(scalar);
            if (r_scalar->kind != ND_REC_F32 || r_scalar->len != L * 4) {
                rc = nd::fail(ND_ERR_ARG, "record %zu (%s): want %zu f32", i - 1, nm, L);
                goto fail;
            }
            std::vector<float> &dst = nm[2] == 'p' && nm[3] == 'r' ? m->a_pre
                                      : nm[2] == 'p'                ? m->a_post
                                                                    : m->a_res;
            dst.resize(L);
            std::memcpy(dst.data(), r_scalar->data, L * 4);
        }
        F32(m->b_pre, b_pre, L * nl);
        F32(m->b_post, b_post, L * nl);
        F32(m->b_res, b_res, L * nl * nl);
        CQ(m->phi_pre, phi_pre, L * nl, nl * d);
        CQ(m->phi_post, phi_post, L * nl, nl * d);
        CQ(m->phi_res, phi_res, L * nl * nl, nl * d);
        for (int pi = 0; pi < 2; ++pi) {
            REC(perm);
            if (r_perm->kind != ND_REC_F32 || r_perm->len != hn * 4) {
                rc = nd::fail(ND_ERR_ARG, "record %zu (hada perm): want %zu f32", i - 1, hn);
                goto fail;
            }
            std::vector<int32_t> pv(hn);
            const float *pf = static_cast<const float *>(r_perm->data);
            for (size_t k2 = 0; k2 < hn; ++k2) {
                const float f = pf[k2];
                if (!(f >= 0.0f && f < float(hn))) {
                    rc = nd::fail(ND_ERR_ARG, "record %zu: permutation entry %zu out of range", i - 1, k2);
                    goto fail;
                }
                pv[k2] = int32_t(f);
            }
            int32_t **dst = pi == 0 ? &m->p1 : &m->p2;
            if ((rc = dalloc(m->mem, dst, hn))) goto fail;
            hipError_t e = hipMemcpy(*dst, pv.data(), hn * 4, hipMemcpyHostToDevice);
            if (e != hipSuccess) {
                rc = nd::hip_fail(e, "hipMemcpy");
                goto fail;
            }
        }
        const size_t nt = size_t(c.n_orders) * c.e_heads;
        m->sites.resize(c.n_sites);
        for (int s = 0; s < c.n_sites; ++s) {
            Site &st = m->sites[s];
            CQ(st.tables, tables, nt * c.e_slots, size_t(c.e_sub_dim));
            CQ(st.key, key_proj, d, nt * c.e_sub_dim);
            CQ(st.value, value_proj, d, nt * c.e_sub_dim);
            F32(st.taps, engram_taps, size_t(c.e_conv_taps) * d);
        }
        F32(m->final_norm, final_norm, d);
    }
#undef REC
#undef F32
#undef CQ
    m->embed_scale = std::sqrt(float(d));
    m->pre_nx = prep_of(m->phi_pre);
    m->pre_h = prep_of(m->layers[0].q);
    m->pre_attn = prep_of(m->layers[0].out);
    m->pre_x = prep_of(m->embedding);
    {
        auto same = [](const nd_cq *a, const Prep &p) {
            return int(a->in_padded) == p.in_padded && int(a->group) == p.group;
        };
        bool ok = same(m->phi_post, m->pre_nx) && same(m->phi_res, m->pre_nx);
        for (const Layer &l : m->layers)
            ok = ok && same(l.q, m->pre_h) && same(l.k, m->pre_h) && same(l.v, m->pre_h) &&
                 same(l.gate, m->pre_h) && same(l.out, m->pre_attn);
        if (!ok) {
            rc = nd::fail(ND_ERR_ARG, "projections sharing an input must share group size");
            goto fail;
        }
        if (m->pre_h.in_padded > 1024 || m->pre_x.in_padded > 1024 ||
            m->pre_attn.in_padded > kMaxGatePad || m->pre_nx.in_padded > kMaxLanesD ||
            nl * d > kMaxLanesD || size_t(c.num_kv_heads) * c.v_head_dim > size_t(kMaxVDims)) {
            rc = nd::fail(ND_ERR_ARG, "padded projection inputs exceed the fused kernels' LDS");
            goto fail;
        }
        const nd_cq *phi = m->phi_pre;
        if (phi->group != 128 || !(phi->per_byte == 2 || phi->per_byte == 4) ||
            nl * phi->num_groups > size_t(kMaxPhiPairs) ||
            phi->num_groups * kPadGroup > size_t(kMaxLanesD)) {
            rc = nd::fail(ND_ERR_ARG, "phi_pre must be 2- or 4-bit with 128-wide groups");
            goto fail;
        }
    }
    {
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            rc = nd::hip_fail(e, "upload");
            goto fail;
        }
    }
    *out = m;
    return ND_OK;
fail:
    (void)hipStreamSynchronize(ctx->stream);
    delete m;
    return rc ? rc : ND_ERR_ARG;
}

void nd_v3_model_free(nd_v3_model *m) { delete m; }

size_t nd_v3_logit_rows(const nd_v3_model *m)
{
    if (!m) return 0;
    return size_t(m->cfg.out_vocab ? m->cfg.out_vocab : m->cfg.vocab_size);
}

int nd_v3_batch_create(nd_ctx *ctx, const nd_v3_model *m, size_t sessions, size_t max_len,
                       size_t hint, nd_v3_batch **out)
{
    return nd_v3_batch_create_chunked(ctx, m, sessions, max_len, hint, 1, out);
}

int nd_v3_batch_create_chunked(nd_ctx *ctx, const nd_v3_model *m, size_t sessions, size_t max_len,
                               size_t hint, size_t max_chunk, nd_v3_batch **out)
{
    return nd_v3_batch_create_ex(ctx, m, sessions, max_len, hint, max_chunk, 1, out);
}

int nd_v3_batch_create_ex(nd_ctx *ctx, const nd_v3_model *m, size_t sessions, size_t max_len,
                          size_t hint, size_t max_chunk, int kv_int8, nd_v3_batch **out)
{
    ND_ENTER(ctx);
    ND_REQUIRE(m && out, "null argument");
    *out = nullptr;
    const nd_v3_cfg &c = m->cfg;
    ND_REQUIRE(sessions >= 1 && sessions <= 4096, "sessions %zu out of 1..4096", sessions);
    ND_REQUIRE(max_len >= 1 && max_len <= size_t(c.max_seq_len), "max_len %zu out of 1..%d",
               max_len, c.max_seq_len);
    ND_REQUIRE(max_chunk >= 1 && max_chunk <= 256 && sessions * max_chunk <= 16384,
               "max_chunk %zu out of 1..256 (or sessions x max_chunk above 16384)", max_chunk);
    nd_v3_batch *b = new (std::nothrow) nd_v3_batch;
    if (!b) return nd::fail(ND_ERR_NOMEM, "host allocation failed");
    b->device = ctx->device;
    b->B = int(sessions);
    b->max_len = int(max_len);
    b->chunk = int(max_chunk);
    b->R = int(sessions * max_chunk);
    b->kv_f32 = kv_int8 == 0;
    const int B = b->R, L = c.num_layers, nl = c.mhc_lanes, d = c.d_model;
    const int S = b->B;  // sessions: per-session state
    const int qd = c.num_heads * c.qk_head_dim, kd = c.num_kv_heads * c.qk_head_dim;
    const int vd = c.num_kv_heads * c.v_head_dim, od = c.num_heads * c.v_head_dim;
    const int T = c.qkv_conv_taps, nt = c.n_orders * c.e_heads;
    const int reach = (c.e_conv_taps > 0 ? c.e_conv_taps - 1 : 0) * c.e_conv_dilation;
    const size_t rows = nd_v3_logit_rows(m);
    const size_t hnt = hint < 1 ? 1 : (hint > size_t(c.max_seq_len) ? size_t(c.max_seq_len) : hint);
    int rc = ND_OK;
    b->s.resize(S);
    for (auto &sh : b->s) sh.slots.resize(L);
    b->kv.resize(L);
    b->kv_stride.resize(L);
    b->geom.resize(L);
    b->cap.resize(L);
    b->qt.resize(L);
    b->kt.resize(L);
    b->vt.resize(L);
    for (int li = 0; li < L; ++li) {
        // cache.rs:190-199: cap = window (local) or max_seq_len (global);
        // the device block needs only the positions this batch can reach.
        const int ref_cap = is_global(c, li) || c.sliding_window == 0
                                ? c.max_seq_len
                                : (c.sliding_window < c.max_seq_len ? c.sliding_window : c.max_seq_len);
        b->cap[li] = ref_cap;
        // a step of C positions writes C slots before its rows attend: the
        // ring holds window + C - 1 positions so none of them is overwritten
        // while a row of the step still reads it
        const long wide = long(ref_cap) + long(b->chunk) - 1;
        const int dev_cap = int(wide < b->max_len ? wide : b->max_len);
        if (b->kv_f32 && dev_cap > 8192) {
            rc = nd::fail(ND_ERR_ARG, "layer %d: an f32 KV ring of %d positions (the f32 view "
                          "attends over at most 8192)", li, dev_cap);
            goto fail;
        }
        for (auto &sh : b->s) sh.slots[li] = int(hnt < size_t(ref_cap) ? hnt : size_t(ref_cap));
        nd_kv_geom g{c.num_heads, c.num_kv_heads, c.qk_head_dim, c.v_head_dim, dev_cap};
        b->geom[li] = g;
        b->kv_stride[li] = b->kv_f32 ? nd_kv_f32_block_bytes(&g) : nd_kv_block_bytes(&g);
        if ((rc = dalloc(b->mem, &b->kv[li], b->kv_stride[li] * S))) goto fail;
        {
            hipError_t e = hipMemsetAsync(b->kv[li], 0, b->kv_stride[li] * S, ctx->stream);
            if (e != hipSuccess) {
                rc = nd::hip_fail(e, "hipMemsetAsync");
                goto fail;
            }
        }
        const int tt = T > 0 ? T - 1 : 0;
        if ((rc = dalloc(b->mem, &b->qt[li], size_t(S) * tt * qd + 1))) goto fail;
        if ((rc = dalloc(b->mem, &b->kt[li], size_t(S) * tt * kd + 1))) goto fail;
        if ((rc = dalloc(b->mem, &b->vt[li], size_t(S) * tt * vd + 1))) goto fail;
        (void)hipMemsetAsync(b->qt[li], 0, (size_t(S) * tt * qd + 1) * 4, ctx->stream);
        (void)hipMemsetAsync(b->kt[li], 0, (size_t(S) * tt * kd + 1) * 4, ctx->stream);
        (void)hipMemsetAsync(b->vt[li], 0, (size_t(S) * tt * vd + 1) * 4, ctx->stream);
    }
    b->et.resize(c.n_sites);
    for (int s = 0; s < c.n_sites; ++s) {
        if ((rc = dalloc(b->mem, &b->et[s], size_t(S) * reach * d + 1))) goto fail;
        (void)hipMemsetAsync(b->et[s], 0, (size_t(S) * reach * d + 1) * 4, ctx->stream);
    }
#define A(p, cnt) \
    if ((rc = dalloc(b->mem, &b->p, size_t(cnt)))) goto fail;
    A(lanes, size_t(B) * nl * d);
    {
        size_t phi_pad = 0;
        if ((rc = nd_cq_shape(m->phi_pre, nullptr, nullptr, &phi_pad, nullptr, nullptr))) goto fail;
        if ((rc = dalloc(b->mem, &b->nxh, size_t(B) * phi_pad))) goto fail;
    }
    A(u, size_t(B) * d);
    A(bx, size_t(B) * d);
    A(hh, size_t(B) * m->pre_h.in_padded);
    A(q, size_t(B) * qd);
    A(k, size_t(B) * kd);
    A(v, size_t(B) * vd);
    A(gate, size_t(B) * od);
    A(attn, size_t(B) * od);
    A(ah, size_t(B) * m->pre_attn.in_padded);
    A(proj, size_t(B) * d);
    A(p2, size_t(B) * d);
    A(y, size_t(B) * d);
    A(hpre, size_t(B) * nl);
    A(hpost, size_t(B) * nl);
    A(hres, size_t(B) * nl * nl);
    A(emb, size_t(B) * d);
    A(fetched, size_t(B) * nt * c.e_sub_dim);
    // one prepared key input per site: [sites][B][fh_width]
    b->fh_width = size_t(nt) * c.e_sub_dim;
    for (int s = 0; s < c.n_sites; ++s)
        if (m->sites[s].key->in_padded > b->fh_width) b->fh_width = m->sites[s].key->in_padded;
    b->fh_width = (b->fh_width + 3) & ~size_t(3);
    A(fh, size_t(c.n_sites > 0 ? c.n_sites : 1) * B * b->fh_width);
    A(ek, size_t(c.n_sites > 0 ? c.n_sites : 1) * B * d);
    A(ev, size_t(c.n_sites > 0 ? c.n_sites : 1) * B * d);
    A(xh, size_t(S) * m->pre_x.in_padded);
    A(logits, size_t(S) * rows);
    A(gp, size_t(B) * nl);
    A(gr, size_t(B) * nl * nl);
    A(gstate, size_t(B) * 64);
    A(graw, size_t(B) * (nl + nl * nl));
    A(next, size_t(S));
    A(hist_dev, size_t(S) * max_order(c));
    if (b->chunk > 1) {
        A(qn, size_t(B) * qd);
        A(evc, size_t(c.n_sites > 0 ? c.n_sites : 1) * B * d);
    }
#undef A
    {
        hipError_t e = hipStreamCreateWithFlags(&b->side, hipStreamNonBlocking);
        for (int i = 0; i < 2 && e == hipSuccess; ++i) {
            // these only order the two streams on this GPU: no system-scope
            // fence (with one, each record cost ~12 us of idle GPU per layer)
            const unsigned fl = hipEventDisableTiming | hipEventDisableSystemFence;
            e = hipEventCreateWithFlags(&b->ev_in[i], fl);
            if (e == hipSuccess) e = hipEventCreateWithFlags(&b->ev_gates[i], fl);
        }
        if (e != hipSuccess) {
            rc = nd::hip_fail(e, "stream/event creation");
            goto fail;
        }
    }
    {
        // step inputs: tokens, pos, hi[B], lo[L][B], engram rows [B][nt]
        const size_t ints = size_t(B) * (3 + L + nt);
        b->step_bytes = ints * 4;
        if ((rc = dalloc(b->mem, reinterpret_cast<uint8_t **>(&b->step_dev), b->step_bytes))) goto fail;
        hipError_t e = hipSuccess;
        for (int i = 0; i < nd_v3_batch::kStages && e == hipSuccess; ++i) {
            e = hipHostMalloc(&b->stage_host[i], b->step_bytes, hipHostMallocDefault);
            // the host waits on it before rewriting the buffer the copy read;
            // no device data is read through it, so no system-scope fence
            if (e == hipSuccess)
                e = hipEventCreateWithFlags(&b->stage_done[i],
                                            hipEventDisableTiming | hipEventDisableSystemFence);
        }
        if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void **>(&b->next_host), size_t(S) * 4, hipHostMallocDefault);
        if (e != hipSuccess) {
            rc = nd::hip_fail(e, "hipHostMalloc");
            goto fail;
        }
    }
    {
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            rc = nd::hip_fail(e, "batch set-up");
            goto fail;
        }
    }
    *out = b;
    return ND_OK;
fail:
    (void)hipStreamSynchronize(ctx->stream);
    delete b;
    return rc ? rc : ND_ERR_ARG;
}

void nd_v3_batch_free(nd_v3_batch *b) { delete b; }

int nd_v3_batch_set_graphs(nd_v3_batch *b, int on)
{
    nd::clear_error();
    ND_REQUIRE(b, "null batch");
    nd::Hold hold(b->owner, "the batch");
    if (hold.rc) return hold.rc;
    ND_HIP(hipSetDevice(b->device));
    if (!on && b->graph_exec) {
        ND_HIP(hipDeviceSynchronize());
        ND_HIP(hipGraphExecDestroy(b->graph_exec));
        b->graph_exec = nullptr;
    }
    b->graphs = on != 0;
    return ND_OK;
}

int nd_v3_positions(const nd_v3_batch *b, int32_t *pos)
{
    nd::clear_error();
    ND_REQUIRE(b && pos, "null argument");
    nd::Hold hold(const_cast<nd_v3_batch *>(b)->owner, "the batch");
    if (hold.rc) return hold.rc;
    for (int i = 0; i < b->B; ++i) pos[i] = b->s[i].pos;
    return ND_OK;
}

int nd_libm_map(nd_ctx *ctx, int fn, const float *x, size_t n, float *y)
{
    ND_ENTER(ctx);
    ND_REQUIRE(fn >= 0 && fn <= 2, "libm function %d (0 expf, 1 logf, 2 sigmoid)", fn);
    if (n == 0) return ND_OK;
    ND_REQUIRE(x && y, "null buffer");
    const size_t blocks = (n + 255) / 256;
    ND_REQUIRE(blocks <= 0x7fffffffu, "n %zu too large", n);
    hipLaunchKernelGGL(k_libm_map, dim3(unsigned(blocks)), dim3(256), 0, ctx->stream, fn, x, n, y);
    return nd::check_launch("k_libm_map");
}

int nd_argmax_rows(nd_ctx *ctx, const float *x, size_t count, size_t n, int32_t *out)
{
    ND_ENTER(ctx);
    if (count == 0) return ND_OK;
    ND_REQUIRE(x && out, "argmax_rows: null buffer");
    ND_REQUIRE(n >= 1 && n <= 0x7fffffffu, "argmax_rows: row length %zu outside 1..2^31-1", n);
    ND_REQUIRE(count <= 0x7fffffffu, "argmax_rows: %zu rows", count);
    hipLaunchKernelGGL(k_argmax, dim3(unsigned(count)), dim3(kT), 0, ctx->stream, x, int(n), out,
                       nullptr);
    return nd::check_launch("argmax_rows");
}

}  // extern "C"

namespace {

// C consecutive positions for every session (C = 1: one decode step).  Row
// i * C + j of every per-row buffer is position pos + j of session i; the
// layers run once over all rows; only each session's last row is scored.
// One step (or prefill pass) of one batch, in pieces: begin() does the host
// bookkeeping and the upload of the step's inputs; enqueue(phase) queues the
// Engram and embedding prologue (phase -1), layer `phase` (0..L-1) or the
// head (L) on the batch's stream; finish() the copies out.  A batch split
// into session groups runs one StepRun per group and interleaves their
// phases, so the groups' kernels overlap on the GPU.
struct StepRun {
    nd_ctx *ctx;
    const nd_v3_model *m;
    nd_v3_batch *b;
    int C;
    int S = 0, B = 0, Rcap = 0, L = 0, nl = 0, d = 0, qd = 0, kd = 0, vd = 0, od = 0, nt = 0, mo = 0;
    size_t rows = 0;
    int32_t *tok_dev = nullptr, *pos_dev = nullptr, *hi_dev = nullptr, *lo_dev = nullptr,
            *rows_dev = nullptr;
    hipStream_t st = nullptr;
    float qk_scale = 1.0f;
    int kf = 0;
    bool gate_fused = false, gates_in = false;
    const nd_cq *phi = nullptr, *fpo = nullptr, *fre = nullptr;
    float *ev_conv = nullptr;  // [sites][Rcap][d], after the conv
    // tokens == nullptr: this step's tokens are b->next on the device (the
    // previous step's choices); the greedy choices are also written here
    int32_t *argmax_also = nullptr;

    int begin(const int32_t *tokens);
    int enqueue(int phase, bool argmax);
};

int StepRun::begin(const int32_t *tokens)
{
    ND_ENTER(ctx);
    ND_REQUIRE(m && b, "null argument");
    const bool dev_tokens = tokens == nullptr;
    ND_REQUIRE(C >= 1 && C <= b->chunk, "%d positions per step; the batch takes at most %d", C,
               b->chunk);
    ND_REQUIRE(!dev_tokens || C == 1, "device tokens take one position per step");
    const nd_v3_cfg &c = m->cfg;
    S = b->B;
    B = S * C;
    Rcap = b->R;
    L = c.num_layers;
    nl = c.mhc_lanes;
    d = c.d_model;
    qd = c.num_heads * c.qk_head_dim;
    kd = c.num_kv_heads * c.qk_head_dim;
    vd = c.num_kv_heads * c.v_head_dim;
    od = c.num_heads * c.v_head_dim;
    nt = c.n_orders * c.e_heads;
    mo = max_order(c);
    rows = nd_v3_logit_rows(m);
    for (int i = 0; i < S; ++i)
        ND_REQUIRE(b->s[i].pos + C <= b->max_len, "session %d is full (%d positions)", i, b->max_len);

    // ---- host bookkeeping (V3Cache state that only steers addressing) -------
    const int stage = b->stage_next;
    if (b->stage_pending[stage]) ND_HIP(hipEventSynchronize(b->stage_done[stage]));
    b->stage_pending[stage] = false;
    int32_t *si = static_cast<int32_t *>(b->stage_host[stage]);
    int32_t *h_tok = si, *h_pos = si + B, *h_hi = si + 2 * B, *h_lo = si + 3 * B;
    int32_t *h_rows = si + 3 * B + size_t(L) * B;
    for (int row = 0; row < B; ++row) {
        const int i = row;  // buffer row: session row / C, position pos + row % C
        SessionHost &sh = b->s[row / C];
        const int pos = sh.pos + row % C;
        h_pos[i] = pos;
        h_hi[i] = pos;
        const int stride = c.e_seed_heads == 0 ? c.e_heads : c.e_seed_heads;
        if (!dev_tokens) {
        const uint32_t tok = uint32_t(tokens[row]);
        // cache.rs:283-289 push_token, keeping max(order) ids
        sh.hist.push_back(tok);
        if (int(sh.hist.size()) > mo) sh.hist.erase(sh.hist.begin());
        // model.rs:196-200 embedding row of the clamped token
        h_tok[i] = int32_t(tok < uint32_t(c.vocab_size) ? tok : uint32_t(c.vocab_size - 1));
        // engram.rs:30-67 hash of the retained history at its last position
        const int here = int(sh.hist.size()) - 1;
        for (int oi = 0; oi < c.n_orders; ++oi)
            for (int hh = 0; hh < c.e_heads; ++hh) {
                const int table = oi * c.e_heads + hh;
                uint32_t acc = 0x9E3779B9u * uint32_t(oi * stride + hh + 1);
                for (int j = 0; j < c.orders[oi]; ++j) {
                    const uint32_t t2 = j > here ? 0u : sh.hist[here - j];
                    acc = (acc ^ t2) * 0x01000193u;
                }
                acc ^= acc >> 15;
                const uint32_t slot = acc % uint32_t(c.e_slots);
                const bool valid = pos + 1 >= c.orders[oi];
                h_rows[size_t(i) * nt + table] = valid ? int32_t(uint32_t(table) * uint32_t(c.e_slots) + slot) : -1;
            }
        }
        // cache.rs:291-331 ensure + span per layer
        for (int li = 0; li < L; ++li) {
            const int cap = b->cap[li];
            int &slots = sh.slots[li];
            if (!(pos < slots || slots >= cap)) {
                int want = slots * 2 > pos + 1 ? slots * 2 : pos + 1;
                slots = want < cap ? want : cap;
            }
            const int window = is_global(c, li) ? 0 : c.sliding_window;
            int lo = (window && pos + 1 > window) ? pos + 1 - window : 0;
            const int clamp = pos + 1 > slots ? pos + 1 - slots : 0;
            h_lo[size_t(li) * B + i] = lo > clamp ? lo : clamp;
        }
    }
    // this step's rows only: the buffer is sized for a full pass of max_chunk
    const size_t used = size_t(B) * (3 + L + nt) * 4;
    ND_HIP(hipMemcpyAsync(b->step_dev, b->stage_host[stage], used, hipMemcpyHostToDevice,
                          ctx->stream));
    tok_dev = static_cast<int32_t *>(b->step_dev);
    pos_dev = tok_dev + B;
    hi_dev = tok_dev + 2 * B;
    lo_dev = tok_dev + 3 * B;
    rows_dev = tok_dev + 3 * B + size_t(L) * B;
    ND_HIP(hipEventRecord(b->stage_done[stage], ctx->stream));
    b->stage_pending[stage] = true;
    b->stage_next = (stage + 1) % nd_v3_batch::kStages;
    st = ctx->stream;
    if (dev_tokens) {
        // the tokens, history and Engram rows from the previous step's choices
        ND_REQUIRE(c.n_orders <= kMaxOrders, "%d Engram orders", int(c.n_orders));
        StepTokens a{b->next, pos_dev, tok_dev, b->hist_dev, rows_dev, S, mo, int(c.vocab_size),
                     int(c.n_orders), int(c.e_heads),
                     int(c.e_seed_heads == 0 ? c.e_heads : c.e_seed_heads), int(c.e_slots), {}};
        for (int oi = 0; oi < c.n_orders; ++oi) a.orders[oi] = c.orders[oi];
        hipLaunchKernelGGL(k_step_tokens, dim3(unsigned((S + 63) / 64)), dim3(64), 0, st, a);
        if (int rc = nd::check_launch("k_step_tokens")) return rc;
    }
    qk_scale = 1.0f / std::sqrt(float(c.qk_head_dim));
    kf = b->kv_f32 ? 1 : 0;
    gate_fused = c.v_head_dim == 64 && m->pre_attn.group == 128 &&
                 m->pre_attn.in_padded == od && m->layers[0].out->per_byte != 0;
    phi = m->phi_pre;
    // The scatter-up gates ride in the layer's launches (k_layer_in's phi
    // rows, second workgroups of k_qkv_kv and k_post_hada) for single
    // positions when the phi weights fit; else (and for prefill passes)
    // they run on the side stream, joined by events.
    fpo = m->phi_post;
    fre = m->phi_res;
    gates_in = (phi->per_byte == 2 || phi->per_byte == 4) && phi->group == 128 &&
                  fpo->per_byte == phi->per_byte && fre->per_byte == phi->per_byte &&
                  fpo->group == 128 && fre->group == 128 &&
                  fpo->in_padded == phi->in_padded && fre->in_padded == phi->in_padded &&
                  size_t(2 * nl + nl * nl) * phi->num_groups <= size_t(kMaxPhiPairs) &&
                  size_t(2 * nl + nl * nl) * phi->num_groups <=
                      size_t((kMaxPhiPairs + kLayerInThreads - 1) / kLayerInThreads * kLayerInThreads) &&
                  nl * nl <= 64 && fpo->row_bytes % 16 == 0 && fre->row_bytes % 16 == 0 &&
                  C == 1;
    ev_conv = C == 1 ? b->ev : b->evc;
    return ND_OK;
}

#define CK(call) \
    if ((rc = (call))) return rc;
#define LCHK(name) \
    if ((rc = nd::check_launch(name))) return rc;

int StepRun::enqueue(int phase, bool argmax)
{
    const nd_v3_cfg &c = m->cfg;
    hipStream_t side = b->side;
    int rc = ND_OK;
    if (phase < 0) {
        // ---- Engram for this position (model.rs:162-191) -------------------------
        // the prepared key inputs of every site: one fused fetch when every
        // table row is one 128-wide group feeding the key's 128-groups
        const size_t fstride = size_t(B) * b->fh_width;
        bool fused = c.n_sites > 0;
        for (int s = 0; s < c.n_sites && fused; ++s) {
            const nd_cq *t = m->sites[s].tables, *k = m->sites[s].key, *t0 = m->sites[0].tables;
            fused = t->group == 128 && t->in_feat == 128 && t->num_groups == 1 && k->group == 128 &&
                    k->in_feat == size_t(nt) * 128 && k->in_padded == size_t(nt) * 128 &&
                    t->out_feat == t0->out_feat && t->row_bytes == t0->row_bytes &&
                    t->bits == t0->bits && t->per_byte != 0 && t->inv_sqrt_group == t0->inv_sqrt_group &&
                    k->inv_sqrt_group == m->sites[0].key->inv_sqrt_group;
        }
        if (fused) {
            for (int s0 = 0; s0 < c.n_sites; s0 += kMaxSitesLaunch) {
                const int ns = c.n_sites - s0 < kMaxSitesLaunch ? c.n_sites - s0 : kMaxSitesLaunch;
                const nd_cq *t0 = m->sites[s0].tables;
                EngramFetch ef{};
                for (int j = 0; j < ns; ++j) {
                    const nd_cq *t = m->sites[s0 + j].tables;
                    ef.packed[j] = t->packed;
                    ef.norms[j] = t->norms;
                    ef.lv[j] = t->lv;
                    ef.fh[j] = b->fh + size_t(s0 + j) * fstride;
                }
                ef.rows = rows_dev;
                ef.out_feat = int(t0->out_feat);
                ef.row_bytes = int(t0->row_bytes);
                ef.w = t0->bits == 5 ? 2 : int(t0->bits);
                ef.ternary = t0->bits == 5;
                ef.count = B * nt;
                ef.sites = ns;
                ef.inv_t = t0->inv_sqrt_group;
                ef.inv_k = m->sites[s0].key->inv_sqrt_group;
                const int waves = ns * B * nt;
                hipLaunchKernelGGL(k_engram_fetch, dim3((waves + 3) / 4), dim3(256), 0, st, ef);
                LCHK("k_engram_fetch");
            }
        } else {
            for (int s = 0; s < c.n_sites; ++s) {
                const Site &site = m->sites[s];
                CK(nd_cq_dequantize_rows(ctx, site.tables, rows_dev, size_t(B) * nt, b->fetched));
                CK(nd_cq_prepare_input(ctx, site.key, b->fetched, B, b->fh + size_t(s) * fstride));
            }
        }
        // every site's key and value projections, six sites a launch
        for (int s0 = 0; s0 < c.n_sites; s0 += 6) {
            const int ns = c.n_sites - s0 < 6 ? c.n_sites - s0 : 6;
            const nd_cq *ws[12];
            const float *xs[12];
            size_t r0[12], nr[12];
            float *ys[12];
            for (int j = 0; j < ns; ++j) {
                const Site &site = m->sites[s0 + j];
                const float *fh = b->fh + size_t(s0 + j) * fstride;
                ws[2 * j] = site.key;
                ws[2 * j + 1] = site.value;
                xs[2 * j] = xs[2 * j + 1] = fh;
                r0[2 * j] = r0[2 * j + 1] = 0;
                nr[2 * j] = nr[2 * j + 1] = size_t(d);
                ys[2 * j] = b->ek + size_t(s0 + j) * Rcap * d;
                ys[2 * j + 1] = b->ev + size_t(s0 + j) * Rcap * d;
            }
            CK(nd_cq_exact_multi(ctx, st, 2 * ns, ws, xs, size_t(B), r0, nr, ys, "v3 engram key/value"));
        }
        const int reach = (c.e_conv_taps - 1) * c.e_conv_dilation;
        if (C == 1) {
            for (int s0 = 0; s0 < c.n_sites; s0 += kMaxSitesLaunch) {
                const int ns = c.n_sites - s0 < kMaxSitesLaunch ? c.n_sites - s0 : kMaxSitesLaunch;
                EngramConv ec{};
                ec.ev = b->ev + size_t(s0) * Rcap * d;
                ec.site_stride = size_t(Rcap) * d;
                for (int j = 0; j < ns; ++j) {
                    ec.taps[j] = m->sites[s0 + j].taps;
                    ec.tail[j] = b->et[s0 + j];
                }
                hipLaunchKernelGGL(k_engram_conv, dim3((d + 255) / 256, B, ns), dim3(256), 0, st, ec,
                                   pos_dev, c.e_conv_taps, c.e_conv_dilation, mo, reach, d);
                LCHK("k_engram_conv");
            }
        }
        for (int s = 0; s < c.n_sites && C > 1; ++s) {
            const Site &site = m->sites[s];
            {
                hipLaunchKernelGGL(k_engram_conv_rows, dim3((d + 255) / 256, B), dim3(256), 0, st,
                                   b->ev + size_t(s) * Rcap * d, b->evc + size_t(s) * Rcap * d,
                                   site.taps, b->et[s], pos_dev, c.e_conv_taps, c.e_conv_dilation, mo,
                                   reach, d, C);
                LCHK("k_engram_conv_rows");
                hipLaunchKernelGGL(k_tails, dim3((d + 255) / 256, S), dim3(256), 0, st,
                                   b->ev + size_t(s) * Rcap * d, b->et[s], reach, C, d);
                LCHK("k_tails");
            }
        }
        // ---- lane stream (model.rs:194-203) --------------------------------------
        CK(nd_cq_dequantize_rows(ctx, m->embedding, tok_dev, size_t(B), b->emb));
        hipLaunchKernelGGL(k_embed, dim3((d + 255) / 256, B), dim3(256), 0, st, b->emb, b->lanes,
                           m->embed_scale, nl, d);
        LCHK("k_embed");

        return ND_OK;
    }
    if (phase < L) {
        const int li = phase;
        const Layer &l = m->layers[li];
        const int site = site_of(c, li);
        // previous layer's scatter up + this layer's mix down
        if (li > 0 && !gates_in) ND_HIP(hipStreamWaitEvent(st, b->ev_gates[(li - 1) & 1], 0));
        LayerIn in{b->lanes, b->y, b->gp, b->gr, li > 0, b->nxh, m->pre_nx, phi->packed,
                   phi->norms, phi->lv, phi->row_bytes, int(phi->num_groups), li * nl,
                   int(phi->bits == 5), m->b_pre + size_t(li) * nl, m->a_pre[li], li, nl, d,
                   gates_in ? 1 : 0, fpo->packed, fre->packed, fpo->norms, fre->norms, fpo->lv, fre->lv,
                   fpo->row_bytes, fre->row_bytes, li * nl, li * nl * nl, int(fpo->bits == 5),
                   int(fre->bits == 5), b->graw,
                   site >= 0 ? b->ek + size_t(site) * Rcap * d : nullptr,
                   site >= 0 ? ev_conv + size_t(site) * Rcap * d : nullptr, l.norm_in, b->u, b->bx,
                   b->hh, m->pre_h};
        if (phi->per_byte == 2)
            hipLaunchKernelGGL((k_layer_in<2, kLayerInThreads>), dim3(B), dim3(kLayerInThreads), 0, st, in);
        else
            hipLaunchKernelGGL((k_layer_in<4, kLayerInThreads>), dim3(B), dim3(kLayerInThreads), 0, st, in);
        LCHK("k_layer_in");
        if (!gates_in) {
            // side stream: this layer's scatter-up gates from the prepared lanes
            ND_HIP(hipEventRecord(b->ev_in[li & 1], st));
            ND_HIP(hipStreamWaitEvent(side, b->ev_in[li & 1], 0));
            {
                const nd_cq *ws[2] = {m->phi_post, m->phi_res};
                const size_t r0[2] = {size_t(li) * nl, size_t(li) * nl * nl};
                const size_t nr[2] = {size_t(nl), size_t(nl) * nl};
                float *ys[2] = {b->hpost, b->hres};
                CK(nd_cq_exact_set(ctx, side, 2, ws, b->nxh, size_t(B), r0, nr, ys, "v3 phi post/res"));
            }
            MhcGates mg{b->hpost, b->hres, m->b_post + size_t(li) * nl,
                        m->b_res + size_t(li) * nl * nl, m->a_post[li], m->a_res[li], li, nl,
                        b->gp, b->gr};
            hipLaunchKernelGGL(k_mhc_gates, dim3(B), dim3(64), 0, side, mg);
            LCHK("k_mhc_gates");
            ND_HIP(hipEventRecord(b->ev_gates[li & 1], side));
        }
        // q, k, v and gate projections of the prepared h, one launch
        {
            const nd_cq *ws[4] = {l.q, l.k, l.v, l.gate};
            const size_t r0[4] = {0, 0, 0, 0};
            const size_t nr[4] = {size_t(qd), size_t(kd), size_t(vd), size_t(od)};
            float *ys[4] = {b->q, b->k, b->v, b->gate};
            CK(nd_cq_exact_set(ctx, st, 4, ws, b->hh, size_t(B), r0, nr, ys, "v3 qkv/gate"));
        }
        // this layer's scatter-up gates, when they ride in the layer's launches
        MhcIn mi{};
        if (gates_in) {
            mi.on = 1;
            mi.graw = b->graw;
            mi.n = nl;
            mi.layer = li;
            mi.split = kGateSplit;
            mi.b_post = m->b_post + size_t(li) * nl;
            mi.b_res = m->b_res + size_t(li) * nl * nl;
            mi.a_post = m->a_post[li];
            mi.a_res = m->a_res[li];
            mi.gp = b->gp;
            mi.gr = b->gr;
            mi.state = b->gstate;
        }
        const unsigned gy = gates_in ? 2u : 1u;
        const nd_kv_geom &g = b->geom[li];
        QkvKv qk{b->q, b->k, b->v, b->qt[li], b->kt[li], b->vt[li], l.q_taps, l.k_taps,
                 l.v_taps, l.q_norm, l.k_norm, m->rope_tab, pos_dev, qd, kd, vd,
                 c.qkv_conv_taps, c.num_heads, c.num_kv_heads, c.qk_head_dim, c.v_head_dim,
                 b->kv[li], b->kv_stride[li], nd_kv_v_offset(&g), nd_kv_ks_offset(&g),
                 nd_kv_vs_offset(&g), g.cap, C, b->qn};
        if (kf) qk.v_off = nd_kv_f32_v_offset(&g);
        // a decode step over the int8 ring with the gated epilogue forms its
        // q, k and v inside the attention launch (k_attn_step)
        const bool step_attn = C == 1 && !kf && gate_fused && c.qk_head_dim % 16 == 0 &&
                               c.qk_head_dim <= 64 && c.v_head_dim == 64 &&
                               c.qkv_conv_taps <= 4 && g.cap <= ndattn::kAttn2MaxCap &&
                               qd + kd + vd <= 1024 && B <= 65535;
        if (step_attn) mi.split = kGateSplitAttn;
        // conv, norm + RoPE, int8 KV append
        if (!step_attn) {
            const dim3 qg(unsigned(B), gy);
            if (C == 1) {
                if (kf)
                    hipLaunchKernelGGL((k_qkv_kv<false, true, kQkvThreads>), qg, dim3(kQkvThreads), 0, st, qk, mi);
                else
                    hipLaunchKernelGGL((k_qkv_kv<false, false, kQkvThreads>), qg, dim3(kQkvThreads), 0, st, qk, mi);
                LCHK("k_qkv_kv");
            } else {
                // prefill passes run the gates on the side stream
                if (kf)
                    hipLaunchKernelGGL((k_qkv_kv<true, true, kQkvThreads>), dim3(B), dim3(kQkvThreads), 0, st, qk, mi);
                else
                    hipLaunchKernelGGL((k_qkv_kv<true, false, kQkvThreads>), dim3(B), dim3(kQkvThreads), 0, st, qk, mi);
                LCHK("k_qkv_kv");
                const int tt = c.qkv_conv_taps - 1;
                if (tt > 0) {
                    hipLaunchKernelGGL(k_tails, dim3((qd + 255) / 256, S), dim3(256), 0, st, b->q,
                                       b->qt[li], tt, C, qd);
                    hipLaunchKernelGGL(k_tails, dim3((kd + 255) / 256, S), dim3(256), 0, st, b->k,
                                       b->kt[li], tt, C, kd);
                    hipLaunchKernelGGL(k_tails, dim3((vd + 255) / 256, S), dim3(256), 0, st, b->v,
                                       b->vt[li], tt, C, vd);
                    LCHK("k_tails");
                }
            }
        }
        // attention over the int8 ring (query fake-quant fused); with
        // 64-wide heads and 128-wide groups its epilogue also applies
        // the sigmoid gate and the butterfly stages inside each head,
        // and out_proj's load finishes prepare_input
        if (step_attn) {
            const int R = c.num_heads / c.num_kv_heads;
            const size_t groups = size_t(B) * c.num_kv_heads;
            const size_t ablocks = 8 * size_t(R) * ((groups + 7) / 8);
            const size_t lds = size_t((g.cap + 3) & ~3) * 4 + 2 * ndattn::kProdBuf * sizeof(float);
            AttnStep as{qk, ndkv::make_geom(&g), lo_dev + size_t(li) * B, hi_dev, qk_scale,
                        b->attn, b->gate, int(groups), int(ablocks)};
            const dim3 ag(unsigned(ablocks + (gates_in ? size_t(B) : 0)));
            switch (c.qk_head_dim / 16) {
            case 1: hipLaunchKernelGGL((k_attn_step<1>), ag, dim3(ndattn::kAttn2Threads), lds, st, as, mi); break;
            case 2: hipLaunchKernelGGL((k_attn_step<2>), ag, dim3(ndattn::kAttn2Threads), lds, st, as, mi); break;
            case 3: hipLaunchKernelGGL((k_attn_step<3>), ag, dim3(ndattn::kAttn2Threads), lds, st, as, mi); break;
            default: hipLaunchKernelGGL((k_attn_step<4>), ag, dim3(ndattn::kAttn2Threads), lds, st, as, mi); break;
            }
            LCHK("k_attn_step");
            const size_t r0 = 0, nr = size_t(d);
            CK(nd_cq_exact_set(ctx, st, 1, &l.out, b->attn, size_t(B), &r0, &nr, &b->proj,
                               "v3 out projection", m->pre_attn.inv));
        } else if (gate_fused) {
            CK(nd_attend_exact_rows(ctx, &b->geom[li], b->kv[li], b->kv_stride[li], size_t(B), C,
                                    lo_dev + size_t(li) * B, hi_dev, C == 1 ? b->q : b->qn,
                                    qk_scale, kf ? 0 : 1, b->attn, b->gate, kf));
            const size_t r0 = 0, nr = size_t(d);
            CK(nd_cq_exact_set(ctx, st, 1, &l.out, b->attn, size_t(B), &r0, &nr, &b->proj,
                               "v3 out projection", m->pre_attn.inv));
        } else {
            CK(nd_attend_exact_rows(ctx, &b->geom[li], b->kv[li], b->kv_stride[li], size_t(B), C,
                                    lo_dev + size_t(li) * B, hi_dev, C == 1 ? b->q : b->qn,
                                    qk_scale, kf ? 0 : 1, b->attn, nullptr, kf));
            hipLaunchKernelGGL(k_gate_prep, dim3(B), dim3(kT), 0, st, b->attn, b->gate, b->ah, od,
                               m->pre_attn);
            LCHK("k_gate_prep");
            CK(project(ctx, l.out, b->ah, B, 0, d, b->proj));
        }
        HadaArgs ha{b->proj, l.post_norm, l.pre_hada, nd_sigmoidf(l.attn_gate), b->u, b->bx, b->y,
                    l.d1, l.d2, l.b2, l.d3, l.d4, l.w1a, l.w1b, l.w2a, l.w2b, l.w3a, l.w3b,
                    l.cond_v, l.cond_u, m->p1, m->p2, d, l.cond_rank};
        if (step_attn && c.qkv_conv_taps > 1) {
            ha.shift_taps = c.qkv_conv_taps;
            ha.sraw[0] = b->q;
            ha.sraw[1] = b->k;
            ha.sraw[2] = b->v;
            ha.stail[0] = b->qt[li];
            ha.stail[1] = b->kt[li];
            ha.stail[2] = b->vt[li];
            ha.sdim[0] = qd;
            ha.sdim[1] = kd;
            ha.sdim[2] = vd;
        }
        hipLaunchKernelGGL(k_post_hada, dim3(unsigned(B), gy), dim3(1024), 0, st, ha, mi);
        LCHK("k_post_hada");
        return ND_OK;
    }
    // ---- head ---------------------------------------------------------------
    if (!gates_in) ND_HIP(hipStreamWaitEvent(st, b->ev_gates[(L - 1) & 1], 0));
    hipLaunchKernelGGL(k_final, dim3(S), dim3(kT), 0, st, b->lanes, b->y, b->gp, b->gr,
                       m->final_norm, b->xh, nl, d, m->pre_x, C);
    LCHK("k_final");
    CK(project(ctx, m->embedding, b->xh, S, 0, rows, b->logits));
    if (argmax) {
        hipLaunchKernelGGL(k_argmax, dim3(S), dim3(kT), 0, st, b->logits, int(rows), b->next,
                           argmax_also);
        LCHK("k_argmax");
    }
    return ND_OK;
}

// A whole step of one batch: begin, every phase (eagerly, or replayed from
// a captured graph), then the copies out and, with `next`, the wait.
int step_impl(nd_ctx *ctx, const nd_v3_model *m, nd_v3_batch *b, const int32_t *tokens, int C,
              int32_t *next, float *logits)
{
    // the context and the batch belong to this thread for the whole step
    ND_ENTER(ctx);
    ND_REQUIRE(b, "null batch");
    nd::Hold hold(b->owner, "the batch");
    if (hold.rc) return hold.rc;
    StepRun r{ctx, m, b, C};
    if (int rc = r.begin(tokens)) return rc;
    const int S = r.S, L = r.L;
    const size_t rows = r.rows;
    hipStream_t st = r.st;
    auto enqueue = [&](bool argmax) -> int {
        for (int ph = -1; ph <= L; ++ph)
            if (int rc = r.enqueue(ph, argmax)) return rc;
        return ND_OK;
    };
    // One position per session, graphs on: replay the captured step on the
    // batch's own stream (a capture needs a stream of its own: the caller's
    // may be the null stream), fenced to the caller's stream by events.  The
    // capture is taken on the second such step; if it cannot be taken, the
    // batch runs eagerly from then on.
    const bool graph = C == 1 && b->graphs;
    const bool argmax = next != nullptr || graph;
    const hipStream_t user = st;
    bool replayed = false;
    if (graph && (b->graph_exec || b->eager_steps > 0)) {
        if (!b->gstream) {
            ND_HIP(hipStreamCreateWithFlags(&b->gstream, hipStreamNonBlocking));
            ND_HIP(hipEventCreateWithFlags(&b->g_in, hipEventDisableTiming));
            ND_HIP(hipEventCreateWithFlags(&b->g_out, hipEventDisableTiming));
        }
        ND_HIP(hipEventRecord(b->g_in, user));
        ND_HIP(hipStreamWaitEvent(b->gstream, b->g_in, 0));
        if (!b->graph_exec) {
            st = b->gstream;
            ctx->stream = b->gstream;
            r.st = st;
            const hipError_t be = hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed);
            const int crc = be == hipSuccess ? enqueue(true) : ND_ERR_HIP;
            hipGraph_t g = nullptr;
            const hipError_t ce = be == hipSuccess ? hipStreamEndCapture(st, &g) : be;
            ctx->stream = user;
            st = user;
            r.st = st;
            hipGraphExec_t ex = nullptr;
            const bool ok = crc == ND_OK && ce == hipSuccess && g &&
                            hipGraphInstantiate(&ex, g, nullptr, nullptr, 0) == hipSuccess;
            if (g) (void)hipGraphDestroy(g);
            if (ok) {
                b->graph_exec = ex;
            } else {
                // nothing was enqueued: this step and every later one run eagerly
                b->graphs = false;
                (void)hipGetLastError();
                nd::clear_error();
            }
        }
        if (b->graph_exec) {
            ND_HIP(hipGraphLaunch(b->graph_exec, b->gstream));
            ND_HIP(hipEventRecord(b->g_out, b->gstream));
            ND_HIP(hipStreamWaitEvent(user, b->g_out, 0));
            replayed = true;
        }
    }
    if (!replayed) {
        if (int rc = enqueue(argmax)) return rc;
        if (C == 1) ++b->eager_steps;
    }
    if (logits)
        ND_HIP(hipMemcpyAsync(logits, b->logits, size_t(S) * rows * 4, hipMemcpyDeviceToDevice, st));
    if (next) {
        ND_HIP(hipMemcpyAsync(b->next_host, b->next, size_t(S) * 4, hipMemcpyDeviceToHost, st));
        ND_HIP(hipStreamSynchronize(st));
        std::memcpy(next, b->next_host, size_t(S) * 4);
    }
    for (int i = 0; i < S; ++i) b->s[i].pos += C;
    return ND_OK;
}

#undef CK
#undef LCHK

}  // namespace

extern "C" {

int nd_v3_step(nd_ctx *ctx, const nd_v3_model *m, nd_v3_batch *b, const int32_t *tokens,
               int32_t *next, float *logits)
{
    return step_impl(ctx, m, b, tokens, 1, next, logits);
}

int nd_v3_prefill(nd_ctx *ctx, const nd_v3_model *m, nd_v3_batch *b, const int32_t *tokens,
                  size_t count, int32_t *next, float *logits)
{
    nd::clear_error();
    ND_REQUIRE(count >= 1 && count <= 256, "count %zu out of 1..256", count);
    return step_impl(ctx, m, b, tokens, int(count), next, logits);
}

}  // extern "C"

namespace {

// nd_v3_generate in three parts, so that several batches' loops can be
// enqueued step by step in turn (nd_v3_generate_many).  The caller holds
// the context and the batch.
int gen_begin(nd_ctx *ctx, const nd_v3_model *m, nd_v3_batch *b, const int32_t *first, size_t steps)
{
    ND_REQUIRE(m && b && first, "null argument");
    const int S = b->B;
    ND_REQUIRE(b->chunk >= 1, "batch without steps");
    for (int i = 0; i < S; ++i)
        ND_REQUIRE(size_t(b->s[i].pos) + steps <= size_t(b->max_len), "session %d: %zu steps from "
                   "position %d pass its %d positions", i, steps, b->s[i].pos, b->max_len);
    const int mo = max_order(m->cfg);
    const size_t n_out = steps * size_t(S);
    if (n_out > b->gen_cap) {
        ND_HIP(hipStreamSynchronize(ctx->stream));
        if (b->gen_out) ND_HIP(hipFree(b->gen_out));
        b->gen_out = nullptr;
        b->gen_cap = 0;
        ND_HIP(hipMalloc(&b->gen_out, n_out * sizeof(int32_t)));
        b->gen_cap = n_out;
    }
    // the first tokens, and each session's retained ids, right-aligned; the
    // host buffer lives in the batch until the loop's tokens come back
    std::vector<int32_t> &init = b->gen_init;
    init.assign(size_t(S) * (1 + mo), 0);
    for (int i = 0; i < S; ++i) {
        init[i] = first[i];
        const std::vector<uint32_t> &hv = b->s[i].hist;
        const int n = int(hv.size()) < mo ? int(hv.size()) : mo;
        for (int j = 0; j < n; ++j)
            init[S + size_t(i) * mo + (mo - n + j)] = int32_t(hv[hv.size() - n + j]);
    }
    ND_HIP(hipMemcpyAsync(b->next, init.data(), size_t(S) * 4, hipMemcpyHostToDevice, ctx->stream));
    ND_HIP(hipMemcpyAsync(b->hist_dev, init.data() + S, size_t(S) * mo * 4, hipMemcpyHostToDevice,
                          ctx->stream));
    return ND_OK;
}

// Step k of the loop: enqueued, nothing waited for (the host runs ahead of
// the device up to the staging ring's depth).
int gen_step(nd_ctx *ctx, const nd_v3_model *m, nd_v3_batch *b, size_t k)
{
    const int S = b->B;
    StepRun r{ctx, m, b, 1};
    r.argmax_also = b->gen_out + k * S;
    int rc = r.begin(nullptr);
    for (int ph = -1; ph <= r.L && rc == ND_OK; ++ph) rc = r.enqueue(ph, true);
    if (rc == ND_OK)
        for (int i = 0; i < S; ++i) b->s[i].pos += 1;
    return rc;
}

// The tokens back to the host, and the host's copy of the retained ids.
int gen_end(nd_ctx *ctx, const nd_v3_model *m, nd_v3_batch *b, const int32_t *first, size_t steps,
            int32_t *tokens)
{
    const int S = b->B;
    const int mo = max_order(m->cfg);
    const size_t n_out = steps * size_t(S);
    std::vector<int32_t> got(n_out);
    ND_HIP(hipMemcpyAsync(got.data(), b->gen_out, n_out * 4, hipMemcpyDeviceToHost, ctx->stream));
    ND_HIP(hipStreamSynchronize(ctx->stream));
    for (int i = 0; i < S; ++i) {
        // the tokens the steps fed
        std::vector<uint32_t> &hv = b->s[i].hist;
        for (size_t k = 0; k < steps; ++k) {
            hv.push_back(uint32_t(k == 0 ? first[i] : got[(k - 1) * S + i]));
            if (int(hv.size()) > mo) hv.erase(hv.begin());
            tokens[size_t(i) * steps + k] = got[k * S + i];
        }
    }
    return ND_OK;
}

constexpr size_t kMaxGenBatches = 8;

}  // namespace

extern "C" {

int nd_v3_generate(nd_ctx *ctx, const nd_v3_model *m, nd_v3_batch *b, const int32_t *first,
                   size_t steps, int32_t *tokens)
{
    ND_ENTER(ctx);
    ND_REQUIRE(m && b && first && tokens, "null argument");
    nd::Hold hold(b->owner, "the batch");
    if (hold.rc) return hold.rc;
    if (steps == 0) return ND_OK;
    if (int rc = gen_begin(ctx, m, b, first, steps)) return rc;
    for (size_t k = 0; k < steps; ++k)
        if (int rc = gen_step(ctx, m, b, k)) return rc;
    return gen_end(ctx, m, b, first, steps, tokens);
}

int nd_v3_generate_many(nd_ctx *const *ctxs, const nd_v3_model *m, nd_v3_batch *const *bs,
                        size_t n, const int32_t *const *first, size_t steps,
                        int32_t *const *tokens)
{
    nd::clear_error();
    ND_REQUIRE(ctxs && m && bs && first && tokens, "null argument");
    ND_REQUIRE(n >= 1 && n <= kMaxGenBatches, "%zu batches (1..%zu)", n, kMaxGenBatches);
    for (size_t i = 0; i < n; ++i) {
        ND_REQUIRE(ctxs[i] && bs[i] && first[i] && tokens[i], "batch %zu: null argument", i);
        for (size_t j = 0; j < i; ++j)
            ND_REQUIRE(ctxs[j] != ctxs[i] && bs[j] != bs[i], "batch %zu repeats a context or a batch", i);
    }
    std::vector<std::unique_ptr<nd::Entry>> entries;
    std::vector<std::unique_ptr<nd::Hold>> holds;
    for (size_t i = 0; i < n; ++i) {
        entries.emplace_back(new nd::Entry(ctxs[i]));
        if (entries.back()->rc) return entries.back()->rc;
        holds.emplace_back(new nd::Hold(bs[i]->owner, "the batch"));
        if (holds.back()->rc) return holds.back()->rc;
    }
    if (steps == 0) return ND_OK;
    for (size_t i = 0; i < n; ++i)
        if (int rc = gen_begin(ctxs[i], m, bs[i], first[i], steps)) return rc;
    // step k of every batch before step k + 1 of any: each batch's launches
    // go to its own stream, so one batch's single-workgroup-per-session
    // kernels run beside another's wide ones
    for (size_t k = 0; k < steps; ++k)
        for (size_t i = 0; i < n; ++i)
            if (int rc = gen_step(ctxs[i], m, bs[i], k)) return rc;
    for (size_t i = 0; i < n; ++i)
        if (int rc = gen_end(ctxs[i], m, bs[i], first[i], steps, tokens[i])) return rc;
    return ND_OK;
}


}  // extern "C"
