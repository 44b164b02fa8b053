// Exact parallel evaluation of a sequential float fold over non-negative
// terms: s = ((0 + a[0]) + a[1]) + ... + a[n-1], every add rounded to
// nearest-even in fp32, in index order, with the same bits as the loop.
//
// The reference folds its norms' sums of squares and softmax sums as one
// sequential chain (e.g. kernels.rs:33-41, norm.rs:23-30, attention.rs:356).
// Run as a chain on one thread, a 3072-term fold costs some 20k cycles of
// dependent adds.  The method below gets the same bits from mostly parallel
// work:
//
//  1. For non-negative terms the partial sums s_i are non-decreasing and the
//     rounding error of step j is at most 2^-24 s_{j+1}, so
//     |s_i - S_i| <= i 2^-24 s_i, with S_i the exact prefix sum.  A parallel
//     fp32 prefix P_i approximates S_i to a relative (depth) 2^-24.  Hence
//     s_i lies in [P_i (1 - d), P_i (1 + d)] for d = (n + 4c + 128) 2^-23
//     (c: terms per thread), and when both ends share a binade, so does s_i.
//  2. Inside one binade of exponent G the floats are the multiples k u of
//     u = 2^(G-150) (zero and the subnormals with binade 1, all on the 2^-149
//     grid).  A step s -> RN(s + a) whose input and result are both known to
//     be in binade G is exactly s + r u with r = a / u rounded to the nearest
//     integer -- unless a / u is an exact tie (x.5), whose result depends on
//     k's parity.  So a run of consecutive in-binade, tie-free steps adds
//     D u, D = the sum of its r (integers below 2^24, summed exactly in
//     fp32), and D u added to the run's true start is exact.
//  3. The steps near a binade crossing (where the bounds of step 1 straddle
//     a power of two) and the ties stay ordinary fp32 adds.
// The folded sequence -- a few dozen items, crossing terms and run sums --
// is then one short sequential chain.  Terms that are negative, -0, not finite,
// or large enough to risk overflow, and any case that exceeds the scratch
// sizes, take the plain sequential loop instead.
//
// The arithmetic helpers are shared by host and device code, so the CPU
// tests check the same functions the kernels use.
#pragma once

#include "nd_libm.h"

#include <math.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define ND_FOLD_FN __host__ __device__ __forceinline__
#else
#define ND_FOLD_FN static inline
#endif

// Binade of a value x >= 0: its biased exponent, with zero and the
// subnormals in binade 1 (both lie on the 2^-149 grid).
ND_FOLD_FN int nd_fold_cls(float x)
{
    const int e = int(nd_f2u(x) >> 23);
    return e < 1 ? 1 : e;
}

// r = a / u rounded to the nearest integer, u = 2^(G-150), for a term
// a >= +0; true when s -> RN(s + a), for s and the result in binade G, is
// exactly s + r u: a / u is not a tie and a alone stays inside the binade.
// a / u is exact (a power-of-two scaling) wherever it matters: below 2^-126
// it may round, but then r = 0 either way.  G = 0 gives false.
ND_FOLD_FN bool nd_fold_units(float a, int G, float &r)
{
    const float t = ldexpf(a, 150 - G);
    r = rintf(t);
    return t < 0x1p24f && t - floorf(t) != 0.5f;
}

// The relative half-width of the bounds on s_i (step 1 above).
ND_FOLD_FN float nd_fold_delta(int n, int c) { return float(n + 4 * c + 128) * 0x1p-23f; }

// Certain binade of the partial sum whose prefix estimate is P (>= 0), or
// 0 when the bounds straddle a power of two.
ND_FOLD_FN int nd_fold_point_cls(float P, float cm, float cp)
{
    const int lo = nd_fold_cls(P * cm), hi = nd_fold_cls(P * cp);
    return lo == hi ? lo : 0;
}

// D * 2^(G-150), exact: D < 2^24 is an integer, and the product is a
// multiple of the binade's grid (a subnormal or normal float).
ND_FOLD_FN float nd_fold_scale(float D, int G) { return ldexpf(D, G - 150); }

#if defined(__HIPCC__)

// ---- device: the first NT threads of a workgroup fold n terms ---------------

constexpr int kNdFoldItems = 512;   // folded-sequence capacity (more: plain loop)
constexpr int kNdFoldMinN = 128;    // shorter folds: plain loop

template <int NT>
struct NdFoldLds {
    __align__(16) float items[kNdFoldItems];
    float wtot[NT / 64];    // per wave: sum of its chunk totals
    int wflags[NT / 64];    // per wave: its run carry (NdFoldCarry)
    float wD[NT / 64];
    int wcnt[NT / 64];      // per wave: items of its lanes, lane 0's carried run aside
    int wfirst[NT / 64];    // per wave: lane 0's chunk starts with a crossing term
};

// The run a span of chunks leaves open, as seen by the chunk after it.
// flags: bit 0 (kind) the span has a crossing term, so the run open after
// it starts inside it; bit 1 (ex) a run is open at its end; bits 2+ the
// run's binade.  D: the run's sum of units (exact integer below 2^24).  An
// all-in-binade span extends the run open before it; an empty one passes
// it through.
struct NdFoldCarry {
    int flags;
    float D;
};

// a's span, then b's.
__device__ __forceinline__ NdFoldCarry nd_fold_then(NdFoldCarry a, NdFoldCarry b)
{
    const bool bkind = b.flags & 1, bex = (b.flags >> 1) & 1, aex = (a.flags >> 1) & 1;
    NdFoldCarry r;
    r.flags = bkind ? b.flags : (bex ? ((a.flags & 1) | 2 | (b.flags & ~3)) : a.flags);
    r.D = bkind ? b.D : (bex ? (aex ? a.D + b.D : b.D) : a.D);
    return r;
}

// Lane l - k's value within each 16-lane row (row_shr:k), the last lane of
// the previous row (row_bcast:15) or of lanes 0-31 (row_bcast:31), lane
// l - 1 of the wave (wave_shr:1) or lane l + 1 (wave_shl:1); 0 where there
// is none.
template <int CTRL, int ROWS>
__device__ __forceinline__ int nd_dpp(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xf, false);
}

template <int CTRL, int ROWS>
__device__ __forceinline__ float nd_dppf(float v)
{
    return nd_u2f(uint32_t(nd_dpp<CTRL, ROWS>(int(nd_f2u(v)))));
}

template <int CTRL, int ROWS>
__device__ __forceinline__ NdFoldCarry nd_dpp(NdFoldCarry x)
{
    return NdFoldCarry{nd_dpp<CTRL, ROWS>(x.flags), nd_dppf<CTRL, ROWS>(x.D)};
}

// Inclusive scans over a wave of 64 lanes in six steps: Hillis-Steele
// inside each row of 16, then the rows' totals carried forward.
__device__ __forceinline__ float nd_fold_scan_add(float v)
{
    v += nd_dppf<0x111, 0xf>(v);
    v += nd_dppf<0x112, 0xf>(v);
    v += nd_dppf<0x114, 0xf>(v);
    v += nd_dppf<0x118, 0xf>(v);
    v += nd_dppf<0x142, 0xa>(v);
    v += nd_dppf<0x143, 0xc>(v);
    return v;
}

__device__ __forceinline__ int nd_fold_scan_int(int v)
{
    v += nd_dpp<0x111, 0xf>(v);
    v += nd_dpp<0x112, 0xf>(v);
    v += nd_dpp<0x114, 0xf>(v);
    v += nd_dpp<0x118, 0xf>(v);
    v += nd_dpp<0x142, 0xa>(v);
    v += nd_dpp<0x143, 0xc>(v);
    return v;
}

__device__ __forceinline__ NdFoldCarry nd_fold_scan_carry(NdFoldCarry f)
{
    f = nd_fold_then(nd_dpp<0x111, 0xf>(f), f);
    f = nd_fold_then(nd_dpp<0x112, 0xf>(f), f);
    f = nd_fold_then(nd_dpp<0x114, 0xf>(f), f);
    f = nd_fold_then(nd_dpp<0x118, 0xf>(f), f);
    f = nd_fold_then(nd_dpp<0x142, 0xa>(f), f);
    f = nd_fold_then(nd_dpp<0x143, 0xc>(f), f);
    return f;
}

__device__ __forceinline__ float nd_fold_plain(const float *v, int n)
{
    float s = 0.0f;
    for (int i = 0; i < n; ++i) s += v[i];
    return s;
}

// ((0 + v[0]) + v[1]) + ... + v[n-1] with the loop's bits, for terms >= +0.
// Every thread of the workgroup calls it with the same v (written and
// synchronised) and n; its first NT threads (NT a multiple of 64, at most
// the workgroup) do the work, up to CMAX terms each (n <= NT * CMAX; more
// takes the plain loop).  Thread 0 gets the fold, the others an unspecified
// value.  With NT = 64 it has no workgroup barrier (threads past 64 return
// at once); otherwise every thread must call it.  L is free again after the
// caller's next barrier.
//
// Items are the crossing terms and the runs' sums D u, in sequence order;
// a run's item is written by the thread holding its last term, except that
// a run ending a wave's last chunk before a crossing term is written by the
// next wave's lane 0, so that each wave's item count is known after one
// barrier.
template <int NT, int CMAX>
__device__ __forceinline__ float nd_fold_nonneg(const float *v, int n, NdFoldLds<NT> &L)
{
    static_assert(NT % 64 == 0 && NT >= 64, "whole waves");
    static_assert(CMAX >= 1 && CMAX <= 32, "the run map holds one bit per term in 32 bits");
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int c = (n + NT - 1) / NT;
    if (n < kNdFoldMinN || c > CMAX) return tid == 0 ? nd_fold_plain(v, n) : 0.0f;
    if (NW == 1 && w > 0) return 0.0f;
    const int i0 = tid * c;
    const int len = tid >= NT ? 0 : (n - i0 < 0 ? 0 : (n - i0 < c ? n - i0 : c));

    // 1. chunk prefix, then the fp32 exclusive prefix of the chunk totals
    float x[CMAX], loc[CMAX];
    float p = 0.0f;
    bool bad = false;
#pragma unroll
    for (int j = 0; j < CMAX; ++j) {
        const int i = i0 + j < n ? i0 + j : n - 1;
        x[j] = j < len ? v[i] : 0.0f;
        bad |= nd_f2u(x[j]) >= 0x7f800000u;
        p += x[j];
        loc[j] = p;
    }
    bad |= !(p < 0x1p110f);
    const float incl = nd_fold_scan_add(p);
    const float lex = nd_dppf<0x138, 0xf>(incl);
    float base = 0.0f;
    if constexpr (NW > 1) {
        if (lane == 63 && w < NW) L.wtot[w] = incl;
        if (__syncthreads_or(bad)) return tid == 0 ? nd_fold_plain(v, n) : 0.0f;
        for (int k = 0; k < NW - 1; ++k) base += k < w ? L.wtot[k] : 0.0f;
    } else {
        if (__ballot(bad)) return tid == 0 ? nd_fold_plain(v, n) : 0.0f;
    }
    const float excl = base + lex;

    // 2. binade of every partial sum; the in-binade, tie-free steps and
    // their units; the chunk's runs and items
    const float dl = nd_fold_delta(n, c), cm = 1.0f - dl, cp = 1.0f + dl;
    int before = nd_fold_point_cls(excl, cm, cp);
    uint32_t inm = 0;
    float rr[CMAX];
    int gg[CMAX];
    float runD = 0.0f;
    int runG = 0, count = 0;
    bool open = false, any_bound = false, first_bound = false;
#pragma unroll
    for (int j = 0; j < CMAX; ++j) {
        const bool valid = j < len;
        const int after = nd_fold_point_cls(excl + loc[j], cm, cp);
        float r;
        const bool ok = nd_fold_units(x[j], before, r);
        const bool in = valid && ok && before != 0 && before == after;
        const bool bound = valid && !in;
        rr[j] = r;
        gg[j] = before;
        inm |= in ? 1u << j : 0u;
        runD = in ? (open ? runD + r : r) : runD;
        runG = in ? before : runG;
        if (j == 0) first_bound = bound;
        count += bound ? (open ? 2 : 1) : 0;  // the local run it closes, and the term
        any_bound |= bound;
        open = in ? true : (bound ? false : open);
        before = valid ? after : before;
    }
    // the run this chunk ends with is written here when the sequence ends
    // or, inside a wave, the next chunk starts with a crossing term
    const bool holds_last = len > 0 && i0 + len == n;
    const bool next_first = nd_dpp<0x130, 0xf>(first_bound ? 1 : 0) != 0;
    const bool tail = open && (holds_last || (lane != 63 && next_first));
    count += tail ? 1 : 0;

    // 3. the run open at each chunk's start, and item offsets
    NdFoldCarry f{(any_bound ? 1 : 0) | (len > 0 && open ? 2 : 0) | (runG << 2), runD};
    const NdFoldCarry fin = nd_fold_scan_carry(f);
    NdFoldCarry cin = nd_dpp<0x138, 0xf>(fin);
    const int cincl = nd_fold_scan_int(count);
    const int cex = nd_dpp<0x138, 0xf>(cincl);
    int obase = 0, total, lead = 0;
    if constexpr (NW > 1) {
        if (lane == 63 && w < NW) {
            L.wflags[w] = fin.flags;
            L.wD[w] = fin.D;
            L.wcnt[w] = cincl;
        }
        if (lane == 0 && w < NW) L.wfirst[w] = first_bound ? 1 : 0;
        __syncthreads();
        // each wave's carry-in, its lane 0's carried run, its item count
        NdFoldCarry cw{0, 0.0f};
        total = 0;
        for (int k = 0; k < NW; ++k) {
            const int lk = k > 0 && L.wfirst[k] && ((cw.flags >> 1) & 1) ? 1 : 0;
            if (k == w) {
                cin = nd_fold_then(cw, cin);
                lead = lk;
                obase = total;
            }
            total += L.wcnt[k] + lk;
            cw = nd_fold_then(cw, NdFoldCarry{L.wflags[k], L.wD[k]});
        }
    } else {
        total = __builtin_amdgcn_readlane(cincl, 63);
    }
    if (total > kNdFoldItems) return tid == 0 ? nd_fold_plain(v, n) : 0.0f;

    // 4. the items
    int o = obase + lead + cex;
    if (lane == 0 && lead) L.items[obase] = nd_fold_scale(cin.D, cin.flags >> 2);
    bool run = (cin.flags >> 1) & 1, runl = false;
    float D = run ? cin.D : 0.0f;
    int G = cin.flags >> 2;
#pragma unroll
    for (int j = 0; j < CMAX; ++j) {
        if (j < len) {
            if ((inm >> j) & 1u) {
                D = run ? D + rr[j] : rr[j];
                run = runl = true;
                G = gg[j];
            } else {
                if (runl) L.items[o++] = nd_fold_scale(D, G);
                L.items[o++] = x[j];
                run = runl = false;
            }
        }
    }
    if (tail) L.items[o] = nd_fold_scale(D, G);
    if constexpr (NW > 1) __syncthreads();

    // 5. the folded sequence, in order, by thread 0
    if (tid != 0) return 0.0f;
    float s = 0.0f;
    int k = 0;
    const float4 *t4 = reinterpret_cast<const float4 *>(L.items);
    for (; k + 8 <= total; k += 8) {
        const float4 a = t4[k / 4], b = t4[k / 4 + 1];
        s += a.x;
        s += a.y;
        s += a.z;
        s += a.w;
        s += b.x;
        s += b.y;
        s += b.z;
        s += b.w;
    }
    for (; k < total; ++k) s += L.items[k];
    return s;
}

#endif  // __HIPCC__
