// Internal entry points of the reference-order kernels for the Needle-3
// forward (not part of the C ABI).
#pragma once

#include "nd_cq_internal.h"

// n (<= 12) Cactus-Quants weights applied to the same prepared input xh
// ([batch][in_padded]) in one launch on `stream` when they share width,
// group and input size (else one launch each); y[k] receives rows[k] rows
// of weight k from row_start[k], batch-major ([batch][rows[k]]).
// Bit-identical to CqWeight::matvec_rows_prepared / matmul_rows_prepared
// per weight.
// half_inv != 0: xh holds each 128-group with butterfly stages 1..32 done
// (the gated attention epilogue's output); the load applies the last stage
// and the 1/sqrt(128) scale (half_inv), so the dots see prepare_input's bits.
int nd_cq_exact_set(nd_ctx *ctx, hipStream_t stream, int n, const nd_cq *const *w, const float *xh,
                    size_t batch, const size_t *row_start, const size_t *rows, float *const *y,
                    const char *what, float half_inv = 0.0f);

// As nd_cq_exact_set with an input of its own per weight (xhs[k],
// [batch][in_padded]), up to 12 weights: e.g. every Engram site's key and
// value projections in one launch.
int nd_cq_exact_multi(nd_ctx *ctx, hipStream_t stream, int n, const nd_cq *const *w,
                      const float *const *xhs, size_t batch, const size_t *row_start,
                      const size_t *rows, float *const *y, const char *what,
                      float half_inv = 0.0f);

// nd_attend_step_i8_exact with query row i reading the KV block of
// kv + (i / rows_per_block) * kv_stride: several positions of one session
// in one call.  With `gate` ([count][num_heads * 64], v_head_dim 64) each
// output column becomes attn * sigmoid(gate) with butterfly stages 1..32
// of its 128-wide group applied: the input nd_cq_exact_set finishes with
// half_inv (v3/model.rs:309-313, hadamard.rs:24-55).  kv_f32: the blocks
// are f32 KV blocks (nd_kv_f32_block_bytes) read through the f32 view, as
// nd_attend_step_f32_exact.
int nd_attend_exact_rows(nd_ctx *ctx, const nd_kv_geom *g, const void *kv, size_t kv_stride,
                         size_t count, int rows_per_block, const int32_t *lo, const int32_t *hi,
                         const float *q, float scale, int quant_query, float *out,
                         const float *gate = nullptr, int kv_f32 = 0);

// One 128-wide group of a Cactus-Quants row dotted with a prepared
// activation group in the reference's order (cq.rs:838-873): element e into
// lane e % 8, each lane a chain over the 16 elements it holds, the lanes
// summed 0..7.  P codes per byte (4: 2-bit or ternary crumbs, 2: 4-bit).
// cq_group_codes128 loads the group's 128 / P code bytes (16-byte aligned)
// into registers; cq_group_dot128 dots them, `lvl` mapping a code to its
// level (ternary crumbs already remapped), with the 128 activations `x`
// (16-byte aligned).
template <int P>
struct CqGroupCodes {
    static constexpr int W = 8 / P;
    static constexpr int PER_DW = 32 / W;
    static constexpr int NDW = 128 / PER_DW;
    uint32_t dw[NDW];
};

template <int P>
__device__ inline void cq_group_codes128(const uint8_t *codes, CqGroupCodes<P> &c)
{
#pragma unroll
    for (int k = 0; k < CqGroupCodes<P>::NDW; k += 4) {
        const uint4 c4 = *reinterpret_cast<const uint4 *>(codes + 4 * k);
        c.dw[k] = c4.x;
        c.dw[k + 1] = c4.y;
        c.dw[k + 2] = c4.z;
        c.dw[k + 3] = c4.w;
    }
}

template <int P>
__device__ inline float cq_group_dot128(const CqGroupCodes<P> &c, const float *lvl, const float *x)
{
    constexpr int W = CqGroupCodes<P>::W;
    constexpr uint32_t MASK = (1u << W) - 1;
    constexpr int PER_DW = CqGroupCodes<P>::PER_DW;
    float lanes[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t dw = c.dw[(i * 8) / PER_DW];
        const int sh = (i * 8 * W) & 31;
        const float4 xa = *reinterpret_cast<const float4 *>(x + i * 8);
        const float4 xb = *reinterpret_cast<const float4 *>(x + i * 8 + 4);
        lanes[0] += lvl[(dw >> sh) & MASK] * xa.x;
        lanes[1] += lvl[(dw >> (sh + W)) & MASK] * xa.y;
        lanes[2] += lvl[(dw >> (sh + 2 * W)) & MASK] * xa.z;
        lanes[3] += lvl[(dw >> (sh + 3 * W)) & MASK] * xa.w;
        lanes[4] += lvl[(dw >> (sh + 4 * W)) & MASK] * xb.x;
        lanes[5] += lvl[(dw >> (sh + 5 * W)) & MASK] * xb.y;
        lanes[6] += lvl[(dw >> (sh + 6 * W)) & MASK] * xb.z;
        lanes[7] += lvl[(dw >> (sh + 7 * W)) & MASK] * xb.w;
    }
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) acc += lanes[k];
    return acc;
}

// Lanes 2q and 2q + 1 (q < 4) of cq_group_dot128's eight, with its
// arithmetic: a quarter of the dot, for spreading one group over 4 threads.
template <int P>
__device__ inline void cq_group_quarter128(const CqGroupCodes<P> &c, const float *lvl, const float *x,
                                           int q, float &l0, float &l1)
{
    constexpr int W = CqGroupCodes<P>::W;
    constexpr uint32_t MASK = (1u << W) - 1;
    constexpr int PER_DW = CqGroupCodes<P>::PER_DW;
    l0 = 0.0f;
    l1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t dw = c.dw[(i * 8) / PER_DW];
        const int sh = ((i * 8 * W) & 31) + 2 * q * W;
        const float2 xv = *reinterpret_cast<const float2 *>(x + i * 8 + 2 * q);
        l0 += lvl[(dw >> sh) & MASK] * xv.x;
        l1 += lvl[(dw >> (sh + W)) & MASK] * xv.y;
    }
}

// acc += a[0].x; acc += a[0].y; ... acc += a[3].w: 16 dependent adds in one
// asm block, so the compiler can neither reorder the terms nor move LDS
// reads across the block (left to itself it hoists the next group's reads
// and copies this group's registers to make room).
__device__ __forceinline__ float nd_add16(float acc, const float4 (&a)[4])
{
    asm volatile(
        "v_add_f32 %0, %1, %0\n\tv_add_f32 %0, %2, %0\n\tv_add_f32 %0, %3, %0\n\t"
        "v_add_f32 %0, %4, %0\n\tv_add_f32 %0, %5, %0\n\tv_add_f32 %0, %6, %0\n\t"
        "v_add_f32 %0, %7, %0\n\tv_add_f32 %0, %8, %0\n\tv_add_f32 %0, %9, %0\n\t"
        "v_add_f32 %0, %10, %0\n\tv_add_f32 %0, %11, %0\n\tv_add_f32 %0, %12, %0\n\t"
        "v_add_f32 %0, %13, %0\n\tv_add_f32 %0, %14, %0\n\tv_add_f32 %0, %15, %0\n\t"
        "v_add_f32 %0, %16, %0"
        : "+v"(acc)
        : "v"(a[0].x), "v"(a[0].y), "v"(a[0].z), "v"(a[0].w), "v"(a[1].x), "v"(a[1].y),
          "v"(a[1].z), "v"(a[1].w), "v"(a[2].x), "v"(a[2].y), "v"(a[2].z), "v"(a[2].w),
          "v"(a[3].x), "v"(a[3].y), "v"(a[3].z), "v"(a[3].w)
        : "memory");
    return acc;
}

// acc += the first m terms of a (m uniform; m >= 16 adds all 16), in order.
__device__ __forceinline__ float nd_add_first(float acc, const float4 (&a)[4], int m)
{
    if (m >= 16) return nd_add16(acc, a);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const float4 &q = a[u / 4];
        const float t = (u & 3) == 0 ? q.x : (u & 3) == 1 ? q.y : (u & 3) == 2 ? q.z : q.w;
        if (u < m) acc += t;
    }
    return acc;
}

__device__ __forceinline__ void nd_lds_read16(float4 (&a)[4], const float *v)
{
    const float4 *v4 = reinterpret_cast<const float4 *>(v);
#pragma unroll
    for (int u = 0; u < 4; ++u) a[u] = v4[u];
}

// ((acc + v[0]) + v[1]) + ... + v[n-1]: the reference's sequential fold, by
// one thread over n floats in LDS (v 16-byte aligned; nothing past v[n-1] is
// read).  Whole groups of 32 are read into two register sets in turn, so a
// group's reads are in flight while the group before it is added.
__device__ inline float nd_lds_fold(float acc, const float *v, int n)
{
    const int G = n / 32;
    if (G > 0) {
        float4 a[8], b[8];
        auto rd = [&](float4 (&r)[8], int gi) {
            const float4 *v4 = reinterpret_cast<const float4 *>(v + gi * 32);
#pragma unroll
            for (int u = 0; u < 8; ++u) r[u] = v4[u];
        };
        auto add32 = [&](float s, const float4 (&r)[8]) {
            const float4 lo[4] = {r[0], r[1], r[2], r[3]};
            const float4 hi[4] = {r[4], r[5], r[6], r[7]};
            return nd_add16(nd_add16(s, lo), hi);
        };
        rd(a, 0);
        int gi = 0;
        for (; gi + 2 <= G; gi += 2) {
            // Wait for the LDS reads in flight (group gi, issued 32 adds ago)
            // before issuing the next group's: at the loop head the compiler
            // would otherwise wait for all reads after issuing them.
            // 0xc07f: lgkmcnt(0), vmcnt and expcnt not waited on.
            __builtin_amdgcn_s_waitcnt(0xc07f);
            rd(b, gi + 1);
            acc = add32(acc, a);
            rd(a, gi + 2 < G ? gi + 2 : gi + 1);  // past the end: a harmless re-read
            acc = add32(acc, b);
        }
        if (gi < G) acc = add32(acc, a);
    }
    int i = G * 32;
    const float4 *v4 = reinterpret_cast<const float4 *>(v);
    for (; i + 4 <= n; i += 4) {
        const float4 q = v4[i / 4];
        acc += q.x;
        acc += q.y;
        acc += q.z;
        acc += q.w;
    }
    for (; i < n; ++i) acc += v[i];
    return acc;
}
