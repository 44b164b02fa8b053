// Internal entry points of the reference-order kernels for the Needle-3
// forward (not part of the C ABI).
#pragma once

#include "nd_cq_internal.h"

// n (<= 4) Cactus-Quants weights applied to the same prepared input xh
// ([batch][in_padded]) in one launch on `stream` when they share width,
// group and input size (else one launch each); y[k] receives rows[k] rows
// of weight k from row_start[k], batch-major ([batch][rows[k]]).
// Bit-identical to CqWeight::matvec_rows_prepared / matmul_rows_prepared
// per weight.
int nd_cq_exact_set(nd_ctx *ctx, hipStream_t stream, int n, const nd_cq *const *w, const float *xh,
                    size_t batch, const size_t *row_start, const size_t *rows, float *const *y,
                    const char *what);

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
