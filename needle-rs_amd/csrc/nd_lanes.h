// Cross-lane sums for gfx950 kernels that reduce many rows a wave at once.
//
// A per-row shuffle reduction (`__shfl_xor` five times) lowers to five
// ds_bpermute round trips through the LDS pipe, each waited on before the
// next add.  Kernels that finish a row every few hundred instructions spend
// more time in those waits than in their gathers.  The helpers here keep the
// partials of several rows in registers and reduce them together with VALU
// lane moves: v_permlane16_swap for lanes 16 apart, DPP row_ror:8 for 8,
// one ds_swizzle for 4 and DPP quad_perm for 2 and 1.
//
// Lanes are numbered threadIdx.x % 64: every caller launches one-dimensional
// blocks whose width is a multiple of 64, with all lanes of the wave active
// where it calls (DPP and the lane swaps read the partner's register
// directly).
#pragma once

#include <hip/hip_runtime.h>

namespace ndl {

// Lane l reads lane l ^ D of x, for D = 8, 4, 2 or 1 (within 32-lane halves).
template <int D>
__device__ inline float lane_xor(float x)
{
    static_assert(D == 8 || D == 4 || D == 2 || D == 1, "lane distance");
    const int xi = __float_as_int(x);
    if constexpr (D == 8)
        return __int_as_float(__builtin_amdgcn_update_dpp(0, xi, 0x128, 0xf, 0xf, false));  // row_ror:8
    else if constexpr (D == 4)
        return __int_as_float(__builtin_amdgcn_ds_swizzle(xi, 0x101f));  // and 0x1f, xor 4
    else if constexpr (D == 2)
        return __int_as_float(__builtin_amdgcn_update_dpp(0, xi, 0x4e, 0xf, 0xf, false));  // quad_perm [2,3,0,1]
    else
        return __int_as_float(__builtin_amdgcn_update_dpp(0, xi, 0xb1, 0xf, 0xf, false));  // quad_perm [1,0,3,2]
}

// Lane l reads lane l ^ H of x across the whole wave, H = 1 .. 32 -- what
// __shfl_xor(x, H, 64) returns, without its ds_bpermute round trip: DPP
// quad_perm for 1 and 2, a row_shl:4 / row_shr:4 pair for 4, row_ror:8 for
// 8, and for 16 and 32 one v_permlane16_swap / v_permlane32_swap of x with
// itself (an even row, or the lower half, finds its partner's value in the
// second result, the other lanes in the first).
template <int H>
__device__ inline float wave_xor(float x)
{
    static_assert(H == 32 || H == 16 || H == 8 || H == 4 || H == 2 || H == 1, "lane distance");
    const int lane = threadIdx.x & 63;
    if constexpr (H == 32 || H == 16) {
        const uint32_t xi = __float_as_uint(x);
        const auto sw = H == 32 ? __builtin_amdgcn_permlane32_swap(xi, xi, false, false)
                                : __builtin_amdgcn_permlane16_swap(xi, xi, false, false);
        return __uint_as_float((lane & H) ? sw[0] : sw[1]);
    } else if constexpr (H == 4) {
        const int xi = __float_as_int(x);
        const int up = __builtin_amdgcn_update_dpp(0, xi, 0x104, 0xf, 0xf, false);  // row_shl:4, lane + 4
        const int dn = __builtin_amdgcn_update_dpp(0, xi, 0x114, 0xf, 0xf, false);  // row_shr:4, lane - 4
        return __int_as_float((lane & 4) ? dn : up);
    } else {
        return lane_xor<H>(x);
    }
}

// Lane K of x's aligned group of four lanes (DPP quad_perm [K,K,K,K]).
template <int K>
__device__ inline float quad_lane(float x)
{
    static_assert(K >= 0 && K < 4, "quad lane");
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), K * 0x55, 0xf, 0xf, false));
}

// The same for an int (argmax indices ride beside their values).
template <int H>
__device__ inline int wave_xor_int(int x)
{
    return __float_as_int(wave_xor<H>(__int_as_float(x)));
}

// Max and sum over the whole wave, pairing lanes at distances 32, 16, .., 1
// (the tree of the usual shuffle loop, bit for bit); every lane gets the
// result.
__device__ inline float wave_max64(float v)
{
    v = fmaxf(v, wave_xor<32>(v));
    v = fmaxf(v, wave_xor<16>(v));
    v = fmaxf(v, wave_xor<8>(v));
    v = fmaxf(v, wave_xor<4>(v));
    v = fmaxf(v, wave_xor<2>(v));
    return fmaxf(v, wave_xor<1>(v));
}

__device__ inline float wave_sum64(float v)
{
    v += wave_xor<32>(v);
    v += wave_xor<16>(v);
    v += wave_xor<8>(v);
    v += wave_xor<4>(v);
    v += wave_xor<2>(v);
    return v + wave_xor<1>(v);
}

// v summed with its partners at lane distances D, 2 D, .., 32, in that
// order (lanes sharing l mod D end with their group's total).
template <int D>
__device__ inline float wave_sum_from(float v)
{
    if constexpr (D < 64) {
        v += wave_xor<D>(v);
        return wave_sum_from<2 * D>(v);
    } else {
        return v;
    }
}

// Sum over aligned groups of N consecutive lanes (N = 1, 2, 4, 8, 16),
// pairing lanes at distances 1, 2, .., N / 2; every lane of a group gets
// the group's total.
template <int N>
__device__ inline float group_sum(float v)
{
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group size");
    if constexpr (N >= 2) v += wave_xor<1>(v);
    if constexpr (N >= 4) v += wave_xor<2>(v);
    if constexpr (N >= 8) v += wave_xor<4>(v);
    if constexpr (N >= 16) v += wave_xor<8>(v);
    return v;
}

// One Walsh-Hadamard butterfly stage across lanes H apart: the lane with
// bit H clear forms a + b, the other a - b (its partner's value minus its
// own), exactly the butterfly's two results.
template <int H>
__device__ inline float wave_butterfly(float v)
{
    const float p = wave_xor<H>(v);
    return (threadIdx.x & H) ? p - v : v + p;
}

// Stages H = 1, 2, .., 32 in order.
__device__ inline float wave_fwht64(float v)
{
    v = wave_butterfly<1>(v);
    v = wave_butterfly<2>(v);
    v = wave_butterfly<4>(v);
    v = wave_butterfly<8>(v);
    v = wave_butterfly<16>(v);
    return wave_butterfly<32>(v);
}

// One level of the tree at lane distance D over n open partials.  With
// exchange, a lane keeps the upper half of its partials when bit D of its
// index is set, the lower half otherwise, and adds its partner's copy of the
// half it keeps; n halves.  Without exchange every partial adds its partner's.
template <int D>
__device__ inline void sum_level(float *v, int n, int j)
{
    const bool up = (j & D) != 0;
    if (n > 1) {
        const int h = n / 2;
#pragma unroll
        for (int q = 0; q < h; ++q) {
            const float keep = up ? v[q + h] : v[q];
            const float give = up ? v[q] : v[q + h];
            v[q] = keep + lane_xor<D>(give);
        }
    } else {
        v[0] += lane_xor<D>(v[0]);
    }
}

// Sums P per-lane partials (P = 1, 2, 4 or 8) over each 32-lane half of a
// wave.  Every total is the tree a shuffle reduction at lane distances 16, 8,
// 4, 2, 1 forms, bit for bit (each level adds a lane's value and its
// partner's).  The first log2(P) levels exchange halves, so lane j ends with
// the total of partial half_wave_slot<P>(j) and v is overwritten.
template <int P>
__device__ inline int half_wave_slot(int j)
{
    static_assert(P == 1 || P == 2 || P == 4 || P == 8, "partials a lane");
    int s = 0, w = P / 2;
#pragma unroll
    for (int bit = 16; bit >= 1 && w > 0; bit >>= 1, w >>= 1)
        if (j & bit) s += w;
    return s;
}

template <int P>
__device__ inline float half_wave_sum(float (&v)[P], int j)
{
    static_assert(P == 1 || P == 2 || P == 4 || P == 8, "partials a lane");
    // Distance 16: v_permlane16_swap exchanges odd 16-lane rows of its first
    // operand with even rows of its second, so after swapping (lower half,
    // upper half) an even-row lane holds its own and its partner's lower
    // partial and an odd-row lane its partner's and its own upper one.
    if constexpr (P > 1) {
#pragma unroll
        for (int q = 0; q < P / 2; ++q) {
            const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[q]),
                                                             __float_as_uint(v[q + P / 2]), false, false);
            v[q] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
    } else {
        const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[0]), __float_as_uint(v[0]), false, false);
        v[0] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    int n = P > 1 ? P / 2 : 1;
    sum_level<8>(v, n, j);
    n = n > 1 ? n / 2 : 1;
    sum_level<4>(v, n, j);
    n = n > 1 ? n / 2 : 1;
    sum_level<2>(v, n, j);
    n = n > 1 ? n / 2 : 1;
    sum_level<1>(v, n, j);
    return v[0];
}

}  // namespace ndl
