// Format B: one uint8 code per weight, one 256-entry fp32 codebook per 64
// consecutive output rows.  y[o] = sum_k cb[o/64][W[o,k]] * x[k].
//
// The format has no reference function (its nearest analogue is the byte-LUT
// decode of crates/needle-core/src/cq.rs:838-873); the semantics are the
// closed form above.
//
// GEMV (decode, batch 1) is HBM-bound: 1 byte of code per multiply-add, so
// the kernel is shaped around keeping HBM streaming while each code costs a
// byte extract, an LDS gather and one FMA:
//   * one 64-row codebook tile per 4-wave workgroup, 32 lanes per row, the
//     lane's activations in registers (fast path: in = 256*M);
//   * the codebook in LDS as 32 lane-private replicas, so random gathers do
//     not conflict on banks;
//   * code loads split in two halves so the second half is in flight while
//     the first computes; nontemporal loads, since codes are read once.
// Other widths fall back to a kernel with the activations in LDS.
// GEMM (prefill) converts X to bf16 once, dequantises weight tiles to bf16 in
// LDS through the bf16-rounded codebook and feeds v_mfma_f32_16x16x32_bf16
// with fp32 accumulation: 64x64 tiles below M = 96, 128x128 tiles, and
// 256x256 tiles with two waves per SIMD once a launch has a tile per CU.
#include "nd_internal.h"
#include "nd_lanes.h"

#include <hip/hip_bf16.h>

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kTileRows = 64;      // rows sharing one codebook
constexpr int kThreads = 256;      // 4 waves
constexpr int kLanesPerRow = 16;
constexpr int kRowsPerPass = kThreads / kLanesPerRow;  // 16

// Fast path, in = 256*M (M = 1..4; config 1's 768 is M = 3).  One 256-thread
// block owns one 64-row tile.  32 lanes share a row: lane j reads M/2
// 16-byte vectors (bytes 512k + 16j) and, for odd M, one 8-byte vector
// (bytes 512*(M/2) + 8j) -- every load instruction covers two rows x 256 or
// 512 contiguous bytes -- and keeps the matching 8*M activations in
// registers.  A wave's 16 rows (8 passes of two) are all loaded before the
// first gather.  Each pass leaves one partial a lane; the 8 partials are
// summed over their half waves together at the end with VALU lane moves
// (a per-pass shuffle reduction costs five LDS round trips a row, which
// measured 72-75 % of HBM against 85 % for the deferred sum).  Rows past
// `out` are clamped (a valid row is read and its sum discarded) rather than
// predicated.
//
// The codebook sits in LDS as 32 lane-private replicas, entry-major (entry
// e, replica r at dword 32e + r): lane l's gathers all hit bank l % 32, so a
// random gather does not conflict.
template <int M>
struct RowCodes {
    u32x4_t a[M / 2 > 0 ? M / 2 : 1];
    u32x2_t b;
};

template <int M>
__device__ inline void load_row(RowCodes<M> &c, const uint8_t *__restrict__ rp, int j)
{
#pragma unroll
    for (int k = 0; k < M / 2; ++k)
        c.a[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(rp + 512 * k) + j);
    if (M % 2)
        c.b = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(rp + 512 * (M / 2)) + j);
}

template <int M>
__global__ __launch_bounds__(kThreads, 4) void cb8_gemv_kernel(
    const uint8_t *__restrict__ w, size_t w_stride, const float *__restrict__ cb,
    size_t cb_stride, const float *__restrict__ x, size_t x_stride, float *__restrict__ y,
    size_t y_stride, int out)
{
    constexpr int K = 256 * M;
    constexpr int kPasses = 8;  // 16 rows per wave, 2 per pass
    constexpr int kFirst = kPasses;
    __shared__ float4 rep4[256 * 32 / 4];  // 32 KB

    const size_t prob = blockIdx.y;
    w += prob * w_stride;
    cb += prob * cb_stride + size_t(blockIdx.x) * 256;
    x += prob * x_stride;
    y += prob * y_stride;
    const int t = threadIdx.x;
    const int wave = t >> 6;
    const int lane = t & 63;
    const int j = lane & 31;
    const int row0 = blockIdx.x * kTileRows + wave * 16 + (lane >> 5);

    RowCodes<M> c[kPasses];
#pragma unroll
    for (int p = 0; p < kFirst; ++p) {
        const int r = min(row0 + 2 * p, out - 1);
        load_row(c[p], w + size_t(r) * K, j);
    }
    // float4 slot f4 = i*256 + t of the replica array holds entry f4 / 8.
    float cbv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) cbv[i] = cb[(i * kThreads + t) >> 3];
    float xa[M / 2 > 0 ? M / 2 : 1][16], xb[8];
#pragma unroll
    for (int k = 0; k < M / 2; ++k) {
        const float4 *xp = reinterpret_cast<const float4 *>(x + 512 * k + 16 * j);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = xp[q];
            xa[k][4 * q + 0] = v.x;
            xa[k][4 * q + 1] = v.y;
            xa[k][4 * q + 2] = v.z;
            xa[k][4 * q + 3] = v.w;
        }
    }
    if (M % 2) {
        const float4 *xp = reinterpret_cast<const float4 *>(x + 512 * (M / 2) + 8 * j);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const float4 v = xp[q];
            xb[4 * q + 0] = v.x;
            xb[4 * q + 1] = v.y;
            xb[4 * q + 2] = v.z;
            xb[4 * q + 3] = v.w;
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) rep4[i * kThreads + t] = make_float4(cbv[i], cbv[i], cbv[i], cbv[i]);
    __syncthreads();

    const float *cbl = reinterpret_cast<const float *>(rep4) + (lane & 31);
    float sp[kPasses];
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        if (p == 0) {
#pragma unroll
            for (int q = kFirst; q < kPasses; ++q) {
                const int r = min(row0 + 2 * q, out - 1);
                load_row(c[q], w + size_t(r) * K, j);
            }
        }
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < M / 2; ++k) {
            const uint32_t dw[4] = {c[p].a[k].x, c[p].a[k].y, c[p].a[k].z, c[p].a[k].w};
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const uint32_t e = (dw[d] >> (8 * b)) & 0xffu;
                    acc[b] += cbl[e * 32] * xa[k][4 * d + b];
                }
        }
        if (M % 2) {
            const uint32_t dw[2] = {c[p].b.x, c[p].b.y};
#pragma unroll
            for (int d = 0; d < 2; ++d)
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const uint32_t e = (dw[d] >> (8 * b)) & 0xffu;
                    acc[b] += cbl[e * 32] * xb[4 * d + b];
                }
        }
        sp[p] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    }
    // The eight rows' half-wave sums in one lane-exchange tree; lane j ends
    // with the row of pass half_wave_slot<8>(j), and lanes 4k store.
    const float s = ndl::half_wave_sum<kPasses>(sp, j);
    const int r = row0 + 2 * ndl::half_wave_slot<kPasses>(j);
    if ((j & 3) == 0 && r < out) y[r] = s;
}

// Any `in` (multiple of 16): activations staged in LDS instead of registers.
template <int REP>
__global__ __launch_bounds__(kThreads) void cb8_gemv_generic_kernel(
    const uint8_t *__restrict__ w, size_t w_stride, const float *__restrict__ cb,
    size_t cb_stride, const float *__restrict__ x, size_t x_stride, float *__restrict__ y,
    size_t y_stride, int out, int in)
{
    __shared__ float4 rep4[256 * REP / 4];
    __shared__ float stage[256];
    extern __shared__ float xs[];
    float *rep = reinterpret_cast<float *>(rep4);
    const int tile = blockIdx.x;
    const size_t prob = blockIdx.y;
    w += prob * w_stride;
    cb += prob * cb_stride + size_t(tile) * 256;
    x += prob * x_stride;
    y += prob * y_stride;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int j = t & (kLanesPerRow - 1);
    const int rg = t / kLanesPerRow;
    const int nvec = in >> 4;
    stage[t] = cb[t];
    for (int k = t; k < in; k += kThreads) xs[k] = x[k];
    __syncthreads();
    for (int i = 0; i < REP / 4; ++i) {
        const int f4 = i * kThreads + t;
        const float v = stage[(f4 * 4) / REP];
        rep4[f4] = make_float4(v, v, v, v);
    }
    __syncthreads();
    const float *cbl = rep + (lane & (REP - 1));
    const int row0 = tile * kTileRows;
    for (int p = 0; p < kTileRows / kRowsPerPass; ++p) {
        const int r = row0 + rg + kRowsPerPass * p;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (r < out) {
            const uint4 *wr = reinterpret_cast<const uint4 *>(w + size_t(r) * in);
            for (int c = j; c < nvec; c += kLanesPerRow) {
                const uint4 cv = wr[c];
                const uint32_t dw[4] = {cv.x, cv.y, cv.z, cv.w};
#pragma unroll
                for (int d = 0; d < 4; ++d)
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const uint32_t e = (dw[d] >> (8 * b)) & 0xffu;
                        acc[b] += cbl[e * REP] * xs[c * 16 + 4 * d + b];
                    }
            }
        }
        float s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        s += ndl::wave_xor<8>(s);
        s += ndl::wave_xor<4>(s);
        s += ndl::wave_xor<2>(s);
        s += ndl::wave_xor<1>(s);
        if (j == 0 && r < out) y[r] = s;
    }
}

// ---------------------------------------------------------------------------
// GEMM: Y[m][o] = sum_k bf16(X[m][k]) * bf16(cb[o/64][W[o][k]]), fp32 accumulate.
// Block tile 64 (M) x 64 (N, one codebook) with K steps of 32; 4 waves in a
// 2x2 grid, each wave a 32x32 output = 2x2 MFMA 16x16x32 tiles.
// ---------------------------------------------------------------------------
typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4_t;

// fp32 to bf16, round to nearest even: gfx950's v_cvt_pk_bf16_f32 (two
// values an instruction).  It equals the integer form (u + 0x7fff + lsb) >> 16
// on every non-NaN input (a device sweep of all 2^32 patterns found no
// difference; test_gpu_cb8.py pins the ties through the GEMMs); NaNs stay NaN.
typedef __bf16 bf16x2_hw_t __attribute__((ext_vector_type(2)));

__device__ inline uint32_t f32x2_to_bf16x2_rne(float lo, float hi)
{
    const bf16x2_hw_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ inline unsigned short f32_to_bf16_rne(float f)
{
    return static_cast<unsigned short>(f32x2_to_bf16x2_rne(f, 0.0f));
}

constexpr int kGM = 64, kGN = 64, kGK = 128;
constexpr int kLdsPad = 8;  // bf16 elements of padding per LDS row

// X (f32) to bf16, round to nearest even; problem blockIdx.y of a batch at
// element stride xs (input) and n (output).  A block converts kXRuns runs of
// 2048 elements, 8 per thread per run, all loads issued before the stores.
constexpr int kXRuns = 4;

__device__ inline uint4 pack_bf16x8(float4 a, float4 b)
{
    return make_uint4(f32x2_to_bf16x2_rne(a.x, a.y), f32x2_to_bf16x2_rne(a.z, a.w),
                      f32x2_to_bf16x2_rne(b.x, b.y), f32x2_to_bf16x2_rne(b.z, b.w));
}

__global__ __launch_bounds__(256) void x_to_bf16_kernel(const float *__restrict__ X, size_t xs,
                                                        unsigned short *__restrict__ Xb, size_t n)
{
    const float *src = X + blockIdx.y * xs;
    unsigned short *dst = Xb + blockIdx.y * n;
    const size_t base = size_t(blockIdx.x) * (2048 * kXRuns) + threadIdx.x * 8;
    if (base + 2048 * (kXRuns - 1) + 8 <= n) {
        float4 a[kXRuns], b[kXRuns];
#pragma unroll
        for (int r = 0; r < kXRuns; ++r) {
            a[r] = *reinterpret_cast<const float4 *>(src + base + 2048 * r);
            b[r] = *reinterpret_cast<const float4 *>(src + base + 2048 * r + 4);
        }
#pragma unroll
        for (int r = 0; r < kXRuns; ++r)
            *reinterpret_cast<uint4 *>(dst + base + 2048 * r) = pack_bf16x8(a[r], b[r]);
        return;
    }
    // a problem's last block: run by run, the ragged end element by element
    for (int r = 0; r < kXRuns; ++r) {
        const size_t i = base + 2048 * size_t(r);
        if (i >= n) return;
        if (i + 8 <= n) {
            const float4 a = *reinterpret_cast<const float4 *>(src + i);
            const float4 b = *reinterpret_cast<const float4 *>(src + i + 4);
            *reinterpret_cast<uint4 *>(dst + i) = pack_bf16x8(a, b);
        } else {
            for (size_t k = i; k < n; ++k) dst[k] = f32_to_bf16_rne(src[k]);
        }
    }
}

// Y[M][N] = X[M][K] . decode(W[N][K])^T, X already bf16.  A 256-thread block
// owns a 64x64 output tile (4 waves of 32x32, 2x2 MFMA 16x16x32 tiles each)
// and walks K 128 at a time: the next step's X rows and codes are loaded
// into registers while the current step's 16 MFMAs per wave run from LDS.
// The block's codebook sits in LDS already rounded to bf16, so decoding a
// code is one LDS read.
__global__ __launch_bounds__(256) void cb8_gemm_kernel(const unsigned short *__restrict__ Xb,
                                                       const uint8_t *__restrict__ W,
                                                       const float *__restrict__ cb,
                                                       float *__restrict__ Y, int M, int N,
                                                       int K, size_t ws, size_t cs, size_t ys)
{
    __shared__ unsigned short cbh[256];
    __shared__ __align__(16) unsigned short As[kGM][kGK + kLdsPad];
    __shared__ __align__(16) unsigned short Bs[kGN][kGK + kLdsPad];

    // problem blockIdx.z of a batch: X at M*K, the rest at element strides
    Xb += blockIdx.z * size_t(M) * K;
    W += blockIdx.z * ws;
    cb += blockIdx.z * cs;
    Y += blockIdx.z * ys;

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int n0 = blockIdx.x * kGN;
    const int m0 = blockIdx.y * kGM;
    const int wm = (wave >> 1) * 32;  // wave's row offset within the tile
    const int wn = (wave & 1) * 32;   // wave's column offset

    cbh[t] = f32_to_bf16_rne(cb[size_t(n0 / 64) * 256 + t]);

    floatx4_t acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int sr = t >> 2;          // staged row 0..63 (of A and of B)
    const int sc = (t & 3) * 32;    // staged columns sc..sc+31 of the K step
    const bool mrow = m0 + sr < M;
    const unsigned short *xrow = Xb + size_t(mrow ? m0 + sr : 0) * K;
    const uint8_t *wrow = W + size_t(n0 + sr) * K;  // N is a multiple of 64
    uint4 xa[4];
    uint2 wc[4];
    auto load = [&](int k0) {
        const bool on = k0 + sc < K;  // K is a multiple of 32: a 32-column run is all in or out
#pragma unroll
        for (int q = 0; q < 4; ++q)
            xa[q] = on && mrow ? *reinterpret_cast<const uint4 *>(xrow + k0 + sc + 8 * q)
                               : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            wc[q] = on ? *reinterpret_cast<const uint2 *>(wrow + k0 + sc + 8 * q) : make_uint2(0, 0);
        return on;
    };
    auto store = [&](bool on) {
#pragma unroll
        for (int q = 0; q < 4; ++q) *reinterpret_cast<uint4 *>(&As[sr][sc + 8 * q]) = xa[q];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t d[2] = {wc[q].x, wc[q].y};
            uint32_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = cbh[(d[e >> 1] >> (16 * (e & 1))) & 0xffu];
                const uint32_t hi = cbh[(d[e >> 1] >> (16 * (e & 1) + 8)) & 0xffu];
                h[e] = on ? lo | (hi << 16) : 0u;
            }
            *reinterpret_cast<uint4 *>(&Bs[sr][sc + 8 * q]) = make_uint4(h[0], h[1], h[2], h[3]);
        }
    };
    __syncthreads();  // codebook in LDS
    bool on = load(0);
    // MFMA 16x16x32 bf16: lane l supplies A[row l%16][k 8*(l/16) .. +8]
    // and B[k 8*(l/16) .. +8][col l%16].
    const int r16 = lane & 15;
    const int kq = (lane >> 4) * 8;
    for (int k0 = 0; k0 < K; k0 += kGK) {
        store(on);
        __syncthreads();
        if (k0 + kGK < K) on = load(k0 + kGK);
        const int steps = (K - k0 < kGK ? K - k0 : kGK) / 32;
        for (int kk = 0; kk < steps; ++kk) {
            bf16x8_t afrag[2], bfrag[2];
#pragma unroll
            for (int a = 0; a < 2; ++a)
                afrag[a] = *reinterpret_cast<const bf16x8_t *>(&As[wm + a * 16 + r16][kk * 32 + kq]);
#pragma unroll
            for (int b = 0; b < 2; ++b)
                bfrag[b] = *reinterpret_cast<const bf16x8_t *>(&Bs[wn + b * 16 + r16][kk * 32 + kq]);
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag[a], bfrag[b],
                                                                        acc[a][b], 0, 0, 0);
        }
        __syncthreads();
    }
    // C layout: lane l holds C[4*(l/16) + i][l%16], i < 4.
    const int col = lane & 15;
    const int rb = (lane >> 4) * 4;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + wm + a * 16 + rb + i;
                const int n = n0 + wn + b * 16 + col;
                if (m < M) Y[size_t(m) * N + n] = acc[a][b][i];
            }
}

// The same product with 128x128 tiles for M >= 96: 4 waves of 64x64 (4x4
// MFMA tiles each), K steps of 64, each thread staging half a row of A
// (32 bf16) and of B (32 codes).  A decoded code strip serves twice the
// rows of the 64x64 kernel, halving the decode work per MFMA.
constexpr int kBM = 128, kBN = 128, kBK = 64;

__global__ __launch_bounds__(256) void cb8_gemm128_kernel(const unsigned short *__restrict__ Xb,
                                                          const uint8_t *__restrict__ W,
                                                          const float *__restrict__ cb,
                                                          float *__restrict__ Y, int M, int N,
                                                          int K, size_t ws, size_t cs, size_t ys)
{
    __shared__ unsigned short cbh[2][256];
    __shared__ __align__(16) unsigned short As[kBM][kBK + kLdsPad];
    __shared__ __align__(16) unsigned short Bs[kBN][kBK + kLdsPad];

    Xb += blockIdx.z * size_t(M) * K;
    W += blockIdx.z * ws;
    cb += blockIdx.z * cs;
    Y += blockIdx.z * ys;

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int n0 = blockIdx.x * kBN;
    const int m0 = blockIdx.y * kBM;
    const int wm = (wave >> 1) * 64;
    const int wn = (wave & 1) * 64;

    // the tile's two 64-row codebooks, rounded to bf16
    cbh[0][t] = f32_to_bf16_rne(cb[size_t(n0 / 64) * 256 + t]);
    cbh[1][t] = f32_to_bf16_rne(cb[size_t(n0 / 64 + 1) * 256 + t]);

    floatx4_t acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int sr = t >> 1;          // staged row 0..127 (of A and of B)
    const int sc = (t & 1) * 32;    // staged columns sc..sc+31 of the K step
    const bool mrow = m0 + sr < M;
    const unsigned short *xrow = Xb + size_t(mrow ? m0 + sr : 0) * K;
    const uint8_t *wrow = W + size_t(n0 + sr) * K;  // N is a multiple of 128 here
    const unsigned short *cbr = cbh[sr >> 6];
    uint4 xa[4];
    uint2 wc[4];
    auto load = [&](int k0) {
        const bool on = k0 + sc < K;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            xa[q] = on && mrow ? *reinterpret_cast<const uint4 *>(xrow + k0 + sc + 8 * q)
                               : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            wc[q] = on ? *reinterpret_cast<const uint2 *>(wrow + k0 + sc + 8 * q) : make_uint2(0, 0);
        return on;
    };
    auto store = [&](bool on) {
#pragma unroll
        for (int q = 0; q < 4; ++q) *reinterpret_cast<uint4 *>(&As[sr][sc + 8 * q]) = xa[q];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t d[2] = {wc[q].x, wc[q].y};
            uint32_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = cbr[(d[e >> 1] >> (16 * (e & 1))) & 0xffu];
                const uint32_t hi = cbr[(d[e >> 1] >> (16 * (e & 1) + 8)) & 0xffu];
                h[e] = on ? lo | (hi << 16) : 0u;
            }
            *reinterpret_cast<uint4 *>(&Bs[sr][sc + 8 * q]) = make_uint4(h[0], h[1], h[2], h[3]);
        }
    };
    __syncthreads();
    bool on = load(0);
    const int r16 = lane & 15;
    const int kq = (lane >> 4) * 8;
    for (int k0 = 0; k0 < K; k0 += kBK) {
        store(on);
        __syncthreads();
        if (k0 + kBK < K) on = load(k0 + kBK);
        const int steps = (K - k0 < kBK ? K - k0 : kBK) / 32;
        for (int kk = 0; kk < steps; ++kk) {
            bf16x8_t afrag[4], bfrag[4];
#pragma unroll
            for (int a = 0; a < 4; ++a)
                afrag[a] = *reinterpret_cast<const bf16x8_t *>(&As[wm + a * 16 + r16][kk * 32 + kq]);
#pragma unroll
            for (int b = 0; b < 4; ++b)
                bfrag[b] = *reinterpret_cast<const bf16x8_t *>(&Bs[wn + b * 16 + r16][kk * 32 + kq]);
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag[a], bfrag[b],
                                                                        acc[a][b], 0, 0, 0);
        }
        __syncthreads();
    }
    const int col = lane & 15;
    const int rb = (lane >> 4) * 4;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + wm + a * 16 + rb + i;
                const int n = n0 + wn + b * 16 + col;
                if (m < M) Y[size_t(m) * N + n] = acc[a][b][i];
            }
}

// The same product on 256x256 tiles for launches with at least one tile per
// CU.  8 waves, two per SIMD, each a 64x128 output (4x8 MFMA 16x16x32 tiles);
// LDS holds two K steps of 64 so the next step is decoded while the current
// one is multiplied.  Waves 0-3 multiply first and then stage, waves 4-7
// stage first: the two waves sharing a SIMD are out of phase, so one keeps
// the MFMA pipe fed while the other waits on global loads and codebook
// gathers.  Loads read clamped, always valid addresses and are masked at the
// LDS store, so no load sits behind a branch.  Tiles are numbered so that each
// XCD (blocks are dealt round-robin to the 8 XCDs) owns a contiguous run,
// M tiles fastest: blocks sharing an X row block or a W column block meet in
// one L2.  Per output the K order is that of the 128x128 kernel, so the two
// agree bit for bit.
constexpr int kPM = 256, kPN = 256, kPK = 64;
constexpr int kPWM = 64, kPWN = 128;  // wave tile: waves 4 (M) x 2 (N)

__global__ __launch_bounds__(512) void cb8_gemm256_kernel(const float *__restrict__ Xf, size_t xs,
                                                          const uint8_t *__restrict__ W,
                                                          const float *__restrict__ cb,
                                                          float *__restrict__ Y, int M, int N,
                                                          int K, size_t ws, size_t cs, size_t ys,
                                                          int tiles_n, int tiles_m, int xcd_run)
{
    constexpr int TA = kPWM / 16, TB = kPWN / 16;
    constexpr int J = kPM / 64;  // staged 64-row slabs of A and of B
    __shared__ __align__(16) unsigned short As[2][kPM][kPK + kLdsPad];
    __shared__ __align__(16) unsigned short Bs[2][kPN][kPK + kLdsPad];
    __shared__ unsigned short cbh[kPN / 64][256];

    const int id = blockIdx.x;
    const int u = xcd_run ? (id % 8) * xcd_run + id / 8 : id;
    const int z = u / (tiles_n * tiles_m);
    const int m0 = (u % tiles_m) * kPM;
    const int n0 = ((u / tiles_m) % tiles_n) * kPN;
    Xf += z * xs;  // X stays fp32 in HBM; it is rounded to bf16 as it is staged
    W += z * ws;
    cb += z * cs;
    Y += z * ys;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wm = (wave & 3) * kPWM;
    const int wn = (wave >> 2) * kPWN;
    for (int i = t; i < kPN / 64 * 256; i += 512)
        cbh[i / 256][i % 256] = f32_to_bf16_rne(cb[size_t(n0 / 64 + i / 256) * 256 + i % 256]);

    floatx4_t acc[TA][TB];
#pragma unroll
    for (int a = 0; a < TA; ++a)
#pragma unroll
        for (int b = 0; b < TB; ++b) acc[a][b] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int r8 = t >> 3;       // staged row within a 64-row slab
    const int c8 = (t & 7) * 8;  // staged columns c8..c8+7 of the K step
    bool mok[J];
    const float *xp[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int m = m0 + r8 + 64 * j;
        mok[j] = m < M;
        xp[j] = Xf + size_t(m < M ? m : M - 1) * K + c8;
    }
    const uint8_t *wp = W + size_t(n0 + r8) * K + c8;  // N is a multiple of 256 here
    float4 xa[J][2];
    uint2 wc[J];
    bool on = true;
    auto load = [&](int k0) {
        on = k0 + c8 < K;
        // K is a multiple of 32: a run past K belongs to a final half step,
        // and the run 32 columns back is in range
        const int kc = on ? k0 : k0 - 32;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            xa[j][0] = *reinterpret_cast<const float4 *>(xp[j] + kc);
            xa[j][1] = *reinterpret_cast<const float4 *>(xp[j] + kc + 4);
        }
#pragma unroll
        for (int j = 0; j < J; ++j) wc[j] = *reinterpret_cast<const uint2 *>(wp + size_t(64 * j) * K + kc);
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int j = 0; j < J; ++j)
            *reinterpret_cast<uint4 *>(&As[buf][r8 + 64 * j][c8]) =
                on && mok[j] ? pack_bf16x8(xa[j][0], xa[j][1]) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t d[2] = {wc[j].x, wc[j].y};
            uint32_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = cbh[j][(d[e >> 1] >> (16 * (e & 1))) & 0xffu];
                const uint32_t hi = cbh[j][(d[e >> 1] >> (16 * (e & 1) + 8)) & 0xffu];
                h[e] = on ? lo | (hi << 16) : 0u;
            }
            *reinterpret_cast<uint4 *>(&Bs[buf][r8 + 64 * j][c8]) = make_uint4(h[0], h[1], h[2], h[3]);
        }
    };
    const int r16 = lane & 15;
    const int kq = (lane >> 4) * 8;
    auto multiply = [&](int buf, int halves) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            if (kk < halves) {
                bf16x8_t af[TA], bfv[TB];
#pragma unroll
                for (int a = 0; a < TA; ++a)
                    af[a] = *reinterpret_cast<const bf16x8_t *>(&As[buf][wm + a * 16 + r16][kk * 32 + kq]);
#pragma unroll
                for (int b = 0; b < TB; ++b)
                    bfv[b] = *reinterpret_cast<const bf16x8_t *>(&Bs[buf][wn + b * 16 + r16][kk * 32 + kq]);
#pragma unroll
                for (int a = 0; a < TA; ++a)
#pragma unroll
                    for (int b = 0; b < TB; ++b)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[a], bfv[b], acc[a][b], 0, 0, 0);
            }
        }
    };
    const int nk = (K + kPK - 1) / kPK;
    load(0);
    __syncthreads();  // codebooks in LDS
    store(0);
    load(nk > 1 ? kPK : 0);
    __syncthreads();
    const bool first = wave < 4;
    for (int i = 0; i < nk; ++i) {
        const int cur = i & 1;
        const int halves = (K - i * kPK < kPK ? K - i * kPK : kPK) / 32;
        // step i+1 into the other buffer (read last in step i-1, before the
        // barrier that ended it); step i+2's loads go out behind it.  Every
        // step stores and loads -- the last ones repeat the final step into a
        // buffer nothing reads -- so no load sits behind a branch and the
        // waits count the loads in flight exactly (a load behind a branch
        // makes the compiler wait for it at the join)
        const int kl = (i + 2 < nk ? i + 2 : nk - 1) * kPK;
        if (first) {
            multiply(cur, halves);
            store(cur ^ 1);
            load(kl);
        } else {
            store(cur ^ 1);
            load(kl);
            multiply(cur, halves);
        }
        __syncthreads();
    }
    const int col = lane & 15;
    const int rb = (lane >> 4) * 4;
#pragma unroll
    for (int a = 0; a < TA; ++a)
#pragma unroll
        for (int b = 0; b < TB; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + wm + a * 16 + rb + i;
                const int n = n0 + wn + b * 16 + col;
                if (m < M) Y[size_t(m) * N + n] = acc[a][b][i];
            }
}

// M <= 64 (e.g. the rows of 64 sessions at once): each code feeds only 64
// rows, so the launch streams codes and the decode, not the MFMAs, sets the
// pace.  A 256-thread block owns 128 output columns (two codebook groups)
// and all M rows; the codes skip LDS entirely.  Lane (r16, q) of wave w
// loads 16 consecutive codes of rows n0 + 32w + 16t + r16 (t = 0, 1) per
// 64-wide K step -- four lanes cover a row's 64 bytes in one load -- and
// decodes them through a lane-replicated codebook table (entry e, replica r
// in bank r: conflict-free gathers; both groups' bf16 in one word) straight
// into MFMA B fragments.  X is staged in LDS 128 columns at a time, double
// buffered.  Both operands use physical k 16q..16q+7 for the first MFMA of
// a step and 16q+8..+15 for the second, so the K order differs from the
// other tile shapes' (results agree to fp32 rounding, not bit for bit).
constexpr int kRN = 128;          // output columns (N) per block: two codebook groups
constexpr int kRC = 128;          // K per staged X chunk
constexpr int kRXS = kRC + 8;     // padded X row in LDS (bf16)

__global__ __launch_bounds__(256, 2) void cb8_gemm_m64_kernel(const unsigned short *__restrict__ Xb,
                                                              const uint8_t *__restrict__ W,
                                                              const float *__restrict__ cb,
                                                              float *__restrict__ Y, int M, int N,
                                                              int K, size_t ws, size_t cs, size_t ys,
                                                              int tiles_n, int xcd_run)
{
    __shared__ __align__(16) uint32_t tab[256 * 32];
    __shared__ __align__(16) unsigned short xs[2][64 * kRXS];
    // the column tiles of one problem are consecutive in u and land on one
    // XCD (workgroups are dealt to the 8 XCDs round-robin), sharing X in L2
    const int id = blockIdx.x;
    const int u = xcd_run ? (id % 8) * xcd_run + id / 8 : id;
    const int z = u / tiles_n, tn = u - z * tiles_n;
    Xb += size_t(z) * M * K;
    W += z * ws;
    cb += z * cs;
    Y += z * ys;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int r16 = lane & 15, q = lane >> 4;
    const int n0 = tn * kRN;
    const uint8_t *wp0 = W + size_t(n0 + 32 * w + r16) * K + 16 * q;
    const uint8_t *wp1 = wp0 + size_t(16) * K;
    const int nc = K / kRC;
    // codes of chunk c: two 64-wide steps x two row groups.  Past the last
    // chunk the load reads X instead (L2-resident, unused), so every chunk
    // issues the same loads and the waits count them exactly.
    uint4 cw[2][2][2];
    auto cload = [&](int slot, int c) {
        const bool in = c < nc;
        const uint8_t *p0 = in ? wp0 + c * kRC : reinterpret_cast<const uint8_t *>(Xb);
        const uint8_t *p1 = in ? wp1 + c * kRC : reinterpret_cast<const uint8_t *>(Xb);
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
            const u32x4_t c0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p0 + kp * 64));
            const u32x4_t c1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p1 + kp * 64));
            cw[slot][kp][0] = make_uint4(c0.x, c0.y, c0.z, c0.w);
            cw[slot][kp][1] = make_uint4(c1.x, c1.y, c1.z, c1.w);
        }
    };
    // X chunk c: 64 rows x 128 bf16, 16-byte pieces; rows past M are zero
    uint4 xr[4];
    auto xload = [&](int c) {
        const int cc = c < nc ? c : nc - 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = t + 256 * i, row = idx >> 4, col = (idx & 15) * 8;
            xr[i] = *reinterpret_cast<const uint4 *>(Xb + size_t(row < M ? row : M - 1) * K + cc * kRC + col);
            if (row >= M) xr[i] = make_uint4(0, 0, 0, 0);
        }
    };
    auto xstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = t + 256 * i, row = idx >> 4, col = (idx & 15) * 8;
            *reinterpret_cast<uint4 *>(&xs[buf][row * kRXS + col]) = xr[i];
        }
    };
    cload(0, 0);
    xload(0);
    {
        // the table, through a staging row in xs[1] so every write is
        // conflict-free: word e of the staging row, then 8 x 16 bytes a thread
        uint32_t *vals = reinterpret_cast<uint32_t *>(&xs[1][0]);
        vals[t] = f32_to_bf16_rne(cb[size_t(n0 / 64) * 256 + t]) |
                  (uint32_t(f32_to_bf16_rne(cb[size_t(n0 / 64 + 1) * 256 + t])) << 16);
        __syncthreads();
        uint4 *t4 = reinterpret_cast<uint4 *>(tab);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t v = vals[(i * 256 + t) >> 3];
            t4[i * 256 + t] = make_uint4(v, v, v, v);
        }
    }
    xstore(0);
    __syncthreads();
    // waves 0-1 hold rows of the first group (low halves), 2-3 the second
    const uint32_t sel = w >= 2 ? 0x07060302u : 0x05040100u;
    const uint32_t *tl = tab + (lane & 31);
    floatx4_t acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
    auto decode = [&](const uint4 &c, bf16x8_t &f0, bf16x8_t &f1) {
        const uint32_t d[4] = {c.x, c.y, c.z, c.w};
        uint32_t h[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t v0 = tl[((d[k >> 1] >> (16 * (k & 1))) & 0xffu) * 32];
            const uint32_t v1 = tl[((d[k >> 1] >> (16 * (k & 1) + 8)) & 0xffu) * 32];
            h[k] = __builtin_amdgcn_perm(v1, v0, sel);
        }
        f0 = __builtin_bit_cast(bf16x8_t, make_uint4(h[0], h[1], h[2], h[3]));
        f1 = __builtin_bit_cast(bf16x8_t, make_uint4(h[4], h[5], h[6], h[7]));
    };
    auto compute = [&](int buf, int slot) {
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
            bf16x8_t b[2][2];
            decode(cw[slot][kp][0], b[0][0], b[0][1]);
            decode(cw[slot][kp][1], b[1][0], b[1][1]);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const unsigned short *xa = &xs[buf][(16 * mt + r16) * kRXS + kp * 64 + 16 * q];
                const bf16x8_t a0 = *reinterpret_cast<const bf16x8_t *>(xa);
                const bf16x8_t a1 = *reinterpret_cast<const bf16x8_t *>(xa + 8);
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    acc[mt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b[tt][0], acc[mt][tt], 0, 0, 0);
                    acc[mt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b[tt][1], acc[mt][tt], 0, 0, 0);
                }
            }
        }
    };
    // chunk c: X of chunk c + 1 and the codes of chunk c + 1 in flight while
    // chunk c is multiplied.  X is issued first, so storing it waits for X
    // only and the code loads stay in flight across the barrier.
    for (int c0 = 0; c0 < nc; c0 += 2) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int c = c0 + s;
            if (c < nc) {
                xload(c + 1);
                __builtin_amdgcn_sched_barrier(0);
                cload(s ^ 1, c + 1);
                compute(c & 1, s);
                if (c + 1 < nc) xstore((c + 1) & 1);
                __syncthreads();
            }
        }
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 16 * mt + 4 * q + i;
                if (m < M) Y[size_t(m) * N + n0 + 32 * w + 16 * tt + r16] = acc[mt][tt][i];
            }
}

constexpr int kRep = 32;

int launch_gemv(nd_ctx *ctx, size_t count, const uint8_t *w, size_t w_stride, const float *cb,
                size_t cb_stride, const float *x, size_t x_stride, float *y, size_t y_stride,
                size_t out, size_t in)
{
    ND_REQUIRE(w && cb && x && y, "null buffer");
    ND_REQUIRE(out > 0 && in > 0, "empty shape %zux%zu", out, in);
    ND_REQUIRE(in % 16 == 0, "in (%zu) must be a multiple of 16", in);
    ND_REQUIRE(out <= (size_t(1) << 30) && in <= (size_t(1) << 24), "shape too large");
    ND_REQUIRE(count >= 1 && count <= 65535, "count %zu out of range 1..65535", count);
    ND_REQUIRE((reinterpret_cast<uintptr_t>(w) & 15) == 0 && w_stride % 16 == 0,
               "codes must be 16-byte aligned");
    ND_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0 && x_stride % 4 == 0,
               "activations must be 16-byte aligned");
    const int tiles = static_cast<int>((out + kTileRows - 1) / kTileRows);
    dim3 grid(tiles, static_cast<unsigned>(count));
    const bool fast = in % 256 == 0 && in <= 1024 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                      x_stride % 4 == 0;
#define ND_GEMV(MM)                                                                          \
    hipLaunchKernelGGL((cb8_gemv_kernel<MM>), grid, dim3(kThreads), 0, ctx->stream, w, w_stride, \
                       cb, cb_stride, x, x_stride, y, y_stride, int(out))
    if (fast) {
        switch (in / 256) {
        case 1: ND_GEMV(1); break;
        case 2: ND_GEMV(2); break;
        case 3: ND_GEMV(3); break;
        default: ND_GEMV(4); break;
        }
    } else {
        ND_REQUIRE(in * sizeof(float) <= 64 * 1024, "in (%zu) too large", in);
        hipLaunchKernelGGL((cb8_gemv_generic_kernel<kRep>), grid, dim3(kThreads),
                           in * sizeof(float), ctx->stream, w, w_stride, cb, cb_stride, x,
                           x_stride, y, y_stride, int(out), int(in));
    }
#undef ND_GEMV
    return nd::check_launch("cb8_gemv");
}

}  // namespace

extern "C" {

int nd_cb8_gemv(nd_ctx *ctx, const uint8_t *w, const float *cb, const float *x, float *y,
                size_t out, size_t in)
{
    ND_ENTER(ctx);
    return launch_gemv(ctx, 1, w, 0, cb, 0, x, 0, y, 0, out, in);
}

int nd_cb8_gemv_batched(nd_ctx *ctx, size_t count, const uint8_t *w, size_t w_stride,
                        const float *cb, size_t cb_stride, const float *x, size_t x_stride,
                        float *y, size_t y_stride, size_t out, size_t in)
{
    ND_ENTER(ctx);
    return launch_gemv(ctx, count, w, w_stride, cb, cb_stride, x, x_stride, y, y_stride, out, in);
}

int nd_cb8_gemm_batched(nd_ctx *ctx, size_t count, const float *x, size_t x_stride,
                        const uint8_t *w, size_t w_stride, const float *cb, size_t cb_stride,
                        float *y, size_t y_stride, size_t m, size_t out, size_t in)
{
    ND_ENTER(ctx);
    if (count == 0) return ND_OK;
    ND_REQUIRE(x && w && cb && y, "null buffer");
    ND_REQUIRE(m > 0 && out > 0 && in > 0, "empty shape");
    ND_REQUIRE(count <= 65535, "count %zu above 65535", count);
    ND_REQUIRE(out % kGN == 0, "out (%zu) must be a multiple of %d", out, kGN);
    ND_REQUIRE(in % 32 == 0, "in (%zu) must be a multiple of 32", in);
    ND_REQUIRE(m <= (size_t(1) << 24) && out <= (size_t(1) << 24) && in <= (size_t(1) << 24),
               "shape too large");
    ND_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(w) & 7) == 0 &&
                   x_stride % 4 == 0 && w_stride % 8 == 0,
               "x must be 16-byte and w 8-byte aligned, problem by problem");
    const size_t big_tiles = (out / kPN) * ((m + kPM - 1) / kPM) * count;
    const size_t cus = size_t(ctx->num_cus > 0 ? ctx->num_cus : 256);
    const size_t m64_tiles = (out / kRN) * count;
    const bool use_m64 = m <= 64 && out % kRN == 0 && in % kRC == 0 &&
                         (reinterpret_cast<uintptr_t>(w) & 15) == 0 && w_stride % 16 == 0 &&
                         m64_tiles <= 0x7fffffff;
    const bool use_256 = !use_m64 && m >= 96 && out % kPN == 0 && big_tiles >= cus && big_tiles <= 0x7fffffff;
    // X to bf16 once per call, into the context workspace, for the kernels
    // that stage bf16 X; the 256x256 kernel rounds fp32 X as it stages it
    const size_t mk = m * in;
    unsigned short *xb = nullptr;
    if (!use_256) {
        void *wsp = nullptr;
        if (int rc = nd::workspace(ctx, count * mk * sizeof(unsigned short), &wsp)) return rc;
        xb = static_cast<unsigned short *>(wsp);
        hipLaunchKernelGGL(x_to_bf16_kernel, dim3(unsigned((mk + 2048 * kXRuns - 1) / (2048 * kXRuns)), unsigned(count)),
                           dim3(256), 0, ctx->stream, x, x_stride, xb, mk);
        if (int rc = nd::check_launch("x_to_bf16")) return rc;
    }
    if (use_m64) {
        // codes streamed into registers, 128 columns a block
        const int run = m64_tiles % 8 == 0 ? int(m64_tiles / 8) : 0;
        hipLaunchKernelGGL(cb8_gemm_m64_kernel, dim3(unsigned(m64_tiles)), dim3(256), 0, ctx->stream, xb, w,
                           cb, y, int(m), int(out), int(in), w_stride, cb_stride, y_stride,
                           int(out / kRN), run);
    } else if (use_256) {
        // at least one 256x256 tile per CU: below that the 128x128 tiles fill
        // the chip better
        const int run = big_tiles % 8 == 0 ? int(big_tiles / 8) : 0;
        hipLaunchKernelGGL(cb8_gemm256_kernel, dim3(unsigned(big_tiles)), dim3(512), 0, ctx->stream, x,
                           x_stride, w, cb, y, int(m), int(out), int(in), w_stride, cb_stride, y_stride,
                           int(out / kPN), int((m + kPM - 1) / kPM), run);
    } else if (m >= 96 && out % kBN == 0) {
        dim3 grid(static_cast<unsigned>(out / kBN), static_cast<unsigned>((m + kBM - 1) / kBM),
                  static_cast<unsigned>(count));
        hipLaunchKernelGGL(cb8_gemm128_kernel, grid, dim3(256), 0, ctx->stream, xb, w, cb, y,
                           int(m), int(out), int(in), w_stride, cb_stride, y_stride);
    } else {
        dim3 grid(static_cast<unsigned>(out / kGN), static_cast<unsigned>((m + kGM - 1) / kGM),
                  static_cast<unsigned>(count));
        hipLaunchKernelGGL(cb8_gemm_kernel, grid, dim3(256), 0, ctx->stream, xb, w, cb, y, int(m),
                           int(out), int(in), w_stride, cb_stride, y_stride);
    }
    return nd::check_launch("cb8_gemm");
}

int nd_cb8_gemm(nd_ctx *ctx, const float *x, const uint8_t *w, const float *cb, float *y,
                size_t m, size_t out, size_t in)
{
    return nd_cb8_gemm_batched(ctx, 1, x, 0, w, 0, cb, 0, y, 0, m, out, in);
}

}  // extern "C"
