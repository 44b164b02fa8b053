// Format A: Cactus-Quants weights (crates/needle-core/src/cq.rs).
//
// A logical [out, in] matrix stored as packed LSB-first 2/3/4-bit codes (or
// ternary crumbs) per row, one FP16 norm per (row, 128-wide group), levels
// from a shared codebook; reconstruction w_g = (levels[idx] * norm) @ H with
// H the normalised Walsh-Hadamard matrix, applied to the activation instead
// (cq.rs:1-48).
//
// Kernels:
//   cq_prepare   per-group normalised FWHT of the activation (cq.rs:264-274).
//                Same butterfly, same pairing, same final multiply as
//                hadamard.rs:24-55, so the result is bit-identical.
//   cq_gemv      decode GEMV for the byte-aligned widths.  16 lanes per row,
//                each lane keeps its 48 activations in registers and reads
//                one code dword per step; the byte LUT (256 x P levels) sits
//                in LDS in lane-private replicas so the gathers do not
//                conflict on banks; a group's norm multiplies the group dot
//                as in cq.rs:731.
//   cq_gemv_generic   any width/group (3-bit, tiny groups): bit reader.
//   cq_matmul    batched prefill: a 64x64 output tile, the weight tile
//                decoded to fp32 (level * norm) in LDS, fp32 MFMA 16x16x4.
//   cq_dequant   dequantize_row (cq.rs:763-779), bit-identical.
#include "nd_internal.h"
#include "nd_cq_internal.h"
#include "nd_lanes.h"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

namespace {

constexpr uint8_t kTernary = 5;
constexpr size_t kCodebookLen = 28;
constexpr size_t kMaxGroup = 1024;

// cq.rs:948-958
__host__ __device__ inline int ternary_index(uint32_t code)
{
    return code == 3 ? 0 : (code == 1 ? 2 : 1);
}


// ---------------------------------------------------------------------------
// prepare_input: one block per (group, batch row).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(512) void cq_prepare_kernel(const float *__restrict__ x,
                                                         float *__restrict__ xh, int in_feat,
                                                         int in_padded, int group, float inv)
{
    extern __shared__ float buf[];
    const int g = blockIdx.x;
    const size_t b = blockIdx.y;
    const int t = threadIdx.x;
    const float *xr = x + b * size_t(in_feat);
    for (int k = t; k < group; k += blockDim.x) {
        const int col = g * group + k;
        buf[k] = col < in_feat ? xr[col] : 0.0f;
    }
    __syncthreads();
    for (int h = 1; h < group; h <<= 1) {
        for (int i = t; i < group / 2; i += blockDim.x) {
            const int jj = (i / h) * (2 * h) + (i % h);
            const float a = buf[jj];
            const float c = buf[jj + h];
            buf[jj] = a + c;
            buf[jj + h] = a - c;
        }
        __syncthreads();
    }
    float *out = xh + b * size_t(in_padded) + size_t(g) * group;
    for (int k = t; k < group; k += blockDim.x) out[k] = buf[k] * inv;
}

// ---------------------------------------------------------------------------
// GEMV, byte-aligned widths.  P levels per byte (4: 2-bit/ternary, 2: 4-bit).
// ND code dwords per lane; each dword holds 4*P elements of one group.
// ---------------------------------------------------------------------------
constexpr int kThreads = 256;
constexpr int kLanesPerRow = 16;
constexpr int kRowsPerPass = kThreads / kLanesPerRow;  // 16
constexpr int kPasses = 4;                              // 64 rows per block

template <int P>
struct LutVec;
template <>
struct LutVec<4> {
    using T = float4;
};
template <>
struct LutVec<2> {
    using T = float2;
};

// REPL replicas of the P-float entry, entry-major: entry e replica r at
// (e * REPL + r) * P floats.  Lane l reads replica l % REPL.
template <int P, int ND, int REPL>
__global__ __launch_bounds__(kThreads) void cq_gemv_kernel(
    const uint8_t *__restrict__ packed, const float *__restrict__ norms,
    const float *__restrict__ lut, const float *__restrict__ xh, float *__restrict__ y,
    int row_start, int rows, int row_bytes, int num_groups, int group)
{
    using V = typename LutVec<P>::T;
    constexpr int E = 4 * P;  // elements per code dword
    __shared__ V rep[256 * REPL];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int j = t & (kLanesPerRow - 1);
    const int rg = t / kLanesPerRow;
    const int row_dwords = row_bytes >> 2;

    for (int f = t; f < 256 * REPL; f += kThreads) {
        const int e = f / REPL;
        rep[f] = *reinterpret_cast<const V *>(lut + e * P);
    }
    // Lane j owns dwords j + 16*i: elements [E*d, E*d + E).
    float xr[ND][E];
    int gi[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) {
        const int d = j + kLanesPerRow * i;
        gi[i] = (d * E) / group;
        if (d < row_dwords) {
            const float4 *xp = reinterpret_cast<const float4 *>(xh + d * E);
#pragma unroll
            for (int q = 0; q < E / 4; ++q) {
                float4 v = xp[q];
                xr[i][4 * q + 0] = v.x;
                xr[i][4 * q + 1] = v.y;
                xr[i][4 * q + 2] = v.z;
                xr[i][4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < E; ++q) xr[i][q] = 0.0f;
        }
    }
    __syncthreads();

    const V *lutl = rep + (lane & (REPL - 1));
    const int r0 = blockIdx.x * (kRowsPerPass * kPasses);
    uint32_t codes[kPasses][ND];
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        const int r = r0 + rg + kRowsPerPass * p;
        const uint32_t *wr =
            reinterpret_cast<const uint32_t *>(packed + size_t(row_start + r) * row_bytes);
#pragma unroll
        for (int i = 0; i < ND; ++i) {
            const int d = j + kLanesPerRow * i;
            codes[p][i] = (r < rows && d < row_dwords) ? __builtin_nontemporal_load(wr + d) : 0u;
        }
    }
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        const int r = r0 + rg + kRowsPerPass * p;
        const float *nr = norms + size_t(row_start + (r < rows ? r : 0)) * num_groups;
        float total = 0.0f;
#pragma unroll
        for (int i = 0; i < ND; ++i) {
            const int d = j + kLanesPerRow * i;
            float acc[P];
#pragma unroll
            for (int q = 0; q < P; ++q) acc[q] = 0.0f;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t e = (codes[p][i] >> (8 * b)) & 0xffu;
                const V v = lutl[e * REPL];
                const float *vf = reinterpret_cast<const float *>(&v);
#pragma unroll
                for (int q = 0; q < P; ++q) acc[q] += vf[q] * xr[i][b * P + q];
            }
            float dot = acc[0];
#pragma unroll
            for (int q = 1; q < P; ++q) dot += acc[q];
            if (r < rows && d < row_dwords) total += nr[gi[i]] * dot;
        }
        total += ndl::wave_xor<8>(total);
        total += ndl::wave_xor<4>(total);
        total += ndl::wave_xor<2>(total);
        total += ndl::wave_xor<1>(total);
        if (j == 0 && r < rows) y[r] = total;
    }
}

// The streaming form of the same GEMV: a workgroup owns a contiguous run of
// 16-row tiles, builds the LUT replicas and loads its activations once, and
// keeps the codes and norms of the next D tiles in registers while it works
// on the current one.  Lane j of a row owns the ND consecutive code dwords
// from j * ND, read as one run (wide loads).  Past the last row a lane reads the
// last row again and stores nothing, so every load is unconditional and the
// compiler waits for the oldest tile only.  Needs row_dwords == 16 * ND.
template <int ND>
struct CodeRun {
    uint32_t v[ND];
};

template <int P, int ND, int REPL, int D>
__global__ __launch_bounds__(kThreads) void cq_gemv_stream_kernel(
    const uint8_t *__restrict__ packed, const float *__restrict__ norms,
    const float *__restrict__ lut, const float *__restrict__ xh, float *__restrict__ y,
    int row_start, int rows, int row_bytes, int num_groups, int group, int tiles_per_block)
{
    using V = typename LutVec<P>::T;
    using CV = CodeRun<ND>;
    constexpr int E = 4 * P;  // elements per code dword
    __shared__ V rep[256 * REPL];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int j = t & (kLanesPerRow - 1);
    const int rg = t / kLanesPerRow;

    for (int f = t; f < 256 * REPL; f += kThreads) {
        const int e = f / REPL;
        rep[f] = *reinterpret_cast<const V *>(lut + e * P);
    }
    // lane j's activations: elements [j * ND * E, (j + 1) * ND * E)
    // the lane's ND * E <= group elements span groups g0 and g0 + 1 at most
    float xr[ND][E];
    const int g0 = (j * ND * E) / group;
    bool second[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) {
        const int d = j * ND + i;
        second[i] = (d * E) / group != g0;
        const float4 *xp = reinterpret_cast<const float4 *>(xh + d * E);
#pragma unroll
        for (int q = 0; q < E / 4; ++q) {
            const float4 v = xp[q];
            xr[i][4 * q + 0] = v.x;
            xr[i][4 * q + 1] = v.y;
            xr[i][4 * q + 2] = v.z;
            xr[i][4 * q + 3] = v.w;
        }
    }
    __syncthreads();

    const V *lutl = rep + (lane & (REPL - 1));
    const int ntiles = (rows + kRowsPerPass - 1) / kRowsPerPass;
    const int tile0 = blockIdx.x * tiles_per_block;
    const int tile1 = tile0 + tiles_per_block < ntiles ? tile0 + tiles_per_block : ntiles;
    const int g1 = g0 + 1 < num_groups ? g0 + 1 : g0;
    CV cb[D];
    float nb[D][2];
    auto load = [&](int tile, CV &c, float (&nr)[2]) {
        int r = tile * kRowsPerPass + rg;
        r = r < rows ? r : rows - 1;
        const uint8_t *wr = packed + size_t(row_start + r) * row_bytes;
        __builtin_memcpy(&c, wr + size_t(j) * (4 * ND), 4 * ND);
        const float *nrow = norms + size_t(row_start + r) * num_groups;
        nr[0] = nrow[g0];
        nr[1] = nrow[g1];
    };
#pragma unroll
    for (int k = 0; k < D; ++k) load(tile0 + k, cb[k], nb[k]);
    for (int tile = tile0; tile < tile1; tile += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            const int tt = tile + k;
            if (tt < tile1) {
                float total = 0.0f;
#pragma unroll
                for (int i = 0; i < ND; ++i) {
                    const uint32_t dw = cb[k].v[i];
                    float acc[P];
#pragma unroll
                    for (int q = 0; q < P; ++q) acc[q] = 0.0f;
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const uint32_t e = (dw >> (8 * b)) & 0xffu;
                        const V v = lutl[e * REPL];
                        const float *vf = reinterpret_cast<const float *>(&v);
#pragma unroll
                        for (int q = 0; q < P; ++q) acc[q] += vf[q] * xr[i][b * P + q];
                    }
                    float dot = acc[0];
#pragma unroll
                    for (int q = 1; q < P; ++q) dot += acc[q];
                    total += (second[i] ? nb[k][1] : nb[k][0]) * dot;
                }
                total += ndl::wave_xor<8>(total);
                total += ndl::wave_xor<4>(total);
                total += ndl::wave_xor<2>(total);
                total += ndl::wave_xor<1>(total);
                const int r = tt * kRowsPerPass + rg;
                if (j == 0 && r < rows) y[r] = total;
            }
            load(tt + D, cb[k], nb[k]);
        }
    }
}

// Streaming shape shared by the batch-1 GEMVs below.  A launch's row tiles
// are dealt to its workgroups round-robin (tile = blockIdx.x + it *
// gridDim.x), so at any moment the workgroups read one contiguous front of
// the weight.  Each workgroup keeps the codes and norms of its next D tiles
// in registers, issuing a tile's refill right after the tile is consumed;
// scheduling barriers hold that order, so each wait covers the oldest tile
// only and the loads in flight slide instead of draining.  The first D
// tiles are requested before the workgroup's lookup table is built.
// Row results are staged in LDS and written out by whole tiles (coalesced,
// nontemporal) every CAP tiles and at the end: a global store inside the
// loop would put its write round trip under the next wait.  Rows past the
// end reread the last row; the loop body has no branches.

// Batch-1 GEMV on 2-bit (and ternary) rows of 16 * ND code dwords, ND <= 3
// (in <= 768), by product lookup.  Each workgroup first builds, from the
// prepared activation, T(p, e) = lvl(e & 3) * xh[2p] + lvl(e >> 2) * xh[2p+1]
// for every nibble position p of a row and nibble value e, so a code nibble
// costs one 4-byte LDS gather and one add: half the LDS bytes of the level
// table (a 16-byte read per code byte) and half its VALU work.
// Lane j of a 16-lane row group owns code dwords j * ND .. j * ND + ND - 1,
// nibble positions 8 * ND * j + 8 i + s (dword i, nibble s).  Four shifted
// copies of a dword put nibbles 2q and 2q + 1 at bits 7-10 and 11-14 of copy
// q, so a gather address is one and-or with the lane's base; the table keeps
// the even nibbles' entries at e << 7 (subtable k = 4i + q at k << 11) and
// the odd ones' at 32 KiB + (e << 11) (subtable k at k << 7), the subtable
// offset riding in the instruction.  Every entry is a 32-dword block indexed
// [row group & 1][j]: the two row groups of a half-wave read disjoint banks,
// so a gather does not conflict whatever codes the lanes hold.  Two
// 1024-thread workgroups share a CU, each streaming 64-row tiles as above.
// The 16 partial sums of a row meet through DPP row rotations.
constexpr int kNibThreads = 1024;
constexpr int kNibRows = kNibThreads / kLanesPerRow;  // 64 rows per tile
constexpr int kNibDepth = 4;                          // tiles in flight
constexpr int kNibStage = 16;                         // staged tiles (4 KiB)

__device__ inline float row16_sum(float v)
{
    // rotations within a 16-lane DPP row: 8, 4, 2, 1 (row_ror:n = 0x120 + n);
    // every lane has a source, so bound_ctrl is moot and each step fuses
    // into one v_add_f32_dpp
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xf, 0xf, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x122, 0xf, 0xf, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121, 0xf, 0xf, true));
    return v;
}

// ND code dwords from byte offset `off` of the buffer (one load).
template <int ND>
__device__ inline void load_dwords(__amdgpu_buffer_rsrc_t rc, int off, uint32_t *c)
{
    if constexpr (ND == 1) {
        c[0] = __builtin_amdgcn_raw_buffer_load_b32(rc, off, 0, 2);
    } else if constexpr (ND == 2) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rc, off, 0, 2);
        c[0] = v[0];
        c[1] = v[1];
    } else {
        const auto v = __builtin_amdgcn_raw_buffer_load_b96(rc, off, 0, 2);
        c[0] = v[0];
        c[1] = v[1];
        c[2] = v[2];
    }
}

// A workgroup barrier ordering LDS accesses only: unlike __syncthreads it
// does not wait for the global loads in flight.
__device__ inline void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The staged results of tiles it_end - count .. it_end - 1 (rpt rows a
// tile, at stage[(it % cap) * rpt]) written to y, nontemporal; between two
// barriers, so all NT threads of the workgroup call it.  (NT is a constant:
// blockDim.x is a load from the dispatch packet, and its wait would drain
// the loads in flight.)
template <int NT>
__device__ inline void flush_stage(const float *stage, int cap, int rpt, int it_end, int count,
                                   int iters, int rows, float *y)
{
    lds_barrier();
    for (int f = int(threadIdx.x); f < count * rpt; f += NT) {
        const int it = it_end - count + f / rpt;
        const int r = (int(blockIdx.x) + it * int(gridDim.x)) * rpt + f % rpt;
        if (it < iters && r < rows) __builtin_nontemporal_store(stage[(it % cap) * rpt + f % rpt], y + r);
    }
    lds_barrier();
}

template <int ND>
__global__ __launch_bounds__(kNibThreads, 2) void cq_gemv_nib_kernel(
    const uint8_t *__restrict__ packed, const float *__restrict__ norms,
    const float *__restrict__ lut, const float *__restrict__ xh, float *__restrict__ y,
    int row_start, int rows, int row_bytes, int num_groups, int group, int iters)
{
    constexpr int NI = 8 * ND;  // nibble positions per lane
    constexpr int D = kNibDepth;
    __shared__ float tab[16384];  // 64 KiB
    __shared__ float stage[kNibStage * kNibRows];
    const int t = threadIdx.x;
    const int j = t & (kLanesPerRow - 1);
    const int rg = t / kLanesPerRow;  // row of the tile
    // the lane's ND * 16 elements span groups g0 and g0 + 1 at most
    const int g0 = (j * ND * 16) / group;
    const int g1 = g0 + 1 < num_groups ? g0 + 1 : g0;
    // the launch's rows through buffer resources: 32-bit offsets (the caller
    // keeps rows * row_bytes and rows * num_groups * 4 below 2^31)
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(packed + size_t(row_start) * row_bytes), (short)0, rows * row_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rn = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(norms + size_t(row_start) * num_groups), (short)0, rows * num_groups * 4, 0x00020000);
    const int ntiles = (rows + kNibRows - 1) / kNibRows;
    uint32_t cb[D][ND];
    float nb[D][2];
    auto load = [&](int it, int k) {
        int tile = int(blockIdx.x) + it * int(gridDim.x);
        tile = tile < ntiles ? tile : ntiles - 1;
        int r = tile * kNibRows + rg;
        r = r < rows ? r : rows - 1;
        // rows < 2^24 here, so 24-bit multiplies give the offsets; codes are
        // read once: nontemporal
        load_dwords<ND>(rc, int(__umul24(uint32_t(r), uint32_t(row_bytes))) + j * (4 * ND), cb[k]);
        const int no = int(__umul24(uint32_t(r), uint32_t(num_groups * 4)));
        nb[k][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rn, no + 4 * g0, 0, 0));
        nb[k][1] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rn, no + 4 * g1, 0, 0));
    };
#pragma unroll
    for (int k = 0; k < D; ++k) {
        load(k, k);
        __builtin_amdgcn_sched_barrier(0);
    }
    // lut[4c] is the level of code c (byte value c, first crumb), ternary
    // crumb map included
    for (int f = t; f < 16 * NI * kLanesPerRow; f += kNibThreads) {
        const int fj = f % kLanesPerRow, n = (f / kLanesPerRow) % NI, e = f / (kLanesPerRow * NI);
        const int p = fj * NI + n;
        const float v = lut[(e & 3) * 4] * xh[2 * p] + lut[(e >> 2) * 4] * xh[2 * p + 1];
        const int i = n / 8, sn = n % 8, k = 4 * i + sn / 2;
        const int at = (sn & 1) ? 0x8000 | (e << 11) | (k << 7) : (k << 11) | (e << 7);
        tab[at / 4 + fj] = v;
        tab[at / 4 + 16 + fj] = v;
    }
    bool second[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) second[i] = ((j * ND + i) * 16) / group != g0;
    __syncthreads();

    const uint32_t lb = uint32_t(((rg & 1) * kLanesPerRow + j) * 4);
    const char *tb = reinterpret_cast<const char *>(tab);
    for (int it0 = 0; it0 < iters; it0 += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            const int it = it0 + k;
            float total = 0.0f;
#pragma unroll
            for (int i = 0; i < ND; ++i) {
                const uint32_t dw = cb[k][i];
                const uint32_t cq[4] = {dw << 7, dw >> 1, dw >> 9, dw >> 17};
                float dot = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int kk = 4 * i + q;
                    const float lo = *reinterpret_cast<const float *>(tb + ((cq[q] & 0x780u) | lb) + (kk << 11));
                    const float hi =
                        *reinterpret_cast<const float *>(tb + ((cq[q] & 0x7800u) | lb) + (0x8000 | (kk << 7)));
                    dot = q == 0 ? lo + hi : dot + lo + hi;
                }
                total += (second[i] ? nb[k][1] : nb[k][0]) * dot;
            }
            total = row16_sum(total);
            stage[(it % kNibStage) * kNibRows + rg] = total;  // the row's 16 lanes agree
            __builtin_amdgcn_sched_barrier(0);
            load(it + D, k);
            __builtin_amdgcn_sched_barrier(0);
            if ((it + 1) % kNibStage == 0) flush_stage<kNibThreads>(stage, kNibStage, kNibRows, it + 1, kNibStage, iters, rows, y);
        }
    }
    // the loop ran to a multiple of D; flush what the last full stage left
    const int done = (iters + D - 1) / D * D;
    if (done % kNibStage) flush_stage<kNibThreads>(stage, kNibStage, kNibRows, done, done % kNibStage, iters, rows, y);
}

// Batch-1 GEMV on 4-bit rows of 16 * ND code dwords, ND = 4..6 (in 512 to
// 768), by byte lookup: a byte's two levels come from a 256-entry table of
// float2 in LDS (REPL = 32 replicas, lane l reading replica l % 32) and
// multiply the lane's activations held in registers.  An entry's replicas
// fill 256 bytes, so a lookup address is the code byte in bits 8-15 over
// the lane's replica offset in bits 3-7: one v_perm_b32 of the code dword
// and that offset, no shift and mask.  Lane j of a 16-lane
// row group holds code bytes [16 j, 16 j + 16) (elements 32 j .. 32 j + 31,
// one 128-bit load) and, for ND > 4, bytes [256 + 4 B j, 256 + 4 B (j + 1))
// with B = ND - 4 (elements 512 + 8 B j ..): every load of a row group
// covers a contiguous run of its row, and each part lies in one group when
// the group is a multiple of 32.  512-thread workgroups (32-row tiles, one
// 128-byte line of results each), two a CU, streaming as above.
constexpr int kQ4Threads = 512;
constexpr int kQ4Rows = kQ4Threads / kLanesPerRow;  // 32 rows per tile
constexpr int kQ4Repl = 32;                        // 256 B an entry
static_assert(kQ4Repl * 8 == 256, "a lookup address puts the code byte at bit 8");
constexpr int kQ4Depth = 4;
constexpr int kQ4Stage = 32;                        // staged tiles (4 KiB)

template <int ND>
__global__ __launch_bounds__(kQ4Threads) void cq_gemv_q4_kernel(
    const uint8_t *__restrict__ packed, const float *__restrict__ norms,
    const float *__restrict__ lut, const float *__restrict__ xh, float *__restrict__ y,
    int row_start, int rows, int row_bytes, int num_groups, int group, int iters)
{
    constexpr int B = ND - 4;  // dwords of the second part
    constexpr int D = kQ4Depth;
    __shared__ float2 rep[256 * kQ4Repl];  // 64 KiB
    __shared__ float stage[kQ4Stage * kQ4Rows];
    const int t = threadIdx.x, lane = t & 63, j = t & (kLanesPerRow - 1), rg = t / kLanesPerRow;
    // the lane's activations: part A elements 32 j + 8 i + e (i < 4), part B
    // 512 + 8 B j + 8 (i - 4) + e
    float xr[ND][8];
#pragma unroll
    for (int i = 0; i < ND; ++i) {
        const int d = i < 4 ? 4 * j + i : 64 + B * j + (i - 4);
        const float4 *xp = reinterpret_cast<const float4 *>(xh + d * 8);
        const float4 a = xp[0], b = xp[1];
        xr[i][0] = a.x;
        xr[i][1] = a.y;
        xr[i][2] = a.z;
        xr[i][3] = a.w;
        xr[i][4] = b.x;
        xr[i][5] = b.y;
        xr[i][6] = b.z;
        xr[i][7] = b.w;
    }
    // the activations are loop invariants: an empty asm reading them puts
    // the wait for their loads here, so the loop's waits do not count them
    // as pending on every pass
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
        for (int q = 0; q < 8; ++q) asm volatile("" ::"v"(xr[i][q]) : "memory");
    const int ga = (32 * j) / group, gb = B > 0 ? (512 + 8 * B * j) / group : ga;
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(packed + size_t(row_start) * row_bytes), (short)0, rows * row_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rn = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(norms + size_t(row_start) * num_groups), (short)0, rows * num_groups * 4, 0x00020000);
    const int ntiles = (rows + kQ4Rows - 1) / kQ4Rows;
    uint32_t cb[D][ND];
    float na[D], nb[D];
    auto load = [&](int it, int k) {
        int tile = int(blockIdx.x) + it * int(gridDim.x);
        tile = tile < ntiles ? tile : ntiles - 1;
        int r = tile * kQ4Rows + rg;
        r = r < rows ? r : rows - 1;
        const int ro = int(__umul24(uint32_t(r), uint32_t(row_bytes)));
        const auto a = __builtin_amdgcn_raw_buffer_load_b128(rc, ro + 16 * j, 0, 2);
        cb[k][0] = a[0];
        cb[k][1] = a[1];
        cb[k][2] = a[2];
        cb[k][3] = a[3];
        if constexpr (B == 1) {
            cb[k][4] = __builtin_amdgcn_raw_buffer_load_b32(rc, ro + 256 + 4 * j, 0, 2);
        } else if constexpr (B == 2) {
            const auto b = __builtin_amdgcn_raw_buffer_load_b64(rc, ro + 256 + 8 * j, 0, 2);
            cb[k][4] = b[0];
            cb[k][5] = b[1];
        }
        const int no = int(__umul24(uint32_t(r), uint32_t(num_groups * 4)));
        na[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rn, no + 4 * ga, 0, 0));
        nb[k] = B > 0 ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rn, no + 4 * gb, 0, 0))
                      : 0.0f;
    };
#pragma unroll
    for (int k = 0; k < D; ++k) {
        load(k, k);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int f = t; f < 256 * kQ4Repl; f += kQ4Threads)
        rep[f] = *reinterpret_cast<const float2 *>(lut + (f / kQ4Repl) * 2);
    __syncthreads();

    // byte 0 of a lookup address: the lane's replica (8 bytes each)
    const uint32_t lb = uint32_t(lane & (kQ4Repl - 1)) * uint32_t(sizeof(float2));
    const char *repb = reinterpret_cast<const char *>(rep);
    for (int it0 = 0; it0 < iters; it0 += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            const int it = it0 + k;
            float ta = 0.0f, tb = 0.0f;
#pragma unroll
            for (int i = 0; i < ND; ++i) {
                const uint32_t dw = cb[k][i];
                float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    // bytes of (dw, lb): selector 4 + b is byte b of dw, 0 is
                    // byte 0 of lb, 0x0c a zero byte
                    const uint32_t at = __builtin_amdgcn_perm(dw, lb, 0x0c0c0000u | ((4u + b) << 8));
                    const float2 v = *reinterpret_cast<const float2 *>(repb + at);
                    a0 += v.x * xr[i][2 * b];
                    a1 += v.y * xr[i][2 * b + 1];
                }
                if (i < 4)
                    ta += a0 + a1;
                else
                    tb += a0 + a1;
            }
            float total = na[k] * ta + nb[k] * tb;
            total = row16_sum(total);
            stage[(it % kQ4Stage) * kQ4Rows + rg] = total;  // the row's 16 lanes agree
            __builtin_amdgcn_sched_barrier(0);
            load(it + D, k);
            __builtin_amdgcn_sched_barrier(0);
            if ((it + 1) % kQ4Stage == 0) flush_stage<kQ4Threads>(stage, kQ4Stage, kQ4Rows, it + 1, kQ4Stage, iters, rows, y);
        }
    }
    const int done = (iters + D - 1) / D * D;
    if (done % kQ4Stage) flush_stage<kQ4Threads>(stage, kQ4Stage, kQ4Rows, done, done % kQ4Stage, iters, rows, y);
}

// Batch-1 GEMV on 2-bit (and ternary) rows of NG groups of 128 (in <= 768)
// on the matrix cores: v_mfma_scale_f32_16x16x128_f8f6f4 with both
// operands fp4 (e2m1: a sign, two exponent bits, one mantissa bit), for the
// tolerance arithmetic of the row dot.  The lookup kernels above spend ~18
// VALU instructions a row per CU; this one ~7, so it stays bound by HBM
// where the others are held back by the clock.
//
// Codes as fp4 planes.  A 2-bit code c = 2 b1 + b0 placed at bits 0-1, 1-2
// or 2-3 of a zero nibble reads, as e2m1, P1(c) = {0, 0.5, 1, 1.5},
// P2(c) = {0, 1, 2, 4} or P3(c) = {0, 2, -0, -2}.  With the constant these
// span every function of c, so lvl(c) = L0 + beta P1(c) + gamma P2(c) +
// delta P3(c) for any four levels.  `dw & 0x33333333` leaves the even codes
// of a dword at nibble bits 0-1 and `dw & 0xcccccccc` the odd ones at bits
// 2-3; two shifts of each give the other two planes, so 16 codes become
// three planes of 16 nibbles in six VALU operations.
//
// The activation as fp4 pieces.  Over each 32-element block, coef_p * x is
// split into kMf2Pieces pieces, each with its own power-of-two (E8M0)
// scale: piece i is the residual the earlier pieces left, rounded to e2m1
// at scale 2^(s0 - drop(i)), s0 mapping the block's largest magnitude into
// [-6, 6]; from the third piece on each takes three more bits, and ten
// leave under 2^-28 of that magnitude.  Each workgroup builds them as MFMA
// A fragments in LDS while its first tiles load (the hardware's scaled
// f32 -> fp4 conversion rounds to nearest even and its inverse is exact):
// row i of A is piece i, the 128 K of one MFMA the 128 elements of one
// group, in the plane order below.
//
// Per 16 rows, one MFMA per (group, plane): D[i][c] = sum_k A[i][k] B[k][c]
// with column c of B the plane of weight row c; a group's three planes
// accumulate into one D, whose 16 piece rows add up to
// sum_k (lvl(c_k) - L0) x_k.  Lane c + 16 q holds weight row c: as B its
// slice q of each group (codes 32 q .. 32 q + 31, two dwords), and D rows
// 4 q .. 4 q + 3, which it sums and scales by the group's norm; slice 0
// adds L0 X_g (X_g the group's activation sum), and two lane exchanges
// finish the row.  In nibble order B's dword 0 holds codes 32 q + 2 n
// (n = 0..7), dword 1 codes 32 q + 2 n + 1, dwords 2 and 3 the same from
// code 32 q + 16 on; the A fragments follow that order.  Products of fp4
// values are exact; the matrix core adds them in fp32.
//
// Four waves a workgroup, 16 rows each (64-row tiles dealt round-robin),
// two workgroups a CU, kMf2Depth tiles of loads in flight, results staged
// in LDS and written out as in the lookup kernels.  A wave loads its 16
// rows as one contiguous run and regroups them into MFMA slices through
// LDS: loading the slices directly (32 bytes of 16 rows per load) ran at
// 60% of the contiguous rate.  An activation holding a non-finite value
// (which fp4 cannot carry), one whose coef * x or L0 * X_g leaves the fp32
// range, or one whose coef * x exceeds kMf2MaxBlock takes a plain per-lane
// loop over the same rows instead.
constexpr int kMf2Pieces = 10;
constexpr int kMf2Threads = 256;
constexpr int kMf2Rows = 64;    // rows per tile
constexpr int kMf2Depth = 3;    // tiles in flight
constexpr int kMf2Stage = 16;   // staged tiles (4 KiB)
constexpr int kMf2MaxGroups = 6;
// Below this many rows the lookup kernel is as fast or faster (the rows
// sit in the MALL; measured crossover ~700k rows of in 768).  The
// environment variable NEEDLE_AMD_CQ_FP4_MIN_ROWS, read once when a weight
// is created, overrides it for that weight.
constexpr size_t kMf2MinRows = 655360;
// The largest |coef * x| a block may hold on the matrix cores.  Its first
// piece's scale 2^s0 is below max / 3, and one group's three planes sum at
// most 3 x 128 products of a piece (<= 6 * 2^s0) and a plane value (<= 4):
// 9216 * 2^s0 < 2^13.2 * max / 3.  Below 2^116 that stays under 2^128, so no
// partial sum of the MFMAs can overflow where the reference's products do not.
constexpr float kMf2MaxBlock = 0x1p116f;

typedef int nd_v8i __attribute__((ext_vector_type(8)));
typedef float nd_v4f __attribute__((ext_vector_type(4)));

// Orders LDS accesses between the lanes of one wave: a release and an
// acquire fence at wavefront scope around a wave barrier.  A wave executes
// its LDS instructions in order, so this emits no wait; it keeps the
// compiler from moving LDS accesses across it and makes a lane's read of
// another lane's store well-defined.
__device__ inline void nd_wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Exponent of piece i's scale below the block's first: 0, 2, 4, then 3 more
// a piece.  With the block's largest |v| at most 6 * 2^s0, piece 0 leaves at
// most 2^s0, piece 1 at most 2^(s1 - 1), and from there a residual of at
// most 2 * 2^si leaves at most 2^(si - 2): three bits a piece.
__host__ __device__ constexpr int mf2_piece_drop(int i)
{
    return i == 0 ? 0 : (i == 1 ? 2 : 4 + 3 * (i - 2));
}

// The plane coefficients of four crumb levels L0..L3: lvl(c) - L0 =
// beta P1(c) + gamma P2(c) + delta P3(c) at c = 1, 2, 3.
struct Mf2Coef {
    float beta, gamma, delta, l0;
};

inline Mf2Coef mf2_coef(const float *lv)
{
    const double L0 = lv[0], d1 = double(lv[1]) - L0, d2 = double(lv[2]) - L0, d3 = double(lv[3]) - L0;
    const double gam = d1 + d3 - 2.0 * d2, bet = d2 - 2.0 * gam, del = (d1 - 0.5 * bet - gam) * 0.5;
    return {float(bet), float(gam), float(del), lv[0]};
}

// Maximum over a 16-lane DPP row (every lane receives it).
__device__ inline float row16_max(float v)
{
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xf, 0xf, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x122, 0xf, 0xf, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121, 0xf, 0xf, true)));
    return v;
}

// N consecutive floats from byte offset `off` of the buffer, in loads of up
// to three dwords.  (The elements go through __uint_as_float by value:
// hipcc compiles __builtin_bit_cast of a vector element as a read of
// element 0.)
template <int N>
__device__ inline void load_floats(__amdgpu_buffer_rsrc_t rc, int off, float *v)
{
    if constexpr (N >= 3) {
        const auto a = __builtin_amdgcn_raw_buffer_load_b96(rc, off, 0, 0);
        v[0] = __uint_as_float(a[0]);
        v[1] = __uint_as_float(a[1]);
        v[2] = __uint_as_float(a[2]);
        if constexpr (N > 3) load_floats<N - 3>(rc, off + 12, v + 3);
    } else if constexpr (N == 2) {
        const auto a = __builtin_amdgcn_raw_buffer_load_b64(rc, off, 0, 0);
        v[0] = __uint_as_float(a[0]);
        v[1] = __uint_as_float(a[1]);
    } else if constexpr (N == 1) {
        v[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rc, off, 0, 0));
    }
}

template <int NG>
__global__ __launch_bounds__(kMf2Threads, 2) void cq_gemv_mf2_kernel(
    const uint8_t *__restrict__ packed, const float *__restrict__ norms, const float *__restrict__ lut,
    const float *__restrict__ xh, float *__restrict__ y, Mf2Coef cf, int row_start, int rows,
    int iters)
{
    constexpr int D = kMf2Depth;
    constexpr int RB = 32 * NG;  // row bytes
    constexpr int NF = 3 * NG;   // A fragments: (group, plane)
    constexpr int NT = 4 * NF;   // piece tasks: (fragment, 32-element block)
    constexpr int TPT = (NT + 15) / 16;  // tasks per 16-lane group
    __shared__ float stage[kMf2Stage * kMf2Rows];
    __shared__ uint2 xch[4 * 16 * (RB + 8) / 8];  // per wave: 16 rows, padded
    __shared__ uint4 fr[NF][64];                  // A fragments, lane-major
    __shared__ int s0s[NF][4];                    // each block's first scale exponent
    __shared__ float xpart[NG][4];                // each block's activation sum
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, c = lane & 15, q = lane >> 4;
    // 32-bit buffer offsets (the caller keeps rows * RB below 2^31)
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(packed + size_t(row_start) * RB), (short)0, rows * RB, 0x00020000);
    const __amdgpu_buffer_rsrc_t rn = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(norms + size_t(row_start) * NG), (short)0, rows * NG * 4, 0x00020000);
    const int ntiles = (rows + kMf2Rows - 1) / kMf2Rows;
    auto row_of = [&](int it) {
        int tile = int(blockIdx.x) + it * int(gridDim.x);
        tile = tile < ntiles ? tile : ntiles - 1;
        const int r = tile * kMf2Rows + 16 * w + c;
        return r < rows ? r : rows - 1;
    };
    uint32_t cw[D][NG][2];
    float nw[D][NG];
    auto load = [&](int it, int k) {
        int tile = int(blockIdx.x) + it * int(gridDim.x);
        tile = tile < ntiles ? tile : ntiles - 1;
        // the wave's 16 rows as one contiguous run, 512 bytes a load (rows
        // past the end read as zeros and are not stored); codes are read
        // once: nontemporal
        const int base = (tile * kMf2Rows + 16 * w) * RB + 8 * lane;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(rc, base + 512 * g, 0, 2);
            cw[k][g][0] = v[0];
            cw[k][g][1] = v[1];
        }
        load_floats<NG>(rn, int(__umul24(uint32_t(row_of(it)), uint32_t(NG * 4))), nw[k]);
    };

    // The pieces.  Lane l of a 16-lane group, task (fragment f = 3 g + p,
    // block b): elements e = 32 b + 16 (d >> 1) + 4 u + (d & 1) and e + 2,
    // d = l >> 2, u = l & 3 -- nibbles 2 u and 2 u + 1 of dword d of every
    // lane 16 b + i of the fragment.  The activations are loaded before the
    // first tiles, so their wait does not wait for the tiles.
    const int gl = t & 15, gt = t >> 4;
    const int ed = gl >> 2, eu = gl & 3;
    const int eo = 16 * (ed >> 1) + 4 * eu + (ed & 1);
    float xa[TPT], xb[TPT];
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
        const int task = gt + 16 * j;
        const int tk = task < NT ? task : NT - 1;
        const int e = 128 * ((tk >> 2) / 3) + 32 * (tk & 3) + eo;
        xa[j] = xh[e];
        xb[j] = xh[e + 2];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < D; ++k) {
        load(k, k);
        __builtin_amdgcn_sched_barrier(0);
    }
    bool nonfinite = false;
    uint8_t *frb = reinterpret_cast<uint8_t *>(fr);
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
        const int task = gt + 16 * j;
        if (task < NT) {  // uniform over the 16-lane group
            const int f = task >> 2, b = task & 3, g = f / 3, p = f % 3;
            const float coef = p == 0 ? cf.beta : (p == 1 ? cf.gamma : cf.delta);
            float ra = coef * xa[j], rb = coef * xb[j];
            // a non-finite activation, or coef * x past the fp32 range
            nonfinite = nonfinite || !isfinite(ra) || !isfinite(rb);
            // the block's scale: the smallest s0 with max |v| <= 6 * 2^s0
            const float bm = row16_max(fmaxf(fabsf(ra), fabsf(rb)));
            // too close to the top of the range for the MFMA sums
            nonfinite = nonfinite || bm > kMf2MaxBlock;
            int s0 = 0;
            if (bm > 0.0f && isfinite(bm)) {
                const float fm = frexpf(bm / 6.0f, &s0);
                if (fm == 0.5f) --s0;
            }
            uint8_t *dst = frb + (f * 64 + 16 * b) * 16 + 4 * ed + eu;
#pragma unroll
            for (int i = 0; i < kMf2Pieces; ++i) {
                int si = s0 - mf2_piece_drop(i);
                si = si < -126 ? -126 : si;
                const float sc = ldexpf(1.0f, si);
                // RNE(ra / sc) low nibble, RNE(rb / sc) high; back: value * sc
                const uint32_t pk = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, ra, rb, sc, 0);
                const auto back = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(pk, sc, 0);
                ra -= back[0];
                rb -= back[1];
                dst[i * 16] = uint8_t(pk);
            }
            if (gl == 0) s0s[f][b] = s0;
            if (p == 0) {
                float xs = xa[j] + xb[j];
                xs = row16_sum(xs);
                if (gl == 0) xpart[g][b] = xs;
                nonfinite = nonfinite || !isfinite(xa[j]) || !isfinite(xb[j]);
            }
        }
    }
    // fragment rows past the pieces are zero
    for (int z = t; z < NF * 4 * (16 - kMf2Pieces); z += kMf2Threads) {
        const int f = z / (4 * (16 - kMf2Pieces)), rem = z % (4 * (16 - kMf2Pieces));
        fr[f][16 * (rem / (16 - kMf2Pieces)) + kMf2Pieces + rem % (16 - kMf2Pieces)] = make_uint4(0, 0, 0, 0);
    }
    const int bad = __syncthreads_or(nonfinite);
    // after the barrier every thread reads the same group sums, so this
    // test is uniform too
    bool axbad = false;
#pragma unroll
    for (int g = 0; g < NG; ++g)
        axbad = axbad || !isfinite(cf.l0 * (((xpart[g][0] + xpart[g][1]) + xpart[g][2]) + xpart[g][3]));
    if (bad || axbad) {
        // a non-finite activation: lane c + 16 q sums its slices in order
        for (int it = 0; it < iters; ++it) {
            const int r = row_of(it);
            float s = 0.0f;
            for (int g = 0; g < NG; ++g) {
                const uint2 cd = *reinterpret_cast<const uint2 *>(packed + size_t(row_start + r) * RB + 32 * g + 8 * q);
                float part = 0.0f;
                for (int j = 0; j < 32; ++j) {
                    const uint32_t code = ((j < 16 ? cd.x : cd.y) >> (2 * (j & 15))) & 3u;
                    part += lut[4 * code] * xh[128 * g + 32 * q + j];
                }
                s += norms[size_t(row_start + r) * NG + g] * part;
            }
            s += ndl::wave_xor<16>(s);
            s += ndl::wave_xor<32>(s);
            if (q == 0) stage[(it % kMf2Stage) * kMf2Rows + 16 * w + c] = s;
            if ((it + 1) % kMf2Stage == 0)
                flush_stage<kMf2Threads>(stage, kMf2Stage, kMf2Rows, it + 1, kMf2Stage, iters, rows, y);
        }
        if (iters % kMf2Stage)
            flush_stage<kMf2Threads>(stage, kMf2Stage, kMf2Rows, iters, iters % kMf2Stage, iters, rows, y);
        return;
    }
    // The loaded dwords reach their MFMA lanes through LDS: lane L's pair g
    // (byte 512 g + 8 L of the 16 rows) is written at its row and column in
    // the wave's own buffer, rows RS = RB + 8 bytes apart, and lane c + 16 q
    // reads back row c, bytes 32 g + 8 q.  (RS / 8 is odd, so the 16 rows
    // of one such read fall in distinct bank pairs.)  A wave reads only what
    // it wrote, in order: no barrier.
    constexpr int RS = RB + 8;
    uint8_t *xb8 = reinterpret_cast<uint8_t *>(xch) + w * 16 * RS;
    int wo[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int o = 512 * g + 8 * lane;
        wo[g] = (o / RB) * RS + o % RB;
    }
    const int ro = c * RS + 8 * q;
    // this lane's A fragments: piece c of block q
    nd_v8i af[NF];
    int sc[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        const uint4 v = fr[f][lane];
        af[f] = nd_v8i{int(v.x), int(v.y), int(v.z), int(v.w), 0, 0, 0, 0};
        int si = s0s[f][q] - mf2_piece_drop(c < kMf2Pieces ? c : 0);
        sc[f] = (si < -126 ? -126 : si) + 127;
    }
    float axq[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g)
        axq[g] = q == 0 ? cf.l0 * (((xpart[g][0] + xpart[g][1]) + xpart[g][2]) + xpart[g][3]) : 0.0f;
    // loop invariants: wait for them here, not on every pass of the loop
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        asm volatile("" ::"v"(af[f][0]), "v"(af[f][1]), "v"(af[f][2]), "v"(af[f][3]), "v"(sc[f]) : "memory");
    }
#pragma unroll
    for (int g = 0; g < NG; ++g) asm volatile("" ::"v"(axq[g]) : "memory");

    for (int it0 = 0; it0 < iters; it0 += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            const int it = it0 + k;
#pragma unroll
            for (int g = 0; g < NG; ++g)
                *reinterpret_cast<uint2 *>(xb8 + wo[g]) = make_uint2(cw[k][g][0], cw[k][g][1]);
            // the lanes' stores are visible to the wave's reads below
            nd_wave_lds_sync();
            uint2 dds[NG];
#pragma unroll
            for (int g = 0; g < NG; ++g) dds[g] = *reinterpret_cast<const uint2 *>(xb8 + ro + 32 * g);
            // and every read is done before the next pass overwrites the buffer
            nd_wave_lds_sync();
            nd_v4f acc[NG];
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                const uint2 dd = dds[g];
                const uint32_t d0 = dd.x, d1 = dd.y;
                const uint32_t e0 = d0 & 0x33333333u, o0 = d0 & 0xccccccccu;
                const uint32_t e1 = d1 & 0x33333333u, o1 = d1 & 0xccccccccu;
                const nd_v8i b1 = {int(e0), int(o0 >> 2), int(e1), int(o1 >> 2), 0, 0, 0, 0};
                const nd_v8i b2 = {int(e0 << 1), int(o0 >> 1), int(e1 << 1), int(o1 >> 1), 0, 0, 0, 0};
                const nd_v8i b3 = {int(e0 << 2), int(o0), int(e1 << 2), int(o1), 0, 0, 0, 0};
                nd_v4f a = {0.0f, 0.0f, 0.0f, 0.0f};
                // cbsz = blgp = 4: both operands fp4; B's scale 2^0
                a = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[3 * g], b1, a, 4, 4, 0, sc[3 * g], 0, 127);
                a = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[3 * g + 1], b2, a, 4, 4, 0, sc[3 * g + 1], 0, 127);
                a = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[3 * g + 2], b3, a, 4, 4, 0, sc[3 * g + 2], 0, 127);
                acc[g] = a;
            }
            float s = 0.0f;
#pragma unroll
            for (int g = 0; g < NG; ++g)
                s += nw[k][g] * (((acc[g][0] + acc[g][1]) + (acc[g][2] + acc[g][3])) + axq[g]);
            s += ndl::wave_xor<16>(s);
            s += ndl::wave_xor<32>(s);
            if (q == 0) stage[(it % kMf2Stage) * kMf2Rows + 16 * w + c] = s;
            __builtin_amdgcn_sched_barrier(0);
            load(it + D, k);
            __builtin_amdgcn_sched_barrier(0);
            if ((it + 1) % kMf2Stage == 0)
                flush_stage<kMf2Threads>(stage, kMf2Stage, kMf2Rows, it + 1, kMf2Stage, iters, rows, y);
        }
    }
    const int done = (iters + D - 1) / D * D;
    if (done % kMf2Stage)
        flush_stage<kMf2Threads>(stage, kMf2Stage, kMf2Rows, done, done % kMf2Stage, iters, rows, y);
}

// Reads code k of a row with the bit reader of cq.rs:914-925 (any width).
__device__ inline uint32_t read_code(const uint8_t *row, int k, int w, int row_bytes)
{
    const int bit = k * w;
    const int byte = bit >> 3;
    const int shift = bit & 7;
    uint32_t lo = row[byte];
    uint32_t hi = (shift + w > 8 && byte + 1 < row_bytes) ? row[byte + 1] : 0u;
    return ((lo | (hi << 8)) >> shift) & ((1u << w) - 1u);
}

__device__ inline float level_of(const float *lv, uint32_t code, int ternary)
{
    return lv[ternary ? ternary_index(code) : int(code)];
}

// One wave per row, any width: lanes stride the reduction axis and fold
// each group's norm into its terms.
__global__ __launch_bounds__(256) void cq_gemv_generic_kernel(
    const uint8_t *__restrict__ packed, const float *__restrict__ norms,
    const float *__restrict__ lv, const float *__restrict__ xh, float *__restrict__ y,
    int row_start, int rows, int row_bytes, int num_groups, int group, int in_padded, int w,
    int ternary)
{
    __shared__ float lvs[16];
    if (threadIdx.x < 16) lvs[threadIdx.x] = lv[threadIdx.x];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const uint8_t *row = packed + size_t(row_start + r) * row_bytes;
    const float *nr = norms + size_t(row_start + r) * num_groups;
    float total = 0.0f;
    for (int g = 0; g < num_groups; ++g) {
        float acc = 0.0f;
        for (int k = lane; k < group; k += 64) {
            const int kk = g * group + k;
            acc += level_of(lvs, read_code(row, kk, w, row_bytes), ternary) * xh[kk];
        }
        total += nr[g] * acc;
    }
    total = ndl::wave_sum64(total);
    if (lane == 0) y[r] = total;
    (void)in_padded;
}

// ---------------------------------------------------------------------------
// Batched matmul on fp32 MFMA: Y[b][r] = sum_k xh[b][k] * level(W[r][k]) *
// norm[r][k/group].  Tile 64 (batch) x 64 (rows), K steps of 32 (zero-filled
// past in_padded).
// ---------------------------------------------------------------------------
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4_t;
constexpr int kMM = 64, kMN = 64, kMK = 32;

__global__ __launch_bounds__(256) void cq_matmul_kernel(
    const uint8_t *__restrict__ packed, const float *__restrict__ norms,
    const float *__restrict__ lv, const float *__restrict__ xh, float *__restrict__ y,
    int batch, int row_start, int rows, int row_bytes, int num_groups, int group, int in_padded,
    int w, int ternary)
{
    __shared__ float lvs[16];
    __shared__ float As[kMM][kMK + 1];
    __shared__ float Bs[kMN][kMK + 1];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int n0 = blockIdx.x * kMN;  // row tile
    const int m0 = blockIdx.y * kMM;  // batch tile
    const int wm = (wave >> 1) * 32;
    const int wn = (wave & 1) * 32;
    if (t < 16) lvs[t] = lv[t];

    floatx4_t acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int sr = t >> 2;        // staging row 0..63
    const int sc = (t & 3) * 8;   // staging col 0..24
    __syncthreads();
    for (int k0 = 0; k0 < in_padded; k0 += kMK) {
        {
            const int m = m0 + sr;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int k = k0 + sc + q;
                As[sr][sc + q] = (m < batch && k < in_padded) ? xh[size_t(m) * in_padded + k] : 0.0f;
            }
        }
        {
            const int n = n0 + sr;
            if (n < rows) {
                const uint8_t *row = packed + size_t(row_start + n) * row_bytes;
                const float *nr = norms + size_t(row_start + n) * num_groups;
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const int k = k0 + sc + q;
                    Bs[sr][sc + q] = k < in_padded ? level_of(lvs, read_code(row, k, w, row_bytes), ternary) *
                                                         nr[k / group]
                                                   : 0.0f;
                }
            } else {
#pragma unroll
                for (int q = 0; q < 8; ++q) Bs[sr][sc + q] = 0.0f;
            }
        }
        __syncthreads();
        // MFMA 16x16x4 f32: lane l supplies A[l%16][k0+l/16], B[k0+l/16][l%16].
        const int r16 = lane & 15;
        const int kq = lane >> 4;
#pragma unroll
        for (int kk = 0; kk < kMK; kk += 4) {
            float af[2], bf[2];
#pragma unroll
            for (int a = 0; a < 2; ++a) af[a] = As[wm + a * 16 + r16][kk + kq];
#pragma unroll
            for (int b = 0; b < 2; ++b) bf[b] = Bs[wn + b * 16 + r16][kk + kq];
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[a], bf[b], acc[a][b], 0, 0, 0);
        }
        __syncthreads();
    }
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
                if (m < batch && n < rows) y[size_t(m) * rows + n] = acc[a][b][i];
            }
}

// The same product for the byte-aligned widths (4-bit, 2-bit, ternary), the
// prefill path: block tile BM (batch) x 64 (rows), K steps of 32.  X is staged
// with float4 loads; codes 8 at a time (one 16- or 32-bit load), decoded
// through the weight's byte LUT and scaled by the group norm; the next step's
// loads are in flight while the current step's MFMAs run.  Waves 2x2 (BM 64:
// 32x32 each; BM 32: 16x32) or 1x4 (BM 16: 16x16).
template <int P, int BM>
__global__ __launch_bounds__(256) void cq_matmul_b_kernel(
    const uint8_t *__restrict__ packed, const float *__restrict__ norms,
    const float *__restrict__ lut_g, const float *__restrict__ xh, float *__restrict__ y,
    int batch, int row_start, int rows, int row_bytes, int num_groups, int group, int in_padded)
{
    constexpr int BN = 64, BK = 32, LD = BK + 4;
    constexpr int WGM = BM >= 32 ? 2 : 1, WGN = 4 / WGM;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TA = WM / 16, TB = WN / 16;
    constexpr int NA = (BM * BK / 4 + 255) / 256;  // float4s of X per thread per step
    __shared__ __align__(16) float lut[256 * P];
    __shared__ __align__(16) float As[BM][LD];
    __shared__ __align__(16) float Bs[BN][LD];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int wm = (wave % WGM) * WM, wn = (wave / WGM) * WN;
    for (int i = t; i < 256 * P; i += 256) lut[i] = lut_g[i];

    floatx4_t acc[TA][TB];
#pragma unroll
    for (int a = 0; a < TA; ++a)
#pragma unroll
        for (int b = 0; b < TB; ++b) acc[a][b] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // staging: X float4 idx = t + 256 j -> row idx / 8, cols 4 * (idx % 8);
    // codes: row t / 4, run of 8 codes (t % 4) * 8
    const int br = t >> 2, bk = (t & 3) * 8;
    const bool brow = n0 + br < rows;
    const uint8_t *crow = packed + size_t(row_start + (brow ? n0 + br : 0)) * row_bytes;
    const float *nrow = norms + size_t(row_start + (brow ? n0 + br : 0)) * num_groups;
    float4 xa[NA];
    uint32_t code = 0;
    float nrm = 0.0f;
    auto load = [&](int k0) {
#pragma unroll
        for (int j = 0; j < NA; ++j) {
            const int idx = t + 256 * j, r = idx >> 3, c = (idx & 7) * 4;
            const bool on = idx < BM * BK / 4 && m0 + r < batch && k0 + c < in_padded;
            xa[j] = on ? *reinterpret_cast<const float4 *>(xh + size_t(m0 + r) * in_padded + k0 + c)
                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        const int k = k0 + bk;
        const bool on = brow && k < in_padded;
        if (P == 4)
            code = on ? uint32_t(*reinterpret_cast<const uint16_t *>(crow + k / 4)) : 0u;
        else
            code = on ? *reinterpret_cast<const uint32_t *>(crow + k / 2) : 0u;
        nrm = on ? nrow[k / group] : 0.0f;
    };
    auto store = [&]() {
#pragma unroll
        for (int j = 0; j < NA; ++j) {
            const int idx = t + 256 * j;
            if (idx < BM * BK / 4)
                *reinterpret_cast<float4 *>(&As[idx >> 3][(idx & 7) * 4]) = xa[j];
        }
        float v[8];
        if (P == 4) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const float4 l4 = *reinterpret_cast<const float4 *>(lut + ((code >> (8 * q)) & 0xffu) * 4);
                v[4 * q] = l4.x;
                v[4 * q + 1] = l4.y;
                v[4 * q + 2] = l4.z;
                v[4 * q + 3] = l4.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float2 l2 = *reinterpret_cast<const float2 *>(lut + ((code >> (8 * q)) & 0xffu) * 2);
                v[2 * q] = l2.x;
                v[2 * q + 1] = l2.y;
            }
        }
        *reinterpret_cast<float4 *>(&Bs[br][bk]) = make_float4(v[0] * nrm, v[1] * nrm, v[2] * nrm, v[3] * nrm);
        *reinterpret_cast<float4 *>(&Bs[br][bk + 4]) = make_float4(v[4] * nrm, v[5] * nrm, v[6] * nrm, v[7] * nrm);
    };
    __syncthreads();  // the LUT
    load(0);
    // MFMA 16x16x4 f32: lane l supplies A[l%16][k + l/16], B[k + l/16][l%16]
    const int r16 = lane & 15, kq = lane >> 4;
    for (int k0 = 0; k0 < in_padded; k0 += BK) {
        store();
        __syncthreads();
        if (k0 + BK < in_padded) load(k0 + BK);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 4) {
            float af[TA], bf[TB];
#pragma unroll
            for (int a = 0; a < TA; ++a) af[a] = As[wm + a * 16 + r16][kk + kq];
#pragma unroll
            for (int b = 0; b < TB; ++b) bf[b] = Bs[wn + b * 16 + r16][kk + kq];
#pragma unroll
            for (int a = 0; a < TA; ++a)
#pragma unroll
                for (int b = 0; b < TB; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[a], bf[b], acc[a][b], 0, 0, 0);
        }
        __syncthreads();
    }
    // C layout: lane l holds C[4*(l/16) + i][l%16]
    const int col = lane & 15, rb = (lane >> 4) * 4;
#pragma unroll
    for (int a = 0; a < TA; ++a)
#pragma unroll
        for (int b = 0; b < TB; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + wm + a * 16 + rb + i;
                const int n = n0 + wn + b * 16 + col;
                if (m < batch && n < rows) y[size_t(m) * rows + n] = acc[a][b][i];
            }
}

// ---------------------------------------------------------------------------
// dequantize rows: one block per (group, requested row).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(512) void cq_dequant_kernel(
    const uint8_t *__restrict__ packed, const float *__restrict__ norms,
    const float *__restrict__ lv, const int32_t *__restrict__ rows_idx, float *__restrict__ out,
    int out_feat, int in_feat, int row_bytes, int num_groups, int group, int w, int ternary,
    float inv)
{
    extern __shared__ float buf[];
    __shared__ float lvs[16];
    const int g = blockIdx.x;
    const size_t i = blockIdx.y;
    const int t = threadIdx.x;
    if (t < 16) lvs[t] = lv[t];
    int o = rows_idx[i];
    float *dst = out + i * size_t(in_feat);
    if (o < 0) {  // a masked row (e.g. an n-gram without enough history) reads as zeros
        for (int k = t; k < group; k += blockDim.x) {
            const int col = g * group + k;
            if (col < in_feat) dst[col] = 0.0f;
        }
        return;
    }
    o = o >= out_feat ? out_feat - 1 : o;
    const uint8_t *row = packed + size_t(o) * row_bytes;
    const float norm = norms[size_t(o) * num_groups + g];
    __syncthreads();
    for (int k = t; k < group; k += blockDim.x)
        buf[k] = level_of(lvs, read_code(row, g * group + k, w, row_bytes), ternary) * norm;
    __syncthreads();
    for (int h = 1; h < group; h <<= 1) {
        for (int q = t; q < group / 2; q += blockDim.x) {
            const int jj = (q / h) * (2 * h) + (q % h);
            const float a = buf[jj];
            const float c = buf[jj + h];
            buf[jj] = a + c;
            buf[jj + h] = a - c;
        }
        __syncthreads();
    }
    for (int k = t; k < group; k += blockDim.x) {
        const int col = g * group + k;
        if (col < in_feat) dst[col] = buf[k] * inv;
    }
}

int code_width(const nd_cq *w) { return w->bits == kTernary ? 2 : w->bits; }

int check_cq(const nd_cq *w)
{
    ND_REQUIRE(w && w->packed, "null weight");
    return ND_OK;
}

}  // namespace

extern "C" {

int nd_cq_from_blob(nd_ctx *ctx, const uint8_t *blob, size_t blob_len, size_t out_feat,
                    size_t in_feat, size_t group, uint8_t bits, const float *codebook,
                    size_t codebook_len, nd_cq **out)
{
    ND_ENTER(ctx);
    ND_REQUIRE(out, "null output pointer");
    *out = nullptr;
    // Validation order follows CqWeight::from_blob (cq.rs:189-225).
    if (out_feat == 0 || in_feat == 0) return nd::fail(ND_ERR_CQ_EMPTY_SHAPE, "EmptyShape");
    if (group == 0 || group % 8 != 0 || (group & (group - 1)) != 0 || group > kMaxGroup)
        return nd::fail(ND_ERR_CQ_BAD_GROUP, "BadGroup(%zu)", group);
    float levels[16] = {};
    int n_levels = 0;
    if (bits == kTernary) {
        const float s = 1.2240064f / std::sqrt(float(group));
        levels[0] = -s;
        levels[1] = 0.0f;
        levels[2] = s;
        n_levels = 3;
    } else {
        if (codebook_len != kCodebookLen)
            return nd::fail(ND_ERR_CQ_BAD_CODEBOOK_LEN, "BadCodebookLen(%zu)", codebook_len);
        size_t off;
        switch (bits) {
        case 2: off = 0; n_levels = 4; break;
        case 3: off = 4; n_levels = 8; break;
        case 4: off = 12; n_levels = 16; break;
        default: return nd::fail(ND_ERR_CQ_UNSUPPORTED_BITS, "UnsupportedBits(%u)", unsigned(bits));
        }
        ND_REQUIRE(codebook, "null codebook");
        std::memcpy(levels, codebook + off, n_levels * sizeof(float));
    }
    const size_t in_padded = (in_feat + group - 1) / group * group;
    const size_t num_groups = in_padded / group;
    const size_t eff = bits == kTernary ? 2 : bits;
    const size_t row_bytes = in_padded * eff / 8;
    const size_t n_packed = out_feat * row_bytes;
    const size_t n_norm = out_feat * num_groups * 2;
    if (!blob || blob_len < n_packed + n_norm)
        return nd::fail(ND_ERR_CQ_SHORT_BLOB, "ShortBlob { need: %zu, got: %zu }", n_packed + n_norm,
                        blob_len);
    ND_REQUIRE(out_feat < (size_t(1) << 31) && in_padded < (size_t(1) << 24), "shape too large");

    nd_cq *w = new (std::nothrow) nd_cq;
    if (!w) return nd::fail(ND_ERR_NOMEM, "host allocation failed");
    w->device = ctx->device;
    w->out_feat = out_feat;
    w->in_feat = in_feat;
    w->in_padded = in_padded;
    w->group = group;
    w->num_groups = num_groups;
    w->row_bytes = row_bytes;
    w->bits = bits;
    w->n_levels = n_levels;
    std::memcpy(w->levels, levels, sizeof levels);
    w->inv_sqrt_group = 1.0f / std::sqrt(float(group));
    w->per_byte = eff == 2 ? 4 : (eff == 4 ? 2 : 0);
    w->fp4_min_rows = kMf2MinRows;
    if (const char *v = std::getenv("NEEDLE_AMD_CQ_FP4_MIN_ROWS")) {
        char *end = nullptr;
        const unsigned long long n = std::strtoull(v, &end, 10);
        if (*v && end && *end == '\0') w->fp4_min_rows = size_t(n);
    }

    std::vector<float> norms(out_feat * num_groups);
    for (size_t i = 0; i < norms.size(); ++i) {
        const uint8_t *c = blob + n_packed + 2 * i;
        norms[i] = nd_f16_to_f32(uint16_t(c[0] | (c[1] << 8)));
    }
    std::vector<float> lut;
    if (w->per_byte) {
        // cq.rs:932-964
        const uint32_t mask = (1u << eff) - 1;
        lut.resize(256 * w->per_byte);
        for (uint32_t byte = 0; byte < 256; ++byte)
            for (size_t k = 0; k < w->per_byte; ++k) {
                const uint32_t code = (byte >> (k * eff)) & mask;
                const int idx = bits == kTernary ? ternary_index(code) : int(code);
                lut[byte * w->per_byte + k] = levels[idx];
            }
    }
    auto cleanup = [&](int rc) {
        nd_cq_free(w);
        return rc;
    };
    hipError_t e;
    if ((e = hipMalloc(&w->packed, n_packed + 16)) != hipSuccess) return cleanup(nd::hip_fail(e, "hipMalloc"));
    if ((e = hipMalloc(&w->norms, norms.size() * 4)) != hipSuccess) return cleanup(nd::hip_fail(e, "hipMalloc"));
    if ((e = hipMalloc(&w->lv, 16 * 4)) != hipSuccess) return cleanup(nd::hip_fail(e, "hipMalloc"));
    if (!lut.empty() && (e = hipMalloc(&w->lut, lut.size() * 4)) != hipSuccess)
        return cleanup(nd::hip_fail(e, "hipMalloc"));
    if ((e = hipMemsetAsync(w->packed + n_packed, 0, 16, ctx->stream)) != hipSuccess ||
        (e = hipMemcpyAsync(w->packed, blob, n_packed, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess ||
        (e = hipMemcpyAsync(w->norms, norms.data(), norms.size() * 4, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess ||
        (e = hipMemcpyAsync(w->lv, levels, 16 * 4, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess ||
        (!lut.empty() && (e = hipMemcpyAsync(w->lut, lut.data(), lut.size() * 4, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess) ||
        (e = hipStreamSynchronize(ctx->stream)) != hipSuccess)
        return cleanup(nd::hip_fail(e, "upload"));
    *out = w;
    return ND_OK;
}

void nd_cq_free(nd_cq *w)
{
    if (!w) return;
    (void)hipSetDevice(w->device);
    if (w->packed) (void)hipFree(w->packed);
    if (w->norms) (void)hipFree(w->norms);
    if (w->lut) (void)hipFree(w->lut);
    if (w->lv) (void)hipFree(w->lv);
    delete w;
}

int nd_cq_shape(const nd_cq *w, size_t *out_feat, size_t *in_feat, size_t *in_padded,
                size_t *group, uint8_t *bits)
{
    nd::clear_error();
    if (int rc = check_cq(w)) return rc;
    if (out_feat) *out_feat = w->out_feat;
    if (in_feat) *in_feat = w->in_feat;
    if (in_padded) *in_padded = w->in_padded;
    if (group) *group = w->group;
    if (bits) *bits = w->bits;
    return ND_OK;
}

int nd_cq_prepare_input(nd_ctx *ctx, const nd_cq *w, const float *x, size_t batch, float *xh)
{
    ND_ENTER(ctx);
    if (int rc = check_cq(w)) return rc;
    if (batch == 0) return ND_OK;
    ND_REQUIRE(x && xh, "null buffer");
    ND_REQUIRE(batch <= 65535, "batch %zu above 65535", batch);
    const int threads = int(w->group / 2 < 64 ? 64 : (w->group / 2 > 512 ? 512 : w->group / 2));
    dim3 grid(unsigned(w->num_groups), unsigned(batch));
    hipLaunchKernelGGL(cq_prepare_kernel, grid, dim3(threads), w->group * sizeof(float), ctx->stream,
                       x, xh, int(w->in_feat), int(w->in_padded), int(w->group), w->inv_sqrt_group);
    return nd::check_launch("cq_prepare");
}


int nd_cq_matvec_rows_prepared(nd_ctx *ctx, const nd_cq *w, const float *xh, size_t row_start,
                               size_t rows, float *y)
{
    ND_ENTER(ctx);
    if (int rc = check_cq(w)) return rc;
    ND_REQUIRE(row_start + rows <= w->out_feat, "rows %zu+%zu beyond %zu", row_start, rows, w->out_feat);
    if (rows == 0) return ND_OK;
    ND_REQUIRE(xh && y, "null buffer");
    ND_REQUIRE((reinterpret_cast<uintptr_t>(xh) & 15) == 0, "xh must be 16-byte aligned");
    const int row_dwords = int(w->row_bytes / 4);
    const int E = int(4 * w->per_byte);
    const bool fast = w->per_byte != 0 && w->row_bytes % 4 == 0 && size_t(E) <= w->group &&
                      row_dwords <= 16 * 6;
    // the streaming kernel: rows of 16 * ND code dwords, ND <= 6 (in 768: 48
    // dwords at 2 bits, 96 at 4 bits); other rows take the per-dword kernel
    const bool stream = w->per_byte != 0 && w->row_bytes % 64 == 0 && row_dwords / 16 >= 1 &&
                        row_dwords / 16 <= 6 && size_t(E) * (row_dwords / 16) <= w->group;
    // buffer offsets of the streaming kernels are 32-bit, their row products
    // 24-bit
    const bool offsets32 = rows < (size_t(1) << 24) && rows * w->row_bytes < (size_t(1) << 31) &&
                           rows * w->num_groups * 4 < (size_t(1) << 31);
    const size_t slots = 2 * size_t(ctx->num_cus > 0 ? ctx->num_cus : 256);
    const int args_rb = int(w->row_bytes), ng = int(w->num_groups), gr = int(w->group);
    if (w->per_byte == 4 && w->group == 128 && w->num_groups <= size_t(kMf2MaxGroups) &&
        w->row_bytes == 32 * w->num_groups && rows >= w->fp4_min_rows && offsets32) {
        // 2-bit / ternary, groups of 128, in <= 768, tall: fp4 matrix cores
        float lv[4];
        for (uint32_t c = 0; c < 4; ++c) lv[c] = w->levels[w->bits == kTernary ? ternary_index(c) : int(c)];
        const Mf2Coef cf = mf2_coef(lv);
        const size_t tiles = (rows + kMf2Rows - 1) / kMf2Rows;
        const size_t blocks = tiles < slots ? tiles : slots;
        const int iters = int((tiles + blocks - 1) / blocks);
#define ND_MF2(NGV)                                                                              \
    hipLaunchKernelGGL((cq_gemv_mf2_kernel<NGV>), dim3(unsigned(blocks)), dim3(kMf2Threads), 0,   \
                       ctx->stream, w->packed, w->norms, w->lut, xh, y, cf, int(row_start),       \
                       int(rows), iters)
        switch (w->num_groups) {
        case 1: ND_MF2(1); break;
        case 2: ND_MF2(2); break;
        case 3: ND_MF2(3); break;
        case 4: ND_MF2(4); break;
        case 5: ND_MF2(5); break;
        default: ND_MF2(6); break;
        }
#undef ND_MF2
        return nd::check_launch("cq_gemv_mf2");
    }
    if (stream && w->per_byte == 4 && row_dwords <= 16 * 3 && offsets32) {
        // 2-bit / ternary, in <= 768: product lookup, two 1024-thread
        // workgroups per CU, the tiles dealt round-robin
        const size_t tiles = (rows + kNibRows - 1) / kNibRows;
        const size_t blocks = tiles < slots ? tiles : slots;
        const int iters = int((tiles + blocks - 1) / blocks);
#define ND_CQN(NDV)                                                                             \
    hipLaunchKernelGGL((cq_gemv_nib_kernel<NDV>), dim3(unsigned(blocks)), dim3(kNibThreads), 0,  \
                       ctx->stream, w->packed, w->norms, w->lut, xh, y, int(row_start), int(rows), \
                       args_rb, ng, gr, iters)
        switch (row_dwords / 16) {
        case 1: ND_CQN(1); break;
        case 2: ND_CQN(2); break;
        default: ND_CQN(3); break;
        }
#undef ND_CQN
        return nd::check_launch("cq_gemv_nib");
    }
    if (stream && w->per_byte == 2 && row_dwords / 16 >= 4 && w->group % 32 == 0 && offsets32) {
        // 4-bit, in 512 to 768: byte lookup, two 512-thread workgroups per
        // CU, the tiles dealt round-robin
        const size_t tiles = (rows + kQ4Rows - 1) / kQ4Rows;
        const size_t blocks = tiles < slots ? tiles : slots;
        const int iters = int((tiles + blocks - 1) / blocks);
#define ND_CQ4(NDV)                                                                             \
    hipLaunchKernelGGL((cq_gemv_q4_kernel<NDV>), dim3(unsigned(blocks)), dim3(kQ4Threads), 0,    \
                       ctx->stream, w->packed, w->norms, w->lut, xh, y, int(row_start), int(rows), \
                       args_rb, ng, gr, iters)
        switch (row_dwords / 16) {
        case 4: ND_CQ4(4); break;
        case 5: ND_CQ4(5); break;
        default: ND_CQ4(6); break;
        }
#undef ND_CQ4
        return nd::check_launch("cq_gemv_q4");
    }
    if (stream) {
        const size_t tiles = (rows + kRowsPerPass - 1) / kRowsPerPass;
        const size_t slots4 = 2 * slots;
        const int tpb = int(tiles > slots4 ? (tiles + slots4 - 1) / slots4 : 1);
        dim3 grid(unsigned((tiles + tpb - 1) / tpb));
#define ND_CQS(P, NDV, REPL)                                                                   \
    hipLaunchKernelGGL((cq_gemv_stream_kernel<P, NDV, REPL, 4>), grid, dim3(kThreads), 0,       \
                       ctx->stream, w->packed, w->norms, w->lut, xh, y, int(row_start), int(rows), \
                       args_rb, ng, gr, tpb)
        const int nd = row_dwords / 16;
        if (w->per_byte == 4) {
            switch (nd) {
            case 1: ND_CQS(4, 1, 8); break;
            case 2: ND_CQS(4, 2, 8); break;
            case 3: ND_CQS(4, 3, 8); break;
            case 4: ND_CQS(4, 4, 8); break;
            case 5: ND_CQS(4, 5, 8); break;
            default: ND_CQS(4, 6, 8); break;
            }
        } else {
            switch (nd) {
            case 1: ND_CQS(2, 1, 16); break;
            case 2: ND_CQS(2, 2, 16); break;
            case 3: ND_CQS(2, 3, 16); break;
            case 4: ND_CQS(2, 4, 16); break;
            case 5: ND_CQS(2, 5, 16); break;
            default: ND_CQS(2, 6, 16); break;
            }
        }
#undef ND_CQS
        return nd::check_launch("cq_gemv_stream");
    }
    if (fast) {
        const int nd = (row_dwords + 15) / 16;
        dim3 grid(unsigned((rows + 63) / 64));
        const int args_rb = int(w->row_bytes), ng = int(w->num_groups), gr = int(w->group);
#define ND_CQ(P, NDV, REPL)                                                                 \
    hipLaunchKernelGGL((cq_gemv_kernel<P, NDV, REPL>), grid, dim3(kThreads), 0, ctx->stream, \
                       w->packed, w->norms, w->lut, xh, y, int(row_start), int(rows), args_rb, ng, gr)
        if (w->per_byte == 4) {
            switch (nd) {
            case 1: ND_CQ(4, 1, 8); break;
            case 2: ND_CQ(4, 2, 8); break;
            case 3: ND_CQ(4, 3, 8); break;
            case 4: ND_CQ(4, 4, 8); break;
            case 5: ND_CQ(4, 5, 8); break;
            default: ND_CQ(4, 6, 8); break;
            }
        } else {
            switch (nd) {
            case 1: ND_CQ(2, 1, 16); break;
            case 2: ND_CQ(2, 2, 16); break;
            case 3: ND_CQ(2, 3, 16); break;
            case 4: ND_CQ(2, 4, 16); break;
            case 5: ND_CQ(2, 5, 16); break;
            default: ND_CQ(2, 6, 16); break;
            }
        }
#undef ND_CQ
        return nd::check_launch("cq_gemv");
    }
    dim3 grid(unsigned((rows + 3) / 4));
    hipLaunchKernelGGL(cq_gemv_generic_kernel, grid, dim3(256), 0, ctx->stream, w->packed, w->norms,
                       w->lv, xh, y, int(row_start), int(rows), int(w->row_bytes), int(w->num_groups),
                       int(w->group), int(w->in_padded), code_width(w), int(w->bits == kTernary));
    return nd::check_launch("cq_gemv_generic");
}

int nd_cq_matmul_rows_prepared(nd_ctx *ctx, const nd_cq *w, const float *xh, size_t batch,
                               size_t row_start, size_t rows, float *y)
{
    ND_ENTER(ctx);
    if (int rc = check_cq(w)) return rc;
    ND_REQUIRE(row_start + rows <= w->out_feat, "rows %zu+%zu beyond %zu", row_start, rows, w->out_feat);
    if (rows == 0 || batch == 0) return ND_OK;
    ND_REQUIRE(xh && y, "null buffer");
    ND_REQUIRE(batch <= (size_t(1) << 22), "batch too large");
    const bool bytes = (w->per_byte == 2 || w->per_byte == 4) && w->lut && w->in_padded % 8 == 0 &&
                       (reinterpret_cast<uintptr_t>(xh) & 15) == 0;
    if (bytes) {
        // the tallest batch tile that still gives every CU a block
        const size_t cus = size_t(ctx->num_cus > 0 ? ctx->num_cus : 256);
        const size_t nt = (rows + 63) / 64;
        const int bm = nt * ((batch + 63) / 64) >= cus ? 64 : nt * ((batch + 31) / 32) >= cus ? 32 : 16;
        dim3 g2(unsigned(nt), unsigned((batch + bm - 1) / bm));
#define ND_MMB(PP, BMM)                                                                                \
    hipLaunchKernelGGL((cq_matmul_b_kernel<PP, BMM>), g2, dim3(256), 0, ctx->stream, w->packed, w->norms, \
                       w->lut, xh, y, int(batch), int(row_start), int(rows), int(w->row_bytes),          \
                       int(w->num_groups), int(w->group), int(w->in_padded))
        if (w->per_byte == 4) {
            if (bm == 64) ND_MMB(4, 64); else if (bm == 32) ND_MMB(4, 32); else ND_MMB(4, 16);
        } else {
            if (bm == 64) ND_MMB(2, 64); else if (bm == 32) ND_MMB(2, 32); else ND_MMB(2, 16);
        }
#undef ND_MMB
        return nd::check_launch("cq_matmul");
    }
    dim3 grid(unsigned((rows + kMN - 1) / kMN), unsigned((batch + kMM - 1) / kMM));
    hipLaunchKernelGGL(cq_matmul_kernel, grid, dim3(256), 0, ctx->stream, w->packed, w->norms, w->lv,
                       xh, y, int(batch), int(row_start), int(rows), int(w->row_bytes),
                       int(w->num_groups), int(w->group), int(w->in_padded), code_width(w),
                       int(w->bits == kTernary));
    return nd::check_launch("cq_matmul");
}

int nd_cq_dequantize_rows(nd_ctx *ctx, const nd_cq *w, const int32_t *rows, size_t n, float *out)
{
    ND_ENTER(ctx);
    if (int rc = check_cq(w)) return rc;
    if (n == 0) return ND_OK;
    ND_REQUIRE(rows && out, "null buffer");
    ND_REQUIRE(n <= 65535, "n %zu above 65535", n);
    const int threads = int(w->group / 2 < 64 ? 64 : (w->group / 2 > 512 ? 512 : w->group / 2));
    dim3 grid(unsigned(w->num_groups), unsigned(n));
    hipLaunchKernelGGL(cq_dequant_kernel, grid, dim3(threads), w->group * sizeof(float), ctx->stream,
                       w->packed, w->norms, w->lv, rows, out, int(w->out_feat), int(w->in_feat),
                       int(w->row_bytes), int(w->num_groups), int(w->group), code_width(w),
                       int(w->bits == kTernary), w->inv_sqrt_group);
    return nd::check_launch("cq_dequant");
}

}  // extern "C"
