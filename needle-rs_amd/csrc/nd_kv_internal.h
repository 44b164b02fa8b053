// Shared by the int8 KV kernels: the block layout as the kernels see it,
// the geometry check and the bit-exact quantiser (cache.rs:80-104).
#pragma once

#include "nd_internal.h"
#include "nd_lanes.h"

namespace ndkv {

constexpr int kMaxRep = 8;
constexpr int kMaxDim = 256;

// Lane pairs at distances 32 .. 1 through DPP and lane swaps (no LDS).
__device__ inline float wave_max(float v) { return ndl::wave_max64(v); }

__device__ inline float wave_sum(float v) { return ndl::wave_sum64(v); }

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

struct Geom {
    int H, KVH, QK, VD, cap;
    size_t v_off, ks_off, vs_off;
};

inline Geom make_geom(const nd_kv_geom *k)
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

inline int check_geom(const nd_kv_geom *g)
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

}  // namespace ndkv
