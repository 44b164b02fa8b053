"""The f32 KV cache (KvPrecision::F32) on the device vs the oracle.

nd_kv_write_f32 against V3Cache::write_kv's f32 branch (cache.rs:359-362):
the stored floats equal the written ones at slot pos % cap, bit for bit.
nd_attend_step_f32_exact against attend_step over the f32 view
(attention.rs:166-189, 327-377): identical float32 bits on the config-3
geometry (12 x 64 MHA) and the v3 GQA geometry, across ring wraps, on both
sides of the softmax sum's fold limits, and several sessions per call.  The
forward with f32 caches is checked in test_gpu_v3_f32.py.
"""
import numpy as np
import pytest
import torch

import needle_amd as nd
import oracle as O
from conftest import dev, host

pytestmark = pytest.mark.gpu


def _same_bits(a, b):
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _fill(ctx, rng, H, KVH, QK, VD, cap, npos, count=1, scale=1.0):
    """Positions 0..npos-1 written in calls of at most `cap` positions: the
    rows of one call are written in parallel, so a call must not hold two
    positions of one slot (the decode step writes one per session)."""
    g = nd.kv_geom(H, KVH, QK, VD, cap)
    blk, nb = nd.kv_alloc_f32(g, count)
    rows = []
    for i in range(count):
        k = (rng.normal(size=(npos, KVH * QK)) * scale).astype(np.float32)
        v = rng.normal(size=(npos, KVH * VD)).astype(np.float32)
        for p0 in range(0, npos, cap):
            p1 = min(npos, p0 + cap)
            pos = torch.arange(p0, p1, dtype=torch.int32, device="cuda")
            nd.kv_write_f32(ctx, g, blk[i * nb:(i + 1) * nb], 0, pos, dev(k[p0:p1]), dev(v[p0:p1]))
        rows.append((k, v))
    return g, blk, nb, rows


def _oracle(g, block_np, q, lo, hi):
    k, v = nd.kv_unpack_f32(g, block_np)
    return O.attend_step_f32(q, k.reshape(-1), v.reshape(-1), g.cap, lo, hi, g.num_heads,
                             g.num_kv_heads, g.qk_head_dim, g.v_head_dim)


@pytest.mark.parametrize("H,KVH,QK,VD,cap,npos", [(12, 2, 48, 64, 1024, 1500),
                                                  (12, 12, 64, 64, 2048, 2048),
                                                  (4, 2, 16, 32, 17, 40)])
def test_write_f32_ring_slots(ctx, H, KVH, QK, VD, cap, npos):
    """Every position lands at slot pos % cap; a later position overwrites
    the slot, as the reference's ring does once it has wrapped."""
    rng = np.random.default_rng(cap + npos)
    g, blk, nb, rows = _fill(ctx, rng, H, KVH, QK, VD, cap, npos)
    k, v = nd.kv_unpack_f32(g, host(blk))
    kw, vw = rows[0]
    for slot in range(cap):
        last = max(p for p in range(slot, npos, cap)) if slot < npos else None
        if last is None:
            assert not k[slot].any() and not v[slot].any()
            continue
        assert _same_bits(k[slot].reshape(-1), kw[last]), slot
        assert _same_bits(v[slot].reshape(-1), vw[last]), slot


def test_write_f32_one_row_per_session(ctx):
    """kv_stride = block bytes: row i into session i's block (the decode
    step's layout), positions differing per session."""
    H, KVH, QK, VD, cap, count = 12, 2, 48, 64, 64, 5
    rng = np.random.default_rng(5)
    g = nd.kv_geom(H, KVH, QK, VD, cap)
    blk, nb = nd.kv_alloc_f32(g, count)
    pos = np.array([0, 63, 64, 130, 7], np.int32)
    k = rng.normal(size=(count, KVH * QK)).astype(np.float32)
    v = rng.normal(size=(count, KVH * VD)).astype(np.float32)
    nd.kv_write_f32(ctx, g, blk, nb, dev(pos), dev(k), dev(v))
    blocks = host(blk)
    for i in range(count):
        kk, vv = nd.kv_unpack_f32(g, blocks[i * nb:(i + 1) * nb])
        s = int(pos[i]) % cap
        assert _same_bits(kk[s].reshape(-1), k[i]) and _same_bits(vv[s].reshape(-1), v[i])
        others = [j for j in range(cap) if j != s]
        assert not kk[others].any() and not vv[others].any()


@pytest.mark.parametrize("H,KVH,QK,VD", [(12, 2, 48, 64), (12, 12, 64, 64), (4, 2, 16, 32),
                                         (4, 2, 32, 128), (6, 3, 16, 48), (2, 1, 16, 16)])
@pytest.mark.parametrize("n", [1, 2, 33, 512, 2048])
def test_attend_f32_causal(ctx, H, KVH, QK, VD, n):
    """Causal span 0..n-1: config 3's 12 x 64 MHA at ctx 512 and 2048, the
    v3 GQA geometry, and odd head widths (the generic score loop)."""
    rng = np.random.default_rng(n * 13 + H + QK)
    g, blk, nb, _ = _fill(ctx, rng, H, KVH, QK, VD, n, n, scale=2.0)
    q = (rng.normal(size=H * QK) * 3).astype(np.float32)
    out = host(nd.attend_step_f32(ctx, g, blk, nb, dev(np.array([0], np.int32)),
                                  dev(np.array([n - 1], np.int32)), dev(q)[None]))[0]
    assert _same_bits(out, _oracle(g, host(blk), q, 0, n - 1))


@pytest.mark.parametrize("lo,hi", [(0, 0), (5, 5), (3, 16), (1000, 1023), (1000, 2023),
                                   (4000, 5023), (17, 1040)])
def test_attend_f32_ring_window(ctx, lo, hi):
    """A 1024-slot local ring read across its wrap point."""
    H, KVH, QK, VD, cap = 12, 2, 48, 64, 1024
    rng = np.random.default_rng(lo * 31 + hi)
    g, blk, nb, _ = _fill(ctx, rng, H, KVH, QK, VD, cap, hi + 1)
    q = rng.normal(size=H * QK).astype(np.float32)
    out = host(nd.attend_step_f32(ctx, g, blk, nb, dev(np.array([lo], np.int32)),
                                  dev(np.array([hi], np.int32)), dev(q)[None]))[0]
    assert _same_bits(out, _oracle(g, host(blk), q, lo, hi))


@pytest.mark.parametrize("span", [2047, 2048, 2049, 4096, 4097, 8192])
def test_attend_f32_softmax_sum_paths(ctx, span):
    """Spans on both sides of the softmax sum's fold limits (2048..4096) and
    the largest f32 ring (8192)."""
    H, KVH, QK, VD, cap = 12, 2, 48, 64, 8192
    rng = np.random.default_rng(span)
    g, blk, nb, _ = _fill(ctx, rng, H, KVH, QK, VD, cap, cap, scale=2.0)
    q = (rng.normal(size=H * QK) * 3).astype(np.float32)
    lo, hi = cap - span, cap - 1
    out = host(nd.attend_step_f32(ctx, g, blk, nb, dev(np.array([lo], np.int32)),
                                  dev(np.array([hi], np.int32)), dev(q)[None]))[0]
    assert _same_bits(out, _oracle(g, host(blk), q, lo, hi))


def test_attend_f32_batched_sessions(ctx):
    """Six sessions with their own blocks and spans in one launch."""
    H, KVH, QK, VD, cap, count = 12, 2, 48, 64, 2048, 6
    rng = np.random.default_rng(11)
    g, blk, nb, _ = _fill(ctx, rng, H, KVH, QK, VD, cap, cap, count)
    q = rng.normal(size=(count, H * QK)).astype(np.float32)
    lo = np.array([0, 100, 2047, 5, 0, 1024], np.int32)
    hi = np.array([2047, 1900, 2047, 5, 511, 2047], np.int32)
    out = host(nd.attend_step_f32(ctx, g, blk, nb, dev(lo), dev(hi), dev(q)))
    blocks = host(blk)
    for i in range(count):
        want = _oracle(g, blocks[i * nb:(i + 1) * nb], q[i], int(lo[i]), int(hi[i]))
        assert _same_bits(out[i], want), i


def test_attend_f32_bad_span_is_nan(ctx):
    H, KVH, QK, VD, cap = 12, 2, 48, 64, 64
    g = nd.kv_geom(H, KVH, QK, VD, cap)
    blk, nb = nd.kv_alloc_f32(g)
    q = torch.zeros(1, H * QK, device="cuda")
    for lo, hi in [(5, 4), (0, 64), (-1, 3)]:
        out = host(nd.attend_step_f32(ctx, g, blk, nb, dev(np.array([lo], np.int32)),
                                      dev(np.array([hi], np.int32)), q))
        assert np.isnan(out).all()


def test_attend_f32_rejects_large_rings(ctx):
    g = nd.kv_geom(4, 2, 16, 32, 9000)
    blk, nb = nd.kv_alloc_f32(g)
    with pytest.raises(nd.NeedleError):
        nd.attend_step_f32(ctx, g, blk, nb, dev(np.array([0], np.int32)),
                           dev(np.array([10], np.int32)), torch.zeros(1, 64, device="cuda"))
