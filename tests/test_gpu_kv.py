"""int8 KV cache on the GPU vs the oracle.

Bit-exact: quantize_rows / fake_quant / write_kv (codes and scales).
Attention: fp32 max-abs <= 1e-4 against the oracle's attend_step over the
same stored ints (the GPU sums in a different order; expf may differ by an
ulp).
"""
import json
import math
import os

import numpy as np
import pytest
import torch

import needle_amd as nd
import oracle as O
from conftest import dev, host

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _golden_cases():
    return json.load(open(os.path.join(GOLDEN, "kv_quant_vectors.json")))["cases"]


def test_quantize_rows_golden_bit_exact(ctx):
    for case in _golden_cases():
        dim = case["dim"]
        x = np.array(case["in"], np.float32)
        qi, qs = nd.quantize_rows(ctx, dev(x), dim)
        oi, os_ = O.quantize_rows(x, dim)
        assert np.array_equal(host(qi), oi), case["name"]
        assert np.array_equal(host(qs).view(np.uint32), os_.view(np.uint32)), case["name"]
        fq = dev(x.copy())
        nd.fake_quant(ctx, fq, dim)
        want = np.concatenate([O.fake_quant_vec(r) for r in x.reshape(-1, dim)])
        assert np.array_equal(host(fq), want), case["name"]
        tol = np.maximum(np.abs(np.array(case["out"], np.float32)), 1.0) * 1e-5
        assert np.all(np.abs(host(fq) - np.array(case["out"], np.float32)) <= tol)


def test_quantize_ties_round_away_from_zero(ctx):
    """Exact .5 products round away from zero on the device as in the oracle
    (libm's roundf): rows with absmax 127 have scale and inverse 1."""
    from test_oracle_kv import TIE_CODES, TIE_ROW
    x = np.stack([TIE_ROW, -TIE_ROW, TIE_ROW[::-1].copy()]).astype(np.float32)
    qi, qs = nd.quantize_rows(ctx, dev(x), TIE_ROW.size)
    oi, os_ = O.quantize_rows(x, TIE_ROW.size)
    assert np.array_equal(host(qi), oi)
    assert host(qi)[: TIE_ROW.size].tolist() == TIE_CODES
    assert np.array_equal(host(qs).view(np.uint32), os_.view(np.uint32))
    fq = dev(x.copy())
    nd.fake_quant(ctx, fq, TIE_ROW.size)
    assert np.array_equal(host(fq).reshape(-1), np.concatenate([O.fake_quant_vec(r) for r in x]))


@pytest.mark.parametrize("dim", [48, 64, 16, 256, 100])
def test_quantize_rows_random_bit_exact(ctx, dim):
    rng = np.random.default_rng(dim)
    rows = 4096
    mags = 10.0 ** rng.uniform(-9, 7, size=(rows, 1))
    x = (rng.normal(size=(rows, dim)) * mags).astype(np.float32)
    x[0] = 0.0                       # all-zero row keeps scale 1
    x[1] = 0.0
    x[1, 3] = 7.0                    # one spike
    x[2] = np.float32(0.5) * np.arange(dim, dtype=np.float32) / np.float32(dim)
    qi, qs = nd.quantize_rows(ctx, dev(x), dim)
    oi, os_ = O.quantize_rows(x, dim)
    assert np.array_equal(host(qi), oi)
    assert np.array_equal(host(qs).view(np.uint32), os_.view(np.uint32))
    assert host(qs)[0] == 1.0


def test_write_kv_ring_matches_oracle(ctx):
    """A local ring (window 16) written past its window, int8 codes and
    scales equal the oracle V3Cache ring's, slot for slot."""
    H, KVH, QK, VD, W = 12, 2, 48, 64, 16
    ring = O.Ring(True, KVH, QK, VD, hint=4, window=W, max_seq_len=64)
    cache = nd.V3LayerCache(ctx, H, KVH, QK, VD, hint=4, window=W, max_seq_len=64)
    rng = np.random.default_rng(2)
    for pos in range(41):
        k = (rng.normal(size=KVH * QK) * (pos + 1)).astype(np.float32)
        v = rng.normal(size=KVH * VD).astype(np.float32)
        ring.write_kv(pos, k, v)
        cache.write_kv(pos, dev(k), dev(v))
        assert cache.span(pos) == ring.span(pos)
        assert cache.slots == ring.slots
    k, ks, v, vs = nd.kv_unpack(cache.geom, host(cache.block))
    st = ring.store()
    assert np.array_equal(k.reshape(-1), st["k"]) and np.array_equal(v.reshape(-1), st["v"])
    assert np.array_equal(ks.reshape(-1), st["k_scale"]) and np.array_equal(vs.reshape(-1), st["v_scale"])


@pytest.mark.parametrize("ctxlen,batch", [(2048, 1), (2048, 64), (512, 3)])
def test_write_kv_config3_bytes(ctx, ctxlen, batch):
    """Config 3's append at 12 kv heads x 64: positions 0..ctx-1 written
    `batch` positions per call, as a decode loop appends them; every slot's
    K and V codes and scales equal the oracle's quantize_rows of that
    position's rows (cache.rs:113-122, 346-379), byte for byte, and the
    untouched bytes of the block stay zero.  A second pass over the ring
    (positions ctx..ctx+batch-1, slots 0..batch-1) overwrites only its slots."""
    H = KVH = 12
    QK = VD = 64
    rng = np.random.default_rng(ctxlen + batch)
    g = nd.kv_geom(H, KVH, QK, VD, ctxlen)
    blk, nb = nd.kv_alloc(g)
    mags = 10.0 ** rng.uniform(-3, 3, size=(ctxlen + batch, 1))
    k = (rng.normal(size=(ctxlen + batch, KVH * QK)) * mags).astype(np.float32)
    v = rng.normal(size=(ctxlen + batch, KVH * VD)).astype(np.float32)
    k[5] = 0.0  # an all-zero row keeps scale 1
    kd, vd_ = dev(k), dev(v)
    for p0 in range(0, ctxlen, batch):
        p1 = min(ctxlen, p0 + batch)
        pos = torch.arange(p0, p1, dtype=torch.int32, device="cuda")
        nd.kv_write(ctx, g, blk, 0, pos, kd[p0:p1], vd_[p0:p1])
    raw = host(blk)
    kk, kks, vv, vvs = nd.kv_unpack(g, raw)
    kq, ks = O.quantize_rows(k[:ctxlen], QK)
    vq, vs = O.quantize_rows(v[:ctxlen], VD)
    assert np.array_equal(kk.reshape(-1), kq) and np.array_equal(vv.reshape(-1), vq)
    assert np.array_equal(kks.reshape(-1).view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(vvs.reshape(-1).view(np.uint32), vs.view(np.uint32))
    off = nd.kv_offsets(g)
    used = [(0, KVH * ctxlen * QK), (off["v"], off["v"] + KVH * ctxlen * VD),
            (off["ks"], off["ks"] + 4 * KVH * ctxlen), (off["vs"], off["vs"] + 4 * KVH * ctxlen)]
    mask = np.ones(raw.size, bool)
    for a, b in used:
        mask[a:b] = False
    assert not raw[mask].any(), "bytes outside the K/V/scale runs were written"
    # the ring wraps: the next positions land in slots 0..batch-1 only
    pos = torch.arange(ctxlen, ctxlen + batch, dtype=torch.int32, device="cuda")
    nd.kv_write(ctx, g, blk, 0, pos, kd[ctxlen:], vd_[ctxlen:])
    kk2, kks2, vv2, vvs2 = nd.kv_unpack(g, host(blk))
    kq2, ks2 = O.quantize_rows(k[ctxlen:], QK)
    vq2, vs2 = O.quantize_rows(v[ctxlen:], VD)
    assert np.array_equal(kk2[:batch].reshape(-1), kq2) and np.array_equal(vv2[:batch].reshape(-1), vq2)
    assert np.array_equal(kks2[:batch].reshape(-1).view(np.uint32), ks2.view(np.uint32))
    assert np.array_equal(vvs2[:batch].reshape(-1).view(np.uint32), vs2.view(np.uint32))
    assert np.array_equal(kk2[batch:], kk[batch:]) and np.array_equal(vv2[batch:], vv[batch:])
    assert np.array_equal(kks2[batch:], kks[batch:]) and np.array_equal(vvs2[batch:], vvs[batch:])


def _fill(ctx, rng, H, KVH, QK, VD, cap, npos, count=1):
    """`count` blocks, positions 0..npos-1 written (ring-wrapped at cap)."""
    g = nd.kv_geom(H, KVH, QK, VD, cap)
    blk, nb = nd.kv_alloc(g, count)
    ks_raw = rng.normal(size=(count, npos, KVH * QK)).astype(np.float32)
    vs_raw = rng.normal(size=(count, npos, KVH * VD)).astype(np.float32)
    for i in range(count):
        pos = torch.arange(npos, dtype=torch.int32, device="cuda")
        nd.kv_write(ctx, g, blk[i * nb:(i + 1) * nb], 0, pos, dev(ks_raw[i]), dev(vs_raw[i]))
    return g, blk, nb


def _oracle_step(g, block_np, q, lo, hi):
    k, ks, v, vs = nd.kv_unpack(g, block_np)
    return O.attend_step_i8(q, k.reshape(-1), ks.reshape(-1), v.reshape(-1), vs.reshape(-1),
                            g.cap, lo, hi, g.num_heads, g.num_kv_heads, g.qk_head_dim,
                            g.v_head_dim)


@pytest.mark.parametrize("H,KVH,QK,VD", [(12, 2, 48, 64), (12, 12, 64, 64)])
@pytest.mark.parametrize("ctxlen", [1, 7, 512, 2048, 8192])
def test_attend_step_causal(ctx, H, KVH, QK, VD, ctxlen):
    """Config 3 (MHA 12 x 64) and the v3 GQA geometry, causal span 0..ctx-1."""
    rng = np.random.default_rng(ctxlen + H * KVH)
    g, blk, nb = _fill(ctx, rng, H, KVH, QK, VD, ctxlen, ctxlen)
    q = rng.normal(size=H * QK).astype(np.float32)
    lo = torch.tensor([0], dtype=torch.int32, device="cuda")
    hi = torch.tensor([ctxlen - 1], dtype=torch.int32, device="cuda")
    out = host(nd.attend_step_i8(ctx, g, blk, nb, lo, hi, dev(q)[None]))[0]
    want = _oracle_step(g, host(blk), q, 0, ctxlen - 1)
    assert np.max(np.abs(out - want)) <= 1e-4


@pytest.mark.parametrize("H,KVH,QK", [(12, 2, 48), (12, 12, 64)])
@pytest.mark.parametrize("lo,hi", [(0, 0), (5, 5), (3, 16), (1000, 1023), (1000, 2023),
                                   (4000, 5023), (17, 1040)])
def test_attend_step_ring_window(ctx, H, KVH, QK, lo, hi):
    """A 1024-slot local ring read across its wrap point: the v3 GQA geometry
    (lane dots summed in LDS) and the MHA cache (lane dots summed by DPP)."""
    VD, cap = 64, 1024
    rng = np.random.default_rng(lo * 31 + hi)
    g = nd.kv_geom(H, KVH, QK, VD, cap)
    blk, nb = nd.kv_alloc(g)
    n = hi + 1
    k = rng.normal(size=(n, KVH * QK)).astype(np.float32)
    v = rng.normal(size=(n, KVH * VD)).astype(np.float32)
    nd.kv_write(ctx, g, blk, 0, torch.arange(n, dtype=torch.int32, device="cuda"), dev(k), dev(v))
    q = rng.normal(size=H * QK).astype(np.float32)
    out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(np.array([lo], np.int32)),
                                 dev(np.array([hi], np.int32)), dev(q)[None]))[0]
    want = _oracle_step(g, host(blk), q, lo, hi)
    assert np.max(np.abs(out - want)) <= 1e-4


def test_hoisted_scale_geometry(ctx):
    """v3_kv_quant_parity.rs:102-218 geometry (4/2 heads, 17 slots)."""
    H, KVH, QK, VD, SLOTS = 4, 2, 48, 64, 17
    rng = np.random.default_rng(17)
    g, blk, nb = _fill(ctx, rng, H, KVH, QK, VD, SLOTS, SLOTS)
    q = rng.normal(size=H * QK).astype(np.float32)
    for lo, hi in [(0, 0), (0, 9), (3, 16), (5, 5)]:
        out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(np.array([lo], np.int32)),
                                     dev(np.array([hi], np.int32)), dev(q)[None]))[0]
        assert np.max(np.abs(out - _oracle_step(g, host(blk), q, lo, hi))) <= 1e-4


def test_quant_query_fused(ctx):
    """quant_rows(q) then attend_step (v3/model.rs:289-307), fused."""
    H, KVH, QK, VD, n = 12, 2, 48, 64, 300
    rng = np.random.default_rng(3)
    g, blk, nb = _fill(ctx, rng, H, KVH, QK, VD, 512, n)
    q = (rng.normal(size=H * QK) * 3).astype(np.float32)
    out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(np.array([0], np.int32)),
                                 dev(np.array([n - 1], np.int32)), dev(q)[None], quant_query=True))[0]
    qq = O.quant_rows(q, 1, H, QK)
    assert np.max(np.abs(out - _oracle_step(g, host(blk), qq, 0, n - 1))) <= 1e-4


def test_batched_sessions(ctx):
    """Several sessions, one launch, each with its own block and span."""
    H, KVH, QK, VD, cap, count = 12, 12, 64, 64, 2048, 5
    rng = np.random.default_rng(11)
    g, blk, nb = _fill(ctx, rng, H, KVH, QK, VD, cap, cap, count)
    q = rng.normal(size=(count, H * QK)).astype(np.float32)
    lo = np.array([0, 100, 2047, 5, 0], np.int32)
    hi = np.array([2047, 1900, 2047, 5, 511], np.int32)
    out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(lo), dev(hi), dev(q)))
    blocks = host(blk)
    for i in range(count):
        want = _oracle_step(g, blocks[i * nb:(i + 1) * nb], q[i], int(lo[i]), int(hi[i]))
        assert np.max(np.abs(out[i] - want)) <= 1e-4, i


def test_bad_span_is_nan(ctx):
    H, KVH, QK, VD, cap = 12, 2, 48, 64, 64
    g = nd.kv_geom(H, KVH, QK, VD, cap)
    blk, nb = nd.kv_alloc(g)
    q = torch.zeros(1, H * QK, device="cuda")
    for lo, hi in [(5, 4), (0, 64)]:
        out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(np.array([lo], np.int32)),
                                     dev(np.array([hi], np.int32)), q))
        assert np.isnan(out).all()


@pytest.mark.parametrize("seq,window", [(1, 0), (40, 16), (128, 0), (300, 64)])
def test_prefill_attend(ctx, seq, window):
    """attend over the prompt's own int8 K/V with a window (attention.rs:218-287)."""
    H, KVH, QK, VD = 12, 2, 48, 64
    rng = np.random.default_rng(seq + window)
    q = rng.normal(size=(seq, H * QK)).astype(np.float32)
    k = rng.normal(size=(seq, KVH * QK)).astype(np.float32)
    v = rng.normal(size=(seq, KVH * VD)).astype(np.float32)
    out = host(nd.attend_i8_prefill(ctx, H, KVH, QK, VD, dev(q), dev(k), dev(v), window))
    kq, ks = O.quantize_rows(k, QK)
    vq, vs = O.quantize_rows(v, VD)
    want = O.attend_i8(q, kq, ks, vq, vs, seq, H, KVH, QK, VD, window=window).reshape(seq, -1)
    assert np.max(np.abs(out - want)) <= 1e-4
