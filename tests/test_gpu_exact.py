"""Reference-order kernels vs the oracle, bit for bit.

nd_cq_matvec_rows_exact / nd_cq_matmul_rows_exact against the oracle's
CqWeight::matvec_rows_prepared / matmul_rows_prepared (cq.rs:721-757,
632-679), and nd_attend_step_i8_exact against attend_step over the int8 view
(attention.rs:327-377): identical float32 bits, signs of zero included.  The
Needle-3 forward is built on these, so its logits can match to the bit.
"""
import json
import os

import numpy as np
import pytest
import torch

import needle_amd as nd
import oracle as O
from conftest import dev, host
from cq_cases import TERNARY, random_case

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
REAL_CB = np.array(json.load(open(os.path.join(GOLDEN, "cq_codebook.json")))["codebook"], np.float32)


def _same_bits(a, b):
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


# (out, in, group, bits, row_start, rows): the v3 projection shapes (q/k/v,
# gate, out, the Engram key, the LM head, a phi band), then ragged and odd
# widths that take the serial kernel (3-bit, 2-byte groups).
CQ_SHAPES = [
    (576, 768, 128, 2, 0, 576), (96, 768, 128, 2, 0, 96), (768, 768, 128, 2, 0, 768),
    (768, 768, 128, 2, 100, 37), (8192, 768, 128, 4, 0, 8192), (80, 3072, 128, 4, 16, 4),
    (320, 3072, 128, 4, 48, 16), (200, 640, 128, TERNARY, 0, 200), (100, 384, 128, 3, 0, 100),
    (130, 300, 64, 2, 0, 130), (33, 200, 32, 4, 1, 31), (17, 40, 8, 2, 0, 17),
    (40, 96, 16, 2, 0, 40), (9, 2048, 1024, 2, 0, 9),
]


@pytest.mark.parametrize("shape", CQ_SHAPES)
@pytest.mark.parametrize("batch", [1, 3, 64])
def test_cq_exact_bits(ctx, shape, batch):
    out, inn, group, bits, r0, rows = shape
    rng = np.random.default_rng(out * 7 + inn + bits * 1000 + batch)
    c = random_case(rng, out, inn, group, bits, REAL_CB)
    g = nd.CqWeight(ctx, c.blob, out, inn, group, bits, REAL_CB)
    o = O.CqWeight(c.blob, out, inn, group, bits, REAL_CB)
    x = rng.normal(size=(batch, inn)).astype(np.float32)
    x[:, ::7] *= 30.0  # a wide dynamic range, so sums round at every step
    xh = o.prepare_batch(x)
    xh_d = dev(xh)
    if batch == 1:
        got = host(g.matvec_rows_prepared(xh_d[0], r0, rows, exact=True))
        want = o.matvec_rows_prepared(xh[0], r0, rows)
        assert _same_bits(got, want)
    got = host(g.matmul_rows_prepared(xh_d, batch, r0, rows, exact=True))
    want = o.matmul_rows_prepared(xh, batch, r0, rows)
    assert _same_bits(got, want)
    if batch == 1:
        # matmul == matvec bit for bit (cq.rs:1270-1323)
        assert _same_bits(got, o.matvec_rows_prepared(xh[0], r0, rows))


def test_cq_exact_rejects_bad_band(ctx):
    rng = np.random.default_rng(0)
    c = random_case(rng, 16, 128, 128, 2, REAL_CB)
    g = nd.CqWeight(ctx, c.blob, 16, 128, 128, 2, REAL_CB)
    xh = torch.zeros(128, device="cuda")
    with pytest.raises(nd.NeedleError):
        g.matvec_rows_prepared(xh, 10, 7, exact=True)


def _fill(ctx, rng, H, KVH, QK, VD, cap, npos, count=1, scale=1.0):
    g = nd.kv_geom(H, KVH, QK, VD, cap)
    blk, nb = nd.kv_alloc(g, count)
    for i in range(count):
        k = (rng.normal(size=(npos, KVH * QK)) * scale).astype(np.float32)
        v = rng.normal(size=(npos, KVH * VD)).astype(np.float32)
        pos = torch.arange(npos, dtype=torch.int32, device="cuda")
        nd.kv_write(ctx, g, blk[i * nb:(i + 1) * nb], 0, pos, dev(k), dev(v))
    return g, blk, nb


def _oracle(g, block_np, q, lo, hi):
    k, ks, v, vs = nd.kv_unpack(g, block_np)
    return O.attend_step_i8(q, k.reshape(-1), ks.reshape(-1), v.reshape(-1), vs.reshape(-1),
                            g.cap, lo, hi, g.num_heads, g.num_kv_heads, g.qk_head_dim,
                            g.v_head_dim)


@pytest.mark.parametrize("H,KVH,QK,VD", [(12, 2, 48, 64), (12, 12, 64, 64), (4, 2, 16, 32),
                                         (4, 2, 32, 128), (6, 3, 16, 48), (2, 1, 16, 16)])
@pytest.mark.parametrize("n", [1, 2, 33, 384, 2048])
def test_attend_exact_causal(ctx, H, KVH, QK, VD, n):
    rng = np.random.default_rng(n * 13 + H + QK)
    g, blk, nb = _fill(ctx, rng, H, KVH, QK, VD, n, n, scale=2.0)
    q = (rng.normal(size=H * QK) * 3).astype(np.float32)
    for qq in (False, True):
        out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(np.array([0], np.int32)),
                                     dev(np.array([n - 1], np.int32)), dev(q)[None],
                                     quant_query=qq, exact=True))[0]
        qin = O.quant_rows(q, 1, H, QK) if qq else q
        assert _same_bits(out, _oracle(g, host(blk), qin, 0, n - 1)), qq


@pytest.mark.parametrize("lo,hi", [(0, 0), (5, 5), (3, 16), (1000, 1023), (1000, 2023),
                                   (4000, 5023), (17, 1040)])
def test_attend_exact_ring_window(ctx, lo, hi):
    """A 1024-slot local ring read across its wrap point."""
    H, KVH, QK, VD, cap = 12, 2, 48, 64, 1024
    rng = np.random.default_rng(lo * 31 + hi)
    g = nd.kv_geom(H, KVH, QK, VD, cap)
    blk, nb = nd.kv_alloc(g)
    n = hi + 1
    k = rng.normal(size=(n, KVH * QK)).astype(np.float32)
    v = rng.normal(size=(n, KVH * VD)).astype(np.float32)
    nd.kv_write(ctx, g, blk, 0, torch.arange(n, dtype=torch.int32, device="cuda"), dev(k), dev(v))
    q = rng.normal(size=H * QK).astype(np.float32)
    out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(np.array([lo], np.int32)),
                                 dev(np.array([hi], np.int32)), dev(q)[None], exact=True))[0]
    assert _same_bits(out, _oracle(g, host(blk), q, lo, hi))


@pytest.mark.parametrize("span", [1023, 1024, 1025, 2047, 2048, 2049, 2304, 2305, 3333, 4096, 4097])
def test_attend_exact_softmax_sum_paths(ctx, span):
    """Spans of 1024..4096 positions take the parallel fold for the softmax
    sum (its loop sized for 4, 9 or 16 terms a thread), the others the
    chain; all give the chain's bits."""
    H, KVH, QK, VD, cap = 12, 2, 48, 64, 4200
    rng = np.random.default_rng(span)
    g, blk, nb = _fill(ctx, rng, H, KVH, QK, VD, cap, cap, scale=2.0)
    q = (rng.normal(size=H * QK) * 3).astype(np.float32)
    lo, hi = cap - span - 7, cap - 8
    out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(np.array([lo], np.int32)),
                                 dev(np.array([hi], np.int32)), dev(q)[None], exact=True))[0]
    assert _same_bits(out, _oracle(g, host(blk), q, lo, hi))


def test_attend_exact_batched_sessions(ctx):
    H, KVH, QK, VD, cap, count = 12, 2, 48, 64, 2048, 6
    rng = np.random.default_rng(11)
    g, blk, nb = _fill(ctx, rng, H, KVH, QK, VD, cap, cap, count)
    q = rng.normal(size=(count, H * QK)).astype(np.float32)
    lo = np.array([0, 100, 2047, 5, 0, 1024], np.int32)
    hi = np.array([2047, 1900, 2047, 5, 511, 2047], np.int32)
    out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(lo), dev(hi), dev(q), quant_query=True,
                                 exact=True))
    blocks = host(blk)
    for i in range(count):
        want = _oracle(g, blocks[i * nb:(i + 1) * nb], O.quant_rows(q[i], 1, H, QK),
                       int(lo[i]), int(hi[i]))
        assert _same_bits(out[i], want), i


def test_attend_exact_bad_span_is_nan(ctx):
    H, KVH, QK, VD, cap = 12, 2, 48, 64, 64
    g = nd.kv_geom(H, KVH, QK, VD, cap)
    blk, nb = nd.kv_alloc(g)
    q = torch.zeros(1, H * QK, device="cuda")
    for lo, hi in [(5, 4), (0, 64), (-1, 3)]:
        out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(np.array([lo], np.int32)),
                                     dev(np.array([hi], np.int32)), q, exact=True))
        assert np.isnan(out).all()


def test_attend_exact_many_sessions_ragged(ctx):
    """13 sessions x 2 kv heads: 26 head groups, a grid padded to whole XCD rounds."""
    H, KVH, QK, VD, cap, count = 12, 2, 48, 64, 640, 13
    rng = np.random.default_rng(23)
    g, blk, nb = _fill(ctx, rng, H, KVH, QK, VD, cap, cap, count)
    q = rng.normal(size=(count, H * QK)).astype(np.float32)
    hi = rng.integers(0, cap, size=count).astype(np.int32)
    lo = np.maximum(hi - rng.integers(0, cap, size=count), 0).astype(np.int32)
    out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(lo), dev(hi), dev(q), quant_query=True,
                                 exact=True))
    blocks = host(blk)
    for i in range(count):
        want = _oracle(g, blocks[i * nb:(i + 1) * nb], O.quant_rows(q[i], 1, H, QK),
                       int(lo[i]), int(hi[i]))
        assert _same_bits(out[i], want), i


def test_attend_exact_large_cap(ctx):
    """cap above 8192 takes the single-role kernel; same bits."""
    H, KVH, QK, VD, cap = 4, 2, 16, 32, 9000
    rng = np.random.default_rng(29)
    g, blk, nb = _fill(ctx, rng, H, KVH, QK, VD, cap, cap)
    q = rng.normal(size=H * QK).astype(np.float32)
    for lo, hi in [(0, 8999), (4000, 4100)]:
        out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(np.array([lo], np.int32)),
                                     dev(np.array([hi], np.int32)), dev(q)[None], exact=True))[0]
        assert _same_bits(out, _oracle(g, host(blk), q, lo, hi))


def test_attend_exact_cap_8192(ctx):
    """The largest cap of the split-role kernel (scores and products fill 68 KB of LDS)."""
    H, KVH, QK, VD, cap = 12, 2, 48, 64, 8192
    rng = np.random.default_rng(31)
    g, blk, nb = _fill(ctx, rng, H, KVH, QK, VD, cap, cap)
    q = rng.normal(size=H * QK).astype(np.float32)
    for lo, hi in [(0, 8191), (100, 8191), (0, 31)]:
        out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(np.array([lo], np.int32)),
                                     dev(np.array([hi], np.int32)), dev(q)[None], exact=True))[0]
        assert _same_bits(out, _oracle(g, host(blk), q, lo, hi))


@pytest.mark.parametrize("H,KVH,QK", [(12, 2, 48), (12, 12, 64), (8, 4, 48), (12, 4, 64),
                                      (16, 4, 48), (16, 2, 64)])
@pytest.mark.parametrize("cap", [300, 2176, 10000])
def test_attend_exact_grouped_heads(ctx, H, KVH, QK, cap):
    """1, 2, 3, 4, 6 and 8 query heads per kv head (v_head_dim 64, qk 48 or
    64) at caps on both sides of the split-role kernel's 8192 limit; spans
    of 1 position up to the whole ring, across the ring's wrap, three
    sessions with different spans in one call; bit for bit against
    attend_step."""
    VD, count = 64, 3
    rng = np.random.default_rng(cap * 7 + H * 3 + KVH + QK)
    npos = cap + 300  # the ring wraps: positions 300.. overwrite the first slots
    g, blk, nb = _fill(ctx, rng, H, KVH, QK, VD, cap, npos, count, scale=2.0)
    top = npos - 1
    spans = [(top, top), (top - 255, top), (top - 256, top), (top - 511, top),
             (top - 512, top), (top - cap + 1, top), (top - cap + 1, top - 1),
             (top - (cap * 2) // 3, top - 5)]
    spans = [(lo, hi) for lo, hi in spans if hi - lo < cap and lo >= npos - cap]
    blocks = None
    for lo_v, hi_v in spans:
        q = (rng.normal(size=(count, H * QK)) * 3).astype(np.float32)
        lo = np.array([lo_v, lo_v + 1 if lo_v < hi_v else lo_v, hi_v], np.int32)
        hi = np.array([hi_v, hi_v, hi_v], np.int32)
        out = host(nd.attend_step_i8(ctx, g, blk, nb, dev(lo), dev(hi), dev(q), quant_query=True,
                                     exact=True))
        if blocks is None:
            blocks = host(blk)
        for i in range(count):
            want = _oracle(g, blocks[i * nb:(i + 1) * nb], O.quant_rows(q[i], 1, H, QK),
                           int(lo[i]), int(hi[i]))
            assert _same_bits(out[i], want), (lo_v, hi_v, i)
