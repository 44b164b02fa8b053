"""Format A (Cactus-Quants) on the GPU vs the oracle.

Bit-exact: prepare_input (same butterfly) and dequantize_row (same decode,
same butterfly).  Floating point: matvec/matmul within the reference's own
tolerance form, 1e-4 * max(|want|, 1) (cq.rs:1184-1186), which at these
magnitudes is BASELINE's fp32 max-abs 1e-4.
"""
import json
import os

import numpy as np
import pytest
import torch

import needle_amd as nd
import oracle as O
from conftest import dev, host
from cq_cases import TERNARY, WIDTHS, build_case, random_case

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
REAL_CB = np.array(json.load(open(os.path.join(GOLDEN, "cq_codebook.json")))["codebook"], np.float32)


def _pair(ctx, c):
    g = nd.CqWeight(ctx, c.blob, c.out, c.in_feat, c.group, c.bits, c.codebook)
    o = O.CqWeight(c.blob, c.out, c.in_feat, c.group, c.bits, c.codebook)
    return g, o


def _close(got, want):
    return np.all(np.abs(got - want) <= 1e-4 * np.maximum(np.abs(want), 1.0))


@pytest.mark.parametrize("bits", WIDTHS)
@pytest.mark.parametrize("shape", [(5, 16, 16), (3, 40, 8), (9, 128, 128), (4, 200, 64),
                                   (24, 128, 128), (70, 768, 128)])
def test_prepare_dequant_matvec(ctx, bits, shape):
    c = build_case(*shape, bits)
    g, o = _pair(ctx, c)
    rng = np.random.default_rng(shape[0] * 10 + bits)
    x = rng.normal(size=c.in_feat).astype(np.float32)
    xh = g.prepare_input(dev(x))
    assert np.array_equal(host(xh)[0], o.prepare_input(x)), "FWHT must be bit-exact"
    rows = np.arange(c.out, dtype=np.int32)[::-1].copy()
    deq = host(g.dequantize_rows(dev(rows)))
    assert np.array_equal(deq, o.dequantize()[rows]), "dequantize_row must be bit-exact"
    y = host(g.matvec_prepared(xh[0]))
    assert _close(y, o.matvec(x))
    assert np.all(np.abs(y - c.dense @ x.astype(np.float64)) <= 1e-4 * np.maximum(
        np.abs(c.dense @ x.astype(np.float64)), 1.0))


@pytest.mark.parametrize("bits", WIDTHS)
def test_row_bands(ctx, bits):
    """A band equals the same rows of the full matvec (cq.rs:1209-1229)."""
    c = build_case(24, 128, 128, bits)
    g, o = _pair(ctx, c)
    x = np.sin(np.arange(128, dtype=np.float32) * np.float32(0.19)).astype(np.float32)
    xh = g.prepare_input(dev(x))[0]
    full = host(g.matvec_prepared(xh))
    for start, n in [(0, 4), (4, 4), (8, 16), (20, 4), (23, 1)]:
        band = host(g.matvec_rows_prepared(xh, start, n))
        assert _close(band, full[start:start + n])
        assert _close(band, o.matvec_rows_prepared(o.prepare_input(x), start, n))


@pytest.mark.parametrize("bits", WIDTHS)
@pytest.mark.parametrize("shape", [(24, 128, 128), (9, 40, 8), (5, 200, 64), (16, 512, 128)])
def test_matmul(ctx, bits, shape):
    c = build_case(*shape, bits)
    g, o = _pair(ctx, c)
    for batch in (1, 2, 7, 16, 70):
        rng = np.random.default_rng(batch)
        xs = rng.normal(size=(batch, c.in_feat)).astype(np.float32)
        xh_d = g.prepare_input(dev(xs))
        xh = o.prepare_batch(xs)
        for rs, rows in [(0, c.out), (0, 1), (1, min(3, c.out - 1))]:
            got = host(g.matmul_rows_prepared(xh_d, batch, rs, rows))
            want = o.matmul_rows_prepared(xh, batch, rs, rows)
            assert _close(got, want), (batch, rs, rows)


V3_SHAPES = [(576, 768, 2), (96, 768, 2), (128, 768, 2), (768, 768, 2), (8192, 768, 4),
             (80, 3072, 4), (84, 768, 4)]


@pytest.mark.parametrize("out,inn,bits", V3_SHAPES)
def test_v3_shapes_real_codebook(ctx, out, inn, bits):
    """The shipped v3 projection shapes with the shipped codebook."""
    rng = np.random.default_rng(out + bits)
    c = random_case(rng, out, inn, 128, bits, REAL_CB)
    g, o = _pair(ctx, c)
    x = rng.normal(size=inn).astype(np.float32)
    xh = g.prepare_input(dev(x))[0]
    y = host(g.matvec_prepared(xh))
    assert _close(y, o.matvec(x))
    xs = rng.normal(size=(64, inn)).astype(np.float32)
    got = host(g.matmul_rows_prepared(g.prepare_input(dev(xs)), 64, 0, out))
    assert _close(got, o.matmul_rows_prepared(o.prepare_batch(xs), 64, 0, out))


def test_errors_match_cqerror(ctx):
    cb = np.zeros(28, np.float32)
    blob = np.zeros(1 << 16, np.uint8)
    for args, code in [((blob, 4, 128, 128, 7, cb), 11), ((blob, 4, 128, 96, 2, cb), 12),
                       ((blob, 0, 128, 128, 2, cb), 15), ((np.zeros(4, np.uint8), 512, 512, 128, 2, cb), 14),
                       ((blob, 4, 128, 128, 2, cb[:10]), 13)]:
        with pytest.raises(nd.NeedleError) as e:
            nd.CqWeight(ctx, *args)
        assert e.value.code == code


@pytest.mark.parametrize("bits", [2, 4])
def test_matvec_tall_multi_tile(ctx, bits):
    """40,003 rows: several 16-row tiles per workgroup and a ragged last tile."""
    rng = np.random.default_rng(40003 + bits)
    out, inn = 40003, 768
    packed = rng.integers(0, 256, size=out * inn * bits // 8, dtype=np.uint8)
    norms = (np.abs(rng.normal(0.0, 0.02, size=out * (inn // 128))) * np.sqrt(128.0))
    blob = np.concatenate([packed, norms.astype(np.float16).view(np.uint8)])
    g = nd.CqWeight(ctx, blob, out, inn, 128, bits, REAL_CB)
    o = O.CqWeight(blob, out, inn, 128, bits, REAL_CB)
    x = rng.normal(size=768).astype(np.float32)
    xh = g.prepare_input(dev(x))[0]
    y = host(g.matvec_prepared(xh))
    assert _close(y, o.matvec(x))
    band = host(g.matvec_rows_prepared(xh, 17, 39000))
    assert _close(band, y[17:17 + 39000])


@pytest.mark.parametrize("bits", [2, 4])
def test_matvec_streams_past_the_stage(ctx, bits):
    """600,001 rows of in 768: each workgroup of the streaming GEMVs owns more
    tiles than it stages results for (16 tiles of 64 rows at 2 bits, 32 of 32
    at 4 bits, over 2 workgroups a CU), so results are written out mid-loop
    as well as at the end.  Against the oracle, and bit for bit against two
    half-height launches (fewer tiles a workgroup, no mid-loop write): a
    row's arithmetic does not depend on how tiles are dealt."""
    rng = np.random.default_rng(600001 + bits)
    out, inn = 600001, 768
    packed = rng.integers(0, 256, size=out * inn * bits // 8, dtype=np.uint8)
    norms = (np.abs(rng.normal(0.0, 0.02, size=out * (inn // 128))) * np.sqrt(128.0))
    blob = np.concatenate([packed, norms.astype(np.float16).view(np.uint8)])
    del packed
    g = nd.CqWeight(ctx, blob, out, inn, 128, bits, REAL_CB)
    o = O.CqWeight(blob, out, inn, 128, bits, REAL_CB)
    del blob
    x = rng.normal(size=768).astype(np.float32)
    xh = g.prepare_input(dev(x))[0]
    y = host(g.matvec_prepared(xh))
    assert _close(y, o.matvec(x))
    half = out // 2
    lo = host(g.matvec_rows_prepared(xh, 0, half))
    hi = host(g.matvec_rows_prepared(xh, half, out - half))
    assert np.array_equal(np.concatenate([lo, hi]).view(np.uint32), y.view(np.uint32))
    g.close()


# A 2-bit slot that is neither monotone nor symmetric: the fp4 kernel's
# plane coefficients are solved from the four levels, whatever they are.
SKEW_CB = REAL_CB.copy()
SKEW_CB[:4] = np.array([0.31, -0.02, 0.27, -0.4], np.float32)


def _tall_blob(rng, out, inn):
    packed = rng.integers(0, 256, size=out * inn // 4, dtype=np.uint8)
    norms = np.abs(rng.normal(0.0, 0.02, size=out * (inn // 128))) * np.sqrt(128.0)
    return np.concatenate([packed, norms.astype(np.float16).view(np.uint8)])


@pytest.fixture
def fp4_from_16k(monkeypatch):
    """The fp4 matrix-core GEMV from 16,384 rows (by default from 655,360)."""
    monkeypatch.setenv("NEEDLE_AMD_CQ_FP4_MIN_ROWS", "16384")


@pytest.mark.parametrize("bits", [2, TERNARY])
@pytest.mark.parametrize("inn", [128, 256, 384, 512, 640, 768])
def test_matvec_fp4_cores(ctx, fp4_from_16k, bits, inn):
    """20,011 rows of 2-bit or ternary codes, groups of 128, on the fp4
    matrix-core kernel: every group count 1..6, a ragged last tile, a band
    from an odd row, two codebooks, activations of one scale and of
    magnitudes spread over 2^-8 .. 2^3 inside a block, against the oracle at
    the reference's tolerance."""
    rng = np.random.default_rng(inn * 10 + bits)
    out = 20011
    blob = _tall_blob(rng, out, inn)
    xs = [rng.normal(size=inn).astype(np.float32),
          (rng.normal(size=inn) * np.exp2(rng.uniform(-8, 3, size=inn))).astype(np.float32)]
    for cb in (REAL_CB, SKEW_CB):
        g = nd.CqWeight(ctx, blob, out, inn, 128, bits, cb)
        o = O.CqWeight(blob, out, inn, 128, bits, cb)
        for x in xs:
            xh = g.prepare_input(dev(x))[0]
            xo = o.prepare_input(x)
            y = host(g.matvec_prepared(xh))
            assert _close(y, o.matvec_rows_prepared(xo, 0, out))
            band = host(g.matvec_rows_prepared(xh, 7, 17000))
            assert _close(band, o.matvec_rows_prepared(xo, 7, 17000))
        g.close()


@pytest.mark.parametrize("bits", [2, TERNARY])
def test_matvec_fp4_cores_non_finite(ctx, fp4_from_16k, bits):
    """fp4 carries no infinity or NaN: a prepared activation holding one, or
    one whose products with the plane coefficients overflow fp32, takes the
    kernel's plain path, and each row's result is +-inf or NaN exactly where
    the oracle's is."""
    rng = np.random.default_rng(77 + bits)
    out, inn = 20011, 768
    blob = _tall_blob(rng, out, inn)
    g = nd.CqWeight(ctx, blob, out, inn, 128, bits, REAL_CB)
    o = O.CqWeight(blob, out, inn, 128, bits, REAL_CB)
    base = rng.normal(size=inn).astype(np.float32)
    for put in ({300: np.inf}, {5: -np.inf}, {5: np.inf, 700: -np.inf}, {129: np.nan}):
        x = base.copy()
        for k, v in put.items():
            x[k] = v
        y = host(g.matvec_rows_prepared(dev(x), 0, out))
        want = o.matvec_rows_prepared(x, 0, out)
        assert np.array_equal(np.isnan(y), np.isnan(want)), put
        inf = np.isinf(want)
        assert np.array_equal(y[inf], want[inf]), put
        fin = np.isfinite(want)
        assert _close(y[fin], want[fin]), put
    # levels 0, 10, 0, 0: the plane coefficients are -20, 10, 5, so an
    # activation of 2e37 is finite while -20 * 2e37 is not; the reference's
    # terms (10 * 2e37 at most) stay finite, and so must the result
    big_cb = REAL_CB.copy()
    big_cb[:4] = np.array([0.0, 10.0, 0.0, 0.0], np.float32)
    gb = nd.CqWeight(ctx, blob, out, inn, 128, 2, big_cb)
    ob = O.CqWeight(blob, out, inn, 128, 2, big_cb)
    x = base.copy()
    x[200] = np.float32(2e37)
    y = host(gb.matvec_rows_prepared(dev(x), 0, out))
    want = ob.matvec_rows_prepared(x, 0, out)
    assert np.all(np.isfinite(want)) and _close(y, want)
    # 8e36: -20 * 8e36 is finite, but a piece of it times a plane value
    # (up to 4), summed over a group, is not; the block is past the matrix
    # cores' headroom and takes the plain path, and the rows stay finite
    x = base.copy()
    x[200] = np.float32(8e36)
    y = host(gb.matvec_rows_prepared(dev(x), 0, out))
    want = ob.matvec_rows_prepared(x, 0, out)
    assert np.all(np.isfinite(want)) and _close(y, want)
    gb.close()
    # and a finite activation afterwards takes the matrix cores again
    y = host(g.matvec_prepared(dev(base)))
    assert _close(y, o.matvec_rows_prepared(base, 0, out))
    g.close()


def test_matvec_fp4_cores_default_bound(ctx, monkeypatch):
    """700,001 rows of in 768 take the fp4 kernel with no override: against
    the oracle, and bit for bit against two halves of 350,000-odd rows run
    on the same kernel by a weight created with the bound lowered (a row's
    arithmetic does not depend on its tile or lane).  The bound is read when
    a weight is created."""
    monkeypatch.delenv("NEEDLE_AMD_CQ_FP4_MIN_ROWS", raising=False)
    rng = np.random.default_rng(700001)
    out, inn = 700001, 768
    blob = _tall_blob(rng, out, inn)
    g = nd.CqWeight(ctx, blob, out, inn, 128, 2, REAL_CB)
    monkeypatch.setenv("NEEDLE_AMD_CQ_FP4_MIN_ROWS", "16384")
    g16 = nd.CqWeight(ctx, blob, out, inn, 128, 2, REAL_CB)
    o = O.CqWeight(blob, out, inn, 128, 2, REAL_CB)
    del blob
    x = rng.normal(size=inn).astype(np.float32)
    xh = g.prepare_input(dev(x))[0]
    y = host(g.matvec_prepared(xh))
    assert _close(y, o.matvec(x))
    half = out // 2
    lo = host(g16.matvec_rows_prepared(xh, 0, half))
    hi = host(g16.matvec_rows_prepared(xh, half, out - half))
    assert np.array_equal(np.concatenate([lo, hi]).view(np.uint32), y.view(np.uint32))
    # the default-bound weight keeps its bound whatever the variable says now
    assert np.array_equal(host(g.matvec_prepared(xh)).view(np.uint32), y.view(np.uint32))
    g16.close()
    g.close()
