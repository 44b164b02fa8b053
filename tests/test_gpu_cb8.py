"""Format B (uint8 codes, per-64-row fp32 codebooks) on the GPU vs the oracle.

GEMV: max-abs <= 1e-4 against the oracle's fp32 closed form (BASELINE's fp32
bar).  GEMM: bf16 MFMA, max|Y - Y_ref| / max|Y_ref| <= 2e-2.
"""
import numpy as np
import pytest
import torch

import needle_amd as nd
import oracle as O
from conftest import dev, host

pytestmark = pytest.mark.gpu


def _problem(rng, out, inn):
    w = rng.integers(0, 256, size=(out, inn), dtype=np.uint8)
    cb = rng.normal(0.0, 0.02, size=(-(-out // 64), 256)).astype(np.float32)
    x = rng.normal(size=inn).astype(np.float32)
    return w, cb, x


def test_gemv_3072x768_shape(ctx):
    """3072 x 768, 48 codebooks, x ~ N(0,1), seed 1."""
    rng = np.random.default_rng(1)
    w, cb, x = _problem(rng, 3072, 768)
    y = host(nd.cb8_gemv(ctx, dev(w), dev(cb), dev(x)))
    want = O.cb8_gemv(w, cb, x)
    assert np.max(np.abs(y - want)) <= 1e-4
    assert np.max(np.abs(y - O.cb8_gemv_f64(w, cb, x))) <= 1e-4


@pytest.mark.parametrize("out,inn", [(1, 16), (64, 256), (128, 512), (100, 768), (1, 768),
                                     (130, 784), (65, 1024), (200, 1040), (64, 4096)])
def test_gemv_ragged(ctx, out, inn):
    rng = np.random.default_rng(out * 7 + inn)
    w, cb, x = _problem(rng, out, inn)
    y = host(nd.cb8_gemv(ctx, dev(w), dev(cb), dev(x)))
    assert np.max(np.abs(y - O.cb8_gemv(w, cb, x))) <= 1e-4


def test_gemv_extreme_codes(ctx):
    """All-0 and all-255 codes pick the first and last codebook entries."""
    out, inn = 128, 768
    cb = np.arange(2 * 256, dtype=np.float32).reshape(2, 256) * np.float32(1e-3)
    x = np.ones(inn, np.float32)
    for code in (0, 255):
        w = np.full((out, inn), code, np.uint8)
        y = host(nd.cb8_gemv(ctx, dev(w), dev(cb), dev(x)))
        want = np.repeat(cb[:, code] * inn, 64)
        assert np.max(np.abs(y - want)) <= 1e-4 * max(1.0, np.abs(want).max())


def test_gemv_batched_distinct_problems(ctx):
    rng = np.random.default_rng(5)
    count, out, inn = 6, 3072, 768
    W = rng.integers(0, 256, size=(count, out, inn), dtype=np.uint8)
    CB = rng.normal(0, 0.02, size=(count, out // 64, 256)).astype(np.float32)
    X = rng.normal(size=(count, inn)).astype(np.float32)
    Y = torch.zeros(count, out, device="cuda")
    nd.cb8_gemv_batched(ctx, dev(W), dev(CB), dev(X), Y)
    Y = host(Y)
    for i in range(count):
        assert np.max(np.abs(Y[i] - O.cb8_gemv(W[i], CB[i], X[i]))) <= 1e-4


def test_gemv_rejects_misaligned_width(ctx):
    w = torch.zeros(64, 24, dtype=torch.uint8, device="cuda")
    cb = torch.zeros(1, 256, device="cuda")
    x = torch.zeros(24, device="cuda")
    with pytest.raises(nd.NeedleError) as e:
        nd.cb8_gemv(ctx, w, cb, x)
    assert e.value.code == 1 and "multiple of 16" in str(e.value)


@pytest.mark.parametrize("m,out,inn", [(512, 3072, 768), (512, 768, 768), (1, 64, 768),
                                       (100, 192, 768), (200, 256, 96), (130, 384, 160),
                                       (96, 128, 32), (64, 3072, 768), (50, 768, 768),
                                       (1, 256, 128), (33, 384, 1024), (64, 128, 256)])
def test_gemm_bf16_mfma(ctx, m, out, inn):
    """Every tile shape: the M <= 64 streaming kernel (out and K multiples
    of 128), 64x64 below M = 96 or when out is not a multiple of 128, else
    128x128; K not a multiple of the K step, ragged M."""
    rng = np.random.default_rng(m + out + inn)
    w = rng.integers(0, 256, size=(out, inn), dtype=np.uint8)
    cb = rng.normal(0, 0.02, size=(out // 64, 256)).astype(np.float32)
    X = rng.normal(size=(m, inn)).astype(np.float32)
    Y = host(nd.cb8_gemm(ctx, dev(X), dev(w), dev(cb)))
    ref = O.cb8_gemm(X, w, cb)
    rel = np.max(np.abs(Y - ref)) / np.max(np.abs(ref))
    assert rel <= 2e-2, rel
    # bf16 inputs, fp32 accumulation: far tighter than the gate in practice
    assert np.linalg.norm(Y - ref) / np.linalg.norm(ref) <= 5e-3


@pytest.mark.parametrize("R,M,N,K", [(11, 512, 3072, 768), (43, 300, 768, 768),
                                     (43, 300, 768, 800)])
def test_gemm_256_tiles_match_128_tiles(ctx, R, M, N, K):
    """A batched launch with at least one 256x256 tile per CU runs the
    256x256 kernel; each problem alone has too few tiles and runs the
    128x128 one.  Per output both sum K in the same order, so they agree
    bit for bit, with K in whole 64-wide steps and with a final half step
    (K 800).  Ragged M; two problems also against the oracle."""
    rng = np.random.default_rng(R * 1000 + K)
    X = rng.normal(size=(R, M, K)).astype(np.float32)
    W = rng.integers(0, 256, size=(R, N, K), dtype=np.uint8)
    CB = (rng.normal(size=(R, N // 64, 256)) * 0.02).astype(np.float32)
    Y = torch.empty(R, M, N, device="cuda")
    nd.cb8_gemm_batched(ctx, dev(X), dev(W), dev(CB), Y)
    got = host(Y)
    for i in range(R):
        one = host(nd.cb8_gemm(ctx, dev(X[i]), dev(W[i]), dev(CB[i])))
        assert np.array_equal(got[i], one), i
    for i in (0, R - 1):
        want = O.cb8_gemm(X[i], W[i], CB[i])
        assert np.max(np.abs(got[i] - want)) <= 2e-2 * np.max(np.abs(want))
        assert np.linalg.norm(got[i] - want) / np.linalg.norm(want) <= 5e-3


def test_gemm_256_edges(ctx):
    """The 256x256 kernel on its edges: ragged M (300 = 256 + 44 rows),
    16 problems of N 4096 (512 tiles, 64 codebook groups each), codebooks
    holding +-0, a subnormal and a bf16 rounding tie; outputs against the
    f64 closed form (bf16 operands, fp32 sums)."""
    R, M, N, K = 16, 300, 4096, 768
    rng = np.random.default_rng(77)
    X = rng.normal(size=(R, M, K)).astype(np.float32)
    W = rng.integers(0, 256, size=(R, N, K), dtype=np.uint8)
    CB = (rng.normal(size=(R, N // 64, 256)) * 0.02).astype(np.float32)
    CB[:, :, 0] = 0.0
    CB[:, :, 1] = -0.0
    CB[:, :, 2] = np.float32(1e-40)
    CB[:, :, 3] = np.float32(1.0 + 2.0 ** -8)  # a bf16 tie: rounds to even
    Y = torch.empty(R, M, N, device="cuda")
    nd.cb8_gemm_batched(ctx, dev(X), dev(W), dev(CB), Y)
    got = host(Y)

    def bf16(a):
        u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
        u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
        return u.astype(np.uint32).view(np.float32)
    rows = np.arange(N)
    for i in (0, 7, R - 1):
        deq = CB[i][rows // 64][rows[:, None], W[i].astype(np.int64)]  # (N, K)
        ref = bf16(X[i]).astype(np.float64) @ bf16(deq).astype(np.float64).T
        err = np.max(np.abs(got[i] - ref)) / np.max(np.abs(ref))
        assert err <= 1e-5, (i, err)


@pytest.mark.parametrize("R,M,N,K", [(3, 70, 128, 96), (5, 64, 384, 768), (4, 17, 256, 256)])
def test_gemm_batched_equals_single(ctx, R, M, N, K):
    """Problem i of one batched launch is bit-identical to its own launch
    (the 64x64 kernel, and the M <= 64 streaming kernel)."""
    rng = np.random.default_rng(21 + M)
    X = rng.normal(size=(R, M, K)).astype(np.float32)
    W = rng.integers(0, 256, size=(R, N, K), dtype=np.uint8)
    CB = (rng.normal(size=(R, N // 64, 256)) * 0.02).astype(np.float32)
    Y = torch.empty(R, M, N, device="cuda")
    nd.cb8_gemm_batched(ctx, dev(X), dev(W), dev(CB), Y)
    got = host(Y)
    for i in range(R):
        one = host(nd.cb8_gemm(ctx, dev(X[i]), dev(W[i]), dev(CB[i])))
        assert np.array_equal(got[i], one)
        want = O.cb8_gemm(X[i], W[i], CB[i])
        assert np.max(np.abs(got[i] - want)) <= 2e-2 * np.max(np.abs(want))


def _rne_bf16(a):
    """fp32 -> bf16 (as fp32), round to nearest even, by the integer form."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("count,m,out,inn", [(1, 64, 128, 128), (1, 128, 128, 64), (256, 256, 256, 64)])
def test_gemm_bf16_rounding_is_round_to_nearest_even(ctx, count, m, out, inn):
    """The GEMMs round X and the codebook to bf16 by round-to-nearest-even.
    X in [1, 2) with its low 16 bits drawn from the tie and near-tie
    patterns, codebook entries +-1 and +-1/2 (exact in bf16), K <= 128: every
    product and partial sum is exact in fp32, so the output is the exact sum
    of rne(x) * cb[code] whatever the accumulation order, and a rounding
    other than RNE (ties away, truncation) changes it.  The shapes take the
    M <= 64, 128x128 and 256x256 kernels."""
    rng = np.random.default_rng(7 + m)
    hi = rng.integers(0x3F80, 0x4000, size=(count, m, inn), dtype=np.uint32)
    lo = rng.choice(np.array([0x8000, 0x7FFF, 0x8001, 0x0000, 0xFFFF], np.uint32), size=(count, m, inn))
    X = ((hi << 16) | lo).view(np.float32)
    W = rng.integers(0, 256, size=(count, out, inn), dtype=np.uint8)
    CB = rng.choice(np.array([1.0, -1.0, 0.5, -0.5], np.float32), size=(count, out // 64, 256))
    want = np.empty((count, m, out), np.float32)
    for i in range(count):
        wv = CB[i][np.arange(out)[:, None] // 64, W[i]].astype(np.float64)  # [out][in]
        want[i] = (_rne_bf16(X[i]).astype(np.float64) @ wv.T).astype(np.float32)
    # the ties decide: truncation or ties-away would differ somewhere
    assert not np.array_equal(_rne_bf16(X), (X.view(np.uint32) >> 16 << 16).view(np.float32))
    Y = torch.empty(count, m, out, device="cuda")
    nd.cb8_gemm_batched(ctx, dev(X), dev(W), dev(CB), Y)
    got = host(Y)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
