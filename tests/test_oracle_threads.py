"""The oracle's thread splits keep its bits.

The reference splits a CqWeight call across its rayon pool past fixed size
rules -- row bands of max(ceil(rows/threads), 64) for a matvec of >= 128
rows and >= 2^20 multiply-adds, and for a matmul row bands (rows >= 128)
or batch bands of max(ceil(batch/threads), 8) (batch >= 16)
(crates/needle-core/src/cq.rs:301-323, 446-581, constants :815-823) --
and each row's arithmetic is unchanged, so every split equals the serial
loop bit for bit (the reference's own test, cq.rs:1209-1229, checks row
bands).  The oracle restates those rules for the CPU baseline and has a
checker mode that also splits the smaller loops and attention's heads.
Both must give the serial bits, on shapes either side of every threshold.
"""
import json
import os

import numpy as np
import pytest

import oracle as O
from cq_cases import random_case

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
REAL_CB = np.array(json.load(open(os.path.join(GOLDEN, "cq_codebook.json")))["codebook"], np.float32)


@pytest.fixture(autouse=True)
def _serial_after():
    yield
    O.set_threads(1, O.SPLIT_REFERENCE)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# (out, in, bits, row_start, rows): 127/128 rows at 1 M MACs either side of
# should_parallelise, the LM head, a band of a tall weight, ragged bands.
SHAPES = [(128, 8192, 2, 0, 128), (127, 8320, 2, 0, 127), (8192, 768, 4, 0, 8192),
          (1400, 768, 2, 100, 1300), (640, 3072, 4, 0, 640), (96, 768, 2, 0, 96),
          (200, 384, 3, 0, 200)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("threads,split", [(3, O.SPLIT_REFERENCE), (8, O.SPLIT_REFERENCE),
                                           (5, O.SPLIT_ALL)])
def test_matvec_splits_keep_bits(shape, threads, split):
    out, inn, bits, r0, rows = shape
    rng = np.random.default_rng(out + inn + bits)
    c = random_case(rng, out, inn, 128, bits, REAL_CB)
    w = O.CqWeight(c.blob, out, inn, 128, bits, REAL_CB)
    xh = w.prepare_input(rng.normal(size=inn).astype(np.float32) * 5)
    O.set_threads(1, O.SPLIT_REFERENCE)
    want = w.matvec_rows_prepared(xh, r0, rows)
    O.set_threads(threads, split)
    assert np.array_equal(_bits(w.matvec_rows_prepared(xh, r0, rows)), _bits(want))


@pytest.mark.parametrize("rows,batch", [(256, 64), (100, 64), (100, 16), (100, 15), (16, 40),
                                        (300, 7)])
@pytest.mark.parametrize("threads,split", [(4, O.SPLIT_REFERENCE), (7, O.SPLIT_ALL)])
def test_matmul_row_and_batch_bands_keep_bits(rows, batch, threads, split):
    inn = 768
    rng = np.random.default_rng(rows * 100 + batch)
    c = random_case(rng, rows + 8, inn, 128, 2, REAL_CB)
    w = O.CqWeight(c.blob, rows + 8, inn, 128, 2, REAL_CB)
    xh = w.prepare_batch(rng.normal(size=(batch, inn)).astype(np.float32))
    O.set_threads(1, O.SPLIT_REFERENCE)
    want = w.matmul_rows_prepared(xh, batch, 3, rows)
    O.set_threads(threads, split)
    assert np.array_equal(_bits(w.matmul_rows_prepared(xh, batch, 3, rows)), _bits(want))
    # and matmul == matvec per batch row (cq.rs:1270-1323)
    O.set_threads(1, O.SPLIT_REFERENCE)
    for b in (0, batch - 1):
        assert np.array_equal(_bits(want[b * rows:(b + 1) * rows]),
                              _bits(w.matvec_rows_prepared(xh[b], 3, rows)))


def test_attention_heads_on_threads_keep_bits():
    H, KVH, QK, VD, slots = 12, 2, 48, 64, 700
    rng = np.random.default_rng(5)
    k = rng.integers(-127, 128, size=slots * KVH * QK).astype(np.int8)
    v = rng.integers(-127, 128, size=slots * KVH * VD).astype(np.int8)
    ks = (rng.random(slots * KVH) * 0.05 + 1e-3).astype(np.float32)
    vs = (rng.random(slots * KVH) * 0.05 + 1e-3).astype(np.float32)
    q = rng.normal(size=H * QK).astype(np.float32)
    O.set_threads(1, O.SPLIT_REFERENCE)
    want = O.attend_step_i8(q, k, ks, v, vs, slots, 50, 699, H, KVH, QK, VD)
    O.set_threads(6, O.SPLIT_ALL)
    got = O.attend_step_i8(q, k, ks, v, vs, slots, 50, 699, H, KVH, QK, VD)
    assert np.array_equal(_bits(got), _bits(want))


def test_decode_steps_keep_bits_under_every_split():
    import v3_synth as S
    g, recs = S.build_records(S.small_geometry(3), seed=4)
    om = O.V3Model(g, recs, S.CODEBOOK)
    prompt = S.prompt_tokens(20, 9)
    runs = []
    for threads, split in ((1, O.SPLIT_REFERENCE), (4, O.SPLIT_REFERENCE), (4, O.SPLIT_ALL)):
        O.set_threads(threads, split)
        cache = om.new_cache(24, True)
        runs.append(np.stack([cache.decode_step(t) for t in prompt]))
    for r in runs[1:]:
        assert np.array_equal(_bits(r), _bits(runs[0]))


def test_session_splits_keep_bits():
    """The CPU baseline's session-parallel helpers give each session's own
    serial result: decode steps of three sessions at once, attention over
    four sessions' caches, and the row-band Format B GEMM."""
    import v3_synth as S
    g, recs = S.build_records(S.small_geometry(2), seed=8)
    om = O.V3Model(g, recs, S.CODEBOOK)
    prompts = [S.prompt_tokens(6, 40 + i) for i in range(3)]
    serial = []
    for p in prompts:
        c = om.new_cache(8, True)
        serial.append(np.stack([c.decode_step(t) for t in p]))
    caches = [om.new_cache(8, True) for _ in prompts]
    par = np.stack([O.v3_decode_sessions(om, caches, [p[t] for p in prompts], 3)
                    for t in range(6)], axis=1)
    assert np.array_equal(_bits(par), _bits(np.stack(serial)))

    rng = np.random.default_rng(12)
    H, KVH, QK, VD, slots, n = 12, 12, 64, 64, 300, 4
    k = rng.integers(-127, 128, size=(n, slots * KVH * QK)).astype(np.int8)
    v = rng.integers(-127, 128, size=(n, slots * KVH * VD)).astype(np.int8)
    ks = (rng.random((n, slots * KVH)) * 0.05 + 1e-3).astype(np.float32)
    vs = (rng.random((n, slots * KVH)) * 0.05 + 1e-3).astype(np.float32)
    q = rng.normal(size=(n, H * QK)).astype(np.float32)
    got = O.attend_step_i8_sessions(q, k, ks, v, vs, slots, 0, slots - 1, H, KVH, QK, VD, 3)
    for i in range(n):
        want = O.attend_step_i8(q[i], k[i], ks[i], v[i], vs[i], slots, 0, slots - 1, H, KVH, QK, VD)
        assert np.array_equal(_bits(got[i]), _bits(want))

    w = rng.integers(0, 256, size=(192, 96), dtype=np.uint8)
    cb = rng.normal(0, 0.02, size=(3, 256)).astype(np.float32)
    x = rng.normal(size=(5, 96)).astype(np.float32)
    assert np.array_equal(_bits(O.cb8_gemm_omp(x, w, cb, 4)), _bits(O.cb8_gemm(x, w, cb)))


def test_synthetic_cache_runs_a_decode_step():
    import v3_synth as S
    g, recs = S.build_records(S.small_geometry(2), seed=8)
    om = O.V3Model(g, recs, S.CODEBOOK)
    c = om.new_cache(80, True)
    c.fill_synthetic(70, 3)
    lg = c.decode_step(5)
    assert np.isfinite(lg).all()
