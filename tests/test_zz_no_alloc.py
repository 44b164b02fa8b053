"""nd_attend_step_i8_noalloc against nd_attend_step_i8, through the C ABI.

The no-allocation entry point runs the same kernels with its split-K
partials in the library's fixed per-GPU array instead of the context
workspace, so its outputs must equal the allocating entry point's bit for
bit.  Two calls in a row, the second smaller than the first (the array
keeps the first call's partials, which the second must not read), then a
call whose partials exceed the array, which must fail cleanly and leave the
next call working.
"""
import numpy as np
import pytest
import torch

import needle_amd as nd
from conftest import dev, host

pytestmark = pytest.mark.gpu


def _case(ctx, rng, H, KVH, QK, VD, cap, spans):
    g = nd.kv_geom(H, KVH, QK, VD, cap)
    count = len(spans)
    blk, nb = nd.kv_alloc(g, count)
    for i, (lo, hi) in enumerate(spans):
        n = hi + 1
        k = rng.normal(size=(n, KVH * QK)).astype(np.float32)
        v = rng.normal(size=(n, KVH * VD)).astype(np.float32)
        pos = torch.arange(n, dtype=torch.int32, device="cuda")
        nd.kv_write(ctx, g, blk[i * nb:(i + 1) * nb], 0, pos, dev(k), dev(v))
    lo = dev(np.array([s[0] for s in spans], np.int32))
    hi = dev(np.array([s[1] for s in spans], np.int32))
    q = dev(rng.normal(size=(count, H * QK)).astype(np.float32))
    return g, blk, nb, lo, hi, q


def _both(ctx, g, blk, nb, lo, hi, q):
    a = nd.attend_step_i8(ctx, g, blk, nb, lo, hi, q, quant_query=True)
    b = nd.attend_step_i8(ctx, g, blk, nb, lo, hi, q, quant_query=True, noalloc=True)
    return host(a), host(b)


def test_noalloc_equals_allocating_entry_point(ctx):
    rng = np.random.default_rng(77)
    # 1: the Needle-3 geometry (12 q / 2 kv heads, qk 48), three sessions at
    # spans up to 4096: split 8 ways (the partials of 3 x 12 heads x 8 splits)
    first = _case(ctx, rng, 12, 2, 48, 64, 4096, [(0, 4095), (100, 2047), (3000, 3999)])
    a, b = _both(ctx, *first)
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # 2: smaller -- one config-3 session (12 x 64 MHA) at ctx 1500, 3 splits
    second = _case(ctx, rng, 12, 12, 64, 64, 1536, [(0, 1499)])
    a, b = _both(ctx, *second)
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # the first case again, after the smaller one
    a, b = _both(ctx, *first)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_noalloc_rejects_partials_beyond_its_array(ctx):
    # 8 query heads per kv head, 1 kv head, 512 positions (2 chunks of 256):
    # with `count` queries just under 4 x CUs the span splits in two, and the
    # partials (count x 8 heads x 2 splits x 66 floats) exceed the 4 MiB array
    want = 4 * torch.cuda.get_device_properties(0).multi_processor_count
    count = want - 24
    if count * 8 * 2 * 66 <= (1 << 20):
        pytest.skip(f"{want // 4} CUs: no 8-heads-per-kv-head call exceeds the array")
    H, KVH, QK, VD, cap = 8, 1, 64, 64, 512
    g = nd.kv_geom(H, KVH, QK, VD, cap)
    blk, nb = nd.kv_alloc(g, count)
    lo = dev(np.zeros(count, np.int32))
    hi = dev(np.full(count, cap - 1, np.int32))
    q = dev(np.ones((count, H * QK), np.float32))
    with pytest.raises(nd.NeedleError) as e:
        nd.attend_step_i8(ctx, g, blk, nb, lo, hi, q, noalloc=True)
    assert e.value.code == nd.ND_ERR_ARG and "no-allocation scratch" in str(e.value)
    # a call that fits still works afterwards
    rng = np.random.default_rng(5)
    small = _case(ctx, rng, 12, 2, 48, 64, 1024, [(0, 700)])
    a, b = _both(ctx, *small)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
