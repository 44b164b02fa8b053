"""The device greedy pick (nd_argmax_rows; the kernel behind nd_v3_step's
`next`) against the engine's argmax (needle-infer/src/v3_engine.rs:410-420):
a strict `>` scan from -inf, so the first of tied maxima wins, NaN never
wins, and a row of -inf or NaN gives 0.

Ties are planted where the device's parallel scan splits a row: across
lanes of one float4, across float4s, across threads (the lower index held
by the higher thread), across waves, at the first and last index; on rows
whose length is a multiple of 4 (the float4 path), not one (the scalar
path) and at a misaligned start (the scalar path).
"""
import numpy as np
import pytest
import torch

import needle_amd as nd
import oracle as O

pytestmark = pytest.mark.gpu


def _scan(row):
    """v3_engine.rs:410-420 as a Python loop."""
    best, top = 0, -np.inf
    for i, v in enumerate(row.tolist()):
        if v > top:
            top, best = v, i
    return best


def _rows(n, rng):
    rows, names = [], []

    def add(name, r):
        names.append(name)
        rows.append(r.astype(np.float32))

    base = rng.normal(size=n)
    add("random", base)
    for name, idx in (("first_last", (0, n - 1)), ("in_float4", (5, 6)),
                      ("across_float4", (3, 4)), ("across_threads", (1023, 1024)),
                      ("across_waves", (255, 256)), ("thread_order", (4 * 200 + 1, 4 * 3 + 2)),
                      ("far_apart", (n // 2 + 1, n - 2))):
        r = base.copy()
        for i in idx:
            if i < n:
                r[i] = 50.0
        add(name, r)
    add("all_equal", np.full(n, 0.25))
    add("all_neg_inf", np.full(n, -np.inf))
    add("all_nan", np.full(n, np.nan))
    r = np.full(n, -np.inf)
    r[n - 1] = -1e30
    add("last_finite", r)
    r = base.copy()
    r[0] = np.nan
    r[n // 3] = np.nan
    add("nan_between", r)
    r = -np.abs(base) - 1.0
    r[min(10, n - 1)] = -0.0
    r[min(20, n - 1)] = 0.0
    add("signed_zero_tie", r)
    r = base.copy()
    r[n - 1] = np.inf
    r[min(7, n - 1)] = np.inf
    add("two_inf", r)
    return names, np.stack(rows)


@pytest.mark.parametrize("n", [8192, 8190, 4096 + 3, 1024, 5, 1])
@pytest.mark.parametrize("misaligned", [False, True])
def test_argmax_first_maximum(ctx, n, misaligned):
    rng = np.random.default_rng(n)
    names, x = _rows(n, rng)
    want = [_scan(r) for r in x]
    assert want == [O.argmax(r) for r in x]
    flat = np.concatenate([np.zeros(1, np.float32), x.reshape(-1)]) if misaligned else x.reshape(-1)
    t = torch.from_numpy(flat).cuda()
    xd = (t[1:] if misaligned else t).view(x.shape)
    got = nd.argmax_rows(ctx, xd).cpu().numpy().tolist()
    bad = [(nm, g, w) for nm, g, w in zip(names, got, want) if g != w]
    assert not bad, bad


def test_argmax_rejects_bad_input(ctx):
    x = torch.zeros(2, 8, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError):
        nd.argmax_rows(ctx, x)
    y = torch.zeros(8, 2, device="cuda").t()
    with pytest.raises(ValueError):
        nd.argmax_rows(ctx, y)
