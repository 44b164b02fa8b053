"""The device copies of the reference's libm wrappers (math.rs:3-46: libm
0.2.16's expf and logf, and the sigmoid built on expf) against the oracle's
independent restatement, bit for bit, on the GPU: a strided walk over every
float32 bit pattern (every 4099th, both signs, specials, subnormals) and
the dense samples the oracle is pinned on (test_oracle_libm.py).  The
device functions are written as straight-line selects over msun's paths,
so this is what checks that each input class still lands on msun's
arithmetic.  NaN results need only both be NaN."""
import numpy as np
import pytest
import torch

import needle_amd as nd
import oracle as O
from conftest import dev, host
from test_oracle_libm import _exp_sample, _log_sample

pytestmark = pytest.mark.gpu

WALK = (np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32)).view(np.float32)
EDGES = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 88.72283, 88.7228, 89.0,
                  -103.97208, -103.972084, -104.0, 2.0 ** -14, -2.0 ** -14, 2.0 ** -15,
                  0.34657359, -0.34657359, 1.0397208, -1.0397208, 87.33655, -87.33655,
                  np.float32(1.17549435e-38), np.float32(1.4e-45), 3.4028235e38],
                 np.float32)


def _same(got, want):
    both_nan = np.isnan(got) & np.isnan(want)
    return np.array_equal(got.view(np.uint32)[~both_nan], want.view(np.uint32)[~both_nan]) \
        and np.array_equal(np.isnan(got), np.isnan(want))


@pytest.mark.parametrize("fn,oracle,sample", [("expf", O.expf, _exp_sample),
                                              ("logf", O.logf, _log_sample)])
def test_device_libm_equals_oracle(ctx, fn, oracle, sample):
    x = np.ascontiguousarray(np.concatenate([WALK, EDGES, sample()]), np.float32)
    got = host(nd.libm_map(ctx, fn, dev(x)))
    want = oracle(x)
    bad = ~((got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want)))
    assert _same(got, want), (x[bad][:8], got[bad][:8], want[bad][:8])


def test_device_sigmoid_equals_oracle(ctx):
    rng = np.random.default_rng(3)
    x = np.ascontiguousarray(np.concatenate([WALK, EDGES, rng.normal(0, 10, 1_000_000)]), np.float32)
    got = host(nd.libm_map(ctx, "sigmoid", dev(x)))
    with np.errstate(over="ignore"):
        want = (np.float32(1.0) / (np.float32(1.0) + O.expf(-x))).astype(np.float32)
    assert _same(got, want)
