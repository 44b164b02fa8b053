"""nd_fold_rows on the GPU against the sequential float32 sum, bit for bit.

Rows of terms >= +0 go through the exact parallel fold (nd_fold.h); signed,
-0 and infinite rows take its plain-chain path.  The generators aim at the
method's edges: exact ties at every scale, subnormals, powers of two, a
binade crossing on every step, zero prefixes, a huge early term."""
import numpy as np
import pytest

import fold_cases

pytestmark = pytest.mark.gpu

SIZES = (1, 5, 127, 128, 200, 768, 1000, 2048, 3072, 4096)


@pytest.fixture(scope="module")
def ctx():
    import needle_amd as nd
    return nd.Ctx(0)


@pytest.mark.parametrize("kind", fold_cases.KINDS)
def test_fold_rows_bit_exact(ctx, kind):
    import torch
    import needle_amd as nd
    rng = np.random.default_rng(1000 + fold_cases.KINDS.index(kind))
    for n in SIZES:
        x = fold_cases.rows_of(kind, 64, n, rng)
        want = fold_cases.sequential_sums(x)
        got = nd.fold_rows(ctx, torch.from_numpy(x).cuda()).cpu().numpy()
        bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
        assert bad.size == 0, (kind, n, bad[:5], got[bad[:5]], want[bad[:5]])


def test_fold_rows_rejects_bad_sizes(ctx):
    import torch
    import needle_amd as nd
    x = torch.zeros((2, 4097), dtype=torch.float32, device="cuda")
    with pytest.raises(nd.NeedleError):
        nd.fold_rows(ctx, x)
