"""CPU checks of the exact parallel fold (needle-rs_amd/csrc/nd_fold.h).

The fold's arithmetic -- binade bounds, in-binade units, run sums -- is
shared host/device code.  fold_fuzz.cpp models the algorithm on the host
with those functions, and emulates nd_fold_nonneg lane for lane (DPP scans,
wave carries, the threads' item offsets), and compares both bit for bit with
the plain sequential loop over adversarial inputs (ties, subnormals, powers
of two, a binade crossing every step, huge ranges, a crossing at a wave's
first or last chunk); the emulated items must match the sequential list in
count and order.  The plain loop is the truth the
reference's sums follow (kernels.rs:22-24, norm.rs:25,
v3/attention.rs:361-365)."""
import os
import shutil
import subprocess

import numpy as np
import pytest

import fold_cases

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "needle-rs_amd", "csrc")


@pytest.fixture(scope="module")
def fuzz_bin(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    out = str(tmp_path_factory.mktemp("fold") / "fold_fuzz")
    subprocess.run([gxx, "-O2", "-std=c++17", "-ffp-contract=off", "-I", CSRC, "-o", out,
                    os.path.join(HERE, "fold_fuzz.cpp")], check=True)
    return out


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_parallel_fold_model_matches_the_loop(fuzz_bin, seed):
    r = subprocess.run([fuzz_bin, "4000", str(seed)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.strip().splitlines()
    assert lines[-1] == "OK"
    # every generator ran, none mismatched
    kinds = [l for l in lines if l.startswith("kind")]
    assert len(kinds) == 12
    assert "lead items" in lines[-2]
    assert all(" mismatches 0 " in l for l in kinds)


def test_sequential_sums_is_the_loop():
    """The GPU test's truth, numpy's add.accumulate, is the element-by-element
    loop (pairwise summation would differ on these rows)."""
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal((4, 300)).astype(np.float32) * 1e4,
                        np.ones((4, 300), np.float32) * np.float32(1e-4)], axis=1)
    x[:, 0] = 1e8
    want = []
    for row in x:
        s = np.float32(0.0)
        for v in row:
            s = np.float32(s + v)
        want.append(s)
    got = fold_cases.sequential_sums(x)
    assert np.array_equal(got.view(np.uint32), np.array(want, np.float32).view(np.uint32))
    pairwise = x.sum(axis=1, dtype=np.float32)
    assert not np.array_equal(pairwise, got)  # the rows do tell the two orders apart
