"""expf and logf as the reference computes them: math.rs:3-11 calls libm
0.2.16 (Cargo.lock:267-269), whose expf/logf are the FreeBSD msun
algorithms (e_expf.c, e_logf.c).  The oracle restates them (needle_oracle.c)
and so does the device header (needle-rs_amd/csrc/nd_libm.h).

No Rust toolchain runs here, so the restatements are pinned by what the
mathematics fixes -- within 1 ulp of the exactly rounded value everywhere
(the published error bound of both algorithms), the special values and
thresholds the source documents -- and by bit equality between the two
independently written copies, so a slip in either (a wrong constant, a
dropped term) fails a check.
"""
import os
import subprocess

import numpy as np
import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "needle-rs_amd", "csrc")


def _ulps(got, want):
    """|got - want| in units in the last place, both finite float32 >= 0."""
    g = got.view(np.int32).astype(np.int64)
    w = want.view(np.int32).astype(np.int64)
    return np.abs(g - w)


def _exp_sample():
    rng = np.random.default_rng(0)
    a = rng.uniform(-104.0, 89.0, 2_000_000).astype(np.float32)
    b = rng.uniform(-1.0, 1.0, 1_000_000).astype(np.float32)
    # every exponent: |x| from 2^-30 to 2^7 at random mantissas, both signs
    e = rng.integers(0x30800000, 0x43000000, 1_000_000, dtype=np.uint32).view(np.float32)
    c = np.concatenate([a, b, e, -e])
    return c[(c > -104.5) & (c < 89.0)]


def _log_sample():
    rng = np.random.default_rng(1)
    bits = rng.integers(1, 0x7f800000, 4_000_000, dtype=np.uint32)  # positive, incl. subnormal
    near_one = rng.uniform(0.5, 2.0, 1_000_000).astype(np.float32)
    return np.concatenate([bits.view(np.float32), near_one])


def test_expf_within_one_ulp_of_exact():
    x = _exp_sample()
    got = O.expf(x)
    with np.errstate(over="ignore"):
        want = np.exp(x.astype(np.float64)).astype(np.float32)
    assert np.all(np.isfinite(got) == np.isfinite(want))
    fin = np.isfinite(want)
    u = _ulps(got[fin], want[fin])
    assert u.max() <= 1, (x[fin][np.argmax(u)], u.max())
    # correctly rounded for most inputs (about 93% over this sample)
    assert np.mean(u == 0) > 0.9


def test_logf_within_one_ulp_of_exact():
    x = _log_sample()
    got = O.logf(x)
    want = np.log(x.astype(np.float64)).astype(np.float32)
    diff = np.abs(got.view(np.int32).astype(np.int64) -
                  want.view(np.int32).astype(np.int64))
    same_sign = np.signbit(got) == np.signbit(want)
    assert np.all(same_sign | (want == 0))
    assert diff[want != 0].max() <= 1
    assert np.mean(diff == 0) > 0.9


def test_special_values():
    inf, nan = np.float32(np.inf), np.float32(np.nan)
    e = O.expf(np.array([0.0, -0.0, inf, -inf, 89.0, 88.72283, -104.0, -103.97, 1e-9, -1e-9],
                        np.float32))
    assert e[0] == 1.0 and e[1] == 1.0
    assert e[2] == inf and e[3] == 0.0
    assert e[4] == inf and np.isfinite(e[5]) and e[5] > 3.4e38
    assert e[6] == 0.0 and 0.0 < e[7] < 1.2e-38  # a subnormal result, not flushed
    assert e[8] == np.float32(1.0) + np.float32(1e-9) and e[9] == np.float32(1.0) - np.float32(1e-9)
    assert np.isnan(O.expf(np.array([nan], np.float32))[0])
    sub = np.array([1], np.uint32).view(np.float32)[0]
    g = O.logf(np.array([1.0, 0.0, -0.0, -1.0, inf, sub, 2.0, 0.5], np.float32))
    assert g[0] == 0.0
    assert g[1] == -inf and g[2] == -inf
    assert np.isnan(g[3]) and g[4] == inf
    assert abs(g[5] - np.float32(-103.27893)) < 1e-4  # log(2^-149)
    assert g[6] == np.float32(np.log(2.0)) and g[7] == -g[6]


def test_oracle_and_device_header_agree_bitwise(tmp_path):
    """nd_libm.h (the device copy) built for the host vs the oracle's copy."""
    shim = tmp_path / "shim.c"
    shim.write_text(
        '#include <stddef.h>\n#include "nd_libm.h"\n'
        "void t_exp(const float *x, size_t n, float *y) { for (size_t i = 0; i < n; i++) y[i] = nd_expf(x[i]); }\n"
        "void t_log(const float *x, size_t n, float *y) { for (size_t i = 0; i < n; i++) y[i] = nd_logf(x[i]); }\n"
        "void t_sig(const float *x, size_t n, float *y) { for (size_t i = 0; i < n; i++) y[i] = nd_sigmoidf(x[i]); }\n")
    so = tmp_path / "shim.so"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-shared", "-fPIC",
                    "-I", CSRC, str(shim), "-o", str(so)], check=True)
    import ctypes as C
    lib = C.CDLL(str(so))
    f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
    for fn in (lib.t_exp, lib.t_log, lib.t_sig):
        fn.argtypes = [f32p, C.c_size_t, f32p]
    rng = np.random.default_rng(7)
    # a strided walk over every float32 bit pattern plus the dense samples
    walk = (np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32)).view(np.float32)
    for x, mine, theirs in ((np.concatenate([walk, _exp_sample()]), lib.t_exp, O.expf),
                            (np.concatenate([walk, _log_sample()]), lib.t_log, O.logf)):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        mine(x, x.size, y)
        want = theirs(x)
        both_nan = np.isnan(y) & np.isnan(want)
        assert np.array_equal(y.view(np.uint32)[~both_nan], want.view(np.uint32)[~both_nan])
    x = rng.normal(0, 10, 100_000).astype(np.float32)
    y = np.empty_like(x)
    lib.t_sig(x, x.size, y)
    want = (np.float32(1.0) / (np.float32(1.0) + O.expf(-x))).astype(np.float32)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
