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


# ---- powf, sinf, cosf: the RoPE table's functions --------------------------
# math.rs:13-36 call libm 0.2.16's sinf, cosf and powf, the msun algorithms
# (s_sinf.c, s_cosf.c with k_sinf.c / k_cosf.c and the e_rem_pio2f.c /
# k_rem_pio2.c reductions; e_powf.c).  Their only caller on the path is the
# RoPE table: freq_i = 1 / powf(theta, 2i / qk) and angle = pos * freq_i
# (v3/model.rs:378-413), theta 1e5, qk 48, pos < max_seq_len = 8192.

THETA, QK, MAX_POS = np.float32(100000.0), 48, 8192


def _ulp_dist(got, want):
    """|got - want| in float32 ulps, across zero too (sign-magnitude bits
    mapped onto a monotone integer line)."""
    def line(a):
        b = a.view(np.int32).astype(np.int64)
        return np.where(b < 0, -(b & 0x7fffffff), b)
    return np.abs(line(np.ascontiguousarray(got, np.float32)) -
                  line(np.ascontiguousarray(want, np.float32)))


def _rope_exponents():
    return (np.arange(QK // 2, dtype=np.float32) * np.float32(2)) / np.float32(QK)


def _rope_angles():
    freq = np.float32(1.0) / O.powf(THETA, _rope_exponents())
    pos = np.arange(MAX_POS, dtype=np.float32)
    return (pos[:, None] * freq[None, :]).astype(np.float32).ravel()


def _trig_sample():
    rng = np.random.default_rng(3)
    small = rng.uniform(-10.0, 10.0, 1_000_000).astype(np.float32)
    mid = rng.uniform(-1e5, 1e5, 1_000_000).astype(np.float32)
    # every exponent up to 2^127 (the Payne-Hanek range from 2^28 pi/2 on)
    bits = rng.integers(0x30000000, 0x7f800000, 2_000_000, dtype=np.uint32)
    e = bits.view(np.float32)
    # around multiples of pi/2, where the reduction loses the most bits
    k = rng.integers(1, 1 << 20, 200_000).astype(np.float64)
    near = (k * (np.pi / 2)).astype(np.float32)
    return np.concatenate([_rope_angles(), small, mid, e, -e, near, -near])


def _pow_sample():
    rng = np.random.default_rng(4)
    x = np.concatenate([rng.uniform(0.0, 4.0, 1_000_000),
                        10.0 ** rng.uniform(-30, 30, 1_000_000),
                        rng.integers(1, 0x7f800000, 500_000, dtype=np.uint32).view(np.float32)])
    y = np.concatenate([rng.uniform(-8.0, 8.0, 1_000_000),
                        rng.uniform(-1.0, 1.0, 1_000_000),
                        rng.uniform(-0.7, 0.7, 500_000)])
    x, y = x.astype(np.float32), y.astype(np.float32)
    # the RoPE calls themselves, and integral and half-integral exponents
    rx = np.full(QK // 2, THETA, np.float32)
    ix = rng.uniform(0.1, 3.0, 100_000).astype(np.float32)
    iy = rng.integers(-20, 21, 100_000).astype(np.float32) / np.float32(2)
    # x just off 1 with |y| > 2^27 (the x - x^2/2 + x^3/3 branch)
    nx = (np.float32(1.0) + rng.integers(-7, 8, 20_000).astype(np.float32) * np.float32(2.0 ** -23))
    ny = rng.uniform(2.0 ** 27.5, 2.0 ** 30, 20_000).astype(np.float32) * \
        np.where(rng.random(20_000) < 0.5, -1, 1).astype(np.float32)
    return (np.concatenate([x, rx, ix, nx]).astype(np.float32),
            np.concatenate([y, _rope_exponents(), iy, ny]).astype(np.float32))


def test_sinf_cosf_within_one_ulp_of_exact():
    x = _trig_sample()
    xd = x.astype(np.float64)
    for mine, exact in ((O.sinf, np.sin), (O.cosf, np.cos)):
        got = mine(x)
        want = exact(xd).astype(np.float32)
        u = _ulp_dist(got, want)
        assert u.max() <= 1, (x[np.argmax(u)], u.max())
        assert np.mean(u == 0) > 0.99


def test_powf_within_one_ulp_of_exact():
    x, y = _pow_sample()
    got = O.powf(x, y)
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        want = np.power(x.astype(np.float64), y.astype(np.float64)).astype(np.float32)
    fin = np.isfinite(want) & (want != 0)
    assert np.array_equal(np.isinf(got), np.isinf(want))
    u = _ulp_dist(got[fin], want[fin])
    assert u.max() <= 1, (x[fin][np.argmax(u)], y[fin][np.argmax(u)], u.max())
    assert np.mean(u == 0) > 0.9


def test_trig_and_pow_special_values():
    inf, nan = np.float32(np.inf), np.float32(np.nan)
    s = O.sinf(np.array([0.0, -0.0, 1e-30, -1e-5, inf, -inf, nan], np.float32))
    assert s[0] == 0.0 and not np.signbit(s[0]) and s[1] == 0.0 and np.signbit(s[1])
    assert s[2] == np.float32(1e-30) and s[3] == np.float32(-1e-5)  # |x| < 2^-12: x itself
    assert np.all(np.isnan(s[4:]))
    c = O.cosf(np.array([0.0, -0.0, 1e-5, inf, nan], np.float32))
    assert c[0] == 1.0 and c[1] == 1.0 and c[2] == 1.0 and np.all(np.isnan(c[3:]))
    sub = np.array([1], np.uint32).view(np.float32)[0]
    cases = [  # (x, y, expected) from e_powf.c's documented special cases
        (nan, 0.0, 1.0), (1.0, nan, 1.0), (-1.0, inf, 1.0), (-1.0, -inf, 1.0),
        (2.0, inf, inf), (2.0, -inf, 0.0), (0.5, inf, 0.0), (0.5, -inf, inf),
        (0.0, -1.0, inf), (-0.0, -1.0, -inf), (-0.0, -2.0, inf), (-0.0, 3.0, -0.0),
        (-2.0, 3.0, -8.0), (-2.0, 2.0, 4.0), (-2.0, 0.5, nan), (inf, -0.5, 0.0),
        (-inf, 3.0, -inf), (4.0, 0.5, 2.0), (3.0, 2.0, 9.0), (7.0, -1.0, np.float32(1.0) / np.float32(7.0)),
        (2.0, 128.0, inf), (2.0, 127.0, np.float32(2.0) ** 127), (2.0, -149.0, sub), (2.0, -151.0, 0.0),
        (2.0, -126.0, np.float32(2.0) ** -126), (100000.0, 0.5, np.float32(np.sqrt(np.float32(100000.0))))]
    x = np.array([c[0] for c in cases], np.float32)
    y = np.array([c[1] for c in cases], np.float32)
    want = np.array([c[2] for c in cases], np.float32)
    got = O.powf(x, y)
    for a, b, g, w in zip(x, y, got, want):
        assert (np.isnan(g) and np.isnan(w)) or (g == w and np.signbit(g) == np.signbit(w)), (a, b, g, w)


def test_rope_table_against_f64():
    """The table the forward uses: every (pos < 8192, frequency) entry within
    1 ulp of the exactly rounded cos/sin of its float angle, and each
    frequency within 1 ulp of 1 / theta^(2i/qk)."""
    e = _rope_exponents()
    p = O.powf(THETA, e)
    want = np.power(np.float64(THETA), e.astype(np.float64)).astype(np.float32)
    assert _ulp_dist(p, want).max() <= 1
    a = _rope_angles()
    assert _ulp_dist(O.cosf(a), np.cos(a.astype(np.float64)).astype(np.float32)).max() <= 1
    assert _ulp_dist(O.sinf(a), np.sin(a.astype(np.float64)).astype(np.float32)).max() <= 1


def test_device_header_trig_and_pow_agree_bitwise(tmp_path):
    """nd_libm.h's sinf / cosf / powf (the copy the device library uses for
    its RoPE table) built for the host vs the oracle's copy, bit for bit."""
    shim = tmp_path / "shim.c"
    shim.write_text(
        '#include <stddef.h>\n#include "nd_libm.h"\n'
        "void t_sin(const float *x, size_t n, float *y) { for (size_t i = 0; i < n; i++) y[i] = nd_sinf(x[i]); }\n"
        "void t_cos(const float *x, size_t n, float *y) { for (size_t i = 0; i < n; i++) y[i] = nd_cosf(x[i]); }\n"
        "void t_pow(const float *x, const float *e, size_t n, float *y) "
        "{ for (size_t i = 0; i < n; i++) y[i] = nd_powf(x[i], e[i]); }\n")
    so = tmp_path / "shim.so"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-shared", "-fPIC",
                    "-I", CSRC, str(shim), "-o", str(so), "-lm"], check=True)
    import ctypes as C
    lib = C.CDLL(str(so))
    f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
    lib.t_sin.argtypes = lib.t_cos.argtypes = [f32p, C.c_size_t, f32p]
    lib.t_pow.argtypes = [f32p, f32p, C.c_size_t, f32p]

    def same(a, b):
        nan = np.isnan(a) & np.isnan(b)
        return np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan])

    walk = (np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32)).view(np.float32)
    x = np.ascontiguousarray(np.concatenate([walk, _trig_sample()]), np.float32)
    for fn, theirs in ((lib.t_sin, O.sinf), (lib.t_cos, O.cosf)):
        y = np.empty_like(x)
        fn(x, x.size, y)
        assert same(y, theirs(x))
    px, py = _pow_sample()
    rng = np.random.default_rng(9)
    wx = walk[rng.permutation(walk.size)]
    wy = walk[rng.permutation(walk.size)]
    px = np.ascontiguousarray(np.concatenate([px, wx, np.abs(wx)]), np.float32)
    with np.errstate(invalid="ignore"):
        py = np.ascontiguousarray(np.concatenate([py, wy, wy * np.float32(1e-30)]), np.float32)
    y = np.empty_like(px)
    lib.t_pow(px, py, px.size, y)
    assert same(y, O.powf(px, py))
