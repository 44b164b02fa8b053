"""Pins the oracle's Cactus-Quants, FWHT, f16 and Format-B restatements.

Mirrors needle-rs's own unit tests (crates/needle-core/src/cq.rs:966-1431,
hadamard.rs:69-173, math.rs:70-130) and adds closed forms and brute force
that a dropped term, a wrong index or a transposed operand would fail.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle as O
from cq_cases import TERNARY, WIDTHS, build_case, fake_codebook, pack_lsb, random_case, sylvester


# ---- math.rs ----------------------------------------------------------------

def test_f16_known_values():
    """math.rs:77-93."""
    f = O.f16_to_f32
    assert f(0x0000) == 0.0 and math.copysign(1, f(0x8000)) == -1
    assert f(0x3C00) == 1.0 and f(0xBC00) == -1.0 and f(0x4000) == 2.0
    assert np.float32(f(0x3555)) == np.float32(0.33325195)
    assert f(0x7BFF) == 65504.0
    assert np.float32(f(0x0001)) == np.float32(5.9604645e-8)
    assert np.float32(f(0x03FF)) == np.float32(6.0975552e-5)
    assert np.float32(f(0x0400)) == np.float32(6.1035156e-5)
    assert math.isinf(f(0x7C00)) and f(0x7C00) > 0
    assert math.isinf(f(0xFC00)) and f(0xFC00) < 0
    assert math.isnan(f(0x7E00))


def test_f16_every_half_matches_numpy():
    """Exhaustive: every binary16 pattern equals numpy's exact widening."""
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(b)) for b in bits], np.float32)
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.isnan(got[~fin]).all()


# ---- hadamard.rs ------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 2, 4, 8, 16, 128, 512, 1024])
def test_fwht_matches_dense_exactly(n):
    """hadamard.rs:102-120: small-integer inputs make every partial sum exact."""
    i = np.arange(n)
    x = (((i * 7 + i // 5) % 19) - 9).astype(np.float32)
    want = sylvester(n) @ x.astype(np.float64)
    assert np.array_equal(O.fwht(x), want.astype(np.float32))


@pytest.mark.parametrize("n", [8, 128, 512])
def test_fwht_fractional(n):
    """hadamard.rs:122-145."""
    i = np.arange(n, dtype=np.float32)
    x = (np.sin(i * np.float32(0.37)) + np.float32(0.3) * np.cos(i * np.float32(0.11))).astype(np.float32)
    want = sylvester(n) @ x.astype(np.float64)
    l1 = np.abs(x).sum()
    assert np.all(np.abs(O.fwht(x) - want) <= 1e-5 * l1)


def test_fwht_normalized_is_involutive():
    """hadamard.rs:147-158."""
    x = np.cos(np.arange(128, dtype=np.float32) * np.float32(0.11)).astype(np.float32)
    y = O.fwht_normalized(O.fwht_normalized(x))
    assert np.all(np.abs(y - x) < 1e-4)


# ---- cq.rs: bit reader and LUT ----------------------------------------------

@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_read_bits_brute_force(bits):
    """Every field read back equals what an independent LSB-first packer wrote."""
    rng = np.random.default_rng(bits)
    n = 8 * 37
    idx = rng.integers(0, 1 << bits, size=n).astype(np.uint8)
    row = pack_lsb(idx, 1, n, bits)
    got = [O.read_bits(np.append(row, 0), k * bits, bits) for k in range(n)]
    assert np.array_equal(np.array(got), idx)


def test_build_lut_every_byte():
    """cq.rs:932-964: byte b's k-th code is (b >> k*w) & mask, LSB first;
    ternary crumbs map 3->0, 0->1, 1->2, 2->1."""
    lv16 = np.arange(16, dtype=np.float32) + 0.5
    per, lut = O.build_lut(4, lv16)
    assert per == 2
    b = np.arange(256)
    assert np.array_equal(lut.reshape(256, 2), np.stack([lv16[b & 15], lv16[b >> 4]], 1))
    per, lut = O.build_lut(2, lv16[:4])
    assert per == 4
    assert np.array_equal(lut.reshape(256, 4),
                          np.stack([lv16[(b >> (2 * k)) & 3] for k in range(4)], 1))
    tern = np.array([-1.0, 0.0, 1.0], np.float32)
    per, lut = O.build_lut(TERNARY, tern)
    crumb_to_trit = np.array([1, 2, 1, 0])
    assert per == 4
    assert np.array_equal(lut.reshape(256, 4),
                          np.stack([tern[crumb_to_trit[(b >> (2 * k)) & 3]] for k in range(4)], 1))
    assert O.build_lut(3, lv16[:8])[0] == 0


# ---- cq.rs: CqWeight --------------------------------------------------------

def _weight(c):
    return O.CqWeight(c.blob, c.out, c.in_feat, c.group, c.bits, c.codebook)


@pytest.mark.parametrize("bits", WIDTHS)
@pytest.mark.parametrize("shape", [(5, 16, 16), (3, 40, 8), (7, 128, 128)])
def test_dequantize_matches_reconstruction(bits, shape):
    """cq.rs:1146-1161."""
    c = build_case(*shape, bits)
    got = _weight(c).dequantize()
    assert np.all(np.abs(got - c.dense) < 1e-5)


@pytest.mark.parametrize("bits", WIDTHS)
@pytest.mark.parametrize("shape", [(5, 16, 16), (3, 40, 8), (9, 128, 128), (4, 200, 64)])
def test_matvec_matches_dense_multiply(bits, shape):
    """cq.rs:1165-1192 (dense is float64 here)."""
    c = build_case(*shape, bits)
    i = np.arange(c.in_feat, dtype=np.float32)
    x = (np.sin(i * np.float32(0.31)) * np.float32(1.7) + np.float32(0.05) * i).astype(np.float32)
    got = _weight(c).matvec(x)
    want = c.dense @ x.astype(np.float64)
    assert np.all(np.abs(got - want) < 1e-4 * np.maximum(np.abs(want), 1.0))


def test_padding_does_not_leak():
    """cq.rs:1195-1206."""
    c = build_case(6, 40, 32, 2)
    x = (1.0 + np.arange(40)).astype(np.float32)
    got = _weight(c).matvec(x)
    want = c.dense @ x
    assert np.all(np.abs(got - want) < 1e-3 * np.maximum(np.abs(want), 1.0))


@pytest.mark.parametrize("bits", WIDTHS)
def test_row_band_equals_full(bits):
    """cq.rs:1209-1229, bit-exact."""
    c = build_case(24, 128, 128, bits)
    w = _weight(c)
    x = np.sin(np.arange(128, dtype=np.float32) * np.float32(0.19)).astype(np.float32)
    full = w.matvec(x)
    xh = w.prepare_input(x)
    for start, n in [(0, 4), (4, 4), (8, 16), (20, 4), (23, 1)]:
        assert np.array_equal(w.matvec_rows_prepared(xh, start, n), full[start:start + n])


@pytest.mark.parametrize("bits", [2, 4, TERNARY])
@pytest.mark.parametrize("shape", [(6, 768, 128), (5, 40, 8), (3, 200, 64)])
def test_matvec_lane_order_bit_exact(bits, shape):
    """matvec_lut_impl::<P> (cq.rs:721-735) with dot_group::<P> (cq.rs:838-873)
    restated in numpy float32: each group's levels go element k -> lane k % 8,
    a multiply then an add, the lanes summed 0..7, then `total += norm * acc`
    over the groups in order.  The oracle must give exactly these bits."""
    rng = np.random.default_rng(7 + bits)
    c = random_case(rng, *shape, bits, fake_codebook(shape[2]))
    w = _weight(c)
    x = rng.normal(size=c.in_feat).astype(np.float32)
    xh = w.prepare_input(x)
    got = w.matvec_prepared(xh)
    vals = c.levels[c.idx]  # [out, in_pad] decoded levels
    want = np.zeros(c.out, np.float32)
    for o in range(c.out):
        total = np.float32(0)
        for g in range(c.num_groups):
            sl = slice(g * c.group, (g + 1) * c.group)
            acc = _lanes_dot(vals[o, sl], xh[sl])
            total = np.float32(total + np.float32(c.norms_f32[o, g] * acc))
        want[o] = total
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits", WIDTHS)
@pytest.mark.parametrize("shape", [(16, 128, 128), (5, 40, 8), (7, 200, 64), (9, 512, 128)])
def test_matvec_matches_simple_reference(bits, shape):
    """cq.rs:1236-1268."""
    c = build_case(*shape, bits)
    w = _weight(c)
    x = (np.sin(np.arange(c.in_feat, dtype=np.float32) * np.float32(0.29)) * 2).astype(np.float32)
    xh = w.prepare_input(x)
    fast, slow = w.matvec_prepared(xh), w.matvec_prepared_reference(xh)
    l1 = np.abs(xh).sum()
    assert np.all(np.abs(fast - slow) <= 1e-5 * max(l1, 1.0))


@pytest.mark.parametrize("bits", WIDTHS)
@pytest.mark.parametrize("shape", [(24, 128, 128), (9, 40, 8), (5, 200, 64), (16, 512, 128)])
def test_matmul_equals_repeated_matvec(bits, shape):
    """cq.rs:1270-1323: bit-identical, not merely close."""
    c = build_case(*shape, bits)
    w = _weight(c)
    for batch in (1, 2, 7, 16):
        xs = np.stack([(np.sin((np.arange(c.in_feat) + b * 13).astype(np.float32) * np.float32(0.23))
                        * np.float32(1.3)).astype(np.float32) for b in range(batch)])
        xh = w.prepare_batch(xs)
        for rs, rows in [(0, c.out), (0, 1), (1, min(3, c.out - 1))]:
            if rows == 0 or rs + rows > c.out:
                continue
            got = w.matmul_rows_prepared(xh, batch, rs, rows).reshape(batch, rows)
            for b in range(batch):
                assert np.array_equal(got[b], w.matvec_rows_prepared(xh[b], rs, rows))


def test_prepared_input_reusable():
    """cq.rs:1325-1345."""
    a, b = _weight(build_case(4, 128, 128, 2)), _weight(build_case(6, 128, 128, 4))
    x = np.cos(np.arange(128, dtype=np.float32) * np.float32(0.07)).astype(np.float32)
    xh = a.prepare_input(x)
    assert np.array_equal(a.matvec_prepared(xh), a.matvec(x))
    assert np.array_equal(b.matvec_prepared(xh), b.matvec(x))


def test_shipped_v2_blob_sizes():
    """cq.rs:1347-1363."""
    for out, inn, bits, group, want in [(8192, 512, 4, 128, 2_162_688), (512, 512, 2, 128, 69_632),
                                        (256, 512, 2, 128, 34_816), (108, 2048, 4, 128, 114_048),
                                        (432, 2048, 4, 128, 456_192), (32768, 128, 2, 128, 1_114_112)]:
        pad = -(-inn // group) * group
        assert out * O.packed_row_bytes(pad, bits) + out * (pad // group) * 2 == want


def test_shipped_v3_records_parse(golden_dir):
    """Every CQ record of the shipped v3 directory: the blob size the loader
    needs equals the record's nbytes, and a blob of exactly that size parses."""
    recs = json.load(open(os.path.join(golden_dir, "v3_cq_records.json")))["records"]
    cb = np.array(json.load(open(os.path.join(golden_dir, "cq_codebook.json")))["codebook"], np.float32)
    assert len(recs) == 122
    for r in recs:
        out, inn = r["shape"]
        pad = -(-inn // r["group"]) * r["group"]
        need = out * O.packed_row_bytes(pad, r["bits"]) + out * (pad // r["group"]) * 2
        assert need == r["nbytes"], r
    r = [x for x in recs if x["shape"] == [576, 768]][0]
    w = O.CqWeight(np.zeros(r["nbytes"], np.uint8), 576, 768, 128, 2, cb)
    assert (w.row_bytes, w.num_groups, w.in_padded) == (192, 6, 768)
    with pytest.raises(O.CqError):
        O.CqWeight(np.zeros(r["nbytes"] - 1, np.uint8), 576, 768, 128, 2, cb)


def test_rejects_bad_geometry():
    """cq.rs:1365-1393."""
    cb = fake_codebook(128)
    blob = np.zeros(1 << 16, np.uint8)
    cases = [((blob, 4, 128, 128, 7, cb), 1), ((blob, 4, 128, 96, 2, cb), 2),
             ((blob, 4, 128, 100, 2, cb), 2), ((blob, 0, 128, 128, 2, cb), 5),
             ((blob, 4, 0, 128, 2, cb), 5), ((np.zeros(4, np.uint8), 512, 512, 128, 2, cb), 4),
             ((blob, 4, 128, 128, 2, cb[:10]), 3)]
    for args, code in cases:
        with pytest.raises(O.CqError) as e:
            O.CqWeight(*args)
        assert e.value.code == code


def test_real_codebook_matvec():
    """The shipped 28-float Lloyd-Max codebook at the v3 q_proj shape."""
    cb = np.array(json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                              "cq_codebook.json")))["codebook"], np.float32)
    rng = np.random.default_rng(7)
    from cq_cases import random_case
    for bits in (2, 4):
        c = random_case(rng, 64, 768, 128, bits, cb)
        w = _weight(c)
        x = rng.normal(size=768).astype(np.float32)
        want = c.dense @ x.astype(np.float64)
        assert np.all(np.abs(w.matvec(x) - want) < 1e-4 * np.maximum(np.abs(want), 1.0))


# ---- Format B ---------------------------------------------------------------

def test_cb8_gemv_against_f64_brute_force():
    rng = np.random.default_rng(11)
    out, inn = 192, 768
    w = rng.integers(0, 256, size=(out, inn), dtype=np.uint8)
    cb = (rng.normal(0, 0.02, size=(out // 64, 256))).astype(np.float32)
    x = rng.normal(size=inn).astype(np.float32)
    dense = cb[np.arange(out)[:, None] // 64, w].astype(np.float64)
    want = dense @ x.astype(np.float64)
    got = O.cb8_gemv(w, cb, x)
    assert np.max(np.abs(got - want)) < 2e-6
    assert np.max(np.abs(O.cb8_gemv_f64(w, cb, x) - want)) < 1e-12
    # The codebook tile is o // 64: swapping two tiles' codebooks must change rows.
    cb2 = cb[::-1].copy()
    assert np.max(np.abs(O.cb8_gemv(w, cb2, x) - got)) > 1e-3
    X = rng.normal(size=(5, inn)).astype(np.float32)
    Y = O.cb8_gemm(X, w, cb)
    assert np.max(np.abs(Y - X.astype(np.float64) @ dense.T)) < 2e-6


def _lanes_dot(u, x):
    """cq.rs:879-895 / :838-873's eight-lane order in numpy float32: element
    k into lane k % 8 (a multiply, then an add), lanes summed 0..7, then the
    tail added in order."""
    u = u.astype(np.float32)
    x = x.astype(np.float32)
    n = u.size - u.size % 8
    lanes = np.zeros(8, np.float32)
    for c in range(0, n, 8):
        lanes = lanes + u[c:c + 8] * x[c:c + 8]
    s = np.float32(0)
    for v in lanes:
        s = np.float32(s + v)
    for k in range(n, u.size):
        s = np.float32(s + u[k] * x[k])
    return s


@pytest.mark.parametrize("inn", [768, 96, 100, 7])
def test_cb8_lanes_kernels_follow_the_eight_lane_order(inn):
    """The CPU baseline's Format B kernels: the eight-lane order exactly (a
    numpy restatement, tail included when `in` is not a multiple of 8),
    within float rounding of the f64 closed form, and the same bits on any
    thread count."""
    rng = np.random.default_rng(31 + inn)
    out = 130
    w = rng.integers(0, 256, size=(out, inn), dtype=np.uint8)
    cb = rng.normal(0, 0.02, size=((out + 63) // 64, 256)).astype(np.float32)
    x = rng.normal(size=inn).astype(np.float32)
    dense = cb[np.arange(out)[:, None] // 64, w]
    got = O.cb8_gemv_lanes(w, cb, x)
    want = np.array([_lanes_dot(dense[o], x) for o in range(out)], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ref = dense.astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(got - ref)) < 2e-6
    assert np.array_equal(O.cb8_gemv_lanes(w, cb, x, 4).view(np.uint32), got.view(np.uint32))
    X = rng.normal(size=(6, inn)).astype(np.float32)
    Y = O.cb8_gemm_lanes(X, w, cb)
    wantY = np.array([[_lanes_dot(dense[o], X[i]) for o in range(out)] for i in range(6)],
                     np.float32)
    assert np.array_equal(Y.view(np.uint32), wantY.view(np.uint32))
    assert np.array_equal(O.cb8_gemm_lanes(X, w, cb, 3).view(np.uint32), Y.view(np.uint32))
    assert np.max(np.abs(Y - X.astype(np.float64) @ dense.T.astype(np.float64))) < 2e-6
