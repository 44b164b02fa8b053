"""Pins the oracle's int8 quantiser, V3Cache ring and attention restatements.

Mirrors crates/needle-core/tests/v3_kv_quant_parity.rs, v3/cache.rs:537-877
and v3/attention.rs:379-457, plus an f64 textbook softmax-attention check.
"""
import json
import os

import numpy as np
import pytest

import oracle as O


def _cases(golden_dir):
    v = json.load(open(os.path.join(golden_dir, "kv_quant_vectors.json")))
    assert v["bits"] == 8
    return v["cases"]


def test_fake_quant_matches_upstream(golden_dir):
    """v3_kv_quant_parity.rs:18-65 at its tolerance, and tighter on the codes:
    the stored integers equal upstream's round(out / scale) exactly.  (The
    dequantised floats agree to 1.4e-7 relative: upstream's own q*scale
    rounds a last ulp differently from the reference's multiply.)"""
    names = []
    for case in _cases(golden_dir):
        dim = case["dim"]
        x = np.array(case["in"], np.float32)
        want = np.array(case["out"], np.float32)
        got = np.concatenate([O.fake_quant_vec(c) for c in x.reshape(-1, dim)])
        tol = np.maximum(np.abs(want), 1.0) * 1e-5
        assert np.all(np.abs(got - want) <= tol), case["name"]
        for r, w in zip(x.reshape(-1, dim), want.reshape(-1, dim)):
            ints, s = O.quant_into(r)
            assert np.array_equal(np.round(w.astype(np.float64) / s), ints.astype(np.float64))
        names.append(case["name"])
    assert names == ["qk_head_dim_48", "v_head_dim_64", "all_zero", "one_spike", "tiny", "huge"]


def test_all_zero_survives():
    """v3_kv_quant_parity.rs:67-73."""
    assert np.all(O.fake_quant_vec(np.zeros(48, np.float32)) == 0)
    ints, s = O.quant_into(np.zeros(48, np.float32))
    assert s == 1.0 and np.all(ints == 0)


def test_error_bounded_by_half_step():
    """v3_kv_quant_parity.rs:75-92."""
    x = (np.sin(np.arange(64, dtype=np.float32) * np.float32(0.37)) * 3).astype(np.float32)
    step = np.abs(x).max() / 127.0
    assert np.all(np.abs(O.fake_quant_vec(x) - x) <= step * 0.5 + 1e-6)


def test_stored_ints_reproduce_fake_quant(golden_dir):
    """cache.rs:93-97: i8 * scale is exactly what fake_quant leaves behind."""
    rng = np.random.default_rng(3)
    for dim in (48, 64):
        for _ in range(200):
            x = (rng.normal(size=dim) * 10 ** rng.uniform(-8, 6)).astype(np.float32)
            ints, s = O.quant_into(x)
            # equal as values (fake_quant keeps round()'s -0.0, the int is 0)
            assert np.array_equal(ints.astype(np.float32) * s, O.fake_quant_vec(x))
            assert ints.min() >= -127 and np.abs(ints).max() == 127


def test_quantizer_closed_form():
    """Independent restatement in numpy: scale=absmax/127, inv=1/scale,
    q = round-half-away(x*inv) clamped to [-128,127]."""
    rng = np.random.default_rng(5)
    x = rng.normal(size=(300, 64)).astype(np.float32) * np.float32(3)
    ints, scales = O.quantize_rows(x, 64)
    absmax = np.abs(x).max(axis=1)
    s = (absmax / np.float32(127)).astype(np.float32)
    inv = (np.float32(1) / s).astype(np.float32)
    p = (x * inv[:, None]).astype(np.float32)
    r = np.sign(p) * np.floor(np.abs(p) + np.float32(0.5))
    assert np.array_equal(scales, s)
    assert np.array_equal(ints.reshape(300, 64), np.clip(r, -128, 127).astype(np.int8))


# ---- v3/cache.rs ring -------------------------------------------------------

TIE_ROW = np.array([127.0, 2.5, -3.5, 0.5, -0.5, 126.5, -126.5, 1.5, -2.5, 3.0,
                    0.0, 0.0, 0.0, 0.0, 0.0, 0.0], np.float32)
TIE_CODES = [127, 3, -4, 1, -1, 127, -127, 2, -3, 3, 0, 0, 0, 0, 0, 0]


def test_roundf_ties_round_away_from_zero():
    """A product x * (1 / scale) on exactly k + 0.5 rounds away from zero:
    the contract of libm's roundf, which the reference's quantiser calls
    (math.rs:39-41; cache.rs:98-104), and which no fixture of the reference
    holds.  A row whose absmax is 127 has scale 127 / 127 = 1 and inverse 1
    exactly, so its codes are the rounded values themselves."""
    ints, scales = O.quantize_rows(TIE_ROW, TIE_ROW.size)
    assert scales[0] == np.float32(1.0)
    assert ints.tolist() == TIE_CODES
    # the row does tell the tie rules apart: half-to-even differs
    assert np.rint(TIE_ROW).astype(int).tolist() != TIE_CODES
    assert np.array_equal(O.fake_quant_vec(TIE_ROW), np.array(TIE_CODES, np.float32))


def test_int8_ring_wraps_and_grows():
    """cache.rs:578-636 with the toy geometry (1 kv head, qk 4, window 4)."""
    r = O.Ring(True, 1, 4, 4, hint=2, window=4, max_seq_len=64)
    for pos in range(10):
        m = np.float32(pos + 1)
        k = m * (np.arange(4, dtype=np.float32) + 1)
        r.write_kv(pos, k, -k)
    assert r.slots == 4
    st = r.store()
    assert st["k"].size == 16 and st["k_scale"].size == 4
    slot = 9 % 4
    want = O.fake_quant_vec(np.float32(10) * (np.arange(4, dtype=np.float32) + 1))
    got = st["k"][slot * 4:(slot + 1) * 4].astype(np.float32) * st["k_scale"][slot]
    assert np.all(np.abs(got - want) <= 1e-4 * np.maximum(np.abs(want), 1))


def test_layers_grow_to_cap():
    """cache.rs:638-665."""
    loc = O.Ring(False, 1, 4, 4, hint=2, window=4, max_seq_len=64)
    glo = O.Ring(False, 1, 4, 4, hint=2, window=0, max_seq_len=64)
    assert loc.slots == 2 and glo.slots == 2
    one = np.ones(4, np.float32)
    loc.write_kv(3, one, one)
    assert loc.slots == 4
    loc.write_kv(99, one, one)
    assert loc.slots == 4
    glo.write_kv(9, one, one)
    assert glo.slots >= 10


def test_global_never_over_reads():
    """cache.rs:699-730."""
    r = O.Ring(False, 2, 48, 64, hint=8, window=0, max_seq_len=8)
    z = np.zeros(96, np.float32)
    for pos in range(12):
        r.write_kv(pos, z, np.zeros(128, np.float32))
        lo, hi = r.span(pos)
        assert hi - lo < r.slots


def test_spans_bound_local_only():
    """cache.rs:795-812."""
    loc = O.Ring(False, 1, 4, 4, hint=8, window=4, max_seq_len=64)
    glo = O.Ring(False, 1, 4, 4, hint=8, window=0, max_seq_len=64)
    z = np.zeros(4, np.float32)
    for pos in range(11):
        loc.write_kv(pos, z, z)
        glo.write_kv(pos, z, z)
    assert loc.span(2) == (0, 2) and loc.span(10) == (7, 10)
    assert glo.span(10) == (0, 10)


# ---- v3/attention.rs --------------------------------------------------------

def test_attend_step_wraps_the_ring():
    """attention.rs:399-431: mean of 20, 30, 40."""
    out = O.attend_step_f32([0.0], [1.0, 1.0, 1.0], [30.0, 40.0, 20.0], 3, 2, 4, 1, 1, 1, 1)
    assert abs(out[0] - 30.0) < 1e-5


def test_window_of_one():
    """attention.rs:433-456."""
    out = O.attend_f32([1.0, 1.0], [1.0, 1.0], [5.0, 9.0], 2, 1, 1, 1, 1, window=1)
    assert list(out) == [5.0, 9.0]
    out = O.attend_f32([1.0, 1.0], [1.0, 1.0], [5.0, 9.0], 2, 1, 1, 1, 1, window=0)
    assert out[0] == 5.0 and abs(out[1] - 7.0) < 1e-6


def _xorshift(seed):
    s = [seed]

    def nxt():
        x = s[0]
        x ^= (x << 13) & 0xFFFFFFFFFFFFFFFF
        x ^= x >> 7
        x ^= (x << 17) & 0xFFFFFFFFFFFFFFFF
        s[0] = x
        return np.float32(np.float32((x >> 11) / float(1 << 53)) * np.float32(2.0) - np.float32(1.0))
    return nxt


def test_hoisted_scale_reader_matches_dequantised_buffer():
    """v3_kv_quant_parity.rs:102-218, same xorshift64 recipe and ranges."""
    H, KVH, QK, V, SLOTS = 4, 2, 48, 64, 17
    nxt = _xorshift(0x243F6A8885A308D3)
    q = np.array([nxt() for _ in range(H * QK)], np.float32)

    def spread(rows, width, lo, hi):
        out = []
        for r in range(rows):
            m = np.float32(lo if r % 2 == 0 else hi)
            out.extend(np.float32(nxt() * m) for _ in range(width))
        return np.array(out, np.float32)

    k_raw = spread(SLOTS * KVH, QK, 1.0, 40.0)
    v_raw = spread(SLOTS * KVH, V, 0.01, 3.0)
    k_deq = np.concatenate([O.fake_quant_vec(c) for c in k_raw.reshape(-1, QK)])
    v_deq = np.concatenate([O.fake_quant_vec(c) for c in v_raw.reshape(-1, V)])
    kq, ks = O.quantize_rows(k_raw, QK)
    vq, vs = O.quantize_rows(v_raw, V)
    for lo, hi in [(0, 0), (0, 9), (3, 16), (5, 5)]:
        a = O.attend_step_f32(q, k_deq, v_deq, SLOTS, lo, hi, H, KVH, QK, V)
        b = O.attend_step_i8(q, kq, ks, vq, vs, SLOTS, lo, hi, H, KVH, QK, V)
        rms = np.sqrt(np.mean(a.astype(np.float64) ** 2))
        assert np.max(np.abs(a - b)) < 1e-5 * max(rms, 1.0)


def _attn_f64(q, kd, vd, slots, lo, hi, H, KVH, QK, VD):
    """Textbook softmax attention in float64 over dequantised K/V."""
    rep = H // KVH
    out = np.zeros((H, VD))
    pos = np.arange(lo, hi + 1) % slots
    K = kd.reshape(slots, KVH, QK).astype(np.float64)
    Vv = vd.reshape(slots, KVH, VD).astype(np.float64)
    for h in range(H):
        s = K[pos, h // rep] @ q.reshape(H, QK)[h].astype(np.float64) / np.sqrt(QK)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ Vv[pos, h // rep]
    return out.reshape(-1)


@pytest.mark.parametrize("H,KVH,QK,VD", [(12, 2, 48, 64), (12, 12, 64, 64), (4, 1, 16, 32)])
def test_attend_step_i8_vs_textbook(H, KVH, QK, VD):
    rng = np.random.default_rng(H * 100 + QK)
    slots = 300
    k = rng.normal(size=slots * KVH * QK).astype(np.float32)
    v = rng.normal(size=slots * KVH * VD).astype(np.float32)
    q = rng.normal(size=H * QK).astype(np.float32)
    kq, ks = O.quantize_rows(k, QK)
    vq, vs = O.quantize_rows(v, VD)
    kd = (kq.reshape(-1, QK).astype(np.float64) * ks[:, None]).reshape(-1)
    vd = (vq.reshape(-1, VD).astype(np.float64) * vs[:, None]).reshape(-1)
    for lo, hi in [(0, 0), (0, 299), (250, 420), (37, 100)]:
        got = O.attend_step_i8(q, kq, ks, vq, vs, slots, lo, hi, H, KVH, QK, VD)
        want = _attn_f64(q, kd, vd, slots, lo, hi, H, KVH, QK, VD)
        assert np.max(np.abs(got - want)) < 2e-6


def test_prefill_equals_stepping_in_oracle():
    """v3_kv_int8.rs:269-282: attend over the stored ints equals attend_step
    at every t, bit for bit (same arithmetic order)."""
    rng = np.random.default_rng(9)
    H, KVH, QK, VD, seq, win = 12, 2, 48, 64, 40, 16
    q = rng.normal(size=seq * H * QK).astype(np.float32)
    k = rng.normal(size=seq * KVH * QK).astype(np.float32)
    v = rng.normal(size=seq * KVH * VD).astype(np.float32)
    kq, ks = O.quantize_rows(k, QK)
    vq, vs = O.quantize_rows(v, VD)
    full = O.attend_i8(q, kq, ks, vq, vs, seq, H, KVH, QK, VD, window=win).reshape(seq, -1)
    ring = O.Ring(True, KVH, QK, VD, hint=4, window=win, max_seq_len=64)
    for t in range(seq):
        ring.write_kv(t, k[t * KVH * QK:(t + 1) * KVH * QK], v[t * KVH * VD:(t + 1) * KVH * VD])
        lo, hi = ring.span(t)
        step = ring.attend_step(q[t * H * QK:(t + 1) * H * QK], lo, hi, H)
        assert np.array_equal(step, full[t]), t
