"""The oracle's Needle-3 forward helpers, pinned.

Each helper of needle_oracle_v3.c is checked against the known-answer tests
the reference ships for it (engram.rs:139-172, mhc.rs:160-238,
v3/kernels.rs:194-226, cache.rs:814-870) and against what the mathematics
fixes, computed independently in float64 (a dense Kronecker product, a
sequence convolution, a rotation's norm, Sinkhorn's doubly-stochastic
limit).  The whole decode step has no reference output to compare with
offline; it is checked for self-consistency here, and is the bit-for-bit
checker of the device forward in test_gpu_v3.py.
"""
import math

import numpy as np
import pytest

import oracle as O
import v3_synth as S


def _sig(x):
    return 1.0 / (1.0 + np.exp(-np.float64(x)))


# ---- Engram hashing (engram.rs:30-67) --------------------------------------

def test_bigram_depends_on_exactly_two_tokens():
    """engram.rs:139-149."""
    a = O.engram_indices([10, 20, 30], [2], 1, 18432)
    b = O.engram_indices([10, 99, 30], [2], 1, 18432)
    assert a[0] == b[0]
    assert a[1] != b[1] and a[2] != b[2]


def test_tables_differ_by_seed():
    """engram.rs:151-161."""
    idx = O.engram_indices([7, 8, 9], [2, 3], 3, 18432)
    row = idx[2 * 6:3 * 6]
    assert len(set(row.tolist())) > 1


def test_validity_follows_the_order():
    """engram.rs:163-171."""
    orders = [2, 3]
    assert not O.ngram_valid(0, 0, orders, 1)
    assert O.ngram_valid(1, 0, orders, 1)
    assert not O.ngram_valid(1, 1, orders, 1)
    assert O.ngram_valid(2, 1, orders, 1)


def test_hash_uses_only_the_order_window():
    """An order-k hash at position p is a function of tokens p-k+1..p (zero
    before the start): changing any other token leaves it alone."""
    rng = np.random.default_rng(0)
    toks = rng.integers(3, 8192, 12).astype(np.uint32)
    base = O.engram_indices(toks, [2, 3], 3, 18432).reshape(12, 6)
    for p in range(12):
        for k, order in enumerate([2, 3]):
            other = toks.copy()
            far = [q for q in range(12) if q > p or q < p - order + 1]
            other[far] = (other[far] + 1000) % 8192
            got = O.engram_indices(other, [2, 3], 3, 18432).reshape(12, 6)
            assert np.array_equal(got[p, 3 * k:3 * k + 3], base[p, 3 * k:3 * k + 3])


# ---- mHC (mhc.rs) -----------------------------------------------------------

def test_offsets_single_out_the_active_lane():
    """mhc.rs:160-167 through mix_down: layer 5 of 4 lanes is lane 1."""
    lanes = np.eye(4, dtype=np.float32)
    gates, _ = O.mix_down(lanes, np.zeros(4), 0.0, np.zeros(4), 5)
    want = np.float32([_sig(-4), _sig(4), _sig(-4), _sig(-4)])
    assert np.allclose(gates, want, atol=1e-7)


def test_mix_down_is_a_gated_lane_sum():
    """mhc.rs:169-193."""
    lanes = np.float32([[1.0, 2.0], [10.0, 20.0]])
    _, u = O.mix_down(lanes, np.zeros(2), 0.0, np.zeros(2), 0)
    hi, lo = _sig(4.0), _sig(-4.0)
    assert abs(u[0] - (hi * 1.0 + lo * 10.0)) < 1e-6
    assert abs(u[1] - (hi * 2.0 + lo * 20.0)) < 1e-6


def test_scatter_rows_stay_doubly_stochastic():
    """mhc.rs:195-238: y drowned by b_post = -100, mass preserved."""
    lanes = np.float32([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]])
    out, post, res = O.scatter_up(lanes, np.zeros(3), np.full(9, 0.3), [7.0, 8.0], 1.0,
                                  np.full(3, -100.0), 1.0, np.zeros(9), 0)
    assert abs(out.sum() - lanes.sum()) < 1e-3
    assert np.allclose(res.sum(0), 1.0, atol=1e-5) and np.allclose(res.sum(1), 1.0, atol=1e-5)


def test_scatter_up_formula():
    """Random gates: lanes' = H_res . lanes + H_post y, with H_post =
    2 sigmoid(a x + b + off) and H_res the Sinkhorn of a x + b."""
    rng = np.random.default_rng(1)
    n, d, layer = 4, 8, 6
    lanes = rng.normal(size=(n, d)).astype(np.float32)
    post_raw = rng.normal(size=n).astype(np.float32)
    res_raw = rng.normal(size=n * n).astype(np.float32)
    y = rng.normal(size=d).astype(np.float32)
    b_post = rng.normal(size=n).astype(np.float32)
    b_res = rng.normal(size=n * n).astype(np.float32)
    out, post, res = O.scatter_up(lanes, post_raw, res_raw, y, 0.7, b_post, 0.4, b_res, layer)
    off = np.where(np.arange(n) == layer % n, 0.0, -4.0)
    want_post = 2.0 * _sig(0.7 * post_raw.astype(np.float64) + b_post + off)
    assert np.allclose(post, want_post, rtol=1e-6)
    want_res = O.sinkhorn(0.4 * res_raw + b_res)
    assert np.allclose(res, want_res, atol=1e-7)
    want = res.astype(np.float64) @ lanes + np.outer(post, y)
    assert np.allclose(out, want, atol=1e-5)


def test_sinkhorn_is_the_log_domain_iteration():
    """kernels.rs:48-74 against a float64 log-domain Sinkhorn (20 rounds)."""
    rng = np.random.default_rng(2)
    for n in (2, 3, 4, 6):
        m = rng.normal(size=(n, n)).astype(np.float32) * 2
        got = O.sinkhorn(m)
        x = m.astype(np.float64)
        for _ in range(20):
            x = x - np.log(np.exp(x - x.max(1, keepdims=True)).sum(1, keepdims=True)) - x.max(1, keepdims=True)
            x = x - np.log(np.exp(x - x.max(0, keepdims=True)).sum(0, keepdims=True)) - x.max(0, keepdims=True)
        assert np.allclose(got, np.exp(x), atol=2e-6)
        assert np.allclose(got.sum(0), 1.0, atol=1e-5)


# ---- HadamardMLP (v3/kernels.rs) -------------------------------------------

def test_block_sizes_match_upstream():
    """kernels.rs:194-199."""
    assert O.hada_blocks(1024) == (32, 32)
    assert O.hada_blocks(512) == (16, 32)
    assert O.hada_blocks(256) == (16, 16)


def test_kron_matches_a_transpose_z_b():
    """kernels.rs:201-216, worked by hand, and random blocks in float64."""
    out = O.kron_apply(np.float32([1, 2, 3, 4]), np.float32([[1, 2], [3, 4]]),
                       np.float32([[0, 1], [1, 0]]))
    assert np.array_equal(out.reshape(-1), np.float32([14, 10, 20, 14]))
    rng = np.random.default_rng(3)
    for ba, bb in ((32, 32), (16, 32), (4, 8)):
        z = rng.normal(size=(ba, bb)).astype(np.float32)
        a = rng.normal(size=(ba, ba)).astype(np.float32)
        b = rng.normal(size=(bb, bb)).astype(np.float32)
        a[0, :] = 0.0  # zero factors are skipped, not mis-summed
        got = O.kron_apply(z.reshape(-1), a, b)
        want = a.T.astype(np.float64) @ z @ b
        assert np.allclose(got, want, atol=1e-4)
        # the same map as the dense Kronecker product on the flattened z
        dense = np.kron(a, b).T.astype(np.float64) @ z.reshape(-1)
        assert np.allclose(got.reshape(-1), dense, atol=1e-4)


def test_hadamard_mlp_structure():
    """kernels.rs:119-180 in float64: conditioning softmax, three Kronecker
    stages with the two permutations, silu, output diagonal."""
    rng = np.random.default_rng(4)
    hn, d, r = 256, 96, 5
    ba, bb = O.hada_blocks(hn)
    w = dict(d1=rng.normal(1, 0.1, hn), d2=rng.normal(1, 0.1, hn), b2=rng.normal(-0.5, 0.1, hn),
             d3=rng.normal(0, 1, hn), d4=rng.normal(1, 0.1, hn),
             w1a=rng.normal(size=(ba, ba)), w1b=rng.normal(size=(bb, bb)) / 4,
             w2a=rng.normal(size=(ba, ba)) / 4, w2b=rng.normal(size=(bb, bb)) / 4,
             w3a=rng.normal(size=(ba, ba)) / 4, w3b=rng.normal(size=(bb, bb)) / 4,
             cond_v=rng.normal(size=(d, r)) / 10, cond_u=rng.normal(size=(r, hn)) / 10)
    w = {k: np.asarray(v, np.float32) for k, v in w.items()}
    p1, p2 = rng.permutation(hn).astype(np.uint32), rng.permutation(hn).astype(np.uint32)
    x = rng.normal(size=d).astype(np.float32)
    got = O.hadamard_mlp(x, w, p1, p2, hn)
    f = {k: v.astype(np.float64) for k, v in w.items()}
    proj = x.astype(np.float64) @ f["cond_v"]
    sm = np.exp(proj - proj.max())
    sm /= sm.sum()
    cond = 1.0 + sm @ f["cond_u"]
    z = np.zeros(hn)
    z[:d] = x
    z *= f["d1"]
    kron = lambda z, a, b: (a.T @ z.reshape(ba, bb) @ b).reshape(-1)
    z = kron(z, f["w1a"], f["w1b"])[p1]
    t = f["d2"] * cond * z + f["b2"]
    z = t / (1.0 + np.exp(-t))
    z = kron(z, f["w2a"], f["w2b"])[p2] * f["d3"]
    want = (kron(z, f["w3a"], f["w3b"]) * f["d4"])[:d]
    assert np.allclose(got, want, atol=2e-4 * max(1.0, np.abs(want).max()))


# ---- convolutions (cache.rs:401-482 against attention.rs:82-100 and
# engram.rs:89-106) ----------------------------------------------------------

def test_conv_step_matches_the_sequence_conv():
    """cache.rs:814-841."""
    dim, T, seq = 40, 3, 6
    taps = np.sin(np.arange(T * dim, dtype=np.float32) * np.float32(0.37)).reshape(T, dim)
    raw = np.cos(np.arange(seq * dim, dtype=np.float32) * np.float32(0.11)).reshape(seq, dim)
    want = np.zeros((seq, dim))
    for t in range(seq):
        for j in range(min(T, t + 1)):
            want[t] += taps[j].astype(np.float64) * raw[t - j]
    tail = np.zeros((T - 1, dim), np.float32)
    for t in range(seq):
        out, tail = O.conv_step(tail, taps, raw[t], t)
        assert np.allclose(out, want[t], atol=1e-5), t


def test_engram_conv_step_matches_the_sequence_conv():
    """cache.rs:843-870: 4 taps, dilation 3, max order 3."""
    d, T, dil, mo, seq = 16, 4, 3, 3, 12
    taps = np.cos(np.arange(T * d, dtype=np.float32) * np.float32(0.23)).reshape(T, d)
    raw = np.sin(np.arange(seq * d, dtype=np.float32) * np.float32(0.19)).reshape(seq, d)
    want = np.zeros((seq, d))
    for p in range(seq):
        for j in range(T):
            back = j * dil
            if back > p or p < j * mo:
                continue
            want[p] += taps[j].astype(np.float64) * raw[p - back]
    tail = np.zeros(((T - 1) * dil, d), np.float32)
    for p in range(seq):
        out, tail = O.engram_conv_step(tail, taps, raw[p], dil, mo, p)
        assert np.allclose(out, want[p], atol=1e-5), p


# ---- norm + RoPE (attention.rs:102-150, model.rs:378-394) -----------------

def test_rope_is_a_norm_preserving_rotation():
    g = dict(S.V3_GEOMETRY)
    cfg = g
    hd = g["qk_head_dim"]
    rng = np.random.default_rng(5)
    x = rng.normal(size=(3, hd)).astype(np.float32)
    scale = rng.normal(0, 0.1, hd).astype(np.float32)
    normed = (1.0 + scale.astype(np.float64)) * x / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6)
    cs, sn = O.rope_at(cfg, 0)
    assert np.all(cs == 1.0) and np.all(sn == 0.0)
    assert np.allclose(O.norm_and_rope(x, scale, cs, sn), normed, atol=1e-5)
    for pos in (1, 7, 1000):
        cs, sn = O.rope_at(cfg, pos)
        half = hd // 2
        freq = 1.0 / (g["rope_theta"] ** (np.arange(half) * 2.0 / hd))
        assert np.allclose(cs, np.cos(pos * freq), atol=2e-4) and np.allclose(sn, np.sin(pos * freq), atol=2e-4)
        got = O.norm_and_rope(x, scale, cs, sn)
        assert np.allclose(np.linalg.norm(got, axis=1), np.linalg.norm(normed, axis=1), rtol=1e-5)
        # half-split pairing: (x_i, x_{i+half}) rotates by the angle of i
        c, s = cs.astype(np.float64), sn.astype(np.float64)
        want = np.concatenate([normed[:, :half] * c - normed[:, half:] * s,
                               normed[:, half:] * c + normed[:, :half] * s], axis=1)
        assert np.allclose(got, want, atol=1e-5)


def test_apply_site_gate():
    """engram.rs:108-132: x += sigmoid(<unit(x), unit(k)> / sqrt(d)) v."""
    rng = np.random.default_rng(6)
    d = 64
    x, k, v = (rng.normal(size=d).astype(np.float32) for _ in range(3))
    got = O.apply_site(x, k, v)
    f = lambda z: z.astype(np.float64) / np.sqrt((z.astype(np.float64) ** 2).mean() + 1e-6)
    alpha = _sig(np.dot(f(x), f(k)) / math.sqrt(d))
    assert np.allclose(got, x + alpha * v, atol=1e-6)


# ---- the whole decode step ---------------------------------------------------

@pytest.fixture(scope="module")
def small():
    g, recs = S.build_records(S.small_geometry(2), seed=3)
    return g, O.V3Model(g, recs, S.CODEBOOK)


def test_decode_is_deterministic_and_cache_local(small):
    """Two caches fed the same tokens give identical logits; a cache fed
    other tokens differs (the cache, not the model, holds the state)."""
    g, om = small
    prompt = S.prompt_tokens(40, 8)
    a, b, c = om.new_cache(64, True), om.new_cache(64, True), om.new_cache(64, True)
    for i, t in enumerate(prompt):
        la, lb = a.decode_step(t), b.decode_step(t)
        lc = c.decode_step((int(t) + 1) % g["vocab_size"] if i == 0 else t)
        assert np.array_equal(la, lb)
    assert not np.array_equal(la, lc)


def test_int8_cache_stays_close_to_f32(small):
    """The int8 KV cache is a small perturbation of the f32 forward (the
    reference's own quality gate is the int8 parity of v3_kv_int8.rs)."""
    g, om = small
    prompt = S.prompt_tokens(48, 9)
    q, f = om.new_cache(64, True), om.new_cache(64, False)
    for t in prompt:
        lq, lf = q.decode_step(t), f.decode_step(t)
    rel = np.abs(lq - lf).max() / np.abs(lf).max()
    assert 0.0 < rel < 0.05, rel


def test_ring_wrap_equals_a_long_ring(small):
    """Local layers see the last `window` positions whether the ring is
    window-sized (wrapping) or holds everything: hint only sizes storage."""
    g, om = small
    prompt = S.prompt_tokens(80, 10)  # > sliding window 32
    a, b = om.new_cache(1, True), om.new_cache(128, True)
    for t in prompt:
        la, lb = a.decode_step(t), b.decode_step(t)
        assert np.array_equal(la, lb)
