"""Random-init Needle-3 weights as canonical container records.

The record order is the one V3Layout::derive walks
(crates/needle-infer/src/v3.rs:236-330): embedding; per layer norm_in,
q/k/v_proj, q/k/v conv taps, q_norm, k_norm, gate_proj, out_proj, post_norm,
attn_gate, pre_hada and the 13 HadamardMLP tensors; the six mHC scalars, the
three mHC projections, the two Hadamard permutations; per Engram site its
tables, key/value projections and taps; final_norm.  Cactus-Quants records
carry a blob exactly as a .cact file stores it (packed LSB-first codes, then
FP16 norms per (row, 128-group), cq.rs:181-238).

Scales are chosen so activations stay O(1) through the stack and greedy
decoding at random init is not degenerate: with the head tied to the
embedding, an embedding as large as the block updates makes every step
repeat the current token, so the embedding is drawn 30x smaller; and
HadamardMLP's silu input is centred (b2 ~ -0.5, where silu's mean over
N(b, 1) crosses zero) with random signs on d3, so the layers do not all push
one fixed direction.  The values are synthetic (no checkpoint is available
offline).
"""
from __future__ import annotations

import math

import numpy as np

# The shipped geometry (needle3.cact header, crates/needle-core/src/v3/config.rs:188-216).
V3_GEOMETRY = dict(
    vocab_size=8192, out_vocab=8192, d_model=768, num_heads=12, num_kv_heads=2, num_layers=20,
    qk_head_dim=48, v_head_dim=64, max_seq_len=8192, hada_n=1024, mhc_lanes=4,
    rope_theta=100000.0, sliding_window=1024, global_layers=[4, 9, 14, 19], qkv_conv_taps=3,
    orders=[2, 3], e_heads=3, e_slots=18432, e_sub_dim=128, sites=[3, 7, 11, 15, 19],
    e_conv_taps=4, e_conv_dilation=3, e_seed_heads=0,
)

# The 28-float cb2|cb3|cb4 Lloyd-Max header codebook (already scaled by
# 1/sqrt(128)), as the needle-rs fixtures record it (tests/cact_vectors.json).
CODEBOOK = np.array([
    -0.1331721395254135, -0.03990209102630615, 0.04003528133034706, 0.13346044719219208,
    -0.18926136195659637, -0.11788499355316162, -0.06614968925714493, -0.02101346105337143,
    0.022101031616330147, 0.06678506731987, 0.11826207488775253, 0.18982602655887604,
    -0.23953154683113098, -0.18070605397224426, -0.14095793664455414, -0.10901255160570145,
    -0.08151296526193619, -0.056527651846408844, -0.03293915092945099, -0.010116109624505043,
    0.012710800394415855, 0.03570791706442833, 0.059458255767822266, 0.08497702330350876,
    0.112741619348526, 0.1446969211101532, 0.184239000082016, 0.2422737032175064], np.float32)

REC_F32, REC_CQ = 1, 3


def small_geometry(num_layers=4):
    """The shipped widths with fewer layers: global layer last, Engram on
    layers 1 and 3, a short sliding window so rings wrap in short tests."""
    g = dict(V3_GEOMETRY)
    g.update(num_layers=num_layers, global_layers=[num_layers - 1], sites=[1, num_layers - 1],
             sliding_window=32, max_seq_len=1024)
    return g


def _f32(name, arr):
    arr = np.ascontiguousarray(arr, np.float32)
    return dict(kind=REC_F32, name=name, data=arr, out=arr.shape[0] if arr.ndim else 1,
                inn=arr.shape[1] if arr.ndim > 1 else (arr.size if arr.ndim == 0 else 1),
                group=0, bits=0)


def _cq(rng, name, out, inn, bits, std, group=128):
    """A CQ blob whose reconstruction has roughly N(0, std^2) entries."""
    pad = -(-inn // group) * group
    row_bytes = pad * bits // 8
    packed = rng.integers(0, 256, size=out * row_bytes, dtype=np.uint8)
    norms = np.abs(rng.normal(1.0, 0.1, size=out * (pad // group))) * std * math.sqrt(group)
    n16 = norms.astype(np.float16).view(np.uint16)
    blob = np.concatenate([packed, n16.view(np.uint8)])
    return dict(kind=REC_CQ, name=name, data=blob, out=out, inn=inn, group=group, bits=bits)


def build_records(geom=None, seed=0):
    g = dict(V3_GEOMETRY if geom is None else geom)
    rng = np.random.default_rng(seed)
    d, L, n = g["d_model"], g["num_layers"], g["mhc_lanes"]
    qd = g["num_heads"] * g["qk_head_dim"]
    kd = g["num_kv_heads"] * g["qk_head_dim"]
    vd = g["num_kv_heads"] * g["v_head_dim"]
    od = g["num_heads"] * g["v_head_dim"]
    T, hn = g["qkv_conv_taps"], g["hada_n"]
    bits = hn.bit_length() - 1
    ba = 1 << (bits // 2)
    bb = hn // ba
    walsh = lambda m: (lambda h: h / math.sqrt(m))(_sylvester(m))
    recs = [_cq(rng, "embedding", g["vocab_size"], d, 4, 1.0 / (30.0 * math.sqrt(d)))]
    for li in range(L):
        recs.append(_f32(f"l{li}.norm_in", rng.normal(0, 0.1, d)))
        recs.append(_cq(rng, f"l{li}.q_proj", qd, d, 2, 1.0 / math.sqrt(d)))
        recs.append(_cq(rng, f"l{li}.k_proj", kd, d, 2, 1.0 / math.sqrt(d)))
        recs.append(_cq(rng, f"l{li}.v_proj", vd, d, 2, 1.0 / math.sqrt(d)))
        if T > 0:
            for nm, dim in (("q", qd), ("k", kd), ("v", vd)):
                taps = rng.normal(0, 0.3, (T, dim))
                taps[0] += 1.0
                recs.append(_f32(f"l{li}.{nm}_taps", taps))
        recs.append(_f32(f"l{li}.q_norm", rng.normal(0, 0.1, g["qk_head_dim"])))
        recs.append(_f32(f"l{li}.k_norm", rng.normal(0, 0.1, g["qk_head_dim"])))
        recs.append(_cq(rng, f"l{li}.gate_proj", od, d, 2, 1.0 / math.sqrt(d)))
        recs.append(_cq(rng, f"l{li}.out_proj", d, od, 2, 1.0 / math.sqrt(od)))
        recs.append(_f32(f"l{li}.post_norm", rng.normal(0, 0.1, d)))
        recs.append(_f32(f"l{li}.attn_gate", rng.normal(0, 1.0, (1,))))
        recs.append(_f32(f"l{li}.pre_hada", rng.normal(0, 0.1, d)))
        for nm in ("d1", "d2"):
            recs.append(_f32(f"l{li}.{nm}", 1.0 + rng.normal(0, 0.1, hn)))
        recs.append(_f32(f"l{li}.b2", rng.normal(-0.5, 0.1, hn)))
        recs.append(_f32(f"l{li}.d3", (1.0 + rng.normal(0, 0.1, hn)) * rng.choice([-1.0, 1.0], hn)))
        recs.append(_f32(f"l{li}.d4", 1.0 + rng.normal(0, 0.1, hn)))
        for nm in ("w1", "w2", "w3"):
            recs.append(_f32(f"l{li}.{nm}a", walsh(ba) + rng.normal(0, 0.05, (ba, ba))))
            recs.append(_f32(f"l{li}.{nm}b", walsh(bb) + rng.normal(0, 0.05, (bb, bb))))
        recs.append(_f32(f"l{li}.cond_v", rng.normal(0, 1.0 / math.sqrt(d), (d, 8))))
        recs.append(_f32(f"l{li}.cond_u", rng.normal(0, 0.1, (8, hn))))
    recs.append(_f32("a_pre", rng.normal(0.5, 0.1, L)))
    recs.append(_f32("a_post", rng.normal(0.5, 0.1, L)))
    recs.append(_f32("a_res", rng.normal(0.5, 0.1, L)))
    recs.append(_f32("b_pre", rng.normal(0, 0.5, (L, n))))
    recs.append(_f32("b_post", rng.normal(0, 0.5, (L, n))))
    recs.append(_f32("b_res", rng.normal(0, 0.5, (L, n, n)).reshape(L, n * n)))
    recs.append(_cq(rng, "phi_pre", L * n, n * d, 4, 1.0 / math.sqrt(n * d)))
    recs.append(_cq(rng, "phi_post", L * n, n * d, 4, 1.0 / math.sqrt(n * d)))
    recs.append(_cq(rng, "phi_res", L * n * n, n * d, 4, 1.0 / math.sqrt(n * d)))
    recs.append(_f32("hada_perm1", rng.permutation(hn).astype(np.float32)))
    recs.append(_f32("hada_perm2", rng.permutation(hn).astype(np.float32)))
    nt = len(g["orders"]) * g["e_heads"]
    for s in range(len(g["sites"])):
        recs.append(_cq(rng, f"e{s}.tables", nt * g["e_slots"], g["e_sub_dim"], 2, 1.0))
        recs.append(_cq(rng, f"e{s}.key_proj", d, nt * g["e_sub_dim"], 2,
                        1.0 / math.sqrt(nt * g["e_sub_dim"])))
        recs.append(_cq(rng, f"e{s}.value_proj", d, nt * g["e_sub_dim"], 2,
                        1.0 / math.sqrt(nt * g["e_sub_dim"])))
        recs.append(_f32(f"e{s}.taps", rng.normal(0, 0.5, (g["e_conv_taps"], d))))
    recs.append(_f32("final_norm", rng.normal(0, 0.1, d)))
    return g, recs


def _sylvester(m):
    h = np.ones((1, 1))
    while h.shape[0] < m:
        h = np.block([[h, h], [h, -h]])
    return h


def prompt_tokens(n, seed, vocab=8192):
    """Uniform random prompt ids in [3, vocab): PAD/EOS/BOS (0/1/2) excluded."""
    return np.random.default_rng(seed).integers(3, vocab, size=n).astype(np.uint32)
