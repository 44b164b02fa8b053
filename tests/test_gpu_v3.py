"""The device Needle-3 forward (decode_step, int8 KV) vs the oracle's.

Same canonical records (random init, v3_synth) on both sides.  The device
forward sums in the reference's order (reference-order projections and
attention, sequential norm chains, libm's exp/log), so the logits match the
oracle's bit for bit at every step -- the only bar under which an int8 KV
cache cannot drift (a last-bit difference upstream of the quantiser can flip
a cached code) -- and greedy tokens are identical (first maximum wins), with
the top-1/top-2 margins reported.
"""
import numpy as np
import pytest
import torch

import needle_amd as nd
import oracle as O
import v3_synth as S

pytestmark = pytest.mark.gpu



def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def small(ctx):
    g, recs = S.build_records(S.small_geometry(4), seed=11)
    return g, recs, O.V3Model(g, recs, S.CODEBOOK), nd.V3Model(ctx, g, recs, S.CODEBOOK)


def _oracle_logits(om, prompt, int8=True):
    cache = om.new_cache(len(prompt), int8)
    return np.stack([cache.decode_step(t) for t in prompt])


def test_small_model_logits_track_the_oracle(small):
    """4 layers, window 32 (the local rings wrap), Engram on layers 1 and 3."""
    g, recs, om, dm = small
    prompt = S.prompt_tokens(48, 3)
    want = _oracle_logits(om, prompt)
    batch = nd.V3Batch(dm, 1, max_len=64)
    got = torch.empty(1, dm.rows, device="cuda")
    errs, first_bad = [], -1
    for t, tok in enumerate(prompt):
        batch.step([tok], logits=got, want_next=False)
        g = got.cpu().numpy()[0]
        errs.append(float(np.max(np.abs(g - want[t]))))
        if first_bad < 0 and not np.array_equal(_bits(g), _bits(want[t])):
            first_bad = t
    print(f"max-abs logit error per step: max {max(errs):.3e}, logit scale {np.abs(want).max():.3e}, "
          f"first step with a differing bit {first_bad}")
    assert first_bad == -1, errs
    assert list(batch.positions()) == [48]


def test_sessions_are_independent(small):
    """Three sessions stepped in one batch (M = 3 projections) each equal
    their own oracle run."""
    g, recs, om, dm = small
    prompts = np.stack([S.prompt_tokens(20, 100 + i) for i in range(3)])
    batch = nd.V3Batch(dm, 3, max_len=32)
    got = torch.empty(3, dm.rows, device="cuda")
    outs = []
    for t in range(prompts.shape[1]):
        batch.step(prompts[:, t], logits=got, want_next=False)
        outs.append(got.cpu().numpy().copy())
    outs = np.stack(outs, axis=1)
    for i in range(3):
        want = _oracle_logits(om, prompts[i])
        assert np.array_equal(_bits(outs[i]), _bits(want)), (i, np.max(np.abs(outs[i] - want)))


def test_greedy_matches_oracle_small(small):
    g, recs, om, dm = small
    prompt = S.prompt_tokens(16, 5)
    toks, margins = O.v3_generate(om, prompt, 48)
    batch = nd.V3Batch(dm, 1, max_len=64)
    got = batch.generate(prompt[None], 48)[0]
    print(f"min top-1/top-2 margin {margins.min():.4e}; distinct tokens {len(set(toks.tolist()))}")
    assert np.array_equal(got, toks.astype(np.int32))


def test_zero_kronecker_factors_are_skipped(ctx):
    """kron_apply skips zero factors (v3/kernels.rs:41-81): layer 0's w1a
    gets an all-zero column (so a row of the intermediate is exactly zero
    too, taking the second pass's skip as well) and a -0.0 entry; layer 1's
    w2a a single zero.  Logits stay bit-identical to the oracle's."""
    g, recs = S.build_records(S.small_geometry(4), seed=19)
    recs = [dict(r) for r in recs]
    for r in recs:
        if r["name"] == "l0.w1a":
            a = np.array(r["data"], np.float32).reshape(32, 32)
            a[:, 3] = 0.0
            a[5, 7] = -0.0
            r["data"] = a
        elif r["name"] == "l1.w2a":
            a = np.array(r["data"], np.float32).reshape(32, 32)
            a[9, 2] = 0.0
            r["data"] = a
    om, dm = O.V3Model(g, recs, S.CODEBOOK), nd.V3Model(ctx, g, recs, S.CODEBOOK)
    prompt = S.prompt_tokens(12, 21)
    want = _oracle_logits(om, prompt)
    batch = nd.V3Batch(dm, 1, max_len=16)
    lg = torch.empty(1, dm.rows, device="cuda")
    for t, tok in enumerate(prompt):
        batch.step([tok], logits=lg, want_next=False)
        assert np.array_equal(_bits(lg.cpu().numpy()[0]), _bits(want[t])), t
    batch.close()


def test_graph_replay_equals_eager_steps(small):
    """With graphs on, single-position steps replay one captured HIP graph
    from the second step on; the default enqueues every kernel.  Both track
    the oracle bit for bit over 24 steps, replay after replay, with eager
    work (a logits copy, a token round trip) between the replays."""
    g, recs, om, dm = small
    prompt = S.prompt_tokens(24, 27)
    want = _oracle_logits(om, prompt)
    a, e = nd.V3Batch(dm, 1, max_len=32), nd.V3Batch(dm, 1, max_len=32)
    a.set_graphs(True)
    la = torch.empty(1, dm.rows, device="cuda")
    le = torch.empty(1, dm.rows, device="cuda")
    for t, tok in enumerate(prompt):
        na = a.step([tok], logits=la)
        ne = e.step([tok], logits=le)
        got_a, got_e = la.cpu().numpy()[0], le.cpu().numpy()[0]
        assert np.array_equal(_bits(got_a), _bits(got_e)), t
        assert np.array_equal(_bits(got_a), _bits(want[t])), t
        assert list(na) == list(ne) == [int(np.argmax(want[t]))]
    a.close()
    e.close()


def test_graph_replay_after_chunked_prefill(small):
    """Prefill passes stay eager; the single-position steps after them are
    captured and replayed, and match a batch stepped eagerly throughout."""
    g, recs, om, dm = small
    prompt = S.prompt_tokens(20, 31)
    a = nd.V3Batch(dm, 2, max_len=48, max_chunk=8)
    e = nd.V3Batch(dm, 2, max_len=48, max_chunk=8)
    a.set_graphs(True)
    toks = np.stack([prompt, prompt[::-1]]).astype(np.int32)
    na = ne = None
    for t in range(0, 16, 8):
        na = a.prefill(toks[:, t:t + 8])
        ne = e.prefill(toks[:, t:t + 8])
    assert list(na) == list(ne)
    la = torch.empty(2, dm.rows, device="cuda")
    le = torch.empty(2, dm.rows, device="cuda")
    for s in range(12):
        na = a.step(na, logits=la)
        ne = e.step(ne, logits=le)
        assert np.array_equal(_bits(la.cpu().numpy()), _bits(le.cpu().numpy())), s
        assert list(na) == list(ne)
    a.close()
    e.close()


def test_model_rejects_a_wrong_record(ctx):
    g, recs = S.build_records(S.small_geometry(2), seed=1)
    bad = list(recs)
    bad[2] = dict(bad[2], out=bad[2]["out"] + 1)  # q_proj with the wrong row count
    with pytest.raises(nd.NeedleError) as e:
        nd.V3Model(ctx, g, bad, S.CODEBOOK)
    assert "q_proj" in str(e.value)
    with pytest.raises(nd.NeedleError):
        nd.V3Model(ctx, g, recs[:-1], S.CODEBOOK)


def test_shipped_geometry_prompt128_greedy256(ctx):
    """The shipped v3 geometry (20 layers, ~121M params), a 128-token
    uniform prompt, 256 greedy steps, int8 KV: tokens identical."""
    g, recs = S.build_records(None, seed=0)
    om = O.V3Model(g, recs, S.CODEBOOK)
    dm = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    prompt = S.prompt_tokens(128, 4)
    toks, margins = O.v3_generate(om, prompt, 256)
    batch = nd.V3Batch(dm, 1, max_len=128 + 256)
    got = batch.generate(prompt[None], 256)[0]
    first_diff = int(np.argmax(got != toks)) if not np.array_equal(got, toks) else -1
    print(f"shipped geometry: min margin {margins.min():.4e}, median {np.median(margins):.4e}, "
          f"distinct {len(set(toks.tolist()))}, first difference at {first_diff}")
    assert np.array_equal(got, toks.astype(np.int32)), first_diff


@pytest.mark.parametrize("taps", [0, 1, 2, 4, 5])
def test_conv_taps_track_the_oracle(ctx, taps):
    """The q/k/v causal conv at other tap counts than the shipped 3: a
    decode step holds a thread's conv operands in registers up to 4 taps
    and loops over them beyond; 0 taps has no conv.  Two sessions stepped
    past the taps' reach, every logit bit for bit the oracle's."""
    geo = S.small_geometry(2)
    geo["qkv_conv_taps"] = taps
    g, recs = S.build_records(geo, seed=21 + taps)
    om = O.V3Model(g, recs, S.CODEBOOK)
    dm = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    prompts = np.stack([S.prompt_tokens(12, 200 + 3 * taps + i) for i in range(2)])
    batch = nd.V3Batch(dm, 2, max_len=16)
    got = torch.empty(2, dm.rows, device="cuda")
    outs = []
    for t in range(prompts.shape[1]):
        batch.step(prompts[:, t], logits=got, want_next=False)
        outs.append(got.cpu().numpy().copy())
    outs = np.stack(outs, axis=1)
    for i in range(2):
        want = _oracle_logits(om, prompts[i])
        assert np.array_equal(_bits(outs[i]), _bits(want)), (taps, i, np.max(np.abs(outs[i] - want)))
    batch.close()
    dm.close()


@pytest.mark.parametrize("qk", [16, 32, 64])
def test_head_dims_track_the_oracle(ctx, qk):
    """q/k head widths other than the shipped 48: a decode step forms each
    query head and its kv head's k and v inside the attention launch, with
    the head read in qk / 16 pieces of 16 codes (1, 2 and 4 here).  Two
    sessions stepped past the sliding window, every logit bit for bit the
    oracle's."""
    geo = S.small_geometry(2)
    geo["qk_head_dim"] = qk
    g, recs = S.build_records(geo, seed=31 + qk)
    om = O.V3Model(g, recs, S.CODEBOOK)
    dm = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    prompts = np.stack([S.prompt_tokens(40, 300 + qk + i) for i in range(2)])
    batch = nd.V3Batch(dm, 2, max_len=48)
    got = torch.empty(2, dm.rows, device="cuda")
    outs = []
    for t in range(prompts.shape[1]):
        batch.step(prompts[:, t], logits=got, want_next=False)
        outs.append(got.cpu().numpy().copy())
    outs = np.stack(outs, axis=1)
    for i in range(2):
        want = _oracle_logits(om, prompts[i])
        assert np.array_equal(_bits(outs[i]), _bits(want)), (qk, i, np.max(np.abs(outs[i] - want)))
    batch.close()
    dm.close()


def test_greedy_ties_take_the_first_index(ctx):
    """Greedy ties go to the first index.  With the tied embedding's upper
    half a copy of its lower half every logit appears twice (rows computed
    by different workgroups, bit-identical), so every step is a tie: the
    tokens must be the oracle's first-maximum choices, all in the lower
    half."""
    g, recs = S.build_records(S.small_geometry(2), seed=41)
    emb = next(r for r in recs if r["name"] == "embedding")
    V, pad = emb["out"], -(-emb["inn"] // emb["group"]) * emb["group"]
    row_bytes, G = pad * emb["bits"] // 8, pad // emb["group"]
    blob = emb["data"].copy()
    codes = blob[:V * row_bytes].reshape(V, row_bytes)
    norms = blob[V * row_bytes:].view(np.uint16).reshape(V, G)
    codes[V // 2:] = codes[:V // 2]
    norms[V // 2:] = norms[:V // 2]
    emb["data"] = blob
    om = O.V3Model(g, recs, S.CODEBOOK)
    dm = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    prompt = S.prompt_tokens(12, 9)
    toks, _ = O.v3_generate(om, prompt, 24)
    batch = nd.V3Batch(dm, 2, max_len=48)
    got = batch.generate(np.stack([prompt, prompt]), 24)
    assert np.array_equal(got[0], toks.astype(np.int32)) and np.array_equal(got[1], got[0])
    assert int(got.max()) < V // 2
    batch.close()
    dm.close()
