"""The device Needle-3 forward with f32 KV caches (KvPrecision::F32, the
default of needle_v3_run and needle_v3_generate(kv_int8 = false),
crates/needle-c/src/v3.rs:219-250) vs the oracle's, and vs the reference's
own numpy transcription of the forward.

With an f32 cache, write_kv stores the keys and values as they are
(cache.rs:359-362), the query is not fake-quantised (v3/model.rs:289-293)
and attention reads the f32 view (attention.rs:166-189).  The device sums
in the reference's order, so the logits equal the oracle's bit for bit at
every step, and greedy tokens are identical.
"""
import os

import numpy as np
import pytest
import torch

import cact_writer as W
import needle_amd as nd
import oracle as O
import v3_synth as S

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "v3_forward_reference.npz")


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def small(ctx):
    g, recs = S.build_records(S.small_geometry(4), seed=11)
    return g, recs, O.V3Model(g, recs, S.CODEBOOK), nd.V3Model(ctx, g, recs, S.CODEBOOK)


def _oracle_logits(om, prompt):
    cache = om.new_cache(len(prompt), False)
    return np.stack([cache.decode_step(t) for t in prompt])


def test_f32_logits_track_the_oracle(small):
    """4 layers, window 32 (the local rings wrap), Engram on layers 1 and 3,
    48 positions: every logit of every step bit-identical."""
    g, recs, om, dm = small
    prompt = S.prompt_tokens(48, 3)
    want = _oracle_logits(om, prompt)
    batch = nd.V3Batch(dm, 1, max_len=64, kv_int8=False)
    got = torch.empty(1, dm.rows, device="cuda")
    for t, tok in enumerate(prompt):
        batch.step([tok], logits=got, want_next=False)
        assert np.array_equal(_bits(got.cpu().numpy()[0]), _bits(want[t])), t
    batch.close()


def test_f32_and_int8_caches_differ(small):
    """The two precisions are different computations (the int8 cache rounds
    K/V and the query): the f32 batch must not be reading an int8 cache."""
    g, recs, om, dm = small
    prompt = S.prompt_tokens(8, 9)
    a = nd.V3Batch(dm, 1, max_len=16, kv_int8=False)
    b = nd.V3Batch(dm, 1, max_len=16, kv_int8=True)
    la = torch.empty(1, dm.rows, device="cuda")
    lb = torch.empty(1, dm.rows, device="cuda")
    for tok in prompt:
        a.step([tok], logits=la, want_next=False)
        b.step([tok], logits=lb, want_next=False)
    want_b = om.new_cache(16, True)
    for tok in prompt:
        wb = want_b.decode_step(tok)
    assert np.array_equal(_bits(lb.cpu().numpy()[0]), _bits(wb))
    assert not np.array_equal(_bits(la.cpu().numpy()[0]), _bits(lb.cpu().numpy()[0]))


def test_f32_sessions_are_independent(small):
    """Three sessions stepped in one batch each equal their own oracle run."""
    g, recs, om, dm = small
    prompts = np.stack([S.prompt_tokens(20, 100 + i) for i in range(3)])
    batch = nd.V3Batch(dm, 3, max_len=32, kv_int8=False)
    got = torch.empty(3, dm.rows, device="cuda")
    outs = []
    for t in range(prompts.shape[1]):
        batch.step(prompts[:, t], logits=got, want_next=False)
        outs.append(got.cpu().numpy().copy())
    outs = np.stack(outs, axis=1)
    for i in range(3):
        assert np.array_equal(_bits(outs[i]), _bits(_oracle_logits(om, prompts[i]))), i


@pytest.mark.parametrize("chunks", [[40], [7, 33], [16, 16, 8], [1, 31, 8]])
def test_f32_prefill_chunks_equal_stepping(small, chunks):
    """Chunked prefill with f32 caches: each pass's last logits, then every
    logit of 8 greedy steps after it, equal the oracle's stepping (the local
    rings are widened by max_chunk - 1 as for int8)."""
    g, recs, om, dm = small
    n = sum(chunks)
    prompt = S.prompt_tokens(n, 41)
    want = _oracle_logits(om, prompt)
    batch = nd.V3Batch(dm, 1, max_len=n + 8, max_chunk=max(chunks), kv_int8=False)
    lg = torch.empty(1, dm.rows, device="cuda")
    t = 0
    nxt = None
    for c in chunks:
        nxt = batch.prefill(prompt[None, t:t + c], logits=lg)
        t += c
        assert np.array_equal(_bits(lg.cpu().numpy()[0]), _bits(want[t - 1])), t
    cache = om.new_cache(n + 8, False)
    for tok in prompt:
        cache.decode_step(tok)
    for s in range(8):
        w = cache.decode_step(int(nxt[0]))
        nxt = batch.step(nxt, logits=lg)
        assert np.array_equal(_bits(lg.cpu().numpy()[0]), _bits(w)), s
    batch.close()


def test_f32_greedy_matches_oracle_small(small):
    g, recs, om, dm = small
    prompt = S.prompt_tokens(16, 5)
    toks, margins = O.v3_generate(om, prompt, 48, int8=False)
    batch = nd.V3Batch(dm, 1, max_len=64, kv_int8=False)
    got = batch.generate(prompt[None], 48)[0]
    print(f"min top-1/top-2 margin {margins.min():.4e}; distinct tokens {len(set(toks.tolist()))}")
    assert np.array_equal(got, toks.astype(np.int32))


def test_f32_forward_matches_the_reference_transcription(ctx):
    """The device forward with an f32 cache against the logits the
    reference's numpy transcription of the forward produced
    (tests/golden/v3_forward_reference.npz: 4 layers at the shipped widths, a
    global layer, Engram, a 32-position window, 40 tokens): the last two
    positions within 2e-5 of the logit scale, the top-16 logits of every
    position likewise, and the greedy token at every position identical."""
    f = np.load(FIXTURE)
    g, recs = S.build_records(S.small_geometry(int(f["geometry_layers"])), seed=int(f["model_seed"]))
    _, held = W.pack_synth(g, recs, S.CODEBOOK)
    dm = nd.V3Model(ctx, g, held, S.CODEBOOK)
    prompt = f["prompt"]
    batch = nd.V3Batch(dm, 1, max_len=64, kv_int8=False)
    lg = torch.empty(1, dm.rows, device="cuda")
    logits = []
    for tok in prompt:
        batch.step([int(tok)], logits=lg, want_next=False)
        logits.append(lg.cpu().numpy()[0].copy())
    logits = np.stack(logits)
    ref = f["last_logits"]
    assert np.abs(logits[-2:] - ref).max() <= 2e-5 * np.abs(ref).max()
    top_ids, top_vals = f["top_ids"], f["top_vals"]
    ours = np.take_along_axis(logits, top_ids, axis=1)
    assert np.abs(ours - top_vals).max() <= 2e-5 * np.abs(top_vals).max()
    assert np.array_equal(logits.argmax(axis=1), top_ids[:, 0])
    batch.close()
    dm.close()


def test_f32_shipped_geometry_greedy(ctx):
    """The shipped geometry (20 layers), a 128-token prompt prefilled in
    32-position passes, then 64 greedy steps with f32 caches: tokens
    identical to the oracle's stepping."""
    g, recs = S.build_records(None, seed=0)
    om = O.V3Model(g, recs, S.CODEBOOK)
    dm = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    prompt = S.prompt_tokens(128, 6)
    toks, margins = O.v3_generate(om, prompt, 64, int8=False)
    batch = nd.V3Batch(dm, 1, max_len=128 + 64, max_chunk=32, kv_int8=False)
    got = batch.generate(prompt[None], 64)[0]
    print(f"shipped geometry, f32 KV: min margin {margins.min():.4e}, "
          f"distinct {len(set(toks.tolist()))}")
    assert np.array_equal(got, toks.astype(np.int32))
    batch.close()
    dm.close()
