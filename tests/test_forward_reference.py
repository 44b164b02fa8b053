"""The oracle's whole Needle-3 forward against the reference's own numpy
transcription of it (tools/needle3_reference.py, `Model.forward`), on the
same container.

tests/golden/make_forward_golden.py packs a seeded random-init 4-layer model
at the shipped widths (a global layer, Engram sites, a 32-position sliding
window) into a `.cact` container, runs the transcription over a 40-token
prompt (so the window wraps) and keeps the last two positions' logits and
the top 16 logits of every position.  The transcription recomputes the whole
prefix in f32 with dense weights; the oracle steps the reference's decode
path with an f32 KV cache and the CQ prepared-input arithmetic.  They are
independent implementations of one architecture, so agreement to float
rounding pins the forward's wiring: Engram, mHC with its Sinkhorn mix,
HadamardMLP, RoPE, the window, the tied LM head.  (The transcription has no
int8 KV cache; the int8 path is pinned by the quantiser fixture and by the
device's bit-exact match with the oracle.)"""
import os

import numpy as np
import pytest

import cact_writer as W
import oracle as O
import v3_synth as S

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "v3_forward_reference.npz")


@pytest.fixture(scope="module")
def run():
    f = np.load(FIXTURE)
    g, recs = S.build_records(S.small_geometry(int(f["geometry_layers"])), seed=int(f["model_seed"]))
    _, held = W.pack_synth(g, recs, S.CODEBOOK)  # the floats as the container holds them
    om = O.V3Model(g, held, S.CODEBOOK)
    prompt = f["prompt"]
    assert np.array_equal(
        prompt, S.prompt_tokens(len(prompt), int(f["prompt_seed"]), g["vocab_size"]).astype(np.int64))
    cache = om.new_cache(64, False)  # f32 KV, as the transcription computes
    logits = np.stack([np.asarray(cache.decode_step(int(t)), np.float32) for t in prompt])
    return f, logits


def test_last_positions_match_the_transcription(run):
    f, logits = run
    ref = f["last_logits"]
    scale = np.abs(ref).max()
    assert np.abs(logits[-2:] - ref).max() <= 2e-5 * scale


def test_top_logits_and_greedy_tokens_match_at_every_position(run):
    f, logits = run
    top_ids, top_vals = f["top_ids"], f["top_vals"]
    ours = np.take_along_axis(logits, top_ids, axis=1)
    assert np.abs(ours - top_vals).max() <= 2e-5 * np.abs(top_vals).max()
    # greedy tokens agree wherever the reference's top two are apart by more
    # than the tolerance (every position of this prompt)
    margin = top_vals[:, 0] - top_vals[:, 1]
    sure = margin > 4e-5 * np.abs(top_vals).max()
    assert sure.all()
    assert np.array_equal(logits.argmax(axis=1), top_ids[:, 0])
