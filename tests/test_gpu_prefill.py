"""Prefill of several positions per pass (nd_v3_prefill) against stepping
(nd_v3_step) and the oracle: V3Model::prefill is bit-identical to stepping
(needle-infer/tests/v3_kv_int8.rs:269-282), and so is this -- the logits of
each pass's last position, and every logit and token of the decode that
follows (so the int8 caches and the conv tails are the same too).

The small geometry's 32-position window makes the local rings wrap within
these prompts; chunks of up to 16 positions exercise the widened ring
(window + chunk - 1 slots), the causal conv and the dilated Engram conv
reaching back into the same pass and into the tails."""
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
    g, recs = S.build_records(S.small_geometry(4), seed=31)
    return g, recs, O.V3Model(g, recs, S.CODEBOOK), nd.V3Model(ctx, g, recs, S.CODEBOOK)


@pytest.mark.parametrize("chunks", [[16, 16, 16], [5, 16, 1, 13, 13], [2, 3, 7, 11, 16, 9]])
def test_prefill_chunks_equal_stepping(small, chunks):
    g, recs, om, dm = small
    n = sum(chunks)
    prompt = S.prompt_tokens(n, 17)
    steps = 12
    ref = nd.V3Batch(dm, 1, max_len=n + steps + 1)
    got = nd.V3Batch(dm, 1, max_len=n + steps + 1, max_chunk=16)
    lr = torch.empty(1, dm.rows, device="cuda")
    lg = torch.empty(1, dm.rows, device="cuda")
    t = 0
    for c in chunks:
        for tok in prompt[t:t + c]:
            nr = ref.step([tok], logits=lr)
        ng = got.prefill(np.array(prompt[t:t + c])[None], logits=lg)
        t += c
        assert np.array_equal(_bits(lr.cpu().numpy()), _bits(lg.cpu().numpy())), t
        assert list(nr) == list(ng)
    # the caches and tails left behind: the decode that follows is identical
    for s in range(steps):
        nr = ref.step(nr, logits=lr)
        ng = got.step(ng, logits=lg)
        assert np.array_equal(_bits(lr.cpu().numpy()), _bits(lg.cpu().numpy())), s
        assert list(nr) == list(ng)
    assert list(got.positions()) == [n + steps]
    ref.close()
    got.close()


def test_prefill_sessions_match_oracle(small):
    """Three sessions, 24-position prompts in passes of 16 then 8, each
    equal to its own oracle run."""
    g, recs, om, dm = small
    B, n = 3, 24
    prompts = np.stack([S.prompt_tokens(n, 40 + i) for i in range(B)]).astype(np.int32)
    batch = nd.V3Batch(dm, B, max_len=n + 1, max_chunk=16)
    lg = torch.empty(B, dm.rows, device="cuda")
    batch.prefill(prompts[:, :16], want_next=False)
    nxt = batch.prefill(prompts[:, 16:], logits=lg)
    got = lg.cpu().numpy()
    for i in range(B):
        cache = om.new_cache(n, True)
        for tok in prompts[i]:
            want = cache.decode_step(int(tok))
        assert np.array_equal(_bits(got[i]), _bits(want)), i
        assert nxt[i] == int(np.argmax(want))
    batch.close()


def test_generate_chunked_equals_stepped(small):
    g, recs, om, dm = small
    prompts = np.stack([S.prompt_tokens(40, 60 + i) for i in range(2)]).astype(np.int32)
    a = nd.V3Batch(dm, 2, max_len=60).generate(prompts, 16)
    b = nd.V3Batch(dm, 2, max_len=60, max_chunk=16).generate(prompts, 16)
    assert np.array_equal(a, b)


def test_prefill_rejects_oversized_pass(small):
    g, recs, om, dm = small
    batch = nd.V3Batch(dm, 1, max_len=64, max_chunk=8)
    with pytest.raises(nd.NeedleError):
        batch.prefill(np.zeros((1, 9), np.int32))
    full = nd.V3Batch(dm, 1, max_len=8, max_chunk=8)
    full.prefill(np.zeros((1, 8), np.int32), want_next=False)
    with pytest.raises(nd.NeedleError) as e:
        full.prefill(np.zeros((1, 1), np.int32))
    assert "full" in str(e.value)
    full.close()
    batch.close()
