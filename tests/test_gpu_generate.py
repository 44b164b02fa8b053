"""nd_v3_generate: the greedy loop of V3Engine::generate_with
(crates/needle-infer/src/v3_engine.rs:254-312) with each step's choice fed
back on the device.  It must give the tokens of host-driven stepping that
feeds `next` back, leave the batch exactly where that stepping leaves it
(caches, conv tails, retained ids, positions: the next steps' logits are
bit-identical), and match the oracle's greedy tokens."""
import numpy as np
import pytest
import torch

import needle_amd as nd
import oracle as O
import v3_synth as S

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _prefilled(dm, prompts, max_len, chunk):
    b = nd.V3Batch(dm, prompts.shape[0], max_len=max_len, max_chunk=chunk)
    n = prompts.shape[1]
    nxt = None
    for t0 in range(0, n, chunk):
        t1 = min(n, t0 + chunk)
        if t1 - t0 == 1:
            nxt = b.step(prompts[:, t0], want_next=(t1 == n))
        else:
            nxt = b.prefill(prompts[:, t0:t1], want_next=(t1 == n))
    return b, nxt


@pytest.mark.parametrize("geom,sessions,prompt,steps,chunk", [
    ("small", 3, 37, 45, 8),      # window 32: the local rings wrap during the loop
    ("shipped", 2, 24, 40, 24),
])
def test_generate_equals_stepping(ctx, geom, sessions, prompt, steps, chunk):
    g, recs = S.build_records(S.small_geometry(4) if geom == "small" else None, seed=5)
    dm = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    prompts = np.stack([S.prompt_tokens(prompt, 40 + i) for i in range(sessions)])
    max_len = prompt + steps + 8
    a, first = _prefilled(dm, prompts, max_len, chunk)
    b, first_b = _prefilled(dm, prompts, max_len, chunk)
    assert np.array_equal(first, first_b)
    # host stepping: each step's next fed back through the host
    want = np.zeros((sessions, steps), np.int32)
    tok = first
    for s in range(steps):
        tok = a.step(tok)
        want[:, s] = tok
    got = b.greedy(first, steps)
    assert np.array_equal(got, want)
    assert np.array_equal(a.positions(), b.positions())
    # both batches continue from the same state, bit for bit
    la = torch.empty(sessions, dm.rows, device="cuda")
    lb = torch.empty(sessions, dm.rows, device="cuda")
    extra = np.stack([S.prompt_tokens(3, 90 + i) for i in range(sessions)])
    for t in range(extra.shape[1]):
        a.step(extra[:, t], logits=la, want_next=False)
        b.step(extra[:, t], logits=lb, want_next=False)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(la.cpu().numpy()), _bits(lb.cpu().numpy())), t
    # a second loop on the same batch continues the retained ids correctly
    tok = a.step(want[:, -1])
    got2 = b.greedy(want[:, -1], 4)
    assert got2[:, 0].tolist() == tok.tolist()
    a.close()
    b.close()
    dm.close()


def test_generate_matches_oracle(ctx):
    """Shipped geometry, one session: prompt 32 stepped, then 48 greedy
    tokens from the device loop against the oracle's greedy run."""
    g, recs = S.build_records(None, seed=0)
    dm = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    om = O.V3Model(g, recs, S.CODEBOOK)
    prompt = S.prompt_tokens(32, 7)
    want, _ = O.v3_generate(om, prompt, 49, hint=32 + 49)
    b, first = _prefilled(dm, np.asarray(prompt, np.int32)[None], 32 + 49, 32)
    assert first[0] == want[0]
    got = b.greedy(first, 48)[0]
    assert np.array_equal(got, want[1:49].astype(np.int32))
    b.close()
    dm.close()


def test_generate_rejects_overflow(ctx):
    g, recs = S.build_records(S.small_geometry(2), seed=9)
    dm = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    b = nd.V3Batch(dm, 1, max_len=8)
    with pytest.raises(nd.NeedleError):
        b.greedy(np.array([1], np.int32), 9)
    assert list(b.positions()) == [0]
    b.close()
    dm.close()


def test_generate_many_equals_each(ctx):
    """nd_v3_generate_many: two batches of one model on two contexts (their
    own streams), stepped in turn from this thread, end exactly where
    nd_v3_generate leaves each alone: tokens, positions and the next
    step's logits, bit for bit."""
    g, recs = S.build_records(S.small_geometry(4), seed=5)
    dm = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    ctxs = [nd.Ctx(0, stream=s) for s in streams]
    shapes = [(3, 37, 8), (2, 20, 16)]  # sessions, prompt, chunk
    steps = 30
    prompts = [np.stack([S.prompt_tokens(n, 70 + 10 * k + i) for i in range(s)])
               for k, (s, n, _) in enumerate(shapes)]

    def prefilled(k, on):
        s, n, chunk = shapes[k]
        b = nd.V3Batch(dm, s, max_len=n + steps + 8, max_chunk=chunk, ctx=on)
        nxt = None
        for t0 in range(0, n, chunk):
            t1 = min(n, t0 + chunk)
            nxt = (b.step(prompts[k][:, t0], want_next=(t1 == n)) if t1 - t0 == 1
                   else b.prefill(prompts[k][:, t0:t1], want_next=(t1 == n)))
        return b, nxt

    alone = [prefilled(k, ctx) for k in range(2)]
    want = [b.greedy(f, steps) for b, f in alone]
    many = [prefilled(k, ctxs[k]) for k in range(2)]
    torch.cuda.synchronize()
    got = nd.V3Batch.greedy_many([b for b, _ in many], [f for _, f in many], steps)
    for k in range(2):
        assert np.array_equal(got[k], want[k]), k
        assert np.array_equal(many[k][0].positions(), alone[k][0].positions())
        s = shapes[k][0]
        la = torch.empty(s, dm.rows, device="cuda")
        lb = torch.empty(s, dm.rows, device="cuda")
        alone[k][0].step(want[k][:, -1], logits=la, want_next=False)
        many[k][0].step(got[k][:, -1], logits=lb, want_next=False)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(la.cpu().numpy()), _bits(lb.cpu().numpy())), k
    for b, _ in alone + many:
        b.close()
    for c in ctxs:
        c.close()
    dm.close()


def test_generate_many_rejects_repeats(ctx):
    g, recs = S.build_records(S.small_geometry(2), seed=9)
    dm = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    b = nd.V3Batch(dm, 1, max_len=16)
    with pytest.raises(nd.NeedleError):
        nd.V3Batch.greedy_many([b, b], [np.array([1], np.int32)] * 2, 2)
    assert list(b.positions()) == [0]
    b.close()
    dm.close()
