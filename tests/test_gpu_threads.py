"""Host threads sharing one device model, as the reference's server shares one
V3Model across sessions, each with its own V3Cache
(crates/needle-infer/src/v3_engine.rs:544-561): every thread steps its own
batch through its own context (and stream), concurrently, and each thread's
logits are bit-identical to the same sessions run alone on one thread."""
import threading

import numpy as np
import pytest
import torch

import needle_amd as nd
import v3_synth as S

pytestmark = pytest.mark.gpu

THREADS = 3
SESSIONS = 2
PROMPT, GREEDY = 20, 20


@pytest.fixture(scope="module")
def model(ctx):
    g, recs = S.build_records(S.small_geometry(4), seed=23)
    m = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    ctx.synchronize()
    return m


def _run(model, prompts, bctx, stream):
    """Prompt then greedy tokens for `prompts` [sessions][PROMPT]; every
    step's logits, copied to the host after the context's stream is done."""
    with torch.cuda.stream(stream):
        b = nd.V3Batch(model, SESSIONS, max_len=PROMPT + GREEDY + 1, ctx=bctx)
        logits = torch.empty(SESSIONS, model.rows, device="cuda")
        out = []
        nxt = None
        for t in range(PROMPT + GREEDY):
            tok = prompts[:, t] if t < PROMPT else nxt
            nxt = b.step(tok, logits=logits, want_next=True)
            bctx.synchronize()
            out.append(logits.cpu().numpy().copy())
        b.close()
    return np.stack(out)


def test_threads_share_one_model(model, ctx):
    prompts = [np.stack([S.prompt_tokens(PROMPT, 300 + 10 * i + j) for j in range(SESSIONS)])
               for i in range(THREADS)]
    # each thread's sessions alone, one after another, on the model's context
    main = torch.cuda.current_stream()
    want = [_run(model, p, ctx, main) for p in prompts]

    ready = threading.Barrier(THREADS)
    got, errors = [None] * THREADS, []

    def worker(i):
        try:
            stream = torch.cuda.Stream()
            c = nd.Ctx(0, stream=stream)
            ready.wait(timeout=60)
            got[i] = _run(model, prompts[i], c, stream)
            c.close()
        except Exception as e:  # reported below, on the test's thread
            errors.append((i, repr(e)))

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(THREADS)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in ts), "a thread did not finish"
    assert not errors, errors
    for i in range(THREADS):
        assert np.array_equal(got[i].view(np.uint32), want[i].view(np.uint32)), i
        # greedy tokens follow from the logits; different prompts, different runs
        assert not np.array_equal(want[i], want[(i + 1) % THREADS])
