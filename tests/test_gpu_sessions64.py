"""Config 5 at its full size: 64 sessions of the shipped Needle-3 geometry,
each prefilled with a 2048-token prompt in 32-position passes, then 128
greedy steps in lockstep (int8 KV; projections batched over the sessions).

This is the multi-session decode the reference runs as independent
V3Model::decode_step calls per session (v3/model.rs:150-375; prefill
:512-523, bit-identical to stepping, needle-infer/tests/v3_kv_int8.rs:190-302).
Checked here:
  * every session's logits at each pass end and at each greedy step, and its
    tokens, equal a batch-1 device run of that session bit for bit (a
    session's result does not depend on the batch it shares);
  * sessions 0 and 63 equal the oracle's decode_step over all 2,176
    positions: logits at every pass end and every greedy step, bit for bit,
    and the greedy tokens (first maximum wins, v3_engine.rs:410-420).
The two oracle sessions run on host threads while the device works (ctypes
releases the GIL); the oracle splits rows and heads across its own threads,
which keeps its bits (each row's arithmetic is unchanged).

The prompts are the ones bench.py times (v3_synth.prompt_tokens(2048, 100 + i)).
"""
import os
import threading

import numpy as np
import pytest
import torch

import needle_amd as nd
import oracle as O
import v3_synth as S

pytestmark = pytest.mark.gpu

SESSIONS, PROMPT, STEPS, CHUNK = 64, 2048, 128, 32
ORACLE_SESSIONS = (0, 63)


def _host_cpus():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def _oracle_session(om, prompt, rows, out):
    """decode_step over the prompt, keeping the logits at each pass end,
    then STEPS greedy steps with their logits and tokens."""
    cache = om.new_cache(PROMPT + STEPS, True)
    passes = np.zeros((PROMPT // CHUNK, rows), np.float32)
    lg = None
    for t, tok in enumerate(prompt):
        lg = cache.decode_step(int(tok))
        if (t + 1) % CHUNK == 0:
            passes[t // CHUNK] = lg
    steps = np.zeros((STEPS, rows), np.float32)
    toks = np.zeros(STEPS, np.int32)
    for s in range(STEPS):
        nxt = int(np.argmax(lg))  # the first maximum, as or_argmax / the engine
        toks[s] = nxt
        lg = cache.decode_step(nxt)
        steps[s] = lg
    out["passes"], out["steps"], out["tokens"] = passes, steps, toks


def _device_run(dm, prompts, rows):
    """Prefill in CHUNK-position passes, then STEPS greedy steps; the logits
    of every pass end and every step stay on the device."""
    B = prompts.shape[0]
    batch = nd.V3Batch(dm, B, max_len=PROMPT + STEPS, max_chunk=CHUNK)
    passes = torch.empty(PROMPT // CHUNK, B, rows, device="cuda")
    steps = torch.empty(STEPS, B, rows, device="cuda")
    toks = np.zeros((B, STEPS), np.int32)
    nxt = None
    for i, t in enumerate(range(0, PROMPT, CHUNK)):
        nxt = batch.prefill(prompts[:, t:t + CHUNK], logits=passes[i],
                            want_next=(t + CHUNK == PROMPT))
    for s in range(STEPS):
        toks[:, s] = nxt
        nxt = batch.step(nxt, logits=steps[s])
    assert list(batch.positions()) == [PROMPT + STEPS] * B
    batch.close()
    return passes, steps, toks


def _same(a, b):
    return torch.equal(a.contiguous().view(torch.int32), b.contiguous().view(torch.int32))


@pytest.mark.timeout(900)
def test_sessions64_ctx2048_greedy128(ctx):
    g, recs = S.build_records(None, seed=0)
    dm = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    rows = dm.rows
    prompts = np.stack([S.prompt_tokens(PROMPT, 100 + i) for i in range(SESSIONS)]).astype(np.int32)

    om = O.V3Model(g, recs, S.CODEBOOK)
    cpus = _host_cpus()
    O.set_threads(max(1, cpus // len(ORACLE_SESSIONS)), O.SPLIT_ALL)
    want = {i: {} for i in ORACLE_SESSIONS}
    workers = [threading.Thread(target=_oracle_session, args=(om, prompts[i], rows, want[i]))
               for i in ORACLE_SESSIONS]
    for w in workers:
        w.start()
    try:
        passes, steps, toks = _device_run(dm, prompts, rows)
        # every session against its own batch-1 run
        bad = []
        for i in range(SESSIONS):
            p1, s1, t1 = _device_run(dm, prompts[i:i + 1], rows)
            if not (_same(p1[:, 0], passes[:, i]) and _same(s1[:, 0], steps[:, i])
                    and np.array_equal(t1[0], toks[i])):
                bad.append(i)
            del p1, s1
        assert not bad, f"sessions differing from their batch-1 run: {bad}"
    finally:
        for w in workers:
            w.join()
        O.set_threads(1, O.SPLIT_REFERENCE)

    for i in ORACLE_SESSIONS:
        w = want[i]
        assert "tokens" in w, f"oracle session {i} did not finish"
        got_p = passes[:, i].cpu().numpy()
        got_s = steps[:, i].cpu().numpy()
        bad_p = [j for j in range(got_p.shape[0])
                 if not np.array_equal(got_p[j].view(np.uint32), w["passes"][j].view(np.uint32))]
        bad_s = [j for j in range(STEPS)
                 if not np.array_equal(got_s[j].view(np.uint32), w["steps"][j].view(np.uint32))]
        print(f"session {i}: {len(set(w['tokens'].tolist()))} distinct greedy tokens; "
              f"pass ends differing {bad_p[:4]}, steps differing {bad_s[:4]}")
        assert not bad_p and not bad_s, (i, bad_p[:8], bad_s[:8])
        assert np.array_equal(toks[i], w["tokens"]), i
    dm.close()
