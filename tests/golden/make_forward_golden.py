"""Golden f32 logits of a seeded random-init Needle-3 model, computed by the
reference's own numpy transcription of the forward
(tools/needle3_reference.py in the reference repository: `Model(path)
.forward(ids)`, a whole-prefix recomputation in f32, no KV cache).

The model is v3_synth's 4-layer geometry at the shipped widths (a global
layer, Engram sites, a 32-position sliding window), packed into a `.cact`
container by tests/cact_writer.py; the prompt has 40 tokens, so the local
layers' window wraps.  Written here, in the container that holds the
reference, to tests/golden/v3_forward_reference.npz; the tests only read
the fixture.  Run: python3 tests/golden/make_forward_golden.py
"""
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REFERENCE_TOOLS = "/root/reference/tools"

GEOMETRY_LAYERS = 4
MODEL_SEED = 11
PROMPT_LEN = 40
PROMPT_SEED = 21
TOP = 16
OUT = os.path.join(HERE, "v3_forward_reference.npz")


def main():
    sys.path.insert(0, os.path.join(REPO, "needle-rs_amd"))
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import cact_writer as W
    import v3_synth as S

    g, recs = S.build_records(S.small_geometry(GEOMETRY_LAYERS), seed=MODEL_SEED)
    data, _ = W.pack_synth(g, recs, S.CODEBOOK)
    ids = S.prompt_tokens(PROMPT_LEN, PROMPT_SEED, g["vocab_size"]).astype(np.int64)

    sys.path.insert(0, REFERENCE_TOOLS)
    import needle3_reference as R

    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "synth.cact")
        with open(path, "wb") as f:
            f.write(data)
        logits = np.asarray(R.Model(path).forward(ids), np.float32)

    order = np.argsort(-logits, axis=1, kind="stable")[:, :TOP]
    np.savez(OUT,
             geometry_layers=np.int64(GEOMETRY_LAYERS), model_seed=np.int64(MODEL_SEED),
             prompt_seed=np.int64(PROMPT_SEED), prompt=ids.astype(np.int64),
             last_logits=logits[-2:].copy(),
             top_ids=order.astype(np.int64),
             top_vals=np.take_along_axis(logits, order, axis=1).astype(np.float32))
    print(OUT, logits.shape, float(np.abs(logits).max()))


if __name__ == "__main__":
    main()
