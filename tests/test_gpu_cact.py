"""A model read from a .cact v3 container (nd_v3_model_from_cact) against the
same model built from its canonical records and against the oracle: the
container holds the float tensors as FP16 and the permutations as FP32, as
needle3.cact does, and the logits agree bit for bit at every step."""
import numpy as np
import pytest
import torch

import cact_writer as W
import needle_amd as nd
import oracle as O
import v3_synth as S

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_model_from_container_matches_records(ctx):
    g, recs = S.build_records(S.small_geometry(4), seed=23)
    data, held = W.pack_synth(g, recs, S.CODEBOOK)
    geom, canon = nd.cact_v3_config(data)
    assert canon == len(held)
    for k, v in g.items():
        assert geom[k] == (pytest.approx(v) if isinstance(v, float) else v), k
    from_file = nd.V3Model.from_cact(ctx, data)
    from_recs = nd.V3Model(ctx, g, held, S.CODEBOOK)
    om = O.V3Model(g, held, S.CODEBOOK)
    cache = om.new_cache(40, True)
    prompt = S.prompt_tokens(40, 9)
    b1, b2 = nd.V3Batch(from_file, 1, max_len=48), nd.V3Batch(from_recs, 1, max_len=48)
    l1 = torch.empty(1, from_file.rows, device="cuda")
    l2 = torch.empty(1, from_recs.rows, device="cuda")
    for t, tok in enumerate(prompt):
        b1.step([tok], logits=l1, want_next=False)
        b2.step([tok], logits=l2, want_next=False)
        want = cache.decode_step(tok)
        a1, a2 = l1.cpu().numpy()[0], l2.cpu().numpy()[0]
        assert np.array_equal(_bits(a1), _bits(a2)), t
        assert np.array_equal(_bits(a1), _bits(want)), t
    b1.close()
    b2.close()


def test_container_errors_reach_the_caller(ctx):
    g, recs = S.build_records(S.small_geometry(4), seed=5)
    data, _ = W.pack_synth(g, recs, S.CODEBOOK)
    with pytest.raises(nd.NeedleError) as e:
        nd.V3Model.from_cact(ctx, W.set_record(data, 2, shape=[16, 768]))
    assert e.value.code == nd.ND_ERR_V3_LAYOUT and "q_proj" in str(e.value)
