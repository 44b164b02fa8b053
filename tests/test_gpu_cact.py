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


def _rung_records(g, recs, kept):
    """A rung's canonical records restated from the slice's definition: kept
    blocks whole; per-layer mHC scalars and phi lane rows of the kept blocks
    (a Cactus-Quants row cut copies packed bytes and FP16 norms); the
    Engram sites on kept blocks; the rest unchanged."""
    L, n = g["num_layers"], g["mhc_lanes"]
    per = 24 + (3 if g["qkv_conv_taps"] > 0 else 0)
    out = [recs[0]]
    for l in kept:
        out += recs[1 + l * per:1 + (l + 1) * per]
    at = 1 + L * per
    for r, w in zip(recs[at:at + 6], (1, 1, 1, n, n, n * n)):
        data = np.ascontiguousarray(np.asarray(r["data"]).reshape(L, w)[kept].reshape(
            (len(kept),) if w == 1 else (len(kept), w)), np.float32)
        out.append(dict(r, data=data, out=len(kept)))
    for r, w in zip(recs[at + 6:at + 9], (n, n, n * n)):
        pad = -(-r["inn"] // r["group"]) * r["group"]
        rb, ng = pad * r["bits"] // 8, pad // r["group"]
        blob = np.asarray(r["data"], np.uint8)
        packed = blob[:r["out"] * rb].reshape(r["out"], rb)
        norms = blob[r["out"] * rb:r["out"] * (rb + 2 * ng)].reshape(r["out"], 2 * ng)
        rows = [row for l in kept for row in range(l * w, (l + 1) * w)]
        cut = np.concatenate([packed[rows].ravel(), norms[rows].ravel()])
        out.append(dict(r, data=cut, out=len(rows)))
    out += recs[at + 9:at + 11]
    for s, layer in enumerate(g["sites"]):
        if layer in kept:
            out += recs[at + 11 + 4 * s:at + 15 + 4 * s]
    out.append(recs[-1])
    rank = {l: i for i, l in enumerate(kept)}
    rg = dict(g, num_layers=len(kept),
              global_layers=[rank[l] for l in g["global_layers"] if l in rank],
              sites=[rank[l] for l in g["sites"] if l in rank])
    return rg, out


@pytest.mark.parametrize("depth", [2, 3])
def test_rung_from_container_matches_sliced_records(ctx, depth):
    """model_from_cact_at_depth on the device against the oracle run on the
    rung's records sliced independently: logits bit-identical every step."""
    g, recs = S.build_records(S.small_geometry(4), seed=29)
    data, held = W.pack_synth(g, recs, S.CODEBOOK)
    kept = nd.v3_ladder(4, depth)
    rg, rrecs = _rung_records(g, held, kept)
    geom, got_kept = nd.cact_v3_config_at_depth(data, depth)
    assert got_kept == kept and geom["num_layers"] == depth
    assert geom["global_layers"] == rg["global_layers"] and geom["sites"] == rg["sites"]
    dm = nd.V3Model.from_cact(ctx, data, depth=depth)
    om = O.V3Model(rg, rrecs, S.CODEBOOK)
    cache = om.new_cache(24, True)
    batch = nd.V3Batch(dm, 1, max_len=32)
    lg = torch.empty(1, dm.rows, device="cuda")
    for t, tok in enumerate(S.prompt_tokens(24, 13)):
        batch.step([tok], logits=lg, want_next=False)
        want = cache.decode_step(tok)
        assert np.array_equal(_bits(lg.cpu().numpy()[0]), _bits(want)), (depth, t)
    batch.close()


def test_full_depth_is_the_ordinary_load(ctx):
    g, recs = S.build_records(S.small_geometry(4), seed=31)
    data, _ = W.pack_synth(g, recs, S.CODEBOOK)
    a, b = nd.V3Model.from_cact(ctx, data), nd.V3Model.from_cact(ctx, data, depth=4)
    ba, bb = nd.V3Batch(a, 1, max_len=16), nd.V3Batch(b, 1, max_len=16)
    la = torch.empty(1, a.rows, device="cuda")
    lb = torch.empty(1, b.rows, device="cuda")
    for tok in S.prompt_tokens(12, 3):
        ba.step([tok], logits=la, want_next=False)
        bb.step([tok], logits=lb, want_next=False)
        assert np.array_equal(_bits(la.cpu().numpy()), _bits(lb.cpu().numpy()))
    ba.close()
    bb.close()
    with pytest.raises(nd.NeedleError):
        nd.V3Model.from_cact(ctx, data, depth=5)
