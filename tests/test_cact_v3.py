"""The .cact v3 container reader (host only): the shipped needle3.cact's
header and directory, laid out from the reference's own fixture
(tests/cact_v3_vectors.json, every record's offset and size) with zero
blobs, walked by nd_v3_cact_config; then the reference's error variants
(CactError cact.rs:58-108, V3GeometryError v3.rs:84-90, V3LayoutError
v3.rs:180-190), each from one planted fault."""
import json
import os

import pytest

import cact_writer as W
import needle_amd as nd
import v3_synth as S

GEO = json.load(open(os.path.join(W.GOLDEN, "v3_geometry.json")))["geometry"]


@pytest.fixture(scope="module")
def shipped():
    return W.skeleton()


def _err(data, code):
    with pytest.raises(nd.NeedleError) as e:
        nd.cact_v3_config(data)
    assert e.value.code == code, str(e.value)
    return str(e.value)


def test_shipped_directory(shipped):
    assert len(shipped) == 35335380
    geom, canon = nd.cact_v3_config(shipped)
    # 1 embedding + 20 layers x 27 + 6 scalars + 3 phi + 2 perms + 5 sites x 4
    # + final_norm; the heads manifest, six head tensors and the tokenizer follow
    assert canon == 1 + 20 * 27 + 6 + 3 + 2 + 5 * 4 + 1 == 573
    for k in ("vocab_size", "out_vocab", "d_model", "num_heads", "num_kv_heads", "num_layers",
              "qk_head_dim", "v_head_dim", "max_seq_len", "hada_n", "mhc_lanes",
              "sliding_window", "qkv_conv_taps", "global_layers", "rope_theta"):
        assert geom[k] == GEO[k], k
    assert geom["orders"] == GEO["engram_orders"]
    assert geom["sites"] == GEO["engram_layers"]
    assert geom["e_slots"] == GEO["engram_slots"] and geom["e_sub_dim"] == GEO["engram_sub_dim"]
    # heads recovered as tables / orders (v3.rs:25-48)
    assert geom["e_heads"] == GEO["num_engram_tables"] // len(GEO["engram_orders"]) == 3
    # the random-init model the benches and tests run has exactly this geometry
    for k, v in S.V3_GEOMETRY.items():
        assert geom[k] == v, k


def test_too_short(shipped):
    assert "TooShort { need: 196, got: 100 }" in _err(shipped[:100], nd.ND_ERR_CACT)
    assert "TooShort { need: 25872, got: 20000 }" in _err(shipped[:20000], nd.ND_ERR_CACT)


def test_bad_tag_and_codebook(shipped):
    assert "BadTag(0x05e12a83)" in _err(W.set_word(shipped, 0, 0x05E12A83), nd.ND_ERR_CACT)
    assert "BadCodebookLen(27)" in _err(W.set_word(shipped, 2, 27), nd.ND_ERR_CACT)


def test_directory_faults(shipped):
    assert "BadNdim { index: 5, ndim: 5 }" in _err(W.set_record(shipped, 5, ndim=5),
                                                   nd.ND_ERR_CACT)
    bad = W.set_record(shipped, 7, offset=len(shipped) - 10)
    assert "BlobOutOfRange { index: 7" in _err(bad, nd.ND_ERR_CACT)


def test_geometry_faults(shipped):
    assert "NoEngramOrders" in _err(W.set_word(shipped, 26, 0), nd.ND_ERR_V3_GEOMETRY)
    assert "TableCountNotDivisible { tables: 7, orders: 2 }" in _err(
        W.set_word(shipped, 22, 7), nd.ND_ERR_V3_GEOMETRY)
    assert "SubDimMismatch { declared: 64, derived: 128 }" in _err(
        W.set_word(shipped, 21, 64), nd.ND_ERR_V3_GEOMETRY)
    assert "HeadsNotDivisible { heads: 12, kv_heads: 5 }" in _err(
        W.set_word(shipped, 9, 5), nd.ND_ERR_V3_GEOMETRY)


def test_layout_faults(shipped):
    # a directory that ends before the canon does
    assert "TooFewTensors { need: 501, got: 500 }" in _err(W.set_word(shipped, 1, 500),
                                                           nd.ND_ERR_V3_LAYOUT)
    # k_proj's record in q_proj's slot (v3.rs:355-358)
    msg = _err(W.set_record(shipped, 2, shape=[96, 768]), nd.ND_ERR_V3_LAYOUT)
    assert 'BadShape { index: 2, what: "q_proj", want: [576, 768], got: [96, 768] }' in msg
    msg = _err(W.set_record(shipped, 560, shape=[110592, 64]), nd.ND_ERR_V3_LAYOUT)
    assert 'what: "engram tables", want: [110592, 128], got: [110592, 64]' in msg


def test_dtype_faults(shipped):
    # a float record where a CQ tensor belongs, and the tokenizer's RAW
    # dtype where a float belongs
    assert "DtypeMismatch { index: 2, want: 3, got: 1 }" in _err(
        W.set_record(shipped, 2, dtype=1), nd.ND_ERR_CACT)
    assert "DtypeMismatch { index: 1, want: 1, got: 4 }" in _err(
        W.set_record(shipped, 1, dtype=4), nd.ND_ERR_CACT)
    assert "RaggedBlob { index: 1, nbytes: 1535 }" in _err(
        W.set_record(shipped, 1, nbytes=1535), nd.ND_ERR_CACT)


def test_trailing_records_are_not_read(shipped):
    """The heads manifest, head tensors and tokenizer are past the canon: a
    fault there does not stop the model from loading."""
    geom, canon = nd.cact_v3_config(W.set_record(shipped, 575, dtype=9))
    assert canon == 573


# ---- ladder rungs (v3/ladder.rs, v3.rs:612-734) -------------------------------

LADDER = json.load(open(os.path.join(W.GOLDEN, "v3_ladder_rungs.json")))


def _order_brute(L):
    """The ladder order restated from its definition: both endpoints, then
    repeatedly the midpoint of the widest gap between chosen blocks, the
    leftmost of equal gaps first."""
    chosen = [0, L - 1]
    while len(chosen) < L:
        s = sorted(chosen)
        gaps = [(s[i + 1] - s[i], -s[i], s[i], s[i + 1]) for i in range(len(s) - 1)
                if s[i + 1] - s[i] > 1]
        _, _, a, b = max(gaps)
        chosen.append((a + b) // 2)
    return chosen


def test_ladder_rungs_match_upstream():
    """Every depth of the 20-block stack keeps upstream's blocks
    (tests/v3_ladder_rungs.json, upstream ladder_config)."""
    assert _order_brute(20) == LADDER["ladder_order"]
    for rung in LADDER["rungs"]:
        assert nd.v3_ladder(20, rung["depth"]) == rung["selected"], rung["depth"]


@pytest.mark.parametrize("L", [2, 3, 4, 7, 12, 33])
def test_ladder_nests_and_keeps_both_ends(L):
    order = _order_brute(L)
    prev = []
    for depth in range(2, L + 1):
        kept = nd.v3_ladder(L, depth)
        assert kept == sorted(order[:depth])
        assert kept[0] == 0 and kept[-1] == L - 1
        assert set(prev) < set(kept)
        prev = kept


def test_ladder_refuses_depths_outside():
    for bad in (0, 1, 21, 100):
        with pytest.raises(nd.NeedleError) as e:
            nd.v3_ladder(20, bad)
        assert e.value.code == nd.ND_ERR_ARG and "outside the ladder" in str(e.value)


def test_rung_geometry_of_the_shipped_container(shipped):
    """config_at_depth on the shipped directory: kept blocks renumbered,
    global layers and Engram sites following them, as upstream's
    ladder_config gives for every depth."""
    full, _ = nd.cact_v3_config(shipped)
    for rung in LADDER["rungs"]:
        d = rung["depth"]
        geom, kept = nd.cact_v3_config_at_depth(shipped, d)
        assert kept == rung["selected"]
        assert geom["num_layers"] == d
        assert geom["global_layers"] == rung["global_layers"], d
        assert geom["sites"] == rung["engram_sites"], d
        for k in ("d_model", "num_heads", "num_kv_heads", "sliding_window", "orders", "e_slots"):
            assert geom[k] == full[k]
    for bad in (0, 1, 21):
        with pytest.raises(nd.NeedleError):
            nd.cact_v3_config_at_depth(shipped, bad)


def test_rung_reads_only_the_kept_blocks(shipped):
    """model_from_cact_at_depth decodes the kept blocks only: a bad float
    record in block 1 stops the full read and the 3-block rung (blocks
    0, 9, 19) does not see it; a bad record in a kept block still stops it."""
    per_layer = 27
    bad1 = W.set_record(shipped, 1 + 1 * per_layer, dtype=4)  # block 1 norm_in as RAW
    with pytest.raises(nd.NeedleError) as e:
        nd.cact_v3_config(bad1)
    assert "DtypeMismatch { index: 28, want: 1, got: 4 }" in str(e.value)
    geom, kept = nd.cact_v3_config_at_depth(bad1, 3)
    assert kept == [0, 9, 19] and geom["num_layers"] == 3
    bad9 = W.set_record(shipped, 1 + 9 * per_layer, dtype=4)
    with pytest.raises(nd.NeedleError) as e:
        nd.cact_v3_config_at_depth(bad9, 3)
    assert "DtypeMismatch { index: 244, want: 1, got: 4 }" in str(e.value)
    # shapes are checked for every block, kept or not (V3Layout::derive)
    with pytest.raises(nd.NeedleError) as e:
        nd.cact_v3_config_at_depth(W.set_record(shipped, 1 + 1 * per_layer + 1, shape=[96, 768]), 3)
    assert e.value.code == nd.ND_ERR_V3_LAYOUT and "q_proj" in str(e.value)


def test_kv_bytes_closed_forms_and_published_figures(shipped):
    """V3Config::kv_bytes_at on the shipped geometry: the reference's own
    closed forms (config.rs:255-282: 512 x 20 x 224 and
    (16 x 1024 + 4 x 8192) x 224 at one byte per element, only the global
    layers growing past the window) and the sizes its docs publish (42.0 /
    11.2 MB at 8192, 8.8 / 2.3 MB at 512, docs/c-ffi.md:121-122 and
    README.md:66; 3.5 MB for the 8-block rung and 2.6 MB for the 6-block
    one at 512, README.md:148 and docs/v3-port-record.md:164)."""
    geom, _ = nd.cact_v3_config(shipped)
    per = 2 * (48 + 64)
    assert nd.v3_kv_bytes(geom, 512, False) == 512 * 20 * per * 4
    assert nd.v3_kv_bytes(geom, 8192, False) == (16 * 1024 + 4 * 8192) * per * 4
    assert nd.v3_kv_bytes(geom, 8192, True) == (16 * 1024 + 4 * 8192) * (per + 2 * 8)
    grow = nd.v3_kv_bytes(geom, 2048, False) - nd.v3_kv_bytes(geom, 1024, False)
    assert grow == 4 * 1024 * per * 4
    MB = float(1 << 20)
    assert round(nd.v3_kv_bytes(geom, 8192, False) / MB, 1) == 42.0
    assert round(nd.v3_kv_bytes(geom, 8192, True) / MB, 1) == 11.2
    assert round(nd.v3_kv_bytes(geom, 512, False) / MB, 1) == 8.8
    assert round(nd.v3_kv_bytes(geom, 512, True) / MB, 1) == 2.3
    g8, _ = nd.cact_v3_config_at_depth(shipped, 8)
    g6, _ = nd.cact_v3_config_at_depth(shipped, 6)
    assert round(nd.v3_kv_bytes(g8, 512, False) / MB, 1) == 3.5
    assert round(nd.v3_kv_bytes(g6, 512, False) / MB, 1) == 2.6
    # int8: one byte plus an f32 scale per head vector -- a touch over a
    # quarter of f32, never at or above a half (v3_kv_int8.rs:58-62)
    a, b = nd.v3_kv_bytes(geom, 2048, False), nd.v3_kv_bytes(geom, 2048, True)
    assert b * 3 < a < b * 5


def test_kv_bytes_null_cfg():
    assert nd.lib().nd_v3_kv_bytes(None, 512, 1) == 0
    assert "null" in nd.lib().nd_last_error().decode()
