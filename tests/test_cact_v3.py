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
