"""Extract the reference's own tracked fixtures for this path into small,
self-contained data files under tests/golden/.

Reads JSON data files only (no reference code is imported or run):
  tests/v3_kv_quant_vectors.json  -> kv_quant_vectors.json   (upstream fake_quant KAT)
  tests/cact_vectors.json         -> cq_codebook.json        (28-float cb2|cb3|cb4)
  tests/cact_v3_vectors.json      -> v3_geometry.json, v3_cq_records.json, v3_directory.json
  tests/v3_ladder_rungs.json      -> v3_ladder_rungs.json    (upstream ladder_config per depth)
Run from the repo root:  python tests/golden/make_fixtures.py [/root/reference]
"""
import json
import os
import sys

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
OUT = os.path.dirname(os.path.abspath(__file__))


def dump(name, obj):
    with open(os.path.join(OUT, name), "w") as f:
        json.dump(obj, f, indent=1)
        f.write("\n")


kv = json.load(open(os.path.join(REF, "tests/v3_kv_quant_vectors.json")))
kv["provenance"] = ("needle-rs tests/v3_kv_quant_vectors.json: upstream "
                    "needle.model.quantize.fake_quant(x, x.shape[-1], 8)")
dump("kv_quant_vectors.json", kv)

v2 = json.load(open(os.path.join(REF, "tests/cact_vectors.json")))
dump("cq_codebook.json", {
    "provenance": "needle-rs tests/cact_vectors.json 'codebook' (cb2|cb3|cb4, "
                  "already scaled by 1/sqrt(group)), exported from needle2.cact",
    "codebook": v2["codebook"],
})

v3 = json.load(open(os.path.join(REF, "tests/cact_v3_vectors.json")))
dump("v3_geometry.json", {
    "provenance": "needle-rs tests/cact_v3_vectors.json 'geometry' (needle3.cact header)",
    "geometry": v3["geometry"],
    "container_bytes": v3["container_bytes"],
})
cq = [dict(index=r["index"], shape=r["shape"], nbytes=r["nbytes"], group=r["group"],
           bits=r["bits"]) for r in v3["records"] if r["dtype"] == 3]
dump("v3_cq_records.json", {
    "provenance": "needle-rs tests/cact_v3_vectors.json 'records' with dtype 3 (CQ)",
    "records": cq,
})
dump("v3_directory.json", {
    "provenance": "needle-rs tests/cact_v3_vectors.json: the whole needle3.cact directory "
                  "(every record's dtype, ndim, shape, offset, nbytes, group, bits) and sizes",
    "container_bytes": v3["container_bytes"],
    "header_bytes": v3["header_bytes"],
    "record_bytes": v3["record_bytes"],
    "codebook_len": v3["codebook_len"],
    "records": [[r["index"], r["dtype"], r["ndim"], r["shape"], r["offset"], r["nbytes"],
                 r["group"], r["bits"]] for r in v3["records"]],
})
lad = json.load(open(os.path.join(REF, "tests/v3_ladder_rungs.json")))
dump("v3_ladder_rungs.json", {
    "provenance": "needle-rs tests/v3_ladder_rungs.json: upstream ladder_config for every "
                  "depth of the 20-block stack (kept blocks, renumbered global layers and "
                  "Engram sites)",
    "parent_layers": lad["parent_layers"],
    "ladder_order": lad["ladder_order"],
    "parent_global": lad["parent_global"],
    "parent_engram_sites": lad["parent_engram_sites"],
    "rungs": [dict(depth=r["depth"], selected=r["selected"], global_layers=r["global_layers"],
                   engram_sites=r["engram_sites"]) for r in lad["rungs"]],
})
print(f"wrote {len(kv['cases'])} kv cases, {len(cq)} CQ records, "
      f"{len(v3['records'])} directory records")
