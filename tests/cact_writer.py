"""Needle-3 .cact containers for the tests, in the byte layout that
needle-infer/src/cact.rs reads: 49 little-endian u32 header words (rope_theta's
bits last), the 28-float codebook, one 44-byte directory record per tensor
(u8 dtype, u8 ndim, u16 pad, u32 shape[4], u64 offset, u64 nbytes, u32 group,
u32 bits), blobs 64-byte aligned.

`skeleton()` lays out the shipped needle3.cact exactly as its directory
fixture records it (every offset and size) with zero-filled blobs;
`pack_synth()` writes a random-init model's canonical records.
"""
import json
import os
import struct

import numpy as np

TAG_V3 = 0x05E12A84
HEADER_BYTES = 49 * 4
REC_BYTES = 44
FP16, FP32, CQ, RAW = 1, 2, 3, 4
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden(name):
    return json.load(open(os.path.join(GOLDEN, name)))


def header_words(g, num_tensors):
    """The 49 header words for a geometry in the fixture's key names."""
    w = [0] * 49
    w[0], w[1], w[2] = TAG_V3, num_tensors, 28
    w[3], w[4] = g.get("kv_window", 256), g.get("kv_bits", 8)
    for k, key in enumerate(("vocab_size", "out_vocab", "d_model", "num_heads", "num_kv_heads",
                             "num_layers", "qk_head_dim", "v_head_dim", "max_seq_len", "hada_n",
                             "mhc_lanes", "sliding_window")):
        w[5 + k] = g[key]
    mask = sum(1 << layer for layer in g["global_layers"])
    w[17], w[18] = mask & 0xFFFFFFFF, mask >> 32
    w[19] = g["qkv_conv_taps"]
    w[20], w[21], w[22] = g["engram_slots"], g["engram_sub_dim"], g["num_engram_tables"]
    w[23], w[24], w[25] = g["engram_conv_taps"], g["engram_conv_dilation"], g["engram_seed_heads"]
    w[26] = len(g["engram_orders"])
    for k, o in enumerate(g["engram_orders"][:4]):
        w[27 + k] = o
    w[31] = len(g["engram_layers"])
    for k, s in enumerate(g["engram_layers"][:16]):
        w[32 + k] = s
    w[48] = struct.unpack("<I", struct.pack("<f", g["rope_theta"]))[0]
    return w


def fixture_geometry(synth_geom):
    """A v3_synth geometry in the fixture's key names."""
    g = synth_geom
    return dict(vocab_size=g["vocab_size"], out_vocab=g["out_vocab"], d_model=g["d_model"],
                num_heads=g["num_heads"], num_kv_heads=g["num_kv_heads"],
                num_layers=g["num_layers"], qk_head_dim=g["qk_head_dim"],
                v_head_dim=g["v_head_dim"], max_seq_len=g["max_seq_len"], hada_n=g["hada_n"],
                mhc_lanes=g["mhc_lanes"], sliding_window=g["sliding_window"],
                global_layers=list(g["global_layers"]), qkv_conv_taps=g["qkv_conv_taps"],
                engram_slots=g["e_slots"], engram_sub_dim=g["e_sub_dim"],
                num_engram_tables=len(g["orders"]) * g["e_heads"],
                engram_conv_taps=g["e_conv_taps"], engram_conv_dilation=g["e_conv_dilation"],
                engram_seed_heads=g["e_seed_heads"], engram_orders=list(g["orders"]),
                engram_layers=list(g["sites"]), rope_theta=g["rope_theta"])


def _record(dtype, shape, offset, nbytes, group=0, bits=0):
    shape = list(shape)[:4]
    dims = shape + [0] * (4 - len(shape))
    return struct.pack("<BBH4IQQII", dtype, len(shape), 0, *dims, offset, nbytes, group, bits)


def assemble(geom, codebook, tensors, offsets=None, total=None):
    """tensors: (dtype, shape, group, bits, bytes or None for zeros, nbytes)."""
    n = len(tensors)
    head = struct.pack("<49I", *header_words(geom, n))
    cb = np.asarray(codebook, np.float32).astype("<f4").tobytes()
    dir_end = HEADER_BYTES + len(cb) + n * REC_BYTES
    if offsets is None:
        offsets, at = [], -(-dir_end // 64) * 64
        for t in tensors:
            offsets.append(at)
            at = -(-(at + t[5]) // 64) * 64
        total = offsets[-1] + tensors[-1][5] if tensors else dir_end
    out = bytearray(total)
    out[:HEADER_BYTES] = head
    out[HEADER_BYTES:HEADER_BYTES + len(cb)] = cb
    for i, (dtype, shape, group, bits, data, nbytes) in enumerate(tensors):
        at = HEADER_BYTES + len(cb) + i * REC_BYTES
        out[at:at + REC_BYTES] = _record(dtype, shape, offsets[i], nbytes, group, bits)
        if data is not None:
            out[offsets[i]:offsets[i] + nbytes] = data
    return bytes(out)


def skeleton():
    """The shipped needle3.cact's header and directory (the reference's
    fixture), blobs zero-filled."""
    geo = _golden("v3_geometry.json")["geometry"]
    d = _golden("v3_directory.json")
    cb = _golden("cq_codebook.json")["codebook"]
    tensors, offsets = [], []
    for idx, dtype, ndim, shape, offset, nbytes, group, bits in d["records"]:
        tensors.append((dtype, shape[:ndim], group, bits, None, nbytes))
        offsets.append(offset)
    return assemble(geo, cb, tensors, offsets, d["container_bytes"])


def set_word(data, i, value):
    b = bytearray(data)
    b[4 * i:4 * i + 4] = struct.pack("<I", value)
    return bytes(b)


def set_record(data, index, **fields):
    """Rewrites fields of directory record `index` (dtype, ndim, shape,
    offset, nbytes)."""
    b = bytearray(data)
    at = HEADER_BYTES + 28 * 4 + index * REC_BYTES
    dtype, ndim, _, s0, s1, s2, s3, off, nb, group, bits = struct.unpack(
        "<BBH4IQQII", bytes(b[at:at + REC_BYTES]))
    shape = fields.get("shape", [s0, s1, s2, s3][:ndim])
    dims = list(shape) + [0] * (4 - len(shape))
    b[at:at + REC_BYTES] = struct.pack(
        "<BBH4IQQII", fields.get("dtype", dtype), fields.get("ndim", len(shape)), 0, *dims,
        fields.get("offset", off), fields.get("nbytes", nb), group, bits)
    return bytes(b)


def pack_synth(geom, records, codebook):
    """A container of v3_synth records: CQ blobs as stored, the Hadamard
    permutations as FP32, every other float tensor as FP16, then a heads
    manifest, one head tensor and a RAW record, which a reader must not need.
    Returns (bytes, records with the floats the container holds)."""
    tensors, held = [], []
    for r in records:
        if r["kind"] == CQ:
            data = np.ascontiguousarray(r["data"], np.uint8).tobytes()
            tensors.append((CQ, [r["out"], r["inn"]], r["group"], r["bits"], data, len(data)))
            held.append(r)
            continue
        arr = np.asarray(r["data"], np.float32)
        shape = list(arr.shape) if arr.ndim else [1]
        if r["name"] == "b_res":  # stored [L][n][n], as the shipped container has it
            n = int(round(np.sqrt(arr.shape[1])))
            shape = [arr.shape[0], n, n]
        if "perm" in r["name"]:
            data = arr.astype("<f4").tobytes()
            tensors.append((FP32, shape, 0, 0, data, len(data)))
            kept = arr
        else:
            h = arr.astype(np.float16)
            data = h.astype("<f2").tobytes()
            tensors.append((FP16, shape, 0, 0, data, len(data)))
            kept = h.astype(np.float32)
        held.append(dict(r, data=np.ascontiguousarray(kept, np.float32)))
    tensors.append((FP16, [1], 0, 0, np.array([2], np.float16).tobytes(), 2))
    tensors.append((FP16, [3, 4], 0, 0, np.zeros(12, np.float16).tobytes(), 24))
    tok = b"tokenizer bytes"
    tensors.append((RAW, [], 0, 0, tok, len(tok)))
    return assemble(fixture_geometry(geom), codebook, tensors), held
