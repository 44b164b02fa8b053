"""Synthetic Cactus-Quants tensors, built the way needle-rs's own unit tests
build them (crates/needle-core/src/cq.rs:973-1088): a monotone fake codebook,
indices packed LSB-first by an independent bit packer, FP16 norms, and a
dense reconstruction `w_g = (levels[idx] * norm) @ H` computed with a dense
Sylvester matrix -- not with the butterfly under test.
"""
from __future__ import annotations

import math

import numpy as np

TERNARY = 5
TERNARY_CENTROID = np.float32(1.2240064)
WIDTHS = (2, 3, 4, TERNARY)


def fake_codebook(group: int) -> np.ndarray:
    """cq.rs:973-986: cb2|cb3|cb4, monotone, scaled by 1/sqrt(group)."""
    s = np.float32(1.0) / np.float32(math.sqrt(group))
    cb = []
    for bits in (2, 3, 4):
        levels = 1 << bits
        for i in range(levels):
            v = (np.float32(i) - (np.float32(levels) - np.float32(1.0)) / np.float32(2.0)) / (
                np.float32(levels) / np.float32(2.0))
            cb.append(np.float32(v) * s)
    return np.array(cb, np.float32)


def levels_for(bits: int, group: int, codebook: np.ndarray) -> np.ndarray:
    if bits == TERNARY:
        s = TERNARY_CENTROID / np.float32(math.sqrt(group))
        return np.array([-s, 0.0, s], np.float32)
    off = {2: 0, 3: 4, 4: 12}[bits]
    return codebook[off:off + (1 << bits)].astype(np.float32)


def pack_lsb(idx: np.ndarray, out: int, in_pad: int, bits: int) -> np.ndarray:
    """cq.rs:989-1005: index k of a row occupies bits [k*bits, (k+1)*bits)."""
    idx = idx.reshape(out, in_pad).astype(np.uint32)
    bitarr = np.stack([(idx >> b) & 1 for b in range(bits)], axis=2)  # [out, in_pad, bits]
    bitarr = bitarr.reshape(out, in_pad * bits).astype(np.uint8)
    return np.packbits(bitarr, axis=1, bitorder="little").reshape(-1)


def f32_to_f16_trunc(v: float) -> int:
    """cq.rs:1007-1020: the test helper's truncating narrowing."""
    x = int(np.array(v, np.float32).view(np.uint32))
    sign = (x >> 31) << 15
    exp = ((x >> 23) & 0xFF) - 127
    mant = x & 0x7FFFFF
    if exp < -14:
        return sign
    if exp > 15:
        return sign | 0x7C00
    return sign | ((exp + 15) << 10) | (mant >> 13)


def sylvester(n: int) -> np.ndarray:
    h = np.ones((1, 1), np.float64)
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def f16_bits_to_f32(b: int) -> np.float32:
    return np.array([b], np.uint16).view(np.float16).astype(np.float32)[0]


class Case:
    pass


def build_case(out: int, in_feat: int, group: int, bits: int, codebook=None,
               idx=None, norms=None) -> Case:
    """cq.rs:1028-1088, optionally with caller-supplied codebook, indices and
    norms (random draws for the GPU tests)."""
    cb = fake_codebook(group) if codebook is None else np.asarray(codebook, np.float32)
    levels = levels_for(bits, group, cb)
    n_levels = levels.size
    in_pad = -(-in_feat // group) * group
    num_groups = in_pad // group
    if idx is None:
        i = np.arange(out * in_pad)
        idx = ((i * 7 + i // 13) % n_levels).astype(np.uint8)
    idx = np.asarray(idx, np.uint8).reshape(-1)
    if norms is None:
        norms = np.array([0.25 + (i % 11) * 0.125 for i in range(out * num_groups)], np.float32)
    if bits == TERNARY:
        crumbs = np.where(idx == 0, 3, idx - 1).astype(np.uint8)
        packed = pack_lsb(crumbs, out, in_pad, 2)
    else:
        packed = pack_lsb(idx, out, in_pad, bits)
    n16 = np.array([f32_to_f16_trunc(float(n)) for n in norms], np.uint16)
    blob = np.concatenate([packed, n16.view(np.uint8)])

    H = sylvester(group) / math.sqrt(group)
    normf = np.array([f16_bits_to_f32(int(b)) for b in n16], np.float64).reshape(out, num_groups)
    u = levels.astype(np.float64)[idx.reshape(out, num_groups, group)] * normf[:, :, None]
    dense = np.einsum("ogk,kj->ogj", u, H).reshape(out, in_pad)[:, :in_feat]

    c = Case()
    c.blob, c.codebook, c.levels, c.idx = blob, cb, levels, idx.reshape(out, in_pad)
    c.norms_f32 = normf.astype(np.float32)
    c.out, c.in_feat, c.in_pad, c.group, c.bits = out, in_feat, in_pad, group, bits
    c.num_groups = num_groups
    c.dense = dense  # float64 [out, in_feat]
    return c


def random_case(rng, out, in_feat, group, bits, codebook):
    """A CQ tensor with uniform random codes and N(0, 0.02)*sqrt(group) norms."""
    levels = levels_for(bits, group, np.asarray(codebook, np.float32))
    in_pad = -(-in_feat // group) * group
    idx = rng.integers(0, levels.size, size=out * in_pad).astype(np.uint8)
    norms = np.abs(rng.normal(0.0, 0.02, size=out * (in_pad // group))) * math.sqrt(group)
    return build_case(out, in_feat, group, bits, codebook=codebook, idx=idx,
                      norms=norms.astype(np.float32))
