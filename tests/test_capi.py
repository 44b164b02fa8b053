"""The C ABI library loads and exports every entry point include/needle_amd.h
declares; host-only functions (KV block layout) and the error path work
without a GPU.  No kernel is launched here."""
import ctypes as C

import numpy as np
import pytest

import needle_amd as nd


def test_header_symbols_all_exported():
    L = nd.lib()
    names = nd.header_symbols()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # The ctypes signature table covers the header exactly.
    assert sorted(n for n, _, _ in nd._SIGS) == names


def test_no_error_before_any_failure():
    assert nd.last_error() is None or isinstance(nd.last_error(), str)


def test_kv_block_layout_v3_and_mha():
    g = nd.kv_geom(12, 2, 48, 64, 1024)
    off = nd.kv_offsets(g)
    assert off["v"] == 2 * 1024 * 48
    assert off["ks"] == off["v"] + 2 * 1024 * 64
    assert off["vs"] == off["ks"] + 2 * 1024 * 4
    assert off["total"] == off["vs"] + 2 * 1024 * 4
    # int8 bytes per position per layer match kv_bytes_at (config.rs:162-179):
    # kv_heads*(qk+v) + kv_heads*8 = 240 for the shipped geometry.
    assert off["total"] // 1024 == 2 * (48 + 64) + 2 * 8
    g = nd.kv_geom(12, 12, 64, 64, 2048)
    assert nd.kv_block_bytes(g) == 2048 * (12 * 128 + 12 * 8)
    for off_v in nd.kv_offsets(nd.kv_geom(4, 2, 48, 64, 17)).values():
        assert off_v % 256 == 0


def test_kv_f32_block_layout():
    """f32 blocks: k [kvh][cap][qk] then v [kvh][cap][vd], 256-aligned; per
    position per layer kv_heads*(qk+v)*4 bytes, as kv_bytes_at counts an f32
    cache (config.rs:162-179)."""
    g = nd.kv_geom(12, 2, 48, 64, 1000)
    v_off = (2 * 1000 * 48 * 4 + 255) // 256 * 256
    assert nd.lib().nd_kv_f32_v_offset(g) == v_off
    assert nd.kv_f32_block_bytes(g) == v_off + (2 * 1000 * 64 * 4 + 255) // 256 * 256
    g = nd.kv_geom(12, 2, 48, 64, 1024)
    assert nd.kv_f32_block_bytes(g) // 1024 == 2 * (48 + 64) * 4
    g = nd.kv_geom(4, 2, 48, 64, 17)
    assert nd.lib().nd_kv_f32_v_offset(g) % 256 == 0 and nd.kv_f32_block_bytes(g) % 256 == 0


def test_ctx_create_reports_error_without_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = C.c_void_p()
    rc = nd.lib().nd_ctx_create(0, C.byref(h))
    assert rc != nd.ND_OK
    msg = nd.last_error()
    assert msg and len(msg) > 0
    assert not h.value


def test_null_context_is_an_argument_error():
    rc = nd.lib().nd_ctx_synchronize(None)
    assert rc == 1 and "context" in nd.last_error()
