"""Python mirror of needle-rs's hot-path operator interface over the C ABI
(include/needle_amd.h), for callers that hold torch device tensors.

Names follow the reference: CqWeight.{prepare_input, matvec_rows_prepared,
matmul_rows_prepared, dequantize_row} (crates/needle-core/src/cq.rs),
fake_quant_vec / quantize_rows / V3Cache.write_kv / span
(v3/cache.rs), attend_step / attend (v3/attention.rs).  Every call goes
through libneedle_amd.so; there is no CPU fallback -- a missing library or
GPU raises.  torch supplies device memory and the stream only.
"""
from __future__ import annotations

import ctypes as C
import math
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libneedle_amd.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "needle_amd.h")

ND_OK = 0
ND_ERR_ARG, ND_ERR_CACT, ND_ERR_V3_GEOMETRY, ND_ERR_V3_LAYOUT = 1, 20, 21, 22
ERRORS = {1: "ND_ERR_ARG", 2: "ND_ERR_HIP", 3: "ND_ERR_NOMEM", 4: "ND_ERR_BUSY", 11: "UnsupportedBits",
          12: "BadGroup", 13: "BadCodebookLen", 14: "ShortBlob", 15: "EmptyShape",
          20: "CactError", 21: "V3GeometryError", 22: "V3LayoutError"}


class NeedleError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{ERRORS.get(code, code)}: {msg}")
        self.code = code


class KvGeom(C.Structure):
    _fields_ = [("num_heads", C.c_int32), ("num_kv_heads", C.c_int32),
                ("qk_head_dim", C.c_int32), ("v_head_dim", C.c_int32), ("cap", C.c_int32)]


_lib = None
_vp, _sz = C.c_void_p, C.c_size_t

# (name, restype, argtypes) for every entry point of include/needle_amd.h.
_SIGS = [
    ("nd_last_error", C.c_char_p, []),
    ("nd_ctx_create", C.c_int, [C.c_int, C.POINTER(_vp)]),
    ("nd_ctx_create_on_stream", C.c_int, [C.c_int, _vp, C.POINTER(_vp)]),
    ("nd_ctx_destroy", None, [_vp]),
    ("nd_ctx_synchronize", C.c_int, [_vp]),
    ("nd_malloc", C.c_int, [_vp, _sz, C.POINTER(_vp)]),
    ("nd_free", C.c_int, [_vp, _vp]),
    ("nd_memcpy_htod", C.c_int, [_vp, _vp, _vp, _sz]),
    ("nd_memcpy_dtoh", C.c_int, [_vp, _vp, _vp, _sz]),
    ("nd_cb8_gemv", C.c_int, [_vp, _vp, _vp, _vp, _vp, _sz, _sz]),
    ("nd_cb8_gemv_batched", C.c_int, [_vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz]),
    ("nd_cb8_gemm", C.c_int, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz]),
    ("nd_cb8_gemm_batched", C.c_int, [_vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz]),
    ("nd_cq_from_blob", C.c_int, [_vp, _vp, _sz, _sz, _sz, _sz, C.c_uint8, _vp, _sz, C.POINTER(_vp)]),
    ("nd_cq_free", None, [_vp]),
    ("nd_cq_shape", C.c_int, [_vp, C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_sz),
                              C.POINTER(C.c_uint8)]),
    ("nd_cq_prepare_input", C.c_int, [_vp, _vp, _vp, _sz, _vp]),
    ("nd_cq_matvec_rows_prepared", C.c_int, [_vp, _vp, _vp, _sz, _sz, _vp]),
    ("nd_cq_matmul_rows_prepared", C.c_int, [_vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    ("nd_cq_matvec_rows_exact", C.c_int, [_vp, _vp, _vp, _sz, _sz, _vp]),
    ("nd_cq_matmul_rows_exact", C.c_int, [_vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    ("nd_cq_dequantize_rows", C.c_int, [_vp, _vp, _vp, _sz, _vp]),
    ("nd_fold_rows", C.c_int, [_vp, _vp, _sz, _sz, _vp]),
    ("nd_fake_quant", C.c_int, [_vp, _vp, _sz, _sz]),
    ("nd_quantize_rows", C.c_int, [_vp, _vp, _sz, _sz, _vp, _vp]),
    ("nd_kv_block_bytes", _sz, [C.POINTER(KvGeom)]),
    ("nd_kv_v_offset", _sz, [C.POINTER(KvGeom)]),
    ("nd_kv_ks_offset", _sz, [C.POINTER(KvGeom)]),
    ("nd_kv_vs_offset", _sz, [C.POINTER(KvGeom)]),
    ("nd_kv_write", C.c_int, [_vp, C.POINTER(KvGeom), _vp, _sz, _sz, _vp, _vp, _vp]),
    ("nd_attend_step_i8", C.c_int, [_vp, C.POINTER(KvGeom), _vp, _sz, _sz, _vp, _vp, _vp,
                                    C.c_float, C.c_int, _vp]),
    ("nd_attend_step_i8_exact", C.c_int, [_vp, C.POINTER(KvGeom), _vp, _sz, _sz, _vp, _vp, _vp,
                                          C.c_float, C.c_int, _vp]),
    ("nd_attend_step_i8_noalloc", C.c_int, [_vp, C.POINTER(KvGeom), _vp, _sz, _sz, _vp, _vp, _vp,
                                            C.c_float, C.c_int, _vp]),
    ("nd_v3_model_create", C.c_int, [_vp, _vp, _vp, _sz, _vp, _sz, C.POINTER(_vp)]),
    ("nd_v3_model_free", None, [_vp]),
    ("nd_v3_logit_rows", _sz, [_vp]),
    ("nd_v3_batch_create", C.c_int, [_vp, _vp, _sz, _sz, _sz, C.POINTER(_vp)]),
    ("nd_v3_batch_free", None, [_vp]),
    ("nd_v3_positions", C.c_int, [_vp, _vp]),
    ("nd_v3_step", C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp]),
    ("nd_argmax_rows", C.c_int, [_vp, _vp, _sz, _sz, _vp]),
    ("nd_v3_batch_create_chunked", C.c_int, [_vp, _vp, _sz, _sz, _sz, _sz, C.POINTER(_vp)]),
    ("nd_v3_prefill", C.c_int, [_vp, _vp, _vp, _vp, _sz, _vp, _vp]),
    ("nd_v3_generate", C.c_int, [_vp, _vp, _vp, _vp, _sz, _vp]),
    ("nd_v3_generate_many", C.c_int, [_vp, _vp, _vp, _sz, _vp, _sz, _vp]),
    ("nd_v3_cact_config", C.c_int, [_vp, _sz, _vp, C.POINTER(_sz)]),
    ("nd_v3_model_from_cact", C.c_int, [_vp, _vp, _sz, C.POINTER(_vp)]),
    ("nd_v3_batch_set_graphs", C.c_int, [_vp, C.c_int]),
    ("nd_v3_kv_bytes", _sz, [_vp, _sz, C.c_int]),
    ("nd_v3_ladder", C.c_int, [_sz, _sz, C.POINTER(C.c_int32)]),
    ("nd_v3_cact_config_at_depth", C.c_int, [_vp, _sz, _sz, _vp, C.POINTER(C.c_int32)]),
    ("nd_v3_model_from_cact_at_depth", C.c_int, [_vp, _vp, _sz, _sz, C.POINTER(_vp)]),
    ("nd_kv_f32_block_bytes", _sz, [C.POINTER(KvGeom)]),
    ("nd_kv_f32_v_offset", _sz, [C.POINTER(KvGeom)]),
    ("nd_kv_write_f32", C.c_int, [_vp, C.POINTER(KvGeom), _vp, _sz, _sz, _vp, _vp, _vp]),
    ("nd_attend_step_f32_exact", C.c_int, [_vp, C.POINTER(KvGeom), _vp, _sz, _sz, _vp, _vp, _vp,
                                           C.c_float, _vp]),
    ("nd_v3_batch_create_ex", C.c_int, [_vp, _vp, _sz, _sz, _sz, _sz, C.c_int, C.POINTER(_vp)]),
    ("nd_libm_map", C.c_int, [_vp, C.c_int, _vp, _sz, _vp]),
]


def header_symbols():
    """Function names declared in include/needle_amd.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nd_[a-z0-9_]+)\s*\(", text)))


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `make -C needle-rs_amd` "
                               "(or __graft_entry__.build()); there is no CPU fallback")
        L = C.CDLL(LIB_PATH)
        for name, res, args in _SIGS:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error():
    m = lib().nd_last_error()
    return m.decode() if m else None


def _check(rc):
    if rc != ND_OK:
        raise NeedleError(rc, last_error())


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else C.c_void_p(0)


def _arg(t, dtype, name, numel=0, rows=False):
    """The device pointer of tensor `t` once it is a device tensor of `dtype`
    holding at least `numel` elements, contiguous (with rows=True: each
    slice t[i] contiguous, for the strided batched calls).  The library
    reads exactly the bytes its sizes imply, so a wrong dtype or layout
    would read past the buffer or in the wrong order: raise instead."""
    if not t.is_cuda:
        raise ValueError(f"{name}: a device tensor is required")
    if t.dtype != dtype:
        raise ValueError(f"{name}: dtype {t.dtype}, expected {dtype}")
    ok = (t.dim() == 0 or all(t[i].is_contiguous() for i in range(min(t.shape[0], 1)))) \
        if rows else t.is_contiguous()
    if rows and t.dim() > 1:
        ok = ok and t.stride(0) >= t[0].numel()
    if not ok:
        raise ValueError(f"{name}: layout {tuple(t.shape)} strides {t.stride()} is not contiguous")
    if t.numel() < numel:
        raise ValueError(f"{name}: {t.numel()} elements, at least {numel} needed")
    return C.c_void_p(t.data_ptr())


def _torch():
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("no GPU visible: the HIP path has no CPU fallback")
    return torch


class Ctx:
    """nd_ctx bound to a device and to torch's current stream on it."""

    def __init__(self, device=0, stream=None):
        torch = _torch()
        self.device = device
        if stream is None:
            stream = torch.cuda.current_stream(device)
        self.stream = stream
        h = C.c_void_p()
        _check(lib().nd_ctx_create_on_stream(device, C.c_void_p(stream.cuda_stream), C.byref(h)))
        self.h = h

    def synchronize(self):
        _check(lib().nd_ctx_synchronize(self.h))

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.nd_ctx_destroy(self.h)
            self.h = None

    __del__ = close


# ---- Format B ---------------------------------------------------------------

def cb8_gemv(ctx, w, cb, x, y=None):
    torch = _torch()
    out, inn = w.shape
    if y is None:
        y = torch.empty(out, dtype=torch.float32, device=w.device)
    f32 = torch.float32
    _check(lib().nd_cb8_gemv(ctx.h, _arg(w, torch.uint8, "w"),
                             _arg(cb, f32, "cb", (out + 63) // 64 * 256), _arg(x, f32, "x", inn),
                             _arg(y, f32, "y", out), out, inn))
    return y


def cb8_gemv_batched(ctx, w, cb, x, y):
    """w [count, out, in] u8, cb [count, out/64, 256], x [count, in], y [count, out]."""
    torch = _torch()
    count, out, inn = w.shape
    f32 = torch.float32
    _check(lib().nd_cb8_gemv_batched(
        ctx.h, count, _arg(w, torch.uint8, "w", rows=True), w.stride(0),
        _arg(cb, f32, "cb", rows=True), cb.stride(0), _arg(x, f32, "x", rows=True), x.stride(0),
        _arg(y, f32, "y", rows=True), y.stride(0), out, inn))
    return y


def cb8_gemm(ctx, x, w, cb, y=None):
    torch = _torch()
    m, inn = x.shape
    out = w.shape[0]
    if y is None:
        y = torch.empty(m, out, dtype=torch.float32, device=x.device)
    f32 = torch.float32
    _check(lib().nd_cb8_gemm(ctx.h, _arg(x, f32, "x"), _arg(w, torch.uint8, "w", out * inn),
                             _arg(cb, f32, "cb", (out + 63) // 64 * 256), _arg(y, f32, "y", m * out),
                             m, out, inn))
    return y


def cb8_gemm_batched(ctx, x, w, cb, y):
    """x [count][m][in] f32, w [count][out][in] u8, cb [count][out/64][256],
    y [count][m][out]: one launch."""
    torch = _torch()
    count, m, inn = x.shape
    out = w.shape[1]
    f32 = torch.float32
    _check(lib().nd_cb8_gemm_batched(
        ctx.h, count, _arg(x, f32, "x", rows=True), x.stride(0),
        _arg(w, torch.uint8, "w", rows=True), w.stride(0), _arg(cb, f32, "cb", rows=True),
        cb.stride(0), _arg(y, f32, "y", rows=True), y.stride(0), m, out, inn))
    return y


# ---- Format A ---------------------------------------------------------------

class CqWeight:
    """Device CqWeight (cq.rs:117-810) built from a host blob."""

    def __init__(self, ctx, blob, out_feat, in_feat, group, bits, codebook):
        self.ctx = ctx
        blob = np.ascontiguousarray(blob, np.uint8)
        cb = np.ascontiguousarray(codebook, np.float32)
        h = C.c_void_p()
        _check(lib().nd_cq_from_blob(ctx.h, blob.ctypes.data_as(C.c_void_p), blob.size, out_feat,
                                     in_feat, group, bits, cb.ctypes.data_as(C.c_void_p), cb.size,
                                     C.byref(h)))
        self.h = h
        o, i, p, g, b = _sz(), _sz(), _sz(), _sz(), C.c_uint8()
        _check(lib().nd_cq_shape(h, C.byref(o), C.byref(i), C.byref(p), C.byref(g), C.byref(b)))
        self.out_feat, self.in_feat, self.in_padded = o.value, i.value, p.value
        self.group, self.bits = g.value, b.value

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.nd_cq_free(self.h)
            self.h = None

    __del__ = close

    def prepare_input(self, x, xh=None):
        torch = _torch()
        x2 = x.reshape(-1, self.in_feat)
        if xh is None:
            xh = torch.empty(x2.shape[0], self.in_padded, dtype=torch.float32, device=x.device)
        n = x2.shape[0]
        _check(lib().nd_cq_prepare_input(self.ctx.h, self.h, _arg(x2, torch.float32, "x"), n,
                                         _arg(xh, torch.float32, "xh", n * self.in_padded)))
        return xh

    def matvec_rows_prepared(self, xh, row_start, rows, y=None, exact=False):
        """exact=True: the reference's summation order, bit-identical."""
        torch = _torch()
        if y is None:
            y = torch.empty(rows, dtype=torch.float32, device=xh.device)
        fn = lib().nd_cq_matvec_rows_exact if exact else lib().nd_cq_matvec_rows_prepared
        _check(fn(self.ctx.h, self.h, _arg(xh, torch.float32, "xh", self.in_padded), row_start,
                  rows, _arg(y, torch.float32, "y", rows)))
        return y

    def matvec_prepared(self, xh, y=None):
        return self.matvec_rows_prepared(xh, 0, self.out_feat, y)

    def matvec(self, x):
        return self.matvec_prepared(self.prepare_input(x))

    def matmul_rows_prepared(self, xh, batch, row_start, rows, y=None, exact=False):
        """exact=True: the reference's summation order, bit-identical."""
        torch = _torch()
        if y is None:
            y = torch.empty(batch * rows, dtype=torch.float32, device=xh.device)
        fn = lib().nd_cq_matmul_rows_exact if exact else lib().nd_cq_matmul_rows_prepared
        _check(fn(self.ctx.h, self.h, _arg(xh, torch.float32, "xh", batch * self.in_padded),
                  batch, row_start, rows, _arg(y, torch.float32, "y", batch * rows)))
        return y

    def dequantize_rows(self, rows_i32, out=None):
        torch = _torch()
        n = rows_i32.numel()
        if out is None:
            out = torch.empty(n, self.in_feat, dtype=torch.float32, device=rows_i32.device)
        _check(lib().nd_cq_dequantize_rows(self.ctx.h, self.h, _arg(rows_i32, torch.int32, "rows"),
                                           n, _arg(out, torch.float32, "out", n * self.in_feat)))
        return out


# ---- int8 KV ----------------------------------------------------------------

def fold_rows(ctx, x, y=None):
    """y[r] = the sequential fp32 sum of row r of x ([rows][n], n <= 4096),
    in the reference's order (kernels.rs:22-24, v3/attention.rs:361-365)."""
    torch = _torch()
    rows, n = x.shape
    if y is None:
        y = torch.empty(rows, dtype=torch.float32, device=x.device)
    _check(lib().nd_fold_rows(ctx.h, _arg(x, torch.float32, "x"), rows, n,
                              _arg(y, torch.float32, "y", rows)))
    return y


def argmax_rows(ctx, x, out=None):
    """The greedy token of each row of x ([count][n] fp32): the first maximum
    (needle-infer/src/v3_engine.rs:410-420)."""
    torch = _torch()
    count, n = x.shape
    if out is None:
        out = torch.empty(count, dtype=torch.int32, device=x.device)
    _check(lib().nd_argmax_rows(ctx.h, _arg(x, torch.float32, "x"), count, n,
                                _arg(out, torch.int32, "out", count)))
    return out


LIBM = {"expf": 0, "logf": 1, "sigmoid": 2}


def libm_map(ctx, fn, x, y=None):
    """The device copy of the reference's libm wrapper `fn` ("expf", "logf",
    "sigmoid"; math.rs:3-46) applied to every element of x (fp32)."""
    torch = _torch()
    if y is None:
        y = torch.empty_like(x)
    n = x.numel()
    _check(lib().nd_libm_map(ctx.h, LIBM[fn], _arg(x, torch.float32, "x"), n,
                             _arg(y, torch.float32, "y", n)))
    return y


def fake_quant(ctx, x, dim):
    """fake_quant_vec(x[r], 8) for every row of `dim`, in place."""
    torch = _torch()
    _check(lib().nd_fake_quant(ctx.h, _arg(x, torch.float32, "x"), x.numel() // dim, dim))
    return x


def quantize_rows(ctx, x, head_dim):
    torch = _torch()
    rows = x.numel() // head_dim
    ints = torch.empty(rows * head_dim, dtype=torch.int8, device=x.device)
    scales = torch.empty(rows, dtype=torch.float32, device=x.device)
    _check(lib().nd_quantize_rows(ctx.h, _arg(x, torch.float32, "x"), rows, head_dim, _ptr(ints),
                                  _ptr(scales)))
    return ints, scales


def kv_geom(num_heads, num_kv_heads, qk, vd, cap):
    return KvGeom(num_heads, num_kv_heads, qk, vd, cap)


def kv_block_bytes(g):
    return lib().nd_kv_block_bytes(C.byref(g))


def kv_offsets(g):
    L = lib()
    return dict(v=L.nd_kv_v_offset(C.byref(g)), ks=L.nd_kv_ks_offset(C.byref(g)),
                vs=L.nd_kv_vs_offset(C.byref(g)), total=L.nd_kv_block_bytes(C.byref(g)))


def kv_alloc(g, count=1, device=0):
    """`count` zeroed KV blocks, one after another (stride = block bytes)."""
    torch = _torch()
    nb = kv_block_bytes(g)
    return torch.zeros(count * nb, dtype=torch.uint8, device=device), nb


def kv_write(ctx, g, kv, kv_stride, pos_i32, k, v):
    torch = _torch()
    n = pos_i32.numel()
    blocks = kv_block_bytes(g) + (n - 1) * kv_stride if n else 0
    _check(lib().nd_kv_write(
        ctx.h, C.byref(g), _arg(kv, torch.uint8, "kv", blocks), kv_stride, n,
        _arg(pos_i32, torch.int32, "pos"),
        _arg(k, torch.float32, "k", n * g.num_kv_heads * g.qk_head_dim),
        _arg(v, torch.float32, "v", n * g.num_kv_heads * g.v_head_dim)))


def attend_step_i8(ctx, g, kv, kv_stride, lo_i32, hi_i32, q, scale=None, quant_query=False,
                   out=None, exact=False, noalloc=False):
    """exact=True: nd_attend_step_i8_exact, bit-identical to attend_step.
    noalloc=True: nd_attend_step_i8_noalloc (no device allocation; split-K
    partials in the library's fixed per-GPU array)."""
    torch = _torch()
    count = lo_i32.numel()
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(g.qk_head_dim)))
    if out is None:
        out = torch.empty(count, g.num_heads * g.v_head_dim, dtype=torch.float32, device=q.device)
    fn = lib().nd_attend_step_i8_exact if exact else lib().nd_attend_step_i8
    if noalloc:
        if exact:
            raise ValueError("the no-allocation entry point is the tolerance-order kernel")
        fn = lib().nd_attend_step_i8_noalloc
    blocks = kv_block_bytes(g) + (count - 1) * kv_stride if count else 0
    i32, f32 = torch.int32, torch.float32
    _check(fn(ctx.h, C.byref(g), _arg(kv, torch.uint8, "kv", blocks), kv_stride, count,
              _arg(lo_i32, i32, "lo"), _arg(hi_i32, i32, "hi", count),
              _arg(q, f32, "q", count * g.num_heads * g.qk_head_dim), scale,
              int(bool(quant_query)), _arg(out, f32, "out", count * g.num_heads * g.v_head_dim)))
    return out


# ---- f32 KV (KvPrecision::F32) ----------------------------------------------

def kv_f32_block_bytes(g):
    return lib().nd_kv_f32_block_bytes(C.byref(g))


def kv_alloc_f32(g, count=1, device=0):
    """`count` zeroed f32 KV blocks, one after another (stride = block bytes)."""
    torch = _torch()
    nb = kv_f32_block_bytes(g)
    return torch.zeros(count * nb, dtype=torch.uint8, device=device), nb


def kv_write_f32(ctx, g, kv, kv_stride, pos_i32, k, v):
    """V3Cache::write_kv with KvPrecision::F32 (cache.rs:359-362)."""
    torch = _torch()
    n = pos_i32.numel()
    blocks = kv_f32_block_bytes(g) + (n - 1) * kv_stride if n else 0
    _check(lib().nd_kv_write_f32(
        ctx.h, C.byref(g), _arg(kv, torch.uint8, "kv", blocks), kv_stride, n,
        _arg(pos_i32, torch.int32, "pos"),
        _arg(k, torch.float32, "k", n * g.num_kv_heads * g.qk_head_dim),
        _arg(v, torch.float32, "v", n * g.num_kv_heads * g.v_head_dim)))


def attend_step_f32(ctx, g, kv, kv_stride, lo_i32, hi_i32, q, scale=None, out=None):
    """attend_step over KvStore::F32 (attention.rs:166-189, 327-377),
    bit-identical (nd_attend_step_f32_exact)."""
    torch = _torch()
    count = lo_i32.numel()
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(g.qk_head_dim)))
    if out is None:
        out = torch.empty(count, g.num_heads * g.v_head_dim, dtype=torch.float32, device=q.device)
    blocks = kv_f32_block_bytes(g) + (count - 1) * kv_stride if count else 0
    i32, f32 = torch.int32, torch.float32
    _check(lib().nd_attend_step_f32_exact(
        ctx.h, C.byref(g), _arg(kv, torch.uint8, "kv", blocks), kv_stride, count,
        _arg(lo_i32, i32, "lo"), _arg(hi_i32, i32, "hi", count),
        _arg(q, f32, "q", count * g.num_heads * g.qk_head_dim), scale,
        _arg(out, f32, "out", count * g.num_heads * g.v_head_dim)))
    return out


def kv_unpack_f32(g, block_u8):
    """One f32 device block (CPU uint8 numpy array) as the reference's
    slot-major views: k [cap][kvh][qk] f32, v [cap][kvh][vd]."""
    H, cap, qk, vd = g.num_kv_heads, g.cap, g.qk_head_dim, g.v_head_dim
    vo = lib().nd_kv_f32_v_offset(C.byref(g))
    b = np.asarray(block_u8)
    k = b[:4 * H * cap * qk].view(np.float32).reshape(H, cap, qk).transpose(1, 0, 2)
    v = b[vo:vo + 4 * H * cap * vd].view(np.float32).reshape(H, cap, vd).transpose(1, 0, 2)
    return np.ascontiguousarray(k), np.ascontiguousarray(v)


def kv_unpack(g, block_u8):
    """Split one device block (as a CPU uint8 numpy array) into the
    reference's slot-major views: k [cap][kvh][qk] i8, v, ks [cap][kvh], vs."""
    off = kv_offsets(g)
    H, cap, qk, vd = g.num_kv_heads, g.cap, g.qk_head_dim, g.v_head_dim
    b = np.asarray(block_u8)
    k = b[:H * cap * qk].view(np.int8).reshape(H, cap, qk).transpose(1, 0, 2)
    v = b[off["v"]:off["v"] + H * cap * vd].view(np.int8).reshape(H, cap, vd).transpose(1, 0, 2)
    ks = b[off["ks"]:off["ks"] + 4 * H * cap].view(np.float32).reshape(H, cap).T
    vs = b[off["vs"]:off["vs"] + 4 * H * cap].view(np.float32).reshape(H, cap).T
    return (np.ascontiguousarray(k), np.ascontiguousarray(ks), np.ascontiguousarray(v),
            np.ascontiguousarray(vs))


class V3LayerCache:
    """One layer of V3Cache (cache.rs:125-393) with an int8 device block.

    The device block holds `cap` slots from the start; the reference's
    logical ring size (`slots`, grown by doubling, cache.rs:291-309) is kept
    here because span() clamps with it (cache.rs:322-331).  Physical slot
    pos % cap equals the reference's pos % slots at every write and read:
    while slots < cap every live position is below slots.
    """

    def __init__(self, ctx, num_heads, num_kv_heads, qk, vd, hint, window, max_seq_len):
        self.ctx = ctx
        hint = min(max(hint, 1), max_seq_len)
        self.window = window
        self.cap = min(window, max_seq_len) if window else max_seq_len
        self.slots = min(hint, self.cap)
        self.geom = kv_geom(num_heads, num_kv_heads, qk, vd, self.cap)
        self.block, self.block_bytes = kv_alloc(self.geom, 1, ctx.device)

    def _ensure(self, pos):
        if pos < self.slots or self.slots >= self.cap:
            return
        self.slots = min(max(self.slots * 2, pos + 1), self.cap)

    def write_kv(self, pos, k, v):
        torch = _torch()
        self._ensure(pos)
        p = torch.tensor([pos], dtype=torch.int32, device=k.device)
        kv_write(self.ctx, self.geom, self.block, 0, p, k, v)

    def span(self, pos):
        lo = pos + 1 - self.window if (self.window and pos + 1 > self.window) else 0
        lo = max(lo, max(pos + 1 - self.slots, 0))
        return lo, pos

    def attend_step(self, q, lo, hi, quant_query=False):
        torch = _torch()
        lo_t = torch.tensor([lo], dtype=torch.int32, device=q.device)
        hi_t = torch.tensor([hi], dtype=torch.int32, device=q.device)
        return attend_step_i8(self.ctx, self.geom, self.block, 0, lo_t, hi_t, q,
                              quant_query=quant_query)[0]


def attend_i8_prefill(ctx, num_heads, num_kv_heads, qk, vd, q, k, v, window=0, quant_query=False):
    """attend (attention.rs:218-287) with an int8 store: every prompt row t
    attends to max(0, t+1-window)..=t of the prompt's own quantised K/V."""
    torch = _torch()
    seq = q.shape[0]
    g = kv_geom(num_heads, num_kv_heads, qk, vd, max(seq, 1))
    blk, _ = kv_alloc(g, 1, q.device.index or 0)
    pos = torch.arange(seq, dtype=torch.int32, device=q.device)
    kv_write(ctx, g, blk, 0, pos, k.contiguous(), v.contiguous())
    hi = pos
    lo = torch.clamp(pos + 1 - window, min=0) if window else torch.zeros_like(pos)
    scale = float(np.float32(1.0) / np.float32(math.sqrt(qk)))
    return attend_step_i8(ctx, g, blk, 0, lo.to(torch.int32), hi, q.contiguous(), scale,
                          quant_query)


# ---- Needle-3 forward on the device ----------------------------------------

class V3Cfg(C.Structure):
    _fields_ = [("vocab_size", C.c_int32), ("out_vocab", C.c_int32), ("d_model", C.c_int32),
                ("num_heads", C.c_int32), ("num_kv_heads", C.c_int32), ("num_layers", C.c_int32),
                ("qk_head_dim", C.c_int32), ("v_head_dim", C.c_int32), ("max_seq_len", C.c_int32),
                ("hada_n", C.c_int32), ("mhc_lanes", C.c_int32), ("rope_theta", C.c_float),
                ("sliding_window", C.c_int32), ("n_global", C.c_int32),
                ("global_layers", C.c_int32 * 64), ("qkv_conv_taps", C.c_int32),
                ("n_orders", C.c_int32), ("orders", C.c_int32 * 8), ("e_heads", C.c_int32),
                ("e_slots", C.c_int32), ("e_sub_dim", C.c_int32), ("n_sites", C.c_int32),
                ("sites", C.c_int32 * 64), ("e_conv_taps", C.c_int32),
                ("e_conv_dilation", C.c_int32), ("e_seed_heads", C.c_int32)]


class V3Record(C.Structure):
    _fields_ = [("kind", C.c_int32), ("data", C.c_void_p), ("len", _sz), ("out", _sz),
                ("inn", _sz), ("group", _sz), ("bits", _sz)]


def v3_cfg(g):
    c = V3Cfg()
    for k in ("vocab_size", "out_vocab", "d_model", "num_heads", "num_kv_heads", "num_layers",
              "qk_head_dim", "v_head_dim", "max_seq_len", "hada_n", "mhc_lanes",
              "sliding_window", "qkv_conv_taps", "e_heads", "e_slots", "e_sub_dim",
              "e_conv_taps", "e_conv_dilation", "e_seed_heads"):
        setattr(c, k, g[k])
    c.rope_theta = g["rope_theta"]
    c.n_global = len(g["global_layers"])
    for i, v in enumerate(g["global_layers"]):
        c.global_layers[i] = v
    c.n_orders = len(g["orders"])
    for i, v in enumerate(g["orders"]):
        c.orders[i] = v
    c.n_sites = len(g["sites"])
    for i, v in enumerate(g["sites"]):
        c.sites[i] = v
    return c


def geom_of_cfg(c):
    """The geometry dict (the keys v3_cfg reads) of an nd_v3_cfg."""
    g = {k: getattr(c, k) for k in (
        "vocab_size", "out_vocab", "d_model", "num_heads", "num_kv_heads", "num_layers",
        "qk_head_dim", "v_head_dim", "max_seq_len", "hada_n", "mhc_lanes", "sliding_window",
        "qkv_conv_taps", "e_heads", "e_slots", "e_sub_dim", "e_conv_taps", "e_conv_dilation",
        "e_seed_heads")}
    g["rope_theta"] = c.rope_theta
    g["global_layers"] = [c.global_layers[i] for i in range(c.n_global)]
    g["orders"] = [c.orders[i] for i in range(c.n_orders)]
    g["sites"] = [c.sites[i] for i in range(c.n_sites)]
    return g


def _container_bytes(data):
    if isinstance(data, (str, os.PathLike)):
        with open(data, "rb") as f:
            data = f.read()
    return np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else \
        np.ascontiguousarray(data, np.uint8)


def cact_v3_config(data):
    """A .cact v3 container (path or bytes) read as CactV3::from_bytes +
    config_from_geometry + V3Layout::derive (needle-infer/src/cact.rs:994-1030,
    v3.rs:25-386) do: returns (geometry dict, records up to final_norm).
    Host only; raises NeedleError with the reference's error variant."""
    buf = _container_bytes(data)
    cfg, n = V3Cfg(), _sz()
    _check(lib().nd_v3_cact_config(buf.ctypes.data_as(C.c_void_p), buf.size, C.byref(cfg),
                                   C.byref(n)))
    return geom_of_cfg(cfg), n.value


def v3_kv_bytes(geom, seq_len, kv_int8=True):
    """Key/value cache bytes of one session of `seq_len` positions
    (V3Config::kv_bytes_at, crates/needle-core/src/v3/config.rs:143-179).
    Host only."""
    cfg = v3_cfg(geom)
    return lib().nd_v3_kv_bytes(C.byref(cfg), seq_len, int(bool(kv_int8)))


def v3_ladder(num_layers, depth):
    """The blocks a `depth`-block rung keeps, ascending (ladder_layer_indices,
    crates/needle-core/src/v3/ladder.rs:67-74).  Host only."""
    kept = (C.c_int32 * max(int(depth), 1))()
    _check(lib().nd_v3_ladder(num_layers, depth, kept))
    return [kept[i] for i in range(depth)]


def cact_v3_config_at_depth(data, depth):
    """The geometry of a container's `depth`-block rung and the parent
    blocks it keeps (config_at_depth with model_from_cact_at_depth's
    checks, needle-infer/src/v3.rs:620-664).  Host only."""
    buf = _container_bytes(data)
    cfg = V3Cfg()
    kept = (C.c_int32 * max(int(depth), 1))()
    _check(lib().nd_v3_cact_config_at_depth(buf.ctypes.data_as(C.c_void_p), buf.size, depth,
                                            C.byref(cfg), kept))
    return geom_of_cfg(cfg), [kept[i] for i in range(depth)]


class V3Model:
    """A Needle-3 model on the device, from canonical container records
    (V3Layout::derive order, crates/needle-infer/src/v3.rs:236-330), or from a
    .cact v3 container with `from_cact` (model_from_cact, v3.rs:438-482; with
    `depth`, the ladder rung model_from_cact_at_depth slices, v3.rs:656-734)."""

    @classmethod
    def from_cact(cls, ctx, data, depth=None):
        buf = _container_bytes(data)
        if depth is None:
            geom, _ = cact_v3_config(buf)
        else:
            geom, _ = cact_v3_config_at_depth(buf, depth)
        self = cls.__new__(cls)
        self.ctx, self.geom = ctx, geom
        h = C.c_void_p()
        if depth is None:
            _check(lib().nd_v3_model_from_cact(ctx.h, buf.ctypes.data_as(C.c_void_p), buf.size,
                                               C.byref(h)))
        else:
            _check(lib().nd_v3_model_from_cact_at_depth(ctx.h, buf.ctypes.data_as(C.c_void_p),
                                                        buf.size, depth, C.byref(h)))
        self.h = h
        self.rows = lib().nd_v3_logit_rows(h)
        return self

    def __init__(self, ctx, geom, records, codebook):
        self.ctx, self.geom = ctx, geom
        cfg = v3_cfg(geom)
        keep = [np.ascontiguousarray(r["data"]) for r in records]
        arr = (V3Record * len(records))()
        for i, (r, buf) in enumerate(zip(records, keep)):
            arr[i] = V3Record(r["kind"], buf.ctypes.data, buf.nbytes, r["out"], r["inn"],
                              r["group"], r["bits"])
        cb = np.ascontiguousarray(codebook, np.float32)
        h = C.c_void_p()
        _check(lib().nd_v3_model_create(ctx.h, C.byref(cfg), cb.ctypes.data_as(C.c_void_p), cb.size,
                                        arr, len(records), C.byref(h)))
        self.h = h
        self.rows = lib().nd_v3_logit_rows(h)

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.nd_v3_model_free(self.h)
            self.h = None

    __del__ = close


class V3Batch:
    """`sessions` decode sessions stepped in lockstep on the device, with
    int8 KV caches (kv_int8=True, KvPrecision::Int8) or f32 ones
    (KvPrecision::F32, needle_v3_generate's default); with max_chunk > 1 a
    prompt is prefilled up to max_chunk positions per pass (the reference's
    chunked prefill, bit-identical to stepping).  The batch is stepped
    through `ctx` (the model's context by default): a model is shared by any
    number of threads, each stepping its own batches through its own
    context."""

    def __init__(self, model, sessions, max_len, hint=None, max_chunk=1, kv_int8=True, ctx=None):
        self.model, self.sessions, self.max_chunk = model, sessions, max_chunk
        self.ctx = ctx if ctx is not None else model.ctx
        self.kv_int8 = bool(kv_int8)
        h = C.c_void_p()
        _check(lib().nd_v3_batch_create_ex(self.ctx.h, model.h, sessions, max_len,
                                           hint or max_len, max_chunk, int(self.kv_int8),
                                           C.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.nd_v3_batch_free(self.h)
            self.h = None

    __del__ = close

    def positions(self):
        out = np.zeros(self.sessions, np.int32)
        _check(lib().nd_v3_positions(self.h, out.ctypes.data_as(C.c_void_p)))
        return out

    def set_graphs(self, on):
        """Single-position steps as one replayed HIP graph, or kernel by
        kernel (the default, faster on ROCm 7.2); the results are identical."""
        _check(lib().nd_v3_batch_set_graphs(self.h, int(bool(on))))

    def _logits_arg(self, logits):
        if logits is None:
            return None
        torch = _torch()
        return _arg(logits, torch.float32, "logits", self.sessions * self.model.rows)

    def step(self, tokens, logits=None, want_next=True):
        """Feed tokens[i] to session i (V3Model::decode_step); returns the greedy
        next tokens, and fills `logits` ([sessions][rows] device tensor) if given."""
        tok = np.ascontiguousarray(tokens, np.int32).reshape(self.sessions)
        nxt = np.zeros(self.sessions, np.int32) if want_next else None
        _check(lib().nd_v3_step(self.ctx.h, self.model.h, self.h,
                                tok.ctypes.data_as(C.c_void_p),
                                nxt.ctypes.data_as(C.c_void_p) if want_next else None,
                                self._logits_arg(logits)))
        return nxt

    def prefill(self, tokens, logits=None, want_next=True):
        """tokens [sessions][count]: count consecutive positions per session in
        one pass (V3Model::prefill); returns the greedy token after the last."""
        tok = np.ascontiguousarray(tokens, np.int32).reshape(self.sessions, -1)
        nxt = np.zeros(self.sessions, np.int32) if want_next else None
        _check(lib().nd_v3_prefill(self.ctx.h, self.model.h, self.h,
                                   tok.ctypes.data_as(C.c_void_p), tok.shape[1],
                                   nxt.ctypes.data_as(C.c_void_p) if want_next else None,
                                   self._logits_arg(logits)))
        return nxt

    def greedy(self, first, steps):
        """`steps` greedy steps from first[i] (V3Engine's loop, nd_v3_generate):
        returns [sessions][steps], each step's choice; the device feeds each
        step's choice to the next without a host round trip."""
        tok = np.ascontiguousarray(first, np.int32).reshape(self.sessions)
        out = np.zeros((self.sessions, steps), np.int32)
        _check(lib().nd_v3_generate(self.ctx.h, self.model.h, self.h,
                                    tok.ctypes.data_as(C.c_void_p), steps,
                                    out.ctypes.data_as(C.c_void_p)))
        return out

    @staticmethod
    def greedy_many(batches, firsts, steps):
        """greedy() for several batches of one model at once (nd_v3_generate_many):
        batch i on its own context's stream, the steps enqueued in turn from
        this thread; returns one [sessions][steps] array per batch."""
        n = len(batches)
        model = batches[0].model
        assert all(b.model is model for b in batches), "one model"
        toks = [np.ascontiguousarray(f, np.int32).reshape(b.sessions) for b, f in zip(batches, firsts)]
        outs = [np.zeros((b.sessions, steps), np.int32) for b in batches]
        ctxs = (C.c_void_p * n)(*[b.ctx.h.value for b in batches])
        bs = (C.c_void_p * n)(*[b.h.value for b in batches])
        fs = (C.c_void_p * n)(*[t.ctypes.data for t in toks])
        ts = (C.c_void_p * n)(*[o.ctypes.data for o in outs])
        _check(lib().nd_v3_generate_many(ctxs, model.h, bs, n, fs, steps, ts))
        return outs

    def generate(self, prompts, steps):
        """Prefill each session's prompt, max_chunk positions per pass (or by
        stepping; the reference proves the two bit-identical), then `steps`
        greedy tokens: the prefill's choice, then the device loop's."""
        prompts = np.asarray(prompts, np.int32).reshape(self.sessions, -1)
        nxt = None
        n = prompts.shape[1]
        for t0 in range(0, n, self.max_chunk):
            t1 = min(n, t0 + self.max_chunk)
            last = t1 == n
            if t1 - t0 == 1:
                nxt = self.step(prompts[:, t0], want_next=last)
            else:
                nxt = self.prefill(prompts[:, t0:t1], want_next=last)
        out = np.zeros((self.sessions, steps), np.int32)
        if steps > 0:
            out[:, 0] = nxt
        if steps > 1:
            out[:, 1:] = self.greedy(nxt, steps - 1)
        return out
