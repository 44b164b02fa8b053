"""ctypes view of the CPU oracle (needle_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the CPU baseline -- never by
the shipped library.  Each wrapper calls the C restatement of the
reference function it names; the citations live in needle_oracle.c.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libneedle_oracle.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_sz = C.c_size_t

TERNARY = 5


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


class _AttnDims(C.Structure):
    _fields_ = [("seq", _sz), ("num_heads", _sz), ("num_kv_heads", _sz),
                ("qk_head_dim", _sz), ("v_head_dim", _sz)]


class _Ring(C.Structure):
    _fields_ = [("int8", C.c_int), ("num_kv_heads", _sz), ("qk_head_dim", _sz),
                ("v_head_dim", _sz), ("slots", _sz), ("cap", _sz), ("window", _sz),
                ("k", C.POINTER(C.c_float)), ("v", C.POINTER(C.c_float)),
                ("kq", C.POINTER(C.c_int8)), ("vq", C.POINTER(C.c_int8)),
                ("k_scale", C.POINTER(C.c_float)), ("v_scale", C.POINTER(C.c_float))]


class _Cq(C.Structure):
    _fields_ = [("packed", C.POINTER(C.c_uint8)), ("norms", C.POINTER(C.c_float)),
                ("lut", C.POINTER(C.c_float)), ("per_byte", _sz), ("row_bytes", _sz),
                ("num_groups", _sz), ("out_feat", _sz), ("in_feat", _sz),
                ("in_padded", _sz), ("group", _sz), ("bits", C.c_uint8),
                ("levels", C.c_float * 16), ("n_levels", _sz)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_f16_to_f32.restype = C.c_float
        L.or_expf_n.argtypes = [_f32p, _sz, _f32p]
        L.or_logf_n.argtypes = [_f32p, _sz, _f32p]
        L.or_sinf_n.argtypes = [_f32p, _sz, _f32p]
        L.or_cosf_n.argtypes = [_f32p, _sz, _f32p]
        L.or_powf_n.argtypes = [_f32p, _f32p, _sz, _f32p]
        L.or_fwht.argtypes = [_f32p, _sz]
        L.or_fwht_normalized.argtypes = [_f32p, _sz]
        L.or_packed_row_bytes.argtypes = [_sz, C.c_uint8]
        L.or_packed_row_bytes.restype = _sz
        L.or_read_bits.argtypes = [_u8p, _sz, _sz, C.c_uint32]
        L.or_read_bits.restype = C.c_uint32
        L.or_build_lut.argtypes = [C.c_uint8, _f32p, C.c_void_p]
        L.or_build_lut.restype = _sz
        L.or_cq_from_blob.argtypes = [_u8p, _sz, _sz, _sz, _sz, C.c_uint8, C.c_void_p, _sz,
                                      C.POINTER(C.POINTER(_Cq))]
        L.or_cq_free.argtypes = [C.POINTER(_Cq)]
        L.or_cq_prepare_input.argtypes = [C.POINTER(_Cq), _f32p, _f32p]
        L.or_cq_matvec_rows_prepared.argtypes = [C.POINTER(_Cq), _f32p, _sz, _sz, _f32p]
        L.or_cq_matvec.argtypes = [C.POINTER(_Cq), _f32p, _f32p]
        L.or_cq_matvec_prepared_reference.argtypes = [C.POINTER(_Cq), _f32p, _f32p]
        L.or_cq_matmul_rows_prepared.argtypes = [C.POINTER(_Cq), _f32p, _sz, _sz, _sz, _f32p]
        L.or_cq_dequantize_row.argtypes = [C.POINTER(_Cq), _sz, _f32p]
        L.or_cb8_gemv.argtypes = [_u8p, _f32p, _f32p, _f32p, _sz, _sz]
        L.or_cb8_gemv_omp.argtypes = [_u8p, _f32p, _f32p, _f32p, _sz, _sz]
        L.or_set_threads.argtypes = [C.c_int, C.c_int]
        L.or_set_threads.restype = None
        L.or_get_threads.restype = C.c_int
        L.or_cb8_gemv_f64.argtypes = [_u8p, _f32p, _f32p, _f64p, _sz, _sz]
        L.or_cb8_gemm.argtypes = [_f32p, _u8p, _f32p, _f32p, _sz, _sz, _sz]
        L.or_cb8_gemm_omp.argtypes = [_f32p, _u8p, _f32p, _f32p, _sz, _sz, _sz, C.c_int]
        L.or_cb8_gemv_lanes.argtypes = [_u8p, _f32p, _f32p, _f32p, _sz, _sz, C.c_int]
        L.or_cb8_gemm_lanes.argtypes = [_f32p, _u8p, _f32p, _f32p, _sz, _sz, _sz, C.c_int]
        L.or_attend_step_i8_sessions.argtypes = [_sz, _f32p, _i8p, _f32p, _i8p, _f32p, _sz, _sz,
                                                 _sz, C.POINTER(_AttnDims), _f32p, C.c_int]
        L.or_fake_quant_vec.argtypes = [_f32p, _sz, C.c_uint32]
        L.or_quant_into.argtypes = [_f32p, _sz, _i8p]
        L.or_quant_into.restype = C.c_float
        L.or_quantize_rows.argtypes = [_f32p, _sz, _sz, _i8p, _f32p]
        L.or_quant_rows.argtypes = [_f32p, _sz, _sz, _sz]
        L.or_ring_new.argtypes = [C.c_int, _sz, _sz, _sz, _sz, _sz, _sz]
        L.or_ring_new.restype = C.POINTER(_Ring)
        L.or_ring_free.argtypes = [C.POINTER(_Ring)]
        L.or_ring_write_kv.argtypes = [C.POINTER(_Ring), _sz, _f32p, _f32p]
        L.or_ring_span.argtypes = [C.POINTER(_Ring), _sz, C.POINTER(_sz), C.POINTER(_sz)]
        L.or_ring_attend_step.argtypes = [C.POINTER(_Ring), _f32p, _sz, _sz, _sz, _f32p]
        L.or_attend_step_f32.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz,
                                         C.POINTER(_AttnDims), _f32p]
        L.or_attend_step_i8.argtypes = [_f32p, _i8p, _f32p, _i8p, _f32p, _sz, _sz, _sz,
                                        C.POINTER(_AttnDims), _f32p]
        L.or_attend_f32.argtypes = [_f32p, _f32p, _f32p, C.POINTER(_AttnDims), _sz, _f32p]
        L.or_attend_i8.argtypes = [_f32p, _i8p, _f32p, _i8p, _f32p, C.POINTER(_AttnDims),
                                   _sz, _f32p]
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- math.rs / hadamard.rs --------------------------------------------------

def f16_to_f32(bits: int) -> float:
    return lib().or_f16_to_f32(bits)


def expf(x):
    """libm's expf (math.rs:3-6), elementwise."""
    x = _f32(x).ravel()
    y = np.empty_like(x)
    lib().or_expf_n(x, x.size, y)
    return y


def logf(x):
    """libm's logf (math.rs:8-11), elementwise."""
    x = _f32(x).ravel()
    y = np.empty_like(x)
    lib().or_logf_n(x, x.size, y)
    return y


def sinf(x):
    """libm's sinf (math.rs:23-26), elementwise."""
    x = _f32(x).ravel()
    y = np.empty_like(x)
    lib().or_sinf_n(x, x.size, y)
    return y


def cosf(x):
    """libm's cosf (math.rs:28-31), elementwise."""
    x = _f32(x).ravel()
    y = np.empty_like(x)
    lib().or_cosf_n(x, x.size, y)
    return y


def powf(x, e):
    """libm's powf (math.rs:43-46), elementwise over broadcast x and e."""
    x, e = np.broadcast_arrays(_f32(x), _f32(e))
    x, e = _f32(x).ravel(), _f32(e).ravel()
    y = np.empty_like(x)
    lib().or_powf_n(x, e, x.size, y)
    return y


def fwht(x):
    y = _f32(x).copy()
    lib().or_fwht(y, y.size)
    return y


def fwht_normalized(x):
    y = _f32(x).copy()
    lib().or_fwht_normalized(y, y.size)
    return y


# ---- cq.rs ------------------------------------------------------------------

def packed_row_bytes(in_padded: int, bits: int) -> int:
    return lib().or_packed_row_bytes(in_padded, bits)


def read_bits(row, bit: int, bits: int) -> int:
    return lib().or_read_bits(np.ascontiguousarray(row, np.uint8), bit, bits, (1 << bits) - 1)


def build_lut(bits: int, levels):
    lv = _f32(levels)
    per = lib().or_build_lut(bits, lv, None)
    if per == 0:
        return 0, np.zeros(0, np.float32)
    out = np.zeros(256 * per, np.float32)
    lib().or_build_lut(bits, lv, out.ctypes.data)
    return per, out


class CqError(Exception):
    NAMES = {1: "UnsupportedBits", 2: "BadGroup", 3: "BadCodebookLen",
             4: "ShortBlob", 5: "EmptyShape"}

    def __init__(self, code):
        super().__init__(self.NAMES.get(code, str(code)))
        self.code = code


class CqWeight:
    """The oracle's CqWeight (cq.rs:117-810)."""

    def __init__(self, blob, out_feat, in_feat, group, bits, codebook):
        blob = np.ascontiguousarray(blob, np.uint8)
        cb = _f32(codebook)
        p = C.POINTER(_Cq)()
        rc = lib().or_cq_from_blob(blob, blob.size, out_feat, in_feat, group, bits,
                                   cb.ctypes.data, cb.size, C.byref(p))
        if rc:
            raise CqError(rc)
        self._p = p
        c = p.contents
        self.out_feat, self.in_feat, self.in_padded = c.out_feat, c.in_feat, c.in_padded
        self.group, self.bits, self.num_groups = c.group, c.bits, c.num_groups
        self.row_bytes, self.per_byte = c.row_bytes, c.per_byte
        self.levels = np.array(c.levels[:c.n_levels], np.float32)

    def __del__(self):
        if getattr(self, "_p", None) is not None and _lib is not None:
            _lib.or_cq_free(self._p)
            self._p = None

    def norms(self):
        c = self._p.contents
        return np.ctypeslib.as_array(c.norms, (self.out_feat * self.num_groups,)).copy()

    def prepare_input(self, x):
        x = _f32(x)
        xh = np.zeros(self.in_padded, np.float32)
        lib().or_cq_prepare_input(self._p, x, xh)
        return xh

    def prepare_batch(self, xs):
        xs = _f32(xs).reshape(-1, self.in_feat)
        return np.stack([self.prepare_input(r) for r in xs]).astype(np.float32)

    def matvec(self, x):
        y = np.zeros(self.out_feat, np.float32)
        lib().or_cq_matvec(self._p, _f32(x), y)
        return y

    def matvec_rows_prepared(self, xh, row_start, rows):
        y = np.zeros(rows, np.float32)
        lib().or_cq_matvec_rows_prepared(self._p, _f32(xh), row_start, rows, y)
        return y

    def matvec_prepared(self, xh):
        return self.matvec_rows_prepared(xh, 0, self.out_feat)

    def matvec_prepared_reference(self, xh):
        y = np.zeros(self.out_feat, np.float32)
        lib().or_cq_matvec_prepared_reference(self._p, _f32(xh), y)
        return y

    def matmul_rows_prepared(self, xh, batch, row_start, rows):
        y = np.zeros(batch * rows, np.float32)
        lib().or_cq_matmul_rows_prepared(self._p, _f32(xh).reshape(-1), batch, row_start,
                                         rows, y)
        return y

    def dequantize_row(self, o):
        out = np.zeros(self.in_feat, np.float32)
        lib().or_cq_dequantize_row(self._p, o, out)
        return out

    def dequantize(self):
        return np.stack([self.dequantize_row(o) for o in range(self.out_feat)])


# ---- Format B ---------------------------------------------------------------

def cb8_gemv(w, cb, x):
    w = np.ascontiguousarray(w, np.uint8)
    out, inn = w.shape
    y = np.zeros(out, np.float32)
    lib().or_cb8_gemv(w, _f32(cb), _f32(x), y, out, inn)
    return y


SPLIT_REFERENCE, SPLIT_ALL = 0, 1


def set_threads(threads, split=SPLIT_REFERENCE):
    """Threads for the reference's rayon splits (cq.rs:301-323, 446-581).
    SPLIT_REFERENCE keeps its size rules; SPLIT_ALL also splits the smaller
    row loops and attention's heads (the same bits, a faster checker)."""
    lib().or_set_threads(int(threads), int(split))


def get_threads():
    return lib().or_get_threads()


def cb8_gemv_omp(w, cb, x, y):
    out, inn = w.shape
    lib().or_cb8_gemv_omp(w, cb, x, y, out, inn)


def cb8_gemv_f64(w, cb, x):
    w = np.ascontiguousarray(w, np.uint8)
    out, inn = w.shape
    y = np.zeros(out, np.float64)
    lib().or_cb8_gemv_f64(w, _f32(cb), _f32(x), y, out, inn)
    return y


def cb8_gemm(x, w, cb):
    x = _f32(x)
    w = np.ascontiguousarray(w, np.uint8)
    m = x.shape[0]
    out, inn = w.shape
    y = np.zeros((m, out), np.float32)
    lib().or_cb8_gemm(x, w, _f32(cb), y, m, out, inn)
    return y


def cb8_gemm_omp(x, w, cb, threads, y=None):
    """cb8_gemm with output-row bands on `threads` threads (the same bits)."""
    x = _f32(x)
    w = np.ascontiguousarray(w, np.uint8)
    m = x.shape[0]
    out, inn = w.shape
    if y is None:
        y = np.zeros((m, out), np.float32)
    lib().or_cb8_gemm_omp(x, w, _f32(cb), y, m, out, inn, int(threads))
    return y


def cb8_gemv_lanes(w, cb, x, threads=1, y=None):
    """Format B GEMV in the reference's eight-lane order (the CPU baseline's kernel)."""
    w = np.ascontiguousarray(w, np.uint8)
    out, inn = w.shape
    if y is None:
        y = np.zeros(out, np.float32)
    lib().or_cb8_gemv_lanes(w, _f32(cb), _f32(x), y, out, inn, int(threads))
    return y


def cb8_gemm_lanes(x, w, cb, threads=1, y=None):
    """Format B GEMM in matmul_rows_prepared's order (the CPU baseline's kernel)."""
    x = _f32(x)
    w = np.ascontiguousarray(w, np.uint8)
    m = x.shape[0]
    out, inn = w.shape
    if y is None:
        y = np.zeros((m, out), np.float32)
    lib().or_cb8_gemm_lanes(x, w, _f32(cb), y, m, out, inn, int(threads))
    return y


# ---- v3/cache.rs ------------------------------------------------------------

def fake_quant_vec(x, bits=8):
    y = _f32(x).copy()
    lib().or_fake_quant_vec(y, y.size, bits)
    return y


def quant_into(x):
    x = _f32(x)
    d = np.zeros(x.size, np.int8)
    s = lib().or_quant_into(x, x.size, d)
    return d, np.float32(s)


def quantize_rows(x, head_dim):
    x = _f32(x).reshape(-1)
    rows = x.size // head_dim
    ints = np.zeros(x.size, np.int8)
    scales = np.ones(rows, np.float32)
    lib().or_quantize_rows(x, rows, head_dim, ints, scales)
    return ints, scales


def quant_rows(x, seq, heads, head_dim):
    y = _f32(x).copy()
    lib().or_quant_rows(y, seq, heads, head_dim)
    return y


class Ring:
    """One layer of the oracle's V3Cache (cache.rs:125-393)."""

    def __init__(self, int8, num_kv_heads, qk, vd, hint, window, max_seq_len):
        self._p = lib().or_ring_new(int(int8), num_kv_heads, qk, vd, hint, window, max_seq_len)
        self.num_kv_heads, self.qk, self.vd = num_kv_heads, qk, vd

    def __del__(self):
        if getattr(self, "_p", None) is not None and _lib is not None:
            _lib.or_ring_free(self._p)
            self._p = None

    @property
    def slots(self):
        return self._p.contents.slots

    @property
    def cap(self):
        return self._p.contents.cap

    def write_kv(self, pos, k, v):
        lib().or_ring_write_kv(self._p, pos, _f32(k), _f32(v))

    def span(self, pos):
        lo, hi = _sz(), _sz()
        lib().or_ring_span(self._p, pos, C.byref(lo), C.byref(hi))
        return lo.value, hi.value

    def store(self):
        c = self._p.contents
        s, H = c.slots, c.num_kv_heads
        if c.int8:
            return dict(
                k=np.ctypeslib.as_array(c.kq, (s * H * c.qk_head_dim,)).copy(),
                v=np.ctypeslib.as_array(c.vq, (s * H * c.v_head_dim,)).copy(),
                k_scale=np.ctypeslib.as_array(c.k_scale, (s * H,)).copy(),
                v_scale=np.ctypeslib.as_array(c.v_scale, (s * H,)).copy())
        return dict(k=np.ctypeslib.as_array(c.k, (s * H * c.qk_head_dim,)).copy(),
                    v=np.ctypeslib.as_array(c.v, (s * H * c.v_head_dim,)).copy())

    def attend_step(self, q, lo, hi, num_heads):
        out = np.zeros(num_heads * self.vd, np.float32)
        lib().or_ring_attend_step(self._p, _f32(q), lo, hi, num_heads, out)
        return out


# ---- v3/attention.rs --------------------------------------------------------

def _dims(seq, nh, nkv, qk, vd):
    return _AttnDims(seq, nh, nkv, qk, vd)


def attend_step_f32(q, k, v, slots, lo, hi, nh, nkv, qk, vd):
    out = np.zeros(nh * vd, np.float32)
    d = _dims(1, nh, nkv, qk, vd)
    lib().or_attend_step_f32(_f32(q), _f32(k), _f32(v), slots, lo, hi, C.byref(d), out)
    return out


def attend_step_i8(q, k, ks, v, vs, slots, lo, hi, nh, nkv, qk, vd):
    out = np.zeros(nh * vd, np.float32)
    d = _dims(1, nh, nkv, qk, vd)
    lib().or_attend_step_i8(_f32(q), np.ascontiguousarray(k, np.int8), _f32(ks),
                            np.ascontiguousarray(v, np.int8), _f32(vs), slots, lo, hi,
                            C.byref(d), out)
    return out


def attend_step_i8_sessions(q, k, ks, v, vs, slots, lo, hi, nh, nkv, qk, vd, threads, out=None):
    """attend_step for each session i over its own cache (k[i], ks[i], v[i],
    vs[i], each `slots` positions), sessions split across `threads`."""
    count = q.shape[0]
    if out is None:
        out = np.zeros((count, nh * vd), np.float32)
    d = _dims(1, nh, nkv, qk, vd)
    lib().or_attend_step_i8_sessions(count, _f32(q), np.ascontiguousarray(k, np.int8), _f32(ks),
                                     np.ascontiguousarray(v, np.int8), _f32(vs), slots, lo, hi,
                                     C.byref(d), out, int(threads))
    return out


def attend_f32(q, k, v, seq, nh, nkv, qk, vd, window=0):
    out = np.zeros(seq * nh * vd, np.float32)
    d = _dims(seq, nh, nkv, qk, vd)
    lib().or_attend_f32(_f32(q), _f32(k), _f32(v), C.byref(d), window or 0, out)
    return out


def attend_i8(q, k, ks, v, vs, seq, nh, nkv, qk, vd, window=0):
    out = np.zeros(seq * nh * vd, np.float32)
    d = _dims(seq, nh, nkv, qk, vd)
    lib().or_attend_i8(_f32(q), np.ascontiguousarray(k, np.int8), _f32(ks),
                       np.ascontiguousarray(v, np.int8), _f32(vs), C.byref(d),
                       window or 0, out)
    return out


# ---- v3 forward (needle_oracle_v3.c) ----------------------------------------

class V3Cfg(C.Structure):
    _fields_ = [("vocab_size", _sz), ("out_vocab", _sz), ("d_model", _sz), ("num_heads", _sz),
                ("num_kv_heads", _sz), ("num_layers", _sz), ("qk_head_dim", _sz),
                ("v_head_dim", _sz), ("max_seq_len", _sz), ("hada_n", _sz), ("mhc_lanes", _sz),
                ("rope_theta", C.c_float), ("sliding_window", _sz), ("n_global", _sz),
                ("global_layers", _sz * 64), ("qkv_conv_taps", _sz), ("n_orders", _sz),
                ("orders", _sz * 8), ("e_heads", _sz), ("e_slots", _sz), ("e_sub_dim", _sz),
                ("n_sites", _sz), ("sites", _sz * 64), ("e_conv_taps", _sz),
                ("e_conv_dilation", _sz), ("e_seed_heads", _sz)]


class V3Record(C.Structure):
    _fields_ = [("kind", C.c_int), ("data", C.c_void_p), ("len", _sz), ("out", _sz),
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


_v3_bound = False


def _v3_lib():
    global _v3_bound
    L = lib()
    if not _v3_bound:
        L.or_v3_model_new.argtypes = [C.POINTER(V3Cfg), _f32p, C.POINTER(V3Record), _sz]
        L.or_v3_model_new.restype = C.c_void_p
        L.or_v3_model_free.argtypes = [C.c_void_p]
        L.or_v3_cache_new.argtypes = [C.POINTER(V3Cfg), _sz, C.c_int]
        L.or_v3_cache_new.restype = C.c_void_p
        L.or_v3_cache_free.argtypes = [C.c_void_p]
        L.or_v3_decode_step.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, _f32p]
        L.or_v3_generate.argtypes = [C.c_void_p, C.c_void_p, np.ctypeslib.ndpointer(np.uint32),
                                     _sz, _sz, np.ctypeslib.ndpointer(np.uint32), _f32p]
        L.or_argmax.argtypes = [_f32p, _sz]
        L.or_argmax.restype = C.c_uint32
        L.or_v3_decode_sessions.argtypes = [C.c_void_p, C.POINTER(C.c_void_p),
                                            np.ctypeslib.ndpointer(np.uint32), _sz, _f32p, C.c_int]
        L.or_v3_cache_fill_synthetic.argtypes = [C.c_void_p, _sz, C.c_uint64]
        L.or_sinkhorn.argtypes = [_f32p, _sz]
        L.or_kron_apply.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _f32p]
        L.or_engram_indices.argtypes = [np.ctypeslib.ndpointer(np.uint32), _sz,
                                        np.ctypeslib.ndpointer(np.uintp), _sz, _sz, C.c_uint32,
                                        _sz, np.ctypeslib.ndpointer(np.uint32)]
        L.or_ngram_valid.argtypes = [_sz, _sz, np.ctypeslib.ndpointer(np.uintp), _sz]
        L.or_ngram_valid.restype = C.c_int
        L.or_v3_rope_at.argtypes = [C.POINTER(V3Cfg), _sz, _f32p, _f32p]
        L.or_v3_set_rope_variant.argtypes = [C.c_int]
        L.or_v3_set_rope_variant.restype = None
        L.or_v3_apply_site.argtypes = [_f32p, _f32p, _f32p, _sz]
        L.or_v3_conv_step.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz]
        L.or_v3_engram_conv_step.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _sz]
        L.or_v3_norm_and_rope.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz]
        L.or_v3_mix_down.argtypes = [_f32p, _f32p, C.c_float, _f32p, _sz, _sz, _sz, _f32p]
        L.or_v3_scatter_up.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_float, _f32p, C.c_float,
                                       _f32p, _sz, _sz, _sz]
        L.or_hadamard_mlp.argtypes = [_f32p, _sz, C.c_void_p, np.ctypeslib.ndpointer(np.uint32),
                                      np.ctypeslib.ndpointer(np.uint32), _sz, _f32p]
        L.or_hada_blocks.argtypes = [_sz, C.POINTER(_sz), C.POINTER(_sz)]
        _v3_bound = True
    return L


class V3Model:
    """The oracle's V3Model built from canonical records (v3_synth.build_records)."""

    def __init__(self, geom, records, codebook):
        L = _v3_lib()
        self.geom = geom
        self.cfg = v3_cfg(geom)
        self._keep = [np.ascontiguousarray(r["data"]) for r in records]
        arr = (V3Record * len(records))()
        for i, (r, buf) in enumerate(zip(records, self._keep)):
            arr[i] = V3Record(r["kind"], buf.ctypes.data, buf.nbytes, r["out"], r["inn"],
                              r["group"], r["bits"])
        self.codebook = np.ascontiguousarray(codebook, np.float32)
        self._p = L.or_v3_model_new(C.byref(self.cfg), self.codebook, arr, len(records))
        if not self._p:
            raise ValueError("records do not match the v3 layout")
        self.rows = geom["out_vocab"] or geom["vocab_size"]

    def __del__(self):
        if getattr(self, "_p", None) and _lib is not None:
            _lib.or_v3_model_free(self._p)
            self._p = None

    def new_cache(self, hint, int8=True):
        return V3Cache(self, hint, int8)


class V3Cache:
    def __init__(self, model, hint, int8):
        self.model = model
        self._p = _v3_lib().or_v3_cache_new(C.byref(model.cfg), hint, int(int8))

    def __del__(self):
        if getattr(self, "_p", None) and _lib is not None:
            _lib.or_v3_cache_free(self._p)
            self._p = None

    def decode_step(self, token):
        out = np.zeros(self.model.rows, np.float32)
        _v3_lib().or_v3_decode_step(self.model._p, self._p, int(token), out)
        return out

    def fill_synthetic(self, pos, seed):
        """For timing only: this fresh cache (hint >= pos + the steps to be
        timed) put at position `pos` with seeded contents, as if `pos`
        tokens had been decoded."""
        _v3_lib().or_v3_cache_fill_synthetic(self._p, int(pos), int(seed))


def v3_decode_sessions(model, caches, tokens, threads):
    """One decode_step per session, sessions split across `threads`;
    returns the logits [sessions][rows]."""
    n = len(caches)
    arr = (C.c_void_p * n)(*[c._p for c in caches])
    tok = np.ascontiguousarray(tokens, np.uint32)
    out = np.zeros((n, model.rows), np.float32)
    _v3_lib().or_v3_decode_sessions(model._p, arr, tok, n, out, int(threads))
    return out


def v3_generate(model, prompt, steps, int8=True, hint=None):
    """Greedy tokens after stepping the prompt, and each step's top-1/top-2 margin."""
    prompt = np.ascontiguousarray(prompt, np.uint32)
    cache = model.new_cache(hint or (len(prompt) + steps), int8)
    toks = np.zeros(steps, np.uint32)
    margins = np.zeros(steps, np.float32)
    _v3_lib().or_v3_generate(model._p, cache._p, prompt, len(prompt), steps, toks, margins)
    return toks, margins


def argmax(x):
    """The engine's greedy pick (v3_engine.rs:410-420): first maximum under
    a strict `>` scan from -inf."""
    return int(_v3_lib().or_argmax(_f32(x).reshape(-1), np.asarray(x).size))


def sinkhorn(m):
    m = _f32(m).copy()
    n = int(round(m.size ** 0.5))
    _v3_lib().or_sinkhorn(m, n)
    return m.reshape(n, n)


def kron_apply(z, a, b):
    ba, bb = a.shape[0], b.shape[0]
    out = np.zeros(ba * bb, np.float32)
    _v3_lib().or_kron_apply(_f32(z).reshape(-1), _f32(a).reshape(-1), _f32(b).reshape(-1), ba, bb, out)
    return out.reshape(ba, bb)


def engram_indices(tokens, orders, heads, slots, seed_heads=0):
    tokens = np.ascontiguousarray(tokens, np.uint32)
    orders = np.ascontiguousarray(orders, np.uintp)
    out = np.zeros(len(tokens) * len(orders) * heads, np.uint32)
    _v3_lib().or_engram_indices(tokens, len(tokens), orders, len(orders), heads, slots,
                                seed_heads, out)
    return out


def ngram_valid(p, table, orders, heads):
    return bool(_v3_lib().or_ngram_valid(p, table, np.ascontiguousarray(orders, np.uintp), heads))


ROPE_LIBM, ROPE_POWF_CR, ROPE_GLIBC = 0, 1, 2


def set_rope_variant(variant):
    """The routines behind the oracle's RoPE table: ROPE_LIBM (the
    reference's libm 0.2.16 restated; the default), ROPE_POWF_CR (theta^e
    correctly rounded) or ROPE_GLIBC (the C library's powf/cosf/sinf)."""
    _v3_lib().or_v3_set_rope_variant(int(variant))


def rope_at(geom, pos):
    half = geom["qk_head_dim"] // 2
    c, s = np.zeros(half, np.float32), np.zeros(half, np.float32)
    _v3_lib().or_v3_rope_at(C.byref(v3_cfg(geom)), pos, c, s)
    return c, s


# ---- v3 helper steps (mhc.rs, engram.rs, cache.rs, attention.rs) -----------

def apply_site(x, k, v):
    """engram.rs:111-132 on copies; returns the updated x."""
    x = _f32(x).copy()
    _v3_lib().or_v3_apply_site(x, _f32(k), _f32(v), x.size)
    return x


def conv_step(tail, taps, raw, pos):
    """cache.rs:401-438: (out, new tail); tail is (taps - 1) x dim."""
    taps = _f32(taps)
    n_taps, dim = taps.shape
    tail = _f32(tail).copy().reshape(-1)
    x = _f32(raw).copy()
    if tail.size == 0:
        tail = np.zeros(1, np.float32)
    _v3_lib().or_v3_conv_step(tail, taps.reshape(-1), x, dim, n_taps, pos)
    return x, tail[:max(n_taps - 1, 0) * dim].reshape(max(n_taps - 1, 0), dim)


def engram_conv_step(tail, taps, raw, dil, max_order, pos):
    """cache.rs:445-482: (out, new tail); tail is (taps - 1) * dil x d."""
    taps = _f32(taps)
    n_taps, d = taps.shape
    reach = (n_taps - 1) * dil
    tail = _f32(tail).copy().reshape(-1)
    if tail.size == 0:
        tail = np.zeros(1, np.float32)
    x = _f32(raw).copy()
    _v3_lib().or_v3_engram_conv_step(tail, taps.reshape(-1), x, d, n_taps, dil, max_order, pos)
    return x, tail[:reach * d].reshape(reach, d)


def norm_and_rope(buf, scale, cs, sn):
    """attention.rs:108-150 for one position: buf is (heads, head_dim)."""
    buf = _f32(buf).copy()
    heads, hd = buf.shape
    _v3_lib().or_v3_norm_and_rope(buf.reshape(-1), _f32(scale), _f32(cs), _f32(sn), heads, hd)
    return buf


def mix_down(lanes, rows, a_pre, b_pre, layer):
    """mhc.rs:79-102: (gates, u) for lanes (n x d) and raw rows (n)."""
    lanes = _f32(lanes)
    n, d = lanes.shape
    rows = _f32(rows).copy()
    u = np.zeros(d, np.float32)
    _v3_lib().or_v3_mix_down(lanes.reshape(-1), rows, float(a_pre), _f32(b_pre), layer, n, d, u)
    return rows, u


def scatter_up(lanes, post, res, y, a_post, b_post, a_res, b_res, layer):
    """mhc.rs:109-152: (lanes, post gates, res gates) after the scatter."""
    lanes = _f32(lanes).copy()
    n, d = lanes.shape
    post = _f32(post).copy()
    res = _f32(res).copy().reshape(-1)
    _v3_lib().or_v3_scatter_up(lanes.reshape(-1), post, res, _f32(y), float(a_post), _f32(b_post),
                               float(a_res), _f32(b_res).reshape(-1), layer, n, d)
    return lanes, post, res.reshape(n, n)


class _V3Mlp(C.Structure):
    _fields_ = [(n, C.POINTER(C.c_float)) for n in
                ("d1", "d2", "b2", "d3", "d4", "w1a", "w1b", "w2a", "w2b", "w3a", "w3b",
                 "cond_v", "cond_u")] + [("cond_rank", _sz)]


def hada_blocks(n):
    a, b = _sz(), _sz()
    _v3_lib().or_hada_blocks(n, C.byref(a), C.byref(b))
    return a.value, b.value


def hadamard_mlp(x, w, p1, p2, hada_n):
    """v3/kernels.rs:119-180.  w: dict of d1 d2 b2 d3 d4 (hada_n), w1a..w3b
    (square factors), cond_v (d x r), cond_u (r x hada_n)."""
    x = _f32(x)
    keep = {k: _f32(v).reshape(-1) for k, v in w.items()}
    m = _V3Mlp(*[keep[k].ctypes.data_as(C.POINTER(C.c_float)) for k in
                 ("d1", "d2", "b2", "d3", "d4", "w1a", "w1b", "w2a", "w2b", "w3a", "w3b",
                  "cond_v", "cond_u")], np.asarray(w["cond_v"]).shape[1])
    out = np.zeros(x.size, np.float32)
    _v3_lib().or_hadamard_mlp(x, x.size, C.byref(m), np.ascontiguousarray(p1, np.uint32),
                              np.ascontiguousarray(p2, np.uint32), hada_n, out)
    return out
