"""ctypes/numpy face of the CPU oracle (oracle/moex_oracle.c). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
checker (or the timed CPU baseline). The product path never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "liboracle.so")
AHD = 256

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        L = ctypes.CDLL(_LIB)
        c = ctypes
        L.orc_tq_tables.argtypes = [_f32p, _f32p, _i8p, _i8p, _f32p, _f32p, _f32p]
        L.orc_round_f16_array.argtypes = [_f32p, _f32p, c.c_long]
        L.orc_int8_quant_row.argtypes = [_f32p, _i8p, _f32p]
        L.orc_tq_half_sum.argtypes = [_f32p]
        L.orc_tq_half_sum.restype = c.c_float
        L.orc_tq_wht.argtypes = [_f32p, _f32p, c.c_int]
        L.orc_tq_quant.argtypes = [_f32p, c.c_int, _i32p, _f32p]
        L.orc_turbo_pack.argtypes = [_i32p, _i32p, _u8p, _u8p]
        L.orc_turbo_unpack.argtypes = [_u8p, _u8p, _i32p, _i32p]
        L.orc_kv_append.argtypes = [_f32p, _f32p, c.c_long, c.c_int, c.c_int, c.c_int, c.c_int, c.c_int,
                                    c.c_void_p, c.c_void_p, _f32p, _f32p]
        rows_args = [_f32p, c.c_void_p, c.c_long, c.c_int, c.c_int, c.c_void_p, c.c_void_p, _f32p, _f32p,
                     c.c_int, c.c_int, c.c_int, _i32p, c.c_int, _f64p]
        L.orc_attn_rows_f64.argtypes = rows_args
        L.orc_attn_rows_fa_emul.argtypes = rows_args
        L.orc_qk_norm_rope_row.argtypes = [_f32p, _u16p, c.c_int, c.c_int, c.c_float, c.c_float, c.c_int, _f32p]
        L.orc_quantize_rows_i8.argtypes = [_u16p, c.c_long, c.c_long, _i8p, _f32p]
        L.orc_dense_i8_f64.argtypes = [_i8p, _f32p, _f32p, c.c_long, c.c_long, c.c_long, _f64p]
        L.orc_dense_i8_fp16x.argtypes = [_i8p, _f32p, _f32p, c.c_long, c.c_long, c.c_long, _f64p]
        L.orc_quantize_rows_q4.argtypes = [_u16p, c.c_long, c.c_long, _u8p, _f32p]
        L.orc_quantize_rows_q6.argtypes = [_u16p, c.c_long, c.c_long, _u8p, _u8p, _f32p]
        mat_args = [c.c_int, c.c_void_p, c.c_void_p, _f32p, _f32p, c.c_long, c.c_long, c.c_long, _f64p]
        L.orc_dense_mat_f64.argtypes = mat_args
        L.orc_dense_mat_fp16x.argtypes = mat_args
        _lib = L
    return _lib


def tables():
    s1 = np.zeros(128, np.float32); s2 = np.zeros(128, np.float32)
    i4 = np.zeros(16, np.int8); i3 = np.zeros(8, np.int8)
    k = np.zeros(2, np.float32); m4 = np.zeros(15, np.float32); m3 = np.zeros(7, np.float32)
    lib().orc_tq_tables(s1, s2, i4, i3, k, m4, m3)
    return dict(S1=s1, S2=s2, I4=i4, I3=i3, K4=k[0], K3=k[1], M4=m4, M3=m3)


def round_f16(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_round_f16_array(x.reshape(-1), y.reshape(-1), x.size)
    return y


def int8_quant_row(x):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(AHD, np.int8); s = np.zeros(1, np.float32)
    lib().orc_int8_quant_row(x, q, s)
    return q, s[0]


def half_sum(v128):
    return np.float32(lib().orc_tq_half_sum(np.ascontiguousarray(v128, np.float32)))


def wht(x, inverse=False):
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(AHD, np.float32)
    lib().orc_tq_wht(x, y, 1 if inverse else 0)
    return y


def tq_quant(x, bits):
    idx = np.zeros(AHD, np.int32); n = np.zeros(2, np.float32)
    lib().orc_tq_quant(np.ascontiguousarray(x, np.float32), bits, idx, n)
    return idx, n


def turbo_pack(ik, iv):
    kb = np.zeros(128, np.uint8); vb = np.zeros(96, np.uint8)
    lib().orc_turbo_pack(np.ascontiguousarray(ik, np.int32), np.ascontiguousarray(iv, np.int32), kb, vb)
    return kb, vb


def turbo_unpack(kb, vb):
    ik = np.zeros(AHD, np.int32); iv = np.zeros(AHD, np.int32)
    lib().orc_turbo_unpack(np.ascontiguousarray(kb, np.uint8), np.ascontiguousarray(vb, np.uint8), ik, iv)
    return ik, iv


class HostCache:
    """Host copy of a KVCache (kernels.cuh:1121): int8 k,v [KV][max_t][256] + ks,vs [KV][max_t], or turbo
    k [KV][max_t][128], v [KV][max_t][96] (uint8) + ks,vs [KV][max_t][2]."""

    def __init__(self, KV, max_t, turbo):
        self.KV, self.max_t, self.turbo = KV, max_t, int(turbo)
        kb, vb, ns = (128, 96, 2) if turbo else (AHD, AHD, 1)
        self.k = np.zeros((KV, max_t, kb), np.int8)
        self.v = np.zeros((KV, max_t, vb), np.int8)
        self.ks = np.zeros((KV, max_t, ns), np.float32) if turbo else np.zeros((KV, max_t), np.float32)
        self.vs = np.zeros_like(self.ks)


def kv_append(cache, k, v, ld, T, pos0):
    """Quantize-append T tokens (k, v: float32 arrays, token stride ld)."""
    k = np.ascontiguousarray(k, np.float32).reshape(-1)
    v = np.ascontiguousarray(v, np.float32).reshape(-1)
    lib().orc_kv_append(k, v, ld, T, cache.KV, pos0, cache.max_t, cache.turbo,
                        cache.k.ctypes.data, cache.v.ctypes.data, cache.ks.reshape(-1), cache.vs.reshape(-1))


def _rows(fn, qo, gate, ld, H, cache, pos0, rows):
    qo = np.ascontiguousarray(qo, np.float32).reshape(-1)
    rows = np.ascontiguousarray(np.asarray(rows, np.int32).reshape(-1))
    out = np.zeros((len(rows) // 2, AHD), np.float64)
    g = None
    if gate is not None:
        g = np.ascontiguousarray(gate, np.float32).reshape(-1)
    fn(qo, None if g is None else g.ctypes.data, ld, H, cache.KV, cache.k.ctypes.data, cache.v.ctypes.data,
       cache.ks.reshape(-1), cache.vs.reshape(-1), cache.max_t, cache.turbo, pos0, rows, len(rows) // 2, out.reshape(-1))
    return out


def attn_rows_f64(qo, gate, ld, H, cache, pos0, rows):
    """fp64 reference attention for (token, head) rows (tests/test_fa.cu:59-80; turbo: + inverse WHT)."""
    return _rows(lib().orc_attn_rows_f64, qo, gate, ld, H, cache, pos0, rows)


def attn_rows_fa_emul(qo, gate, ld, H, cache, pos0, rows):
    """Precision model of the reference attn_fa_k (fp16 Q, fp16 P*vscale, fp32 softmax): its error estimate."""
    return _rows(lib().orc_attn_rows_fa_emul, qo, gate, ld, H, cache, pos0, rows)


def qk_norm_rope_row(x, w_f16_bits, pos, rot, theta, eps, wht_fwd=False):
    out = np.zeros(AHD, np.float32)
    lib().orc_qk_norm_rope_row(np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w_f16_bits, np.uint16),
                               pos, rot, theta, eps, 1 if wht_fwd else 0, out)
    return out


# ---- dense int8 projections ----
def quantize_rows_i8(w16):
    """quantize_rows_i8_k (kernels.cuh:144-156): fp16 [O][I] (np.float16) -> (int8 [O][I], float32 [O])."""
    w16 = np.ascontiguousarray(w16, np.float16)
    O, I = w16.shape
    q = np.zeros((O, I), np.int8); s = np.zeros(O, np.float32)
    lib().orc_quantize_rows_i8(w16.view(np.uint16).reshape(-1), O, I, q.reshape(-1), s)
    return q, s


def dense_i8_f64(q, s, x):
    """y [S][O] = s * (q . x), exact in fp64 (x: float32 [S][I])."""
    q = np.ascontiguousarray(q, np.int8); s = np.ascontiguousarray(s, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    O, I = q.shape; S = x.shape[0]
    y = np.zeros((S, O), np.float64)
    lib().orc_dense_i8_f64(q.reshape(-1), s, x.reshape(-1), S, I, O, y.reshape(-1))
    return y


def dense_i8_fp16x(q, s, x):
    """The prefill GEMM's precision model: activations rounded to fp16, products exact, fp64 sums."""
    q = np.ascontiguousarray(q, np.int8); s = np.ascontiguousarray(s, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    O, I = q.shape; S = x.shape[0]
    y = np.zeros((S, O), np.float64)
    lib().orc_dense_i8_fp16x(q.reshape(-1), s, x.reshape(-1), S, I, O, y.reshape(-1))
    return y


# ---- the other dense forms (struct Mat, kernels.cuh:186-196) ----
MAT_Q4, MAT_Q6, MAT_F16 = 1, 2, 3


def quantize_rows_q4(w16):
    """quantize_rows_q4_k (kernels.cuh:576-590): fp16 [O][I] -> (uint8 [O][I/2] nibbles, float32 [O][I/64] scales)."""
    w16 = np.ascontiguousarray(w16, np.float16)
    O, I = w16.shape
    q = np.zeros((O, I // 2), np.uint8); s = np.zeros((O, I // 64), np.float32)
    lib().orc_quantize_rows_q4(w16.view(np.uint16).reshape(-1), O, I, q.reshape(-1), s.reshape(-1))
    return q, s


def quantize_rows_q6(w16):
    """quantize_rows_q6_k (kernels.cuh:552-573): fp16 [O][I] -> (low plane [O][I/2], high plane [O][I/4], scales)."""
    w16 = np.ascontiguousarray(w16, np.float16)
    O, I = w16.shape
    q = np.zeros((O, I // 2), np.uint8); qh = np.zeros((O, I // 4), np.uint8); s = np.zeros((O, I // 64), np.float32)
    lib().orc_quantize_rows_q6(w16.view(np.uint16).reshape(-1), O, I, q.reshape(-1), qh.reshape(-1), s.reshape(-1))
    return q, qh, s


def _mat_call(fn, fmt, w, wh, s, x):
    x = np.ascontiguousarray(x, np.float32)
    S, I = x.shape
    w = np.ascontiguousarray(w)
    O = w.shape[0]
    if fmt == MAT_F16:
        w = w.view(np.uint16)
        s = np.zeros(1, np.float32)
    s = np.ascontiguousarray(s, np.float32).reshape(-1)
    wh = None if wh is None else np.ascontiguousarray(wh, np.uint8)
    y = np.zeros((S, O), np.float64)
    fn(fmt, w.ctypes.data, None if wh is None else wh.ctypes.data, s, x.reshape(-1), S, I, O, y.reshape(-1))
    return y


def dense_mat_f64(fmt, w, wh, s, x):
    """y [S][O] = W . x with the exact weights (code * group scale, or fp16), fp64 sums."""
    return _mat_call(lib().orc_dense_mat_f64, fmt, w, wh, s, x)


def dense_mat_fp16x(fmt, w, wh, s, x):
    """The int4 / int6 / fp16 GEMMs' precision model: weights fp16(fp32(code * scale)), activations fp16."""
    return _mat_call(lib().orc_dense_mat_fp16x, fmt, w, wh, s, x)
