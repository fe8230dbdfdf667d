"""moex_amd -- MI355X (gfx950) attention hot path of moex behind its C ABI (include/moex_attn.h).

This module is the Python face of libmoex_attn.so: ctypes bindings that keep the reference's entry-point names
and argument order (src/kernels.cuh: attn_decode :1850, attn_fa :1713, attn_prefill :1435, kv_alloc :1867,
kv_bytes :1875, and the raw launches attn_gqa_k :1745, attn_combine_k :1317, attn_decode_k :1244,
turbo_out_k :1731, qk_norm_rope_k :1185). Device buffers are passed as torch tensors (or raw int addresses);
streams as torch.cuda.Stream (or a raw hipStream_t int). There is no fallback: if the library is missing the
import-time load raises.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmoex_attn.so")
AHD = 256
TQ_KB, TQ_VB = 128, 96


class Mat(ctypes.Structure):
    """struct Mat (kernels.cuh:186-196) as moex_mat (include/moex_dense.h): one of f16; q, s (int8, row scales);
    q4, s (int4 gs64); q6, q6h, s (int6 gs64). Fields take torch tensors or device addresses; the struct holds the
    addresses only, so the caller keeps the tensors alive while it is used."""
    _fields_ = [("f16", ctypes.c_void_p), ("q", ctypes.c_void_p), ("s", ctypes.c_void_p), ("q4", ctypes.c_void_p),
                ("q6", ctypes.c_void_p), ("q6h", ctypes.c_void_p)]

    def __init__(self, f16=None, q=None, s=None, q4=None, q6=None, q6h=None):
        super().__init__(_p(f16), _p(q), _p(s), _p(q4), _p(q6), _p(q6h))


class KVCache(ctypes.Structure):
    """struct KVCache (kernels.cuh:1121): int8 *k, *v; float *ks, *vs; int turbo."""
    _fields_ = [("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("ks", ctypes.c_void_p), ("vs", ctypes.c_void_p),
                ("turbo", ctypes.c_int)]


_lib = None


def build():
    """Compile libmoex_attn.so for gfx950 in place (hipcc via moex_amd/csrc/Makefile)."""
    import subprocess
    subprocess.run(["make", "-s", "-B", "-j8", "-C", os.path.join(_HERE, "csrc")], check=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run moex_amd.build() (hipcc, gfx950)")
    L = ctypes.CDLL(LIB_PATH)
    vp, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    L.moex_kv_alloc.argtypes = [i, i, i]
    L.moex_kv_alloc.restype = KVCache
    L.moex_kv_bytes.argtypes = [i, i, i]
    L.moex_kv_bytes.restype = ctypes.c_size_t
    L.moex_kv_free.argtypes = [KVCache]
    L.moex_attn_decode.argtypes = [vp, vp, vp, vp, vp, vp, KVCache, vp, i, i, vp, i, i, f, f, i, i, vp, vp, i]
    L.moex_attn_decode_noalloc.argtypes = [vp, vp, vp, vp, vp, vp, KVCache, vp, i, i, vp, i, i, f, f, i, i, vp, i]
    L.moex_attn_fa.argtypes = [vp, vp, KVCache, vp, i, i, vp, i, i, i, vp]
    L.moex_attn_prefill.argtypes = [vp, vp, KVCache, vp, i, i, vp, i, i, i, vp]
    L.moex_qk_norm_rope.argtypes = [vp, vp, vp, vp, vp, vp, KVCache, i, i, vp, i, i, f, f, i, i, vp]
    L.moex_kv_append.argtypes = [vp, vp, KVCache, i, vp, i, i, i, vp]
    L.moex_attn_gqa.argtypes = [vp, KVCache, i, i, vp, i, vp, i, i, vp]
    L.moex_attn_gqa_out.argtypes = [vp, KVCache, i, i, vp, i, vp, i, i, vp]
    L.moex_attn_combine.argtypes = [vp, vp, vp, i, i, i, i, vp]
    L.moex_attn_decode_heads.argtypes = [vp, vp, KVCache, vp, i, i, vp, i, i, vp, i, i, vp]
    L.moex_turbo_out.argtypes = [vp, vp, i, i, i, vp]
    L.moex_set_int.argtypes = [vp, i, vp]
    L.moex_set_soft_error.argtypes = [vp]
    L.moex_set_skip.argtypes = [i, vp]
    L.moex_fa_on.restype = i
    L.moex_fa_supported.restype = i
    L.moex_decode_splits.argtypes = [i]
    L.moex_decode_splits.restype = i
    L.moex_gqa_splits.argtypes = [i, i, i, i]
    L.moex_gqa_splits.restype = i
    L.moex_version.restype = ctypes.c_char_p
    L.moex_attn_workspace_bytes.argtypes = [i, i, i, i]
    L.moex_attn_workspace_bytes.restype = ctypes.c_size_t
    L.moex_workspace_held.restype = ctypes.c_size_t
    L.moex_quantize_rows_i8.argtypes = [vp, vp, vp, i, i, vp]
    L.moex_gemv_i8.argtypes = [vp, vp, vp, vp, i, i, vp]
    L.moex_gemm_i8.argtypes = [vp, vp, vp, vp, i, i, i, vp]
    L.moex_quantize_rows_q4.argtypes = [vp, vp, vp, i, i, vp]
    L.moex_quantize_rows_q6.argtypes = [vp, vp, vp, vp, i, i, vp]
    L.moex_gemv.argtypes = [ctypes.POINTER(Mat), vp, vp, i, i, vp]
    L.moex_gemm.argtypes = [ctypes.POINTER(Mat), vp, vp, i, i, i, vp]
    _lib = L
    return L


EXPORTS = ["moex_kv_alloc", "moex_kv_bytes", "moex_kv_free", "moex_attn_decode", "moex_attn_decode_noalloc", "moex_attn_fa", "moex_attn_prefill",
           "moex_qk_norm_rope", "moex_kv_append", "moex_attn_gqa", "moex_attn_gqa_out", "moex_attn_combine", "moex_attn_decode_heads",
           "moex_turbo_out", "moex_set_int", "moex_set_soft_error", "moex_set_skip", "moex_fa_on",
           "moex_fa_supported", "moex_decode_splits", "moex_gqa_splits", "moex_version",
           "moex_attn_workspace_bytes", "moex_workspace_held",
           "moex_quantize_rows_i8", "moex_gemv_i8", "moex_gemm_i8", "moex_quantize_rows_q4", "moex_quantize_rows_q6",
           "moex_gemv", "moex_gemm"]


def _p(x):
    """device pointer of a torch tensor / int / None"""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _s(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


# ---- cache storage ----
class DeviceKVCache:
    """A KVCache whose arrays are torch tensors (caller-owned device memory, like the engine's buffers)."""

    def __init__(self, KV, max_t, turbo=False, device="cuda"):
        import torch
        self.KV, self.max_t, self.turbo = KV, max_t, int(bool(turbo))
        kb, vb, ns = (TQ_KB, TQ_VB, 2) if turbo else (AHD, AHD, 1)
        self.k = torch.empty((KV, max_t, kb), dtype=torch.int8 if not turbo else torch.uint8, device=device)
        self.v = torch.empty((KV, max_t, vb), dtype=torch.int8 if not turbo else torch.uint8, device=device)
        shape = (KV, max_t, 2) if turbo else (KV, max_t)
        self.ks = torch.empty(shape, dtype=torch.float32, device=device)
        self.vs = torch.empty(shape, dtype=torch.float32, device=device)

    @property
    def c(self):
        return KVCache(self.k.data_ptr(), self.v.data_ptr(), self.ks.data_ptr(), self.vs.data_ptr(), self.turbo)


def kv_alloc(KV, max_t, turbo=0):
    """kv_alloc (kernels.cuh:1867): library-owned arrays (free with kv_free)."""
    return lib().moex_kv_alloc(KV, max_t, turbo)


def kv_free(kv):
    lib().moex_kv_free(kv)


def kv_bytes(KV, max_t, turbo):
    """kv_bytes (kernels.cuh:1875)."""
    return lib().moex_kv_bytes(KV, max_t, turbo)


def _kv(kv):
    return kv.c if isinstance(kv, DeviceKVCache) else kv


# ---- entry points (reference names and argument order) ----
def attn_decode(q, k, v, qn, kn, qo, kv, out, H, KV, pos_d, max_t, rot, theta, eps, T, ld, st=None, part=None, ns=1):
    """attn_decode (kernels.cuh:1850): norm + RoPE + KV append + attention + gate."""
    lib().moex_attn_decode(_p(q), _p(k), _p(v), _p(qn), _p(kn), _p(qo), _kv(kv), _p(out), H, KV, _p(pos_d), max_t,
                           rot, theta, eps, T, ld, _s(st), _p(part), ns)


def attn_decode_noalloc(q, k, v, qn, kn, qo, kv, out, H, KV, pos_d, max_t, rot, theta, eps, T, ld, st=None, ns=1):
    """attn_decode without part: the split partials in the library's own device array (no allocation)."""
    lib().moex_attn_decode_noalloc(_p(q), _p(k), _p(v), _p(qn), _p(kn), _p(qo), _kv(kv), _p(out), H, KV, _p(pos_d),
                                   max_t, rot, theta, eps, T, ld, _s(st), ns)


def attn_fa(qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, T, st=None):
    """attn_fa (kernels.cuh:1713): FA-2 causal prefill (q_gate None: no gate)."""
    lib().moex_attn_fa(_p(qo), _p(q_gate), _kv(kv), _p(out), H, KV, _p(pos_d), max_t, ld, T, _s(st))


def attn_prefill(qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, T, st=None):
    """attn_prefill (kernels.cuh:1435): int8 prefill fallback."""
    lib().moex_attn_prefill(_p(qo), _p(q_gate), _kv(kv), _p(out), H, KV, _p(pos_d), max_t, ld, T, _s(st))


def qk_norm_rope(q, k, v, qn, kn, qo, kv, H, KV, pos_d, max_t, rot, theta, eps, ld, T, st=None):
    """qk_norm_rope_k (kernels.cuh:1185)."""
    lib().moex_qk_norm_rope(_p(q), _p(k), _p(v), _p(qn), _p(kn), _p(qo), _kv(kv), H, KV, _p(pos_d), max_t, rot, theta,
                            eps, ld, T, _s(st))


def kv_append(k, v, kv, KV, pos_d, max_t, ld, T, st=None):
    """quantize-append of already normalized/rotated k and raw v (kernels.cuh:1210-1235)."""
    lib().moex_kv_append(_p(k), _p(v), _kv(kv), KV, _p(pos_d), max_t, ld, T, _s(st))


def attn_gqa(qo, kv, H, KV, pos_d, max_t, part, T, ns, st=None):
    """attn_gqa_k (kernels.cuh:1745), grid (KV, T, ns)."""
    lib().moex_attn_gqa(_p(qo), _kv(kv), H, KV, _p(pos_d), max_t, _p(part), T, ns, _s(st))


def attn_gqa_out(qo, kv, H, KV, pos_d, max_t, part, T, ns, st=None):
    """attn_gqa whose turbo partials are rotated back (combine with the gate then gives the output; no turbo_out)."""
    lib().moex_attn_gqa_out(_p(qo), _kv(kv), H, KV, _p(pos_d), max_t, _p(part), T, ns, _s(st))


def attn_combine(part, q_gate, out, H, ns, ld, T, st=None):
    """attn_combine_k (kernels.cuh:1317), grid (H, T)."""
    lib().moex_attn_combine(_p(part), _p(q_gate), _p(out), H, ns, ld, T, _s(st))


def attn_decode_heads(qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, part, T, ns, st=None):
    """attn_decode_k (kernels.cuh:1244), grid (H, T, ns)."""
    lib().moex_attn_decode_heads(_p(qo), _p(q_gate), _kv(kv), _p(out), H, KV, _p(pos_d), max_t, ld, _p(part), T, ns,
                                 _s(st))


def turbo_out(out, q_gate, H, ld, T, st=None):
    """turbo_out_k (kernels.cuh:1731)."""
    lib().moex_turbo_out(_p(out), _p(q_gate), H, ld, T, _s(st))


def set_int(p, v, st=None):
    """set_int_k (kernels.cuh:1879)."""
    lib().moex_set_int(_p(p), v, _s(st))


def set_skip(v, st=None):
    lib().moex_set_skip(v, _s(st))


def decode_splits(n_ctx):
    return lib().moex_decode_splits(n_ctx)


def gqa_splits(T, KV, ns, turbo=0):
    """split count moex_attn_decode uses for the GQA kernel when allowed ns (pass it to attn_gqa and attn_combine)"""
    return lib().moex_gqa_splits(T, KV, ns, int(turbo))


def fa_on():
    return bool(lib().moex_fa_on())


def fa_supported():
    return bool(lib().moex_fa_supported())


def attn_workspace_bytes(H, KV, max_t, T):
    """Workspace bytes one attn_fa call of these sizes takes on its stream (for a VRAM audit beside kv_bytes)."""
    return int(lib().moex_attn_workspace_bytes(H, KV, max_t, T))


def workspace_held():
    """Bytes the library's per-stream workspaces hold now."""
    return int(lib().moex_workspace_held())


# ---- dense int8 projections (include/moex_dense.h): the qkv projection before attn_decode, o_proj after it ----
def quantize_rows_i8(W, q, s, O, I, st=None):
    """quantize_rows_i8_k (kernels.cuh:144-156): fp16 W [O][I] -> int8 q [O][I] + fp32 s [O] (absmax/127)."""
    lib().moex_quantize_rows_i8(_p(W), _p(q), _p(s), O, I, _s(st))


def gemv_i8(q, s, x, y, I, O, st=None):
    """gemv(Mat{q, s}, x, y, I, O) (kernels.cuh:214-219, gemv_i8 :98-141): y = s * (q . x)."""
    lib().moex_gemv_i8(_p(q), _p(s), _p(x), _p(y), I, O, _s(st))


def gemm_i8(q, s, X, Y, S, I, O, st=None):
    """gemm(Mat{q, s}, X, Y, S, I, O) (kernels.cuh:339-350): S <= 8 one GEMV pass, else the fp16 MFMA GEMM."""
    lib().moex_gemm_i8(_p(q), _p(s), _p(X), _p(Y), S, I, O, _s(st))


def quantize_rows_q4(W, q4, s, O, I, st=None):
    """quantize_rows_q4_k (kernels.cuh:576-590): fp16 W [O][I] -> int4 gs64 q4 [O][I/2] + fp32 s [O][I/64]."""
    lib().moex_quantize_rows_q4(_p(W), _p(q4), _p(s), O, I, _s(st))


def quantize_rows_q6(W, q6, q6h, s, O, I, st=None):
    """quantize_rows_q6_k (kernels.cuh:552-573): fp16 W [O][I] -> int6 gs64 planes q6 [O][I/2], q6h [O][I/4] + s."""
    lib().moex_quantize_rows_q6(_p(W), _p(q6), _p(q6h), _p(s), O, I, _s(st))


def gemv(m, x, y, I, O, st=None):
    """gemv(const Mat&, x, y, I, O) (kernels.cuh:214-219) for a Mat in any form."""
    lib().moex_gemv(ctypes.byref(m), _p(x), _p(y), I, O, _s(st))


def gemm(m, X, Y, S, I, O, st=None):
    """gemm(const Mat&, X, Y, S, I, O) (kernels.cuh:339-369) for a Mat in any form."""
    lib().moex_gemm(ctypes.byref(m), _p(X), _p(Y), S, I, O, _s(st))

