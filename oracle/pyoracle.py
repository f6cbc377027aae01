"""ctypes view of the CPU oracle (liboracle.so). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, as the checker; the shipped
library never does. Each wrapper names the reference function it restates (see oracle.h for file:line citations).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")

# KernelEpilogue (reference include/kernels.h:82) and GemmKind (include/gemm.h:15-20).
K_STORE, K_ADD, K_PARTIAL, K_SWIGLU = 0, 1, 2, 3
GEMM_STORE, GEMM_ADD, GEMM_SWIGLU, GEMM_PARTIAL = 0, 1, 2, 3
SEED = 88172645463325252  # the reference tests' xorshift64 seed (tests/q8.c:19)

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = ctypes.c_void_p


def _declare(L):
    sz, i32, u64, f32 = ctypes.c_size_t, ctypes.c_int, ctypes.c_uint64, ctypes.c_float
    sig = {
        "orc_quantize": (i32, [P, P, P, i32, i32]),
        "orc_quantize_rows": (i32, [P, P, P, sz, i32, i32, i32]),
        "orc_silu_gate": (f32, [f32, f32]),
        "orc_q8_dots": (None, [P, P, P, sz, i32, P, P, P, i32, i32]),
        "orc_matmul_q8": (None, [P, P, P, P, P, P, P, P, sz, i32, i32, i32, i32]),
        "orc_group_dots": (None, [P, P, sz, i32, P, sz, i32, i32, i32]),
        "orc_gemm_q8": (None, [P, P, i32, i32, i32, P, i32, P, P, P, P, i32, i32]),
        "orc_matmul_f32": (None, [P, P, P, P, sz, i32, i32, i32]),
        "orc_gemm_f32": (None, [P, i32, i32, i32, P, i32, P, P, sz, i32, i32]),
        "orc_bf16_from_f32": (ctypes.c_uint16, [f32]),
        "orc_f32_from_bf16": (f32, [ctypes.c_uint16]),
        "orc_bf16_vnni_elements": (sz, [i32, i32]),
        "orc_s8_vnni_bytes": (sz, [i32, i32]),
        "orc_pack_bf16_vnni": (None, [P, P, i32, i32, sz]),
        "orc_pack_s8_vnni": (None, [P, P, i32, i32, sz]),
        "orc_gemm_bf16": (None, [P, i32, i32, i32, P, i32, P, P, i32, i32]),
        "orc_matmul_q8_threads": (None, [P, P, P, P, P, i32, i32, i32, i32]),
        "orc_rmsnorm": (None, [P, P, P, i32, f32]),
        "orc_rope_apply": (None, [P, P, P, i32, i32, i32]),
        "orc_kv_store": (None, [P, P, sz, i32, i32, i32, i32, sz, sz]),
        "orc_attention": (i32, [P, P, P, P, P, i32, i32, i32, i32, i32, sz, sz]),
        "orc_rng_next": (u64, [P]),
        "orc_rng_uniform": (f32, [P]),
        "orc_fill_uniform": (None, [P, sz, P, f32]),
        "orc_fill_normal": (None, [P, sz, P, f32, f32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def ptr(a):
    return None if a is None else a.ctypes.data_as(P)


class Rng:
    """The reference tests' xorshift64 stream (tests/q8.c:19-30), advanced in C."""

    def __init__(self, seed=SEED):
        self.state = ctypes.c_uint64(seed)

    def uniform(self, n, scale=1.0):
        out = np.empty(n, np.float32)
        lib().orc_fill_uniform(ptr(out), n, ctypes.byref(self.state), scale)
        return out

    def normal(self, n, mean=0.0, std=1.0):
        out = np.empty(n, np.float32)
        lib().orc_fill_normal(ptr(out), n, ctypes.byref(self.state), mean, std)
        return out

    def int8(self, n):
        """Uniform int8 in [-127, 127] as tests/q8.c:71 draws them: (next() % 255) - 127."""
        out = np.empty(n, np.int8)
        L = lib()
        for i in range(n):
            out[i] = int(L.orc_rng_next(ctypes.byref(self.state)) % 255) - 127
        return out


def quantize(x, gs):
    """k_quantize (src/gemv.c:589-624) over the last axis of x; raises on a non-finite value."""
    x = np.ascontiguousarray(x, np.float32)
    rows = x.reshape(-1, x.shape[-1])
    m, n = rows.shape
    q = np.zeros((m, n), np.int8)
    s = np.zeros((m, n // gs), np.float32)
    if lib().orc_quantize_rows(ptr(q), ptr(s), ptr(rows), n, m, n, gs):
        raise FloatingPointError("nonfinite activation during INT8 quantization")
    return q.reshape(x.shape), s.reshape(x.shape[:-1] + (n // gs,))


def matmul_q8(xq, xs, wq, ws, gs, kind=K_STORE, out=None, w3q=None, w3s=None, xf=None, ld=0):
    """k_matmul_q8 / _add / _swiglu / _ld on the scalar instruction set (src/gemv.c:401-528, 565-587)."""
    d = wq.shape[0]
    n = xf.shape[-1] if xq is None else xq.shape[-1]
    if ld == 0:
        ld = wq.shape[1]
    out = np.zeros(d, np.float32) if out is None else out
    lib().orc_matmul_q8(ptr(out), ptr(xq), ptr(xs), ptr(xf), ptr(wq), ptr(ws), ptr(w3q), ptr(w3s), ld, n, d, gs, kind)
    return out


def group_dots(xq, wq, gs):
    m, k = xq.shape
    n = wq.shape[0]
    dots = np.zeros((k // gs, m, n), np.int32)
    lib().orc_group_dots(ptr(dots), ptr(xq), xq.strides[0], m, ptr(wq), wq.strides[0], n, k, gs)
    return dots


def gemm_q8(xq, xs, wq, ws, gs, kind=GEMM_STORE, c=None, w3q=None, w3s=None):
    m, k = xq.shape
    n = wq.shape[0]
    c = np.zeros((m, n), np.float32) if c is None else c
    lib().orc_gemm_q8(ptr(xq), ptr(xs), m, k, gs, ptr(c), c.strides[0] // 4, ptr(wq), ptr(ws), ptr(w3q), ptr(w3s), n,
                      kind)
    return c


def matmul_f32(x, w, kind=K_STORE, out=None, w3=None):
    d, n = w.shape
    out = np.zeros(d, np.float32) if out is None else out
    lib().orc_matmul_f32(ptr(out), ptr(x), ptr(w), ptr(w3), w.strides[0] // 4, n, d, kind)
    return out


def gemm_f32(a, w, kind=GEMM_STORE, c=None, w3=None):
    m, k = a.shape
    n = w.shape[0]
    c = np.zeros((m, n), np.float32) if c is None else c
    lib().orc_gemm_f32(ptr(a), a.strides[0] // 4, m, k, ptr(c), c.strides[0] // 4, ptr(w), ptr(w3), w.strides[0] // 4,
                       n, kind)
    return c


def bf16_from_f32(x):
    x = np.ascontiguousarray(x, np.float32).ravel()
    L = lib()
    return np.array([L.orc_bf16_from_f32(float(v)) for v in x], np.uint16)


def pack_bf16_vnni(w):
    rows, cols = w.shape
    dst = np.zeros(lib().orc_bf16_vnni_elements(rows, cols), np.uint16)
    lib().orc_pack_bf16_vnni(ptr(dst), ptr(w), rows, cols, w.strides[0] // 4)
    return dst


def pack_s8_vnni(w):
    rows, cols = w.shape
    dst = np.zeros(lib().orc_s8_vnni_bytes(rows, cols), np.int8)
    lib().orc_pack_s8_vnni(ptr(dst), ptr(w), rows, cols, w.strides[0])
    return dst


def gemm_bf16(a, pw, n, kind=GEMM_STORE, c=None, pw3=None):
    m, k = a.shape
    c = np.zeros((m, n), np.float32) if c is None else c
    lib().orc_gemm_bf16(ptr(a), a.strides[0] // 4, m, k, ptr(c), c.strides[0] // 4, ptr(pw), ptr(pw3), n, kind)
    return c


def rmsnorm(x, weight, eps=1e-5):
    """k_rmsnorm / k_rmsnorm_rows (src/kernels.c:8-21), row by row; x (size,) or (rows, size)."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    rows = x.reshape(-1, x.shape[-1])
    o = out.reshape(rows.shape)
    for r in range(rows.shape[0]):
        lib().orc_rmsnorm(ptr(o[r]), ptr(rows[r]), ptr(weight), rows.shape[1], eps)
    return out


def rope_apply(q, k, table, n_heads, n_kv_heads, head_dim):
    """k_rope_apply (src/kernels_simd.c:203-225) on copies of one row's q and k."""
    q, k = np.array(q, np.float32), np.array(k, np.float32)
    lib().orc_rope_apply(ptr(q), ptr(k), ptr(np.ascontiguousarray(table, np.float32)), n_heads, n_kv_heads, head_dim)
    return q, k


def kv_strides(n_kv_heads, head_dim, seq_len, head_major):
    """(pos_stride, head_base) of the rows or head-major K/V layout (src/attention.c:1415-1418)."""
    return (head_dim, seq_len * head_dim) if head_major else (n_kv_heads * head_dim, head_dim)


def attention(q, key_cache, value_cache, n_heads, n_kv_heads, head_dim, seq_len, position, pos_stride, head_base):
    """The scalar decode attention (src/attention.c:606-641) for one position; None where the reference fails."""
    out = np.zeros(n_heads * head_dim, np.float32)
    att = np.zeros(n_heads * seq_len, np.float32)
    rc = lib().orc_attention(ptr(out), ptr(np.ascontiguousarray(q, np.float32)), ptr(key_cache), ptr(value_cache),
                             ptr(att), n_heads, n_kv_heads, head_dim, seq_len, position, pos_stride, head_base)
    return None if rc else out


def quantize_weights(w, gs):
    """The one documented rule for synthetic Q8_0 weights: the activation rule k_quantize applied per row (roundf,
    half away from zero), so CPU and GPU read the same bytes."""
    return quantize(w, gs)
