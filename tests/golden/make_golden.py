"""Writes the golden vectors under tests/golden/ by running the reference itself.

The reference (LucianCrainic/llama3.x.c) is C; oracle/Makefile's `ref` target compiles its own sources into
oracle/_ref/libllama_ref.so (this container only: the sources are not on the GPU box). This script loads that
library, selects the reference's scalar instruction set (kernels_select(KERNELS_SCALAR), include/kernels.h:15-17) so the
portable kernels run, feeds it seeded inputs and stores inputs and outputs as small .npz fixtures. The tests check the
CPU oracle against these fixtures bit for bit, and the GPU kernels against the oracle.

Usage: python tests/golden/make_golden.py   (rebuilds oracle/_ref first)
"""
import ctypes
import hashlib
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle import pyoracle as orc  # noqa: E402  (the seeded generator only)

P = ctypes.c_void_p
KERNELS_SCALAR, KERNELS_AVX512 = 0, 1


class K8Weight(ctypes.Structure):  # include/kernels.h:101-104
    _fields_ = [("q", P), ("s", P)]


class K8Input(ctypes.Structure):  # include/kernels.h:105-109
    _fields_ = [("q", P), ("s", P), ("f", P)]


class GemmSegment(ctypes.Structure):  # include/gemm.h:22-30
    _fields_ = [("c", P), ("ldc", ctypes.c_int), ("w", P), ("w3", P), ("ldw", ctypes.c_size_t), ("n", ctypes.c_int),
                ("kind", ctypes.c_int)]


class GemmBf16Segment(ctypes.Structure):  # include/gemm.h:89-96
    _fields_ = [("c", P), ("ldc", ctypes.c_int), ("w", P), ("w3", P), ("n", ctypes.c_int), ("kind", ctypes.c_int)]


class GemmQ8Segment(ctypes.Structure):  # include/gemm.h:118-125
    _fields_ = [("c", P), ("ldc", ctypes.c_int), ("w", K8Weight), ("w3", K8Weight), ("pw", P), ("pw3", P),
                ("n", ctypes.c_int), ("kind", ctypes.c_int)]


class AlignedBuffer(ctypes.Structure):  # include/gemm.h:78-81
    _fields_ = [("base", P), ("data", P), ("bytes", ctypes.c_size_t)]


def ptr(a):
    return None if a is None else a.ctypes.data_as(P)


def load_reference():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref"], check=True)
    L = ctypes.CDLL(os.path.join(ROOT, "oracle", "_ref", "libllama_ref.so"))
    L.kernels_select.restype = ctypes.c_int
    L.bf16_from_f32.restype = ctypes.c_uint16
    L.bf16_from_f32.argtypes = [ctypes.c_float]
    L.bf16_vnni_elements.restype = ctypes.c_size_t
    L.s8_vnni_bytes.restype = ctypes.c_size_t
    L.k_gemm_bf16_panel_bytes.restype = ctypes.c_size_t
    L.gemm_amx_unavailable.restype = ctypes.c_char_p
    return L


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def ref_quantize(L, x, gs):
    n = x.shape[-1]
    q = np.zeros(n, np.int8)
    s = np.zeros(n // gs, np.float32)
    L.k_quantize(ptr(q), ptr(s), ptr(x), n, gs)
    return q, s


def quantize_cases(L):
    """k_quantize (src/gemv.c:589-624) on seeded, crafted and edge inputs, scalar and AVX-512 (bitwise equal there)."""
    rng = orc.Rng()
    cases = {}
    for n in (2048, 4096, 8192, 14336):
        cases[f"normal_{n}"] = (rng.normal(n, 0.0, 1.0), 64)
    # roundf ties with scale exactly 1 (group max 127), after tests/kernels.c:110-116, then every .5 in range
    ties = np.zeros(64, np.float32)
    ties[:8] = [127, 2.5, -3.5, 0.5, -0.5, 1.5, -126.5, 0]
    ties[8:] = np.arange(-27.5, 28.5, 1.0, dtype=np.float32)[:56]
    cases["ties"] = (ties, 64)
    halves = np.concatenate([[127.0], np.arange(-126.5, 127, 2.0)[:63]]).astype(np.float32)
    cases["halves"] = (halves, 64)
    # a zero group, negative zeros, a subnormal scale, a scale that underflows to zero, huge values, clamp edges
    edge = np.zeros(6 * 64, np.float32)
    edge[64:128] = -0.0
    edge[128:192] = rng.uniform(64) * 1e-39
    edge[192:256] = np.float32(1.4e-45) * np.sign(rng.uniform(64))
    edge[256:320] = rng.uniform(64) * 3.0e38
    edge[320:384] = rng.uniform(64)
    edge[320] = 1.0
    edge[321] = -1.0
    cases["edges"] = (edge, 64)
    for gs in (2, 4, 16, 32, 128):
        cases[f"gs{gs}"] = (rng.normal(256, 0.0, 2.0), gs)
    out = {}
    for name, (x, gs) in cases.items():
        x = np.ascontiguousarray(x, np.float32)
        assert L.kernels_select(KERNELS_SCALAR)
        q, s = ref_quantize(L, x, gs)
        if gs % 16 == 0 and L.kernels_select(KERNELS_AVX512):
            q2, s2 = ref_quantize(L, x, gs)
            assert np.array_equal(q, q2) and np.array_equal(s.view(np.uint32), s2.view(np.uint32)), name
        out[f"{name}/x"], out[f"{name}/gs"], out[f"{name}/q"], out[f"{name}/s"] = x, np.int32(gs), q, s
    return out


def synth_q8_weights(L, rng, d, n, gs, std=0.02):
    w = rng.normal(d * n, 0.0, std).reshape(d, n)
    q = np.zeros((d, n), np.int8)
    s = np.zeros((d, n // gs), np.float32)
    assert L.kernels_select(KERNELS_SCALAR)
    for r in range(d):
        L.k_quantize(ptr(q[r]), ptr(s[r]), ptr(w[r]), n, gs)
    return q, s


def gemv_cases(L):
    """The scalar Q8 GEMV entry points (src/gemv.c:512-528, 565-587) and the C1 workload."""
    out = {}
    assert L.kernels_select(KERNELS_SCALAR)
    # C1: W 2048x2048 ~ N(0, 0.02) quantized Q8_0 gs 64, x 2048 ~ N(0, 1) quantized by k_quantize; inputs are
    # regenerated by the tests from the same stream, so only their digest and the output are stored.
    rng = orc.Rng()
    wq, ws = synth_q8_weights(L, rng, 2048, 2048, 64)
    x = rng.normal(2048, 0.0, 1.0)
    xq, xs = ref_quantize(L, x, 64)
    y = np.zeros(2048, np.float32)
    L.k_matmul_q8(ptr(y), ctypes.byref(K8Input(ptr(xq), ptr(xs), ptr(x))), K8Weight(ptr(wq), ptr(ws)), 2048, 2048, 64)
    out["c1/digest"] = np.frombuffer(digest(wq, ws, x, xq, xs).encode(), np.uint8)
    out["c1/y"] = y
    assert L.kernels_select(KERNELS_AVX512)
    y2 = np.zeros(2048, np.float32)
    L.k_matmul_q8(ptr(y2), ctypes.byref(K8Input(ptr(xq), ptr(xs), ptr(x))), K8Weight(ptr(wq), ptr(ws)), 2048, 2048, 64)
    out["c1/y_avx512"] = y2
    assert L.kernels_select(KERNELS_SCALAR)
    # small shapes, every entry point, W8A8 and W8A32
    i = 0
    for gs in (2, 4, 32, 64, 128):
        for n_groups, d in ((1, 1), (2, 5), (3, 17), (5, 33)):
            n = gs * n_groups
            rng = orc.Rng(orc.SEED + 1000 + i)
            x = rng.normal(n, 0.0, 1.0)
            xq, xs = ref_quantize(L, x, gs)
            mats = [synth_q8_weights(L, rng, d, n, gs) for _ in range(3)]
            base = rng.uniform(d, 3.0)
            key = f"s{i}"
            out[f"{key}/x"], out[f"{key}/gs"], out[f"{key}/base"] = x, np.int32(gs), base
            for j, (q, s) in enumerate(mats):
                out[f"{key}/wq{j}"], out[f"{key}/ws{j}"] = q, s
            for mode, inp in (("w8a8", K8Input(ptr(xq), ptr(xs), ptr(x))), ("w8a32", K8Input(None, None, ptr(x)))):
                w0, w1, w2 = (K8Weight(ptr(q), ptr(s)) for q, s in mats)
                y = base.copy()
                L.k_matmul_q8(ptr(y), ctypes.byref(inp), w0, n, d, gs)
                out[f"{key}/{mode}/store"] = y
                y = base.copy()
                L.k_matmul_q8_add(ptr(y), ctypes.byref(inp), w0, n, d, gs)
                out[f"{key}/{mode}/add"] = y
                y = base.copy()
                L.k_matmul_q8_swiglu(ptr(y), ctypes.byref(inp), w0, w1, n, d, gs)
                out[f"{key}/{mode}/swiglu"] = y
                yq, yk, yv = base.copy(), np.zeros(d, np.float32), np.zeros(d, np.float32)
                L.k_matmul_q8_qkv(ptr(yq), ptr(yk), ptr(yv), ctypes.byref(inp), w0, w1, w2, n, d, d, gs)
                out[f"{key}/{mode}/qkv"] = np.concatenate([yq, yk, yv])
            i += 1
    return out


def gemm_q8_cases(L):
    """The portable batched Q8 GEMM (src/gemm.c:839-854, 963-1029) on the scalar instruction set, all kinds, with
    padded output rows (ldc = n + 5), and the exact int32 group dots of the reference's AMX probe where AMX runs."""
    out = {}
    assert L.kernels_select(KERNELS_SCALAR)
    shapes = [(5, 7, 16, 4), (33, 20, 128, 64), (1, 9, 32, 2), (40, 33, 192, 64), (17, 16, 256, 128), (3, 5, 320, 64)]
    for i, (m, n, k, gs) in enumerate(shapes):
        rng = orc.Rng(orc.SEED + 2000 + i)
        x = rng.normal(m * k, 0.0, 1.0).reshape(m, k)
        xq = np.zeros((m, k), np.int8)
        xs = np.zeros((m, k // gs), np.float32)
        L.k_quantize_rows(ptr(xq), ptr(xs), ptr(x), ctypes.c_size_t(k), m, k, gs)
        (wq, ws), (w3q, w3s) = synth_q8_weights(L, rng, n, k, gs), synth_q8_weights(L, rng, n, k, gs)
        ldc = n + 5
        base = rng.uniform(m * ldc, 3.0).reshape(m, ldc)
        key = f"g{i}"
        out[f"{key}/shape"] = np.array([m, n, k, gs], np.int32)
        for name, a in (("x", x), ("xq", xq), ("xs", xs), ("wq", wq), ("ws", ws), ("w3q", w3q), ("w3s", w3s),
                        ("base", base)):
            out[f"{key}/{name}"] = a
        for kind, kname in ((0, "store"), (1, "add"), (2, "swiglu"), (3, "partial")):
            c = base.copy()
            seg = GemmQ8Segment(ptr(c), ldc, K8Weight(ptr(wq), ptr(ws)), K8Weight(ptr(w3q), ptr(w3s)), None, None, n,
                                kind)
            L.k_gemm_q8(ptr(xq), ptr(xs), m, k, gs, ctypes.byref(seg), 1)
            out[f"{key}/{kname}"] = c
        if gs % 64 == 0 and L.gemm_amx_unavailable() is None:
            packed = np.zeros(L.s8_vnni_bytes(n, k), np.int8)
            L.pack_s8_vnni(ptr(packed), ptr(wq), n, k, ctypes.c_size_t(k))
            dots = np.zeros((k // gs, m, n), np.int32)
            xpad = np.zeros(((m + 31) // 32 * 32, k), np.int8)
            xpad[:m] = xq
            if L.k_gemm_q8_amx_dots_test(ptr(dots), ptr(xpad), m, k, gs, ptr(packed), n):
                out[f"{key}/amx_dots"] = dots
    return out


def f32_cases(L):
    """Scalar FP32 GEMV (src/gemv.c:252-396) and the portable FP32 GEMM with one K block (k_gemm_f32_portable, kc 0)."""
    out = {}
    assert L.kernels_select(KERNELS_SCALAR)
    L.k_gemm_f32_portable.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, ctypes.c_int, ctypes.c_int]
    for i, (m, n, k) in enumerate([(1, 7, 16), (5, 17, 33), (9, 33, 100), (4, 16, 256)]):
        rng = orc.Rng(orc.SEED + 3000 + i)
        lda, ldc = k + 3, n + 7
        a = rng.uniform(m * lda, 2.0).reshape(m, lda)
        w, w3 = rng.uniform(n * k).reshape(n, k), rng.uniform(n * k).reshape(n, k)
        base = rng.uniform(m * ldc, 4.0).reshape(m, ldc)
        key = f"f{i}"
        for name, arr in (("a", a), ("w", w), ("w3", w3), ("base", base)):
            out[f"{key}/{name}"] = arr
        out[f"{key}/shape"] = np.array([m, n, k], np.int32)
        for kind, kname in ((0, "store"), (1, "add"), (2, "swiglu")):
            c = base.copy()
            seg = GemmSegment(ptr(c), ldc, ptr(w), ptr(w3), k, n, kind)
            L.k_gemm_f32_portable(ptr(a), lda, m, k, ctypes.byref(seg), 1, 0)
            out[f"{key}/gemm_{kname}"] = c
        x = np.ascontiguousarray(a[0, :k])
        for kname, fn in (("store", L.k_matmul), ("add", L.k_matmul_add)):
            y = base[0, :n].copy()
            fn(ptr(y), ptr(x), ptr(w), k, n)
            out[f"{key}/gemv_{kname}"] = y
        y = base[0, :n].copy()
        L.k_matmul_swiglu(ptr(y), ptr(x), ptr(w), ptr(w3), k, n)
        out[f"{key}/gemv_swiglu"] = y
    return out


def bf16_cases(L):
    """bf16_from_f32 (src/gemm.c:335-342) on the specials of tests/bf16.c:101-112, ties and a strided sweep; the packing
    helpers (src/gemm.c:355-398); the portable BF16 GEMM (src/gemm.c:667-771) on the scalar instruction set."""
    out = {}
    specials = [0x00000000, 0x80000000, 0x7f800000, 0xff800000, 0x7fc00000, 0xffc00000, 0x7f800001, 0xff800001,
                0x7f80ffff, 0x7fffffff, 0xffffffff, 0x7f7fffff, 0xff7fffff, 0x7f7f8000, 0x7f7f7fff, 0x7f7f0000,
                0x00000001, 0x00007fff, 0x00008000, 0x00008001, 0x00018000, 0x0000ffff, 0x00010000, 0x007fffff,
                0x00800000, 0x807fffff, 0x80000001, 0x80008000]
    bits = list(specials)
    for e in range(0, 256, 3):
        for mh in (0, 1, 63, 127):
            for low in (0x7fff, 0x8000, 0x8001):
                u = (e << 23) | (mh << 16) | low
                bits += [u, u | 0x80000000]
    bits += list(range(0, 1 << 32, 0x10001 * 97))
    bits = np.array(bits, np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    out["convert/bits"] = bits
    # Converted memory to memory through the reference's own packer (a 1-row matrix: column l lands at element
    # (l / 2) * 32 + l % 2), so NaN payloads never pass through a Python float.
    cols = len(vals)
    packed = np.zeros(L.bf16_vnni_elements(1, cols), np.uint16)
    L.pack_bf16_vnni(ptr(packed), ptr(vals), 1, cols, ctypes.c_size_t(cols))
    idx = np.arange(cols)
    out["convert/bf16"] = packed[(idx // 2) * 32 + (idx % 2)]
    assert L.kernels_select(KERNELS_SCALAR)
    for i, (m, n, k) in enumerate([(1, 5, 8), (5, 17, 40), (17, 33, 64), (3, 16, 97)]):
        rng = orc.Rng(orc.SEED + 4000 + i)
        lda, ldc = k + 3, n + 7
        a = rng.uniform(m * lda, 2.0).reshape(m, lda)
        w, w3 = rng.uniform(n * k).reshape(n, k), rng.uniform(n * k).reshape(n, k)
        base = rng.uniform(m * ldc, 4.0).reshape(m, ldc)
        pw = np.zeros(L.bf16_vnni_elements(n, k), np.uint16)
        pw3 = np.zeros_like(pw)
        L.pack_bf16_vnni(ptr(pw), ptr(w), n, k, ctypes.c_size_t(k))
        L.pack_bf16_vnni(ptr(pw3), ptr(w3), n, k, ctypes.c_size_t(k))
        wi = (rng.uniform(n * k) * 127).astype(np.int8).reshape(n, k)
        ps = np.zeros(L.s8_vnni_bytes(n, k), np.int8)
        L.pack_s8_vnni(ptr(ps), ptr(wi), n, k, ctypes.c_size_t(k))
        key = f"b{i}"
        for name, arr in (("a", a), ("w", w), ("w3", w3), ("base", base), ("pw", pw), ("wi", wi), ("ps", ps)):
            out[f"{key}/{name}"] = arr
        out[f"{key}/shape"] = np.array([m, n, k], np.int32)
        panel_bytes = L.k_gemm_bf16_panel_bytes(m, k)
        raw = np.zeros(panel_bytes + 64, np.uint8)
        base_addr = raw.ctypes.data
        aligned = (base_addr + 63) // 64 * 64
        panel = AlignedBuffer(ctypes.c_void_p(base_addr), ctypes.c_void_p(aligned), panel_bytes)
        for kind, kname in ((0, "store"), (1, "add"), (2, "swiglu")):
            c = base.copy()
            seg = GemmBf16Segment(ptr(c), ldc, ptr(pw), ptr(pw3), n, kind)
            L.k_gemm_bf16(ptr(a), lda, m, k, ctypes.byref(seg), 1, ctypes.byref(panel))
            out[f"{key}/{kname}"] = c
    return out


def main():
    L = load_reference()
    groups = {"quantize": quantize_cases, "gemv_q8": gemv_cases, "gemm_q8": gemm_q8_cases, "f32": f32_cases,
              "bf16": bf16_cases}
    for name, fn in groups.items():
        data = fn(L)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **data)
        print(f"{path}: {len(data)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
