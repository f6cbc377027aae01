"""Writes the golden vectors under tests/golden/ by running the reference itself.

The reference (LucianCrainic/llama3.x.c) is C; oracle/Makefile's `ref` target compiles its own sources into
oracle/_ref/libllama_ref.so (only where the reference's sources are; they do not travel with the tests). This
script loads that library, selects the reference's scalar instruction set (kernels_select(KERNELS_SCALAR), include/kernels.h:15-17) so the
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


class Config(ctypes.Structure):  # include/runtime.h:9-16
    _fields_ = [(f, ctypes.c_int) for f in ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size",
                                           "seq_len", "format", "max_seq_len", "shared", "head_dim")] + \
               [(f, ctypes.c_float) for f in ("norm_eps", "rope_theta", "rope_factor", "rope_low", "rope_high")] + \
               [(f, ctypes.c_int) for f in ("rope_type", "rope_original", "bos_id", "eos_id", "eot_id", "eom_id")] + \
               [("name", ctypes.c_char * 128)]


class AttentionWork(ctypes.Structure):  # include/kernels.h:127-132
    _fields_ = [("partial", P), ("max_chunks", ctypes.c_int), ("n_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("workers", ctypes.c_int), ("external", ctypes.c_int), ("capacity", ctypes.c_size_t)]


def rope_config(head_dim, llama3):
    c = Config()
    c.head_dim = head_dim
    if llama3:  # Llama 3.1 scaling
        c.rope_theta, c.rope_type, c.rope_factor, c.rope_low, c.rope_high, c.rope_original = 500000.0, 1, 8.0, 1.0, 4.0, 8192
    else:
        c.rope_theta, c.rope_type = 10000.0, 0
    return c


def forward_cases(L):
    """The forward around the matmuls on the scalar instruction set: k_rmsnorm and _rows (src/kernels.c:8-21,
    src/kernels_simd.c:247-255), k_rope_table and k_rope_apply (src/kernels_simd.c:194-225), the decode attention
    k_attention / k_attention_layout (src/attention.c:606-641, 1362-1377) and the batched k_attention_batch
    (src/attention.c:1379-1384)."""
    rng = orc.Rng(orc.SEED + 900)
    out = {}
    assert L.kernels_select(KERNELS_SCALAR)
    for size in (1, 100, 2048, 3072, 4096):
        x, w = rng.normal(size, 0.0, 2.0), rng.normal(size, 1.0, 0.1)
        o = np.zeros(size, np.float32)
        L.k_rmsnorm(ptr(o), ptr(x), ptr(w), size, ctypes.c_float(1e-5))
        out[f"rms{size}/x"], out[f"rms{size}/w"], out[f"rms{size}/out"] = x, w, o
    xr, wr = rng.normal(3 * 512, 0.0, 1.0).reshape(3, 512), rng.normal(512, 1.0, 0.1)
    orow = np.zeros_like(xr)
    L.k_rmsnorm_rows(ptr(orow), ptr(xr), ptr(wr), 3, 512, ctypes.c_float(1e-5))
    out["rmsrows/x"], out["rmsrows/w"], out["rmsrows/out"] = xr, wr, orow
    for hd, llama3 in ((128, True), (64, False)):
        cfg = rope_config(hd, llama3)
        for pos in (0, 1, 7, 1000, 8191, 100000):
            t = np.zeros(2 * hd, np.float32)
            L.k_rope_table(ctypes.byref(cfg), pos, ptr(t))
            out[f"ropetab{hd}_{pos}/table"] = t
        t = out[f"ropetab{hd}_1000/table"]
        nh, nkv = 8, 2
        q, k = rng.normal(nh * hd, 0.0, 1.0), rng.normal(nkv * hd, 0.0, 1.0)
        out[f"rope{hd}/q"], out[f"rope{hd}/k"] = q.copy(), k.copy()
        L.k_rope_apply(ptr(q), ptr(k), ptr(t), nh, nkv, hd)
        out[f"rope{hd}/q_out"], out[f"rope{hd}/k_out"] = q, k
    for (nh, nkv, hd, seq, pos) in ((4, 2, 16, 8, 0), (4, 2, 16, 8, 7), (8, 2, 64, 48, 47), (32, 8, 128, 20, 19)):
        key = f"att{nh}_{nkv}_{hd}_{seq}_{pos}"
        kv_dim = nkv * hd
        kc, vc = rng.normal(seq * kv_dim, 0.0, 1.0), rng.normal(seq * kv_dim, 0.0, 1.0)
        q = rng.normal(nh * hd, 0.0, 1.0)
        work = AttentionWork()
        L.k_attention_init(ctypes.byref(work), nh, nkv, hd, seq)
        att = np.zeros(nh * seq, np.float32)
        o = np.zeros(nh * hd, np.float32)
        L.k_attention(ptr(o), ptr(q), ptr(kc), ptr(vc), ptr(att), ctypes.byref(work), nh, nkv, hd, seq, pos)
        # the same cache values in the head-major layout [kv_head][position][head_dim]
        kh = np.ascontiguousarray(kc.reshape(seq, nkv, hd).transpose(1, 0, 2)).reshape(-1)
        vh = np.ascontiguousarray(vc.reshape(seq, nkv, hd).transpose(1, 0, 2)).reshape(-1)
        oh = np.zeros(nh * hd, np.float32)
        L.k_attention_layout(ptr(oh), ptr(q), ptr(kh), ptr(vh), ptr(att), ctypes.byref(work), nh, nkv, hd, seq, pos,
                             ctypes.c_size_t(hd), ctypes.c_size_t(seq * hd))
        assert np.array_equal(o.view(np.uint32), oh.view(np.uint32)), key
        out[f"{key}/k"], out[f"{key}/v"], out[f"{key}/q"], out[f"{key}/out"] = kc, vc, q, o
        L.k_attention_free(ctypes.byref(work))
    # batched: m rows at positions pos0 .. pos0 + m - 1 over a cache holding all of them
    nh, nkv, hd, seq, pos0, m = 8, 2, 64, 48, 20, 6
    kv_dim = nkv * hd
    kc, vc = rng.normal(seq * kv_dim, 0.0, 1.0), rng.normal(seq * kv_dim, 0.0, 1.0)
    q = rng.normal(m * nh * hd, 0.0, 1.0)
    work = AttentionWork()
    L.k_attention_bytes_rows.restype = ctypes.c_size_t
    mem = np.zeros(L.k_attention_bytes_rows(nh, nkv, hd, seq, m) // 4 + 16, np.float32)
    L.k_attention_init_rows(ctypes.byref(work), nh, nkv, hd, seq, m, ptr(mem))
    att = np.zeros(m * nh * seq, np.float32)
    o = np.zeros(m * nh * hd, np.float32)
    L.k_attention_batch(ptr(o), ptr(q), ptr(kc), ptr(vc), ptr(att), ctypes.byref(work), nh, nkv, hd, seq, pos0, m)
    out["attbatch/k"], out["attbatch/v"], out["attbatch/q"], out["attbatch/out"] = kc, vc, q, o
    out["attbatch/shape"] = np.array([nh, nkv, hd, seq, pos0, m], np.int32)
    return out


def main():
    L = load_reference()
    groups = {"quantize": quantize_cases, "gemv_q8": gemv_cases, "gemm_q8": gemm_q8_cases, "f32": f32_cases,
              "bf16": bf16_cases, "forward": forward_cases}
    only = sys.argv[1:]
    for name, fn in groups.items():
        if only and name not in only:
            continue
        data = fn(L)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **data)
        print(f"{path}: {len(data)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
