"""GPU parity of the FP32 and BF16 paths through the C ABI: the FP32 GEMV (run's decode), the FP32 GEMM and the BF16
GEMM (batched prefill).

Budgets are the reference's own (float64 references): FP32 GEMV and GEMM 2e-5 * sum|w x| + 1e-6 (tests/gemm.c:405-425,
tests/kernels.c), ADD adds |base|, SWIGLU 2e-5 * (mag (|g| + 1) + mag3 (|r| + 1)) + 1e-6; BF16 2e-6 * sum|w x| + 1e-6
on BF16-rounded operands (tests/bf16.c:158-170). Golden fixtures written by the reference (tests/golden/f32.npz,
bf16.npz) are matched within the same budgets, padded output columns must stay untouched.
"""
import os

import numpy as np
import pytest

import llama_hip as lh
from oracle import pyoracle as orc
from tests import hip_util as hu

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def device():
    L = hu.lib()
    assert L.llhip_init() == 0, lh.last_error()
    yield L


def silu(v):
    return v / (1.0 + np.exp(-v))


def ref_f32(a, w):
    a64, w64 = a.astype(np.float64), w.astype(np.float64)
    return a64 @ w64.T, np.abs(a64) @ np.abs(w64).T


def check_kind(got, base, r, mag, r3, mag3, kind, rel=2e-5, what=""):
    if kind in (lh.GEMM_ADD, "add"):
        hu.assert_within_budget(got, base + r, mag + np.abs(base), rel=rel, what=what)
    elif kind in (lh.GEMM_SWIGLU, "swiglu"):
        tol = 2e-5 * (mag * (np.abs(r3) + 1) + mag3 * (np.abs(r) + 1)) + 1e-6
        err = np.abs(got - silu(r) * r3)
        assert np.all(err <= tol), f"{what}: swiglu outside budget, worst {np.max(err - tol)}"
    else:
        hu.assert_within_budget(got, r, mag, rel=rel, what=what)


# ---- FP32 GEMV -----------------------------------------------------------------------------------------------------


@pytest.mark.parametrize("d,n", [(7, 16), (33, 100), (4096, 4096), (1024, 3072), (129, 14336), (64, 13)])
def test_f32_gemv_all_kinds(d, n):
    L = hu.lib()
    rng = orc.Rng(orc.SEED + 51 * d + n)
    x = rng.uniform(n, 2.0)
    w, w3 = rng.uniform(d * n).reshape(d, n), rng.uniform(d * n).reshape(d, n)
    base = rng.uniform(d, 4.0)
    r, mag = ref_f32(x[None, :], w)
    r3, mag3 = ref_f32(x[None, :], w3)
    r, mag, r3, mag3 = r[0], mag[0], r3[0], mag3[0]
    dx, dw, dw3 = hu.dev(x), hu.dev(w), hu.dev(w3)
    for kind, fn in (("store", L.k_matmul), ("add", L.k_matmul_add)):
        out = hu.dev(base)
        fn(lh.ptr(out), lh.ptr(dx), lh.ptr(dw), n, d)
        check_kind(hu.host(out), base, r, mag, r3, mag3, kind, what=f"k_matmul {kind} {d}x{n}")
    out = hu.dev(base)
    L.k_matmul_swiglu(lh.ptr(out), lh.ptr(dx), lh.ptr(dw), lh.ptr(dw3), n, d)
    check_kind(hu.host(out), base, r, mag, r3, mag3, "swiglu", what=f"k_matmul_swiglu {d}x{n}")
    # QKV: three projections of one input (the reference test's layout: v uses w3)
    q, k, v = hu.empty(d, hu.torch().float32), hu.empty(d, hu.torch().float32), hu.empty(d, hu.torch().float32)
    L.k_matmul_qkv(lh.ptr(q), lh.ptr(k), lh.ptr(v), lh.ptr(dx), lh.ptr(dw), lh.ptr(dw3), lh.ptr(dw3), n, d, d)
    hu.assert_within_budget(hu.host(q), r, mag, what="qkv.q")
    hu.assert_within_budget(hu.host(k), r3, mag3, what="qkv.k")
    hu.assert_within_budget(hu.host(v), r3, mag3, what="qkv.v")


def test_f32_gemv_golden_ld_and_worker():
    g = np.load(os.path.join(GOLDEN, "f32.npz"))
    L = hu.lib()
    for key in sorted({k.split("/")[0] for k in g.files if k.endswith("/shape")}):
        m, n, k = (int(v) for v in g[f"{key}/shape"])
        a, w, w3, base = (g[f"{key}/{x}"] for x in ("a", "w", "w3", "base"))
        x = np.ascontiguousarray(a[0, :k])
        r, mag = ref_f32(x[None, :], w)
        for kname, fn in (("store", L.k_matmul), ("add", L.k_matmul_add)):
            y = base[0, :n].copy()
            fn(lh.ptr(y), lh.ptr(x), lh.ptr(w), k, n)
            want = g[f"{key}/gemv_{kname}"]
            extra = np.abs(base[0, :n]) if kname == "add" else 0
            hu.assert_within_budget(y, want, mag[0] + extra, rel=4e-5, what=f"{key} gemv {kname} vs reference")
        y = base[0, :n].copy()
        L.k_matmul_swiglu(lh.ptr(y), lh.ptr(x), lh.ptr(w), lh.ptr(w3), k, n)
        np.testing.assert_allclose(y, g[f"{key}/gemv_swiglu"], rtol=1e-4, atol=1e-5)
    # shard forms: stride ld > n, static member split
    rng = orc.Rng(orc.SEED + 52)
    d, n, ld = 45, 300, 320
    w = rng.uniform(d * ld).reshape(d, ld)
    x = rng.uniform(n, 2.0)
    r, mag = ref_f32(x[None, :], w[:, :n])
    out = np.zeros(d, np.float32)
    L.k_matmul_ld(lh.ptr(out), lh.ptr(x), lh.ptr(w), ld, n, d, lh.K_PARTIAL)
    hu.assert_within_budget(out, r[0], mag[0], what="k_matmul_ld")
    out = np.zeros(d, np.float32)
    for member in range(4):
        L.k_matmul_ld_worker(lh.ptr(out), lh.ptr(x), lh.ptr(w), ld, n, d, lh.K_STORE, member, 4, None,
                             lh.RowsDoneFn(), None)
    hu.assert_within_budget(out, r[0], mag[0], what="k_matmul_ld_worker union")
    w3 = rng.uniform(d * ld).reshape(d, ld)
    r3, mag3 = ref_f32(x[None, :], w3[:, :n])
    out = np.zeros(d, np.float32)
    L.k_matmul_swiglu_ld(lh.ptr(out), lh.ptr(x), lh.ptr(w), lh.ptr(w3), ld, n, d)
    check_kind(out, 0, r[0], mag[0], r3[0], mag3[0], "swiglu", what="k_matmul_swiglu_ld")


# ---- FP32 GEMM -----------------------------------------------------------------------------------------------------


@pytest.mark.parametrize("m,n,k", [(1, 7, 16), (5, 17, 33), (130, 257, 100), (512, 384, 3072), (64, 96, 8192),
                                   (200, 129, 65)])
def test_f32_gemm_all_kinds(m, n, k):
    L = hu.lib()
    rng = orc.Rng(orc.SEED + 61 * m + n + k)
    lda, ldc = k + 3, n + 7
    a = rng.uniform(m * lda, 2.0).reshape(m, lda)
    w, w3 = rng.uniform(n * k).reshape(n, k), rng.uniform(n * k).reshape(n, k)
    base = rng.uniform(m * ldc, 4.0).reshape(m, ldc)
    r, mag = ref_f32(a[:, :k], w)
    r3, mag3 = ref_f32(a[:, :k], w3)
    da, dw, dw3 = hu.dev(a), hu.dev(w), hu.dev(w3)
    for kind in (lh.GEMM_STORE, lh.GEMM_ADD, lh.GEMM_SWIGLU, lh.GEMM_PARTIAL):
        c = hu.dev(base)
        seg = lh.GemmSegment(lh.ptr(c), ldc, lh.ptr(dw), lh.ptr(dw3), k, n, kind)
        L.k_gemm_f32(lh.ptr(da), lda, m, k, seg, 1)
        got = hu.host(c)
        assert np.array_equal(hu.bits(got[:, n:]), hu.bits(base[:, n:])), "row padding was written"
        check_kind(got[:, :n], base[:, :n], r, mag, r3, mag3, kind, what=f"gemm_f32 {m}x{n}x{k} kind {kind}")


def test_f32_gemm_golden_segments_and_host_buffers():
    g = np.load(os.path.join(GOLDEN, "f32.npz"))
    L = hu.lib()
    for key in sorted({k.split("/")[0] for k in g.files if k.endswith("/shape")}):
        m, n, k = (int(v) for v in g[f"{key}/shape"])
        a, w, w3, base = (g[f"{key}/{x}"] for x in ("a", "w", "w3", "base"))
        r, mag = ref_f32(a[:, :k], w)
        for kname, kind in (("store", 0), ("add", 1), ("swiglu", 2)):
            c = base.copy()  # host buffers: staged through the device
            seg = lh.GemmSegment(lh.ptr(c), c.shape[1], lh.ptr(w), lh.ptr(w3), k, n, kind)
            L.k_gemm_f32_portable(lh.ptr(a), a.shape[1], m, k, seg, 1, 0)
            want = g[f"{key}/gemm_{kname}"]
            assert np.array_equal(hu.bits(c[:, n:]), hu.bits(base[:, n:]))
            if kname == "swiglu":
                np.testing.assert_allclose(c[:, :n], want[:, :n], rtol=1e-4, atol=1e-5)
            else:
                extra = np.abs(base[:, :n]) if kname == "add" else 0
                hu.assert_within_budget(c[:, :n], want[:, :n], mag + extra, rel=4e-5, what=f"{key} {kname}")
    # three segments sharing A
    rng = orc.Rng(orc.SEED + 62)
    m, k = 70, 256
    a = rng.uniform(m * k, 2.0).reshape(m, k)
    ws = [rng.uniform(nn * k).reshape(nn, k) for nn in (64, 32, 32)]
    outs = [np.zeros((m, nn), np.float32) for nn in (64, 32, 32)]
    segs = (lh.GemmSegment * 3)(*[lh.GemmSegment(lh.ptr(o), o.shape[1], lh.ptr(w), None, k, o.shape[1],
                                                 lh.GEMM_STORE) for o, w in zip(outs, ws)])
    L.k_gemm_f32(lh.ptr(a), k, m, k, segs, 3)
    for o, w in zip(outs, ws):
        r, mag = ref_f32(a, w)
        hu.assert_within_budget(o, r, mag, what="qkv segments")


# ---- BF16 GEMM -----------------------------------------------------------------------------------------------------


def bf16_round(x):
    """Finite float32 values rounded to BF16 (nearest, ties to even) and widened back; a sample is checked against the
    oracle's bf16_from_f32 (src/gemm.c:335-342)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)).view(np.float32)
    sample = np.ravel(x)[:257]
    assert np.array_equal(orc.bf16_from_f32(sample), (np.ravel(r)[:257].view(np.uint32) >> 16).astype(np.uint16))
    return r


@pytest.mark.parametrize("m,n,k", [(1, 5, 8), (5, 17, 40), (17, 33, 64), (130, 200, 97), (256, 256, 3072),
                                   (64, 512, 8192)])
def test_bf16_gemm_all_kinds(m, n, k):
    L = hu.lib()
    rng = orc.Rng(orc.SEED + 71 * m + n + k)
    lda, ldc = k + 3, n + 7
    a = rng.uniform(m * lda, 2.0).reshape(m, lda)
    w, w3 = rng.uniform(n * k).reshape(n, k), rng.uniform(n * k).reshape(n, k)
    base = rng.uniform(m * ldc, 4.0).reshape(m, ldc)
    pw, pw3 = np.zeros(L.bf16_vnni_elements(n, k), np.uint16), np.zeros(L.bf16_vnni_elements(n, k), np.uint16)
    L.pack_bf16_vnni(lh.ptr(pw), lh.ptr(w), n, k, k)
    L.pack_bf16_vnni(lh.ptr(pw3), lh.ptr(w3), n, k, k)
    ab, wb, w3b = bf16_round(a[:, :k].copy()), bf16_round(w), bf16_round(w3)
    r, mag = ref_f32(ab, wb)
    r3, mag3 = ref_f32(ab, w3b)
    panel = lh.AlignedBuffer()
    L.aligned_buffer_alloc(panel, L.k_gemm_bf16_panel_bytes(m, k), 1)
    da, dpw, dpw3 = hu.dev(a), hu.dev(pw), hu.dev(pw3)
    try:
        for kind in (lh.GEMM_STORE, lh.GEMM_ADD, lh.GEMM_SWIGLU):
            c = hu.dev(base)
            seg = lh.GemmBf16Segment(lh.ptr(c), ldc, lh.ptr(dpw), lh.ptr(dpw3), n, kind)
            L.k_gemm_bf16(lh.ptr(da), lda, m, k, seg, 1, panel)
            got = hu.host(c)
            assert np.array_equal(hu.bits(got[:, n:]), hu.bits(base[:, n:])), "row padding was written"
            check_kind(got[:, :n], base[:, :n], r, mag, r3, mag3, kind, rel=2e-6, what=f"bf16 {m}x{n}x{k} {kind}")
    finally:
        L.aligned_buffer_free(panel)


@pytest.mark.parametrize("m,k,lda", [(37, 200, 200), (37, 203, 203), (20, 203, 208), (5, 3072, 3072)])
def test_bf16_panel_bits(m, k, lda):
    """The activation panel k_gemm_bf16 writes: row r holds bf16_from_f32 of A's row (the oracle's conversion, taken
    from its VNNI packing so NaN payloads pass unchanged), zeros from k to the padded width; aligned rows take the
    16-byte path, odd strides and the row tail the per-value one. Specials: NaN payloads, infinities, denormals,
    rounding ties and values that round up to infinity."""
    L = hu.lib()
    rng = orc.Rng(orc.SEED + 5 * m + k + lda)
    a = rng.normal(m * lda, 0.0, 3.0).reshape(m, lda)
    specials = np.array([0x7FC00001, 0xFF800001, 0x7F800001, 0x7F800000, 0xFF800000, 0x00000001, 0x807FFFFF,
                         0x3F808000, 0x3F818000, 0xBF808000, 0x7F7FFFFF, 0xFF7FFFFF, 0x00000000, 0x80000000],
                        np.uint32).view(np.float32)
    flat = a.reshape(-1)
    idx = (np.arange(specials.size * 7) * 131) % flat.size
    flat[idx] = np.tile(specials, 7)
    kpad = (k + 31) // 32 * 32
    vnni = orc.pack_bf16_vnni(np.ascontiguousarray(a[:, :k]))
    r, c = np.meshgrid(np.arange(m), np.arange(k), indexing="ij")
    want = vnni[(r // 16) * 16 * kpad + (c // 2) * 32 + (r % 16) * 2 + c % 2]
    n = 16
    w = rng.uniform(n * k).reshape(n, k)
    pw = np.zeros(L.bf16_vnni_elements(n, k), np.uint16)
    L.pack_bf16_vnni(lh.ptr(pw), lh.ptr(w), n, k, k)
    panel = lh.AlignedBuffer()
    L.aligned_buffer_alloc(panel, L.k_gemm_bf16_panel_bytes(m, k), 1)
    da, dpw, out = hu.dev(a), hu.dev(pw), hu.empty((m, n), hu.torch().float32)
    try:
        seg = lh.GemmBf16Segment(lh.ptr(out), n, lh.ptr(dpw), None, n, lh.GEMM_STORE)
        L.k_gemm_bf16(lh.ptr(da), lda, m, k, seg, 1, panel)
        L.llhip_synchronize()
        got = np.zeros((m, kpad), np.uint16)
        L.llhip_memcpy_d2h(got.ctypes.data, panel.data, got.nbytes)
        assert np.array_equal(got[:, :k], want), np.argwhere(got[:, :k] != want)[:5]
        assert not got[:, k:].any()
    finally:
        L.aligned_buffer_free(panel)


def test_bf16_gemm_reference_golden():
    g = np.load(os.path.join(GOLDEN, "bf16.npz"))
    L = hu.lib()
    for key in sorted({k.split("/")[0] for k in g.files if k.endswith("/shape")}):
        m, n, k = (int(v) for v in g[f"{key}/shape"])
        a, w, w3, base, pw = (g[f"{key}/{x}"] for x in ("a", "w", "w3", "base", "pw"))
        pw3 = orc.pack_bf16_vnni(w3)
        r, mag = ref_f32(bf16_round(a[:, :k].copy()), bf16_round(w))
        panel = lh.AlignedBuffer()
        L.aligned_buffer_alloc(panel, L.k_gemm_bf16_panel_bytes(m, k), 1)
        for kname, kind in (("store", 0), ("add", 1), ("swiglu", 2)):
            c = base.copy()
            seg = lh.GemmBf16Segment(lh.ptr(c), c.shape[1], lh.ptr(pw), lh.ptr(pw3), n, kind)
            L.k_gemm_bf16(lh.ptr(a), a.shape[1], m, k, seg, 1, panel)
            want = g[f"{key}/{kname}"]
            assert np.array_equal(hu.bits(c[:, n:]), hu.bits(base[:, n:]))
            if kname == "swiglu":
                np.testing.assert_allclose(c[:, :n], want[:, :n], rtol=1e-4, atol=1e-5)
            else:
                extra = np.abs(base[:, :n]) if kname == "add" else 0
                hu.assert_within_budget(c[:, :n], want[:, :n], mag + extra, rel=4e-6, what=f"{key} {kname}")
        L.aligned_buffer_free(panel)


# ---- pipelined FP32 / BF16 kernels: aligned shapes, split K --------------------------------------------------------


@pytest.mark.parametrize("m,n,k", [(300, 200, 1024), (513, 136, 3072), (40, 130, 16 * 37), (256, 256, 8192),
                                   (600, 600, 512)])
@pytest.mark.parametrize("mode", ["f32", "f32-fp32", "bf16", "bf16-wide"])
def test_pipelined_gemm_split_k(m, n, k, mode, monkeypatch):
    """Rows 16-byte aligned and K a multiple of 16 take the pipelined kernel: for FP32 mm_gemm_f32x3 (products from
    exact BF16 parts, pairs of 16-value K steps; 37 steps leave a pair's second half empty) or, with
    LLAMA_HIP_F32_FORM=fp32, mm_gemm_lds (FP32 products). Every split count (0 = the automatic choice) meets the budget
    for every kind and for three segments sharing A; a repeated call with the same split count gives the same bits
    (the arrival counters are back at zero and partial sums are added in split order)."""
    L = hu.lib()
    L.llhip_set_bf16_tile(2 if mode == "bf16-wide" else 1)
    if mode == "f32-fp32":
        monkeypatch.setenv("LLAMA_HIP_F32_FORM", "fp32")
    mode = mode[:4]
    rng = orc.Rng(orc.SEED + 81 * m + n + k)
    lda, ldc = k + 4, n + 7
    a = rng.uniform(m * lda, 2.0).reshape(m, lda)
    w, w3 = rng.uniform(n * k).reshape(n, k), rng.uniform(n * k).reshape(n, k)
    base = rng.uniform(m * ldc, 4.0).reshape(m, ldc)
    da = hu.dev(a)
    panel = lh.AlignedBuffer()
    if mode == "bf16":
        pw, pw3 = np.zeros(L.bf16_vnni_elements(n, k), np.uint16), np.zeros(L.bf16_vnni_elements(n, k), np.uint16)
        L.pack_bf16_vnni(lh.ptr(pw), lh.ptr(w), n, k, k)
        L.pack_bf16_vnni(lh.ptr(pw3), lh.ptr(w3), n, k, k)
        dw, dw3 = hu.dev(pw), hu.dev(pw3)
        ab, wb, w3b = bf16_round(a[:, :k].copy()), bf16_round(w), bf16_round(w3)
        r, mag = ref_f32(ab, wb)
        r3, mag3 = ref_f32(ab, w3b)
        rel = 2e-6
        L.aligned_buffer_alloc(panel, L.k_gemm_bf16_panel_bytes(m, k), 1)
    else:
        dw, dw3 = hu.dev(w), hu.dev(w3)
        r, mag = ref_f32(a[:, :k], w)
        r3, mag3 = ref_f32(a[:, :k], w3)
        rel = 2e-5

    def gemm(c, kind, splits):
        L.llhip_set_gemm_splits(splits)
        if mode == "bf16":
            seg = lh.GemmBf16Segment(lh.ptr(c), ldc, lh.ptr(dw), lh.ptr(dw3), n, kind)
            L.k_gemm_bf16(lh.ptr(da), lda, m, k, seg, 1, panel)
        else:
            seg = lh.GemmSegment(lh.ptr(c), ldc, lh.ptr(dw), lh.ptr(dw3), k, n, kind)
            L.k_gemm_f32(lh.ptr(da), lda, m, k, seg, 1)

    try:
        for splits in (0, 1, 2, 3, 7):
            for kind in (lh.GEMM_STORE, lh.GEMM_ADD, lh.GEMM_SWIGLU):
                c = hu.dev(base)
                gemm(c, kind, splits)
                got = hu.host(c)
                assert lh.last_error() == "", lh.last_error()
                assert np.array_equal(hu.bits(got[:, n:]), hu.bits(base[:, n:])), "row padding was written"
                check_kind(got[:, :n], base[:, :n], r, mag, r3, mag3, kind, rel=rel,
                           what=f"{mode} {m}x{n}x{k} kind {kind} splits {splits}")
                if kind == lh.GEMM_STORE:
                    again = hu.dev(base)
                    gemm(again, kind, splits)
                    assert np.array_equal(hu.bits(hu.host(again)), hu.bits(got)), f"splits {splits} not repeatable"
        # three segments sharing A (QKV), automatic splits
        L.llhip_set_gemm_splits(0)
        widths = (n, max(16, n // 4), max(16, n // 4))
        outs = [hu.dev(np.zeros((m, nn), np.float32)) for nn in widths]
        wts = [w[:nn] for nn in widths]
        if mode == "bf16":
            packed = []
            for nn, wt in zip(widths, wts):
                pk = np.zeros(L.bf16_vnni_elements(nn, k), np.uint16)
                L.pack_bf16_vnni(lh.ptr(pk), lh.ptr(np.ascontiguousarray(wt)), nn, k, k)
                packed.append(hu.dev(pk))
            segs = (lh.GemmBf16Segment * 3)(*[lh.GemmBf16Segment(lh.ptr(o), nn, lh.ptr(p), None, nn, lh.GEMM_STORE)
                                              for o, p, nn in zip(outs, packed, widths)])
            L.k_gemm_bf16(lh.ptr(da), lda, m, k, segs, 3, panel)
        else:
            dws = [hu.dev(np.ascontiguousarray(wt)) for wt in wts]
            segs = (lh.GemmSegment * 3)(*[lh.GemmSegment(lh.ptr(o), nn, lh.ptr(d), None, k, nn, lh.GEMM_STORE)
                                          for o, d, nn in zip(outs, dws, widths)])
            L.k_gemm_f32(lh.ptr(da), lda, m, k, segs, 3)
        for o, nn in zip(outs, widths):
            hu.assert_within_budget(hu.host(o), r[:, :nn], mag[:, :nn], rel=rel, what=f"{mode} segment of {nn}")
    finally:
        L.llhip_set_gemm_splits(0)
        L.llhip_set_bf16_tile(0)
        L.aligned_buffer_free(panel)
