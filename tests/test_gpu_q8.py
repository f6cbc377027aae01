"""GPU parity of the Q8_0 hot path through the C ABI: quantizer, decode GEMV, batched GEMM, int32 probes.

The oracle (oracle/, pinned to the reference by tests/test_oracle.py) is the checker. The bar: int8 activations, their
scales and the int32 group dots are bitwise the oracle's; FP32 outputs lie within the reference's budget
2e-5 * sum|w x| + 1e-6 of the float64 dequantized reference (tests/q8.c:128-133), which also bounds the difference to
the reference's own scalar results; the floored relative error d / (|ref| + 1e-3) (tests/q8_engine.c:71) is checked
against the stated tolerance 1e-4.
"""
import ctypes
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
    assert L.llhip_init() == 0, hu.lh.last_error()
    print("device:", L.llhip_device_name().decode(), flush=True)
    yield L


def synth_weights(rng, d, n, gs, std=0.02):
    return orc.quantize_weights(rng.normal(d * n, 0.0, std).reshape(d, n), gs)


# ---- quantizer -----------------------------------------------------------------------------------------------------


def test_quantize_golden_bitwise_device_and_host():
    g = np.load(os.path.join(GOLDEN, "quantize.npz"))
    L = hu.lib()
    names = sorted({k.split("/")[0] for k in g.files})
    for name in names:
        x, gs = g[f"{name}/x"], int(g[f"{name}/gs"])
        n = x.shape[0]
        want_q, want_s = g[f"{name}/q"], g[f"{name}/s"]
        # device-resident buffers
        xd, qd, sd = hu.dev(x), hu.empty(n, hu.torch().int8), hu.empty(n // gs, hu.torch().float32)
        L.k_quantize(lh.ptr(qd), lh.ptr(sd), lh.ptr(xd), n, gs)
        assert np.array_equal(hu.host(qd), want_q), name
        assert np.array_equal(hu.bits(hu.host(sd)), hu.bits(want_s)), name
        # host buffers (staged through the device)
        q, s = np.zeros(n, np.int8), np.zeros(n // gs, np.float32)
        L.k_quantize(lh.ptr(q), lh.ptr(s), lh.ptr(x), n, gs)
        assert np.array_equal(q, want_q) and np.array_equal(hu.bits(s), hu.bits(want_s)), name


@pytest.mark.parametrize("m,n,gs,ldx", [(1, 4096, 64, 4096), (7, 14336, 64, 14400), (33, 2048, 128, 2048),
                                        (5, 768, 32, 800), (3, 96, 2, 96), (4, 200, 8, 203), (2, 1024, 1024, 1024)])
def test_quantize_rows_bitwise(m, n, gs, ldx):
    rng = orc.Rng(orc.SEED + 11 * m + n)
    x = rng.normal(m * ldx, 0.0, 1.5).reshape(m, ldx)
    x[0, :gs] = 0.0  # an all-zero group
    want_q, want_s = orc.quantize(np.ascontiguousarray(x[:, :n]), gs)
    L = hu.lib()
    xd = hu.dev(x)
    qd, sd = hu.empty((m, n), hu.torch().int8), hu.empty((m, n // gs), hu.torch().float32)
    L.k_quantize_rows(lh.ptr(qd), lh.ptr(sd), lh.ptr(xd), ldx, m, n, gs)
    assert np.array_equal(hu.host(qd), want_q)
    assert np.array_equal(hu.bits(hu.host(sd)), hu.bits(want_s))


def test_quantize_nonfinite_fails_at_the_next_host_visible_point():
    L = hu.lib()
    lh.record_failures()
    try:
        x = np.ones(256, np.float32)
        x[100] = np.nan
        q, s = np.zeros(256, np.int8), np.zeros(4, np.float32)
        L.k_quantize(lh.ptr(q), lh.ptr(s), lh.ptr(x), 256, 64)  # host buffers: the call itself waits and fails
        assert "nonfinite activation during INT8 quantization" in lh.last_error()
        L.llhip_clear_error()
        x[100] = np.inf
        xd, qd, sd = hu.dev(x), hu.empty(256, hu.torch().int8), hu.empty(4, hu.torch().float32)
        L.k_quantize(lh.ptr(qd), lh.ptr(sd), lh.ptr(xd), 256, 64)  # device buffers: reported by the next wait
        L.llhip_synchronize()
        assert "nonfinite activation during INT8 quantization" in lh.last_error()
        L.llhip_clear_error()
        L.llhip_synchronize()  # the flag was consumed
        assert lh.last_error() == ""
    finally:
        L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
        L.llhip_clear_error()


# ---- decode GEMV ---------------------------------------------------------------------------------------------------


def c1_inputs():
    rng = orc.Rng()
    wq, ws = synth_weights(rng, 2048, 2048, 64)
    x = rng.normal(2048, 0.0, 1.0)
    xq, xs = orc.quantize(x, 64)
    return wq, ws, x, xq, xs


def test_c1_gemv_parity_and_probe():
    """C1: the 1B wq GEMV (2048 x 2048, gs 64): outputs within budget of the float64 reference and of the reference's
    own scalar output (golden), int32 group dots bitwise."""
    L = hu.lib()
    wq, ws, x, xq, xs = c1_inputs()
    golden = np.load(os.path.join(GOLDEN, "gemv_q8.npz"))["c1/y"]
    want = orc.matmul_q8(xq, xs, wq, ws, 64)
    assert np.array_equal(hu.bits(want), hu.bits(golden))  # the oracle is the reference here, bit for bit
    ref, mag = hu.dequant_reference(xq, xs, wq, ws, 64)
    wqd, wsd, xqd, xsd = hu.dev(wq), hu.dev(ws), hu.dev(xq), hu.dev(xs)
    out = hu.empty(2048, hu.torch().float32)
    L.k_matmul_q8(lh.ptr(out), lh.k8(xqd, xsd, None), lh.w8(wqd, wsd), 2048, 2048, 64)
    got = hu.host(out)
    hu.assert_within_budget(got, ref, mag, what="C1 vs float64")
    hu.assert_within_budget(got, golden, mag, rel=4e-5, what="C1 vs reference scalar")
    assert hu.max_rel_error(got, ref) < 1e-4
    dots = np.zeros((32, 2048), np.int32)
    L.llhip_q8_gemv_group_dots(lh.ptr(dots), lh.ptr(xqd), lh.ptr(xsd), lh.ptr(wqd), lh.ptr(wsd), 0, 2048, 2048, 64)
    want_dots = orc.group_dots(xq.reshape(1, -1), wq, 64)[:, 0, :]
    assert np.array_equal(dots, want_dots)


@pytest.mark.parametrize("d,n,gs", [(4096, 4096, 64), (1024, 14336, 64), (333, 4096, 128), (77, 2048, 32),
                                    (64, 1088, 64), (5, 256, 16), (9, 64, 4), (3, 12, 2), (17, 320, 64)])
def test_gemv_shapes_budget_and_probe(d, n, gs):
    L = hu.lib()
    rng = orc.Rng(orc.SEED + d * 7 + n)
    wq, ws = synth_weights(rng, d, n, gs)
    x = rng.normal(n, 0.0, 1.0)
    xq, xs = orc.quantize(x, gs)
    ref, mag = hu.dequant_reference(xq, xs, wq, ws, gs)
    out = hu.empty(d, hu.torch().float32)
    dxq, dxs, dwq, dws = hu.dev(xq), hu.dev(xs), hu.dev(wq), hu.dev(ws)  # held: the call only sees their addresses
    L.k_matmul_q8(lh.ptr(out), lh.k8(dxq, dxs), lh.w8(dwq, dws), n, d, gs)
    hu.assert_within_budget(hu.host(out), ref, mag, what=f"gemv {d}x{n} gs {gs}")
    dots = np.zeros((n // gs, d), np.int32)
    L.llhip_q8_gemv_group_dots(lh.ptr(dots), lh.ptr(xq), lh.ptr(xs), lh.ptr(wq), lh.ptr(ws), 0, n, d, gs)
    assert np.array_equal(dots, orc.group_dots(xq.reshape(1, -1), wq, gs)[:, 0, :])


def f32_input_reference(x, wq, ws, gs):
    """float64 sum and magnitude of W.x for the W8A32 GEMV: dequantized weights, the FP32 input as it is."""
    wd = wq.astype(np.float64) * np.repeat(ws.astype(np.float64), gs, axis=-1)
    xd = x.astype(np.float64)
    return wd @ xd, np.abs(wd) @ np.abs(xd)


@pytest.mark.parametrize("d,n,gs", [(4096, 4096, 64), (1024, 14336, 64), (512, 16384, 64), (333, 4096, 128),
                                    (77, 2048, 32), (64, 1088, 64), (5, 256, 16), (17, 320, 64), (40, 8192, 256)])
def test_w8a32_gemv_shapes_budget(d, n, gs):
    """W8A32 (FP32 activations, src/gemv.c:141-181) through every epilogue: store and add within the budget of the
    float64 reference, SwiGLU and the three-matrix QKV form against the oracle (the reference's scalar loop)."""
    L = hu.lib()
    rng = orc.Rng(orc.SEED + 3 * d + n + gs)
    wq, ws = synth_weights(rng, d, n, gs)
    w3q, w3s = synth_weights(rng, d, n, gs)
    x = rng.normal(n, 0.0, 1.0)
    base = rng.normal(d, 0.0, 1.0)
    ref, mag = f32_input_reference(x, wq, ws, gs)
    dx, dwq, dws, dw3q, dw3s = hu.dev(x), hu.dev(wq), hu.dev(ws), hu.dev(w3q), hu.dev(w3s)
    inp = lh.k8(None, None, dx)
    out = hu.empty(d, hu.torch().float32)
    L.k_matmul_q8(lh.ptr(out), inp, lh.w8(dwq, dws), n, d, gs)
    hu.assert_within_budget(hu.host(out), ref, mag, what=f"w8a32 store {d}x{n} gs {gs}")
    acc = hu.dev(base)
    L.k_matmul_q8_add(lh.ptr(acc), inp, lh.w8(dwq, dws), n, d, gs)
    hu.assert_within_budget(hu.host(acc), ref + base, mag + np.abs(base), what=f"w8a32 add {d}x{n}")
    sw = hu.empty(d, hu.torch().float32)
    L.k_matmul_q8_swiglu(lh.ptr(sw), inp, lh.w8(dwq, dws), lh.w8(dw3q, dw3s), n, d, gs)
    got = hu.host(sw).astype(np.float64)
    ref3, mag3 = f32_input_reference(x, w3q, w3s, gs)
    # silu(a) * b with both dots inside their budgets t: the error carries through |silu'| <= 1.1
    ta, tb = 2e-5 * mag + 1e-6, 2e-5 * mag3 + 1e-6
    silu = ref / (1.0 + np.exp(-ref))
    tol = 1.1 * np.abs(ref3) * ta + np.abs(silu) * tb + 1.1 * ta * tb + 1e-6
    assert np.all(np.abs(got - silu * ref3) <= tol), f"w8a32 swiglu {d}x{n}"
    want = orc.matmul_q8(None, None, wq, ws, gs, orc.K_SWIGLU, w3q=w3q, w3s=w3s, xf=x)
    assert np.all(np.abs(got - want) <= 2 * tol), f"w8a32 swiglu {d}x{n} vs oracle"
    qkv = [hu.empty(d, hu.torch().float32) for _ in range(3)]
    L.k_matmul_q8_qkv(lh.ptr(qkv[0]), lh.ptr(qkv[1]), lh.ptr(qkv[2]), inp, lh.w8(dwq, dws), lh.w8(dw3q, dw3s),
                      lh.w8(dwq, dws), n, d, d, gs)
    for j, (r, m) in enumerate([(ref, mag), (ref3, mag3), (ref, mag)]):
        hu.assert_within_budget(hu.host(qkv[j]), r, m, what=f"w8a32 qkv[{j}] {d}x{n}")


def test_gemv_entry_points_against_reference_golden():
    """Every GEMV entry point, W8A8 and W8A32, on the reference's own golden small cases (host buffers)."""
    g = np.load(os.path.join(GOLDEN, "gemv_q8.npz"))
    L = hu.lib()
    keys = sorted({k.split("/")[0] for k in g.files if k.endswith("/gs")})
    for key in keys:
        gs, x, base = int(g[f"{key}/gs"]), g[f"{key}/x"], g[f"{key}/base"]
        n, d = x.shape[0], base.shape[0]
        w = [(g[f"{key}/wq{j}"], g[f"{key}/ws{j}"]) for j in range(3)]
        xq, xs = orc.quantize(x, gs)
        for mode in ("w8a8", "w8a32"):
            inp = lh.k8(xq, xs, x) if mode == "w8a8" else lh.k8(None, None, x)
            aq, as_ = (xq, xs) if mode == "w8a8" else (None, None)
            ref = [hu.dequant_reference(xq, xs, q, s, gs) for q, s in w] if mode == "w8a8" else None
            for kname in ("store", "add", "swiglu", "qkv"):
                want = g[f"{key}/{mode}/{kname}"]
                if kname == "qkv":
                    y = [base.copy(), np.zeros(d, np.float32), np.zeros(d, np.float32)]
                    L.k_matmul_q8_qkv(lh.ptr(y[0]), lh.ptr(y[1]), lh.ptr(y[2]), inp, lh.w8(*w[0]), lh.w8(*w[1]),
                                      lh.w8(*w[2]), n, d, d, gs)
                    got = np.concatenate(y)
                else:
                    got = base.copy()
                    if kname == "store":
                        L.k_matmul_q8(lh.ptr(got), inp, lh.w8(*w[0]), n, d, gs)
                    elif kname == "add":
                        L.k_matmul_q8_add(lh.ptr(got), inp, lh.w8(*w[0]), n, d, gs)
                    else:
                        L.k_matmul_q8_swiglu(lh.ptr(got), inp, lh.w8(*w[0]), lh.w8(*w[1]), n, d, gs)
                oracle = _oracle_gemv(kname, aq, as_, x, w, gs, base)
                np.testing.assert_allclose(oracle, want, rtol=0, atol=0)  # the oracle is bitwise the reference
                if ref is not None and kname in ("store", "add"):
                    r, mag = ref[0]
                    r = r + (base if kname == "add" else 0)
                    hu.assert_within_budget(got, r, mag + (np.abs(base) if kname == "add" else 0),
                                            what=f"{key} {mode} {kname}")
                else:
                    scale = np.maximum(np.abs(want), 1.0)
                    assert np.all(np.abs(got - want) <= 1e-4 * scale), (key, mode, kname, got, want)


def _oracle_gemv(kname, aq, as_, x, w, gs, base):
    if kname == "qkv":
        return np.concatenate([orc.matmul_q8(aq, as_, w[0][0], w[0][1], gs, xf=x, out=base.copy()),
                               orc.matmul_q8(aq, as_, w[1][0], w[1][1], gs, xf=x),
                               orc.matmul_q8(aq, as_, w[2][0], w[2][1], gs, xf=x)])
    kind = {"store": orc.K_STORE, "add": orc.K_ADD, "swiglu": orc.K_SWIGLU}[kname]
    return orc.matmul_q8(aq, as_, w[0][0], w[0][1], gs, kind, out=base.copy(), w3q=w[1][0], w3s=w[1][1], xf=x)


def test_gemv_ld_and_worker_forms():
    L = hu.lib()
    rng = orc.Rng(orc.SEED + 404)
    d, n, ld, gs = 50, 512, 640, 64
    wq, ws = synth_weights(rng, d, ld, gs)
    xq, xs = orc.quantize(rng.normal(n, 0.0, 1.0), gs)
    ref, mag = hu.dequant_reference(xq, xs, wq[:, :n], ws[:, : n // gs], gs)
    base = rng.uniform(d, 2.0)
    for kind in (lh.K_STORE, lh.K_PARTIAL, lh.K_ADD):
        out = base.copy()
        wv = lh.w8(wq, ws)
        L.k_matmul_q8_ld(lh.ptr(out), lh.k8(xq, xs), wv, ld, n, d, gs, kind)
        want = ref + (base if kind == lh.K_ADD else 0)
        hu.assert_within_budget(out, want, mag + np.abs(base), what=f"_ld kind {kind}")
    # the worker form: the union of the members' static shares is the whole result; done() sees each share
    seen = []
    cb = lh.RowsDoneFn(lambda ctx, r0, r1: seen.append((r0, r1)))
    out = np.zeros(d, np.float32)
    for worker in range(3):
        L.k_matmul_q8_ld_worker(lh.ptr(out), lh.k8(xq, xs), lh.w8(wq, ws), ld, n, d, gs, lh.K_STORE, worker, 3, None,
                                cb, None)
    hu.assert_within_budget(out, ref, mag, what="_ld_worker union")
    assert seen == [(0, 16), (16, 33), (33, 50)]
    # the SwiGLU shard form
    w3q, w3s = synth_weights(rng, d, ld, gs)
    r3, _ = hu.dequant_reference(xq, xs, w3q[:, :n], w3s[:, : n // gs], gs)
    out = np.zeros(d, np.float32)
    L.k_matmul_q8_swiglu_ld(lh.ptr(out), lh.k8(xq, xs), lh.w8(wq, ws), lh.w8(w3q, w3s), ld, n, d, gs)
    want = ref / (1 + np.exp(-ref)) * r3
    np.testing.assert_allclose(out, want, rtol=1e-4, atol=1e-5)


def test_gemv_qkv_device_resident_and_graph_replay():
    """The three-segment QKV launch on device buffers, captured into a graph and replayed with eager work between
    the replays; every replay equals the eager result bitwise."""
    L = hu.lib()
    T = hu.torch()
    rng = orc.Rng(orc.SEED + 505)
    n, dq, dkv, gs = 2048, 2048, 512, 64
    ws_ = [synth_weights(rng, d, n, gs) for d in (dq, dkv, dkv)]
    x = rng.normal(n, 0.0, 1.0)
    xd = hu.dev(x)
    xqd, xsd = hu.empty(n, T.int8), hu.empty(n // gs, T.float32)
    wdev = [(hu.dev(q), hu.dev(s)) for q, s in ws_]
    outs = [hu.empty(d, T.float32) for d in (dq, dkv, dkv)]

    def step():
        L.k_quantize(lh.ptr(xqd), lh.ptr(xsd), lh.ptr(xd), n, gs)
        L.k_matmul_q8_qkv(lh.ptr(outs[0]), outs[1].data_ptr(), outs[2].data_ptr(), lh.k8(xqd, xsd, xd),
                          lh.w8(*wdev[0]), lh.w8(*wdev[1]), lh.w8(*wdev[2]), n, dq, dkv, gs)

    step()
    eager = [hu.host(o) for o in outs]
    xq, xs = orc.quantize(x, gs)
    for (q, s), got in zip(ws_, eager):
        ref, mag = hu.dequant_reference(xq, xs, q, s, gs)
        hu.assert_within_budget(got, ref, mag, what="qkv")
    assert L.llhip_graph_begin() == 0
    step()
    graph = L.llhip_graph_end()
    assert graph, lh.last_error()
    try:
        for replay in range(4):
            for o in outs:
                o.fill_(-1.0)
            T.cuda.synchronize()
            assert L.llhip_graph_launch(graph) == 0
            got = [hu.host(o) for o in outs]
            for a, b in zip(got, eager):
                assert np.array_equal(hu.bits(a), hu.bits(b)), replay
    finally:
        L.llhip_graph_destroy(graph)


def test_registered_host_weights_resolve_to_hbm():
    L = hu.lib()
    rng = orc.Rng(orc.SEED + 606)
    d, n, gs = 300, 1024, 64
    wq, ws = synth_weights(rng, d, n, gs)
    xq, xs = orc.quantize(rng.normal(n, 0.0, 1.0), gs)
    assert L.llhip_register_host(lh.ptr(wq), wq.nbytes) == 0
    assert L.llhip_register_host(lh.ptr(ws), ws.nbytes) == 0
    try:
        assert L.llhip_resolve(lh.ptr(wq) + 64) is not None
        out = np.zeros(d, np.float32)
        L.k_matmul_q8(lh.ptr(out), lh.k8(xq, xs), lh.w8(wq, ws), n, d, gs)
        ref, mag = hu.dequant_reference(xq, xs, wq, ws, gs)
        hu.assert_within_budget(out, ref, mag, what="registered weights")
    finally:
        L.llhip_unregister_host(lh.ptr(wq))
        L.llhip_unregister_host(lh.ptr(ws))


# ---- batched GEMM ---------------------------------------------------------------------------------------------------


def gemm_case(m, n, k, gs, seed):
    rng = orc.Rng(orc.SEED + seed)
    x = rng.normal(m * k, 0.0, 1.0).reshape(m, k)
    xq, xs = orc.quantize(x, gs)
    (wq, ws), (w3q, w3s) = synth_weights(rng, n, k, gs), synth_weights(rng, n, k, gs)
    return xq, xs, wq, ws, w3q, w3s, rng


@pytest.mark.parametrize("m,n,k,gs", [(1, 64, 64, 64), (33, 20, 128, 64), (40, 33, 192, 64), (130, 257, 1024, 64),
                                      (256, 384, 4096, 64), (77, 200, 2048, 128), (64, 96, 512, 32), (5, 7, 16, 4),
                                      (129, 129, 640, 64), (600, 200, 1024, 64), (300, 136, 14336, 64),
                                      (50, 70, 1024, 256), (513, 65, 320, 64)])
def test_gemm_q8_all_kinds_within_budget(m, n, k, gs):
    L = hu.lib()
    T = hu.torch()
    xq, xs, wq, ws, w3q, w3s, rng = gemm_case(m, n, k, gs, m * 31 + n)
    ldc = n + 5
    base = rng.uniform(m * ldc, 3.0).reshape(m, ldc)
    ref, mag = hu.dequant_reference(xq, xs, wq, ws, gs)
    r3, mag3 = hu.dequant_reference(xq, xs, w3q, w3s, gs)
    dx = [hu.dev(a) for a in (xq, xs, wq, ws, w3q, w3s)]
    for kind in (lh.GEMM_STORE, lh.GEMM_ADD, lh.GEMM_SWIGLU, lh.GEMM_PARTIAL):
        c = hu.dev(base)
        seg = lh.GemmQ8Segment(lh.ptr(c), ldc, lh.w8(dx[2], dx[3]), lh.w8(dx[4], dx[5]), None, None, n, kind)
        L.k_gemm_q8(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, gs, seg, 1)
        got = hu.host(c)
        assert np.array_equal(hu.bits(got[:, n:]), hu.bits(base[:, n:])), "row padding was written"
        got = got[:, :n]
        if kind == lh.GEMM_ADD:
            hu.assert_within_budget(got, base[:, :n] + ref, mag + np.abs(base[:, :n]), what=f"add {m}x{n}x{k}")
        elif kind == lh.GEMM_SWIGLU:
            want = ref / (1 + np.exp(-ref)) * r3
            tol = 2e-5 * (mag * (np.abs(r3) + 1) + mag3 * (np.abs(ref) + 1)) + 1e-6  # tests/q8.c:130
            assert np.all(np.abs(got - want) <= tol), f"swiglu {m}x{n}x{k}"
        else:
            hu.assert_within_budget(got, ref, mag, what=f"store {m}x{n}x{k}")
    del T


@pytest.mark.parametrize("m", [1, 2, 3, 4, 7, 16, 17, 32])
@pytest.mark.parametrize("n,k,gs", [(300, 4096, 64), (136, 14336, 256), (70, 2048, 128), (100, 2368, 64),
                                    (48, 2496, 192)])
def test_gemm_q8_short_batches(m, n, k, gs):
    """At most 32 rows take the skinny kernel (weights streamed once, K split over a block's waves): every kind and a
    three-segment QKV call within the budget, and each output equal to the tiled kernel's within the budget (a forced
    split count selects the tiled kernel). k = 2368 and 2496 give an odd number of K steps per wave, so a pair of
    steps loaded together reaches into the next wave's range or past the row's end."""
    L = hu.lib()
    xq, xs, wq, ws, w3q, w3s, rng = gemm_case(m, n, k, gs, 1212 + m + n)
    ldc = n + 3
    base = rng.uniform(m * ldc, 3.0).reshape(m, ldc)
    ref, mag = hu.dequant_reference(xq, xs, wq, ws, gs)
    r3, mag3 = hu.dequant_reference(xq, xs, w3q, w3s, gs)
    dx = [hu.dev(a) for a in (xq, xs, wq, ws, w3q, w3s)]

    def run(kind, splits):
        L.llhip_set_gemm_splits(splits)
        c = hu.dev(base)
        seg = lh.GemmQ8Segment(lh.ptr(c), ldc, lh.w8(dx[2], dx[3]), lh.w8(dx[4], dx[5]), None, None, n, kind)
        L.k_gemm_q8(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, gs, seg, 1)
        got = hu.host(c)
        assert lh.last_error() == "", lh.last_error()
        assert np.array_equal(hu.bits(got[:, n:]), hu.bits(base[:, n:])), "row padding was written"
        return got[:, :n]

    try:
        for kind in (lh.GEMM_STORE, lh.GEMM_ADD, lh.GEMM_SWIGLU):
            got, tiled = run(kind, 0), run(kind, 1)
            what = f"skinny m {m} {n}x{k} gs {gs} kind {kind}"
            if kind == lh.GEMM_ADD:
                hu.assert_within_budget(got, base[:, :n] + ref, mag + np.abs(base[:, :n]), what=what)
                hu.assert_within_budget(got, tiled, 2 * (mag + np.abs(base[:, :n])), what=what + " vs tiled")
            elif kind == lh.GEMM_SWIGLU:
                want = ref / (1 + np.exp(-ref)) * r3
                tol = 2e-5 * (mag * (np.abs(r3) + 1) + mag3 * (np.abs(ref) + 1)) + 1e-6
                assert np.all(np.abs(got - want) <= tol), what
                assert np.all(np.abs(got - tiled) <= 2 * tol), what + " vs tiled"
            else:
                hu.assert_within_budget(got, ref, mag, what=what)
                hu.assert_within_budget(got, tiled, 2 * mag, what=what + " vs tiled")
        # three segments sharing the activations
        L.llhip_set_gemm_splits(0)
        widths = (n, max(16, n // 4), max(16, n // 4))
        outs = [hu.dev(np.zeros((m, nn), np.float32)) for nn in widths]
        mats = [(hu.dev(wq[:nn]), hu.dev(ws[:nn])) for nn in widths]  # kept alive across the call
        segs = (lh.GemmQ8Segment * 3)(*[lh.GemmQ8Segment(lh.ptr(o), nn, lh.w8(*w), lh.K8Weight(), None, None, nn,
                                                         lh.GEMM_STORE) for o, w, nn in zip(outs, mats, widths)])
        L.k_gemm_q8(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, gs, segs, 3)
        for o, nn in zip(outs, widths):
            hu.assert_within_budget(hu.host(o), ref[:, :nn], mag[:, :nn], what=f"skinny segment of {nn}")
    finally:
        L.llhip_set_gemm_splits(0)


@pytest.mark.parametrize("m", [17, 32])
@pytest.mark.parametrize("n", [6152, 6168])
def test_gemm_q8_short_batches_two_weight_tiles(m, n):
    """17-32 rows on a grid of at least 384 sixteen-row tiles take blocks of two weight tiles sharing each activation
    load: every kind within the budget, bitwise equal to the same product split into segments narrow enough for blocks
    of one tile (the same per-output sums in the same order). n = 6152 leaves the last block's second tile empty and
    its first half full; 6168 leaves the second tile half full."""
    L = hu.lib()
    k, gs = 4096, 64
    xq, xs, wq, ws, w3q, w3s, rng = gemm_case(m, n, k, gs, 3100 + m + n)
    ref, mag = hu.dequant_reference(xq, xs, wq, ws, gs)
    r3, mag3 = hu.dequant_reference(xq, xs, w3q, w3s, gs)
    dx = [hu.dev(a) for a in (xq, xs, wq, ws, w3q, w3s)]
    base = rng.uniform(m * n, 3.0).reshape(m, n)
    for kind in (lh.GEMM_STORE, lh.GEMM_ADD, lh.GEMM_SWIGLU):
        c = hu.dev(base)
        seg = lh.GemmQ8Segment(lh.ptr(c), n, lh.w8(dx[2], dx[3]), lh.w8(dx[4], dx[5]), None, None, n, kind)
        L.k_gemm_q8(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, gs, seg, 1)
        got = hu.host(c)
        assert lh.last_error() == "", lh.last_error()
        what = f"two-tile skinny m {m} n {n} kind {kind}"
        if kind == lh.GEMM_ADD:
            hu.assert_within_budget(got, base + ref, mag + np.abs(base), what=what)
        elif kind == lh.GEMM_SWIGLU:
            want = ref / (1 + np.exp(-ref)) * r3
            tol = 2e-5 * (mag * (np.abs(r3) + 1) + mag3 * (np.abs(ref) + 1)) + 1e-6
            assert np.all(np.abs(got - want) <= tol), what
        else:
            hu.assert_within_budget(got, ref, mag, what=what)
        # the same product as 24 segments of at most 16 * 15 rows (each call's grid stays under 384 tiles)
        one = hu.dev(base)
        bounds = list(range(0, n, 16 * 15)) + [n]
        parts = []
        for lo, hi in zip(bounds[:-1], bounds[1:]):
            parts.append((lo, hi, hu.dev(wq[lo:hi]), hu.dev(ws[lo:hi]), hu.dev(w3q[lo:hi]), hu.dev(w3s[lo:hi])))
        for lo, hi, a, b, a3, b3 in parts:
            sub = one[:, lo:hi]
            seg = lh.GemmQ8Segment(lh.ptr(sub), n, lh.w8(a, b), lh.w8(a3, b3), None, None, hi - lo, kind)
            L.k_gemm_q8(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, gs, seg, 1)
        assert np.array_equal(hu.bits(hu.host(one)), hu.bits(got)), what + " vs one-tile blocks"


@pytest.mark.parametrize("m,n,k,gs", [(5, 300, 4096, 64), (40, 136, 14336, 256), (257, 70, 2048, 128)])
def test_gemm_q8_split_k(m, n, k, gs):
    """Grids of few tiles split K over several blocks per tile (partials added in split order by a second kernel).
    Every forced split count meets the budget for every kind, repeats bit for bit, and leaves the int32 group dots of
    the probe exact; 0 is the automatic choice."""
    L = hu.lib()
    xq, xs, wq, ws, w3q, w3s, rng = gemm_case(m, n, k, gs, 909 + m)
    ldc = n + 3
    base = rng.uniform(m * ldc, 3.0).reshape(m, ldc)
    ref, mag = hu.dequant_reference(xq, xs, wq, ws, gs)
    r3, mag3 = hu.dequant_reference(xq, xs, w3q, w3s, gs)
    dx = [hu.dev(a) for a in (xq, xs, wq, ws, w3q, w3s)]
    want_dots = orc.group_dots(xq, wq, gs)
    try:
        for splits in (0, 1, 2, 3, 7):
            L.llhip_set_gemm_splits(splits)
            for kind in (lh.GEMM_STORE, lh.GEMM_ADD, lh.GEMM_SWIGLU):
                c = hu.dev(base)
                seg = lh.GemmQ8Segment(lh.ptr(c), ldc, lh.w8(dx[2], dx[3]), lh.w8(dx[4], dx[5]), None, None, n, kind)
                L.k_gemm_q8(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, gs, seg, 1)
                got = hu.host(c)
                assert lh.last_error() == "", lh.last_error()
                assert np.array_equal(hu.bits(got[:, n:]), hu.bits(base[:, n:])), "row padding was written"
                what = f"{m}x{n}x{k} gs {gs} kind {kind} splits {splits}"
                if kind == lh.GEMM_ADD:
                    hu.assert_within_budget(got[:, :n], base[:, :n] + ref, mag + np.abs(base[:, :n]), what=what)
                elif kind == lh.GEMM_SWIGLU:
                    want = ref / (1 + np.exp(-ref)) * r3
                    tol = 2e-5 * (mag * (np.abs(r3) + 1) + mag3 * (np.abs(ref) + 1)) + 1e-6
                    assert np.all(np.abs(got[:, :n] - want) <= tol), what
                else:
                    hu.assert_within_budget(got[:, :n], ref, mag, what=what)
                    again = hu.dev(base)
                    seg = lh.GemmQ8Segment(lh.ptr(again), ldc, lh.w8(dx[2], dx[3]), lh.K8Weight(), None, None, n,
                                           kind)
                    L.k_gemm_q8(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, gs, seg, 1)
                    assert np.array_equal(hu.bits(hu.host(again)), hu.bits(got)), what + " not repeatable"
            dots = np.zeros((k // gs, m, n), np.int32)
            L.llhip_q8_group_dots(lh.ptr(dots), lh.ptr(xq), m, k, gs, lh.ptr(wq), n)
            assert lh.last_error() == ""
            assert np.array_equal(dots, want_dots), f"probe splits {splits}"
    finally:
        L.llhip_set_gemm_splits(0)


@pytest.mark.parametrize("m,n,k", [(33, 20, 128), (40, 33, 192), (130, 257, 1024), (256, 384, 4096), (129, 129, 640),
                                   (600, 200, 1024), (300, 136, 14336), (513, 65, 320), (257, 513, 2048),
                                   (1, 64, 64)])
@pytest.mark.parametrize("scales", [1, 2])
def test_gemm_q8_wide_tiles(m, n, k, scales):
    """The 256 x 256 int8 kernels (gs = 64), forced: every kind within the budget at every forced split count, and a
    three-segment call.
    scales = 1 (q8_gemm_wide, the scale products on the vector unit): bit for bit the 256 x 128 kernel's result (both
    add each group's ((float)dot * ws) * xs in group order, and split partials in split order), so the two tilings
    differ in nothing but speed.
    scales = 2 (q8_gemm_wide_smma, xs * ws from a bf16 MFMA over exact three-part splits of the scales): within
    1e-6 * sum|w x| of the scales = 1 result, the same exact group dots rescaled with the product rounded once instead
    of twice (a dropped or mispaired part would be off by 2^-16 to 2^-8 of a term)."""
    L = hu.lib()
    gs = 64
    xq, xs, wq, ws, w3q, w3s, rng = gemm_case(m, n, k, gs, 4242 + m + n)
    ldc = n + 3
    base = rng.uniform(m * ldc, 3.0).reshape(m, ldc)
    ref, mag = hu.dequant_reference(xq, xs, wq, ws, gs)
    r3, mag3 = hu.dequant_reference(xq, xs, w3q, w3s, gs)
    dx = [hu.dev(a) for a in (xq, xs, wq, ws, w3q, w3s)]

    def run(kind, tile, splits, where=scales):
        L.llhip_set_q8_tile(tile)
        L.llhip_set_gemm_splits(splits)
        L.llhip_set_q8_scales(where)
        c = hu.dev(base)
        seg = lh.GemmQ8Segment(lh.ptr(c), ldc, lh.w8(dx[2], dx[3]), lh.w8(dx[4], dx[5]), None, None, n, kind)
        L.k_gemm_q8(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, gs, seg, 1)
        got = hu.host(c)
        assert lh.last_error() == "", lh.last_error()
        assert np.array_equal(hu.bits(got[:, n:]), hu.bits(base[:, n:])), "row padding was written"
        return got[:, :n]

    try:
        for splits in (1, 2, 3, 0):
            for kind in (lh.GEMM_STORE, lh.GEMM_ADD, lh.GEMM_SWIGLU, lh.GEMM_PARTIAL):
                what = f"wide {m}x{n}x{k} kind {kind} splits {splits}"
                got = run(kind, 2, splits)
                if kind == lh.GEMM_ADD:
                    hu.assert_within_budget(got, base[:, :n] + ref, mag + np.abs(base[:, :n]), what=what)
                elif kind == lh.GEMM_SWIGLU:
                    want = ref / (1 + np.exp(-ref)) * r3
                    tol = 2e-5 * (mag * (np.abs(r3) + 1) + mag3 * (np.abs(ref) + 1)) + 1e-6  # tests/q8.c:130
                    assert np.all(np.abs(got - want) <= tol), what
                else:
                    hu.assert_within_budget(got, ref, mag, what=what)
                if splits and scales == 1:  # the automatic count differs between the tilings (a wide grid has half
                    # the tiles)
                    assert np.array_equal(hu.bits(got), hu.bits(run(kind, 1, splits))), what + " vs 256 x 128"
                if scales == 2:
                    other = run(kind, 2, splits, 1)
                    if kind == lh.GEMM_SWIGLU:  # |d silu(a) b| <= 1.1 |b| |da| + |silu(a)| |db|
                        bound = 1e-6 * (mag * (np.abs(r3) + 1) + mag3 * (np.abs(ref) + 1)) + 1e-9
                    else:
                        bound = 1e-6 * mag + 1e-9
                    assert np.all(np.abs(got - other) <= bound), what + " vs the vector-unit scale products"
        L.llhip_set_q8_tile(2)
        L.llhip_set_gemm_splits(1)
        L.llhip_set_q8_scales(scales)
        widths = (n, max(16, n // 4), max(16, n // 4))
        outs = [hu.dev(np.zeros((m, nn), np.float32)) for nn in widths]
        mats = [(hu.dev(wq[:nn]), hu.dev(ws[:nn])) for nn in widths]  # kept alive across the call
        segs = (lh.GemmQ8Segment * 3)(*[lh.GemmQ8Segment(lh.ptr(o), nn, lh.w8(*w), lh.K8Weight(), None, None, nn,
                                                         lh.GEMM_STORE) for o, w, nn in zip(outs, mats, widths)])
        L.k_gemm_q8(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, gs, segs, 3)
        for o, nn in zip(outs, widths):
            hu.assert_within_budget(hu.host(o), ref[:, :nn], mag[:, :nn], what=f"wide segment of {nn}")
    finally:
        L.llhip_set_q8_tile(0)
        L.llhip_set_gemm_splits(0)
        L.llhip_set_q8_scales(0)


@pytest.mark.parametrize("m,n,k,kind", [(512, 20480, 128, lh.GEMM_SWIGLU), (512, 40960, 128, lh.GEMM_STORE),
                                        (300, 40960, 192, lh.GEMM_ADD), (512, 20416, 128, lh.GEMM_SWIGLU)])
def test_gemm_q8_wide_grid_tail_on_narrow_tiles(m, n, k, kind):
    """A wide grid whose last round would hold at most half the CUs, in whole column tiles across every row tile (here
    2 x 160 = 320 wide tiles on 256 CUs): its last columns go to the 256 x 128 kernel. Every kind within the budget,
    those columns bit for bit the 256 x 128 kernel's over the whole matrix, and the rest within twice the budget of it.
    n = 20416 leaves the last wide tile partly past n (a narrower tail)."""
    L = hu.lib()
    gs = 64
    xq, xs, wq, ws, w3q, w3s, rng = gemm_case(m, n, k, gs, 5150 + m + n)
    ref, mag = hu.dequant_reference(xq, xs, wq, ws, gs)
    r3, mag3 = hu.dequant_reference(xq, xs, w3q, w3s, gs)
    base = rng.uniform(m * n, 3.0).reshape(m, n)
    dx = [hu.dev(a) for a in (xq, xs, wq, ws, w3q, w3s)]

    def run(tile):
        L.llhip_set_q8_tile(tile)
        c = hu.dev(base)
        seg = lh.GemmQ8Segment(lh.ptr(c), n, lh.w8(dx[2], dx[3]), lh.w8(dx[4], dx[5]), None, None, n, kind)
        L.k_gemm_q8(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, gs, seg, 1)
        got = hu.host(c)
        assert lh.last_error() == "", lh.last_error()
        return got

    try:
        got, narrow = run(2), run(1)
        what = f"wide grid with a narrow tail {m}x{n}x{k} kind {kind}"
        width, cus = (128 if kind == lh.GEMM_SWIGLU else 256), L.llhip_device_cu_count()
        tiles = -(-n // width)  # per row tile; two row tiles
        assert 2 * tiles > cus and (2 * tiles) % cus % 2 == 0 and 2 * ((2 * tiles) % cus) <= cus, "not a tail case"
        n1 = (tiles - (2 * tiles) % cus // 2) * width  # wide columns: the whole rounds' tiles
        assert 0 < n1 < n
        assert np.array_equal(hu.bits(got[:, n1:]), hu.bits(narrow[:, n1:])), what + ": tail columns"
        if kind == lh.GEMM_ADD:
            hu.assert_within_budget(got, base + ref, mag + np.abs(base), what=what)
            hu.assert_within_budget(got, narrow, 2 * (mag + np.abs(base)), what=what + " vs 256 x 128")
        elif kind == lh.GEMM_SWIGLU:
            want = ref / (1 + np.exp(-ref)) * r3
            tol = 2e-5 * (mag * (np.abs(r3) + 1) + mag3 * (np.abs(ref) + 1)) + 1e-6
            assert np.all(np.abs(got - want) <= tol), what
            assert np.all(np.abs(got - narrow) <= 2 * tol), what + " vs 256 x 128"
        else:
            hu.assert_within_budget(got, ref, mag, what=what)
            hu.assert_within_budget(got, narrow, 2 * mag, what=what + " vs 256 x 128")
    finally:
        L.llhip_set_q8_tile(0)


@pytest.mark.parametrize("m,n,k", [(300, 256, 1024), (513, 640, 320), (257, 128, 4096), (1024, 384, 2048),
                                   (512, 24576, 128)])
def test_gemm_q8_swiglu_quantized(m, n, k):
    """llhip_gemm_q8_swiglu_quantize: hb quantized in the wide int8 kernel's epilogue, bitwise k_gemm_q8 GEMM_SWIGLU then
    k_quantize_rows of its output; it declines (returns 0, writes nothing) where the launcher would not run the wide
    kernel unsplit, and a non-finite hb value fails as k_quantize_rows does. n = 24576 at 512 rows is 384 wide tiles
    on 256 CUs: the last 8192 columns go to the 256 x 128 kernel, whose epilogue quantizes each tile's 64-column
    group across its two waves."""
    L = hu.lib()
    gs = 64
    xq, xs, wq, ws, w3q, w3s, rng = gemm_case(m, n, k, gs, 6161 + m + n)
    t = hu.torch()
    dx = [hu.dev(a) for a in (xq, xs, wq, ws, w3q, w3s)]
    w1, w3 = lh.w8(dx[2], dx[3]), lh.w8(dx[4], dx[5])
    try:
        L.llhip_set_q8_tile(2)
        L.llhip_set_gemm_splits(1)
        hq, hs = hu.empty((m, n), t.int8), hu.empty((m, n // 64), t.float32)
        assert L.llhip_gemm_q8_swiglu_quantize(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, gs, ctypes.byref(w1), ctypes.byref(w3),
                                               n, lh.ptr(hq), lh.ptr(hs)) == 1
        hb = hu.dev(np.zeros((m, n), np.float32))
        seg = lh.GemmQ8Segment(lh.ptr(hb), n, w1, w3, None, None, n, lh.GEMM_SWIGLU)
        L.k_gemm_q8(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, gs, seg, 1)
        q2, s2 = hu.empty((m, n), t.int8), hu.empty((m, n // 64), t.float32)
        L.k_quantize_rows(lh.ptr(q2), lh.ptr(s2), lh.ptr(hb), n, m, n, gs)
        assert lh.last_error() == "", lh.last_error()
        assert np.array_equal(hu.host(hq), hu.host(q2)), "quantized values"
        assert np.array_equal(hu.bits(hu.host(hs)), hu.bits(hu.host(s2))), "scales"
        # declined: the 256 x 128 kernel forced, or split K, or another group size; nothing is written (a wide grid of
        # more tiles than the split workspace holds is never split, so a forced split count leaves it as it is)
        wide_tiles = -(-m // 256) * -(-n // 128)
        for tile, splits in ((1, 1), (2, 2)) if wide_tiles <= 256 else ((1, 1),):
            L.llhip_set_q8_tile(tile)
            L.llhip_set_gemm_splits(splits)
            hq0 = hu.dev(np.full((m, n), 7, np.int8))
            assert L.llhip_gemm_q8_swiglu_quantize(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, gs, ctypes.byref(w1),
                                                   ctypes.byref(w3), n, lh.ptr(hq0), lh.ptr(hs)) == 0
            assert np.all(hu.host(hq0) == 7)
        L.llhip_set_q8_tile(2)
        L.llhip_set_gemm_splits(1)
        assert L.llhip_gemm_q8_swiglu_quantize(lh.ptr(dx[0]), lh.ptr(dx[1]), m, k, 32, ctypes.byref(w1),
                                               ctypes.byref(w3), n, lh.ptr(hq), lh.ptr(hs)) == 0
        if m == 300:
            lh.record_failures()
            try:
                xs_bad = xs.copy()
                xs_bad[5, 0] = np.inf  # row 5's dots become infinite, its SwiGLU values non-finite
                assert L.llhip_gemm_q8_swiglu_quantize(lh.ptr(dx[0]), lh.ptr(hu.dev(xs_bad)), m, k, gs,
                                                       ctypes.byref(w1), ctypes.byref(w3), n, lh.ptr(hq),
                                                       lh.ptr(hs)) == 1
                L.llhip_synchronize()
                assert "nonfinite activation during INT8 quantization" in lh.last_error(), lh.last_error()
            finally:
                L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
                L.llhip_clear_error()
    finally:
        L.llhip_set_q8_tile(0)
        L.llhip_set_gemm_splits(0)


def test_gemm_q8_qkv_segments_and_gemv_agreement():
    """Three segments sharing the activations (QKV), and each GEMM row against the GEMV of that row."""
    L = hu.lib()
    m, k, gs = 70, 1024, 64
    xq, xs, wq, ws, _, _, rng = gemm_case(m, 96, k, gs, 707)
    mats = [synth_weights(rng, n, k, gs) for n in (96, 32, 32)]
    dxq, dxs = hu.dev(xq), hu.dev(xs)
    outs = [hu.empty((m, n), hu.torch().float32) for n in (96, 32, 32)]
    dw = [(hu.dev(q), hu.dev(s)) for q, s in mats]
    segs = (lh.GemmQ8Segment * 3)(*[lh.GemmQ8Segment(lh.ptr(o), o.shape[1], lh.w8(*w), lh.K8Weight(), None, None,
                                                     o.shape[1], lh.GEMM_STORE) for o, w in zip(outs, dw)])
    L.k_gemm_q8(lh.ptr(dxq), lh.ptr(dxs), m, k, gs, segs, 3)
    for o, (q, s), w in zip(outs, mats, dw):
        got = hu.host(o)
        ref, mag = hu.dequant_reference(xq, xs, q, s, gs)
        hu.assert_within_budget(got, ref, mag, what="qkv segment")
        for i in (0, m // 2, m - 1):
            row = hu.empty(q.shape[0], hu.torch().float32)
            L.k_matmul_q8(lh.ptr(row), lh.k8(dxq[i], dxs[i]), lh.w8(*w), k, q.shape[0], gs)
            hu.assert_within_budget(hu.host(row), got[i], mag[i] * 2, what="gemm row vs gemv")


@pytest.mark.parametrize("m,n,k,gs", [(33, 20, 128, 64), (130, 200, 1024, 64), (64, 64, 512, 128), (300, 130, 448, 64),
                                      (40, 24, 768, 256)])
def test_gemm_q8_int32_probe_bitwise(m, n, k, gs):
    L = hu.lib()
    xq, _, wq, _, _, _, _ = gemm_case(m, n, k, gs, 808 + m)
    dots = np.zeros((k // gs, m, n), np.int32)
    L.llhip_q8_group_dots(lh.ptr(dots), lh.ptr(xq), m, k, gs, lh.ptr(wq), n)
    assert lh.last_error() == ""
    assert np.array_equal(dots, orc.group_dots(xq, wq, gs))


@pytest.mark.parametrize("m,n,k,gs", [(33, 20, 128, 64), (70, 130, 1024, 128), (5, 17, 256, 256)])
def test_amx_dots_probe_from_packed_weights(m, n, k, gs):
    """testing.h:69 k_gemm_q8_amx_dots_test: the exact int32 group dots from weights in the pack_s8_vnni layout
    (unpacked on the device, then the MFMA probe); 0 for a group size the MFMA probe does not take."""
    L = hu.lib()
    xq, _, wq, _, _, _, _ = gemm_case(m, n, k, gs, 1111 + m)
    packed = np.zeros(L.s8_vnni_bytes(n, k), np.int8)
    L.pack_s8_vnni(lh.ptr(packed), lh.ptr(wq), n, k, k)
    dots = np.zeros((k // gs, m, n), np.int32)
    assert L.k_gemm_q8_amx_dots_test(lh.ptr(dots), lh.ptr(xq), m, k, gs, lh.ptr(packed), n) == 1, lh.last_error()
    assert np.array_equal(dots, orc.group_dots(xq, wq, gs))
    assert L.k_gemm_q8_amx_dots_test(lh.ptr(dots), lh.ptr(xq), m, k, 32, lh.ptr(packed), n) == 0


def test_gemm_q8_reference_golden_and_backends():
    """The reference's golden portable-GEMM cases: the MFMA backend (gs % 64 == 0) and the generic one, each within
    budget of the reference's outputs; the probe equals the reference's AMX int32 dots where the fixture has them."""
    g = np.load(os.path.join(GOLDEN, "gemm_q8.npz"))
    L = hu.lib()
    for key in sorted({k.split("/")[0] for k in g.files if k.endswith("/shape")}):
        m, n, k, gs = (int(v) for v in g[f"{key}/shape"])
        xq, xs, base = g[f"{key}/xq"], g[f"{key}/xs"], g[f"{key}/base"]
        wq, ws, w3q, w3s = (g[f"{key}/{a}"] for a in ("wq", "ws", "w3q", "w3s"))
        ref, mag = hu.dequant_reference(xq, xs, wq, ws, gs)
        backends = [lh.Q8_GEMM_PORTABLE] + ([lh.Q8_GEMM_HIP_MFMA] if gs % 64 == 0 else [])
        assert L.k_gemm_q8_pick(gs, None, 1) == (lh.Q8_GEMM_HIP_MFMA if gs % 64 == 0 else lh.Q8_GEMM_PORTABLE)
        for backend in backends:
            c = base.copy()
            seg = lh.GemmQ8Segment(lh.ptr(c), c.shape[1], lh.w8(wq, ws), lh.w8(w3q, w3s), None, None, n,
                                   lh.GEMM_STORE)
            assert L.k_gemm_q8_backend_test(backend, lh.ptr(xq), lh.ptr(xs), m, k, gs, seg, 1) == 1
            hu.assert_within_budget(c[:, :n], g[f"{key}/store"][:, :n], mag, rel=4e-5, what=f"{key} backend {backend}")
            hu.assert_within_budget(c[:, :n], ref, mag, what=f"{key} backend {backend} vs float64")
            assert np.array_equal(hu.bits(c[:, n:]), hu.bits(base[:, n:]))
        assert L.k_gemm_q8_backend_test(lh.Q8_GEMM_AMX, lh.ptr(xq), lh.ptr(xs), m, k, gs, None, 1) == 0
        if f"{key}/amx_dots" in g.files:
            dots = np.zeros((k // gs, m, n), np.int32)
            L.llhip_q8_group_dots(lh.ptr(dots), lh.ptr(xq), m, k, gs, lh.ptr(wq), n)
            assert np.array_equal(dots, g[f"{key}/amx_dots"]), key


# ---- the deferred (fused) quantization ------------------------------------------------------------------------------


@pytest.mark.parametrize("d,n", [(4096, 4096), (512, 14336), (300, 2048), (17, 1088)])
def test_fused_quantize_gemv(d, n):
    """k_quantize on device buffers is consumed by the next GEMV reading them: the output is within budget, q and s
    hold the quantization bitwise afterwards, and a second consumer reads them from memory."""
    L = hu.lib()
    T = hu.torch()
    gs = 64
    rng = orc.Rng(orc.SEED + 909 + d)
    wq, ws = synth_weights(rng, d, n, gs)
    x = rng.normal(n, 0.0, 1.0)
    xq, xs = orc.quantize(x, gs)
    ref, mag = hu.dequant_reference(xq, xs, wq, ws, gs)
    xd, dwq, dws = hu.dev(x), hu.dev(wq), hu.dev(ws)
    qd, sd = T.zeros(n, dtype=T.int8, device="cuda"), T.zeros(n // gs, dtype=T.float32, device="cuda")
    out, out2 = hu.empty(d, T.float32), hu.dev(np.ones(d, np.float32))
    T.cuda.synchronize()
    L.k_quantize(lh.ptr(qd), lh.ptr(sd), lh.ptr(xd), n, gs)
    L.k_matmul_q8(lh.ptr(out), lh.k8(qd, sd, xd), lh.w8(dwq, dws), n, d, gs)
    L.k_matmul_q8_add(lh.ptr(out2), lh.k8(qd, sd, xd), lh.w8(dwq, dws), n, d, gs)
    hu.assert_within_budget(hu.host(out), ref, mag, what="fused")
    hu.assert_within_budget(hu.host(out2), ref + 1.0, mag + 1.0, what="second consumer")
    assert np.array_equal(hu.host(qd), xq) and np.array_equal(hu.bits(hu.host(sd)), hu.bits(xs))


def test_recorded_quantization_is_launched_by_other_calls():
    L = hu.lib()
    T = hu.torch()
    n, gs = 2048, 64
    rng = orc.Rng(orc.SEED + 910)
    x = rng.normal(n, 0.0, 1.0)
    xq, xs = orc.quantize(x, gs)
    xd = hu.dev(x)
    for trigger in ("synchronize", "other_call"):
        qd, sd = T.zeros(n, dtype=T.int8, device="cuda"), T.zeros(n // gs, dtype=T.float32, device="cuda")
        T.cuda.synchronize()
        L.k_quantize(lh.ptr(qd), lh.ptr(sd), lh.ptr(xd), n, gs)
        if trigger == "other_call":
            other = hu.empty(64, T.float32)
            y = hu.dev(np.ones(64, np.float32))
            w = hu.dev(np.ones((64, 64), np.float32))
            L.k_matmul(lh.ptr(other), lh.ptr(y), lh.ptr(w), 64, 64)
        L.llhip_synchronize()
        assert np.array_equal(hu.host(qd), xq) and np.array_equal(hu.bits(hu.host(sd)), hu.bits(xs)), trigger


def test_fused_quantization_flags_nonfinite():
    L = hu.lib()
    T = hu.torch()
    lh.record_failures()
    try:
        n, d, gs = 1024, 64, 64
        x = np.ones(n, np.float32)
        x[7] = np.nan
        wq = np.ones((d, n), np.int8)
        ws = np.full((d, n // gs), 0.01, np.float32)
        xd, dwq, dws = hu.dev(x), hu.dev(wq), hu.dev(ws)
        qd, sd, out = hu.empty(n, T.int8), hu.empty(n // gs, T.float32), hu.empty(d, T.float32)
        L.k_quantize(lh.ptr(qd), lh.ptr(sd), lh.ptr(xd), n, gs)
        L.k_matmul_q8(lh.ptr(out), lh.k8(qd, sd, xd), lh.w8(dwq, dws), n, d, gs)
        L.llhip_synchronize()
        assert "nonfinite activation during INT8 quantization" in lh.last_error()
    finally:
        L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
        L.llhip_clear_error()


# ---- launch shapes of the streaming GEMV ----------------------------------------------------------------------------


@pytest.mark.parametrize("n", [1088, 4096, 14336])
def test_gemv_every_launch_shape(n):
    """Every waves-per-row split (1, 2, 4, 8), block size and grid size gives the same int32 group dots and in-budget
    outputs, for
    a three-segment QKV (rows of one step straddle segments), a SwiGLU pair and the ADD epilogue, fused and not."""
    L = hu.lib()
    T = hu.torch()
    gs = 64
    rng = orc.Rng(orc.SEED + 4242 + n)
    rows = (200, 56, 40)
    ws = [synth_weights(rng, d, n, gs) for d in rows]
    x = rng.normal(n, 0.0, 1.0)
    xq, xs = orc.quantize(x, gs)
    refs = [hu.dequant_reference(xq, xs, q, s, gs) for q, s in ws]
    xd = hu.dev(x)
    dws = [(hu.dev(q), hu.dev(s)) for q, s in ws]
    base = rng.uniform(rows[0], 3.0)
    try:
        for split in (1, 2, 4, 8):
            for blocks, waves in ((1, 8), (3, 8), (2, 16), (4, 16)):
                L.llhip_set_gemv_shape(split, blocks, waves)
                what = f"n {n} split {split} blocks/CU {blocks} waves/block {waves}"
                for fused in (True, False):
                    qd, sd = T.zeros(n, dtype=T.int8, device="cuda"), T.zeros(n // gs, dtype=T.float32, device="cuda")
                    outs = [hu.empty(d, T.float32) for d in rows]
                    T.cuda.synchronize()
                    if fused:
                        L.k_quantize(lh.ptr(qd), lh.ptr(sd), lh.ptr(xd), n, gs)
                    else:
                        qd.copy_(T.from_numpy(xq))
                        sd.copy_(T.from_numpy(xs))
                        T.cuda.synchronize()
                    inp = lh.k8(qd, sd, xd)
                    L.k_matmul_q8_qkv(lh.ptr(outs[0]), lh.ptr(outs[1]), lh.ptr(outs[2]), inp, lh.w8(*dws[0]),
                                      lh.w8(*dws[1]), lh.w8(*dws[2]), n, rows[0], rows[1], gs)
                    for o, (r, mag) in zip(outs, refs):
                        hu.assert_within_budget(hu.host(o), r, mag, what=f"qkv {what} fused {fused}")
                    assert np.array_equal(hu.host(qd), xq), what
                    # SwiGLU with the same matrix as value and gate: silu(r) * r
                    sw = hu.empty(rows[1], T.float32)
                    L.k_matmul_q8_swiglu(lh.ptr(sw), inp, lh.w8(*dws[1]), lh.w8(*dws[1]), n, rows[1], gs)
                    r1, m1 = refs[1]
                    got = hu.host(sw)
                    want = r1 / (1.0 + np.exp(-r1)) * r1
                    tol = 2e-5 * (m1 * (np.abs(r1) + 1) * 2) + 1e-6
                    assert np.all(np.abs(got - want) <= tol), f"swiglu {what}"
                    acc = hu.dev(base)
                    L.k_matmul_q8_add(lh.ptr(acc), inp, lh.w8(*dws[0]), n, rows[0], gs)
                    hu.assert_within_budget(hu.host(acc), base + refs[0][0], refs[0][1] + np.abs(base), what=f"add {what}")
                dots = np.zeros((n // gs, rows[0]), np.int32)
                L.llhip_q8_gemv_group_dots(lh.ptr(dots), lh.ptr(xq), lh.ptr(xs), lh.ptr(ws[0][0]), lh.ptr(ws[0][1]), 0,
                                           n, rows[0], gs)
                assert np.array_equal(dots, orc.group_dots(xq.reshape(1, -1), ws[0][0], gs)[:, 0, :]), what
    finally:
        L.llhip_set_gemv_shape(0, 0, 0)


def test_fused_quantization_with_output_over_its_input():
    """k_quantize(q, s, x) then k_matmul_q8_add(x, q/s): the residual output is the quantizer's own input. The result
    is x + W q(x) with q taken from x before any output is written (the fused kernel steps aside for this case)."""
    L = hu.lib()
    T = hu.torch()
    n = d = 4096
    gs = 64
    rng = orc.Rng(orc.SEED + 5151)
    wq, ws = synth_weights(rng, d, n, gs)
    x = rng.normal(n, 0.0, 1.0)
    xq, xs = orc.quantize(x, gs)
    ref, mag = hu.dequant_reference(xq, xs, wq, ws, gs)
    xd, dwq, dws = hu.dev(x), hu.dev(wq), hu.dev(ws)
    qd, sd = T.zeros(n, dtype=T.int8, device="cuda"), T.zeros(n // gs, dtype=T.float32, device="cuda")
    T.cuda.synchronize()
    L.k_quantize(lh.ptr(qd), lh.ptr(sd), lh.ptr(xd), n, gs)
    L.k_matmul_q8_add(lh.ptr(xd), lh.k8(qd, sd, xd), lh.w8(dwq, dws), n, d, gs)
    hu.assert_within_budget(hu.host(xd), x + ref, mag + np.abs(x), what="residual over the quantized input")
    assert np.array_equal(hu.host(qd), xq)
