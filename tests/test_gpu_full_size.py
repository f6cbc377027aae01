"""GPU parity at the full sizes of the benchmarked workloads, through the C ABI.

The smaller parity tests compare every output with the oracle. At full size a float64 reference of every output is
too slow on the host, so these tests check what does not depend on size:
  - the quantized activations are bit-identical to the oracle's k_quantize (all of them);
  - sampled output rows (first, last, tile and segment boundaries, a few random ones) are within the reference's
    budget of a float64 product of the dequantized (Q8) or BF16-rounded operands;
  - a GEMM row equals the GEMV of that row within the budget (tests/q8.c:158-183 checks the same on the CPU);
  - GEMV outputs of the 1B decode set are checked in full (every row), the classifier in row chunks.
Weights ~N(0, 0.02), activations ~N(0, 1), from the reference tests' xorshift stream (oracle.Rng), quantized by the
Q8_0 rule with gs 64.
"""
import numpy as np
import pytest

import llama_hip as lh
from oracle import pyoracle as orc
from tests import hip_util as hu

pytestmark = pytest.mark.gpu
GS = 64


@pytest.fixture(scope="module", autouse=True)
def device():
    L = hu.lib()
    assert L.llhip_init() == 0, lh.last_error()
    yield L


def q8_weights(rng, n, k):
    return orc.quantize_weights(rng.normal(n * k, 0.0, 0.02).reshape(n, k), GS)


def dequant(q, s):
    return q.astype(np.float64) * np.repeat(s.astype(np.float64), GS, axis=-1)


def sample_rows(m, extra=()):
    rng = np.random.default_rng(m)
    rows = {0, 1, m // 2, m - 2, m - 1, *[r for r in extra if 0 <= r < m]}
    rows.update(int(r) for r in rng.integers(0, m, 3))
    return sorted(rows)


def swiglu_check(got, r, mag, r3, mag3, what):
    want = r / (1 + np.exp(-r)) * r3
    tol = 2e-5 * (mag * (np.abs(r3) + 1) + mag3 * (np.abs(r) + 1)) + 1e-6  # tests/q8.c:130
    err = np.abs(np.asarray(got, np.float64) - want)
    assert np.all(err <= tol), f"{what}: swiglu outside budget, worst {np.max(err - tol):.3g}"


# ---- Llama-3.2-1B decode set (configs C1 and C2) ------------------------------------------------------------------


def test_1b_decode_set_full_outputs():
    """One 1B decode step's matmuls on device buffers: k_quantize (recorded, fused into the next GEMV), QKV (2048 +
    512 + 512 rows), Wo + residual, W1/W3 SwiGLU (8192 rows), W2 + residual (k = 8192), classifier (128256 rows)."""
    L = hu.lib()
    T = hu.torch()
    rng = orc.Rng(orc.SEED + 1001)
    dim, kv, hidden, vocab = 2048, 512, 8192, 128256
    x = rng.normal(dim, 0.0, 1.0)
    h = rng.normal(hidden, 0.0, 1.0)
    xq_want, xs_want = orc.quantize(x, GS)
    hq_want, hs_want = orc.quantize(h, GS)
    xq_want, xs_want, hq_want, hs_want = (a.reshape(-1) for a in (xq_want, xs_want, hq_want, hs_want))
    xd = dequant(xq_want, xs_want)
    hd = dequant(hq_want, hs_want)

    dx, dh = hu.dev(x), hu.dev(h)
    dxq, dxs = hu.empty(dim, T.int8), hu.empty(dim // GS, T.float32)
    dhq, dhs = hu.empty(hidden, T.int8), hu.empty(hidden // GS, T.float32)
    inp, hinp = lh.K8Input(lh.ptr(dxq), lh.ptr(dxs), None), lh.K8Input(lh.ptr(dhq), lh.ptr(dhs), None)

    def check(out, w, src, extra=0.0, what=""):
        wd = dequant(*w)
        hu.assert_within_budget(out, wd @ src + extra, np.abs(wd) @ np.abs(src) + np.abs(extra), what=what)

    # QKV
    wq, wk, wv = q8_weights(rng, dim, dim), q8_weights(rng, kv, dim), q8_weights(rng, kv, dim)
    dq = [tuple(hu.dev(a) for a in w) for w in (wq, wk, wv)]
    outs = [hu.empty(r, T.float32) for r in (dim, kv, kv)]
    L.k_quantize(lh.ptr(dxq), lh.ptr(dxs), lh.ptr(dx), dim, GS)
    L.k_matmul_q8_qkv(lh.ptr(outs[0]), lh.ptr(outs[1]), lh.ptr(outs[2]), inp, lh.w8(*dq[0]), lh.w8(*dq[1]),
                      lh.w8(*dq[2]), dim, dim, kv, GS)
    assert np.array_equal(hu.host(dxq), xq_want) and np.array_equal(hu.bits(hu.host(dxs)), hu.bits(xs_want))
    for o, w, name in zip(outs, (wq, wk, wv), ("q", "k", "v")):
        check(hu.host(o), w, xd, what=f"1B {name}")
    # Wo + residual
    wo = q8_weights(rng, dim, dim)
    resid = rng.normal(dim, 0.0, 1.0)
    dres = hu.dev(resid)
    dwo = tuple(hu.dev(a) for a in wo)
    L.k_quantize(lh.ptr(dxq), lh.ptr(dxs), lh.ptr(dx), dim, GS)
    L.k_matmul_q8_add(lh.ptr(dres), inp, lh.w8(*dwo), dim, dim, GS)
    check(hu.host(dres), wo, xd, resid.astype(np.float64), what="1B wo + residual")
    # W1/W3 SwiGLU
    w1, w3 = q8_weights(rng, hidden, dim), q8_weights(rng, hidden, dim)
    d1, d3 = tuple(hu.dev(a) for a in w1), tuple(hu.dev(a) for a in w3)
    hb = hu.empty(hidden, T.float32)
    L.k_quantize(lh.ptr(dxq), lh.ptr(dxs), lh.ptr(dx), dim, GS)
    L.k_matmul_q8_swiglu(lh.ptr(hb), inp, lh.w8(*d1), lh.w8(*d3), dim, hidden, GS)
    w1d, w3d = dequant(*w1), dequant(*w3)
    swiglu_check(hu.host(hb), w1d @ xd, np.abs(w1d) @ np.abs(xd), w3d @ xd, np.abs(w3d) @ np.abs(xd), "1B w1/w3")
    # W2 + residual (k = 8192)
    w2 = q8_weights(rng, dim, hidden)
    d2 = tuple(hu.dev(a) for a in w2)
    res2 = rng.normal(dim, 0.0, 1.0)
    dres2 = hu.dev(res2)
    L.k_quantize(lh.ptr(dhq), lh.ptr(dhs), lh.ptr(dh), hidden, GS)
    L.k_matmul_q8_add(lh.ptr(dres2), hinp, lh.w8(*d2), hidden, dim, GS)
    assert np.array_equal(hu.host(dhq), hq_want) and np.array_equal(hu.bits(hu.host(dhs)), hu.bits(hs_want))
    check(hu.host(dres2), w2, hd, res2.astype(np.float64), what="1B w2 + residual")
    # classifier, checked in row chunks
    wc = q8_weights(rng, vocab, dim)
    dwc = tuple(hu.dev(a) for a in wc)
    logits = hu.empty(vocab, T.float32)
    L.k_quantize(lh.ptr(dxq), lh.ptr(dxs), lh.ptr(dx), dim, GS)
    L.k_matmul_q8(lh.ptr(logits), inp, lh.w8(*dwc), dim, vocab, GS)
    got = hu.host(logits)
    for r0 in range(0, vocab, 16384):
        r1 = min(vocab, r0 + 16384)
        check(got[r0:r1], (wc[0][r0:r1], wc[1][r0:r1]), xd, what=f"1B classifier rows {r0}..{r1}")


# ---- Llama-3.1-8B INT8 prefill, 2048 tokens (config C4) -----------------------------------------------------------


def test_8b_int8_prefill_full_size():
    """k_quantize_rows of the 2048 x 4096 and 2048 x 14336 activations (bitwise, all rows) and the four GEMMs of a
    layer at full size: QKV (three segments), Wo + residual, W1/W3 SwiGLU, W2 + residual (k = 14336). Sampled rows
    against float64; two rows against the GEMV."""
    L = hu.lib()
    T = hu.torch()
    rng = orc.Rng(orc.SEED + 1002)
    m, dim, kv, hidden = 2048, 4096, 1024, 14336
    x = rng.normal(m * dim, 0.0, 1.0).reshape(m, dim)
    h = rng.normal(m * hidden, 0.0, 1.0).reshape(m, hidden)
    dx, dh = hu.dev(x), hu.dev(h)
    dxq, dxs = hu.empty((m, dim), T.int8), hu.empty((m, dim // GS), T.float32)
    dhq, dhs = hu.empty((m, hidden), T.int8), hu.empty((m, hidden // GS), T.float32)
    L.k_quantize_rows(lh.ptr(dxq), lh.ptr(dxs), lh.ptr(dx), dim, m, dim, GS)
    L.k_quantize_rows(lh.ptr(dhq), lh.ptr(dhs), lh.ptr(dh), hidden, m, hidden, GS)
    xq, xs = orc.quantize(x, GS)
    hq, hs = orc.quantize(h, GS)
    assert np.array_equal(hu.host(dxq), xq) and np.array_equal(hu.bits(hu.host(dxs)), hu.bits(xs))
    assert np.array_equal(hu.host(dhq), hq) and np.array_equal(hu.bits(hu.host(dhs)), hu.bits(hs))
    rows = sample_rows(m, extra=(255, 256, 1023, 1024))
    xd, hd = dequant(xq[rows], xs[rows]), dequant(hq[rows], hs[rows])

    def seg(out, w, w3=None, kind=lh.GEMM_STORE):
        return lh.GemmQ8Segment(lh.ptr(out), out.shape[1], lh.w8(*w), lh.w8(*w3) if w3 else lh.K8Weight(), None,
                                None, out.shape[1], kind)

    # QKV
    mats = [q8_weights(rng, n, dim) for n in (dim, kv, kv)]
    dm = [tuple(hu.dev(a) for a in w) for w in mats]
    outs = [hu.empty((m, n), T.float32) for n in (dim, kv, kv)]
    segs = (lh.GemmQ8Segment * 3)(*[seg(o, w) for o, w in zip(outs, dm)])
    L.k_gemm_q8(lh.ptr(dxq), lh.ptr(dxs), m, dim, GS, segs, 3)
    for o, w, name in zip(outs, mats, ("q", "k", "v")):
        wd = dequant(*w)
        hu.assert_within_budget(hu.host(o)[rows], xd @ wd.T, np.abs(xd) @ np.abs(wd).T, what=f"8B {name}")
    # the GEMM's rows against the GEMV of the same rows
    q_host = hu.host(outs[0])
    wd = dequant(*mats[0])
    for r in (0, m - 1):
        row = hu.empty(dim, T.float32)
        L.k_matmul_q8(lh.ptr(row), lh.k8(dxq[r], dxs[r]), lh.w8(*dm[0]), dim, dim, GS)
        mag = np.abs(dequant(xq[r], xs[r])) @ np.abs(wd).T
        hu.assert_within_budget(hu.host(row), q_host[r], 2 * mag, what=f"8B gemm row {r} vs gemv")
    # Wo + residual
    wo = q8_weights(rng, dim, dim)
    dwo = tuple(hu.dev(a) for a in wo)
    base = rng.normal(m * dim, 0.0, 1.0).reshape(m, dim)
    c = hu.dev(base)
    L.k_gemm_q8(lh.ptr(dxq), lh.ptr(dxs), m, dim, GS, seg(c, dwo, kind=lh.GEMM_ADD), 1)
    wd = dequant(*wo)
    hu.assert_within_budget(hu.host(c)[rows], base[rows] + xd @ wd.T, np.abs(xd) @ np.abs(wd).T + np.abs(base[rows]),
                            what="8B wo + residual")
    # W1/W3 SwiGLU
    w1, w3 = q8_weights(rng, hidden, dim), q8_weights(rng, hidden, dim)
    d1, d3 = tuple(hu.dev(a) for a in w1), tuple(hu.dev(a) for a in w3)
    hb = hu.empty((m, hidden), T.float32)
    L.k_gemm_q8(lh.ptr(dxq), lh.ptr(dxs), m, dim, GS, seg(hb, d1, d3, lh.GEMM_SWIGLU), 1)
    w1d, w3d = dequant(*w1), dequant(*w3)
    swiglu_check(hu.host(hb)[rows], xd @ w1d.T, np.abs(xd) @ np.abs(w1d).T, xd @ w3d.T, np.abs(xd) @ np.abs(w3d).T,
                 "8B w1/w3")
    del d1, d3, hb
    # W2 + residual (k = 14336)
    w2 = q8_weights(rng, dim, hidden)
    d2 = tuple(hu.dev(a) for a in w2)
    base2 = rng.normal(m * dim, 0.0, 1.0).reshape(m, dim)
    c2 = hu.dev(base2)
    L.k_gemm_q8(lh.ptr(dhq), lh.ptr(dhs), m, hidden, GS, seg(c2, d2, kind=lh.GEMM_ADD), 1)
    wd = dequant(*w2)
    hu.assert_within_budget(hu.host(c2)[rows], base2[rows] + hd @ wd.T,
                            np.abs(hd) @ np.abs(wd).T + np.abs(base2[rows]), what="8B w2 + residual")
    assert lh.last_error() == ""


# ---- Llama-3.2-3B FP32 / BF16 prefill, 512 tokens (config C3) -----------------------------------------------------


def bf16_round(x):
    """Finite float32 values rounded to BF16 (nearest, ties to even) and widened back."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)).view(np.float32)


@pytest.mark.parametrize("mode", ["f32", "bf16"])
def test_3b_prefill_full_size(mode):
    """The four GEMMs of a 3B layer at 512 tokens in FP32 or BF16 mode (the grids split K): QKV, Wo + residual,
    W1/W3 SwiGLU, W2 + residual (k = 8192). Sampled rows against float64 of the (BF16-rounded) operands."""
    L = hu.lib()
    rng = orc.Rng(orc.SEED + 1003 + (mode == "bf16"))
    m, dim, kv, hidden = 512, 3072, 1024, 8192
    x = rng.normal(m * dim, 0.0, 1.0).reshape(m, dim)
    h = rng.normal(m * hidden, 0.0, 1.0).reshape(m, hidden)
    rows = sample_rows(m, extra=(255, 256))
    rel = 2e-6 if mode == "bf16" else 2e-5
    panel = lh.AlignedBuffer()
    L.aligned_buffer_alloc(panel, L.k_gemm_bf16_panel_bytes(m, hidden), 1)
    dx, dh = hu.dev(x), hu.dev(h)
    xr = bf16_round(x[rows]) if mode == "bf16" else x[rows]
    hr = bf16_round(h[rows]) if mode == "bf16" else h[rows]
    xr, hr = xr.astype(np.float64), hr.astype(np.float64)

    def weights(n, k):
        w = rng.normal(n * k, 0.0, 0.02).reshape(n, k)
        ref = (bf16_round(w) if mode == "bf16" else w).astype(np.float64)
        return (hu.dev(orc.pack_bf16_vnni(w)) if mode == "bf16" else hu.dev(w)), ref

    def gemm(a, lda, k, outs_ws, kind):
        if mode == "bf16":
            segs = (lh.GemmBf16Segment * len(outs_ws))(
                *[lh.GemmBf16Segment(lh.ptr(o), o.shape[1], lh.ptr(w), lh.ptr(w3) if w3 is not None else None,
                                     o.shape[1], kind) for o, w, w3 in outs_ws])
            L.k_gemm_bf16(lh.ptr(a), lda, m, k, segs, len(outs_ws), panel)
        else:
            segs = (lh.GemmSegment * len(outs_ws))(
                *[lh.GemmSegment(lh.ptr(o), o.shape[1], lh.ptr(w), lh.ptr(w3) if w3 is not None else None, k,
                                 o.shape[1], kind) for o, w, w3 in outs_ws])
            L.k_gemm_f32(lh.ptr(a), lda, m, k, segs, len(outs_ws))

    try:
        # QKV
        mats = [weights(n, dim) for n in (dim, kv, kv)]
        outs = [hu.dev(np.zeros((m, n), np.float32)) for n in (dim, kv, kv)]
        gemm(dx, dim, dim, [(o, w, None) for o, (w, _) in zip(outs, mats)], lh.GEMM_STORE)
        for o, (_, wr), name in zip(outs, mats, ("q", "k", "v")):
            hu.assert_within_budget(hu.host(o)[rows], xr @ wr.T, np.abs(xr) @ np.abs(wr).T, rel=rel,
                                    what=f"3B {mode} {name}")
        # Wo + residual
        wo, wor = weights(dim, dim)
        base = rng.normal(m * dim, 0.0, 1.0).reshape(m, dim)
        c = hu.dev(base)
        gemm(dx, dim, dim, [(c, wo, None)], lh.GEMM_ADD)
        hu.assert_within_budget(hu.host(c)[rows], base[rows] + xr @ wor.T,
                                np.abs(xr) @ np.abs(wor).T + np.abs(base[rows]), rel=rel, what=f"3B {mode} wo")
        # W1/W3 SwiGLU
        (w1, w1r), (w3, w3r) = weights(hidden, dim), weights(hidden, dim)
        hb = hu.dev(np.zeros((m, hidden), np.float32))
        gemm(dx, dim, dim, [(hb, w1, w3)], lh.GEMM_SWIGLU)
        r, r3 = xr @ w1r.T, xr @ w3r.T
        want = r / (1 + np.exp(-r)) * r3
        mag, mag3 = np.abs(xr) @ np.abs(w1r).T, np.abs(xr) @ np.abs(w3r).T
        tol = (rel if mode == "bf16" else 2e-5) * (mag * (np.abs(r3) + 1) + mag3 * (np.abs(r) + 1)) + 1e-6
        assert np.all(np.abs(hu.host(hb)[rows] - want) <= tol), f"3B {mode} w1/w3"
        # W2 + residual (k = 8192)
        w2, w2r = weights(dim, hidden)
        base2 = rng.normal(m * dim, 0.0, 1.0).reshape(m, dim)
        c2 = hu.dev(base2)
        gemm(dh, hidden, hidden, [(c2, w2, None)], lh.GEMM_ADD)
        hu.assert_within_budget(hu.host(c2)[rows], base2[rows] + hr @ w2r.T,
                                np.abs(hr) @ np.abs(w2r).T + np.abs(base2[rows]), rel=rel, what=f"3B {mode} w2")
        assert lh.last_error() == ""
    finally:
        L.aligned_buffer_free(panel)
