"""The reference's k_gemm_q8 shape matrix replayed through the GPU library: tests/q8.c:224-231 (gs 2, 4, 32, 64,
128; k = 2 gs and 5 gs; m 1, 2, 3, 17, 33, 40; n 1, 5, 16, 17, 33) and its large shapes (tests/q8.c:267-273), each
with the reference's operands (uniform activations scaled by row, int8 weights uniform in [-127, 127], every seventh
weight scale zero, garbage int8 in the activation rows past m up to a multiple of 32) and its checks: k_quantize_rows
bitwise the oracle's per-token quantizer, every kind (STORE, ADD, SWIGLU, PARTIAL) within the budget of the double
reference from the dequantized operands (tests/q8.c:128-133), and the row padding past n untouched.

Every dispatch edge is taken: the launcher's own choice (the short-batch kernel for m <= 32 and gs % 64 == 0, the
tiled kernels above, the generic kernel for other group sizes), and for gs % 64 == 0 also forced split counts (which
send short batches to the tiled kernel) and, for gs = 64, the 256 x 256 kernels with either form of the scale
products."""
import numpy as np
import pytest

import llama_hip as lh
from oracle import pyoracle as orc
from tests import hip_util as hu

pytestmark = pytest.mark.gpu

MS, NS = (1, 2, 3, 17, 33, 40), (1, 5, 16, 17, 33)
LARGE = [(64, 130, 2048, 64), (64, 33, 8192, 64), (37, 520, 1024, 64), (128, 70, 2048, 128), (64, 600, 4096, 64),
         (96, 257, 3072, 64), (16, 48, 128, 64), (16, 48, 512, 64), (16, 48, 1024, 64), (16, 48, 2048, 64),
         (16, 48, 4096, 64), (16, 48, 8192, 64), (16, 48, 14336, 64), (64, 4096, 2048, 64), (64, 14336, 4096, 64),
         (53, 1024, 2048, 64)]
KINDS = (lh.GEMM_STORE, lh.GEMM_ADD, lh.GEMM_SWIGLU, lh.GEMM_PARTIAL)


def make_case(rng, m, n, k, gs):
    """The operands of tests/q8.c:53-77, drawn with numpy."""
    groups = k // gs
    x = (rng.uniform(-1, 1, (m, k)) * (1.0 + (np.arange(m) % 3))[:, None]).astype(np.float32)
    rows = (m + 31) // 32 * 32
    xq_pad = rng.integers(-127, 128, (rows, k)).astype(np.int8)  # garbage in the padding rows
    xs_pad = rng.uniform(0, 1, (rows, groups)).astype(np.float32)
    wq = rng.integers(-127, 128, (n, k)).astype(np.int8)
    wq3 = rng.integers(-127, 128, (n, k)).astype(np.int8)
    ws = (np.abs(rng.uniform(-1, 1, n * groups)) * 0.02).astype(np.float32)
    ws[np.arange(n * groups) % 7 == 3] = 0.0
    ws3 = (np.abs(rng.uniform(-1, 1, n * groups)) * 0.02).astype(np.float32)
    return x, xq_pad, xs_pad, wq, ws.reshape(n, groups), wq3, ws3.reshape(n, groups)


def forcings(m, gs):
    """(q8 tile, splits, scale products) settings: the launcher's choice, then the forced edges for gs % 64 == 0."""
    out = [(0, 0, 0)]
    if gs % 64 == 0:
        out.append((1, 2, 0))  # split K in two on the 256 x 128 kernel (short batches included)
    if gs == 64:
        out += [(2, 1, 1), (2, 3, 2), (2, 1, 2)]  # 256 x 256, unsplit and split, either form of the scale products
    return out


def check_case(L, rng, m, n, k, gs):
    T = hu.torch()
    x, xq_pad, xs_pad, wq, ws, wq3, ws3 = make_case(rng, m, n, k, gs)
    # k_quantize_rows writes the first m rows of the padded buffers, bitwise the per-token quantizer
    xq_d, xs_d, x_d = hu.dev(xq_pad), hu.dev(xs_pad), hu.dev(x)
    L.k_quantize_rows(lh.ptr(xq_d), lh.ptr(xs_d), lh.ptr(x_d), k, m, k, gs)
    q_got, s_got = hu.host(xq_d), hu.host(xs_d)
    q_want, s_want = orc.quantize(x, gs)
    assert np.array_equal(q_got[:m], q_want) and np.array_equal(hu.bits(s_got[:m]), hu.bits(s_want)), (m, n, k, gs)
    assert np.array_equal(q_got[m:], xq_pad[m:]), "k_quantize_rows wrote past its rows"
    ref, mag = hu.dequant_reference(q_want, s_want, wq, ws, gs)
    r3, mag3 = hu.dequant_reference(q_want, s_want, wq3, ws3, gs)
    ldc = n + 5
    base = rng.uniform(-3, 3, (m, ldc)).astype(np.float32)
    w_d = [hu.dev(a) for a in (wq, ws, wq3, ws3)]
    for tile, splits, scales in forcings(m, gs):
        L.llhip_set_q8_tile(tile)
        L.llhip_set_gemm_splits(splits)
        L.llhip_set_q8_scales(scales)
        for kind in KINDS:
            c = hu.dev(base)
            seg = lh.GemmQ8Segment(lh.ptr(c), ldc, lh.w8(w_d[0], w_d[1]), lh.w8(w_d[2], w_d[3]), None, None, n, kind)
            L.k_gemm_q8(lh.ptr(xq_d), lh.ptr(xs_d), m, k, gs, seg, 1)
            got = hu.host(c)
            what = f"m={m} n={n} k={k} gs={gs} kind={kind} tile={tile} splits={splits} scales={scales}"
            assert lh.last_error() == "", (what, lh.last_error())
            old = base[:, :n].astype(np.float64)
            if kind == lh.GEMM_ADD:
                want, tol = old + ref, 2e-5 * (mag + np.abs(old)) + 1e-6
            elif kind == lh.GEMM_SWIGLU:
                want = ref / (1 + np.exp(-ref)) * r3
                tol = 2e-5 * (mag * (np.abs(r3) + 1) + mag3 * (np.abs(ref) + 1)) + 1e-6
            else:
                want, tol = ref, 2e-5 * mag + 1e-6
            err = np.abs(got[:, :n] - want)
            assert np.all(err <= tol), (what, float(np.max(err - tol)))
            assert np.array_equal(hu.bits(got[:, n:]), hu.bits(base[:, n:])), what + ": wrote into the row padding"
    del T


@pytest.mark.parametrize("gs", [2, 4, 32, 64, 128])
def test_gemm_q8_reference_matrix(gs):
    L = hu.lib()
    rng = np.random.default_rng(224 + gs)
    try:
        for mult in (2, 5):
            for m in MS:
                for n in NS:
                    check_case(L, rng, m, n, gs * mult, gs)
    finally:
        L.llhip_set_q8_tile(0)
        L.llhip_set_gemm_splits(0)
        L.llhip_set_q8_scales(0)


@pytest.mark.parametrize("m,n,k,gs", LARGE)
def test_gemm_q8_reference_large_shapes(m, n, k, gs):
    L = hu.lib()
    rng = np.random.default_rng(267 + m + n + k)
    try:
        check_case(L, rng, m, n, k, gs)
    finally:
        L.llhip_set_q8_tile(0)
        L.llhip_set_gemm_splits(0)
        L.llhip_set_q8_scales(0)
