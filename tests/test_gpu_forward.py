"""GPU parity of the forward around the matmuls through the C ABI: RMSNorm, RoPE (table and rotation), the K/V cache
store and causal attention (decode and batched, rows and head-major layouts).

The oracle (oracle/, pinned bitwise to the reference's scalar kernels by tests/test_oracle.py) is the checker. The bar:
RoPE, its table and the cache store are bitwise the reference's; RMSNorm differs only in the order of its sum of squares
(relative 1e-5); attention sums scores, exponentials and values in other orders (split over 64-position chunks, as the
reference's own split-K form does), so it is checked against a float64 evaluation within 1e-5 of sum_t w_t |v_t| plus
1e-6, and against the oracle within twice that.
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
    assert L.llhip_init() == 0, lh.last_error()
    yield L


def golden():
    return np.load(os.path.join(GOLDEN, "forward.npz"))


# ---- RMSNorm ---------------------------------------------------------------------------------------------------------


def test_rmsnorm_golden_device_host_and_in_place():
    L = hu.lib()
    g = golden()
    for size in (1, 100, 2048, 3072, 4096):
        x, w, want = g[f"rms{size}/x"], g[f"rms{size}/w"], g[f"rms{size}/out"]
        tol = 1e-5 * np.abs(want) + 1e-7
        out = np.zeros_like(x)
        L.k_rmsnorm(lh.ptr(out), lh.ptr(x), lh.ptr(w), size, 1e-5)  # host buffers
        assert np.all(np.abs(out - want) <= tol), size
        dx, dw = hu.dev(x), hu.dev(w)
        L.k_rmsnorm(lh.ptr(dx), lh.ptr(dx), lh.ptr(dw), size, 1e-5)  # device, in place
        assert np.all(np.abs(hu.host(dx) - want) <= tol), size
    x, w, want = g["rmsrows/x"], g["rmsrows/w"], g["rmsrows/out"]
    dx, dw, do = hu.dev(x), hu.dev(w), hu.empty(x.shape, hu.torch().float32)
    L.k_rmsnorm_rows(lh.ptr(do), lh.ptr(dx), lh.ptr(dw), 3, 512, 1e-5)
    assert np.all(np.abs(hu.host(do) - want) <= 1e-5 * np.abs(want) + 1e-7)


@pytest.mark.parametrize("rows,size", [(1, 8192), (64, 4096), (7, 1000)])
def test_rmsnorm_rows_against_oracle(rows, size):
    L = hu.lib()
    rng = orc.Rng(orc.SEED + rows * 13 + size)
    x, w = rng.normal(rows * size, 0.0, 2.0).reshape(rows, size), rng.normal(size, 1.0, 0.2)
    want = orc.rmsnorm(x, w, 1e-6)
    dx, dw, do = hu.dev(x), hu.dev(w), hu.empty((rows, size), hu.torch().float32)
    L.k_rmsnorm_rows(lh.ptr(do), lh.ptr(dx), lh.ptr(dw), rows, size, 1e-6)
    assert np.all(np.abs(hu.host(do) - want) <= 1e-5 * np.abs(want) + 1e-7)


@pytest.mark.parametrize("rows,size,gs", [(1, 4096, 64), (37, 4096, 64), (5, 2048, 64), (9, 3072, 32), (3, 8192, 64),
                                          (4, 640, 128), (6, 96, 4), (2, 1024, 256), (130, 4096, 64)])
def test_rmsnorm_quantize_rows_fused(rows, size, gs):
    """llhip_rmsnorm_quantize_rows: bitwise k_rmsnorm_rows then k_quantize_rows (the same normalized values, the same
    quantization), over rows up to 8192 values and group sizes 4-256, with values at rounding ties of the quantizer;
    and a non-finite value fails as k_quantize_rows does."""
    L = hu.lib()
    rng = orc.Rng(orc.SEED + 3100 + rows * 7 + size + gs)
    x = rng.normal(rows * size, 0.0, 2.0).reshape(rows, size)
    x[0, :8] = [0.0, -0.0, 1e-30, 3.5, -3.5, 127.0, -127.0, 0.5]
    w = rng.normal(size, 1.0, 0.2)
    dx, dw = hu.dev(x), hu.dev(w)
    groups = size // gs
    t = hu.torch()
    q1, s1 = hu.empty((rows, size), t.int8), hu.empty((rows, groups), t.float32)
    q2, s2, xb = hu.empty((rows, size), t.int8), hu.empty((rows, groups), t.float32), hu.empty((rows, size), t.float32)
    L.llhip_rmsnorm_quantize_rows(lh.ptr(q1), lh.ptr(s1), lh.ptr(dx), lh.ptr(dw), rows, size, 1e-5, gs)
    L.k_rmsnorm_rows(lh.ptr(xb), lh.ptr(dx), lh.ptr(dw), rows, size, 1e-5)
    L.k_quantize_rows(lh.ptr(q2), lh.ptr(s2), lh.ptr(xb), size, rows, size, gs)
    assert lh.last_error() == "", lh.last_error()
    assert np.array_equal(hu.host(q1), hu.host(q2)), "quantized values"
    assert np.array_equal(hu.bits(hu.host(s1)), hu.bits(hu.host(s2))), "scales"
    # against the oracle: its RMSNorm then quantization, within one step of the grid where the normalized value's
    # reduction order moves it across a rounding boundary
    want_q, want_s = orc.quantize(orc.rmsnorm(x, w, 1e-5), gs)
    assert np.allclose(hu.host(s1), want_s, rtol=1e-5, atol=0)
    assert np.max(np.abs(hu.host(q1).astype(int) - want_q.astype(int))) <= 1
    if rows == 1:
        lh.record_failures()
        try:
            x[0, 5] = np.inf
            L.llhip_rmsnorm_quantize_rows(lh.ptr(q1), lh.ptr(s1), lh.ptr(hu.dev(x)), lh.ptr(dw), rows, size, 1e-5, gs)
            L.llhip_synchronize()
            assert "nonfinite activation during INT8 quantization" in lh.last_error(), lh.last_error()
        finally:
            L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
            L.llhip_clear_error()


# ---- RoPE --------------------------------------------------------------------------------------------------------------


def rope_config(head_dim, llama3):
    c = lh.Config()
    c.head_dim = head_dim
    if llama3:
        c.rope_theta, c.rope_type, c.rope_factor, c.rope_low, c.rope_high, c.rope_original = 500000.0, 1, 8.0, 1.0, 4.0, 8192
    else:
        c.rope_theta, c.rope_type = 10000.0, 0
    return c


def test_rope_table_bitwise_host_and_device():
    """k_rope_table runs on the host with the C library, as the reference does: bitwise its tables (Llama 3.1 scaling at
    head_dim 128, plain theta 10000 at 64), written to host memory in place and to device memory by a copy."""
    L = hu.lib()
    g = golden()
    for hd, llama3 in ((128, True), (64, False)):
        cfg = rope_config(hd, llama3)
        for pos in (0, 1, 7, 1000, 8191, 100000):
            want = g[f"ropetab{hd}_{pos}/table"]
            t = np.zeros(2 * hd, np.float32)
            L.k_rope_table(ctypes.byref(cfg), pos, lh.ptr(t))
            assert np.array_equal(hu.bits(t), hu.bits(want)), (hd, pos)
            dt = hu.empty(2 * hd, hu.torch().float32)
            L.k_rope_table(ctypes.byref(cfg), pos, lh.ptr(dt))
            assert np.array_equal(hu.bits(hu.host(dt)), hu.bits(want)), (hd, pos)


def test_rope_apply_bitwise_golden_and_rows():
    L = hu.lib()
    g = golden()
    for hd in (128, 64):
        q, k, t = g[f"rope{hd}/q"].copy(), g[f"rope{hd}/k"].copy(), g[f"ropetab{hd}_1000/table"]
        L.k_rope_apply(lh.ptr(q), lh.ptr(k), lh.ptr(t), 8, 2, hd)  # host buffers
        assert np.array_equal(hu.bits(q), hu.bits(g[f"rope{hd}/q_out"]))
        assert np.array_equal(hu.bits(k), hu.bits(g[f"rope{hd}/k_out"]))
        dq, dk, dt = hu.dev(g[f"rope{hd}/q"]), hu.dev(g[f"rope{hd}/k"]), hu.dev(t)
        L.k_rope_apply(lh.ptr(dq), lh.ptr(dk), lh.ptr(dt), 8, 2, hd)
        assert np.array_equal(hu.bits(hu.host(dq)), hu.bits(g[f"rope{hd}/q_out"]))
        assert np.array_equal(hu.bits(hu.host(dk)), hu.bits(g[f"rope{hd}/k_out"]))
    # rows with padded strides: each row bitwise the oracle's single-row rotation with its own table
    rng = orc.Rng(orc.SEED + 505)
    rows, nh, nkv, hd = 5, 8, 2, 64
    qs, ks, ts = nh * hd + 16, nkv * hd + 8, 2 * hd + 4
    q, k, t = rng.normal(rows * qs, 0, 1).reshape(rows, qs), rng.normal(rows * ks, 0, 1).reshape(rows, ks), \
        rng.normal(rows * ts, 0, 1).reshape(rows, ts)
    dq, dk, dt = hu.dev(q), hu.dev(k), hu.dev(t)
    L.k_rope_apply_rows(lh.ptr(dq), qs, lh.ptr(dk), ks, lh.ptr(dt), ts, rows, nh, nkv, hd)
    gq, gk = hu.host(dq), hu.host(dk)
    for r in range(rows):
        wq, wk = orc.rope_apply(q[r, :nh * hd], k[r, :nkv * hd], t[r, :2 * hd], nh, nkv, hd)
        assert np.array_equal(hu.bits(gq[r, :nh * hd]), hu.bits(wq)) and np.array_equal(hu.bits(gk[r, :nkv * hd]), hu.bits(wk))
        assert np.array_equal(hu.bits(gq[r, nh * hd:]), hu.bits(q[r, nh * hd:]))  # row padding untouched
        assert np.array_equal(hu.bits(gk[r, nkv * hd:]), hu.bits(k[r, nkv * hd:]))


# ---- the K/V cache -----------------------------------------------------------------------------------------------------


@pytest.mark.parametrize("layout", ["rows", "head"])
def test_kv_store_both_layouts(layout):
    L = hu.lib()
    assert L.kernels_kv_layout_select(layout.encode()) == 1
    try:
        assert L.kernels_kv_layout_name() == layout.encode()
        nkv, hd, seq, pos0, count, ld = 4, 32, 50, 17, 6, 4 * 32 + 8
        ps, hb = ctypes.c_size_t(), ctypes.c_size_t()
        L.k_kv_strides(nkv, hd, seq, ctypes.byref(ps), ctypes.byref(hb))
        assert (ps.value, hb.value) == orc.kv_strides(nkv, hd, seq, layout == "head")
        rng = orc.Rng(orc.SEED + 606)
        cache0 = rng.normal(seq * nkv * hd, 0, 1)
        src = rng.normal(count * ld, 0, 1).reshape(count, ld)
        want = cache0.copy()
        orc.lib().orc_kv_store(orc.ptr(want), orc.ptr(src), ld, pos0, count, nkv, hd, ps.value, hb.value)
        dc, ds = hu.dev(cache0), hu.dev(src)
        L.k_kv_store(lh.ptr(dc), lh.ptr(ds), ld, pos0, count, nkv, hd, seq)
        assert np.array_equal(hu.bits(hu.host(dc)), hu.bits(want))
        hc = cache0.copy()  # host cache
        L.k_kv_store(lh.ptr(hc), lh.ptr(src), ld, pos0, count, nkv, hd, seq)
        assert np.array_equal(hu.bits(hc), hu.bits(want))
    finally:
        L.kernels_kv_layout_select(b"head")


# ---- attention ---------------------------------------------------------------------------------------------------------


def attention_f64(q, kc, vc, nh, nkv, hd, pos, ps, hb):
    """float64 decode attention and the magnitude sum_t w_t |v_t| per output."""
    kv_mul = nh // nkv
    q = q.astype(np.float64).reshape(nh, hd)
    out, mag = np.zeros((nh, hd)), np.zeros((nh, hd))
    t = np.arange(pos + 1)
    for h in range(nh):
        base = (h // kv_mul) * hb
        idx = base + t[:, None] * ps + np.arange(hd)[None, :]
        K, V = kc[idx].astype(np.float64), vc[idx].astype(np.float64)
        s = K @ q[h] / np.sqrt(hd)
        w = np.exp(s - s.max())
        w /= w.sum()
        out[h], mag[h] = w @ V, w @ np.abs(V)
    return out.reshape(-1), mag.reshape(-1)


def check_attention(got, q, kc, vc, nh, nkv, hd, seq, pos, ps, hb, what):
    ref, mag = attention_f64(q, kc, vc, nh, nkv, hd, pos, ps, hb)
    tol = 1e-5 * mag + 1e-6
    assert np.all(np.abs(got - ref) <= tol), (what, np.max(np.abs(got - ref) - tol))
    orc_out = orc.attention(q, kc, vc, nh, nkv, hd, seq, pos, ps, hb)
    assert np.all(np.abs(got - orc_out) <= 2 * tol), what


def test_attention_golden_cases_both_layouts():
    L = hu.lib()
    g = golden()
    for key in sorted({k.split("/")[0] for k in g.files if k.startswith("att") and not k.startswith("attbatch")}):
        nh, nkv, hd, seq, pos = (int(v) for v in key[3:].split("_"))
        q, kc, vc = g[f"{key}/q"], g[f"{key}/k"], g[f"{key}/v"]
        work = lh.AttentionWork()
        L.k_attention_init(ctypes.byref(work), nh, nkv, hd, seq)
        out = np.zeros(nh * hd, np.float32)
        L.k_attention(lh.ptr(out), lh.ptr(q), lh.ptr(kc), lh.ptr(vc), None, ctypes.byref(work), nh, nkv, hd, seq, pos)
        ps, hb = orc.kv_strides(nkv, hd, seq, False)
        check_attention(out, q, kc, vc, nh, nkv, hd, seq, pos, ps, hb, key)
        assert np.all(np.abs(out - g[f"{key}/out"]) <= 2e-5 * np.abs(vc).max() + 1e-6), key
        kh = np.ascontiguousarray(kc.reshape(seq, nkv, hd).transpose(1, 0, 2)).reshape(-1)
        vh = np.ascontiguousarray(vc.reshape(seq, nkv, hd).transpose(1, 0, 2)).reshape(-1)
        dq, dk, dv, do = hu.dev(q), hu.dev(kh), hu.dev(vh), hu.empty(nh * hd, hu.torch().float32)
        L.k_attention_kv(lh.ptr(do), lh.ptr(dq), lh.ptr(dk), lh.ptr(dv), None, ctypes.byref(work), nh, nkv, hd, seq,
                         pos)  # the default head-major layout
        ps, hb = orc.kv_strides(nkv, hd, seq, True)
        check_attention(hu.host(do), q, kh, vh, nh, nkv, hd, seq, pos, ps, hb, key + " head")
        L.k_attention_free(ctypes.byref(work))


@pytest.mark.parametrize("nh,nkv,hd,seq,positions", [(32, 8, 128, 600, (0, 63, 64, 65, 599)),
                                                     (8, 8, 64, 200, (1, 127, 199)), (12, 4, 96, 130, (129,)),
                                                     (16, 1, 256, 70, (69,)), (4, 2, 32, 40, (39,)),
                                                     (24, 8, 128, 300, (0, 127, 130, 299)),
                                                     (64, 8, 128, 150, (1, 64, 149)), (32, 8, 64, 200, (5, 127, 199)),
                                                     (16, 2, 64, 100, (63, 99)),
                                                     (8, 2, 64, 16500, (16383, 16384, 16499))])
def test_attention_decode_shapes(nh, nkv, hd, seq, positions):
    """Decode attention at chunk boundaries (63, 64, 65) and GQA ratios 1-16, head_dim 32-256, head-major layout.
    head_dim 64 or 128 with up to 8 query heads per KV head take the decode kernel (the 3B model's 3, the 1B and 8B
    models' 4, and 8); the others the general one. The last case reaches 16384 positions (258 chunks to merge)."""
    L = hu.lib()
    rng = orc.Rng(orc.SEED + nh * 31 + hd + seq)
    kc, vc = rng.normal(seq * nkv * hd, 0, 1), rng.normal(seq * nkv * hd, 0, 1)
    dk, dv = hu.dev(kc), hu.dev(vc)
    ps, hb = orc.kv_strides(nkv, hd, seq, True)
    for pos in positions:
        q = rng.normal(nh * hd, 0, 1)
        dq, do = hu.dev(q), hu.empty(nh * hd, hu.torch().float32)
        L.k_attention_layout(lh.ptr(do), lh.ptr(dq), lh.ptr(dk), lh.ptr(dv), None, None, nh, nkv, hd, seq, pos, ps, hb)
        check_attention(hu.host(do), q, kc, vc, nh, nkv, hd, seq, pos, ps, hb, f"pos {pos}")


@pytest.mark.parametrize("nh,nkv,hd,seq,pos0,m", [(8, 2, 64, 48, 20, 6), (32, 8, 128, 300, 0, 130),
                                                  (32, 8, 128, 300, 100, 64), (4, 2, 32, 2400, 2300, 40)])
def test_attention_batch_rows(nh, nkv, hd, seq, pos0, m):
    """k_attention_batch: row i attends to positions 0..pos0 + i, each row as the decode attention at its position; the
    reference's own batched output on the golden case. The last case: 40 rows past position 2300 (37 chunks)."""
    L = hu.lib()
    g = golden()
    rng = orc.Rng(orc.SEED + 700 + m)
    if (nh, nkv, hd, seq, pos0, m) == tuple(int(v) for v in g["attbatch/shape"]):
        kc, vc, q = g["attbatch/k"], g["attbatch/v"], g["attbatch/q"]
    else:
        kc, vc, q = rng.normal(seq * nkv * hd, 0, 1), rng.normal(seq * nkv * hd, 0, 1), rng.normal(m * nh * hd, 0, 1)
    dq, dk, dv, do = hu.dev(q), hu.dev(kc), hu.dev(vc), hu.empty(m * nh * hd, hu.torch().float32)
    L.k_attention_batch(lh.ptr(do), lh.ptr(dq), lh.ptr(dk), lh.ptr(dv), None, None, nh, nkv, hd, seq, pos0, m)
    got = hu.host(do).reshape(m, -1)
    ps, hb = orc.kv_strides(nkv, hd, seq, False)
    for i in range(m):
        check_attention(got[i], q.reshape(m, -1)[i], kc, vc, nh, nkv, hd, seq, pos0 + i, ps, hb, f"row {i}")
    if (nh, nkv, hd, seq, pos0, m) == tuple(int(v) for v in g["attbatch/shape"]):
        assert np.all(np.abs(got.reshape(-1) - g["attbatch/out"]) <= 2e-5 * np.abs(vc).max() + 1e-6)


@pytest.mark.parametrize("nh,nkv,hd,seq,pos0,m,layout", [
    (32, 8, 128, 2100, 0, 2048, "head"),   # the 8B prompt (rows sampled below)
    (16, 16, 64, 300, 7, 200, "rows"),     # kv_mul 1: 128-row tiles
    (16, 8, 128, 400, 130, 77, "head"),    # kv_mul 2, a ragged last tile
    (32, 4, 64, 260, 64, 96, "rows"),      # kv_mul 8: 16-row tiles, starting on a chunk boundary
    (64, 4, 128, 200, 33, 50, "head"),     # kv_mul 16: 8-row tiles
    (8, 2, 128, 1500, 1400, 16, "rows"),   # 16 rows, 23 chunks each
    (24, 8, 128, 2100, 0, 2048, "head"),   # the 3B prompt: kv_mul 3, 42-row tiles of 126 query vectors
    (12, 4, 64, 300, 21, 100, "rows"),     # kv_mul 3, a ragged last tile
    (20, 4, 64, 200, 0, 60, "head"),       # kv_mul 5: 25-row tiles, 3 vectors idle
    (48, 8, 128, 160, 3, 50, "rows"),      # kv_mul 6: 21-row tiles, 2 vectors idle
    (32, 8, 128, 600, 0, 512, "head"),     # a short 8B prompt: 64 blocks
    (24, 8, 128, 700, 40, 512, "rows"),    # the 3B heads from position 40
    (32, 8, 64, 300, 0, 130, "head"),      # 1B heads, 130 rows
    (32, 8, 128, 2100, 1792, 256, "head"), # a 256-row batch late in an 8B prompt: tiles split over 4 blocks each
    (32, 8, 128, 2100, 1984, 64, "rows"),  # 64 rows at 1984: 16 blocks per tile
    (24, 8, 128, 4100, 3968, 128, "head"), # 3B heads at 3968: 8 blocks per tile
    (32, 8, 64, 2100, 1792, 256, "rows"),  # 1B heads late: 4 blocks per tile
])
def test_attention_batch_flash_shapes(nh, nkv, hd, seq, pos0, m, layout, monkeypatch, splits=None):
    """Batches of at least 16 rows with 64 or 128 dimensions per head run the flash kernel (its products from exact
    BF16 parts on the BF16 matrix cores): every checked row within the float64 budget of the decode attention at its position and within twice it of the
    oracle, for GQA ratios 1-16 (those that do not divide 128 leave the tile's last vectors idle), both layouts, ragged
    tiles, short prompts and long contexts. A short batch late in a sequence splits each tile's positions over several
    blocks whose partials attn_merge combines (the last four cases, and the 16-row one)."""
    if splits:
        monkeypatch.setenv("LLAMA_HIP_FLASH_SPLITS", str(splits))
    L = hu.lib()
    rng = orc.Rng(orc.SEED + 900 + m + hd)
    kc, vc, q = rng.normal(seq * nkv * hd, 0, 1), rng.normal(seq * nkv * hd, 0, 1), rng.normal(m * nh * hd, 0, 1)
    ps, hb = orc.kv_strides(nkv, hd, seq, layout == "head")
    dq, dk, dv, do = hu.dev(q), hu.dev(kc), hu.dev(vc), hu.empty(m * nh * hd, hu.torch().float32)
    L.k_attention_batch_layout(lh.ptr(do), lh.ptr(dq), lh.ptr(dk), lh.ptr(dv), None, None, nh, nkv, hd, seq, pos0, m,
                               ps, hb)
    got = hu.host(do).reshape(m, -1)
    assert not lh.last_error()
    rows = range(m) if m <= 200 else sorted(r for r in {0, 1, 63, 64, 127, 128, 300, 1000, m - 2, m - 1} if r < m)
    for i in rows:
        check_attention(got[i], q.reshape(m, -1)[i], kc, vc, nh, nkv, hd, seq, pos0 + i, ps, hb, f"row {i}")


@pytest.mark.parametrize("shape", [(16, 8, 128, 400, 130, 77, "head"), (32, 4, 64, 260, 64, 96, "rows"),
                                   (24, 8, 128, 2100, 0, 2048, "head"), (32, 8, 128, 2100, 1792, 256, "head")])
def test_attention_flash_fp32_form(shape, monkeypatch):
    """LLAMA_HIP_FLASH_FORM=fp32 keeps the flash kernel whose products run on the FP32 matrix cores (attn_flash; the
    default forms them from exact BF16 parts, attn_flash3): ragged tiles, 64 dimensions, the 3B prompt, a split late
    batch, each row within the float64 budget."""
    monkeypatch.setenv("LLAMA_HIP_FLASH_FORM", "fp32")
    test_attention_batch_flash_shapes(*shape, monkeypatch)


@pytest.mark.parametrize("nh,nkv,hd,seq,pos0,m,gs,layout,form", [
    (32, 8, 128, 600, 0, 512, 64, "head", None),      # 8B heads: quantized in the flash kernel's epilogue
    (24, 8, 128, 300, 10, 100, 32, "rows", None),     # kv_mul 3 (idle vectors), groups of 32
    (32, 8, 64, 300, 0, 130, 64, "head", None),       # 64 dimensions, a group per head
    (16, 4, 128, 200, 3, 40, 128, "head", None),      # a group of a whole head
    (32, 8, 128, 2100, 1792, 256, 64, "head", None),  # a late batch split over blocks: merged, then quantized
    (8, 2, 128, 200, 50, 8, 64, "rows", None),        # 8 rows: the tile kernels, then quantized
    (32, 8, 128, 600, 0, 200, 16, "head", "fp32"),    # the FP32-product kernel, then quantized
])
def test_attention_batch_quantize_fused(nh, nkv, hd, seq, pos0, m, gs, layout, form, monkeypatch):
    """llhip_attention_batch_quantize: bitwise k_attention_batch_kv then k_quantize_rows of its rows, whether the
    flash kernel quantizes in its epilogue or the rows are quantized after it."""
    if form:
        monkeypatch.setenv("LLAMA_HIP_FLASH_FORM", form)
    L = hu.lib()
    assert L.kernels_kv_layout_select(layout.encode()) == 1
    try:
        T = hu.torch()
        rng = orc.Rng(orc.SEED + 950 + m + hd + gs)
        kc, vc, q = rng.normal(seq * nkv * hd, 0, 1), rng.normal(seq * nkv * hd, 0, 1), rng.normal(m * nh * hd, 0, 1)
        dq, dk, dv = hu.dev(q), hu.dev(kc), hu.dev(vc)
        n = nh * hd
        out, out2 = hu.empty(m * n, T.float32), hu.empty(m * n, T.float32)
        xq, xq2 = hu.empty(m * n, T.int8), hu.empty(m * n, T.int8)
        xs, xs2 = hu.empty(m * n // gs, T.float32), hu.empty(m * n // gs, T.float32)
        L.llhip_attention_batch_quantize(lh.ptr(xq), lh.ptr(xs), gs, lh.ptr(out), lh.ptr(dq), lh.ptr(dk), lh.ptr(dv), nh,
                                         nkv, hd, seq, pos0, m)
        L.k_attention_batch_kv(lh.ptr(out2), lh.ptr(dq), lh.ptr(dk), lh.ptr(dv), None, None, nh, nkv, hd, seq, pos0, m)
        L.k_quantize_rows(lh.ptr(xq2), lh.ptr(xs2), lh.ptr(out2), n, m, n, gs)
        assert not lh.last_error()
        assert np.array_equal(hu.host(xq), hu.host(xq2))
        assert np.array_equal(hu.bits(hu.host(xs)), hu.bits(hu.host(xs2)))
    finally:
        assert L.kernels_kv_layout_select(b"head") == 1


@pytest.mark.parametrize("splits,shape", [(3, (16, 8, 128, 400, 130, 77, "head")), (16, (32, 8, 128, 600, 0, 512, "head")),
                                          (5, (12, 4, 64, 300, 21, 100, "rows")), (2, (24, 8, 128, 2100, 0, 2048, "head"))])
def test_attention_flash_forced_splits(splits, shape, monkeypatch):
    """LLAMA_HIP_FLASH_SPLITS forces the blocks per tile: shares that hold no chunk (3 shares of a 4-chunk tile), more
    shares than a tile's chunks, an odd count and the whole 3B prompt, each row within the float64 budget."""
    test_attention_batch_flash_shapes(*shape, monkeypatch, splits=splits)


def test_attention_flash_nonfinite_score_fails():
    L = hu.lib()
    lh.record_failures()
    try:
        nh, nkv, hd, seq, m = 8, 2, 64, 40, 20
        rng = orc.Rng(orc.SEED + 909)
        kc, vc, q = rng.normal(seq * nkv * hd, 0, 1), rng.normal(seq * nkv * hd, 0, 1), rng.normal(m * nh * hd, 0, 1)
        kc[15 * nkv * hd + 70] = np.inf  # position 15, KV head 1
        dq, dk, dv, do = hu.dev(q), hu.dev(kc), hu.dev(vc), hu.empty(m * nh * hd, hu.torch().float32)
        L.k_attention_batch(lh.ptr(do), lh.ptr(dq), lh.ptr(dk), lh.ptr(dv), None, None, nh, nkv, hd, seq, 10, m)
        L.llhip_synchronize()
        assert "nonfinite value in softmax" in lh.last_error()
        L.llhip_clear_error()
        L.k_attention_batch(lh.ptr(do), lh.ptr(dq), lh.ptr(dk), lh.ptr(dv), None, None, nh, nkv, hd, seq, 0, 15)
        L.llhip_synchronize()  # rows 0..14 stop before position 15: the split kernel (15 rows), no failure
        assert lh.last_error() == ""
        L.k_attention_batch(lh.ptr(do), lh.ptr(dq), lh.ptr(dk), lh.ptr(dv), None, None, nh, nkv, hd, seq, 0, 16)
        L.llhip_synchronize()  # row 15 reaches it: the flash kernel's failure
        assert "nonfinite value in softmax" in lh.last_error()
    finally:
        L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
        L.llhip_clear_error()


def test_attention_nonfinite_score_fails_and_bookkeeping():
    L = hu.lib()
    lh.record_failures()
    try:
        nh, nkv, hd, seq = 4, 2, 16, 10
        rng = orc.Rng(orc.SEED + 808)
        kc, vc, q = rng.normal(seq * nkv * hd, 0, 1), rng.normal(seq * nkv * hd, 0, 1), rng.normal(nh * hd, 0, 1)
        kc[5 * nkv * hd + 3] = np.inf
        out = np.zeros(nh * hd, np.float32)
        L.k_attention(lh.ptr(out), lh.ptr(q), lh.ptr(kc), lh.ptr(vc), None, None, nh, nkv, hd, seq, seq - 1)
        assert "nonfinite value in softmax" in lh.last_error()
        L.llhip_clear_error()
        L.k_attention(lh.ptr(out), lh.ptr(q), lh.ptr(kc), lh.ptr(vc), None, None, nh, nkv, hd, seq, 4)  # before it
        assert lh.last_error() == ""
        L.k_attention(lh.ptr(out), lh.ptr(q), lh.ptr(kc), lh.ptr(vc), None, None, nh, nkv, hd, seq, seq)
        assert "outside the cache" in lh.last_error()
        L.llhip_clear_error()
        L.k_attention(lh.ptr(out), lh.ptr(q), lh.ptr(kc), lh.ptr(vc), None, None, 6, 4, hd, seq, 3)
        assert "not supported" in lh.last_error()
        L.llhip_clear_error()
    finally:
        L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
        L.llhip_clear_error()
    work = lh.AttentionWork()
    L.k_attention_init(ctypes.byref(work), 32, 8, 128, 8192)
    assert work.max_chunks == 128 and work.n_heads == 32 and work.head_dim == 128 and not work.partial
    assert L.k_attention_chunk_count(ctypes.byref(work), 8, 63) == 1 and L.k_attention_chunk_count(None, 8, 64) == 2
    assert L.k_attention_bytes(32, 8, 128, 8192) == 32 * 128 * 132 * 4  # 130 floats per chunk, rounded to 4
    L.k_attention_free(ctypes.byref(work))
    assert L.kernels_attention_select(b"tiled", b"group") == 1 and L.kernels_attention_select(b"x", None) == 0


# ---- embedding rows ------------------------------------------------------------------------------------------------


def test_embed_q8_rows_bitwise_host_device_and_bad_id():
    """Embedding lookup of a Q8_0 table (src/tp.c:395-396, 444-456): each value is the int8 converted exactly times its
    group's scale, one float product, so the row is bitwise numpy's float32 product. Groups straddle rows (dim 96,
    gs 64). Host operands and device operands (ids read on the device) give the same bits."""
    L = hu.lib()
    rng = np.random.default_rng(orc.SEED + 909)
    vocab, dim, gs = 778, 96, 64
    table = rng.integers(-127, 128, vocab * dim, dtype=np.int8)
    scales = rng.uniform(1e-4, 2e-2, vocab * dim // gs).astype(np.float32)
    ids = np.array([0, 777, 5, 5, 400, 1], np.int32)
    flat = ids[:, None].astype(np.int64) * dim + np.arange(dim)
    want = table[flat].astype(np.float32) * scales[flat // gs]
    out = np.full((len(ids), dim), np.nan, np.float32)
    L.k_embed_q8_rows(lh.ptr(out), lh.ptr(table), lh.ptr(scales), lh.ptr(ids), len(ids), dim, gs, vocab)
    assert np.array_equal(out.view(np.int32), want.view(np.int32))
    dt, ds, di = hu.dev(table), hu.dev(scales), hu.dev(ids)
    do = hu.empty(len(ids) * dim, hu.torch().float32)
    L.k_embed_q8_rows(lh.ptr(do), lh.ptr(dt), lh.ptr(ds), lh.ptr(di), len(ids), dim, gs, vocab)
    assert np.array_equal(hu.host(do).reshape(len(ids), dim).view(np.int32), want.view(np.int32))
    lh.record_failures()
    try:
        bad = np.array([3, vocab], np.int32)
        L.k_embed_q8_rows(lh.ptr(out), lh.ptr(table), lh.ptr(scales), lh.ptr(bad), 2, dim, gs, vocab)
        assert "embedding row id outside the table" in lh.last_error()
        L.llhip_clear_error()
        L.k_embed_q8_rows(lh.ptr(out), lh.ptr(table), lh.ptr(scales), lh.ptr(ids), 1, dim, 7, vocab)
        assert "groups of 7" in lh.last_error()
        L.llhip_clear_error()
    finally:
        L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
        L.llhip_clear_error()


# ---- RMSNorm recorded into the next GEMV's prologue -----------------------------------------------------------------


def synth_q8(rng, d, n, gs=64):
    return orc.quantize_weights(rng.normal(d * n, 0.0, 0.02).reshape(d, n), gs)


@pytest.mark.parametrize("kind", ["store", "swiglu", "qkv", "add_residual"])
def test_rmsnorm_quantize_gemv_fusion(kind):
    """k_rmsnorm -> k_quantize -> Q8 GEMV on device memory, the reference's decode order (tp.c:399-401, 419-420): the
    GEMV normalizes and quantizes in its prologue. The normalized row matches the oracle's within 1e-5, the quantized
    row is bitwise the quantization of that normalized row, and the GEMV output is within the budget of its float64
    reference. add_residual adds into the norm's own input, which the fused kernel must not do (it falls back to
    separate launches): the same checks hold."""
    L = hu.lib()
    rng = orc.Rng(orc.SEED + 1200 + len(kind))
    n, d, gs = 4096, 1024, 64
    x = rng.normal(n, 0.0, 2.0)
    w = rng.normal(n, 1.0, 0.1)
    wq, ws = synth_q8(rng, d, n)
    w3q, w3s = synth_q8(rng, d, n)
    base = rng.normal(n, 0.0, 1.0) if kind == "add_residual" else None
    dx = hu.dev(x if base is None else x)
    dw, dxb = hu.dev(w), hu.empty(n, hu.torch().float32)
    dxq, dxs = hu.empty(n, hu.torch().int8), hu.empty(n // gs, hu.torch().float32)
    dwq, dws, dw3q, dw3s = hu.dev(wq), hu.dev(ws), hu.dev(w3q), hu.dev(w3s)
    inp = lh.k8(dxq, dxs)
    outs = [hu.empty(d if kind != "add_residual" else n, hu.torch().float32) for _ in range(3)]
    L.k_rmsnorm(lh.ptr(dxb), lh.ptr(dx), lh.ptr(dw), n, 1e-5)
    L.k_quantize(lh.ptr(dxq), lh.ptr(dxs), lh.ptr(dxb), n, gs)
    if kind == "store":
        L.k_matmul_q8(lh.ptr(outs[0]), inp, lh.w8(dwq, dws), n, d, gs)
    elif kind == "swiglu":
        L.k_matmul_q8_swiglu(lh.ptr(outs[0]), inp, lh.w8(dwq, dws), lh.w8(dw3q, dw3s), n, d, gs)
    elif kind == "qkv":
        L.k_matmul_q8_qkv(lh.ptr(outs[0]), lh.ptr(outs[1]), lh.ptr(outs[2]), inp, lh.w8(dwq, dws), lh.w8(dw3q, dw3s),
                          lh.w8(dwq, dws), n, d, d, gs)
    else:  # x += W x_normed with a square W: the output is the norm's input
        wsq, wss = synth_q8(rng, n, n)
        dwsq, dwss = hu.dev(wsq), hu.dev(wss)
        L.k_matmul_q8_add(lh.ptr(dx), inp, lh.w8(dwsq, dwss), n, n, gs)
    xb = hu.host(dxb)
    want_xb = orc.rmsnorm(x, w)
    assert np.all(np.abs(xb - want_xb) <= 1e-5 * np.abs(want_xb) + 1e-7)
    xq, xs = hu.host(dxq), hu.host(dxs)
    q2, s2 = orc.quantize(xb, gs)
    assert np.array_equal(xq, q2) and np.array_equal(hu.bits(xs), hu.bits(s2))
    if kind == "add_residual":
        ref, mag = hu.dequant_reference(xq, xs, wsq, wss, gs)
        hu.assert_within_budget(hu.host(dx), x + ref, mag + np.abs(x), what="residual add")
        return
    ref, mag = hu.dequant_reference(xq, xs, wq, ws, gs)
    got = hu.host(outs[0])
    if kind == "swiglu":
        ref3, mag3 = hu.dequant_reference(xq, xs, w3q, w3s, gs)
        ta, tb = 2e-5 * mag + 1e-6, 2e-5 * mag3 + 1e-6
        silu = ref / (1.0 + np.exp(-ref))
        tol = 1.1 * np.abs(ref3) * ta + np.abs(silu) * tb + 1.1 * ta * tb + 1e-6
        assert np.all(np.abs(got - silu * ref3) <= tol)
    else:
        hu.assert_within_budget(got, ref, mag, what=kind)
    if kind == "qkv":
        ref3, mag3 = hu.dequant_reference(xq, xs, w3q, w3s, gs)
        hu.assert_within_budget(hu.host(outs[1]), ref3, mag3, what="k")
        hu.assert_within_budget(hu.host(outs[2]), ref, mag, what="v")


def test_recorded_rmsnorm_runs_before_any_other_call():
    """A recorded k_rmsnorm whose output is read by something other than a k_quantize -> GEMV pair still runs first:
    before a RoPE call on its output, before a quantization of another buffer, and at a synchronization."""
    L = hu.lib()
    rng = orc.Rng(orc.SEED + 1300)
    n = 256
    x, w = rng.normal(n, 0.0, 1.0), rng.normal(n, 1.0, 0.1)
    want = orc.rmsnorm(x, w)
    dx, dw, dxb = hu.dev(x), hu.dev(w), hu.empty(n, hu.torch().float32)
    table = np.zeros(2 * 64, np.float32)
    table[:64] = 1.0  # cos 1, sin 0: the identity rotation
    dt = hu.dev(table)
    L.k_rmsnorm(lh.ptr(dxb), lh.ptr(dx), lh.ptr(dw), n, 1e-5)
    L.k_rope_apply(lh.ptr(dxb), None, lh.ptr(dt), n // 64, 0, 64)  # reads and rewrites the normalized row
    got = hu.host(dxb)
    assert np.all(np.abs(got - want) <= 1e-5 * np.abs(want) + 1e-7)
    other = hu.dev(rng.normal(n, 0.0, 1.0))
    dxq, dxs = hu.empty(n, hu.torch().int8), hu.empty(n // 64, hu.torch().float32)
    dxb.zero_()
    hu.torch().cuda.synchronize()
    L.k_rmsnorm(lh.ptr(dxb), lh.ptr(dx), lh.ptr(dw), n, 1e-5)
    L.k_quantize(lh.ptr(dxq), lh.ptr(dxs), lh.ptr(other), n, 64)  # not the norm's output: the norm runs on its own
    got = hu.host(dxb)
    assert np.all(np.abs(got - want) <= 1e-5 * np.abs(want) + 1e-7)
    q2, s2 = orc.quantize(hu.host(other), 64)
    assert np.array_equal(hu.host(dxq), q2)


@pytest.mark.parametrize("rows,nh,nkv,hd,seq,pos0,layout", [(5, 32, 8, 128, 64, 3, "head"), (37, 8, 2, 64, 100, 60, "head"),
                                                             (3, 4, 4, 32, 10, 7, "rows"), (130, 24, 8, 128, 300, 0, "head")])
def test_rope_kv_store_rows_fused(rows, nh, nkv, hd, seq, pos0, layout):
    """llhip_rope_kv_store_rows: bitwise k_rope_apply_rows of q and k then k_kv_store of k and v (the caches, q and the
    rotated k), in either cache layout."""
    L = hu.lib()
    assert L.kernels_kv_layout_select(layout.encode()) == 1
    try:
        rng = orc.Rng(orc.SEED + 4100 + rows + nh + hd + pos0)
        d, kvl = nh * hd, nkv * hd
        q, k, v = (rng.normal(rows * n, 0, 1).reshape(rows, n) for n in (d, kvl, kvl))
        table = rng.uniform(rows * 2 * hd, 1.0).reshape(rows, 2 * hd)
        kc0, vc0 = rng.normal(seq * kvl, 0, 1), rng.normal(seq * kvl, 0, 1)
        out = []
        for fused in (True, False):
            dq, dk, dv, dt = hu.dev(q), hu.dev(k), hu.dev(v), hu.dev(table)
            dkc, dvc = hu.dev(kc0), hu.dev(vc0)
            if fused:
                L.llhip_rope_kv_store_rows(lh.ptr(dq), d, lh.ptr(dk), lh.ptr(dv), kvl, lh.ptr(dt), 2 * hd, rows, nh, nkv,
                                           hd, lh.ptr(dkc), lh.ptr(dvc), pos0, seq)
            else:
                L.k_rope_apply_rows(lh.ptr(dq), d, lh.ptr(dk), kvl, lh.ptr(dt), 2 * hd, rows, nh, nkv, hd)
                L.k_kv_store(lh.ptr(dkc), lh.ptr(dk), kvl, pos0, rows, nkv, hd, seq)
                L.k_kv_store(lh.ptr(dvc), lh.ptr(dv), kvl, pos0, rows, nkv, hd, seq)
            assert lh.last_error() == "", lh.last_error()
            out.append([hu.bits(hu.host(a)) for a in (dq, dk, dkc, dvc)])
        for what, a, b in zip(("q", "k", "key cache", "value cache"), *out):
            assert np.array_equal(a, b), what
        wq, wk = orc.rope_apply(q[0], k[0], table[0], nh, nkv, hd)  # the oracle on the first row
        assert np.array_equal(out[0][0][0], hu.bits(wq)) and np.array_equal(out[0][1][0], hu.bits(wk))
    finally:
        L.kernels_kv_layout_select(b"head")


# ---- RoPE and the cache stores recorded into the decode attention ----------------------------------------------------


@pytest.mark.parametrize("layout,interrupt,shape", [("head", None, (32, 8, 128, 200, 130)),
                                                    ("rows", None, (32, 8, 128, 200, 130)),
                                                    ("head", "sync", (32, 8, 128, 200, 130)),
                                                    ("head", "position", (32, 8, 128, 200, 130)),
                                                    ("head", None, (24, 8, 128, 300, 127)),
                                                    ("head", None, (32, 8, 64, 200, 128)),
                                                    ("rows", None, (64, 8, 128, 150, 63))])
def test_rope_kv_store_attention_fusion(layout, interrupt, shape):
    """The reference's decode order (tp.c:409-413): k_rope_apply(q, k), k_kv_store of k and of v at the position,
    k_attention_kv at that position. Device-resident, the three recorded calls run inside the attention launch: q and k
    come back rotated bitwise as the oracle rotates them, the cache rows hold the rotated k and v bitwise, and the
    output is within the attention tolerance of the oracle on the updated cache. A synchronization in between, or an
    attention at another position, runs the recorded calls on their own first: the same results."""
    L = hu.lib()
    assert L.kernels_kv_layout_select(layout.encode()) == 1
    try:
        rng = orc.Rng(orc.SEED + 1400 + len(layout) + (0 if interrupt is None else len(interrupt)) + sum(shape))
        nh, nkv, hd, seq, pos = shape
        kv_dim = nkv * hd
        ps, hb = orc.kv_strides(nkv, hd, seq, layout == "head")
        kc0, vc0 = rng.normal(seq * kv_dim, 0, 1), rng.normal(seq * kv_dim, 0, 1)
        q, k, v = rng.normal(nh * hd, 0, 1), rng.normal(kv_dim, 0, 1), rng.normal(kv_dim, 0, 1)
        g = golden()
        # the reference's table row for 128 dimensions; any 2 * hd values otherwise (the rotation only reads them)
        table = g["ropetab128_1000/table"] if hd == 128 else rng.uniform(2 * hd, 1.0).astype(np.float32)
        dq, dk, dv, dt = hu.dev(q), hu.dev(k), hu.dev(v), hu.dev(table)
        dkc, dvc, do = hu.dev(kc0), hu.dev(vc0), hu.empty(nh * hd, hu.torch().float32)
        L.k_rope_apply(lh.ptr(dq), lh.ptr(dk), lh.ptr(dt), nh, nkv, hd)
        L.k_kv_store(lh.ptr(dkc), lh.ptr(dk), kv_dim, pos, 1, nkv, hd, seq)
        if interrupt == "sync":
            L.llhip_synchronize()
        L.k_kv_store(lh.ptr(dvc), lh.ptr(dv), kv_dim, pos, 1, nkv, hd, seq)
        apos = pos if interrupt != "position" else pos + 1
        L.k_attention_kv(lh.ptr(do), lh.ptr(dq), lh.ptr(dkc), lh.ptr(dvc), None, None, nh, nkv, hd, seq, apos)
        wq, wk = orc.rope_apply(q, k, table, nh, nkv, hd)
        kc, vc = kc0.copy(), vc0.copy()
        orc.lib().orc_kv_store(orc.ptr(kc), orc.ptr(wk), kv_dim, pos, 1, nkv, hd, ps, hb)
        orc.lib().orc_kv_store(orc.ptr(vc), orc.ptr(v), kv_dim, pos, 1, nkv, hd, ps, hb)
        assert np.array_equal(hu.bits(hu.host(dq)), hu.bits(wq)) and np.array_equal(hu.bits(hu.host(dk)), hu.bits(wk))
        assert np.array_equal(hu.bits(hu.host(dkc)), hu.bits(kc)) and np.array_equal(hu.bits(hu.host(dvc)), hu.bits(vc))
        check_attention(hu.host(do), wq, kc, vc, nh, nkv, hd, seq, apos, ps, hb, f"{layout} {interrupt}")
    finally:
        L.kernels_kv_layout_select(b"head")
