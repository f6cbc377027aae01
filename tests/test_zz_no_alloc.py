"""k_attention_batch_layout_noalloc, the attention entry point that allocates nothing (its split-K partials live in a
fixed per-device array): equal bit for bit to k_attention_batch_layout on calls in a row, each smaller than the one
before (a 16-row batch at position 1000 on the flash kernel, its positions split over 16 blocks per tile, then 8 rows
and one decode row on the split kernels, each writing and reading the array); no HBM claimed by the calls; replayable
from a HIP graph captured around it; a 2048-row batch, which needs no partials, accepted; host buffers, a split call
too large for the array and an uninitialized library refused with a message."""
import os
import subprocess
import sys

import numpy as np
import pytest

import llama_hip as lh
from tests import hip_util as hu

pytestmark = pytest.mark.gpu

NH, NKV, HD, SEQ = 32, 8, 128, 4096  # Llama-3.1-8B heads
SCRATCH_FLOATS = 4 << 20


def head_major(rng, seq):
    """Random K and V caches in the head-major layout ([kv_head][position][head_dim]) and their strides."""
    k = rng.standard_normal((NKV, seq, HD), dtype=np.float32)
    v = rng.standard_normal((NKV, seq, HD), dtype=np.float32)
    return k, v, HD, seq * HD


def run(L, name, out, q, k, v, pos0, m, ps, hb, seq=SEQ):
    getattr(L, name)(lh.ptr(out), lh.ptr(q), lh.ptr(k), lh.ptr(v), None, None, NH, NKV, HD, seq, pos0, m, ps, hb)


def test_noalloc_attention_equals_the_workspace_form():
    L = hu.lib()
    T = hu.torch()
    assert L.llhip_init() == 0, lh.last_error()
    rng = np.random.default_rng(31)
    k, v, ps, hb = head_major(rng, SEQ)
    kd, vd = hu.dev(k), hu.dev(v)
    # 16 rows (attn_flash split + attn_merge_shares), 8 rows (attn_tile + attn_merge), a decode row
    cases = [(1000, 16), (1000, 8), (300, 1)]
    for pos0, m in cases:
        assert m * NH * ((pos0 + m - 1) // 64 + 1) * 132 <= SCRATCH_FLOATS
    outs = []
    claimed = L.llhip_hbm_claimed()
    for pos0, m in cases:
        q = hu.dev(rng.standard_normal((m, NH * HD), dtype=np.float32))
        out = hu.empty((m, NH * HD), T.float32)
        run(L, "k_attention_batch_layout_noalloc", out, q, kd, vd, pos0, m, ps, hb)
        L.llhip_synchronize()
        assert not lh.last_error()
        outs.append((q, hu.host(out)))
    assert L.llhip_hbm_claimed() == claimed  # nothing allocated through the library
    for (pos0, m), (q, got) in zip(cases, outs):
        want = hu.empty((m, NH * HD), T.float32)
        run(L, "k_attention_batch_layout", want, q, kd, vd, pos0, m, ps, hb)
        assert np.array_equal(got, hu.host(want)), (pos0, m)
        assert np.isfinite(got).all()


def test_noalloc_attention_replays_from_a_graph():
    """Captured once, replayed three times with eager work and synchronizations in between; every replay equals the
    eager result."""
    L = hu.lib()
    T = hu.torch()
    assert L.llhip_init() == 0, lh.last_error()
    rng = np.random.default_rng(32)
    k, v, ps, hb = head_major(rng, 2048)
    kd, vd = hu.dev(k), hu.dev(v)
    q = hu.dev(rng.standard_normal((1, NH * HD), dtype=np.float32))
    eager = hu.empty((1, NH * HD), T.float32)
    run(L, "k_attention_batch_layout_noalloc", eager, q, kd, vd, 2047, 1, ps, hb, seq=2048)
    L.llhip_synchronize()
    want = hu.host(eager)
    out = hu.empty((1, NH * HD), T.float32)
    assert L.llhip_graph_begin() == 0, lh.last_error()
    run(L, "k_attention_batch_layout_noalloc", out, q, kd, vd, 2047, 1, ps, hb, seq=2048)
    graph = L.llhip_graph_end()
    assert graph, lh.last_error()
    try:
        for i in range(3):
            out.zero_()
            T.cuda.synchronize()
            other = hu.empty((4, NH * HD), T.float32)  # eager work on the same array between replays
            q4 = hu.dev(rng.standard_normal((4, NH * HD), dtype=np.float32))
            run(L, "k_attention_batch_layout_noalloc", other, q4, kd, vd, 100, 4, ps, hb, seq=2048)
            L.llhip_synchronize()
            ref4 = hu.empty((4, NH * HD), T.float32)
            run(L, "k_attention_batch_layout", ref4, q4, kd, vd, 100, 4, ps, hb, seq=2048)
            assert np.array_equal(hu.host(other), hu.host(ref4)), i
            assert L.llhip_graph_launch(graph) == 0, lh.last_error()
            L.llhip_synchronize()
            assert np.array_equal(hu.host(out), want), i
    finally:
        L.llhip_graph_destroy(graph)


def test_noalloc_flash_split_narrowed_to_the_array():
    """256 rows at position 1792 (8B heads): the workspace form splits each tile's positions over 4 blocks, whose
    partials (256 x 32 x 4 x 132 floats) would overflow the 4 Mi array, so the allocation-free form splits them over 3;
    the two agree to FP32 summation order, and both to the float64 attention of sampled rows."""
    L = hu.lib()
    T = hu.torch()
    assert L.llhip_init() == 0, lh.last_error()
    rng = np.random.default_rng(33)
    seq, pos0, m = 2048, 1792, 256
    assert m * NH * 4 * 132 > SCRATCH_FLOATS >= m * NH * 3 * 132
    k, v, ps, hb = head_major(rng, seq)
    kd, vd = hu.dev(k), hu.dev(v)
    qh = rng.standard_normal((m, NH * HD), dtype=np.float32)
    q = hu.dev(qh)
    got, want = hu.empty((m, NH * HD), T.float32), hu.empty((m, NH * HD), T.float32)
    claimed = L.llhip_hbm_claimed()
    run(L, "k_attention_batch_layout_noalloc", got, q, kd, vd, pos0, m, ps, hb, seq=seq)
    L.llhip_synchronize()
    assert not lh.last_error() and L.llhip_hbm_claimed() == claimed
    run(L, "k_attention_batch_layout", want, q, kd, vd, pos0, m, ps, hb, seq=seq)
    g, w = hu.host(got), hu.host(want)
    assert np.all(np.abs(g - w) <= 1e-5 * np.abs(w).max() + 1e-6)
    kv_mul = NH // NKV
    for r in (0, 101, m - 1):  # the float64 attention of row r: query head h reads KV head h // kv_mul
        for h in (0, 13, NH - 1):
            kk = k[h // kv_mul, :pos0 + r + 1].astype(np.float64)
            vv = v[h // kv_mul, :pos0 + r + 1].astype(np.float64)
            s = kk @ qh[r, h * HD:(h + 1) * HD].astype(np.float64) / np.sqrt(HD)
            p = np.exp(s - s.max())
            ref = (p / p.sum()) @ vv
            assert np.all(np.abs(g[r, h * HD:(h + 1) * HD] - ref) <= 1e-5 * np.abs(vv).max() + 1e-6), (r, h)


def test_noalloc_attention_refusals():
    L = hu.lib()
    T = hu.torch()
    assert L.llhip_init() == 0, lh.last_error()
    rng = np.random.default_rng(33)
    k, v, ps, hb = head_major(rng, 256)
    kd, vd = hu.dev(k), hu.dev(v)
    lh.record_failures()
    try:
        # a 2048-row batch runs the flash kernel, which keeps no partials: accepted, and equal to the workspace form
        big = 2048
        kb, vb, bps, bhb = head_major(rng, big)
        kb, vb = hu.dev(kb), hu.dev(vb)
        q = hu.dev(rng.standard_normal((big, NH * HD), dtype=np.float32))
        out, want = hu.empty((big, NH * HD), T.float32), hu.empty((big, NH * HD), T.float32)
        run(L, "k_attention_batch_layout_noalloc", out, q, kb, vb, 0, big, bps, bhb, seq=big)
        assert lh.last_error() == "", lh.last_error()
        run(L, "k_attention_batch_layout", want, q, kb, vb, 0, big, bps, bhb, seq=big)
        assert np.array_equal(hu.host(out), hu.host(want))
        # 8 rows at position 16384 take the split kernels: 8 * 32 * 257 chunks * 132 floats exceed the array
        far, m8 = 16392, 8
        q8 = hu.empty((m8, NH * HD), T.float32)
        out8 = hu.empty((m8, NH * HD), T.float32)
        kf, vf = hu.empty((NKV, far, HD), T.float32), hu.empty((NKV, far, HD), T.float32)
        run(L, "k_attention_batch_layout_noalloc", out8, q8, kf, vf, far - m8, m8, HD, far * HD, seq=far)
        assert "floats of scratch; it holds 4194304" in lh.last_error(), lh.last_error()
        L.llhip_clear_error()
        qh = rng.standard_normal((1, NH * HD), dtype=np.float32)  # host memory: staging would allocate
        outh = np.zeros((1, NH * HD), np.float32)
        run(L, "k_attention_batch_layout_noalloc", outh, qh, kd, vd, 10, 1, ps, hb, seq=256)
        assert "every buffer must be device memory" in lh.last_error(), lh.last_error()
        assert not outh.any()
    finally:
        L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
        L.llhip_clear_error()


def test_noalloc_attention_needs_an_initialized_library():
    """In a process whose library has not opened the device (torch has), the call refuses rather than open it."""
    code = """
import sys
sys.path.insert(0, {pkg!r})
import torch
import llama_hip as lh
L = lh.load()
lh.record_failures()
b = torch.zeros(8 * 64 * 128, device="cuda")
torch.cuda.synchronize()
p = b.data_ptr()
L.k_attention_batch_layout_noalloc(p, p, p, p, None, None, 8, 8, 128, 64, 0, 1, 128, 64 * 128)
print(lh.last_error())
""".format(pkg=os.path.dirname(lh.LIB_PATH))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "the library is not initialized on this device" in r.stdout, r.stdout
