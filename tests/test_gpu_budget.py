"""The HBM budget on the device (src/loader.c:28-56): the default is the device's memory, allocations the library
hands out are claimed and given back, and one beyond LLAMA_HBM_BUDGET_GIB fails with the reference's message."""
import numpy as np
import pytest

import llama_hip as lh
from tests import hip_util as hu

pytestmark = pytest.mark.gpu


def test_budget_claims_and_the_reference_failure(monkeypatch):
    L = hu.lib()
    assert L.llhip_init() == 0, lh.last_error()
    monkeypatch.delenv("LLAMA_HBM_BUDGET_GIB", raising=False)
    assert L.placement_hbm_budget() == hu.torch().cuda.get_device_properties(0).total_memory
    base = L.llhip_hbm_claimed()
    assert base >= 512 * 128 * 1024  # the split-K workspace is claimed when the device opens
    p = L.llhip_malloc(1 << 20)
    assert p and L.llhip_hbm_claimed() == base + (1 << 20)
    host = np.zeros(1 << 20, np.float32)
    assert L.llhip_register_host(lh.ptr(host), host.nbytes) == 0
    assert L.llhip_hbm_claimed() == base + (1 << 20) + host.nbytes
    assert L.llhip_unregister_host(lh.ptr(host)) == 0
    L.llhip_free(p)
    assert L.llhip_hbm_claimed() == base
    monkeypatch.setenv("LLAMA_HBM_BUDGET_GIB", f"{(base + (1 << 19)) / 2 ** 30:.12f}")
    lh.record_failures()
    try:
        assert not L.llhip_malloc(1 << 20)
        msg = lh.last_error()
        assert msg.startswith("llhip_malloc need 1048576 bytes of HBM but LLAMA_HBM_BUDGET_GIB leaves "), msg
        L.llhip_clear_error()
        q = L.llhip_malloc(1 << 18)  # within what is left
        assert q and lh.last_error() == ""
        L.llhip_free(q)
        assert L.llhip_hbm_claimed() == base
    finally:
        L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
        L.llhip_clear_error()


def test_failed_batch_allocation_leaves_nothing_claimed(tmp_path, monkeypatch):
    """engine_forward_batch allocates its rows on the first call: when the budget refuses part of them, what was
    already allocated is released (the claim returns to where it was), and a later call with room succeeds and gives
    the same logits as an engine that never failed."""
    import ctypes
    import os

    from llama_hip import checkpoint as ck
    cfg = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=512, seq_len=64)
    norms, t = ck.normal_model(cfg, 3)
    path = os.path.join(tmp_path, "m.bin")
    ck.write_q8_v3(path, cfg, 64, norms, ck.q8_tensors(cfg, t, 64), shared=False)
    L = hu.lib()
    assert L.llhip_init() == 0, lh.last_error()
    monkeypatch.delenv("LLAMA_HBM_BUDGET_GIB", raising=False)
    tokens = np.arange(16, dtype=np.int32) * 7
    ref = lh.Model()
    L.engine_load(ctypes.byref(ref), path.encode())
    want = np.ctypeslib.as_array(L.engine_forward_batch(ctypes.byref(ref), lh.ptr(tokens), 16, 0, lh.LOGITS_LAST),
                                 shape=(512,)).copy()
    L.engine_free(ctypes.byref(ref))
    model = lh.Model()
    L.engine_load(ctypes.byref(model), path.encode())
    try:
        claimed = L.llhip_hbm_claimed()
        # room for the first few row buffers (64 rows x 256 floats each), not for all of them
        monkeypatch.setenv("LLAMA_HBM_BUDGET_GIB", f"{(claimed + 3 * 64 * 256 * 4 + 1024) / 2 ** 30:.12f}")
        lh.record_failures()
        assert not L.engine_forward_batch(ctypes.byref(model), lh.ptr(tokens), 16, 0, lh.LOGITS_LAST)
        assert "LLAMA_HBM_BUDGET_GIB leaves" in lh.last_error(), lh.last_error()
        assert L.llhip_hbm_claimed() == claimed
        L.llhip_clear_error()
        monkeypatch.delenv("LLAMA_HBM_BUDGET_GIB")
        got = L.engine_forward_batch(ctypes.byref(model), lh.ptr(tokens), 16, 0, lh.LOGITS_LAST)
        assert got, lh.last_error()
        assert np.array_equal(np.ctypeslib.as_array(got, shape=(512,)), want)
    finally:
        L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
        L.llhip_clear_error()
        L.engine_free(ctypes.byref(model))
