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
