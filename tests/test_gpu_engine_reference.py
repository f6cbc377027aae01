"""The engine end to end against the reference's own engine (src/engine.c, src/tp.c, src/runq.c / src/run.c, built
from its sources into oracle/_ref/ as the raw-logits probes probe-int8 / probe-fp32), and the drop-in: the same
probes with gemv.c, gemm.c and prefill.c replaced by libllama3x_hip.so (probe-int8-hip / probe-fp32-hip).

Gates are the reference's (docs/architecture.md:268-274, tools/compare_engines.py): W8A8 against W8A8 is statistical
(rms 0.2, argmax 0.9, max 16: any change of FP32 order can flip a quantization), FP32 against FP32 is per position
(max |d| 1e-3, same argmax), BF16 against FP32 is statistical (rms 0.05, argmax 0.97, max 2). The reference's own
W8A8 noise on the random model here, its scalar against its AVX-512 path, is rms 0.003 with argmax 0.98; the tests
also require the GPU within a fixed multiple of that floor. Weights are random-init (~N(0, 0.02), norms 1), so the
logits have no ties; the reference's sinusoid fixture (tests/fixtures.py), whose logits are nearly tied, is compared
on the magnitudes only."""
import ctypes
import os
import struct

import numpy as np
import pytest

import llama_hip as lh
from llama_hip import checkpoint as ck
from tests import hip_util as hu
from tests import ref_probe as rp
from tests.golden import ref_fixtures as rf

pytestmark = pytest.mark.gpu

GS = 64
CFG = dict(dim=512, hidden_dim=1536, n_layers=3, n_heads=8, n_kv_heads=2, vocab_size=4096, seq_len=256, rope_type=1,
           rope_factor=8.0, rope_low=1.0, rope_high=4.0, rope_original=64)
V = CFG["vocab_size"]
TOKENS = [int(t) for t in np.random.default_rng(2).integers(0, V, 96)]


def need(*names):
    missing = [n for n in names if not rp.have(n)]
    if missing:
        pytest.skip(f"oracle/_ref/{missing[0]} not built (make -C oracle ref dropin)")


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    """The same random model as FP32 (version 3 and legacy) and Q8_0 (version 3 and version 2), untied."""
    root = tmp_path_factory.mktemp("models")
    norms, t = ck.normal_model(CFG, 5)
    paths = {k: str(root / f"{k}.bin") for k in ("f32", "f32_legacy", "q8", "q8_v2")}
    ck.write_f32_v3(paths["f32"], CFG, norms, t, shared=False)
    ck.write_q8_v3(paths["q8"], CFG, GS, norms, ck.q8_tensors(CFG, t, GS), shared=False)
    # legacy FP32: seven ints (negative vocabulary: untied), the body, the unused RoPE table before the classifier
    body = open(paths["f32"], "rb").read()[256:]
    cls = V * CFG["dim"] * 4
    legacy = struct.pack("<7i", *(CFG[k] for k in ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads")), -V,
                         CFG["seq_len"])
    table = bytes(CFG["seq_len"] * (CFG["dim"] // CFG["n_heads"]) * 4)
    open(paths["f32_legacy"], "wb").write(legacy + body[:-cls] + table + body[-cls:])
    # version 2 INT8: the 41-byte header (flag byte at 36, group size at 37) padded to 256, the same body
    q8 = open(paths["q8"], "rb").read()
    head = struct.pack("<Ii7iBi", rf.MAGIC, 2, *(CFG[k] for k in ("dim", "hidden_dim", "n_layers", "n_heads",
                                                                  "n_kv_heads", "vocab_size", "seq_len")), 0, GS)
    open(paths["q8_v2"], "wb").write(head + bytes(256 - len(head)) + q8[256:])
    return paths


def engine_rows(path, tokens, vocab, mode="tokens", batch=None, monkeypatch=None, env=None):
    """Our engine's logits at every position: per token (engine_forward), or engine_forward_batch in microbatches of
    engine_max_batch rows (LLAMA_PREFILL_BATCH=batch) with every row's logits, as the probe's batch mode runs."""
    L = hu.lib()
    assert L.llhip_init() == 0, lh.last_error()
    for k, v in {**(env or {}), **({"LLAMA_PREFILL_BATCH": str(batch)} if batch else {})}.items():
        monkeypatch.setenv(k, v)
    model = lh.Model()
    out = np.empty((len(tokens), vocab), np.float32)
    try:
        L.engine_load(ctypes.byref(model), path.encode())
        assert model.implementation, lh.last_error()
        if mode == "tokens":
            for pos, tok in enumerate(tokens):
                p = L.engine_forward(ctypes.byref(model), int(tok), pos)
                assert p, lh.last_error()
                out[pos] = np.ctypeslib.as_array(p, shape=(vocab,))
        else:
            ids = np.asarray(tokens, np.int32)
            step = L.engine_max_batch(ctypes.byref(model))
            for at in range(0, len(tokens), step):
                n = min(step, len(tokens) - at)
                p = L.engine_forward_batch(ctypes.byref(model), lh.ptr(ids[at:at + n]), n, at, lh.LOGITS_ALL)
                assert p, lh.last_error()
                out[at:at + n] = np.ctypeslib.as_array(p, shape=(n, vocab))
    finally:
        L.engine_free(ctypes.byref(model))
        for k in {**(env or {}), **({"LLAMA_PREFILL_BATCH": 1} if batch else {})}:
            monkeypatch.delenv(k, raising=False)
    return out


def within_floor(ref, got, floor, what, factor=4.0):
    """got's distance from the reference engine stays within `factor` times the reference's own noise between two of
    its instruction sets (floor: compare() of those two runs), besides the reference's gate."""
    s = rp.compare(ref, got)[1]
    assert s["rms"] <= factor * max(floor["rms"], 1e-6), (what, s, floor)
    return s


def test_baseline_logits_of_the_reference(tmp_path):
    """tests/baseline_logits.json: the reference's regression numbers, the first 12 logits at positions 0..3 of tokens
    65..68 on its default fixture (tests/test_runtime.py:55-66), within its rel 2e-5 / abs 2e-6, from the version-2
    INT8 file (group size 2: the generic kernels) and the legacy FP32 file, and from both after upgrade_v3."""
    import json
    import math
    base = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "baseline_logits.json")))
    root = rf.create(tmp_path / "fx")
    L = hu.lib()
    assert L.llhip_init() == 0, lh.last_error()
    for upgraded in (False, True):
        if upgraded:
            rf.upgrade_v3(root)
        for name, key in (("int8.bin", "runq"), ("fp32.bin", "run")):
            model = lh.Model()
            L.engine_load(ctypes.byref(model), str(root / name).encode())
            assert model.implementation, lh.last_error()
            try:
                got = []
                for p in range(4):
                    out = L.engine_forward(ctypes.byref(model), 65 + p, p)
                    assert out, lh.last_error()
                    got += list(np.ctypeslib.as_array(out, shape=(model.config.vocab_size,))[:12])
            finally:
                L.engine_free(ctypes.byref(model))
            for i, (a, e) in enumerate(zip(got, base[key])):
                assert math.isclose(a, e, rel_tol=2e-5, abs_tol=2e-6), (name, upgraded, i, a, e)


def test_q8_engine_against_runq(models, monkeypatch):
    """W8A8: our engine per token and in 32-row batches against runq's engine (probe-int8) in the same modes, at the
    reference's statistical gate and within 4x its own scalar / AVX-512 noise floor; version 2 reads the same."""
    need("probe-int8")
    ref_tok = rp.run("probe-int8", models["q8"], TOKENS, V)
    floor = rp.compare(rp.run("probe-int8", models["q8"], TOKENS, V, env={"LLAMA_KERNELS": "scalar"}), ref_tok)[1]
    ref_batch = rp.run("probe-int8", models["q8"], TOKENS, V, mode="batch", batch=32)
    got_tok = engine_rows(models["q8"], TOKENS, V, monkeypatch=monkeypatch)
    got_batch = engine_rows(models["q8"], TOKENS, V, mode="batch", batch=32, monkeypatch=monkeypatch)
    rp.gate_statistical(ref_tok, got_tok, what="per token", **rp.W8A8)
    rp.gate_statistical(ref_batch, got_batch, what="batch 32", **rp.W8A8)
    rp.gate_statistical(got_tok, got_batch, what="our batch against our tokens", **rp.W8A8)
    within_floor(ref_tok, got_tok, floor, "per token")
    within_floor(ref_batch, got_batch, floor, "batch 32")
    # version 2 carries no RoPE metadata (the defaults: theta 500000, no scaling), so it matches the scaled version 3
    # file at position 0 only, and runq on the same file everywhere
    v2 = engine_rows(models["q8_v2"], TOKENS[:16], V, monkeypatch=monkeypatch)
    assert np.array_equal(v2[0], got_tok[0])
    rp.gate_statistical(rp.run("probe-int8", models["q8_v2"], TOKENS[:16], V), v2, what="version 2", **rp.W8A8)


def test_q8_engine_on_the_reference_fixture(tmp_path, monkeypatch):
    """The reference's own gs-64 fixture (tests/fixtures.py TP_WIDE_CONFIG, version 3 with Llama 3.1 RoPE scaling):
    nearly tied logits, so only the magnitudes are gated (max |d| and rms within the W8A8 gate)."""
    need("probe-int8")
    root = rf.create(tmp_path / "wide", config=rf.TP_WIDE_CONFIG, gs=64)
    rf.upgrade_v3(root, config=rf.TP_WIDE_CONFIG, gs=64, scaling=True)
    vocab = rf.TP_WIDE_CONFIG[5]
    tokens = [int(t) for t in np.random.default_rng(1).integers(0, vocab, 48)]
    path = str(root / "int8.bin")
    for mode, batch in (("tokens", None), ("batch", 16)):
        ref = rp.run("probe-int8", path, tokens, vocab, mode=mode, batch=batch)
        got = engine_rows(path, tokens, vocab, mode=mode, batch=batch, monkeypatch=monkeypatch)
        s = rp.gate_statistical(ref, got, what=f"fixture {mode}", rms_max=0.2, argmax_min=0.0, max_abs=16.0)
        # logits up to about 2.3 here; an activation quantized the other way moves them by about 2e-3
        assert s["max_abs"] < 1e-2 and s["rms"] < 1e-3, (mode, s)


def test_w8a32_engine_against_runq(models, monkeypatch):
    """LLAMA_Q8_ACTIVATIONS=fp32: no quantizer in the way, so the FP32 gate (max 1e-3, argmax 100%) against runq's
    W8A32 engine. With LLAMA_PREFILL_BATCH=8 a batch runs its rows one token at a time (src/engine.c:65-81): ALL gives
    every row, equal to the per-token logits bit for bit, LAST the last row's, NONE only the cache rows."""
    need("probe-int8")
    env = {"LLAMA_Q8_ACTIVATIONS": "fp32"}
    ref = rp.run("probe-int8", models["q8"], TOKENS[:48], V, env=env)
    got = engine_rows(models["q8"], TOKENS[:48], V, monkeypatch=monkeypatch, env=env)
    rp.gate_strict(ref, got, rp.FP32_MAX_ABS, "w8a32 per token")
    batch = engine_rows(models["q8"], TOKENS[:48], V, mode="batch", batch=8, monkeypatch=monkeypatch, env=env)
    assert np.array_equal(batch, got)
    L = hu.lib()
    monkeypatch.setenv("LLAMA_Q8_ACTIVATIONS", "fp32")
    monkeypatch.setenv("LLAMA_PREFILL_BATCH", "8")
    model = lh.Model()
    try:
        L.engine_load(ctypes.byref(model), models["q8"].encode())
        assert L.engine_max_batch(ctypes.byref(model)) == 8 and model.prefill_gemm == 0
        ids = np.asarray(TOKENS[:16], np.int32)
        assert not L.engine_forward_batch(ctypes.byref(model), lh.ptr(ids[:8]), 8, 0, lh.LOGITS_NONE)
        assert not lh.last_error()
        p = L.engine_forward_batch(ctypes.byref(model), lh.ptr(ids[8:]), 8, 8, lh.LOGITS_LAST)
        assert p and np.array_equal(np.ctypeslib.as_array(p, shape=(V,)), got[15])
    finally:
        L.engine_free(ctypes.byref(model))


def test_gemm_off_batches_run_per_token(models, monkeypatch):
    """LLAMA_PREFILL_GEMM=off with LLAMA_PREFILL_BATCH=8: batches run token by token, bit for bit the per-token
    engine (the batched GEMM never runs)."""
    got = engine_rows(models["q8"], TOKENS[:24], V, monkeypatch=monkeypatch)
    off = engine_rows(models["q8"], TOKENS[:24], V, mode="batch", batch=8, monkeypatch=monkeypatch,
                      env={"LLAMA_PREFILL_GEMM": "off"})
    assert np.array_equal(off, got)


@pytest.mark.parametrize("fmt", ["f32", "f32_legacy"])
def test_fp32_engine_against_run(models, monkeypatch, fmt):
    """FP32 checkpoints (version 3 and legacy): the FP32 GEMVs per token and the FP32 GEMM in 32-row batches, against
    run's engine (probe-fp32) at the FP32 gate (max |d| 1e-3, same argmax at every position)."""
    need("probe-fp32")
    L = hu.lib()
    ref = rp.run("probe-fp32", models[fmt], TOKENS, V)
    got = engine_rows(models[fmt], TOKENS, V, monkeypatch=monkeypatch)
    assert L.engine_precision() == b"fp32" and L.engine_group_size() == 0
    rp.gate_strict(ref, got, rp.FP32_MAX_ABS, f"{fmt} per token")
    ref_b = rp.run("probe-fp32", models[fmt], TOKENS, V, mode="batch", batch=32)
    got_b = engine_rows(models[fmt], TOKENS, V, mode="batch", batch=32, monkeypatch=monkeypatch)
    rp.gate_strict(ref_b, got_b, rp.FP32_MAX_ABS, f"{fmt} batch 32")


def test_bf16_engine_against_run(models, monkeypatch):
    """LLAMA_PRECISION=bf16: the batched GEMMs on BF16 copies packed at load (every batch, the all-row classifier
    too), against run's BF16 mode and against its FP32 per-token logits, at the BF16 gate."""
    need("probe-fp32")
    L = hu.lib()
    env = {"LLAMA_PRECISION": "bf16"}
    ref_bf16 = rp.run("probe-fp32", models["f32"], TOKENS, V, mode="batch", batch=32, env=env)
    ref_f32 = rp.run("probe-fp32", models["f32"], TOKENS, V)
    got = engine_rows(models["f32"], TOKENS, V, mode="batch", batch=32, monkeypatch=monkeypatch, env=env)
    assert L.engine_precision() == b"bf16_from_fp32"
    rp.gate_statistical(ref_bf16, got, what="bf16 against run's bf16", **rp.BF16)
    rp.gate_statistical(ref_f32, got, what="bf16 against run's fp32", **rp.BF16)
    assert rp.compare(ref_bf16, got)[1]["rms"] <= rp.compare(ref_f32, ref_bf16)[1]["rms"]


def test_dropin_probes_against_the_reference(models):
    """The reference's own engine.c and tp.c on libllama3x_hip.so (its gemv.c, gemm.c and prefill.c left out of the
    link, unchanged headers): runq per token and in batches at the W8A8 gate, run at the FP32 gate, run's BF16 mode at
    the BF16 gate, each against the all-CPU build of the same probe."""
    need("probe-int8", "probe-fp32", "probe-int8-hip", "probe-fp32-hip")
    ref = rp.run("probe-int8", models["q8"], TOKENS, V)
    floor = rp.compare(rp.run("probe-int8", models["q8"], TOKENS, V, env={"LLAMA_KERNELS": "scalar"}), ref)[1]
    got = rp.run("probe-int8-hip", models["q8"], TOKENS, V)
    rp.gate_statistical(ref, got, what="drop-in runq per token", **rp.W8A8)
    within_floor(ref, got, floor, "drop-in runq per token")
    # with the checkpoint mapping registered on first use (resident weights instead of staging per call): the same
    # kernels on the same bytes, so bit for bit the staged run
    resident = rp.run("probe-int8-hip", models["q8"], TOKENS, V, env={"LLAMA_HIP_REGISTER_MAPPINGS": "1"})
    assert np.array_equal(resident, got)
    ref = rp.run("probe-int8", models["q8"], TOKENS, V, mode="batch", batch=32)
    got = rp.run("probe-int8-hip", models["q8"], TOKENS, V, mode="batch", batch=32)
    rp.gate_statistical(ref, got, what="drop-in runq batch 32", **rp.W8A8)
    within_floor(ref, got, floor, "drop-in runq batch 32")
    assert np.array_equal(rp.run("probe-int8-hip", models["q8"], TOKENS, V, mode="batch", batch=32,
                                 env={"LLAMA_HIP_REGISTER_MAPPINGS": "1"}), got)
    for mode in ("tokens", "batch"):
        ref = rp.run("probe-fp32", models["f32"], TOKENS, V, mode=mode, batch=32)
        got = rp.run("probe-fp32-hip", models["f32"], TOKENS, V, mode=mode, batch=32)
        rp.gate_strict(ref, got, rp.FP32_MAX_ABS, f"drop-in run {mode}")
        resident = rp.run("probe-fp32-hip", models["f32"], TOKENS, V, mode=mode, batch=32,
                          env={"LLAMA_HIP_REGISTER_MAPPINGS": "1"})
        assert np.array_equal(resident, got), mode
    env = {"LLAMA_PRECISION": "bf16"}
    ref = rp.run("probe-fp32", models["f32"], TOKENS, V, mode="batch", batch=32, env=env)
    got = rp.run("probe-fp32-hip", models["f32"], TOKENS, V, mode="batch", batch=32, env=env)
    rp.gate_statistical(ref, got, what="drop-in run bf16", **rp.BF16)


def test_8b_shapes_against_runq(tmp_path, monkeypatch):
    """Llama-3.1-8B layer shapes (dim 4096, hidden 14336, 32 query / 8 KV heads of 128, vocabulary 128256, RoPE theta
    500000 with Llama 3.1 scaling, gs 64, untied), two layers of random-init weights: 24 positions per token and in
    one batch against runq at the W8A8 gate."""
    need("probe-int8")
    cfg = dict(dim=4096, hidden_dim=14336, n_layers=2, n_heads=32, n_kv_heads=8, vocab_size=128256, seq_len=8192,
               rope_theta=500000.0, rope_type=1, rope_factor=8.0, rope_low=1.0, rope_high=4.0, rope_original=8192)
    path = str(tmp_path / "8b2.bin")
    ck.write_q8_v3_normal(path, cfg, 64, seed=21)
    vocab = cfg["vocab_size"]
    tokens = [int(t) for t in np.random.default_rng(9).integers(0, vocab, 24)]
    for mode, batch in (("tokens", None), ("batch", 24)):
        ref = rp.run("probe-int8", path, tokens, vocab, mode=mode, batch=batch)
        got = engine_rows(path, tokens, vocab, mode=mode, batch=batch, monkeypatch=monkeypatch)
        rp.gate_statistical(ref, got, what=f"8b shapes {mode}", **rp.W8A8)
    os.unlink(path)


def test_engine_kv_stats_and_context(models):
    """engine_kv_stats (runtime.h:113): both caches reserved over the context, the first `position` positions
    active, no NUMA node for device memory; the default context is min(seq_len, 4096) and an explicit one is
    exact (src/engine.c:147-150)."""
    L = hu.lib()
    model = lh.Model()
    L.engine_load_context(ctypes.byref(model), models["q8"].encode(), 100)
    try:
        assert model.config.seq_len == 100 and L.engine_max_batch(ctypes.byref(model)) == 100
        st = lh.KvStats()
        L.engine_kv_stats(ctypes.byref(model), 10, 1, ctypes.byref(st))
        row = CFG["dim"] // CFG["n_heads"] * CFG["n_kv_heads"] * 4
        assert st.reserved_bytes == 2 * CFG["n_layers"] * 100 * row and st.active_bytes == 2 * CFG["n_layers"] * 10 * row
        assert st.node == -1 and st.verified == 0
        lh.record_failures()
        try:
            assert not L.engine_forward(ctypes.byref(model), 1, 100)
            assert lh.last_error() == "forward input out of range: token=1 position=100"
        finally:
            L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
            L.llhip_clear_error()
    finally:
        L.engine_free(ctypes.byref(model))
