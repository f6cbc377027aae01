"""End to end at Llama-3.1-8B size: a Q8_0 checkpoint of random-init weights (~N(0, 0.02), RMSNorm weights 1.0,
32 layers, 32 query / 8 KV heads of 128, vocabulary 128256, RoPE theta 500000 with Llama 3.1 scaling, gs 64), 2048
random token ids prefilled in one engine_forward_batch with every row's logits, then 256 greedy engine_forward steps,
against runq's engine on the CPU (the reference built from its sources: probe-int8).

W8A8 requantizes every activation, so any change of FP32 order flips some roundings, and 32 layers of random weights
carry those flips into the logits. The reference's own gate for such comparisons is statistical (rms 0.2, argmax
0.9, max 16; docs/architecture.md:274, written for real checkpoints). On this random model the reference does not
meet its own argmax bar against itself: its batched prefill against its per-token path gives rms 0.086 and argmax
0.79 over the last 256 prompt positions (measured on the MI355X). So the test measures that floor on the same file
and requires the engine to stay at it: every comparison within the rms and max bars of the gate, and within 1.25x the
floor's rms and 0.08 (0.15 for the 64 decode rows) of its argmax agreement.

Compared: our batched rows and our token-by-token replay of the prompt (last 256 positions) with each other and
with the reference's batched and per-token rows; our first 64 greedy decode steps with the reference's per-token
forwards of the same tokens (probe tail mode, tools/compare_engines.py --tail).

The same file in W8A32 (FP32 activations, no requantization) pins the whole 32-layer forward tightly: 64 positions
against the reference's W8A32 engine at its FP32-class gate."""
import ctypes
import os
import shutil
import sys
import time

import numpy as np
import pytest

import llama_hip as lh
from llama_hip import checkpoint as ck
from tests import hip_util as hu
from tests import ref_probe as rp

pytestmark = pytest.mark.gpu

CFG = dict(dim=4096, hidden_dim=14336, n_layers=32, n_heads=32, n_kv_heads=8, vocab_size=128256, seq_len=8192,
           rope_theta=500000.0, rope_type=1, rope_factor=8.0, rope_low=1.0, rope_high=4.0, rope_original=8192)
PROMPT, DECODE, LAST, COMPARED = 2048, 256, 256, 64


def say(*a):
    print("[c5]", *a, flush=True)
    sys.stdout.flush()


def scratch_dir(tmp_path):
    """/dev/shm when it can hold the 8.5 GB file with room to spare (it is host memory), else tmp_path."""
    shm = "/dev/shm"
    if os.path.isdir(shm) and shutil.disk_usage(shm).free > 40 << 30:
        d = os.path.join(shm, f"llhip-c5-{os.getpid()}")
        os.makedirs(d, exist_ok=True)
        return d
    return str(tmp_path)


def at_floor(ref, got, floor, what, argmax_slack):
    s = rp.gate_statistical(ref, got, what=what, rms_max=0.2, argmax_min=0.0, max_abs=16.0)
    say(f"{what}: rms {s['rms']:.4f} argmax {s['argmax']:.3f} max {s['max_abs']:.3f}")
    assert s["rms"] <= 1.25 * floor["rms"], (what, s, floor)
    assert s["argmax"] >= floor["argmax"] - argmax_slack, (what, s, floor)


@pytest.fixture(scope="module")
def c5_checkpoint(tmp_path_factory):
    """The 8B Q8_0 checkpoint of random-init weights, written once for the module's tests."""
    if not rp.have("probe-int8"):
        pytest.skip("oracle/_ref/probe-int8 not built (make -C oracle ref)")
    d = scratch_dir(tmp_path_factory.mktemp("c5"))
    path = os.path.join(d, "c5-8b-q8.bin")
    try:
        t = time.time()
        size = ck.write_q8_v3_normal(path, CFG, 64, seed=88172645463325252)
        assert os.path.getsize(path) == size
        say(f"wrote {size / 1e9:.2f} GB in {time.time() - t:.1f} s")
        yield path
    finally:
        if os.path.exists(path):
            os.unlink(path)
        if d.startswith("/dev/shm/"):
            shutil.rmtree(d, ignore_errors=True)


def test_c5_8b_prefill_2048_then_256_greedy_steps(c5_checkpoint, monkeypatch):
    L = hu.lib()
    assert L.llhip_init() == 0, lh.last_error()
    path = c5_checkpoint
    model = lh.Model()
    try:
        V = CFG["vocab_size"]
        tokens = np.random.default_rng(2048).integers(0, V, PROMPT).astype(np.int32)
        L.engine_load(ctypes.byref(model), path.encode())
        assert model.implementation, lh.last_error()
        assert model.config.seq_len == 4096 and L.engine_max_batch(ctypes.byref(model)) == PROMPT
        t = time.time()
        p = L.engine_forward_batch(ctypes.byref(model), lh.ptr(tokens), PROMPT, 0, lh.LOGITS_ALL)
        assert p, lh.last_error()
        rows = np.ctypeslib.as_array(p, shape=(PROMPT, V))
        assert np.isfinite(rows).all()
        ours_batch, last_row = rows[-LAST:].copy(), rows[-1].copy()
        say(f"prefill of {PROMPT} tokens with every row's logits in {time.time() - t:.2f} s")
        # the classifier GEMM ran in 256-row pieces whose logits copied while the next piece computed; at this
        # classifier's 128256 columns every piece takes the whole batch's unsplit tiles, so one GEMM over all rows
        # (the same prompt again: the same cache rows, bit for bit) gives the same bits
        pieces = rows.copy()
        monkeypatch.setenv("LLAMA_HIP_LOGITS_PIECE", "0")
        p = L.engine_forward_batch(ctypes.byref(model), lh.ptr(tokens), PROMPT, 0, lh.LOGITS_ALL)
        monkeypatch.delenv("LLAMA_HIP_LOGITS_PIECE")
        assert p, lh.last_error()
        assert np.array_equal(np.ctypeslib.as_array(p, shape=(PROMPT, V)), pieces)
        del pieces
        # greedy decode from the prefill's last row
        greedy, decode = [], []
        logits = last_row
        t = time.time()
        for step in range(DECODE):
            tok = int(np.argmax(logits))
            greedy.append(tok)
            p = L.engine_forward(ctypes.byref(model), tok, PROMPT + step)
            assert p, (step, lh.last_error())
            logits = np.ctypeslib.as_array(p, shape=(V,)).copy()
            assert np.isfinite(logits).all(), step
            if step < COMPARED:
                decode.append(logits)
        say(f"{DECODE} greedy steps in {time.time() - t:.2f} s; first tokens {greedy[:8]}")
        assert all(0 <= g < V for g in greedy)
        # LAST of the same batch is its ALL row up to the classifier: the last row's GEMV there, one GEMM over every
        # row here, which agree within the kernel budget 2e-5 * sum|w x| (tests/q8.c:158-183); with N(0, 0.02)
        # weights over 4096 RMSNorm-ed inputs sum|w x| is about 50, so 1e-3
        p = L.engine_forward_batch(ctypes.byref(model), lh.ptr(tokens), PROMPT, 0, lh.LOGITS_LAST)
        assert p
        last = np.ctypeslib.as_array(p, shape=(V,))
        assert np.max(np.abs(last - last_row)) <= 1e-3 and int(np.argmax(last)) == int(np.argmax(last_row))
        # the prompt token by token (rewrites the cache rows in order)
        t = time.time()
        ours_tokens = np.empty((LAST, V), np.float32)
        for pos in range(PROMPT):
            p = L.engine_forward(ctypes.byref(model), int(tokens[pos]), pos)
            assert p, (pos, lh.last_error())
            if pos >= PROMPT - LAST:
                ours_tokens[pos - PROMPT + LAST] = np.ctypeslib.as_array(p, shape=(V,))
        say(f"token-by-token replay in {time.time() - t:.2f} s")
        L.engine_free(ctypes.byref(model))
        # the reference on the CPU: its batched rows, and its per-token forwards of the last 256 prompt positions and
        # of our first 64 greedy tokens after them
        t = time.time()
        ref_batch = rp.run("probe-int8", path, list(tokens), V, mode="batch", batch=256, timeout=900)[-LAST:].copy()
        ref_tail = rp.run("probe-int8", path, list(tokens) + greedy[:COMPARED], V, mode="tail",
                          tail=LAST + COMPARED, batch=256, timeout=900)
        say(f"reference (CPU, {rp.threads()} threads): two 2048-token prefills and {LAST + COMPARED} per-token "
            f"forwards in {time.time() - t:.1f} s")
        ref_tokens, ref_decode = ref_tail[:LAST], ref_tail[LAST:]
        floor = rp.compare(ref_tokens, ref_batch)[1]
        say(f"reference batched against its per-token (the floor): rms {floor['rms']:.4f} argmax {floor['argmax']:.3f}")
        at_floor(ours_tokens, ours_batch, floor, "our batched against our per-token", 0.08)
        at_floor(ref_batch, ours_batch, floor, "our batched against the reference's batched", 0.08)
        at_floor(ref_tokens, ours_tokens, floor, "our per-token against the reference's per-token", 0.08)
        at_floor(ref_decode, np.stack(decode), floor, "our 64 greedy steps against the reference's", 0.15)
    finally:
        if model.implementation:
            L.engine_free(ctypes.byref(model))


W8A32_POSITIONS = 64


def test_c5_8b_w8a32_full_depth_at_the_fp32_gate(c5_checkpoint, monkeypatch):
    """The same 32-layer 8B file with LLAMA_Q8_ACTIVATIONS=fp32 (src/engine.c:132-135): W8A32 has no quantizer to
    flip, so the whole forward is held to the reference's FP32-class gate (docs/architecture.md:272: every position
    finite, max |d| <= 1e-3, the same argmax) against runq's W8A32 engine on the same tokens, position by position over
    64 positions. The bar is widened only to what the reference shows against itself on this file (its scalar kernels
    against its AVX-512 kernels, twice their max |d|) should that exceed 1e-3; the argmax must agree everywhere. A
    batch of the 64 tokens runs them one at a time (W8A32 takes no batched GEMM, src/engine.c:65-81), bit for bit the
    per-token rows."""
    L = hu.lib()
    assert L.llhip_init() == 0, lh.last_error()
    path = c5_checkpoint
    V = CFG["vocab_size"]
    tokens = np.random.default_rng(32).integers(0, V, W8A32_POSITIONS).astype(np.int32)
    monkeypatch.setenv("LLAMA_Q8_ACTIVATIONS", "fp32")
    monkeypatch.setenv("LLAMA_PREFILL_BATCH", str(W8A32_POSITIONS))  # W8A32's default batch is one row
    model = lh.Model()
    ours = np.empty((W8A32_POSITIONS, V), np.float32)
    try:
        L.engine_load(ctypes.byref(model), path.encode())
        assert model.implementation, lh.last_error()
        assert L.engine_max_batch(ctypes.byref(model)) == W8A32_POSITIONS and model.prefill_gemm == 0
        t = time.time()
        for pos in range(W8A32_POSITIONS):
            p = L.engine_forward(ctypes.byref(model), int(tokens[pos]), pos)
            assert p, (pos, lh.last_error())
            ours[pos] = np.ctypeslib.as_array(p, shape=(V,))
        say(f"W8A32: {W8A32_POSITIONS} positions in {time.time() - t:.2f} s")
        p = L.engine_forward_batch(ctypes.byref(model), lh.ptr(tokens), W8A32_POSITIONS, 0, lh.LOGITS_ALL)
        assert p, lh.last_error()
        assert np.array_equal(np.ctypeslib.as_array(p, shape=(W8A32_POSITIONS, V)), ours)
    finally:
        if model.implementation:
            L.engine_free(ctypes.byref(model))
    env = {"LLAMA_Q8_ACTIVATIONS": "fp32"}
    t = time.time()
    ref = rp.run("probe-int8", path, list(tokens), V, env=env, timeout=900)
    ref_scalar = rp.run("probe-int8", path, list(tokens), V, env={**env, "LLAMA_KERNELS": "scalar"}, timeout=1800)
    say(f"reference W8A32 (CPU, {rp.threads()} threads), AVX-512 and scalar kernels: {time.time() - t:.1f} s")
    floor = rp.compare(ref, ref_scalar)[1]
    rows, s = rp.compare(ref, ours)
    say(f"W8A32 ours against the reference: max |d| {s['max_abs']:.2e} rms {s['rms']:.2e} argmax {s['argmax']:.3f}; "
        f"the reference's scalar against its AVX-512: max |d| {floor['max_abs']:.2e} rms {floor['rms']:.2e} "
        f"argmax {floor['argmax']:.3f}")
    bar = max(rp.FP32_MAX_ABS, 2.0 * floor["max_abs"])
    rp.gate_strict(ref, ours, bar, f"W8A32 at 8B, {W8A32_POSITIONS} positions (bar {bar:.2e})")


def test_c5_8b_dropin_on_resident_weights(c5_checkpoint):
    """The drop-in at full size: the reference's own engine (engine.c, tp.c, runq.c and its probe, tests/probe.c)
    linked against the library in place of gemv.c, gemm.c and prefill.c (oracle/_ref/probe-int8-hip), on the 8B file,
    with LLAMA_HIP_REGISTER_MAPPINGS=1: its read-only checkpoint mapping is uploaded on first use and every later
    matmul reads the resident copy. Its logits are held to the reference's (all CPU, probe-int8, the same tokens) at
    the W8A8 gate's rms and max, and at the argmax floor this file shows the reference against itself (0.79, less the
    0.08 the C5 comparisons allow), and its decode rate per token comes from the difference of two runs of 4 and 36 tokens (load and upload
    cancel; the reference's RMSNorm, RoPE and attention stay on the CPU)."""
    if not rp.have("probe-int8-hip"):
        pytest.skip("oracle/_ref/probe-int8-hip not built (make -C oracle dropin)")
    path = c5_checkpoint
    V = CFG["vocab_size"]
    tokens = [int(t) for t in np.random.default_rng(36).integers(0, V, 36)]
    env = {"LLAMA_HIP_REGISTER_MAPPINGS": "1"}
    timings = {}
    for n in (4, 4, 36):  # the first run warms the file's pages
        t = time.time()
        got = rp.run("probe-int8-hip", path, tokens[:n], V, env=env, timeout=900)
        timings[n] = time.time() - t
    sec = (timings[36] - timings[4]) / 32
    say(f"drop-in (the reference's engine on the library, resident weights): {sec * 1e3:.2f} ms/token, "
        f"{1 / sec:.1f} tok/s; 36 tokens in {timings[36]:.2f} s including load and upload")
    t = time.time()
    ref = rp.run("probe-int8", path, tokens, V, timeout=900)
    say(f"the reference on the CPU ({rp.threads()} threads): 36 tokens in {time.time() - t:.2f} s")
    s = rp.gate_statistical(ref, got, what="drop-in at 8B", rms_max=0.2, argmax_min=0.71, max_abs=16.0)
    say(f"drop-in against the reference: rms {s['rms']:.4f} argmax {s['argmax']:.3f} max {s['max_abs']:.3f}")
