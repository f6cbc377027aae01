"""Running the reference's raw-logits probe (tests/probe.c of LucianCrainic/llama3.x.c, built from its sources into
oracle/_ref/ by oracle/Makefile) and the logit gates of its tools/compare_engines.py, for the end-to-end tests.

probe-int8 / probe-fp32 are runq / run on the CPU: the oracle of the engine. probe-int8-hip / probe-fp32-hip are the
same programs with gemv.c, gemm.c and prefill.c replaced by libllama3x_hip.so: the drop-in under test."""
import math
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref")


def probe_path(name):
    return os.path.join(REF, name)


def have(name):
    return os.access(probe_path(name), os.X_OK)


def threads():
    """Worker threads for the reference's team: the CPUs this process may use, at most 16."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def run(name, checkpoint, tokens, vocab, mode="tokens", batch=None, tail=None, env=None, timeout=600):
    """Logits from the probe, one float32 row per position it reports (compare_engines.py:46-64):
    mode "tokens" runs engine_forward per token (every position's row); "batch" runs engine_forward_batch in
    microbatches of `batch` rows with LLAMA_PREFILL_LOGITS=all (every row); "tail" runs the prompt but its last `tail`
    tokens through the batched prefill without logits, then those per token (the last `tail` rows)."""
    cmd = [probe_path(name)]
    e = {**os.environ, "LLAMA_BACKEND": "teams", "LLAMA_THREADS": str(threads()), **(env or {})}
    if mode == "batch":
        cmd += ["batch", str(checkpoint)]
        e.update(LLAMA_PREFILL_BATCH=str(batch), LLAMA_PREFILL_LOGITS="all")
    elif mode == "tail":
        cmd += ["tail", str(checkpoint), str(tail)]
        if batch:
            e["LLAMA_PREFILL_BATCH"] = str(batch)
    else:
        cmd += [str(checkpoint)]
    cmd += [str(t) for t in tokens]
    r = subprocess.run(cmd, capture_output=True, env=e, timeout=timeout)
    if r.returncode != 0:
        raise AssertionError(f"{name} failed (exit {r.returncode}): {r.stderr.decode(errors='replace')[-2000:]}")
    rows = tail if mode == "tail" else len(tokens)
    out = np.frombuffer(r.stdout, np.float32)
    assert out.size == rows * vocab, (name, out.size, rows, vocab)
    return out.reshape(rows, vocab)


def compare(a, b):
    """Per position of reference rows a and candidate rows b: max |delta|, rms of delta, max relative delta (against
    max(|a|, 1)), argmax agreement and finiteness, as compare_engines.py:67-80 computes them; plus the summary over the
    positions (compare_engines.py:146-150)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    d = np.abs(b - a)
    rows = dict(max_abs=d.max(axis=1), rms=np.sqrt((d ** 2).mean(axis=1)),
                max_rel=(d / np.maximum(np.abs(a), 1.0)).max(axis=1),
                argmax=a.argmax(axis=1) == b.argmax(axis=1), finite=np.isfinite(b).all(axis=1))
    summary = dict(max_abs=float(rows["max_abs"].max()), rms=math.sqrt(float((rows["rms"] ** 2).mean())),
                   max_rel=float(rows["max_rel"].max()), argmax=float(rows["argmax"].mean()),
                   finite=bool(rows["finite"].all()))
    return rows, summary


def gate_strict(a, b, max_abs, what):
    """The per-position gate (compare_engines.py:139-141): every row finite, max |delta| <= max_abs, same argmax."""
    rows, s = compare(a, b)
    bad = [i for i in range(len(a)) if not (rows["finite"][i] and rows["argmax"][i] and rows["max_abs"][i] <= max_abs)]
    assert not bad, f"{what}: positions {bad[:8]} over the gate (max |d| {max_abs}); summary {s}"
    return s


def gate_statistical(a, b, rms_max, argmax_min, max_abs, what):
    """The statistical gate (compare_engines.py:141-154) that W8A8 comparisons use: every row finite and within
    max_abs, the rms over all positions within rms_max and the argmax agreement at least argmax_min."""
    rows, s = compare(a, b)
    assert s["finite"], f"{what}: non-finite logits; summary {s}"
    assert s["max_abs"] <= max_abs and s["rms"] <= rms_max and s["argmax"] >= argmax_min, f"{what}: summary {s}"
    return s


# The gates of the reference's architecture notes (docs/architecture.md:268-274).
W8A8 = dict(rms_max=0.2, argmax_min=0.9, max_abs=16.0)  # W8A8 against W8A8: any change of FP32 order requantizes
FP32_MAX_ABS = 1e-3                                     # FP32 engines against each other: max 1e-3, argmax 100%
BF16 = dict(rms_max=0.05, argmax_min=0.97, max_abs=2.0)  # BF16 against FP32 per token
