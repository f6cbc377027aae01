"""The fixture generator (tests/golden/ref_fixtures.py) and the logit gates (tests/ref_probe.py) that the end-to-end
tests use, pinned on the CPU: the reference's own probes, built from its sources (oracle/_ref), reproduce its
regression numbers (tests/baseline_logits.json, tests/test_runtime.py:55-66) on the files written here, and each gate
rejects a planted mistake."""
import json
import math
import os

import numpy as np
import pytest

from tests import ref_probe as rp
from tests.golden import ref_fixtures as rf

BASE = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "baseline_logits.json")))


@pytest.mark.parametrize("upgraded", [False, True])
def test_reference_fixture_reproduces_baseline(tmp_path, upgraded):
    """The first 12 logits at positions 0..3 of tokens 65..68 (tests/unit.c:58-63) from the version-2 INT8 and legacy
    FP32 files (and their version-3 upgrades, which change only the header) within rel 2e-5 / abs 2e-6."""
    if not (rp.have("probe-int8") and rp.have("probe-fp32")):
        pytest.skip("oracle/_ref probes not built (make -C oracle ref)")
    root = rf.create(tmp_path / "fx")
    if upgraded:
        rf.upgrade_v3(root)
    vocab = rf.CONFIG[5]
    for name, key, probe in (("int8.bin", "runq", "probe-int8"), ("fp32.bin", "run", "probe-fp32")):
        got = rp.run(probe, root / name, [65, 66, 67, 68], vocab)[:, :12].reshape(-1)
        for i, (a, e) in enumerate(zip(got, BASE[key])):
            assert math.isclose(float(a), e, rel_tol=2e-5, abs_tol=2e-6), (name, i, a, e)


def test_fixture_bytes():
    """Q8_0 of the generator in double precision: ties round to even, the scale is float32(max|w| / 127), and a zero
    group has a zero scale and zero values (fixtures.py:56-64)."""
    w = np.array([0.5, -1.5, 2.5, 127.0, 0, 0, 0, 0], np.float32)
    q, s = rf.quantize(w, 4)
    assert s.tolist() == [1.0, 0.0] and q.tolist() == [0, -2, 2, 127, 0, 0, 0, 0]
    f = rf.floats(3, 0.2)
    assert f.dtype == np.float32 and f[1] == np.float32(0.12 * math.sin(0.71 + 0.2))


def test_gates_reject_planted_mistakes():
    """A wrong row, a flipped argmax or a non-finite value fails the gate that must catch it; noise below the gate
    passes."""
    rng = np.random.default_rng(0)
    a = rng.standard_normal((20, 300)).astype(np.float32)
    noisy = a + rng.normal(0, 0.01, a.shape).astype(np.float32)
    rp.gate_statistical(a, noisy, what="noise", **rp.W8A8)
    with pytest.raises(AssertionError):
        rp.gate_strict(a, noisy, rp.FP32_MAX_ABS, "noise above 1e-3")
    shifted = noisy.copy()
    shifted[3] = a[4]  # a row of the wrong position
    with pytest.raises(AssertionError):
        rp.gate_statistical(a, shifted, what="wrong row", **rp.BF16)
    flipped = a.copy()
    for i in range(3):  # three of twenty argmaxes moved: agreement 0.85 < 0.9
        flipped[i, a[i].argmin()] = a[i].max() + 1
    with pytest.raises(AssertionError):
        rp.gate_statistical(a, flipped, what="argmax", rms_max=10, argmax_min=0.9, max_abs=100)
    bad = a.copy()
    bad[5, 7] = np.nan
    with pytest.raises(AssertionError):
        rp.gate_statistical(a, bad, what="nan", **rp.W8A8)
