"""The device quantizer's reciprocal shortcut, checked on the CPU against the oracle. CPU only.

The HIP quantizer (llama3.x.c_amd/csrc/gemv.hip, quantize_fast) forms r = x * rcp(scale) and takes rint(r), as the low
byte of t = r + 1.5 * 2^23, instead of rounding the exact quotient x / scale, unless some value of the call has
|r - (t - 1.5 * 2^23)| > 0.5 - 2^-12 (r within 2^-12 of a rounding tie, or not finite), or the scale is zero, not
normal or infinite: then the exact quotient decides for all values of the call. The argument: |r - fl(x / scale)| <
2.3e-5 when rcp is within 1 ulp, so outside the margin both round to the same integer. Here the same steps run in
float32 numpy (denormals kept, as in the kernels) with the reciprocal perturbed by -1, 0 and +1 ulp, on random groups,
subnormal inputs and inputs built to sit next to every rounding tie, and must reproduce the oracle's k_quantize bit for
bit.
"""
import numpy as np

from oracle import pyoracle as orc

F32_MIN = np.float32(1.17549435e-38)


MAGIC = np.float32(12582912.0)  # 1.5 * 2^23
F32_MAX = np.float32(3.40282347e38)


def fast_quantize(x, gs, ulp_shift, per_call=16):
    """The device steps: per group the reciprocal of the scale, per value r = x * inv, t = r + M (r rounded to an
    integer, ties to even, in the low mantissa bits), the int8 value the low byte of t's bits; a call of `per_call`
    consecutive values of one lane falls back to the exact quotient when any of them is near a tie or not finite, or
    the scale is not normal and finite."""
    x = np.asarray(x, np.float32).reshape(-1, gs)
    peak = np.max(np.abs(x), axis=1)
    scale = (peak / np.float32(127.0)).astype(np.float32)
    ok = (scale >= F32_MIN) & (scale <= F32_MAX)
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        inv = np.where(ok, (np.float32(1.0) / np.where(ok, scale, 1)).astype(np.float32), np.float32(0))
        for _ in range(abs(ulp_shift)):
            inv = np.nextafter(inv, np.float32(np.inf if ulp_shift > 0 else 0)).astype(np.float32)
        r = (x * inv[:, None]).astype(np.float32)
        t = (r + MAGIC).astype(np.float32)
        k = (t - MAGIC).astype(np.float32)
        near = ~(np.abs((r - k).astype(np.float32)) <= np.float32(0.5 - 2.0 ** -12))
        slow_value = near | ~ok[:, None]
        # one branch per call: a lane's per_call consecutive values go the exact way together
        slow = np.repeat(slow_value.reshape(x.shape[0], -1, per_call).any(axis=2), per_call, axis=1)
        low_byte = (t.view(np.uint32) & np.uint32(0xFF)).astype(np.uint8).view(np.int8)
        # wherever the fast value is taken it is rint(r) and within the int8 range
        assert np.all(np.where(slow, 0, np.abs(k)) <= 127)
        assert np.array_equal(np.where(slow, 0, low_byte), np.where(slow, 0, k).astype(np.int8))
    q_ref, s_ref = orc.quantize(x, gs)
    q = np.where(slow, q_ref, low_byte)
    return q.astype(np.int8), scale, slow.mean()


def adversarial(rng, gs, groups):
    """Groups whose max is 127 * scale exactly, with members at k + 0.5 +- a few ulps of the scaled value."""
    out = []
    for g in range(groups):
        scale = np.float32(abs(rng.normal(1, 0.0, 1.0)[0]) * 10.0 ** rng.uniform(1, 6.0)[0] + 1e-6)
        ks = np.floor(rng.uniform(gs - 1, 126.0)).astype(np.float32)
        jitter = np.round(rng.uniform(gs - 1, 4.0)).astype(np.int32)
        vals = []
        for k, j in zip(ks, jitter):
            v = np.float32((k + np.float32(0.5)) * scale)
            for _ in range(abs(int(j))):
                v = np.nextafter(v, np.float32(np.inf) if j > 0 else np.float32(-np.inf))
            vals.append(v)
        vals = np.array(vals, np.float32) * np.where(rng.uniform(gs - 1) < 0, -1, 1).astype(np.float32)
        out.append(np.concatenate([[np.float32(127) * scale], vals]))
    return np.concatenate(out).astype(np.float32)


def test_fast_path_reproduces_k_quantize_bitwise():
    rng = orc.Rng(orc.SEED + 31)
    cases = [rng.normal(64 * 4096, 0.0, 1.0), rng.normal(64 * 1024, 0.0, 1e-3), rng.normal(64 * 1024, 0.0, 1e4),
             adversarial(rng, 64, 2000)]
    tiny = rng.normal(64 * 64, 0.0, 1.0) * np.float32(1e-38)
    cases.append(tiny.astype(np.float32))
    # subnormal members of groups whose scale is just normal (x / scale up to ~1: a flushing multiply would give 0)
    sub = (rng.normal(64 * 256, 0.0, 1.0) * np.float32(2.0 ** -127)).astype(np.float32).reshape(-1, 64)
    sub = np.clip(sub, np.float32(-2.0 ** -126) * np.float32(0.99), np.float32(2.0 ** -126) * np.float32(0.99))
    sub[:, 0] = np.float32(127.0) * np.float32(2.0 ** -126)
    cases.append(sub.ravel())
    for x in cases:
        want_q, want_s = orc.quantize(x.reshape(-1, 64), 64)
        for shift in (-1, 0, 1):
            for per_call in (1, 4, 16):
                q, s, exact_share = fast_quantize(x, 64, shift, per_call)
                assert np.array_equal(s.view(np.uint32), want_s.ravel().view(np.uint32))
                assert np.array_equal(q.ravel(), want_q.ravel()), (shift, per_call)
                if x is cases[-1] and per_call == 1:
                    assert exact_share < 0.5  # the subnormal inputs mostly take the fast path


def test_margin_catches_a_plausible_slip():
    """Without the margin (always clamp(rint(r))), the adversarial inputs disagree with k_quantize for some reciprocal
    error: the fallback is what makes the shortcut exact. rint's ties-to-even also differs from roundf's
    half-away-from-zero on exact ties, which only the fallback resolves."""
    rng = orc.Rng(orc.SEED + 32)
    x = adversarial(rng, 64, 3000).reshape(-1, 64)
    want_q, _ = orc.quantize(x, 64)
    peak = np.max(np.abs(x), axis=1)
    scale = (peak / np.float32(127.0)).astype(np.float32)
    mismatches = 0
    for shift in (-1, 1):
        inv = (np.float32(1.0) / scale).astype(np.float32)
        inv = np.nextafter(inv, np.float32(np.inf if shift > 0 else 0)).astype(np.float32)
        r = (x * inv[:, None]).astype(np.float32)
        naive = np.clip(np.rint(r), -127, 127).astype(np.int8)
        mismatches += int(np.sum(naive != want_q))
    assert mismatches > 0
    ties = np.array([0.5, 1.5, 2.5, -0.5, -2.5, 126.5] + [127.0] * 58, np.float32) * np.float32(0.25)
    q_ties, _ = orc.quantize(ties.reshape(1, 64), 64)
    s = np.float32(127.0 * 0.25) / np.float32(127.0)
    assert not np.array_equal(np.clip(np.rint(ties / s), -127, 127).astype(np.int8), q_ties.ravel())
