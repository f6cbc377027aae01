"""Helpers shared by the GPU parity tests: device buffers through torch, the library handle, tolerance checks.

The HIP library runs on its own stream; torch's copies run on torch's stream. Every helper that moves data synchronizes
both, so a test never reads or writes a buffer another stream is still using.
"""
import numpy as np

import llama_hip as lh

_torch = None


def torch():
    global _torch
    if _torch is None:
        import torch as t

        _torch = t
    return _torch


def lib():
    return lh.load()


def dev(a):
    """A device copy of a numpy array (a torch CUDA tensor of the same dtype and shape)."""
    t = torch()
    out = t.from_numpy(np.ascontiguousarray(a)).to("cuda")
    t.cuda.synchronize()
    return out


def empty(shape, dtype):
    t = torch()
    out = t.empty(shape, dtype=dtype, device="cuda")
    t.cuda.synchronize()
    return out


def host(x):
    """Numpy copy of a device tensor, after the library's stream has finished."""
    lib().llhip_synchronize()
    return x.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def dequant_reference(xq, xs, wq, ws, gs):
    """float64 sum and magnitude of W.x from the dequantized operands (the reference's double reference,
    tests/q8.c:86-96). xq (k,) or (m, k); wq (n, k)."""
    xd = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), gs, axis=-1)
    wd = wq.astype(np.float64) * np.repeat(ws.astype(np.float64), gs, axis=-1)
    return xd @ wd.T, np.abs(xd) @ np.abs(wd).T


def assert_within_budget(got, want, mag, rel=2e-5, floor=1e-6, what=""):
    """|got - want| <= rel * mag + floor elementwise: the reference's kernel budget (tests/q8.c:128-133)."""
    got = np.asarray(got, np.float64)
    err = np.abs(got - want)
    tol = rel * mag + floor
    bad = ~(err <= tol)
    if bad.any():
        i = np.argmax(err - tol)
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside {rel}*sum|wx|+{floor}; worst at {i}: got "
                             f"{got.ravel()[i]!r} want {np.ravel(want)[i]!r} err {err.ravel()[i]:.3g} tol "
                             f"{np.ravel(tol)[i]:.3g}")


def max_rel_error(got, want, floor=1e-3):
    """max |got - want| / (|want| + floor), the floored relative error of tests/q8_engine.c:71."""
    return float(np.max(np.abs(np.asarray(got, np.float64) - want) / (np.abs(want) + floor)))
