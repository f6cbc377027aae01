"""LLAMA_HIP_REGISTER_MAPPINGS=1: host weights inside a read-only file mapping are uploaded once, on first use, and the
registration follows the mapping. The reference unmaps its checkpoint when the model is freed (src/engine.c:55), and
a process that loads another checkpoint may get the same addresses back; the library must then read the new file,
or the new place in the same file, not the copy of the old one.

The switch is read once per process, so the checks run in a child process with it set. Each GEMV on mapped weights
is compared bit for bit with the same call on the weights in plain host memory (staged per call: the same kernel on
the same bytes), and the HBM claim shows when a copy is made and dropped."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r'''
import ctypes, os, sys
import numpy as np
sys.path[:0] = [sys.argv[1], os.path.join(sys.argv[1], "llama3.x.c_amd")]
import llama_hip as lh
L = lh.load()
assert L.llhip_init() == 0
tmp = sys.argv[2]
n, k, gs = 256, 512, 64
wbytes = n * k + n * (k // gs) * 4
size = (wbytes + 4095) // 4096 * 4096
libc = ctypes.CDLL(None, use_errno=True)
libc.mmap.restype = ctypes.c_void_p
libc.mmap.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_long]
libc.munmap.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
PROT_READ, PROT_WRITE, MAP_PRIVATE, MAP_FIXED, MAP_ANONYMOUS = 1, 2, 2, 0x10, 0x20

def weights(seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(-127, 128, (n, k), dtype=np.int8)
    s = (rng.random((n, k // gs), dtype=np.float32) * 0.01 + 0.001).astype(np.float32)
    raw = np.zeros(size, np.uint8)
    raw[:n * k] = q.reshape(-1).view(np.uint8)
    raw[n * k:wbytes] = s.reshape(-1).view(np.uint8)
    return raw

rng = np.random.default_rng(7)
x = rng.standard_normal(k).astype(np.float32)
xq, xs = np.empty(k, np.int8), np.empty(k // gs, np.float32)
L.k_quantize(lh.ptr(xq), lh.ptr(xs), lh.ptr(x), k, gs)

def gemv(base):
    out = np.empty(n, np.float32)
    w = lh.K8Weight(base, base + n * k)
    L.k_matmul_q8(lh.ptr(out), lh.K8Input(lh.ptr(xq), lh.ptr(xs), None), w, k, n, gs)
    assert lh.last_error() == "", lh.last_error()
    return out

def mapped(path, addr=None, fixed=False, offset=0):
    fd = os.open(path, os.O_RDONLY)
    p = libc.mmap(addr, size, PROT_READ, MAP_PRIVATE | (MAP_FIXED if fixed else 0), fd, offset)
    os.close(fd)
    assert p not in (None, ctypes.c_void_p(-1).value), ctypes.get_errno()
    return p

A, B, C = weights(1), weights(2), weights(3)
want = {}
for name, raw in (("A", A), ("B", B), ("C", C)):
    want[name] = gemv(raw.ctypes.data)  # plain host memory: staged per call
with open(os.path.join(tmp, "A"), "wb") as f:
    f.write(A.tobytes())
with open(os.path.join(tmp, "B"), "wb") as f:  # B, then C one page further on
    f.write(B.tobytes() + bytes(4096) + C.tobytes())
assert not np.array_equal(want["A"], want["B"]) and not np.array_equal(want["B"], want["C"])
base_claim = L.llhip_hbm_claimed()

a = mapped(os.path.join(tmp, "A"))
assert np.array_equal(gemv(a), want["A"])
assert L.llhip_resolve(ctypes.c_void_p(a)), "the mapping was registered on first use"
claim_a = L.llhip_hbm_claimed()
assert claim_a >= base_claim + size
assert np.array_equal(gemv(a), want["A"]) and L.llhip_hbm_claimed() == claim_a  # resident: no second copy

# the same addresses, another file: the registration follows the mapping
assert libc.munmap(a, size) == 0
b = mapped(os.path.join(tmp, "B"), a, fixed=True)
assert b == a
assert np.array_equal(gemv(b), want["B"])
assert L.llhip_hbm_claimed() == claim_a  # A's copy dropped, B's made

# the same addresses and file, another place in it (C, mapped from offset size + 4096)
assert libc.munmap(b, size) == 0
b = mapped(os.path.join(tmp, "B"), a, fixed=True, offset=size + 4096)
assert b == a
assert np.array_equal(gemv(b), want["C"])
assert L.llhip_hbm_claimed() == claim_a

# the same addresses, anonymous memory holding B's bytes: not a file mapping, so staged, and the copy dropped
assert libc.munmap(b, size) == 0
c = libc.mmap(a, size, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_FIXED, -1, 0)
assert c == a
ctypes.memmove(c, B.ctypes.data, size)
assert np.array_equal(gemv(c), want["B"])
assert not L.llhip_resolve(ctypes.c_void_p(c))
assert L.llhip_hbm_claimed() == base_claim
libc.munmap(c, size)
print("mappings ok", flush=True)
'''


def test_registered_mapping_follows_the_file_mapped_at_its_addresses(tmp_path):
    env = dict(os.environ, LLAMA_HIP_REGISTER_MAPPINGS="1")
    r = subprocess.run([sys.executable, "-c", CHILD, ROOT, str(tmp_path)], env=env, capture_output=True, text=True,
                       timeout=180)
    assert r.returncode == 0 and "mappings ok" in r.stdout, (r.stdout[-2000:], r.stderr[-4000:])
