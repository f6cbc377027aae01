"""The reference's deterministic synthetic checkpoints, written by code of this repository.

The algorithm is the one of LucianCrainic/llama3.x.c tests/fixtures.py (create at :20-79, upgrade_v3 at :82-114): every
weight value is float32(0.12 * sin(0.71 i + phase)), the norms are 1, the Q8_0 scale of a group is max|w| / 127 taken in
double precision and stored as float32, each value round(w / scale) with round-half-to-even in double precision (0
where the scale is 0). Three files per model:
  fp32.bin   the legacy FP32 layout (28-byte header, a negative vocabulary size for an untied classifier, the unused
             RoPE table of seq x head_dim zeros);
  int8.bin   the version-2 Q8_0 layout (256-byte header: shared flag byte at 36, group size at 37);
and, after upgrade_v3, both rewritten as version 3 (256-byte header with the Llama 3 metadata, no RoPE table).
The reference's own regression numbers (tests/baseline_logits.json, copied beside this file as data) were produced by
its engines on the default CONFIG with group size 2 and a tied classifier; test_reference_fixture_reproduces_baseline
checks that the files written here give those numbers through the reference's probes."""
import math
import struct
from pathlib import Path

import numpy as np

CONFIG = (4, 8, 2, 2, 1, 128010, 32)            # (dim, hidden, layers, heads, kv_heads, vocab, seq): fixtures.py:7
TP_WIDE_CONFIG = (128, 256, 2, 4, 2, 128010, 64)  # fixtures.py:13, with group size 64
MAGIC = 0x616B3432


def floats(n, phase):
    """float32(0.12 * sin(0.71 i + phase)), i < n. math.sin per value, so the doubles are the C library's."""
    return np.fromiter((0.12 * math.sin(i * 0.71 + phase) for i in range(n)), np.float64, n).astype(np.float32)


def quantize(w, gs):
    """Q8_0 in double precision as fixtures.py:56-64 does it: (int8 values, float32 scales)."""
    g = w.astype(np.float64).reshape(-1, gs)
    scale = np.abs(g).max(axis=1) / 127
    safe = np.where(scale > 0, scale, 1.0)
    q = np.where(scale[:, None] > 0, np.round(g / safe[:, None]), 0.0)
    return q.astype(np.int8).reshape(-1), scale.astype(np.float32)


def tensors(config, shared=True):
    """The embedding, then per role (wq, wk, wv, wo, w1, w2, w3) the layers back to back, then the untied classifier."""
    d, h, layers, heads, kvheads, v, seq = config
    kv = d // heads * kvheads
    weights = [floats(v * d, 0.2)]
    for n, phase in [(d * d, 1), (d * kv, 2), (d * kv, 3), (d * d, 4), (d * h, 5), (h * d, 6), (d * h, 7)]:
        for layer in range(layers):
            weights.append(floats(n, phase + layer))
    if not shared:
        cls = np.zeros(v * d, np.float32)
        cls[65 * d:66 * d] = np.tile(np.array([10, -10], np.float32), d // 2)
        weights.append(cls)
    return weights


def create(root, config=None, gs=2, shared=True):
    """fp32.bin (legacy) and int8.bin (version 2) of `config` under root."""
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    config = config or CONFIG
    d, h, layers, heads, kvheads, v, seq = config
    w = tensors(config, shared)
    ones = np.ones(layers * d, np.float32).tobytes()
    with (root / "fp32.bin").open("wb") as f:
        f.write(struct.pack("<7i", d, h, layers, heads, kvheads, v if shared else -v, seq))
        f.write(w[0].tobytes())
        f.write(ones)
        for t in w[1:1 + 4 * layers]:
            f.write(t.tobytes())
        f.write(ones)
        for t in w[1 + 4 * layers:1 + 7 * layers]:
            f.write(t.tobytes())
        f.write(np.ones(d, np.float32).tobytes())
        f.write(bytes(seq * (d // heads) * 4))
        if not shared:
            f.write(w[-1].tobytes())
    with (root / "int8.bin").open("wb") as f:
        head = struct.pack("<Ii7iBi", MAGIC, 2, d, h, layers, heads, kvheads, v, seq, int(shared), gs)
        f.write(head + bytes(256 - len(head)))
        f.write(ones * 2 + np.ones(d, np.float32).tobytes())
        for t in w:
            q, s = quantize(t, gs)
            f.write(q.tobytes())
            f.write(s.tobytes())
    return root


def v3_header(config, precision, gs, shared, epsilon=1e-5, theta=500000.0, scaling=False):
    """fixtures.py:90-96: the version-3 header; the ten special tokens end the vocabulary."""
    d, h, layers, heads, kvheads, vocab, seq = config
    base = vocab - 10
    data = bytearray(256)
    struct.pack_into("<9I", data, 0, MAGIC, 3, *config)
    struct.pack_into("<3I2fI3f3I4i", data, 36, precision, int(shared), gs, epsilon, theta, int(scaling), 32.0, 1.0,
                     4.0, 8192, seq, d // heads, base, base + 1, base + 9, base + 8)
    data[100:116] = b"synthetic-phase2"
    return bytes(data)


def upgrade_v3(root, config=None, gs=2, epsilon=1e-5, theta=500000.0, scaling=False):
    """Rewrites fp32.bin and int8.bin of root as version 3 (fixtures.py:82-106: the legacy RoPE table dropped)."""
    root = Path(root)
    config = config or CONFIG
    d, h, layers, heads, kvheads, vocab, seq = config
    fp = (root / "fp32.bin").read_bytes()
    shared = struct.unpack_from("<i", fp, 20)[0] > 0
    table = seq * (d // heads) * 4
    before = len(fp) - table - (0 if shared else vocab * d * 4)
    payload = fp[28:before] + fp[before + table:]
    (root / "fp32.bin").write_bytes(v3_header(config, 0, 0, shared, epsilon, theta, scaling) + payload)
    quant = (root / "int8.bin").read_bytes()
    (root / "int8.bin").write_bytes(v3_header(config, 1, gs, shared, epsilon, theta, scaling) + quant[256:])
    return root


if __name__ == "__main__":
    import sys

    create(sys.argv[1])
