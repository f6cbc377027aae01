"""Writer of version-3 INT8 (Q8_0) and FP32 checkpoints, the formats engine_load reads (src/runtime.c:179-260 for the header,
src/shards.c:77-99 for the tensor order), and a seeded synthetic model for tests and benchmarks.

Header (256 bytes, little-endian): magic 0x616b3432, version 3, the seven Config ints (dim, hidden_dim, n_layers,
n_heads, n_kv_heads, vocab_size, seq_len), precision (1 = INT8), shared classifier flag, group size, norm_eps,
rope_theta, rope_type, rope_factor, rope_low, rope_high, rope_original, max_seq_len, head_dim, bos/eos/eot/eom ids,
a 128-byte NUL-terminated name, 28 zero bytes. Body: FP32 rms_att[L], rms_ffn[L], rms_final; then each INT8 tensor as
its values followed by its FP32 group scales: the embedding, wq[L], wk[L], wv[L], wo[L], w1[L], w2[L], w3[L], and the
classifier unless it is tied to the embedding."""
import struct

import numpy as np

MAGIC = 0x616B3432
ROLES = ("wq", "wk", "wv", "wo", "w1", "w2", "w3")


def header(cfg, gs, shared, name="synthetic", precision=1):
    """The 256 header bytes of cfg (a dict with the Config fields); precision 1 is INT8 (Q8_0), 0 FP32 (gs 0)."""
    h = struct.pack("<II7iiii", MAGIC, 3, cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["n_heads"],
                    cfg["n_kv_heads"], cfg["vocab_size"], cfg["seq_len"], precision, int(shared), gs)
    # the special tokens must lie in the vocabulary (src/runtime.c:163-166): Llama 3's ids where they fit, else the
    # last ten ids as the reference's synthetic fixtures place them (tests/fixtures.py:88, 95)
    v = cfg["vocab_size"]
    base = v - 10
    ids = (128000, 128001, 128009, -1) if v > 128009 else (base, base + 1, base + 9, base + 8)
    h += struct.pack("<ffifffiiiiiii", cfg.get("norm_eps", 1e-5), cfg.get("rope_theta", 500000.0),
                     cfg.get("rope_type", 0), cfg.get("rope_factor", 1.0), cfg.get("rope_low", 1.0),
                     cfg.get("rope_high", 4.0), cfg.get("rope_original", 8192), cfg.get("max_seq_len", cfg["seq_len"]),
                     cfg["dim"] // cfg["n_heads"], cfg.get("bos_id", ids[0]), cfg.get("eos_id", ids[1]),
                     cfg.get("eot_id", ids[2]), cfg.get("eom_id", ids[3]))
    h += name.encode()[:127].ljust(128, b"\0")
    assert len(h) == 228
    return h + bytes(28)


def quantize_q8(w, gs):
    """Q8_0 of FP32 rows: per group of gs values scale = max|w| / 127, q = round(w / scale) (half away from zero)."""
    g = np.asarray(w, np.float32).reshape(-1, gs)
    scale = (np.abs(g).max(axis=1) / np.float32(127.0)).astype(np.float32)
    safe = np.where(scale > 0, scale, np.float32(1.0))
    r = g / safe[:, None]
    q = (np.sign(r) * np.floor(np.abs(r) + np.float32(0.5))).clip(-127, 127).astype(np.int8)
    return q.reshape(np.shape(w)), scale


def write_q8_v3(path, cfg, gs, norms, tensors, shared=True):
    """Writes a checkpoint. norms: rms_att (L, dim), rms_ffn (L, dim), rms_final (dim,) float32. tensors: "embed" and
    each role of ROLES as (q int8 [L][rows][cols] or [rows][cols] for embed/cls, s float32 with one scale per gs
    values), plus "cls" when not shared."""
    with open(path, "wb") as f:
        f.write(header(cfg, gs, shared))
        for key in ("rms_att", "rms_ffn", "rms_final"):
            f.write(np.ascontiguousarray(norms[key], np.float32).tobytes())

        def put(q, s):
            f.write(np.ascontiguousarray(q, np.int8).tobytes())
            f.write(np.ascontiguousarray(s, np.float32).tobytes())

        put(*tensors["embed"])
        for role in ROLES:
            q, s = tensors[role]
            for layer in range(cfg["n_layers"]):
                put(q[layer], s[layer])
        if not shared:
            put(*tensors["cls"])


def synthetic(cfg, gs, seed, scale=0.05):
    """A seeded random model of cfg: norms near 1, weights ~N(0, scale) quantized to Q8_0. Returns (norms, tensors)."""
    rng = np.random.default_rng(seed)
    d, h, L, v = cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["vocab_size"]
    kv = d // cfg["n_heads"] * cfg["n_kv_heads"]
    norms = {"rms_att": rng.uniform(0.8, 1.2, (L, d)).astype(np.float32),
             "rms_ffn": rng.uniform(0.8, 1.2, (L, d)).astype(np.float32),
             "rms_final": rng.uniform(0.8, 1.2, d).astype(np.float32)}
    shapes = {"wq": (d, d), "wk": (kv, d), "wv": (kv, d), "wo": (d, d), "w1": (h, d), "w2": (d, h), "w3": (h, d)}
    tensors = {"embed": quantize_q8(rng.normal(0, 1.0, (v, d)).astype(np.float32), gs)}
    for role, (rows, cols) in shapes.items():
        q, s = quantize_q8(rng.normal(0, scale, (L, rows, cols)).astype(np.float32), gs)
        tensors[role] = (q, s.reshape(L, rows * cols // gs))
    tensors["cls"] = tensors["embed"]
    return norms, tensors


def file_bytes(cfg, gs, shared=True):
    """The exact size of a version-3 INT8 checkpoint of cfg (src/runtime.c:279-293)."""
    d, h, L, v = cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["vocab_size"]
    kv = d // cfg["n_heads"] * cfg["n_kv_heads"]
    t = lambda n: n + n // gs * 4
    size = 256 + (2 * L + 1) * d * 4 + t(v * d) + L * sum(t(n) for n in (d * d, d * kv, d * kv, d * d, d * h, h * d, d * h))
    return size + (0 if shared else t(v * d))


def write_random_q8_v3(path, cfg, gs, seed, shared=False):
    """A large synthetic checkpoint written tensor by tensor (for benchmarks): uniform int8 values in [-127, 127],
    scales uniform in [1e-4, 2e-4] (weights of magnitude about 0.01), norms near 1."""
    rng = np.random.default_rng(seed)
    d, h, L, v = cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["vocab_size"]
    kv = d // cfg["n_heads"] * cfg["n_kv_heads"]
    with open(path, "wb") as f:
        f.write(header(cfg, gs, shared, name="synthetic-8b"))
        for count in (L * d, L * d, d):
            f.write(rng.uniform(0.8, 1.2, count).astype(np.float32).tobytes())

        def put(count):
            f.write(rng.integers(-127, 128, count, dtype=np.int8).tobytes())
            f.write(rng.uniform(1e-4, 2e-4, count // gs).astype(np.float32).tobytes())

        put(v * d)
        for count in (d * d, kv * d, kv * d, d * d, h * d, d * h, h * d):
            for _ in range(L):
                put(count)
        if not shared:
            put(v * d)


def write_f32_v3(path, cfg, norms, tensors, shared=True):
    """A version-3 FP32 checkpoint (precision 0, group size 0; src/shards.c:60-77 order): the embedding, rms_att[L],
    wq, wk, wv, wo (layers back to back), rms_ffn[L], w1, w2, w3, rms_final, and the classifier unless tied. tensors:
    float32 arrays "embed" [vocab][dim], each role [L][rows][cols], and "cls" when not shared."""
    with open(path, "wb") as f:
        f.write(header(cfg, 0, shared, precision=0))
        put = lambda a: f.write(np.ascontiguousarray(a, np.float32).tobytes())
        put(tensors["embed"])
        put(norms["rms_att"])
        for role in ("wq", "wk", "wv", "wo"):
            put(tensors[role])
        put(norms["rms_ffn"])
        for role in ("w1", "w2", "w3"):
            put(tensors[role])
        put(norms["rms_final"])
        if not shared:
            put(tensors["cls"])


def write_q8_v3_normal(path, cfg, gs, seed, std=0.02, shared=False, name="synthetic-normal"):
    """A large seeded checkpoint of random-init weights: every matrix (the embedding and classifier too) ~N(0, std)
    quantized by the Q8_0 rule of quantize_q8 (scale = max|w| / 127 per group of gs, q = round half away from zero),
    RMSNorm weights 1.0. Tensors are generated and quantized on the GPU when torch has one (seconds for an 8B model),
    else with numpy, and written in file order without holding the model in host memory. Returns the file size."""
    d, h, L, v = cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["vocab_size"]
    kv = d // cfg["n_heads"] * cfg["n_kv_heads"]
    try:
        import torch
        cuda = torch.cuda.is_available()
    except ImportError:
        cuda = False
    if cuda:
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
    else:
        rng = np.random.default_rng(seed)
    chunk = 1 << 26  # values per generated piece (a multiple of every group size used)

    def q8_piece(count):
        if cuda:
            w = torch.randn(count // gs, gs, device="cuda", generator=gen, dtype=torch.float32) * std
            s = w.abs().amax(dim=1) / 127.0
            r = w / torch.where(s > 0, s, torch.ones_like(s))[:, None]
            q = (torch.sign(r) * torch.floor(r.abs() + 0.5)).clamp_(-127, 127).to(torch.int8)
            return q.cpu().numpy().reshape(-1), s.cpu().numpy()
        w = (rng.standard_normal(count, dtype=np.float32) * np.float32(std)).reshape(-1, gs)
        q, s = quantize_q8(w, gs)
        return q.reshape(-1), s

    with open(path, "wb") as f:
        f.write(header(cfg, gs, shared, name=name))
        f.write(np.ones(2 * L * d + d, np.float32).tobytes())

        def put(count):
            # values, then the scales of the whole tensor: pieces are generated once, the scales kept until the end
            scales = []
            for at in range(0, count, chunk):
                q, s = q8_piece(min(chunk, count - at))
                f.write(q.tobytes())
                scales.append(s)
            f.write(np.concatenate(scales).astype(np.float32).tobytes())

        put(v * d)
        for count in (d * d, kv * d, kv * d, d * d, h * d, d * h, h * d):
            for _ in range(L):
                put(count)
        if not shared:
            put(v * d)
    return file_bytes(cfg, gs, shared)


def normal_model(cfg, seed, std=0.02, shared=False):
    """A seeded random-init FP32 model of cfg: every matrix ~N(0, std) (the embedding and the untied classifier
    too), RMSNorm weights 1.0. Returns (norms, tensors) for write_f32_v3; q8_tensors quantizes the same weights."""
    rng = np.random.default_rng(seed)
    d, h, L, v = cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["vocab_size"]
    kv = d // cfg["n_heads"] * cfg["n_kv_heads"]
    norms = {"rms_att": np.ones((L, d), np.float32), "rms_ffn": np.ones((L, d), np.float32),
             "rms_final": np.ones(d, np.float32)}
    shapes = {"wq": (d, d), "wk": (kv, d), "wv": (kv, d), "wo": (d, d), "w1": (h, d), "w2": (d, h), "w3": (h, d)}
    g = lambda *shape: (rng.standard_normal(shape, dtype=np.float32) * np.float32(std))
    tensors = {"embed": g(v, d)}
    for role, (rows, cols) in shapes.items():
        tensors[role] = g(L, rows, cols)
    tensors["cls"] = tensors["embed"] if shared else g(v, d)
    return norms, tensors


def q8_tensors(cfg, tensors, gs):
    """The Q8_0 form of normal_model's tensors, as write_q8_v3 takes them."""
    L = cfg["n_layers"]
    out = {}
    for key, w in tensors.items():
        q, s = quantize_q8(w, gs)
        out[key] = (q, s.reshape(L, -1)) if w.ndim == 3 else (q, s)
    return out
