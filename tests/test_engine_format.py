"""The version-3 INT8 checkpoint reader of engine_load (src/runtime.c:179-310, src/shards.c:77-99) on the CPU: the
writer's size agrees with the reference's layout arithmetic, and malformed files fail with the reference's messages
before anything touches the device."""
import ctypes
import os
import struct

import pytest

import llama_hip as lh
from llama_hip import checkpoint as ck

CFG = dict(dim=64, hidden_dim=128, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=96, seq_len=16,
           rope_theta=10000.0)
GS = 32


@pytest.fixture
def record():
    L = lh.load()
    lh.record_failures()
    yield L
    L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
    L.llhip_clear_error()


def write(tmp_path, name="m.bin", shared=True, mutate=None, extra=b"", cut=0):
    norms, t = ck.synthetic(CFG, GS, 5)
    path = os.path.join(tmp_path, name)
    ck.write_q8_v3(path, CFG, GS, norms, t, shared=shared)
    data = bytearray(open(path, "rb").read())
    if mutate:
        mutate(data)
    data = bytes(data[:len(data) - cut]) + extra
    open(path, "wb").write(data)
    return path


def test_writer_size_matches_the_layout(tmp_path):
    """4-byte norms, then values + scales per tensor; 96 x 64 embedding, 2 layers of 7 matrices (kv = 32)."""
    want = 256 + 5 * 64 * 4 + (96 * 64) * 9 // 8 + 2 * (64 * 64 * 2 + 32 * 64 * 2 + 128 * 64 * 3) * 9 // 8
    assert ck.file_bytes(CFG, GS) == want
    assert os.path.getsize(write(tmp_path)) == want
    assert os.path.getsize(write(tmp_path, "u.bin", shared=False)) == want + 96 * 64 * 9 // 8
    h = open(write(tmp_path), "rb").read(256)
    assert struct.unpack_from("<II7i", h) == (0x616B3432, 3, 64, 128, 2, 4, 2, 96, 16)
    assert struct.unpack_from("<iii", h, 36) == (1, 1, GS) and struct.unpack_from("<i", h, 80) == (16,)


@pytest.mark.parametrize("case,message", [
    ("magic", "unsupported attention dimensions"),  # no tag: read as a legacy FP32 header, whose dims do not divide
    ("version", "unsupported checkpoint version 4 for this executable"),
    ("precision", "unsupported checkpoint precision 2"),
    ("fp32_gs", "FP32 checkpoint must have group size zero"),
    ("gs", "unsupported INT8 group size 48: must divide dim and hidden_dim and fit int32 accumulation"),
    ("reserved", "unsupported nonzero reserved checkpoint metadata"),
    ("name", "unterminated model name"),
    ("shared", "invalid classifier flag in"),
    ("dims", "invalid checkpoint dimensions: all seven dimensions must be positive"),
    ("heads", "unsupported attention dimensions: dim must be divisible by heads, heads must be divisible by KV heads, "
              "head size must be even"),
    ("odd_head", "unsupported attention dimensions"),
    ("eps", "invalid RMSNorm, RoPE theta, head dimension or context metadata"),
    ("theta", "invalid RMSNorm, RoPE theta, head dimension or context metadata"),
    ("head_dim", "invalid RMSNorm, RoPE theta, head dimension or context metadata"),
    ("max_seq", "invalid RMSNorm, RoPE theta, head dimension or context metadata"),
    ("rope_type", "unsupported RoPE scaling type 2"),
    ("rope_factor", "invalid RoPE scaling metadata"),
    ("rope_band", "invalid RoPE scaling metadata"),
    ("bos", "invalid special token metadata"),
    ("eom", "invalid special token metadata"),
    ("truncated", "truncated checkpoint"),
    ("trailing", "version 3 checkpoint has unexpected trailing bytes"),
    ("missing", "cannot open checkpoint"),
])
def test_malformed_checkpoints_fail_like_the_reference(tmp_path, record, case, message):
    """Each check of src/runtime.c:147-170 and 179-296, in the reference's order, before the device is touched."""
    L = record
    i32 = lambda off, v: (lambda d: struct.pack_into("<i", d, off, v))
    f32 = lambda off, v: (lambda d: struct.pack_into("<f", d, off, v))
    edits = {"magic": i32(0, 0x12345678), "version": i32(4, 4), "precision": i32(36, 2), "fp32_gs": i32(36, 0),
             "gs": i32(44, 48), "reserved": lambda d: d.__setitem__(240, 1),
             "name": lambda d: d.__setitem__(slice(100, 228), b"x" * 128), "shared": i32(40, 2), "dims": i32(16, 0),
             "heads": i32(20, 3), "odd_head": lambda d: (i32(20, 64)(d), i32(24, 2)(d), i32(80, 1)(d)),
             "eps": f32(48, 0.0), "theta": f32(52, 1.0), "head_dim": i32(80, 8), "max_seq": i32(76, 32),
             "rope_type": i32(56, 2), "rope_factor": f32(60, 0.5), "rope_band": f32(68, 0.5), "bos": i32(84, 96),
             "eom": i32(96, -2)}
    if case == "missing":
        path = os.path.join(tmp_path, "absent.bin")
    else:
        path = write(tmp_path, mutate=edits.get(case), extra=b"\0" * 4 if case == "trailing" else b"",
                     cut=100 if case == "truncated" else 0)
    model = lh.Model()
    L.engine_load(ctypes.byref(model), path.encode())
    assert message in lh.last_error(), (case, lh.last_error())
    assert not model.implementation


@pytest.mark.parametrize("context", [-1, CFG["seq_len"] + 1])
def test_context_beyond_the_checkpoint_fails(tmp_path, record, context):
    """src/engine.c:147-148: a context below zero or above the checkpoint's fails before anything is allocated."""
    L = record
    model = lh.Model()
    L.engine_load_context(ctypes.byref(model), write(tmp_path).encode(), context)
    assert lh.last_error() == "requested context exceeds checkpoint context" and not model.implementation


def test_version2_and_fp32_headers_pass_the_checks(tmp_path, record):
    """The other formats reach the device step (which fails here, on a machine without the GPU, or loads there):
    version 2 INT8 (flag byte at 36, group size at 37), version 3 FP32 (precision 0, group size 0) and the legacy
    FP32 header; and their malformed forms fail with the reference's messages."""
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    from tests.golden import ref_fixtures as rf
    root = rf.create(os.path.join(tmp_path, "fx"), config=(8, 16, 1, 2, 1, 40, 8), gs=4)
    L = record
    for name in ("int8.bin", "fp32.bin"):
        model = lh.Model()
        L.engine_load(ctypes.byref(model), os.path.join(root, name).encode())
        err = lh.last_error()
        assert not any(k in err for k in ("checkpoint", "invalid", "unsupported")), (name, err)
        L.engine_free(ctypes.byref(model))
        L.llhip_clear_error()
    data = bytearray(open(os.path.join(root, "fp32.bin"), "rb").read())
    struct.pack_into("<i", data, 20, -2 ** 31)
    bad = os.path.join(tmp_path, "bad.bin")
    open(bad, "wb").write(data)
    model = lh.Model()
    L.engine_load(ctypes.byref(model), bad.encode())
    assert "invalid vocabulary size in" in lh.last_error() and not model.implementation
    L.llhip_clear_error()
    data = bytearray(open(os.path.join(root, "int8.bin"), "rb").read())
    struct.pack_into("<i", data, 37, 3)  # group size 3 does not divide dim 8
    open(bad, "wb").write(data)
    L.engine_load(ctypes.byref(model), bad.encode())
    assert "unsupported INT8 group size 3" in lh.last_error() and not model.implementation
