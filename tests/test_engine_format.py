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
    ("magic", "unsupported INT8 checkpoint: expected ak42 version 2 or 3"),
    ("version", "unsupported checkpoint version 4 for this executable"),
    ("precision", "checkpoint precision requires run executable"),
    ("gs", "unsupported INT8 group size 48: must divide dim and hidden_dim and fit int32 accumulation"),
    ("reserved", "unsupported nonzero reserved checkpoint metadata"),
    ("truncated", "truncated checkpoint"),
    ("trailing", "version 3 checkpoint has unexpected trailing bytes"),
    ("missing", "cannot open checkpoint"),
])
def test_malformed_checkpoints_fail_like_the_reference(tmp_path, record, case, message):
    L = record
    edits = {"magic": lambda d: struct.pack_into("<I", d, 0, 0x12345678),
             "version": lambda d: struct.pack_into("<i", d, 4, 4),
             "precision": lambda d: struct.pack_into("<i", d, 36, 0),
             "gs": lambda d: struct.pack_into("<i", d, 44, 48),
             "reserved": lambda d: d.__setitem__(240, 1)}
    if case == "missing":
        path = os.path.join(tmp_path, "absent.bin")
    else:
        path = write(tmp_path, mutate=edits.get(case), extra=b"\0" * 4 if case == "trailing" else b"",
                     cut=100 if case == "truncated" else 0)
    model = lh.Model()
    L.engine_load(ctypes.byref(model), path.encode())
    assert message in lh.last_error(), (case, lh.last_error())
    assert not model.implementation
