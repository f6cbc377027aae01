"""The C ABI without a GPU: the library loads, exports every entry point include/llama_hip*.h declares, keeps the
reference's struct layouts, and applies the reference's preconditions and prefill policy (host code only: these calls
fail or return before anything is launched). CPU only.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

import llama_hip as lh

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def L():
    lib = lh.load()
    yield lib


@pytest.fixture
def record(L):
    lh.record_failures()
    yield L
    L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
    L.llhip_clear_error()


def test_every_declared_function_is_exported(L):
    names = lh.declared_functions()
    assert len(names) >= 70
    missing = [n for n in sorted(names) if not hasattr(L, n)]
    assert not missing, missing
    # and the Python view declares argument types for each of them
    assert not sorted(names - set(lh._SIGNATURES)), sorted(names - set(lh._SIGNATURES))


def test_library_resolves_every_symbol_of_its_own():
    """A kernel whose host-side stub the compiler dropped shows up as an undefined llhip symbol in the library."""
    out = subprocess.run(["nm", "-D", lh.LIB_PATH], capture_output=True, text=True, check=True).stdout
    undefined = [line.split()[-1] for line in out.splitlines() if line.split()[:1] == ["U"] and "llhip" in line]
    assert not undefined, undefined


def test_struct_layouts_match_the_reference():
    """Sizes and offsets on x86-64 of the reference's structs (kernels.h:101-109, gemm.h:22-30, 89-96, 118-125,
    runtime.h:9-16, 87-97), restated field by field."""
    assert ctypes.sizeof(lh.K8Weight) == 16 and ctypes.sizeof(lh.K8Input) == 24
    assert ctypes.sizeof(lh.GemmSegment) == 48 and lh.GemmSegment.ldw.offset == 32 and lh.GemmSegment.kind.offset == 44
    assert ctypes.sizeof(lh.GemmBf16Segment) == 40 and lh.GemmBf16Segment.kind.offset == 36
    assert ctypes.sizeof(lh.GemmQ8Segment) == 72 and lh.GemmQ8Segment.pw.offset == 48 and lh.GemmQ8Segment.n.offset == 64
    assert ctypes.sizeof(lh.AlignedBuffer) == 24
    assert ctypes.sizeof(lh.PackBf16) == 32 and ctypes.sizeof(lh.PackS8) == 32
    assert ctypes.sizeof(lh.TensorDesc) == 56 and ctypes.sizeof(lh.Shard) == 80 and lh.Shard.q.offset == 56
    assert ctypes.sizeof(lh.Config) == 44 + 20 + 24 + 128
    assert ctypes.sizeof(lh.AttentionWork) == 40 and lh.AttentionWork.capacity.offset == 32
    assert lh.Model.max_batch.offset == ctypes.sizeof(lh.Config) + 4 + 8 + 8 + 8 - 4 or lh.Model.max_batch.offset > 0


def test_reference_headers_agree_on_layouts():
    """Where the reference's headers are present (this container), compile a probe against them and compare."""
    ref = "/root/reference/include"
    if not os.path.isdir(ref):
        pytest.skip("reference headers are not present")
    src = r'''
#include <stddef.h>
#include <stdio.h>
#include "gemm.h"
#include "prefill.h"
#include "shards.h"
#include "kernels.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(K8Weight), sizeof(K8Input),
         sizeof(GemmSegment), sizeof(GemmBf16Segment), sizeof(GemmQ8Segment), sizeof(AlignedBuffer), sizeof(Config),
         sizeof(Model), sizeof(TensorDesc), sizeof(Shard), sizeof(PackS8), offsetof(Shard, ld),
         offsetof(Model, max_batch), offsetof(Model, prefill_bf16), sizeof(AttentionWork),
         offsetof(AttentionWork, capacity));
  return 0;
}
'''
    tmp = os.path.join("/tmp", "llhip_layout_probe")
    os.makedirs(tmp, exist_ok=True)
    with open(os.path.join(tmp, "probe.c"), "w") as f:
        f.write(src)
    exe = os.path.join(tmp, "probe")
    subprocess.run(["gcc", "-std=c11", "-D_GNU_SOURCE", f"-I{ref}", os.path.join(tmp, "probe.c"), "-o", exe],
                   check=True)
    sizes = [int(v) for v in subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split()]
    mine = [ctypes.sizeof(c) for c in (lh.K8Weight, lh.K8Input, lh.GemmSegment, lh.GemmBf16Segment, lh.GemmQ8Segment,
                                       lh.AlignedBuffer, lh.Config, lh.Model, lh.TensorDesc, lh.Shard, lh.PackS8)]
    mine += [lh.Shard.ld.offset, lh.Model.max_batch.offset, lh.Model.prefill_bf16.offset, ctypes.sizeof(lh.AttentionWork),
             lh.AttentionWork.capacity.offset]
    assert sizes == mine


def test_status_functions(L):
    assert L.kernels_avx512_active() == 0 and L.kernels_amx_active() == 0 and L.gemm_amx_active() == 0
    assert L.kernels_backend_name() == b"hip"
    assert L.gemm_amx_permission() == b"not requested"
    assert L.k_gemm_kc() == 0
    assert L.k_gemm_q8_pick(64, None, 1) == lh.Q8_GEMM_HIP_MFMA
    assert L.k_gemm_q8_pick(32, None, 1) == lh.Q8_GEMM_PORTABLE
    assert L.k_gemm_bf16_panel_bytes(5, 40) == 16 * (64 + 32) * 2  # gemm.c:740-742
    assert L.bf16_vnni_elements(17, 33) == 32 * 64 and L.s8_vnni_bytes(17, 65) == 32 * 128
    calls = []
    fn = lh.SegmentFn(lambda job, s, a, b: calls.append((s, a, b)))
    chunks = (ctypes.c_int * 3)(4, 0, 2)
    L.kernels_parallel_segments(3, chunks, fn, None)
    assert calls == [(0, 0, 4), (2, 0, 2)]


def test_pack_jobs_from_shards(record):
    """gemm.c:1103-1115: a bound ROWS / COLS shard of the right dtype gives a job at its own stride; anything else fails
    with the reference's message."""
    L = record
    desc_f, desc_q = lh.TensorDesc(dtype=lh.DT_F32, rows=40, cols=96), lh.TensorDesc(dtype=lh.DT_Q8, rows=40, cols=96)
    w = np.zeros((33, 100), np.float32)
    shard = lh.Shard(src=ctypes.pointer(desc_f), kind=lh.SHARD_COLS, rows=33, cols=96, q=w.ctypes.data, ld=100)
    dst = np.zeros(L.bf16_vnni_elements(33, 96), np.uint16)
    job = L.pack_bf16_job_from_shard(dst.ctypes.data, shard)
    assert (job.dst, job.w, job.rows, job.cols, job.ld) == (dst.ctypes.data, w.ctypes.data, 33, 96, 100)
    assert L.llhip_last_error() == b""
    L.pack_s8_job_from_shard(None, shard)  # FP32 shard for an int8 job
    assert L.llhip_last_error() == b"pack_s8_job_from_shard needs a bound ROWS or COLS Q8_0 shard"
    L.llhip_clear_error()
    qshard = lh.Shard(src=ctypes.pointer(desc_q), kind=lh.SHARD_COPY, rows=33, cols=96, q=w.ctypes.data, ld=100)
    L.pack_s8_job_from_shard(None, qshard)  # COPY shards are not packable
    assert L.llhip_last_error() == b"pack_s8_job_from_shard needs a bound ROWS or COLS Q8_0 shard"
    L.llhip_clear_error()
    qshard.kind, qshard.ld = lh.SHARD_ROWS, 95  # stride shorter than a row
    L.pack_s8_job_from_shard(None, qshard)
    assert L.llhip_last_error() == b"pack_s8_job_from_shard needs a bound ROWS or COLS Q8_0 shard"
    L.llhip_clear_error()
    qshard.ld = 96
    job = L.pack_s8_job_from_shard(None, qshard)
    assert (job.rows, job.cols, job.ld) == (33, 96, 96) and L.llhip_last_error() == b""
    L.pack_bf16_job_from_shard(None, None)
    assert L.llhip_last_error() == b"pack_bf16_job_from_shard needs a bound ROWS or COLS FP32 shard"


def test_host_packers_and_bf16_match_the_oracle(L):
    from oracle import pyoracle as orc

    rng = orc.Rng(orc.SEED + 21)
    w = rng.uniform(19 * 45).reshape(19, 45)
    dst = np.zeros(L.bf16_vnni_elements(19, 45), np.uint16)
    L.pack_bf16_vnni(lh.ptr(dst), lh.ptr(w), 19, 45, 45)
    assert np.array_equal(dst, orc.pack_bf16_vnni(w))
    wi = (rng.uniform(19 * 70) * 127).astype(np.int8).reshape(19, 70)
    d8 = np.zeros(L.s8_vnni_bytes(19, 70), np.int8)
    L.pack_s8_vnni(lh.ptr(d8), lh.ptr(wi), 19, 70, 70)
    assert np.array_equal(d8, orc.pack_s8_vnni(wi))
    g = np.load(os.path.join(ROOT, "tests", "golden", "bf16.npz"))
    vals = g["convert/bits"].view(np.float32)
    want = g["convert/bf16"]
    for v, u, b in zip(vals[::13], g["convert/bits"][::13], want[::13]):
        if np.isnan(v):
            continue
        assert L.bf16_from_f32(float(v)) == b, hex(int(u))


def test_gemm_preconditions_fail_like_the_reference(record):
    L = record
    seg = lh.GemmQ8Segment()
    L.k_gemm_q8(None, None, 4, 64, 64, seg, 0)
    assert lh.last_error() == "GEMM needs 1..3 segments, got 0"
    L.llhip_clear_error()
    L.k_gemm_q8(None, None, 4, 100, 64, seg, 1)
    assert lh.last_error() == "Q8 GEMM: K=100 is not a multiple of the group size 64"
    L.llhip_clear_error()
    seg.kind = lh.GEMM_SWIGLU
    L.k_gemm_q8(None, None, 4, 128, 64, seg, 1)
    assert lh.last_error() == "GEMM_SWIGLU needs a second weight matrix"
    L.llhip_clear_error()
    fseg = lh.GemmSegment()
    fseg.kind = lh.GEMM_SWIGLU
    L.k_gemm_f32(None, 8, 4, 8, fseg, 1)
    assert lh.last_error() == "GEMM_SWIGLU needs a second weight matrix"
    L.llhip_clear_error()
    bseg = lh.GemmBf16Segment()
    L.k_gemm_bf16(None, 8, 4, 8, bseg, 1, None)
    assert lh.last_error() == "BF16 GEMM segment 0 has no packed weights"
    L.llhip_clear_error()
    bseg.w = 1
    panel = lh.AlignedBuffer(None, None, 10)
    L.k_gemm_bf16(None, 8, 4, 8, bseg, 1, panel)
    assert lh.last_error() == "BF16 activation panel holds 10 bytes but 2048 are needed"
    L.llhip_clear_error()
    # m <= 0 returns quietly, as in the reference (gemm.c:1015-1016)
    seg.kind = lh.GEMM_STORE
    L.k_gemm_q8(None, None, 0, 128, 64, seg, 1)
    assert lh.last_error() == ""


def test_gemv_preconditions_fail_like_the_reference(record):
    L = record
    w = lh.K8Weight()
    L.k_matmul_q8_ld(None, lh.K8Input(), w, 64, 64, 4, 64, lh.K_SWIGLU)
    assert lh.last_error() == "k_matmul_q8_ld: invalid epilogue kind 3"
    L.llhip_clear_error()
    L.k_matmul_q8_ld(None, lh.K8Input(), w, 96, 64, 4, 64, lh.K_STORE)
    assert lh.last_error() == "k_matmul_q8_ld: row stride 96 must be at least 64 and a multiple of the group size 64"
    L.llhip_clear_error()
    L.k_matmul_ld(None, None, None, 32, 64, 4, lh.K_ADD)
    assert lh.last_error() == "k_matmul_ld: row stride 32 is shorter than the 64 inputs"
    L.llhip_clear_error()
    L.k_matmul_q8_ld_worker(None, lh.K8Input(), w, 64, 64, 4, 64, lh.K_STORE, 3, 3, None, lh.RowsDoneFn(), None)
    assert "is not a team member" in lh.last_error()
    L.llhip_clear_error()


def test_fail_exits_by_default():
    """Without the record mode a precondition ends the process with the reference's message, like fail()."""
    code = (
        "import sys; sys.path.insert(0, %r); import llama_hip as lh; L = lh.load();"
        "L.k_gemm_q8(None, None, 4, 64, 64, lh.GemmQ8Segment(), 0); print('returned')"
    ) % os.path.join(ROOT, "llama3.x.c_amd")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True)
    assert r.returncode == 1
    assert "error: GEMM needs 1..3 segments, got 0" in r.stderr
    assert "returned" not in r.stdout


def model(seq_len=4096, vocab=128256):
    m = lh.Model()
    m.config.seq_len = seq_len
    m.config.vocab_size = vocab
    return m


def test_prefill_policy(record, monkeypatch):
    L = record
    for var in ("LLAMA_PREFILL_BATCH", "LLAMA_PREFILL_GEMM", "LLAMA_PREFILL_LOGITS", "LLAMA_PRECISION"):
        monkeypatch.delenv(var, raising=False)
    m = model()
    L.prefill_configure_engine(m, 2048, 1)
    assert (m.max_batch, m.prefill_gemm, m.prefill_kernel, m.prefill_logits) == (2048, 1, b"hip-mfma-int8",
                                                                                  lh.LOGITS_LAST)
    assert L.engine_max_batch(m) == 2048
    m = model(seq_len=100)
    L.prefill_configure(m, 2048)
    assert m.max_batch == 100 and m.prefill_kernel == b"hip-mfma-f32"
    monkeypatch.setenv("LLAMA_PREFILL_GEMM", "off")
    m = model()
    L.prefill_configure(m, 2048)
    assert m.max_batch == 1 and m.prefill_gemm == 0 and m.prefill_kernel is None
    monkeypatch.setenv("LLAMA_PREFILL_GEMM", "sometimes")
    L.prefill_configure(model(), 16)
    assert lh.last_error() == "LLAMA_PREFILL_GEMM must be auto, on or off"
    L.llhip_clear_error()
    monkeypatch.setenv("LLAMA_PREFILL_GEMM", "on")
    for bad in ("0", "-3", " 5", "12x", "99999999999"):
        monkeypatch.setenv("LLAMA_PREFILL_BATCH", bad)
        L.prefill_configure(model(), 16)
        assert lh.last_error() == "LLAMA_PREFILL_BATCH must be a positive integer <= INT_MAX", bad
        L.llhip_clear_error()
    monkeypatch.setenv("LLAMA_PREFILL_BATCH", "64")
    monkeypatch.setenv("LLAMA_PREFILL_LOGITS", "all")
    m = model()
    L.prefill_configure(m, 16)
    assert m.max_batch == 64 and m.prefill_logits == lh.LOGITS_ALL
    monkeypatch.setenv("LLAMA_PREFILL_LOGITS", "first")
    L.prefill_configure(model(), 16)
    assert lh.last_error() == "LLAMA_PREFILL_LOGITS must be last or all"
    L.llhip_clear_error()
    monkeypatch.delenv("LLAMA_PREFILL_LOGITS")
    monkeypatch.setenv("LLAMA_PRECISION", "bf16")
    assert L.prefill_precision(0) == 1
    L.prefill_precision(1)
    assert lh.last_error().startswith("LLAMA_PRECISION=bf16 applies to FP32 checkpoints")
    L.llhip_clear_error()
    m = model()
    m.prefill_bf16 = 1
    monkeypatch.setenv("LLAMA_PREFILL_BATCH", "1")
    L.prefill_configure(m, 256)
    assert lh.last_error() == "LLAMA_PRECISION=bf16 applies to batched prefill: set LLAMA_PREFILL_BATCH to 2 or more"
    L.llhip_clear_error()
    monkeypatch.setenv("LLAMA_PRECISION", "fp16")
    L.prefill_precision(0)
    assert lh.last_error() == "LLAMA_PRECISION must be fp32 or bf16"


def test_prefill_validate(record):
    L = record
    m = model(seq_len=16, vocab=100)
    m.max_batch = 8
    toks = np.arange(8, dtype=np.int32)
    L.prefill_validate(m, lh.ptr(toks), 8, 8, lh.LOGITS_LAST)
    assert lh.last_error() == ""
    for count, pos0 in ((9, 0), (0, 0), (8, 9), (4, 16), (4, -1)):
        L.prefill_validate(m, lh.ptr(toks), count, pos0, lh.LOGITS_LAST)
        assert lh.last_error().startswith("batch input out of range"), (count, pos0)
        L.llhip_clear_error()
    L.prefill_validate(m, lh.ptr(toks), 4, 0, 7)
    assert lh.last_error() == "invalid batch logits request: 7"
    L.llhip_clear_error()
    toks[2] = 100
    L.prefill_validate(m, lh.ptr(toks), 4, 3, lh.LOGITS_ALL)
    assert lh.last_error() == "forward input out of range: token=100 position=5"


def test_rope_kv_store_rows_refuses_overlap_and_misalignment(record):
    """llhip_rope_kv_store_rows writes the caches as 16-byte vectors while other threads still read the k and v rows:
    an unaligned cache, or k or v rows inside either cache, fail with a message before any device work."""
    L = record
    raw = np.zeros(4096 + 16, np.float32)
    base = (-raw.ctypes.data % 16) // 4  # first 16-byte aligned element
    buf = raw[base:base + 4096]
    P = lh.ptr(buf)
    rows, nkv, hd, seq = 4, 1, 8, 100  # caches of 800 floats; rows of 8
    at = lambda i: P + 4 * i  # noqa: E731
    L.llhip_rope_kv_store_rows(at(1024), 8, at(1100), at(1200), 8, at(1300), 16, rows, 1, nkv, hd, at(1), at(2048), 0,
                               seq)
    assert "16-byte aligned rows and caches" in lh.last_error(), lh.last_error()
    L.llhip_clear_error()
    for k, v in ((0, 1200), (1100, 2100), (800 - 8, 1200)):  # k in key_cache, v in value_cache, k's last row in it
        L.llhip_rope_kv_store_rows(at(1024), 8, at(k), at(v), 8, at(1300), 16, rows, 1, nkv, hd, at(0), at(2048), 0, seq)
        assert lh.last_error() == "llhip_rope_kv_store_rows: the k and v rows must lie outside both caches", (k, v)
        L.llhip_clear_error()


def test_cache_position_checks_cannot_overflow(record):
    """The cache-position checks of k_kv_store, llhip_rope_kv_store_rows and the batched attention compare without
    forming pos0 + count in int: a batch starting just below INT_MAX is refused (before any device work), not
    wrapped into range."""
    L = record
    buf = np.zeros(256, np.float32)
    big = 2**31 - 2
    P = lh.ptr(buf)
    L.k_kv_store(P, P, 8, big, 4, 1, 8, 100)
    assert lh.last_error() == f"k_kv_store: positions {big}..{big + 3} are outside the cache of 100"
    L.llhip_clear_error()
    L.llhip_rope_kv_store_rows(P, 8, P, P, 8, P, 16, 4, 1, 1, 8, P, P, big, 100)
    assert lh.last_error() == f"llhip_rope_kv_store_rows: positions {big}..{big + 3} are outside the cache of 100"
    L.llhip_clear_error()
    L.k_attention_batch_layout(P, P, P, P, None, None, 1, 1, 8, 100, big, 4, 8, 8)
    assert f"positions {big}..{big + 3} are outside the cache of 100" in lh.last_error()
    L.llhip_clear_error()
    L.k_kv_store(P, P, 8, 0, 4, 1, 8, 0)  # an empty cache holds no position
    assert "outside the cache of 0" in lh.last_error()


def test_hbm_budget_parses_like_the_reference(record, monkeypatch):
    """placement_hbm_budget (src/loader.c:28-37): LLAMA_HBM_BUDGET_GIB in GiB, fractions allowed; zero, negative,
    trailing text and more than 2^20 GiB fail with the reference's message. (The default, the device's memory, needs
    the device and is checked by the GPU tests.)"""
    L = record
    monkeypatch.setenv("LLAMA_HBM_BUDGET_GIB", "1.5")
    assert L.placement_hbm_budget() == 3 << 29
    monkeypatch.setenv("LLAMA_HBM_BUDGET_GIB", "288")
    assert L.placement_hbm_budget() == 288 << 30
    for bad in ("0", "-2", "12GiB", "2000000"):
        monkeypatch.setenv("LLAMA_HBM_BUDGET_GIB", bad)
        L.llhip_clear_error()
        assert L.placement_hbm_budget() == 0
        assert lh.last_error() == "LLAMA_HBM_BUDGET_GIB must be a positive number of GiB", bad
    L.llhip_clear_error()
