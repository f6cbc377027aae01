#!/usr/bin/env python3
"""Throughput of the llama3.x.c matmul hot path on one MI355X.

Headline (`value`): Llama-3.1-8B Q8_0 decode, tokens/s of the decode-step matmul set at batch 1: per layer the
activation quantization and the W8A8 GEMVs of QKV (one three-segment launch), Wo (+residual), W1/W3 (SwiGLU) and W2
(+residual), for 32 layers, then the classifier (128256 x 4096); gs = 64. A step is one token's set, replayed from a
HIP graph with every input already in HBM; attention, RMSNorm and RoPE are not part of the set.

Alongside (`prefill`): the 8B INT8 W8A8 prefill of a 2048-token prompt: per layer quantize the 2048 rows and run the
int8-MFMA GEMMs (QKV, Wo + residual, W1/W3 SwiGLU, W2 + residual), then the last row's classifier GEMV.
`decode_1b` and `gemv_2048`: the Llama-3.2-1B decode matmul set and one cold 2048 x 2048 GEMV, launch-amortized.
`forward_decode`: the whole 8B decode token on the device (the embedding row, the matmul set plus RMSNorm, RoPE, the K/V
cache store and attention over 2048 cached positions), also from a HIP graph.
`decode_batch`: one decode step of 4, 16 and 32 sequences through the same matmul set as k_quantize_rows + k_gemm_q8
on that many rows (the short-batch int8 kernel streams each weight matrix once for all of them), classifier included
(`--no-batch` skips it).
`engine`: the engine end to end at the configuration of a Llama-3.1-8B Q8_0 forward (a version-3 checkpoint of
random-init weights written to /dev/shm): a 2048-token prompt through engine_forward_batch, then 256 greedy
engine_forward steps (`--no-engine` skips it; `--engine` runs only it).

Weights ~N(0, 0.02) and activations ~N(0, 1) are drawn on the device (torch, seeded) and quantized by the library's
own k_quantize rule; the data is synthetic. `roofline` is the dominant kernel of the decode step (the SwiGLU GEMV),
its 32 launches captured into one graph and timed with HIP events on the library stream. `cpu_baseline` runs the
reference's own gemm-bench (oracle/_ref, built from the reference's sources) on this host's cores (one socket's
physical cores, read with lscpu): its W8A8 GEMV on the decode shapes and its Q8 GEMM on the 2048-row prefill shapes.
"""
import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "llama3.x.c_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
BF16_PEAK_TFS = 2500.0  # MI355X dense bf16 MFMA
F32_PEAK_TFS = 157.3  # MI355X fp32 matrix

# Llama-3.1-8B
DIM, KV_DIM, HIDDEN, VOCAB, LAYERS, GS = 4096, 1024, 14336, 128256, 32, 64
PROMPT = 2048
BATCH_DEFAULT = 256  # the reference's default prefill batch for Q8_0 (src/engine.c:98)


def q8_bytes(rows, k, gs=GS):
    """Algorithmic bytes of one Q8_0 GEMV: int8 weights, their FP32 scales, the int8 input and its scales, the FP32
    output (read too for the residual kinds is not counted)."""
    return rows * k + rows * (k // gs) * 4 + k + (k // gs) * 4 + rows * 4


def weight_bytes(rows, k, gs=GS):
    return rows * k + rows * (k // gs) * 4


class Model8B:
    """Device-resident Q8_0 weights of the 8B matmul set, drawn and quantized on the GPU."""

    def __init__(self, torch, lh, seed):
        self.torch, self.lh = torch, lh
        L = lh.load()
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
        self.layers = []
        shapes = [("wq", DIM, DIM), ("wk", KV_DIM, DIM), ("wv", KV_DIM, DIM), ("wo", DIM, DIM), ("w1", HIDDEN, DIM),
                  ("w3", HIDDEN, DIM), ("w2", DIM, HIDDEN)]
        total = sum(r * k for _, r, k in shapes) * LAYERS + VOCAB * DIM
        self.q_all = torch.empty(total, dtype=torch.int8, device="cuda")
        self.s_all = torch.empty(total // GS, dtype=torch.float32, device="cuda")
        scratch = torch.empty(VOCAB * DIM, dtype=torch.float32, device="cuda")
        self.cursor = 0

        def make(rows, k):
            n = rows * k
            w = scratch[:n].view(rows, k)
            w.normal_(0.0, 0.02, generator=gen)
            q = self.q_all[self.cursor: self.cursor + n].view(rows, k)
            s = self.s_all[self.cursor // GS: (self.cursor + n) // GS].view(rows, k // GS)
            self.cursor += n
            torch.cuda.synchronize()
            L.k_quantize_rows(q.data_ptr(), s.data_ptr(), w.data_ptr(), k, rows, k, GS)
            L.llhip_synchronize()
            return q, s

        for _ in range(LAYERS):
            self.layers.append({name: make(r, k) for name, r, k in shapes})
        self.cls = make(VOCAB, DIM)
        del scratch
        torch.cuda.synchronize()
        torch.cuda.empty_cache()


def decode_set(torch, lh, model, seed):
    """Buffers and the call sequence of one token's matmul set."""
    L = lh.load()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 1)
    f32 = dict(dtype=torch.float32, device="cuda")
    acts = [{k: torch.randn(n, generator=gen, **f32) for k, n in (("att", DIM), ("o", DIM), ("ffn", DIM),
                                                                    ("h", HIDDEN))} for _ in range(LAYERS)]
    x_cls = torch.randn(DIM, generator=gen, **f32)
    xq_d, xs_d = torch.empty(DIM, dtype=torch.int8, device="cuda"), torch.empty(DIM // GS, **f32)
    xq_h, xs_h = torch.empty(HIDDEN, dtype=torch.int8, device="cuda"), torch.empty(HIDDEN // GS, **f32)
    q, k, v = torch.empty(DIM, **f32), torch.empty(KV_DIM, **f32), torch.empty(KV_DIM, **f32)
    resid, hb, logits = torch.zeros(DIM, **f32), torch.empty(HIDDEN, **f32), torch.empty(VOCAB, **f32)
    torch.cuda.synchronize()
    P = lh.ptr

    def w8(pair):
        return lh.K8Weight(P(pair[0]), P(pair[1]))

    inputs_d, inputs_h = lh.K8Input(P(xq_d), P(xs_d), None), lh.K8Input(P(xq_h), P(xs_h), None)

    def run_step():
        for l, lay in enumerate(model.layers):
            a = acts[l]
            L.k_quantize(P(xq_d), P(xs_d), P(a["att"]), DIM, GS)
            L.k_matmul_q8_qkv(P(q), P(k), P(v), inputs_d, w8(lay["wq"]), w8(lay["wk"]), w8(lay["wv"]), DIM, DIM,
                              KV_DIM, GS)
            L.k_quantize(P(xq_d), P(xs_d), P(a["o"]), DIM, GS)
            L.k_matmul_q8_add(P(resid), inputs_d, w8(lay["wo"]), DIM, DIM, GS)
            L.k_quantize(P(xq_d), P(xs_d), P(a["ffn"]), DIM, GS)
            L.k_matmul_q8_swiglu(P(hb), inputs_d, w8(lay["w1"]), w8(lay["w3"]), DIM, HIDDEN, GS)
            L.k_quantize(P(xq_h), P(xs_h), P(a["h"]), HIDDEN, GS)
            L.k_matmul_q8_add(P(resid), inputs_h, w8(lay["w2"]), HIDDEN, DIM, GS)
        L.k_quantize(P(xq_d), P(xs_d), P(x_cls), DIM, GS)
        L.k_matmul_q8(P(logits), inputs_d, w8(model.cls), DIM, VOCAB, GS)

    return run_step


N_HEADS, N_KV_HEADS, HEAD_DIM = 32, 8, 128
CONTEXT = 2048  # the position the full decode token is measured at (its attention reads 2048 cached positions)


def forward_decode_set(torch, lh, model, seed):
    """One token of the device-resident 8B forward at position CONTEXT - 1, in the reference's decode order
    (src/tp.c:395-432): the token's embedding row (the classifier's Q8_0 table, as a tied model looks it up), per layer
    RMSNorm, quantize + QKV, RoPE, K/V cache store, attention over the cache, quantize +
    Wo (+ residual), RMSNorm, quantize + W1/W3 SwiGLU, quantize + W2 (+ residual); then the final RMSNorm and the
    classifier. Synthetic cache contents, norm weights and rope table; the matmul weights are the decode set's."""
    import ctypes
    L = lh.load()
    P = lh.ptr
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 7)
    f32 = dict(dtype=torch.float32, device="cuda")
    cache = [(torch.randn(CONTEXT * KV_DIM, generator=gen, **f32), torch.randn(CONTEXT * KV_DIM, generator=gen, **f32))
             for _ in range(LAYERS)]
    norms = torch.rand(2 * LAYERS + 1, DIM, generator=gen, **f32) + 0.5
    x, xb, att = torch.randn(DIM, generator=gen, **f32) * 0.1, torch.empty(DIM, **f32), torch.empty(DIM, **f32)
    q, k, v = torch.empty(DIM, **f32), torch.empty(KV_DIM, **f32), torch.empty(KV_DIM, **f32)
    hb, logits = torch.empty(HIDDEN, **f32), torch.empty(VOCAB, **f32)
    xq_d, xs_d = torch.empty(DIM, dtype=torch.int8, device="cuda"), torch.empty(DIM // GS, **f32)
    xq_h, xs_h = torch.empty(HIDDEN, dtype=torch.int8, device="cuda"), torch.empty(HIDDEN // GS, **f32)
    cfg = lh.Config()
    cfg.head_dim, cfg.rope_theta, cfg.rope_type = HEAD_DIM, 500000.0, 1
    cfg.rope_factor, cfg.rope_low, cfg.rope_high, cfg.rope_original = 8.0, 1.0, 4.0, 8192
    table = torch.empty(2 * HEAD_DIM, **f32)
    token = torch.tensor([VOCAB // 3], dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    pos = CONTEXT - 1
    L.k_rope_table(ctypes.byref(cfg), pos, P(table))
    inputs_d, inputs_h = lh.K8Input(P(xq_d), P(xs_d), None), lh.K8Input(P(xq_h), P(xs_h), None)
    assert L.kernels_kv_layout_head() == 1

    def w8(pair):
        return lh.K8Weight(P(pair[0]), P(pair[1]))

    def run_step():
        L.k_embed_q8_rows(P(x), P(model.cls[0]), P(model.cls[1]), P(token), 1, DIM, GS, VOCAB)
        for l, lay in enumerate(model.layers):
            kc, vc = cache[l]
            L.k_rmsnorm(P(xb), P(x), P(norms[2 * l]), DIM, 1e-5)
            L.k_quantize(P(xq_d), P(xs_d), P(xb), DIM, GS)
            L.k_matmul_q8_qkv(P(q), P(k), P(v), inputs_d, w8(lay["wq"]), w8(lay["wk"]), w8(lay["wv"]), DIM, DIM,
                              KV_DIM, GS)
            L.k_rope_apply(P(q), P(k), P(table), N_HEADS, N_KV_HEADS, HEAD_DIM)
            L.k_kv_store(P(kc), P(k), KV_DIM, pos, 1, N_KV_HEADS, HEAD_DIM, CONTEXT)
            L.k_kv_store(P(vc), P(v), KV_DIM, pos, 1, N_KV_HEADS, HEAD_DIM, CONTEXT)
            L.k_attention_kv(P(att), P(q), P(kc), P(vc), None, None, N_HEADS, N_KV_HEADS, HEAD_DIM, CONTEXT, pos)
            L.k_quantize(P(xq_d), P(xs_d), P(att), DIM, GS)
            L.k_matmul_q8_add(P(x), inputs_d, w8(lay["wo"]), DIM, DIM, GS)
            L.k_rmsnorm(P(xb), P(x), P(norms[2 * l + 1]), DIM, 1e-5)
            L.k_quantize(P(xq_d), P(xs_d), P(xb), DIM, GS)
            L.k_matmul_q8_swiglu(P(hb), inputs_d, w8(lay["w1"]), w8(lay["w3"]), DIM, HIDDEN, GS)
            L.k_quantize(P(xq_h), P(xs_h), P(hb), HIDDEN, GS)
            L.k_matmul_q8_add(P(x), inputs_h, w8(lay["w2"]), HIDDEN, DIM, GS)
        L.k_rmsnorm(P(xb), P(x), P(norms[2 * LAYERS]), DIM, 1e-5)
        L.k_quantize(P(xq_d), P(xs_d), P(xb), DIM, GS)
        L.k_matmul_q8(P(logits), inputs_d, w8(model.cls), DIM, VOCAB, GS)

    return run_step, x


def decode_fp_sets(torch, lh, model, seed, steps, warmup):
    """The 8B decode-step matmul set in the two other forms the reference runs (src/gemv.c:141-181 and 252-396):
    W8A32 (runq with LLAMA_Q8_ACTIVATIONS=fp32: the Q8_0 weights above, the FP32 activations handed to the GEMVs
    unquantized) and FP32 (run's k_matmul*: FP32 weights ~N(0, 0.02), 30 GB per token, drawn here and freed after).
    Each is one HIP graph per token, in the decode order of src/tp.c:352-374 / 401-435; tok/s and the algorithmic bytes
    of the step over its time against 8 TB/s."""
    L = lh.load()
    P = lh.ptr
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 9)
    f32 = dict(dtype=torch.float32, device="cuda")
    acts = [{k: torch.randn(n, generator=gen, **f32) for k, n in (("att", DIM), ("o", DIM), ("ffn", DIM),
                                                                    ("h", HIDDEN))} for _ in range(LAYERS)]
    x_cls = torch.randn(DIM, generator=gen, **f32)
    q, k, v = torch.empty(DIM, **f32), torch.empty(KV_DIM, **f32), torch.empty(KV_DIM, **f32)
    resid, hb, logits = torch.zeros(DIM, **f32), torch.empty(HIDDEN, **f32), torch.empty(VOCAB, **f32)
    torch.cuda.synchronize()

    def timed(run_step):
        run_step()
        L.llhip_synchronize()
        assert L.llhip_graph_begin() == 0
        run_step()
        graph = L.llhip_graph_end()
        if not graph:
            raise SystemExit(f"graph capture failed: {lh.last_error()}")
        sec = time_graph(torch, L, graph, steps, warmup) / steps
        L.llhip_graph_destroy(graph)
        return sec

    def w8(pair):
        return lh.K8Weight(P(pair[0]), P(pair[1]))

    def a32(x):
        return lh.K8Input(None, None, P(x))

    def a32_step():
        for lay, a in zip(model.layers, acts):
            L.k_matmul_q8_qkv(P(q), P(k), P(v), a32(a["att"]), w8(lay["wq"]), w8(lay["wk"]), w8(lay["wv"]), DIM, DIM,
                              KV_DIM, GS)
            L.k_matmul_q8_add(P(resid), a32(a["o"]), w8(lay["wo"]), DIM, DIM, GS)
            L.k_matmul_q8_swiglu(P(hb), a32(a["ffn"]), w8(lay["w1"]), w8(lay["w3"]), DIM, HIDDEN, GS)
            L.k_matmul_q8_add(P(resid), a32(a["h"]), w8(lay["w2"]), HIDDEN, DIM, GS)
        L.k_matmul_q8(P(logits), a32(x_cls), w8(model.cls), DIM, VOCAB, GS)

    def a32_bytes(rows, kk):  # weights and scales, the FP32 input, the FP32 output
        return weight_bytes(rows, kk) + 4 * kk + 4 * rows

    a32_sec = timed(a32_step)
    a32_b = LAYERS * (a32_bytes(DIM + 2 * KV_DIM, DIM) + a32_bytes(DIM, DIM) + 2 * weight_bytes(HIDDEN, DIM)
                      + 4 * DIM + 4 * HIDDEN + a32_bytes(DIM, HIDDEN)) + a32_bytes(VOCAB, DIM)
    out = {"w8a32": {"value": round(1 / a32_sec, 2), "unit": "tok/s", "ms_per_token": round(a32_sec * 1e3, 4),
                     "bytes_per_step": a32_b, "hbm_frac": round(a32_b / a32_sec / 1e9 / HBM_PEAK_GBS, 4),
                     "workload": "Llama-3.1-8B Q8_0 decode-step matmul set with FP32 activations (W8A32, "
                                 "LLAMA_Q8_ACTIVATIONS=fp32): 32 x (QKV, Wo +resid, W1/W3 SwiGLU, W2 +resid) + "
                                 "classifier, gs 64, HIP graph"}}
    print(f"# decode W8A32: {a32_sec * 1e3:.3f} ms/token, {a32_b / a32_sec / 1e9:.0f} GB/s", file=sys.stderr,
          flush=True)

    shapes = [("wq", DIM, DIM), ("wk", KV_DIM, DIM), ("wv", KV_DIM, DIM), ("wo", DIM, DIM), ("w1", HIDDEN, DIM),
              ("w3", HIDDEN, DIM), ("w2", DIM, HIDDEN)]
    per_layer = sum(r * c for _, r, c in shapes)
    w_all = torch.empty(per_layer * LAYERS + VOCAB * DIM, **f32)
    w_all.normal_(0.0, 0.02, generator=gen)
    layers, at = [], 0
    for _ in range(LAYERS):
        lay = {}
        for name, r, c in shapes:
            lay[name] = w_all[at: at + r * c]
            at += r * c
        layers.append(lay)
    cls = w_all[at:]
    torch.cuda.synchronize()

    def f32_step():
        for lay, a in zip(layers, acts):
            L.k_matmul_qkv(P(q), P(k), P(v), P(a["att"]), P(lay["wq"]), P(lay["wk"]), P(lay["wv"]), DIM, DIM, KV_DIM)
            L.k_matmul_add(P(resid), P(a["o"]), P(lay["wo"]), DIM, DIM)
            L.k_matmul_swiglu(P(hb), P(a["ffn"]), P(lay["w1"]), P(lay["w3"]), DIM, HIDDEN)
            L.k_matmul_add(P(resid), P(a["h"]), P(lay["w2"]), HIDDEN, DIM)
        L.k_matmul(P(logits), P(x_cls), P(cls), DIM, VOCAB)

    def f32_bytes(rows, kk):
        return 4 * rows * kk + 4 * kk + 4 * rows

    f32_sec = timed(f32_step)
    f32_b = LAYERS * (f32_bytes(DIM + 2 * KV_DIM, DIM) + f32_bytes(DIM, DIM) + 2 * 4 * HIDDEN * DIM + 4 * DIM
                      + 4 * HIDDEN + f32_bytes(DIM, HIDDEN)) + f32_bytes(VOCAB, DIM)
    del w_all, layers, cls
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    out["fp32"] = {"value": round(1 / f32_sec, 2), "unit": "tok/s", "ms_per_token": round(f32_sec * 1e3, 4),
                   "bytes_per_step": f32_b, "hbm_frac": round(f32_b / f32_sec / 1e9 / HBM_PEAK_GBS, 4),
                   "workload": "Llama-3.1-8B FP32 decode-step matmul set (run's k_matmul*, FP32 weights ~N(0, 0.02), "
                               "30 GB per token): 32 x (QKV, Wo +resid, W1/W3 SwiGLU, W2 +resid) + classifier, HIP "
                               "graph"}
    print(f"# decode FP32: {f32_sec * 1e3:.3f} ms/token, {f32_b / f32_sec / 1e9:.0f} GB/s", file=sys.stderr,
          flush=True)
    return out


def time_graph(torch, L, graph, steps, warmup):
    stream = torch.cuda.ExternalStream(L.llhip_stream())
    for _ in range(warmup):
        L.llhip_graph_launch(graph)
    L.llhip_synchronize()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        L.llhip_graph_launch(graph)
    end.record(stream)
    end.synchronize()
    L.llhip_synchronize()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1000.0


def time_per_launch(torch, L, calls, reps=5):
    """Average GPU duration of one launch among `calls`: the calls are captured back to back into one HIP graph, the
    graph is replayed `reps` times between HIP events on the library stream, and the median replay is divided by the
    number of launches (the small gaps between graph nodes are included, so this never flatters the kernel)."""
    L.llhip_synchronize()
    assert L.llhip_graph_begin() == 0
    for call in calls:
        call()
    graph = L.llhip_graph_end()
    if not graph:
        raise SystemExit("graph capture of the roofline launches failed")
    stream = torch.cuda.ExternalStream(L.llhip_stream())
    L.llhip_graph_launch(graph)
    L.llhip_synchronize()
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        L.llhip_graph_launch(graph)
        e1.record(stream)
        e1.synchronize()
        times.append(e0.elapsed_time(e1) / 1000.0)
    L.llhip_synchronize()
    L.llhip_graph_destroy(graph)
    return sorted(times)[len(times) // 2] / len(calls)


def copy_probe(torch, mib, reps=5):
    """A plain copy kernel of known size (torch's elementwise multiply by 1 of `mib` MiB of FP32 into another buffer),
    launched `reps` times: the calibration of the FETCH_SIZE / WRITE_SIZE counters in a --pmc run."""
    n = mib * (1 << 20) // 4
    src, dst = torch.ones(n, device="cuda"), torch.empty(n, device="cuda")
    for _ in range(reps):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    print(f"# copy probe: {reps} x {mib} MiB read + {mib} MiB written", file=sys.stderr, flush=True)


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed counter summary (profiles/traffic.json, written from two
    rocprofv3 --pmc runs of this script, FETCH_SIZE and WRITE_SIZE, scaled by the copy probe); None when absent."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)[kernel]
        return int(rec["fetch_bytes"] + rec["write_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def prefill_set(torch, lh, model, seed):
    L = lh.load()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 2)
    f32 = dict(dtype=torch.float32, device="cuda")
    x_in = torch.randn(PROMPT, DIM, generator=gen, **f32)
    h_in = torch.randn(PROMPT, HIDDEN, generator=gen, **f32)
    xq = torch.empty(PROMPT, HIDDEN, dtype=torch.int8, device="cuda")
    xs = torch.empty(PROMPT, HIDDEN // GS, **f32)
    q, k, v = torch.empty(PROMPT, DIM, **f32), torch.empty(PROMPT, KV_DIM, **f32), torch.empty(PROMPT, KV_DIM, **f32)
    resid, hb = torch.zeros(PROMPT, DIM, **f32), torch.empty(PROMPT, HIDDEN, **f32)
    logits = torch.empty(VOCAB, **f32)
    torch.cuda.synchronize()
    P = lh.ptr

    def w8(pair):
        return lh.K8Weight(P(pair[0]), P(pair[1]))

    def seg(c, pair, n, kind, pair3=None):
        return lh.GemmQ8Segment(P(c), n, w8(pair), w8(pair3) if pair3 else lh.K8Weight(), None, None, n, kind)

    gemms = []  # (callable, ops) of every GEMM launch, for the roofline
    for lay in model.layers:
        qkv = (lh.GemmQ8Segment * 3)(seg(q, lay["wq"], DIM, lh.GEMM_STORE), seg(k, lay["wk"], KV_DIM, lh.GEMM_STORE),
                                     seg(v, lay["wv"], KV_DIM, lh.GEMM_STORE))
        wo = seg(resid, lay["wo"], DIM, lh.GEMM_ADD)
        w13 = seg(hb, lay["w1"], HIDDEN, lh.GEMM_SWIGLU, lay["w3"])
        w2 = seg(resid, lay["w2"], DIM, lh.GEMM_ADD)
        gemms.append((lambda s=qkv: L.k_gemm_q8(P(xq), P(xs), PROMPT, DIM, GS, s, 3), 2 * PROMPT * DIM * (DIM + 2 * KV_DIM)))
        gemms.append((lambda s=wo: L.k_gemm_q8(P(xq), P(xs), PROMPT, DIM, GS, s, 1), 2 * PROMPT * DIM * DIM))
        gemms.append((lambda s=w13: L.k_gemm_q8(P(xq), P(xs), PROMPT, DIM, GS, s, 1), 2 * PROMPT * DIM * HIDDEN * 2))
        gemms.append((lambda s=w2: L.k_gemm_q8(P(xq), P(xs), PROMPT, HIDDEN, GS, s, 1), 2 * PROMPT * HIDDEN * DIM))
    last = lh.K8Input(P(xq), P(xs), None)

    def run():
        for i, (call, _) in enumerate(gemms):
            if i % 4 == 3:
                L.k_quantize_rows(P(xq), P(xs), P(h_in), HIDDEN, PROMPT, HIDDEN, GS)
            else:
                L.k_quantize_rows(P(xq), P(xs), P(x_in), DIM, PROMPT, DIM, GS)
            call()
        # the classifier on the last row only (tp.c:610-618)
        L.k_quantize(P(xq), P(xs), P(x_in[PROMPT - 1]), DIM, GS)
        L.k_matmul_q8(P(logits), last, w8(model.cls), DIM, VOCAB, GS)

    ops = sum(o for _, o in gemms) + 2 * VOCAB * DIM
    return run, gemms, ops


def decode_batch_set(torch, lh, model, seed, m):
    """One decode step of m sequences (a token each) through the 8B matmul set: k_quantize_rows + k_gemm_q8 on m rows
    per projection, the classifier on every row. Below 33 rows k_gemm_q8 streams each weight matrix once for all rows
    (the short-batch kernel), so the step reads the weights once for m tokens."""
    L = lh.load()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 5 + m)
    f32 = dict(dtype=torch.float32, device="cuda")
    x_in, h_in = torch.randn(m, DIM, generator=gen, **f32), torch.randn(m, HIDDEN, generator=gen, **f32)
    xq, xs = torch.empty(m, HIDDEN, dtype=torch.int8, device="cuda"), torch.empty(m, HIDDEN // GS, **f32)
    q, k, v = torch.empty(m, DIM, **f32), torch.empty(m, KV_DIM, **f32), torch.empty(m, KV_DIM, **f32)
    resid, hb, logits = torch.zeros(m, DIM, **f32), torch.empty(m, HIDDEN, **f32), torch.empty(m, VOCAB, **f32)
    torch.cuda.synchronize()
    P = lh.ptr

    def seg(c, pair, n, kind, pair3=None):
        w3 = lh.K8Weight(P(pair3[0]), P(pair3[1])) if pair3 else lh.K8Weight()
        return lh.GemmQ8Segment(P(c), n, lh.K8Weight(P(pair[0]), P(pair[1])), w3, None, None, n, kind)

    calls = []
    for lay in model.layers:
        qkv = (lh.GemmQ8Segment * 3)(seg(q, lay["wq"], DIM, lh.GEMM_STORE), seg(k, lay["wk"], KV_DIM, lh.GEMM_STORE),
                                     seg(v, lay["wv"], KV_DIM, lh.GEMM_STORE))
        calls += [(DIM, x_in, qkv, 3), (DIM, x_in, seg(resid, lay["wo"], DIM, lh.GEMM_ADD), 1),
                  (DIM, x_in, seg(hb, lay["w1"], HIDDEN, lh.GEMM_SWIGLU, lay["w3"]), 1),
                  (HIDDEN, h_in, seg(resid, lay["w2"], DIM, lh.GEMM_ADD), 1)]
    calls.append((DIM, x_in, seg(logits, model.cls, VOCAB, lh.GEMM_STORE), 1))

    def run_step():
        for kdim, src, segs, nseg in calls:
            L.k_quantize_rows(P(xq), P(xs), P(src), kdim, m, kdim, GS)
            L.k_gemm_q8(P(xq), P(xs), m, kdim, GS, segs, nseg)

    return run_step


def decode_batch(torch, lh, model, seed, steps, warmup, sizes=(4, 16, 32)):
    """The batched decode step at several batch sizes: tok/s = m tokens per step, and the weights' bytes per step over
    its time (the activations are a few MB)."""
    L = lh.load()
    step_bytes = LAYERS * (q8_bytes(DIM + 2 * KV_DIM, DIM) + q8_bytes(DIM, DIM) + 2 * weight_bytes(HIDDEN, DIM)
                           + q8_bytes(DIM, HIDDEN)) + q8_bytes(VOCAB, DIM)
    out = {"unit": "tok/s", "workload": "Llama-3.1-8B Q8_0 decode step of m sequences: 32 x (quantize_rows + QKV, "
                                        "Wo +resid, W1/W3 SwiGLU, W2 +resid as k_gemm_q8 on m rows) + classifier on "
                                        "m rows, gs 64, HIP graph", "weight_bytes_per_step": step_bytes}
    for m in sizes:
        run = decode_batch_set(torch, lh, model, seed, m)
        run()
        L.llhip_synchronize()
        assert L.llhip_graph_begin() == 0
        run()
        graph = L.llhip_graph_end()
        if not graph:
            raise SystemExit(f"graph capture of the batched decode failed: {lh.last_error()}")
        sec = time_graph(torch, L, graph, steps, warmup) / steps
        L.llhip_graph_destroy(graph)
        out[f"m{m}"] = {"value": round(m / sec, 1), "ms_per_step": round(sec * 1e3, 4),
                        "weights_gb_s": round(step_bytes / sec / 1e9, 1)}
        print(f"# batched decode, {m} sequences: {sec * 1e3:.3f} ms/step, {m / sec:.0f} tok/s, "
              f"{step_bytes / sec / 1e9:.0f} GB/s of weights", file=sys.stderr, flush=True)
    return out


def prefill_3b(torch, lh, seed, steps=3):
    """The FP32 / BF16 batched-prefill GEMMs on the Llama-3.2-3B shapes: 512 tokens, dim 3072, kv_dim 1024, hidden
    8192, 28 layers of QKV (three segments), Wo (+residual), W1/W3 (SwiGLU) and W2 (+residual). Weights ~N(0, 0.02)
    drawn on the device, BF16 weights packed on the device into the pack_bf16_vnni layout (16-row tiles, K pairs;
    torch's float -> bfloat16 cast rounds to nearest even like bf16_from_f32 for finite values)."""
    L = lh.load()
    T, D, KVD, H, NL = 512, 3072, 1024, 8192, 28
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 3)
    f32 = dict(dtype=torch.float32, device="cuda")
    shapes = [("wq", D, D), ("wk", KVD, D), ("wv", KVD, D), ("wo", D, D), ("w1", H, D), ("w3", H, D), ("w2", D, H)]

    def vnni(w):
        n, k = w.shape
        b = w.to(torch.bfloat16).view(torch.int16).reshape(n // 16, 16, k // 2, 2).permute(0, 2, 1, 3)
        return b.contiguous().reshape(-1)

    layers = []
    for _ in range(NL):
        lay = {}
        for name, n, k in shapes:
            w = torch.empty(n, k, **f32)
            w.normal_(0.0, 0.02, generator=gen)
            lay[name] = (w, vnni(w))
        layers.append(lay)
    x, h = torch.randn(T, D, generator=gen, **f32), torch.randn(T, H, generator=gen, **f32)
    q, kk, v = torch.empty(T, D, **f32), torch.empty(T, KVD, **f32), torch.empty(T, KVD, **f32)
    resid, hb = torch.zeros(T, D, **f32), torch.empty(T, H, **f32)
    panel = lh.AlignedBuffer()
    L.aligned_buffer_alloc(panel, L.k_gemm_bf16_panel_bytes(T, H), 1)
    torch.cuda.synchronize()
    P = lh.ptr
    flops = 2 * T * NL * sum(n * k for _, n, k in shapes)

    def f32seg(c, w, n, k, kind, w3=None):
        return lh.GemmSegment(P(c), n, P(w), P(w3) if w3 is not None else None, k, n, kind)

    def bfseg(c, pw, n, kind, pw3=None):
        return lh.GemmBf16Segment(P(c), n, P(pw), P(pw3) if pw3 is not None else None, n, kind)

    def run(mode):
        for lay in layers:
            if mode == "f32":
                qkv = (lh.GemmSegment * 3)(f32seg(q, lay["wq"][0], D, D, 0), f32seg(kk, lay["wk"][0], KVD, D, 0),
                                           f32seg(v, lay["wv"][0], KVD, D, 0))
                L.k_gemm_f32(P(x), D, T, D, qkv, 3)
                L.k_gemm_f32(P(x), D, T, D, f32seg(resid, lay["wo"][0], D, D, 1), 1)
                L.k_gemm_f32(P(x), D, T, D, f32seg(hb, lay["w1"][0], H, D, 2, lay["w3"][0]), 1)
                L.k_gemm_f32(P(h), H, T, H, f32seg(resid, lay["w2"][0], D, H, 1), 1)
            else:
                qkv = (lh.GemmBf16Segment * 3)(bfseg(q, lay["wq"][1], D, 0), bfseg(kk, lay["wk"][1], KVD, 0),
                                               bfseg(v, lay["wv"][1], KVD, 0))
                L.k_gemm_bf16(P(x), D, T, D, qkv, 3, panel)
                L.k_gemm_bf16(P(x), D, T, D, bfseg(resid, lay["wo"][1], D, 1), 1, panel)
                L.k_gemm_bf16(P(x), D, T, D, bfseg(hb, lay["w1"][1], H, 2, lay["w3"][1]), 1, panel)
                L.k_gemm_bf16(P(h), H, T, H, bfseg(resid, lay["w2"][1], D, 1), 1, panel)

    out = {}
    for mode, peak in (("bf16", BF16_PEAK_TFS), ("f32", F32_PEAK_TFS)):
        run(mode)
        L.llhip_synchronize()
        assert L.llhip_graph_begin() == 0
        run(mode)
        graph = L.llhip_graph_end()
        sec = time_graph(torch, L, graph, steps, 1) / steps
        L.llhip_graph_destroy(graph)
        tf = flops / sec / 1e12
        out[mode] = {"value": round(T / sec, 1), "unit": "tok/s", "ms_per_prompt": round(sec * 1e3, 3),
                     "tflops": round(tf, 1), "peak_tflops": peak, "frac": round(tf / peak, 4)}
        if mode == "f32" and os.environ.get("LLAMA_HIP_F32_FORM", "bf16x3") != "fp32":
            # FP32-accurate products from exact three-part BF16 splits: six BF16 MFMA flops per FP32 flop, so the
            # FP32 rate can pass the FP32 matrix peak; the matrix cores' own use is against the BF16 peak
            out[mode]["mfma"] = {"form": "bf16 x3 parts", "bf16_tflops": round(6 * tf, 1), "bf16_peak": BF16_PEAK_TFS,
                                 "bf16_frac": round(6 * tf / BF16_PEAK_TFS, 4)}
        print(f"# 3B {mode} prefill: {sec * 1e3:.2f} ms/prompt, {T / sec:.0f} tok/s, {tf:.0f} TFLOP/s",
              file=sys.stderr, flush=True)
    L.aligned_buffer_free(panel)
    out["workload"] = ("Llama-3.2-3B FP32 / BF16 batched prefill GEMMs, 512 tokens, 28 layers (QKV, Wo +resid, W1/W3 "
                       "SwiGLU, W2 +resid), FP32 activations")
    out["flops_per_prompt"] = flops
    return out


def decode_1b(torch, lh, seed, steps=50):
    """C2, the Llama-3.2-1B decode-step matmul set (dim 2048, kv_dim 512, hidden 8192, 16 layers, classifier 128256 x
    2048, gs 64: per layer quantize, QKV, Wo +resid, W1/W3 SwiGLU, W2 +resid), replayed from one HIP graph; and C1, one
    2048 x 2048 GEMV (the 1B wq), launch-amortized (64 launches in one graph) and cold: the 64 launches read 64 copies
    of the weights, 286 MB, more than the 256 MB last-level cache. Weights ~N(0, 0.02) quantized by k_quantize_rows,
    activations ~N(0, 1)."""
    L = lh.load()
    D, KVD, H, NL, V = 2048, 512, 8192, 16, 128256
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 5)
    f32 = dict(dtype=torch.float32, device="cuda")
    P = lh.ptr

    def q8(rows, k):
        w = torch.empty(rows, k, **f32)
        w.normal_(0.0, 0.02, generator=gen)
        q = torch.empty(rows, k, dtype=torch.int8, device="cuda")
        s = torch.empty(rows, k // GS, **f32)
        torch.cuda.synchronize()
        L.k_quantize_rows(P(q), P(s), P(w), k, rows, k, GS)
        L.llhip_synchronize()
        return q, s

    shapes = [("wq", D, D), ("wk", KVD, D), ("wv", KVD, D), ("wo", D, D), ("w1", H, D), ("w3", H, D), ("w2", D, H)]
    layers = [{name: q8(r, k) for name, r, k in shapes} for _ in range(NL)]
    cls = q8(V, D)
    acts = [{n: torch.randn(size, generator=gen, **f32) for n, size in (("att", D), ("o", D), ("ffn", D), ("h", H))}
            for _ in range(NL)]
    x_cls = torch.randn(D, generator=gen, **f32)
    xq_d, xs_d = torch.empty(D, dtype=torch.int8, device="cuda"), torch.empty(D // GS, **f32)
    xq_h, xs_h = torch.empty(H, dtype=torch.int8, device="cuda"), torch.empty(H // GS, **f32)
    q, k, v = torch.empty(D, **f32), torch.empty(KVD, **f32), torch.empty(KVD, **f32)
    resid, hb, logits = torch.zeros(D, **f32), torch.empty(H, **f32), torch.empty(V, **f32)
    torch.cuda.synchronize()

    def w8(pair):
        return lh.K8Weight(P(pair[0]), P(pair[1]))

    ind, inh = lh.K8Input(P(xq_d), P(xs_d), None), lh.K8Input(P(xq_h), P(xs_h), None)

    def step():
        for lay, a in zip(layers, acts):
            L.k_quantize(P(xq_d), P(xs_d), P(a["att"]), D, GS)
            L.k_matmul_q8_qkv(P(q), P(k), P(v), ind, w8(lay["wq"]), w8(lay["wk"]), w8(lay["wv"]), D, D, KVD, GS)
            L.k_quantize(P(xq_d), P(xs_d), P(a["o"]), D, GS)
            L.k_matmul_q8_add(P(resid), ind, w8(lay["wo"]), D, D, GS)
            L.k_quantize(P(xq_d), P(xs_d), P(a["ffn"]), D, GS)
            L.k_matmul_q8_swiglu(P(hb), ind, w8(lay["w1"]), w8(lay["w3"]), D, H, GS)
            L.k_quantize(P(xq_h), P(xs_h), P(a["h"]), H, GS)
            L.k_matmul_q8_add(P(resid), inh, w8(lay["w2"]), H, D, GS)
        L.k_quantize(P(xq_d), P(xs_d), P(x_cls), D, GS)
        L.k_matmul_q8(P(logits), ind, w8(cls), D, V, GS)

    step()
    L.llhip_synchronize()
    assert L.llhip_graph_begin() == 0
    step()
    graph = L.llhip_graph_end()
    sec = time_graph(torch, L, graph, steps, 3) / steps
    L.llhip_graph_destroy(graph)
    # the 8B step's accounting (main): QKV as one GEMV of 3072 rows, W1/W3 as two weight streams sharing one input
    per_step = NL * (q8_bytes(D + 2 * KVD, D) + q8_bytes(D, D) + 2 * weight_bytes(H, D) + D + D // GS * 4 + H * 4
                     + q8_bytes(D, H)) + q8_bytes(V, D)
    c2 = {"value": round(1.0 / sec, 1), "unit": "tok/s", "ms_per_token": round(sec * 1e3, 4),
          "bytes_per_step": per_step, "hbm_frac": round(per_step / sec / 1e9 / HBM_PEAK_GBS, 4),
          "workload": "C2: Llama-3.2-1B decode-step matmul set (16 layers of quantize + QKV, Wo +resid, W1/W3 "
                      "SwiGLU, W2 +resid; classifier 128256 x 2048), gs 64, one HIP graph per token"}
    print(f"# 1B decode matmul set: {sec * 1e3:.3f} ms/token, {1 / sec:.0f} tok/s, "
          f"{per_step / sec / 1e9:.0f} GB/s", file=sys.stderr, flush=True)
    del layers, cls
    torch.cuda.empty_cache()
    # C1: the 2048 x 2048 GEMV from cold weights, 64 launches per graph
    copies = [q8(D, D) for _ in range(64)]
    x = torch.randn(D, generator=gen, **f32)
    xq, xs, out = torch.empty(D, dtype=torch.int8, device="cuda"), torch.empty(D // GS, **f32), torch.empty(D, **f32)
    L.k_quantize(P(xq), P(xs), P(x), D, GS)
    L.llhip_synchronize()
    inp = lh.K8Input(P(xq), P(xs), None)
    avg = time_per_launch(torch, L, [lambda c=c: L.k_matmul_q8(P(out), inp, w8(c), D, D, GS) for c in copies], reps=5)
    c1_bytes = q8_bytes(D, D)
    c1 = {"us_per_gemv": round(avg * 1e6, 3), "bytes": c1_bytes, "hbm_frac": round(c1_bytes / avg / 1e9 / HBM_PEAK_GBS, 4),
          "workload": "C1: one 2048 x 2048 Q8_0 GEMV (gs 64, pre-quantized input), 64 launches in one HIP graph over "
                      "64 weight copies (286 MB, beyond the last-level cache)"}
    print(f"# C1 GEMV 2048x2048 cold: {avg * 1e6:.2f} us, {c1_bytes / avg / 1e9:.0f} GB/s", file=sys.stderr, flush=True)
    del copies
    torch.cuda.empty_cache()
    return c2, c1


def host_topology():
    """Sockets, physical cores per socket and logical CPUs of this host (lscpu), and the CPUs this process may use."""
    topo = {"sockets": 1, "cores_per_socket": os.cpu_count() or 1, "threads_per_core": 1,
            "logical_cpus": os.cpu_count() or 1, "model": "?"}
    try:
        out = subprocess.run(["lscpu", "-J"], capture_output=True, text=True, timeout=30).stdout
        fields = {e["field"].rstrip(":"): e["data"] for e in json.loads(out)["lscpu"]}
        topo.update(sockets=int(fields.get("Socket(s)", 1)), cores_per_socket=int(fields.get("Core(s) per socket", 1)),
                    threads_per_core=int(fields.get("Thread(s) per core", 1)),
                    logical_cpus=int(fields.get("CPU(s)", os.cpu_count() or 1)), model=fields.get("Model name", "?"))
    except (OSError, ValueError, KeyError, subprocess.SubprocessError):
        pass
    try:
        topo["usable_cpus"] = len(os.sched_getaffinity(0))
    except AttributeError:
        topo["usable_cpus"] = topo["logical_cpus"]
    return topo


def gemm_bench(exe, threads, args, timeout=600):
    env = dict(os.environ, LLAMA_THREADS=str(threads), LLAMA_BACKEND="teams", LLAMA_KERNELS="auto")
    r = subprocess.run([exe] + args, env=env, capture_output=True, text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError(f"gemm-bench failed ({r.returncode}): {r.stderr[-500:]}")
    return [json.loads(line) for line in r.stdout.splitlines() if line.startswith("{")]


def cpu_baseline(threads=None, budget_s=30.0):
    """The reference's own instrument, gemm-bench (tests/gemm_bench.c, built from its sources into oracle/_ref), on
    this host's cores: the W8A8 GEMV on the five 8B decode shapes with cold weights, scaled to one token (32 x the
    layer set + the classifier), and the W8A8 Q8 GEMM at m = 2048 on the four 8B prefill shapes, scaled to a
    2048-token prompt (32 x the layer; the activation quantization it reports is added). Threads:
    one socket's physical cores (the reference's single-socket configuration), capped by the CPUs this process may
    use. Falls back to the oracle's threaded scalar GEMV when the reference was not built here."""
    topo = host_topology()
    if threads is None:
        threads = max(1, min(topo["cores_per_socket"], topo["usable_cpus"]))
    host = {k: topo[k] for k in ("model", "sockets", "cores_per_socket", "threads_per_core", "logical_cpus",
                                 "usable_cpus")}
    exe = os.path.join(ROOT, "oracle", "_ref", "gemm-bench")
    shapes = [(DIM, DIM), (KV_DIM, DIM), (HIDDEN, DIM), (DIM, HIDDEN), (VOCAB, DIM)]
    per_token = {(DIM, DIM): 2 * LAYERS, (KV_DIM, DIM): 2 * LAYERS, (HIDDEN, DIM): 2 * LAYERS, (DIM, HIDDEN): LAYERS,
                 (VOCAB, DIM): 1}
    if os.path.exists(exe):
        reps = 100  # about 10 s of wall time on 16 host threads
        t0 = time.time()
        med, isa = {}, "?"
        for rec in gemm_bench(exe, threads, ["--kernel", "q8", "--gemv", "--m", "1", "--reps", str(reps),
                                             "--cold-mib", "1200", "--shapes", ",".join(f"{n}x{k}" for n, k in shapes)]):
            if rec["kernel"] == "gemv_rows_q8":
                med[(rec["n"], rec["k"])] = rec["median_s"]
                isa = rec["isa"]
        token_s = sum(med[sh] * c for sh, c in per_token.items())
        decode_wall = time.time() - t0
        # prefill: the Q8 GEMM of a 2048-row batch on QKV (6144 x 4096), Wo, W1 and W3 (14336 x 4096 each), W2
        t0 = time.time()
        pre_shapes = [(DIM + 2 * KV_DIM, DIM), (DIM, DIM), (HIDDEN, DIM), (DIM, HIDDEN)]
        per_layer = {(DIM + 2 * KV_DIM, DIM): 1, (DIM, DIM): 1, (HIDDEN, DIM): 2, (DIM, HIDDEN): 1}
        gmed, quant = {}, {}
        for rec in gemm_bench(exe, threads, ["--kernel", "q8", "--m", str(PROMPT), "--reps", "3", "--shapes",
                                             ",".join(f"{n}x{k}" for n, k in pre_shapes)]):
            if rec["kernel"] == "gemm_q8":
                gmed[(rec["n"], rec["k"])] = rec["median_s"]
                quant[(rec["n"], rec["k"])] = rec.get("quant_median_s", 0.0)
                impl = rec.get("impl", "?")
        # per layer the rows are quantized before QKV, Wo, W1/W3 (once for both) and W2
        layer_s = sum(gmed[sh] * c for sh, c in per_layer.items()) + sum(quant[sh] for sh in pre_shapes)
        prompt_s = LAYERS * layer_s + med[(VOCAB, DIM)]  # plus the last row's classifier GEMV
        ops = 2 * PROMPT * LAYERS * sum(n * k * c for (n, k), c in per_layer.items())
        return {"value": round(1.0 / token_s, 3), "unit": "tok/s", "cores": threads, "kind": "reference",
                "sample": f"reference gemm-bench --kernel q8 --gemv (isa {isa}, {threads} threads, {reps} reps, cold "
                          f"copies over 1200 MiB) on the 8B shapes 4096x4096, 1024x4096, 14336x4096, 4096x14336, "
                          f"128256x4096; per-token time = 32 x (2 wq/wo + 2 wk/wv + 2 w1/w3 + w2) + classifier "
                          f"= {token_s * 1e3:.2f} ms; wall {decode_wall:.1f} s",
                "weight_gbs": round(7973699584 / token_s / 1e9, 1),
                "prefill": {"value": round(PROMPT / prompt_s, 2), "unit": "tok/s", "tops": round(ops / prompt_s / 1e12, 3),
                            "sample": f"reference gemm-bench --kernel q8 --m {PROMPT} ({impl}, {threads} threads, 3 "
                                      f"reps) on 6144x4096, 4096x4096, 14336x4096, 4096x14336; per prompt 32 x "
                                      f"(QKV + Wo + 2 x W1/W3 + W2 + the row quantizations) + the last row's "
                                      f"classifier = {prompt_s:.2f} s; wall {time.time() - t0:.1f} s"},
                "host": host,
                "cores_note": "one socket's physical cores" + (" = all host cores" if threads == topo["logical_cpus"]
                                                               else f" of {topo['logical_cpus']} host CPUs")}
    # fallback: the oracle's scalar GEMV on one 4096x4096 matrix, threaded, scaled to a token by bytes
    import numpy as np

    from oracle import pyoracle as orc

    rng = orc.Rng()
    wq = (rng.uniform(DIM * DIM) * 120).astype(np.int8).reshape(DIM, DIM)
    ws = np.full((DIM, DIM // GS), 0.001, np.float32)
    xq = (rng.uniform(DIM) * 120).astype(np.int8)
    xs = np.full(DIM // GS, 0.01, np.float32)
    out = np.zeros(DIM, np.float32)
    L = orc.lib()
    reps, t0 = 0, time.time()
    while time.time() - t0 < min(budget_s, 10.0):
        L.orc_matmul_q8_threads(orc.ptr(out), orc.ptr(xq), orc.ptr(xs), orc.ptr(wq), orc.ptr(ws), DIM, DIM, GS, threads)
        reps += 1
    per_call = (time.time() - t0) / reps
    token_s = per_call * 7973699584 / weight_bytes(DIM, DIM)
    return {"value": round(1.0 / token_s, 3), "unit": "tok/s", "cores": threads, "kind": "port", "host": host,
            "sample": f"oracle scalar Q8 GEMV 4096x4096 x{reps}, {threads} threads, scaled to the 8B token by bytes"}


def engine_bench(lh, L, args, prompts=None):
    """The engine end to end at the configuration of a Llama-3.1-8B Q8_0 forward: a version-3 checkpoint of random-init
    weights (~N(0, 0.02), RMSNorm weights 1.0, untied classifier, RoPE theta 500000 with Llama 3.1 scaling) written to
    /dev/shm (or $TMPDIR), a 2048-token prompt of random ids through engine_forward_batch (the last row's logits),
    then 256 greedy engine_forward steps from position 2048 (logits to the host and their argmax every step), timed on
    the host clock. Returns the result object; a failure names its stage."""
    prompts = args.prefill_steps if prompts is None else prompts
    decode_steps = 256
    import ctypes
    import shutil
    import tempfile

    import numpy as np

    from llama_hip import checkpoint as ck
    cfg = dict(dim=DIM, hidden_dim=HIDDEN, n_layers=LAYERS, n_heads=N_HEADS, n_kv_heads=N_KV_HEADS, vocab_size=VOCAB,
               seq_len=8192, rope_theta=500000.0, rope_type=1, rope_factor=8.0, rope_low=1.0, rope_high=4.0,
               rope_original=8192)
    base = "/dev/shm" if os.path.isdir("/dev/shm") and shutil.disk_usage("/dev/shm").free > 40 << 30 else None
    stage = "write"
    with tempfile.TemporaryDirectory(dir=base) as tmp:
        path = os.path.join(tmp, "llama8b_q8_normal.bin")
        model = lh.Model()
        try:
            t0 = time.time()
            ck.write_q8_v3_normal(path, cfg, GS, args.seed)
            print(f"# wrote {os.path.getsize(path) / 1e9:.2f} GB checkpoint in {time.time() - t0:.1f} s",
                  file=sys.stderr, flush=True)
            stage = "load"
            t0 = time.time()
            L.engine_load(ctypes.byref(model), path.encode())
            assert model.implementation, lh.last_error()
            print(f"# engine_load (map + upload to HBM) {time.time() - t0:.1f} s", file=sys.stderr, flush=True)
            stage = "prefill"
            rng = np.random.default_rng(args.seed)
            prompt = rng.integers(0, VOCAB, PROMPT).astype(np.int32)
            pptr = prompt.ctypes.data_as(ctypes.c_void_p)
            out = L.engine_forward_batch(ctypes.byref(model), pptr, PROMPT, 0, lh.LOGITS_LAST)  # warm-up
            assert out, lh.last_error()
            t0 = time.perf_counter()
            for _ in range(prompts):
                out = L.engine_forward_batch(ctypes.byref(model), pptr, PROMPT, 0, lh.LOGITS_LAST)
            psec = (time.perf_counter() - t0) / prompts
            assert out, lh.last_error()
            logits = np.ctypeslib.as_array(out, shape=(VOCAB,)).copy()
            assert np.isfinite(logits).all()
            print(f"# engine prefill: {PROMPT} tokens in {psec * 1e3:.2f} ms, {PROMPT / psec:.0f} tok/s",
                  file=sys.stderr, flush=True)
            stage = "prefill with every row's logits"
            out_all = L.engine_forward_batch(ctypes.byref(model), pptr, PROMPT, 0, lh.LOGITS_ALL)  # warm-up (the
            assert out_all, lh.last_error()  # engine pins its host buffer for the batch's logits on the first call)
            t0 = time.perf_counter()
            for _ in range(prompts):
                out_all = L.engine_forward_batch(ctypes.byref(model), pptr, PROMPT, 0, lh.LOGITS_ALL)
            asec = (time.perf_counter() - t0) / prompts
            assert out_all, lh.last_error()
            assert np.isfinite(np.ctypeslib.as_array(out_all, shape=(PROMPT, VOCAB))[-1]).all()
            print(f"# engine prefill with every row's logits ({PROMPT} x {VOCAB} floats to the host): "
                  f"{asec * 1e3:.2f} ms", file=sys.stderr, flush=True)
            stage = "decode"
            t0 = time.perf_counter()
            for step in range(decode_steps):
                out = L.engine_forward(ctypes.byref(model), int(np.argmax(logits)), PROMPT + step)
                assert out, lh.last_error()
                logits = np.ctypeslib.as_array(out, shape=(VOCAB,))
            sec = (time.perf_counter() - t0) / decode_steps
            assert np.isfinite(logits).all()
            print(f"# engine decode: {decode_steps} greedy steps at positions {PROMPT}..{PROMPT + decode_steps - 1}, "
                  f"{sec * 1e3:.3f} ms/token, {1.0 / sec:.1f} tok/s", file=sys.stderr, flush=True)
            # the same prompt in the reference's default batches for Q8_0 (256 rows, src/engine.c:98): a second load
            # with LLAMA_PREFILL_BATCH=256, the prompt in 8 calls, the last row's logits from the last
            stage = "prefill in batches of 256"
            L.engine_free(ctypes.byref(model))
            saved = os.environ.get("LLAMA_PREFILL_BATCH")
            os.environ["LLAMA_PREFILL_BATCH"] = str(BATCH_DEFAULT)
            try:
                L.engine_load(ctypes.byref(model), path.encode())
            finally:
                if saved is None:
                    os.environ.pop("LLAMA_PREFILL_BATCH")
                else:
                    os.environ["LLAMA_PREFILL_BATCH"] = saved
            assert model.implementation and L.engine_max_batch(ctypes.byref(model)) == BATCH_DEFAULT, lh.last_error()

            def batched():
                out = None
                for c in range(0, PROMPT, BATCH_DEFAULT):
                    want = lh.LOGITS_LAST if c + BATCH_DEFAULT >= PROMPT else lh.LOGITS_NONE
                    out = L.engine_forward_batch(ctypes.byref(model), prompt[c:].ctypes.data_as(ctypes.c_void_p),
                                                 BATCH_DEFAULT, c, want)
                assert out, lh.last_error()
                return out
            batched()  # warm-up
            t0 = time.perf_counter()
            for _ in range(prompts):
                out = batched()
            bsec = (time.perf_counter() - t0) / prompts
            assert np.isfinite(np.ctypeslib.as_array(out, shape=(VOCAB,))).all()
            print(f"# engine prefill in batches of {BATCH_DEFAULT}: {bsec * 1e3:.2f} ms, {PROMPT / bsec:.0f} tok/s",
                  file=sys.stderr, flush=True)
        except Exception as e:
            raise RuntimeError(f"engine {stage}: {e}") from e
        finally:
            if model.implementation:
                L.engine_free(ctypes.byref(model))
    return {"metric": "8B Q8_0 engine decode tok/s (engine_forward, logits to host)",
            "value": round(1.0 / sec, 2), "unit": "tok/s", "n_gpus": 1, "steps": decode_steps, "warmup": 0,
            "ms_per_step": round(sec * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "int8 W8A8", "data": "synthetic",
            "config": {"workload": f"Llama-3.1-8B Q8_0 version-3 checkpoint of random-init weights (~N(0, 0.02), "
                                   f"norms 1, untied), {decode_steps} greedy engine_forward steps at positions "
                                   f"{PROMPT}..{PROMPT + decode_steps - 1} after the prompt, logits to the host"},
            "prefill": {"value": round(PROMPT / psec, 1), "unit": "tok/s", "ms_per_prompt": round(psec * 1e3, 3),
                        "workload": f"engine_forward_batch of a {PROMPT}-token prompt of random ids from position 0, "
                                    f"the last row's logits"},
            "prefill_batches": {"value": round(PROMPT / bsec, 1), "unit": "tok/s", "ms_per_prompt": round(bsec * 1e3, 3),
                                "workload": f"the same prompt in the reference's default Q8_0 batches of "
                                            f"{BATCH_DEFAULT} rows (LLAMA_PREFILL_BATCH={BATCH_DEFAULT}, "
                                            f"{PROMPT // BATCH_DEFAULT} calls), the last row's logits"},
            "prefill_all_logits": {"value": round(PROMPT / asec, 1), "unit": "tok/s",
                                   "ms_per_prompt": round(asec * 1e3, 3),
                                   "workload": f"the same prompt with every row's logits ({PROMPT} x {VOCAB} FP32, "
                                               f"1.05 GB) copied to the host"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--prefill-steps", type=int, default=3)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-batch", action="store_true", help="skip the batched decode step (4, 16, 32 sequences)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=None,
                    help="threads of the CPU baseline (default: one socket's physical cores, as lscpu reports them)")
    ap.add_argument("--seed", type=int, default=88172645463325252 % (1 << 31))
    ap.add_argument("--no-1b", action="store_true",
                    help="skip the Llama-3.2-1B decode matmul set and the cold 2048 x 2048 GEMV (C2, C1)")
    ap.add_argument("--no-c3", action="store_true",
                    help="skip the FP32 / BF16 prefill GEMMs on the Llama-3.2-3B shapes (512 tokens)")
    ap.add_argument("--no-forward", action="store_true",
                    help="skip the full device decode token (matmuls + RMSNorm, RoPE, K/V store, attention)")
    ap.add_argument("--no-engine", action="store_true", help="skip the engine's end-to-end measurement")
    ap.add_argument("--no-fp", action="store_true",
                    help="skip the W8A32 and FP32 decode-step matmul sets (the FP32 one draws 30 GB of weights)")
    ap.add_argument("--engine", action="store_true",
                    help="measure engine_load + engine_forward on a synthetic 8B checkpoint instead")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="also launch a plain copy kernel of this many MiB (counter calibration for --pmc runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import llama_hip as lh

    L = lh.load()
    if L.llhip_init() != 0:
        raise SystemExit(f"no usable MI355X: {lh.last_error()}")
    if args.engine:
        print(json.dumps(engine_bench(lh, L, args)), flush=True)
        return
    t_setup = time.time()
    model = Model8B(torch, lh, args.seed)
    run_step = decode_set(torch, lh, model, args.seed)
    print(f"# weights resident: {model.cursor / 1e9:.2f} GB int8 + scales, setup {time.time() - t_setup:.1f} s",
          file=sys.stderr, flush=True)

    # decode: one token's matmul set as a HIP graph
    run_step()
    L.llhip_synchronize()
    assert L.llhip_graph_begin() == 0
    run_step()
    graph = L.llhip_graph_end()
    if not graph:
        raise SystemExit(f"graph capture failed: {lh.last_error()}")
    seconds = time_graph(torch, L, graph, args.steps, args.warmup)
    tok_s = args.steps / seconds
    step_bytes = LAYERS * (q8_bytes(DIM + 2 * KV_DIM, DIM) + q8_bytes(DIM, DIM) + 2 * weight_bytes(HIDDEN, DIM)
                           + DIM + DIM // GS * 4 + HIDDEN * 4 + q8_bytes(DIM, HIDDEN)) + q8_bytes(VOCAB, DIM)
    print(f"# decode: {seconds / args.steps * 1e3:.3f} ms/token, {tok_s:.1f} tok/s, "
          f"{step_bytes / (seconds / args.steps) / 1e9:.0f} GB/s over the step", file=sys.stderr, flush=True)

    # roofline of the dominant kernel: the W1/W3 SwiGLU GEMV with the activation quantization fused in (the launch
    # the step makes: k_quantize followed by k_matmul_q8_swiglu), one launch per layer
    sw_calls = []
    P = lh.ptr
    xq_probe = torch.empty(DIM, dtype=torch.int8, device="cuda")
    xs_probe = torch.empty(DIM // GS, dtype=torch.float32, device="cuda")
    xf = torch.randn(DIM, device="cuda")
    hb = torch.empty(HIDDEN, device="cuda")
    torch.cuda.synchronize()
    inp = lh.K8Input(P(xq_probe), P(xs_probe), None)

    def swiglu(w1, w3):
        L.k_quantize(P(xq_probe), P(xs_probe), P(xf), DIM, GS)
        L.k_matmul_q8_swiglu(P(hb), inp, lh.K8Weight(P(w1[0]), P(w1[1])), lh.K8Weight(P(w3[0]), P(w3[1])), DIM,
                             HIDDEN, GS)

    for lay in model.layers:
        sw_calls.append(lambda w1=lay["w1"], w3=lay["w3"]: swiglu(w1, w3))
    avg = time_per_launch(torch, L, sw_calls)
    # weights and scales of W1 and W3, the FP32 input, the quantized input written back once, the FP32 output
    sw_bytes = 2 * weight_bytes(HIDDEN, DIM) + DIM * 4 + DIM + DIM // GS * 4 + HIDDEN * 4
    achieved = sw_bytes / avg / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic("q8_gemv_swiglu_fused"),
                "kernel": "q8_gemv SwiGLU with fused quantization (W1/W3 2 x 14336x4096, gs 64)",
                "avg_launch_us": round(avg * 1e6, 2), "bytes_per_launch": sw_bytes}
    if args.copy_probe_mib:
        copy_probe(torch, args.copy_probe_mib)

    result = {
        "metric": "8B Q8_0 decode tok/s (%HBM peak); 2048-tok prefill tok/s (%MFMA peak)",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(seconds / args.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 W8A8 (int32 group dots, fp32 scales)", "data": "synthetic",
        "config": {"workload": "Llama-3.1-8B Q8_0 decode-step matmul set, batch 1: 32 x (quantize + QKV 6144x4096, "
                               "Wo 4096x4096 +resid, W1/W3 2x14336x4096 SwiGLU, W2 4096x14336 +resid) + classifier "
                               "128256x4096, gs 64, HIP graph",
                   "algorithmic_bytes_per_step": step_bytes,
                   "step_hbm_frac": round(step_bytes / (seconds / args.steps) / 1e9 / HBM_PEAK_GBS, 4)},
        "roofline": roofline,
    }

    if not args.no_forward:
        # the whole decode token on the device, at position CONTEXT - 1 (graph replays rewrite the same cache slot)
        run_fwd, x_state = forward_decode_set(torch, lh, model, args.seed)
        x0 = x_state.clone()
        run_fwd()
        L.llhip_synchronize()
        assert L.llhip_graph_begin() == 0
        run_fwd()
        fgraph = L.llhip_graph_end()
        if not fgraph:
            raise SystemExit(f"graph capture of the forward token failed: {lh.last_error()}")
        fsteps = max(5, args.steps // 2)
        x_state.copy_(x0)
        fsec = time_graph(torch, L, fgraph, fsteps, 2) / fsteps
        L.llhip_graph_destroy(fgraph)
        result["forward_decode"] = {
            "value": round(1.0 / fsec, 2), "unit": "tok/s", "ms_per_token": round(fsec * 1e3, 4),
            "matmul_share": round((seconds / args.steps) / fsec, 3),
            "workload": f"Llama-3.1-8B Q8_0 decode token on the device at position {CONTEXT - 1}: embedding row, 32 x (RMSNorm, "
                        "quantize + QKV, RoPE, K/V store, attention over the head-major cache, quantize + Wo +resid, "
                        "RMSNorm, quantize + W1/W3 SwiGLU, quantize + W2 +resid) + RMSNorm + classifier, HIP graph"}
        print(f"# device decode token at position {CONTEXT - 1}: {fsec * 1e3:.3f} ms, {1 / fsec:.1f} tok/s",
              file=sys.stderr, flush=True)

    if not args.no_prefill:
        run_prefill, gemms, ops = prefill_set(torch, lh, model, args.seed)
        run_prefill()
        L.llhip_synchronize()
        assert L.llhip_graph_begin() == 0
        run_prefill()
        pgraph = L.llhip_graph_end()
        psec = time_graph(torch, L, pgraph, args.prefill_steps, 1)
        ptok = PROMPT * args.prefill_steps / psec
        # the dominant prefill kernel: the W1/W3 SwiGLU GEMM (2048 x 2 x 14336 x 4096), one launch per layer
        w13 = [c for i, (c, _) in enumerate(gemms) if i % 4 == 2]
        pavg = time_per_launch(torch, L, w13, reps=2)
        w13_ops = 2 * PROMPT * DIM * HIDDEN * 2
        ach = w13_ops / pavg / 1e12
        result["prefill"] = {
            "value": round(ptok, 1), "unit": "tok/s", "ms_per_prompt": round(psec / args.prefill_steps * 1e3, 3),
            "workload": "Llama-3.1-8B INT8 W8A8 prefill, 2048 tokens, 32 layers of quantize_rows + int8-MFMA GEMMs "
                        "(QKV, Wo +resid, W1/W3 SwiGLU, W2 +resid) + last-row classifier GEMV, gs 64",
            "ops_per_prompt": ops, "tops": round(ops / (psec / args.prefill_steps) / 1e12, 1),
            "roofline": {"bound": "mfma", "achieved": round(ach, 1), "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                         "frac": round(ach / INT8_PEAK_TOPS, 4), "traffic": measured_traffic("q8_gemm_w13_2048"),
                         "kernel": "k_gemm_q8 W1/W3 SwiGLU 2048x(2x14336)x4096: q8_gemm_wide_smma over the first "
                                   "12288 columns (768 tiles, three rounds) + q8_gemm_lds over the last 2048",
                         "avg_launch_us": round(pavg * 1e6, 1)},
        }
        L.llhip_graph_destroy(pgraph)
        print(f"# prefill: {psec / args.prefill_steps * 1e3:.2f} ms/prompt, {ptok:.0f} tok/s, "
              f"{ach:.0f} TOP/s in the W1/W3 GEMM", file=sys.stderr, flush=True)
    L.llhip_graph_destroy(graph)

    if not args.no_fp:
        result["decode_w8a32_fp32"] = decode_fp_sets(torch, lh, model, args.seed, max(5, args.steps // 2), 2)
    if not args.no_batch:
        result["decode_batch"] = decode_batch(torch, lh, model, args.seed, max(5, args.steps // 2), 2)
    if not args.no_1b:
        result["decode_1b"], result["gemv_2048"] = decode_1b(torch, lh, args.seed)
    if not args.no_c3:
        result["prefill_3b"] = prefill_3b(torch, lh, args.seed)
    if not args.no_engine:
        # the engine end to end (engine_load of a written 8B checkpoint, engine_forward_batch, engine_forward); its
        # failure (say, no room for the 8.5 GB file) is reported here with its stage and leaves the line above intact
        lh.record_failures()  # a library failure returns with its message instead of ending the process
        try:
            eng = engine_bench(lh, L, args, prompts=2)
            result["engine"] = {"decode": {"value": eng["value"], "unit": "tok/s", "ms_per_token": eng["ms_per_step"],
                                           "workload": eng["config"]["workload"]},
                                "prefill": eng["prefill"], "prefill_all_logits": eng["prefill_all_logits"],
                                "prefill_batches": eng["prefill_batches"]}
        except Exception as err:  # noqa: BLE001 - the main metric must still print
            result["engine"] = {"error": f"{type(err).__name__}: {err}"}
        finally:
            L.llhip_set_fail_mode(lh.LLHIP_FAIL_EXIT)
            L.llhip_clear_error()
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args.cpu_threads)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
