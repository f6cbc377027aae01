// The reference-named C entry points of the matmul hot path: argument checks with the reference's failure messages,
// pointer residency, then one launch per call. Citations are LucianCrainic/llama3.x.c file:line.
#include <cstring>

#include "common.h"

using namespace llhip;

namespace {

// ---- activation quantization (src/gemv.c:589-624, src/gemm.c:819-830) --------------------------------------------

void quantize_rows(const char *name, int8_t *q, float *s, const float *x, size_t ldx, int m, int n, int gs) {
  if (gs <= 0) {
    raise("%s: group size %d must be positive", name, gs);
    return;
  }
  const int groups = n / gs;
  if (m <= 0 || groups <= 0)
    return;
  if (!q || !s || !x) {
    raise("%s: null buffer", name);
    return;
  }
  Call call(name, true); // a recorded k_rmsnorm of x may be taken along
  const size_t used = (size_t)groups * gs;
  Ref X = call.in2d(x, used * sizeof(float), ldx * sizeof(float), (size_t)m);
  Ref Q = call.out2d(q, used, (size_t)n, (size_t)m, false);
  Ref S = call.out(s, (size_t)m * groups * sizeof(float), false);
  if (!call.ready())
    return;
  if (m == 1 && !call.staged() && quantize_fusion_enabled() && n % gs == 0) {
    // one device-resident row: the next GEMV reading (q, s) quantizes it (and normalizes it, when a k_rmsnorm of
    // this row was recorded) in its prologue
    defer_quantize(PendingQuantize{call.ptr<int8_t>(Q), call.ptr<float>(S), call.ptr<const float>(X), n, gs, nullptr,
                                   nullptr, 0.0f});
    return;
  }
  if (!flush_pending_quantize())
    return;
  QuantizeJob job{call.ptr<int8_t>(Q), call.ptr<float>(S), call.ptr<const float>(X), ldx, m, n, gs};
  if (launch_quantize(job, call.stream()))
    call.finish();
}

// ---- the Q8 GEMV drivers (src/gemv.c:441-528, 565-587) ----------------------------------------------------------

struct Q8Member {
  float *out;
  K8Weight w, w3;
  int d;
};

void q8_gemv(const char *name, const Q8Member *members, int count, const K8Input *x, int n, size_t ld, int gs,
             Epilogue epi, int32_t *probe = nullptr) {
  if (!x) {
    raise("%s: null input", name);
    return;
  }
  if (gs <= 0) {
    raise("%s: group size %d must be positive", name, gs);
    return;
  }
  if (ld == 0)
    ld = (size_t)n;
  const bool w8a8 = x->q != nullptr;
  if (!w8a8 && !x->f) {
    raise("%s: the input has neither quantized values nor FP32 activations", name);
    return;
  }
  int total = 0;
  for (int i = 0; i < count; i++)
    total += members[i].d > 0 ? members[i].d : 0;
  const int groups = n / gs;
  if (total <= 0)
    return;
  Call call(name, true);
  const size_t used = (size_t)(groups > 0 ? groups : 0) * gs;
  const size_t sld = ld / (size_t)gs;
  Ref XQ, XS, XF;
  if (w8a8) {
    XQ = call.in(x->q, used);
    XS = call.in(x->s, (size_t)groups * sizeof(float));
  } else {
    XF = call.in(x->f, used * sizeof(float));
  }
  Ref WQ[3], WS[3], W3Q[3], W3S[3], OUT[3];
  for (int i = 0; i < count; i++) {
    const Q8Member &mb = members[i];
    if (mb.d <= 0)
      continue;
    WQ[i] = call.in2d(mb.w.q, used, ld, (size_t)mb.d);
    WS[i] = call.in2d(mb.w.s, (size_t)groups * sizeof(float), sld * sizeof(float), (size_t)mb.d);
    if (epi == EPI_SWIGLU) {
      W3Q[i] = call.in2d(mb.w3.q, used, ld, (size_t)mb.d);
      W3S[i] = call.in2d(mb.w3.s, (size_t)groups * sizeof(float), sld * sizeof(float), (size_t)mb.d);
    }
    OUT[i] = call.out(mb.out, (size_t)mb.d * sizeof(float), epi == EPI_ADD);
  }
  if (!call.ready())
    return;
  GemvJob job{};
  int nseg = 0;
  for (int i = 0; i < count; i++) {
    if (members[i].d <= 0)
      continue;
    job.seg[nseg++] = GemvSegment{call.ptr<float>(OUT[i]),        call.ptr<const int8_t>(WQ[i]),
                                  call.ptr<const float>(WS[i]),   call.ptr<const int8_t>(W3Q[i]),
                                  call.ptr<const float>(W3S[i]), members[i].d};
  }
  job.nseg = nseg;
  job.xq = call.ptr<const int8_t>(XQ);
  job.xs = call.ptr<const float>(XS);
  job.xf = call.ptr<const float>(XF);
  job.n = groups * gs;
  job.gs = gs;
  job.ld = ld;
  job.epi = epi;
  job.probe = probe;
  PendingQuantize pq;
  if (w8a8 && take_pending_quantize(x->q, x->s, job.n, gs, &pq)) {
    GemvJob fused = job;
    fused.xf_quantize = true;
    fused.xf = pq.x;
    fused.xq_out = pq.q;
    fused.xs_out = pq.s;
    fused.xq = nullptr;
    fused.xs = nullptr;
    fused.norm_w = pq.norm_w;
    fused.norm_out = pq.norm_out;
    fused.norm_eps = pq.norm_eps;
    if (gemv_fast_path(fused)) {
      if (launch_q8_gemv(fused, call.stream()))
        call.finish();
      return;
    }
    // not a shape the fused kernel takes: normalize and quantize first, as recorded
    if (!launch_pending_quantize(pq, call.stream()))
      return;
  } else if (!flush_pending_quantize()) {
    return;
  }
  if (launch_q8_gemv(job, call.stream()))
    call.finish();
}

Epilogue ld_kind(int kind, const char *name, bool *ok) {
  *ok = true;
  if (kind == K_STORE || kind == K_PARTIAL)
    return EPI_STORE;
  if (kind == K_ADD)
    return EPI_ADD;
  *ok = raise("%s: invalid epilogue kind %d", name, kind); // src/gemv.c:533-536
  return EPI_STORE;
}

bool worker_share(const char *name, int d, int worker, int workers, int *r0, int *r1) {
  if (workers < 1 || worker < 0 || worker >= workers)
    return raise("%s: member %d of %d is not a team member", name, worker, workers);
  *r0 = (int)((long long)d * worker / workers); // the static split of src/gemv.c:488-495
  *r1 = (int)((long long)d * (worker + 1) / workers);
  return true;
}

// ---- FP32 GEMV (src/gemv.c:252-396, 538-564) -------------------------------------------------------------------

struct F32Member {
  float *out;
  const float *w, *w3;
  int d;
};

void f32_gemv(const char *name, const F32Member *members, int count, const float *x, int n, size_t ld, Epilogue epi) {
  if (ld == 0)
    ld = (size_t)n;
  int total = 0;
  for (int i = 0; i < count; i++)
    total += members[i].d > 0 ? members[i].d : 0;
  if (total <= 0)
    return;
  if (!x) {
    raise("%s: null input", name);
    return;
  }
  Call call(name);
  const size_t nn = n > 0 ? (size_t)n : 0;
  Ref X = call.in(x, nn * sizeof(float));
  Ref W[3], W3[3], OUT[3];
  for (int i = 0; i < count; i++) {
    if (members[i].d <= 0)
      continue;
    W[i] = call.in2d(members[i].w, nn * sizeof(float), ld * sizeof(float), (size_t)members[i].d);
    if (epi == EPI_SWIGLU)
      W3[i] = call.in2d(members[i].w3, nn * sizeof(float), ld * sizeof(float), (size_t)members[i].d);
    OUT[i] = call.out(members[i].out, (size_t)members[i].d * sizeof(float), epi == EPI_ADD);
  }
  if (!call.ready())
    return;
  F32GemvJob job{};
  int nseg = 0;
  for (int i = 0; i < count; i++)
    if (members[i].d > 0)
      job.seg[nseg++] = F32GemvSegment{call.ptr<float>(OUT[i]), call.ptr<const float>(W[i]),
                                       call.ptr<const float>(W3[i]), members[i].d};
  job.nseg = nseg;
  job.x = call.ptr<const float>(X);
  job.n = (int)nn;
  job.ld = ld;
  job.epi = epi;
  if (launch_f32_gemv(job, call.stream()))
    call.finish();
}

// ---- GEMM segments (src/gemm.c:171-191, 744-771, 1006-1029) -----------------------------------------------------

Epilogue gemm_epilogue(GemmKind kind) {
  return kind == GEMM_ADD ? EPI_ADD : kind == GEMM_SWIGLU ? EPI_SWIGLU : EPI_STORE;
}

bool check_count(int count) {
  if (count < 1 || count > GEMM_MAX_SEGMENTS)
    return raise("GEMM needs 1..%d segments, got %d", GEMM_MAX_SEGMENTS, count);
  return true;
}

void gemm_q8(const char *name, bool mfma, const int8_t *xq, const float *xs, int m, int k, int gs,
             const GemmQ8Segment *segments, int count) {
  if (!check_count(count))
    return;
  if (gs <= 0 || k % gs)
    return (void)raise("Q8 GEMM: K=%d is not a multiple of the group size %d", k, gs);
  for (int s = 0; s < count; s++)
    if (segments[s].kind == GEMM_SWIGLU && !segments[s].w3.q)
      return (void)raise("GEMM_SWIGLU needs a second weight matrix");
  if (m <= 0 || k <= 0)
    return;
  const int groups = k / gs;
  Call call(name);
  Ref XQ = call.in(xq, (size_t)m * k);
  Ref XS = call.in(xs, (size_t)m * groups * sizeof(float));
  Ref W[3], WS[3], W3[3], W3S[3], C[3];
  for (int s = 0; s < count; s++) {
    const GemmQ8Segment &g = segments[s];
    if (g.n <= 0)
      continue;
    W[s] = call.in(g.w.q, (size_t)g.n * k);
    WS[s] = call.in(g.w.s, (size_t)g.n * groups * sizeof(float));
    if (g.kind == GEMM_SWIGLU) {
      W3[s] = call.in(g.w3.q, (size_t)g.n * k);
      W3S[s] = call.in(g.w3.s, (size_t)g.n * groups * sizeof(float));
    }
    C[s] = call.out2d(g.c, (size_t)g.n * sizeof(float), (size_t)g.ldc * sizeof(float), (size_t)m, g.kind == GEMM_ADD);
  }
  if (!call.ready())
    return;
  GemmQ8Job job{};
  int nseg = 0;
  for (int s = 0; s < count; s++) {
    const GemmQ8Segment &g = segments[s];
    if (g.n <= 0)
      continue;
    job.seg[nseg++] = GemmSegmentDev{call.ptr<float>(C[s]),        g.ldc,          call.ptr<const void>(W[s]),
                                     call.ptr<const void>(W3[s]),  call.ptr<const float>(WS[s]),
                                     call.ptr<const float>(W3S[s]), (size_t)k,     g.n,
                                     gemm_epilogue(g.kind)};
  }
  if (!nseg)
    return (void)call.finish();
  job.nseg = nseg;
  job.xq = call.ptr<const int8_t>(XQ);
  job.xs = call.ptr<const float>(XS);
  job.m = m;
  job.k = k;
  job.gs = gs;
  bool aligned = ((uintptr_t)job.xq & 15) == 0;
  for (int s = 0; s < nseg; s++)
    aligned = aligned && ((uintptr_t)job.seg[s].w & 15) == 0 && ((uintptr_t)job.seg[s].w3 & 15) == 0;
  const bool ok = mfma && aligned && q8_gemm_fast_path(job.xq, m, k, gs) ? launch_q8_gemm(job, call.stream())
                                                                          : launch_q8_gemm_generic(job, call.stream());
  if (ok)
    call.finish();
}

void gemm_f32(const char *name, const float *a, int lda, int m, int k, const GemmSegment *segments, int count) {
  if (!check_count(count))
    return;
  for (int s = 0; s < count; s++)
    if (segments[s].kind == GEMM_SWIGLU && !segments[s].w3)
      return (void)raise("GEMM_SWIGLU needs a second weight matrix");
  if (m <= 0 || k <= 0)
    return;
  Call call(name);
  Ref A = call.in2d(a, (size_t)k * sizeof(float), (size_t)lda * sizeof(float), (size_t)m);
  Ref W[3], W3[3], C[3];
  for (int s = 0; s < count; s++) {
    const GemmSegment &g = segments[s];
    if (g.n <= 0)
      continue;
    W[s] = call.in2d(g.w, (size_t)k * sizeof(float), g.ldw * sizeof(float), (size_t)g.n);
    if (g.kind == GEMM_SWIGLU)
      W3[s] = call.in2d(g.w3, (size_t)k * sizeof(float), g.ldw * sizeof(float), (size_t)g.n);
    C[s] = call.out2d(g.c, (size_t)g.n * sizeof(float), (size_t)g.ldc * sizeof(float), (size_t)m, g.kind == GEMM_ADD);
  }
  if (!call.ready())
    return;
  GemmF32Job job{};
  int nseg = 0;
  for (int s = 0; s < count; s++) {
    const GemmSegment &g = segments[s];
    if (g.n <= 0)
      continue;
    job.seg[nseg++] = GemmSegmentDev{call.ptr<float>(C[s]), g.ldc,    call.ptr<const void>(W[s]), call.ptr<const void>(W3[s]),
                                     nullptr,               nullptr, g.ldw,                      g.n,
                                     gemm_epilogue(g.kind)};
  }
  if (!nseg)
    return (void)call.finish();
  job.nseg = nseg;
  job.a = call.ptr<const float>(A);
  job.lda = lda;
  job.m = m;
  job.k = k;
  job.bf16 = false;
  if (launch_f32_gemm(job, call.stream()))
    call.finish();
}

} // namespace

extern "C" {

void k_quantize(int8_t *q, float *s, const float *x, int n, int gs) {
  quantize_rows("k_quantize", q, s, x, (size_t)(n > 0 ? n : 0), 1, n, gs);
}

void k_quantize_rows(int8_t *q, float *s, const float *x, size_t ldx, int m, int n, int gs) {
  quantize_rows("k_quantize_rows", q, s, x, ldx, m, n, gs);
}

void k_matmul_q8(float *out, const K8Input *x, K8Weight w, int n, int d, int gs) {
  Q8Member m{out, w, {nullptr, nullptr}, d};
  q8_gemv("k_matmul_q8", &m, 1, x, n, 0, gs, EPI_STORE);
}

void k_matmul_q8_add(float *out, const K8Input *x, K8Weight w, int n, int d, int gs) {
  Q8Member m{out, w, {nullptr, nullptr}, d};
  q8_gemv("k_matmul_q8_add", &m, 1, x, n, 0, gs, EPI_ADD);
}

void k_matmul_q8_qkv(float *q, float *k, float *v, const K8Input *x, K8Weight wq, K8Weight wk, K8Weight wv, int n,
                     int dq, int dkv, int gs) {
  Q8Member m[3] = {{q, wq, {nullptr, nullptr}, dq}, {k, wk, {nullptr, nullptr}, dkv}, {v, wv, {nullptr, nullptr}, dkv}};
  q8_gemv("k_matmul_q8_qkv", m, 3, x, n, 0, gs, EPI_STORE);
}

void k_matmul_q8_swiglu(float *out, const K8Input *x, K8Weight w1, K8Weight w3, int n, int d, int gs) {
  if (!w3.q)
    return (void)raise("k_matmul_q8_swiglu: the SwiGLU gate needs w3");
  Q8Member m{out, w1, w3, d};
  q8_gemv("k_matmul_q8_swiglu", &m, 1, x, n, 0, gs, EPI_SWIGLU);
}

void k_matmul_q8_ld(float *out, const K8Input *x, const K8Weight *w, size_t ld, int n, int d, int gs, int kind) {
  bool ok;
  Epilogue epi = ld_kind(kind, "k_matmul_q8_ld", &ok);
  if (!ok)
    return;
  if (gs <= 0 || ld < (size_t)n || ld % (size_t)gs) // src/gemv.c:567-568
    return (void)raise("k_matmul_q8_ld: row stride %zu must be at least %d and a multiple of the group size %d", ld, n,
                       gs);
  Q8Member m{out, *w, {nullptr, nullptr}, d};
  q8_gemv("k_matmul_q8_ld", &m, 1, x, n, ld, gs, epi);
}

void k_matmul_q8_ld_worker(float *out, const K8Input *x, const K8Weight *w, size_t ld, int n, int d, int gs, int kind,
                           int worker, int workers, llhip_atomic_int *claim, RowsDoneFn done, void *done_ctx) {
  (void)claim; /* every split here is static, as the reference's Q8 split is (src/gemv.c:578) */
  bool ok;
  Epilogue epi = ld_kind(kind, "k_matmul_q8_ld_worker", &ok);
  if (!ok)
    return;
  if (gs <= 0 || ld < (size_t)n || ld % (size_t)gs)
    return (void)raise(
        "k_matmul_q8_ld_worker: row stride %zu must be at least %d and a multiple of the group size %d", ld, n, gs);
  int r0, r1;
  if (!worker_share("k_matmul_q8_ld_worker", d, worker, workers, &r0, &r1))
    return;
  if (r1 > r0) {
    K8Weight share{w->q + (size_t)r0 * ld, w->s + (size_t)r0 * (ld / gs)};
    Q8Member m{out + r0, share, {nullptr, nullptr}, r1 - r0};
    q8_gemv("k_matmul_q8_ld_worker", &m, 1, x, n, ld, gs, epi);
  }
  if (done) {
    if (!synchronize_and_check())
      return;
    if (r1 > r0)
      done(done_ctx, r0, r1);
  }
}

void k_matmul_q8_swiglu_ld(float *out, const K8Input *x, const K8Weight *w1, const K8Weight *w3, size_t ld, int n,
                           int d, int gs) {
  if (gs <= 0 || ld < (size_t)n || ld % (size_t)gs) // src/gemv.c:583-584
    return (void)raise(
        "k_matmul_q8_swiglu_ld: row stride %zu must be at least %d and a multiple of the group size %d", ld, n, gs);
  Q8Member m{out, *w1, *w3, d};
  q8_gemv("k_matmul_q8_swiglu_ld", &m, 1, x, n, ld, gs, EPI_SWIGLU);
}

void k_matmul(float *out, const float *x, const float *w, int n, int d) {
  F32Member m{out, w, nullptr, d};
  f32_gemv("k_matmul", &m, 1, x, n, 0, EPI_STORE);
}

void k_matmul_add(float *out, const float *x, const float *w, int n, int d) {
  F32Member m{out, w, nullptr, d};
  f32_gemv("k_matmul_add", &m, 1, x, n, 0, EPI_ADD);
}

void k_matmul_qkv(float *q, float *k, float *v, const float *x, const float *wq, const float *wk, const float *wv, int n,
                  int dq, int dkv) {
  F32Member m[3] = {{q, wq, nullptr, dq}, {k, wk, nullptr, dkv}, {v, wv, nullptr, dkv}};
  f32_gemv("k_matmul_qkv", m, 3, x, n, 0, EPI_STORE);
}

void k_matmul_swiglu(float *out, const float *x, const float *w1, const float *w3, int n, int d) {
  F32Member m{out, w1, w3, d};
  f32_gemv("k_matmul_swiglu", &m, 1, x, n, 0, EPI_SWIGLU);
}

void k_matmul_ld(float *out, const float *x, const float *w, size_t ld, int n, int d, int kind) {
  bool ok;
  Epilogue epi = ld_kind(kind, "k_matmul_ld", &ok);
  if (!ok)
    return;
  if (ld < (size_t)n) // src/gemv.c:540-541
    return (void)raise("k_matmul_ld: row stride %zu is shorter than the %d inputs", ld, n);
  F32Member m{out, w, nullptr, d};
  f32_gemv("k_matmul_ld", &m, 1, x, n, ld, epi);
}

void k_matmul_ld_worker(float *out, const float *x, const float *w, size_t ld, int n, int d, int kind, int worker,
                        int workers, llhip_atomic_int *claim, RowsDoneFn done, void *done_ctx) {
  (void)claim;
  bool ok;
  Epilogue epi = ld_kind(kind, "k_matmul_ld_worker", &ok);
  if (!ok)
    return;
  if (ld < (size_t)n)
    return (void)raise("k_matmul_ld_worker: row stride %zu is shorter than the %d inputs", ld, n);
  int r0, r1;
  if (!worker_share("k_matmul_ld_worker", d, worker, workers, &r0, &r1))
    return;
  if (r1 > r0) {
    F32Member m{out + r0, w + (size_t)r0 * ld, nullptr, r1 - r0};
    f32_gemv("k_matmul_ld_worker", &m, 1, x, n, ld, epi);
  }
  if (done) {
    if (!synchronize_and_check())
      return;
    if (r1 > r0)
      done(done_ctx, r0, r1);
  }
}

void k_matmul_swiglu_ld(float *out, const float *x, const float *w1, const float *w3, size_t ld, int n, int d) {
  if (ld < (size_t)n) // src/gemv.c:560-561
    return (void)raise("k_matmul_swiglu_ld: row stride %zu is shorter than the %d inputs", ld, n);
  F32Member m{out, w1, w3, d};
  f32_gemv("k_matmul_swiglu_ld", &m, 1, x, n, ld, EPI_SWIGLU);
}

void k_gemm_q8(const int8_t *xq, const float *xs, int m, int k, int gs, const GemmQ8Segment *segments, int count) {
  gemm_q8("k_gemm_q8", true, xq, xs, m, k, gs, segments, count);
}

// No counterpart in the reference: hb = silu(W1 x) * (W3 x) as k_gemm_q8's GEMM_SWIGLU computes it, quantized in the
// GEMM's epilogue by the k_quantize rule (groups of 64) instead of written out in FP32 (the engine's batched forward:
// the SwiGLU GEMM then k_quantize_rows of hb, src/tp.c:580-584); bitwise those two calls. 1 when it ran, 0 (nothing
// launched) when the shape does not take the wide int8 kernel unsplit.
int llhip_gemm_q8_swiglu_quantize(const int8_t *xq, const float *xs, int m, int k, int gs, const K8Weight *w1,
                                  const K8Weight *w3, int n, int8_t *hq, float *hs) {
  const char *name = "llhip_gemm_q8_swiglu_quantize";
  if (!w1 || !w3 || !w1->q || !w1->s || !w3->q || !w3->s || !xq || !xs || !hq || !hs) {
    raise("%s: null buffer", name);
    return 0;
  }
  if (gs != 64 || k % gs || n % 64 || m <= 0 || n <= 0 || k <= 0)
    return 0;
  const int groups = k / gs;
  Call call(name);
  Ref XQ = call.in(xq, (size_t)m * k), XS = call.in(xs, (size_t)m * groups * sizeof(float));
  Ref W = call.in(w1->q, (size_t)n * k), WS = call.in(w1->s, (size_t)n * groups * sizeof(float));
  Ref W3 = call.in(w3->q, (size_t)n * k), W3S = call.in(w3->s, (size_t)n * groups * sizeof(float));
  Ref HQ = call.out(hq, (size_t)m * n, false), HS = call.out(hs, (size_t)m * (n / 64) * sizeof(float), false);
  if (!call.ready())
    return 0;
  GemmQ8Job job{};
  job.seg[0] = GemmSegmentDev{nullptr, n, call.ptr<const void>(W), call.ptr<const void>(W3), call.ptr<const float>(WS),
                              call.ptr<const float>(W3S), (size_t)k, n, EPI_SWIGLU};
  job.seg[0].cq = call.ptr<int8_t>(HQ);
  job.seg[0].cs = call.ptr<float>(HS);
  job.nseg = 1;
  job.xq = call.ptr<const int8_t>(XQ);
  job.xs = call.ptr<const float>(XS);
  job.m = m;
  job.k = k;
  job.gs = gs;
  if (((uintptr_t)job.xq | (uintptr_t)job.seg[0].w | (uintptr_t)job.seg[0].w3) & 15 ||
      !launch_q8_gemm_swiglu_quantized(job, call.stream()))
    return 0;
  return call.finish() ? 1 : 0;
}

Q8GemmBackend k_gemm_q8_pick(int gs, const GemmQ8Segment *segments, int count) {
  (void)segments, (void)count;
  return gs > 0 && gs % 64 == 0 ? Q8_GEMM_HIP_MFMA : Q8_GEMM_PORTABLE;
}

int k_gemm_q8_backend_test(Q8GemmBackend backend, const int8_t *xq, const float *xs, int m, int k, int gs,
                           const GemmQ8Segment *segments, int count) {
  if (backend == Q8_GEMM_HIP_MFMA) {
    if (gs <= 0 || gs % 64)
      return 0;
    gemm_q8("k_gemm_q8_backend_test", true, xq, xs, m, k, gs, segments, count);
    return 1;
  }
  if (backend == Q8_GEMM_PORTABLE) {
    gemm_q8("k_gemm_q8_backend_test", false, xq, xs, m, k, gs, segments, count);
    return 1;
  }
  return 0; /* the CPU backends are not compiled into this library */
}

void llhip_q8_group_dots(int32_t *dots, const int8_t *xq, int m, int k, int gs, const int8_t *wq, int n) {
  if (gs <= 0 || gs % 64 || k % gs)
    return (void)raise("llhip_q8_group_dots: the MFMA probe needs gs %% 64 == 0 and K a multiple of gs (K=%d gs=%d)", k,
                       gs);
  if (m <= 0 || n <= 0 || k <= 0)
    return;
  Call call("llhip_q8_group_dots");
  Ref XQ = call.in(xq, (size_t)m * k), WQ = call.in(wq, (size_t)n * k);
  Ref D = call.out(dots, (size_t)(k / gs) * m * n * sizeof(int32_t), false);
  if (!call.ready())
    return;
  if (!q8_gemm_fast_path(call.ptr<const int8_t>(XQ), m, k, gs))
    return (void)raise("llhip_q8_group_dots: the shape (m %d, K %d) is outside the MFMA kernel's range", m, k);
  if (launch_q8_group_dots(call.ptr<int32_t>(D), call.ptr<const int8_t>(XQ), m, k, gs, call.ptr<const int8_t>(WQ), n,
                           call.stream()))
    call.finish();
}

// testing.h:69: the reference's AMX probe reads the weights in the pack_s8_vnni layout (K padded to 64); here they are
// unpacked on the device and the MFMA kernel's probe forms the dots.
int k_gemm_q8_amx_dots_test(int32_t *dots, const int8_t *xq, int m, int k, int gs, const int8_t *packed, int n) {
  if (gs <= 0 || gs % 64 || k <= 0 || k % gs)
    return 0;
  if (m <= 0 || n <= 0)
    return 1;
  Call call("k_gemm_q8_amx_dots_test");
  Ref XQ = call.in(xq, (size_t)m * k), PK = call.in(packed, s8_vnni_bytes(n, k));
  Ref D = call.out(dots, (size_t)(k / gs) * m * n * sizeof(int32_t), false);
  if (!call.ready())
    return 0;
  if (!q8_gemm_fast_path(call.ptr<const int8_t>(XQ), m, k, gs)) {
    raise("k_gemm_q8_amx_dots_test: the shape (m %d, K %d) is outside the MFMA kernel's range", m, k);
    return 0;
  }
  if ((uintptr_t)call.ptr<const int8_t>(PK) & 3) {
    raise("k_gemm_q8_amx_dots_test: the packed weights must be 4-byte aligned");
    return 0;
  }
  int8_t *wq = nullptr;
  if (!LLHIP_CHECK(hipMallocAsync((void **)&wq, (size_t)n * k, call.stream())))
    return 0;
  const bool ok = launch_s8_vnni_unpack(wq, call.ptr<const int8_t>(PK), n, k, call.stream()) &&
                  launch_q8_group_dots(call.ptr<int32_t>(D), call.ptr<const int8_t>(XQ), m, k, gs, wq, n,
                                       call.stream());
  (void)hipFreeAsync(wq, call.stream());
  if (!ok)
    return 0;
  call.finish();
  return 1;
}

void llhip_set_gemv_shape(int waves_per_row, int blocks_per_cu, int block_waves) {
  // the next launches use it: launch any recorded quantization under the shape it was recorded with
  if (ensure_device() && flush_pending_quantize())
    (void)set_gemv_shape(waves_per_row, blocks_per_cu, block_waves);
}

void llhip_set_gemm_splits(int splits) { set_gemm_splits(splits); }

void llhip_set_bf16_tile(int tile) { set_bf16_tile(tile); }

void llhip_set_q8_tile(int tile) { set_q8_tile(tile); }

void llhip_set_q8_scales(int where) { set_q8_scales(where); }

void llhip_q8_gemv_group_dots(int32_t *dots, const int8_t *xq, const float *xs, const int8_t *wq, const float *ws,
                              size_t ld, int n, int d, int gs) {
  if (gs <= 0 || n % gs || (ld && (ld < (size_t)n || ld % (size_t)gs)))
    return (void)raise("llhip_q8_gemv_group_dots: n=%d and ld=%zu must be multiples of gs=%d", n, ld, gs);
  if (d <= 0 || n <= 0 || !ensure_device())
    return;
  // The GEMV itself stages or resolves its inputs; the probe and the discarded output live in device scratch here.
  hipStream_t stream = device().stream;
  const size_t probe_bytes = (size_t)(n / gs) * d * sizeof(int32_t);
  int32_t *probe = nullptr;
  float *scratch = nullptr;
  if (!LLHIP_CHECK(hipMalloc((void **)&probe, probe_bytes)) ||
      !LLHIP_CHECK(hipMalloc((void **)&scratch, (size_t)d * sizeof(float))))
    return;
  K8Input in{xq, xs, nullptr};
  Q8Member m{scratch, K8Weight{wq, ws}, {nullptr, nullptr}, d};
  q8_gemv("llhip_q8_gemv_group_dots", &m, 1, &in, n, ld, gs, EPI_STORE, probe);
  if (LLHIP_CHECK(hipMemcpyAsync(dots, probe, probe_bytes, hipMemcpyDefault, stream)))
    (void)synchronize_and_check();
  (void)hipFree(probe);
  (void)hipFree(scratch);
}

void k_gemm_f32(const float *a, int lda, int m, int k, const GemmSegment *segments, int count) {
  gemm_f32("k_gemm_f32", a, lda, m, k, segments, count);
}

/* testing.h:61: the portable driver with an explicit K block; the device GEMM has no K blocking, so kc is ignored. */
void k_gemm_f32_portable(const float *a, int lda, int m, int k, const GemmSegment *segments, int count, int kc) {
  (void)kc;
  gemm_f32("k_gemm_f32_portable", a, lda, m, k, segments, count);
}

int k_gemm_f32_simd_test(const float *a, int lda, int m, int k, const GemmSegment *segments, int count, int kc) {
  (void)a, (void)lda, (void)m, (void)k, (void)segments, (void)count, (void)kc;
  return 0; /* testing.h:64: no CPU SIMD microkernel is compiled in */
}

size_t k_gemm_bf16_panel_bytes(int m, int k) {
  const size_t mm = (size_t)(m > 0 ? m : 1), kk = (size_t)(k > 0 ? k : 1);
  return (mm + 15) / 16 * 16 * ((kk + 31) / 32 * 32 + 32) * sizeof(uint16_t); // gemm.c:740-742
}

void k_gemm_bf16(const float *a, int lda, int m, int k, const GemmBf16Segment *segments, int count,
                 AlignedBuffer *panel) {
  if (!check_count(count))
    return;
  for (int s = 0; s < count; s++)
    if (!segments[s].w || (segments[s].kind == GEMM_SWIGLU && !segments[s].w3))
      return (void)raise("BF16 GEMM segment %d has no packed weights", s);
  if (m <= 0 || k <= 0)
    return;
  if (!panel || panel->bytes < k_gemm_bf16_panel_bytes(m, k))
    return (void)raise("BF16 activation panel holds %zu bytes but %zu are needed", panel ? panel->bytes : (size_t)0,
                       k_gemm_bf16_panel_bytes(m, k));
  if (!panel->data)
    return (void)raise("BF16 activation panel has no memory");
  Call call("k_gemm_bf16");
  Ref A = call.in2d(a, (size_t)k * sizeof(float), (size_t)lda * sizeof(float), (size_t)m);
  // the rounded activations, m rows of K rounded up to 32 values (device memory from aligned_buffer_alloc is used in
  // place; a host panel is staged like any other host buffer)
  Ref PANEL = call.out(panel->data, (size_t)m * (size_t)((k + 31) / 32 * 32) * sizeof(uint16_t), false);
  Ref W[3], W3[3], C[3];
  for (int s = 0; s < count; s++) {
    const GemmBf16Segment &g = segments[s];
    if (g.n <= 0)
      continue;
    const size_t packed = bf16_vnni_elements(g.n, k) * sizeof(uint16_t);
    W[s] = call.in(g.w, packed);
    if (g.kind == GEMM_SWIGLU)
      W3[s] = call.in(g.w3, packed);
    C[s] = call.out2d(g.c, (size_t)g.n * sizeof(float), (size_t)g.ldc * sizeof(float), (size_t)m, g.kind == GEMM_ADD);
  }
  if (!call.ready())
    return;
  GemmF32Job job{};
  int nseg = 0;
  for (int s = 0; s < count; s++) {
    const GemmBf16Segment &g = segments[s];
    if (g.n <= 0)
      continue;
    job.seg[nseg++] = GemmSegmentDev{call.ptr<float>(C[s]), g.ldc,    call.ptr<const void>(W[s]), call.ptr<const void>(W3[s]),
                                     nullptr,               nullptr, 0,                          g.n,
                                     gemm_epilogue(g.kind)};
  }
  if (!nseg)
    return (void)call.finish();
  job.nseg = nseg;
  job.a = call.ptr<const float>(A);
  job.lda = lda;
  job.m = m;
  job.k = k;
  job.bf16 = true;
  job.panel = call.ptr<unsigned short>(PANEL);
  if (launch_f32_gemm(job, call.stream()))
    call.finish();
}

} // extern "C"
