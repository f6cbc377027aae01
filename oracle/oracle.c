/* CPU oracle for the llama3.x.c matmul hot path. TEST INFRASTRUCTURE ONLY: see oracle.h for what may use it and how
 * each function is pinned to the reference. Written from the reference's semantics, cited per function. */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- activation quantization ------------------------------------------------------------------------------------ */

/* src/gemv.c:596-623. The max scan keeps the first strictly larger |x| (so -0.0f and 0.0f both leave it at 0); the
 * division and the clamp run in float; roundf rounds half away from zero; the cast to int8 is exact after the clamp. */
int orc_quantize(int8_t *q, float *s, const float *x, int n, int gs) {
  const int groups = n / gs;
  for (int g = 0; g < groups; g++) {
    const float *in = x + (size_t)g * (size_t)gs;
    int8_t *dst = q + (size_t)g * (size_t)gs;
    float peak = 0.0f;
    for (int i = 0; i < gs; i++) {
      if (!isfinite(in[i]))
        return -1;
      const float magnitude = fabsf(in[i]);
      if (magnitude > peak)
        peak = magnitude;
    }
    const float scale = peak / 127.0f;
    s[g] = scale;
    for (int i = 0; i < gs; i++) {
      const float ratio = scale == 0.0f ? 0.0f : in[i] / scale;
      const float clamped = fmaxf(-127.0f, fminf(127.0f, ratio));
      dst[i] = (int8_t)roundf(clamped);
    }
  }
  return 0;
}

/* src/gemm.c:819-830: each row is the per-token quantizer, so the batch is bitwise the per-row result. */
int orc_quantize_rows(int8_t *q, float *s, const float *x, size_t ldx, int m, int n, int gs) {
  for (int r = 0; r < m; r++)
    if (orc_quantize(q + (size_t)r * (size_t)n, s + (size_t)r * (size_t)(n / gs), x + (size_t)r * ldx, n, gs))
      return -1;
  return 0;
}

/* ---- GEMV ------------------------------------------------------------------------------------------------------- */

float orc_silu_gate(float value, float gate) {
  value *= (1.0f / (1.0f + expf(-value)));
  return value * gate;
}

/* src/gemv.c:417-438. One float per row; each whole group adds ((float)i32 * ws) * xs (W8A8), or the group's float
 * sum times ws (W8A32). A tail shorter than gs is not part of any group and is ignored, as in the reference loop. */
void orc_q8_dots(float *out, const int8_t *wq, const float *ws, size_t ld, int rows, const int8_t *xq, const float *xs,
                 const float *xf, int n, int gs) {
  const size_t scale_ld = ld / (size_t)gs;
  for (int r = 0; r < rows; r++) {
    const int8_t *row = wq + (size_t)r * ld;
    const float *row_scale = ws + (size_t)r * scale_ld;
    float total = 0.0f;
    for (int j = 0; j + gs <= n; j += gs) {
      const int g = j / gs;
      if (xq) {
        int32_t dot = 0;
        for (int t = 0; t < gs; t++)
          dot += (int32_t)xq[j + t] * (int32_t)row[j + t];
        total += (float)dot * row_scale[g] * xs[g];
      } else {
        float partial = 0.0f;
        for (int t = 0; t < gs; t++)
          partial += (float)row[j + t] * xf[j + t];
        total += partial * row_scale[g];
      }
    }
    out[r] = total;
  }
}

/* The GEMV epilogues, src/gemv.c:463-470. */
static void gemv_epilogue(float *out, float dot, float gate, int kind) {
  if (kind == ORC_K_ADD)
    *out += dot;
  else if (kind == ORC_K_SWIGLU)
    *out = orc_silu_gate(dot, gate);
  else
    *out = dot;
}

void orc_matmul_q8(float *out, const int8_t *xq, const float *xs, const float *xf, const int8_t *wq, const float *ws,
                   const int8_t *w3q, const float *w3s, size_t ld, int n, int d, int gs, int kind) {
  if (!ld)
    ld = (size_t)n;
  const size_t scale_ld = ld / (size_t)gs;
  for (int r = 0; r < d; r++) {
    float dot, gate = 0.0f;
    orc_q8_dots(&dot, wq + (size_t)r * ld, ws + (size_t)r * scale_ld, ld, 1, xq, xs, xf, n, gs);
    if (kind == ORC_K_SWIGLU)
      orc_q8_dots(&gate, w3q + (size_t)r * ld, w3s + (size_t)r * scale_ld, ld, 1, xq, xs, xf, n, gs);
    gemv_epilogue(out + r, dot, gate, kind);
  }
}

void orc_group_dots(int32_t *dots, const int8_t *xq, size_t ldx, int m, const int8_t *wq, size_t ldw, int n, int k,
                    int gs) {
  const int groups = k / gs;
  for (int g = 0; g < groups; g++)
    for (int r = 0; r < m; r++)
      for (int c = 0; c < n; c++) {
        const int8_t *a = xq + (size_t)r * ldx + (size_t)g * (size_t)gs;
        const int8_t *b = wq + (size_t)c * ldw + (size_t)g * (size_t)gs;
        int32_t dot = 0;
        for (int t = 0; t < gs; t++)
          dot += (int32_t)a[t] * (int32_t)b[t];
        dots[((size_t)g * (size_t)m + (size_t)r) * (size_t)n + (size_t)c] = dot;
      }
}

/* ---- batched GEMMs ---------------------------------------------------------------------------------------------- */

/* The GEMM epilogues, src/gemm.c:155-166, 975-986 and 724-735 (GemmKind). */
static void gemm_epilogue(float *out, float sum, float gate, int kind) {
  if (kind == ORC_GEMM_ADD)
    *out += sum;
  else if (kind == ORC_GEMM_SWIGLU)
    *out = orc_silu_gate(sum, gate);
  else
    *out = sum;
}

void orc_gemm_q8(const int8_t *xq, const float *xs, int m, int k, int gs, float *c, int ldc, const int8_t *wq,
                 const float *ws, const int8_t *w3q, const float *w3s, int n, int kind) {
  const int groups = k / gs;
  for (int i = 0; i < m; i++) {
    const int8_t *x = xq + (size_t)i * (size_t)k;
    const float *x_scale = xs + (size_t)i * (size_t)groups;
    for (int j = 0; j < n; j++) {
      float sum, gate = 0.0f;
      orc_q8_dots(&sum, wq + (size_t)j * (size_t)k, ws + (size_t)j * (size_t)groups, (size_t)k, 1, x, x_scale, NULL, k,
                  gs);
      if (kind == ORC_GEMM_SWIGLU)
        orc_q8_dots(&gate, w3q + (size_t)j * (size_t)k, w3s + (size_t)j * (size_t)groups, (size_t)k, 1, x, x_scale,
                    NULL, k, gs);
      gemm_epilogue(c + (size_t)i * (size_t)ldc + j, sum, gate, kind);
    }
  }
}

/* src/gemv.c:259-266: ascending j into one float. */
static float f32_dot(const float *w, const float *x, int n) {
  float total = 0.0f;
  for (int j = 0; j < n; j++)
    total += w[j] * x[j];
  return total;
}

void orc_matmul_f32(float *out, const float *x, const float *w, const float *w3, size_t ld, int n, int d, int kind) {
  if (!ld)
    ld = (size_t)n;
  for (int r = 0; r < d; r++) {
    const float dot = f32_dot(w + (size_t)r * ld, x, n);
    const float gate = kind == ORC_K_SWIGLU ? f32_dot(w3 + (size_t)r * ld, x, n) : 0.0f;
    gemv_epilogue(out + r, dot, gate, kind);
  }
}

/* src/gemm.c:52-55 sums `val += wc[j] * ar[j]` (weight first); src/gemm.c:126-138 adds the tile to a zeroed
 * accumulator. With one K block the result is the ascending-k sum, as the scalar GEMV computes it. */
void orc_gemm_f32(const float *a, int lda, int m, int k, float *c, int ldc, const float *w, const float *w3,
                  size_t ldw, int n, int kind) {
  for (int i = 0; i < m; i++)
    for (int j = 0; j < n; j++) {
      const float *ar = a + (size_t)i * (size_t)lda;
      float acc = 0.0f, gacc = 0.0f;
      acc += f32_dot(w + (size_t)j * ldw, ar, k);
      if (kind == ORC_GEMM_SWIGLU)
        gacc += f32_dot(w3 + (size_t)j * ldw, ar, k);
      gemm_epilogue(c + (size_t)i * (size_t)ldc + j, acc, gacc, kind);
    }
}

/* ---- BF16 ------------------------------------------------------------------------------------------------------- */

uint16_t orc_bf16_from_f32(float x) {
  uint32_t bits;
  memcpy(&bits, &x, sizeof(bits));
  if ((bits & 0x7fffffffu) > 0x7f800000u) /* NaN: keep sign and the top payload bits, set the quiet bit */
    return (uint16_t)((bits >> 16) | 0x0040u);
  /* Round to nearest even on the 16 dropped bits: add just under half an ulp, plus one when the kept lsb is odd. */
  const uint32_t lsb = (bits >> 16) & 1u;
  bits += 0x7fffu + lsb;
  return (uint16_t)(bits >> 16);
}

float orc_f32_from_bf16(uint16_t v) {
  const uint32_t bits = (uint32_t)v << 16;
  float x;
  memcpy(&x, &bits, sizeof(x));
  return x;
}

static size_t round_up(size_t v, size_t to) {
  return (v + to - 1) / to * to;
}

size_t orc_bf16_vnni_elements(int rows, int cols) {
  return round_up((size_t)rows, 16) * round_up((size_t)cols, 32);
}

size_t orc_s8_vnni_bytes(int rows, int cols) {
  return round_up((size_t)rows, 16) * round_up((size_t)cols, 64);
}

/* src/gemm.c:363-376: tile t (rows 16t..16t+15), K pair p: element ((t * kp/2 + p) * 16 + c) * 2 + e holds
 * w[16t + c][2p + e]. */
void orc_pack_bf16_vnni(uint16_t *dst, const float *w, int rows, int cols, size_t ld) {
  const size_t kp = round_up((size_t)cols, 32), tiles = round_up((size_t)rows, 16) / 16;
  for (size_t t = 0; t < tiles; t++)
    for (size_t p = 0; p < kp / 2; p++)
      for (size_t c = 0; c < 16; c++)
        for (size_t e = 0; e < 2; e++) {
          const size_t row = t * 16 + c, col = 2 * p + e;
          const uint16_t v = row < (size_t)rows && col < (size_t)cols ? orc_bf16_from_f32(w[row * ld + col]) : 0;
          dst[((t * (kp / 2) + p) * 16 + c) * 2 + e] = v;
        }
}

/* src/gemm.c:382-394: the same with K quads, kp = cols rounded up to 64. */
void orc_pack_s8_vnni(int8_t *dst, const int8_t *w, int rows, int cols, size_t ld) {
  const size_t kp = round_up((size_t)cols, 64), tiles = round_up((size_t)rows, 16) / 16;
  for (size_t t = 0; t < tiles; t++)
    for (size_t q = 0; q < kp / 4; q++)
      for (size_t c = 0; c < 16; c++)
        for (size_t e = 0; e < 4; e++) {
          const size_t row = t * 16 + c, col = 4 * q + e;
          dst[((t * (kp / 4) + q) * 16 + c) * 4 + e] = row < (size_t)rows && col < (size_t)cols ? w[row * ld + col] : 0;
        }
}

/* Element (row j, column l) of a matrix packed by orc_pack_bf16_vnni for kp = k rounded up to 32. */
static float packed_bf16(const uint16_t *p, size_t kp, int j, int l) {
  const size_t t = (size_t)j / 16, c = (size_t)j % 16, pair = (size_t)l / 2, e = (size_t)l & 1u;
  return orc_f32_from_bf16(p[((t * (kp / 2) + pair) * 16 + c) * 2 + e]);
}

/* src/gemm.c:667-678 (the sum) and 693-706 (the RNE activation panel), with the epilogue of 724-735. */
void orc_gemm_bf16(const float *a, int lda, int m, int k, float *c, int ldc, const uint16_t *pw, const uint16_t *pw3,
                   int n, int kind) {
  const size_t kp = round_up((size_t)k, 32);
  float *row = malloc((size_t)(k > 0 ? k : 1) * sizeof(float));
  for (int i = 0; i < m; i++) {
    for (int l = 0; l < k; l++)
      row[l] = orc_f32_from_bf16(orc_bf16_from_f32(a[(size_t)i * (size_t)lda + (size_t)l]));
    for (int j = 0; j < n; j++) {
      float sum = 0.0f, gate = 0.0f;
      for (int l = 0; l < k; l++)
        sum += row[l] * packed_bf16(pw, kp, j, l);
      if (kind == ORC_GEMM_SWIGLU)
        for (int l = 0; l < k; l++)
          gate += row[l] * packed_bf16(pw3, kp, j, l);
      gemm_epilogue(c + (size_t)i * (size_t)ldc + j, sum, gate, kind);
    }
  }
  free(row);
}

/* ---- threaded CPU timing rung ------------------------------------------------------------------------------------ */

typedef struct {
  float *out;
  const int8_t *xq, *wq;
  const float *xs, *ws;
  int n, d, gs, worker, workers;
} GemvShare;

static void *gemv_share(void *p) {
  const GemvShare *job = p;
  const int r0 = (int)((long long)job->d * job->worker / job->workers);
  const int r1 = (int)((long long)job->d * (job->worker + 1) / job->workers);
  const size_t scale_ld = (size_t)job->n / (size_t)job->gs;
  if (r1 > r0)
    orc_q8_dots(job->out + r0, job->wq + (size_t)r0 * (size_t)job->n, job->ws + (size_t)r0 * scale_ld, (size_t)job->n,
                r1 - r0, job->xq, job->xs, NULL, job->n, job->gs);
  return NULL;
}

void orc_matmul_q8_threads(float *out, const int8_t *xq, const float *xs, const int8_t *wq, const float *ws, int n,
                           int d, int gs, int threads) {
  if (threads < 1)
    threads = 1;
  if (threads > 1024)
    threads = 1024;
  pthread_t *tid = malloc(sizeof(pthread_t) * (size_t)threads);
  GemvShare *jobs = malloc(sizeof(GemvShare) * (size_t)threads);
  for (int t = 0; t < threads; t++) {
    jobs[t] = (GemvShare){out, xq, wq, xs, ws, n, d, gs, t, threads};
    if (t)
      pthread_create(&tid[t], NULL, gemv_share, &jobs[t]);
  }
  gemv_share(&jobs[0]);
  for (int t = 1; t < threads; t++)
    pthread_join(tid[t], NULL);
  free(tid);
  free(jobs);
}

/* ---- the forward around the matmuls ------------------------------------------------------------------------- */

/* src/kernels.c:8-21 */
void orc_rmsnorm(float *out, const float *x, const float *weight, int size, float epsilon) {
  float ss = 0.0f;
  for (int j = 0; j < size; j++)
    ss += x[j] * x[j];
  ss /= size;
  ss += epsilon;
  ss = 1.0f / sqrtf(ss);
  for (int j = 0; j < size; j++)
    out[j] = weight[j] * (ss * x[j]);
}

/* src/kernels_simd.c:212-225 (the products round before the sum: this file is built with -ffp-contract=off). */
static void rope_pair(float *v, int i, float c, float s) {
  const float a = v[i], b = v[i + 1];
  v[i] = a * c - b * s;
  v[i + 1] = a * s + b * c;
}

void orc_rope_apply(float *q, float *k, const float *table, int n_heads, int n_kv_heads, int head_dim) {
  const float *sines = table + head_dim;
  for (int h = 0; h < n_heads; h++)
    for (int j = 0; j < head_dim; j += 2) {
      const float c = table[j], s = sines[j + 1];
      rope_pair(q, h * head_dim + j, c, s);
      if (h < n_kv_heads)
        rope_pair(k, h * head_dim + j, c, s);
    }
}

/* src/attention.c:1420-1432 */
void orc_kv_store(float *cache, const float *src, size_t src_ld, int pos0, int count, int n_kv_heads, int head_dim,
                  size_t pos_stride, size_t head_base) {
  for (int r = 0; r < count; r++)
    for (int g = 0; g < n_kv_heads; g++)
      memcpy(cache + (size_t)(pos0 + r) * pos_stride + (size_t)g * head_base, src + (size_t)r * src_ld + (size_t)g * head_dim,
             (size_t)head_dim * sizeof(float));
}

/* src/kernels.c:23-45 */
static int softmax(float *x, int size) {
  float max_val = x[0];
  if (!isfinite(max_val))
    return -1;
  for (int i = 1; i < size; i++) {
    if (!isfinite(x[i]))
      return -1;
    if (x[i] > max_val)
      max_val = x[i];
  }
  float sum = 0.0f;
  for (int i = 0; i < size; i++) {
    x[i] = expf(x[i] - max_val);
    sum += x[i];
  }
  for (int i = 0; i < size; i++)
    x[i] /= sum;
  return 0;
}

/* src/attention.c:606-641 */
int orc_attention(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                  int n_heads, int n_kv_heads, int head_dim, int seq_len, int position, size_t pos_stride,
                  size_t head_base) {
  const int kv_mul = n_heads / n_kv_heads;
  for (int h = 0; h < n_heads; h++) {
    const float *qh = q + (size_t)h * head_dim;
    float *a = att + (size_t)h * seq_len;
    for (int t = 0; t <= position; t++) {
      const float *k = key_cache + (size_t)t * pos_stride + (size_t)(h / kv_mul) * head_base;
      float score = 0.0f;
      for (int i = 0; i < head_dim; i++)
        score += qh[i] * k[i];
      score /= sqrtf(head_dim);
      a[t] = score;
    }
    if (softmax(a, position + 1))
      return -1;
    float *xb = out + (size_t)h * head_dim;
    memset(xb, 0, (size_t)head_dim * sizeof(float));
    for (int t = 0; t <= position; t++) {
      const float *v = value_cache + (size_t)t * pos_stride + (size_t)(h / kv_mul) * head_base;
      const float w = a[t];
      for (int i = 0; i < head_dim; i++)
        xb[i] += w * v[i];
    }
  }
  return 0;
}

/* ---- seeded synthetic inputs ------------------------------------------------------------------------------------- */

uint64_t orc_rng_next(uint64_t *state) {
  uint64_t x = *state;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  *state = x;
  return x;
}

float orc_rng_uniform(uint64_t *state) {
  return (float)((double)(orc_rng_next(state) >> 40) / (double)(1ull << 24)) * 2.0f - 1.0f;
}

void orc_fill_uniform(float *dst, size_t n, uint64_t *state, float scale) {
  for (size_t i = 0; i < n; i++)
    dst[i] = orc_rng_uniform(state) * scale;
}

/* A uniform in (0, 1] from the top 24 bits of one draw, so the logarithm below is finite. */
static double open_unit(uint64_t *state) {
  return ((double)(orc_rng_next(state) >> 40) + 1.0) / (double)(1ull << 24);
}

void orc_fill_normal(float *dst, size_t n, uint64_t *state, float mean, float std) {
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < n; i += 2) {
    const double radius = sqrt(-2.0 * log(open_unit(state))), angle = two_pi * open_unit(state);
    dst[i] = (float)(mean + std * radius * cos(angle));
    if (i + 1 < n)
      dst[i + 1] = (float)(mean + std * radius * sin(angle));
  }
}
