// The reference-named C entry points of the forward around the matmuls: RMSNorm, RoPE, the K/V cache and attention
// (include/kernels.h:57-68, 124-179). Argument checks, pointer residency as for the matmuls, one stream-ordered launch
// per call. Citations are LucianCrainic/llama3.x.c file:line.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "common.h"
#include "llama_hip_forward.h"

using namespace llhip;

namespace {

// Positions pos0 .. pos0 + count - 1 lie in a cache of seq_len positions; no sum can overflow.
bool positions_fit(int pos0, int count, int seq_len) {
  return pos0 >= 0 && count >= 0 && seq_len > 0 && pos0 <= seq_len && count <= seq_len - pos0;
}

// src/attention.c:1375-1392: head (the default) is [kv_head][position][head_dim], rows is [position][kv_head][head_dim];
// LLAMA_KV_LAYOUT=rows|head picks one, read at the first use.
int kv_layout_head_flag = -1;

bool kv_head_major() {
  if (kv_layout_head_flag < 0) {
    const char *layout = getenv("LLAMA_KV_LAYOUT");
    kv_layout_head_flag = 1;
    if (layout && *layout && strcmp(layout, "auto")) {
      if (!strcmp(layout, "rows"))
        kv_layout_head_flag = 0;
      else if (strcmp(layout, "head"))
        raise("LLAMA_KV_LAYOUT must be rows or head");
    }
  }
  return kv_layout_head_flag == 1;
}

// The split-K partials of the device attention: grown on demand (never during graph capture), kept for the process.
float *attention_workspace = nullptr;
size_t attention_workspace_floats = 0;

float *attention_partials(size_t floats) {
  if (floats <= attention_workspace_floats)
    return attention_workspace;
  Device &dev = device();
  if (dev.capturing) {
    raise("attention needs %zu floats of workspace during graph capture; run the call once before capturing", floats);
    return nullptr;
  }
  if (attention_workspace) {
    (void)hipStreamSynchronize(dev.stream);
    (void)hipFree(attention_workspace);
    hbm_release(attention_workspace_floats * sizeof(float));
    attention_workspace = nullptr;
    attention_workspace_floats = 0;
  }
  const size_t want = floats + floats / 4 + 1024;
  if (!hbm_claim(want * sizeof(float), "the attention workspace"))
    return nullptr;
  if (hipMalloc((void **)&attention_workspace, want * sizeof(float)) != hipSuccess) {
    (void)hipGetLastError();
    hbm_release(want * sizeof(float));
    attention_workspace = nullptr;
    raise("allocating %zu bytes of attention workspace failed", want * sizeof(float));
    return nullptr;
  }
  attention_workspace_floats = want;
  return attention_workspace;
}

void rmsnorm(const char *name, float *out, const float *x, const float *weight, int rows, int size, float epsilon) {
  if (rows <= 0 || size <= 0)
    return;
  if (!out || !x || !weight) {
    raise("%s: null buffer", name);
    return;
  }
  Call call(name);
  const size_t bytes = (size_t)rows * size * sizeof(float);
  Ref X = call.in(x, bytes), W = call.in(weight, (size_t)size * sizeof(float));
  Ref O = call.out(out, bytes, false);
  if (!call.ready())
    return;
  float *o = call.ptr<float>(O);
  const float *xd = call.ptr<const float>(X);
  const bool apart = (uintptr_t)(o + size) <= (uintptr_t)xd || (uintptr_t)(xd + size) <= (uintptr_t)o;
  if (rows == 1 && !call.staged() && apart && quantize_fusion_enabled()) {
    // one device-resident row into another buffer: recorded, so a k_quantize of the output and the GEMV after it
    // normalize in the GEMV's prologue (any other call runs it first)
    defer_norm(PendingNorm{o, xd, call.ptr<const float>(W), size, epsilon});
    return;
  }
  if (launch_rmsnorm(o, xd, call.ptr<const float>(W), rows, size, epsilon, call.stream()))
    call.finish();
}

void rope(const char *name, float *q, size_t q_stride, float *k, size_t k_stride, const float *table,
          size_t table_stride, int rows, int n_heads, int n_kv_heads, int head_dim) {
  if (rows <= 0 || n_heads <= 0 || head_dim <= 0)
    return;
  if (head_dim % 2 || n_kv_heads < 0 || n_kv_heads > n_heads) {
    raise("%s: head_dim %d must be even and 0 <= n_kv_heads (%d) <= n_heads (%d)", name, head_dim, n_kv_heads,
          n_heads);
    return;
  }
  if (!q || !table || (n_kv_heads > 0 && !k)) {
    raise("%s: null buffer", name);
    return;
  }
  // a table stride of 0 gives every row the same table (src/kernels_simd.c:268-269 adds i * table_stride)
  const bool shared_table = rows == 1 || table_stride == 0;
  if ((!shared_table && table_stride < 2 * (size_t)head_dim) || q_stride < (size_t)n_heads * head_dim ||
      (n_kv_heads > 0 && k_stride < (size_t)n_kv_heads * head_dim)) {
    raise("%s: a row stride is shorter than its row", name);
    return;
  }
  Call call(name);
  const size_t f = sizeof(float);
  Ref T = shared_table ? call.in(table, 2 * (size_t)head_dim * f)
                       : call.in2d(table, 2 * (size_t)head_dim * f, table_stride * f, (size_t)rows);
  Ref Q = call.out2d(q, (size_t)n_heads * head_dim * f, q_stride * f, (size_t)rows, true);
  Ref K = n_kv_heads > 0 ? call.out2d(k, (size_t)n_kv_heads * head_dim * f, k_stride * f, (size_t)rows, true) : Ref{};
  if (!call.ready())
    return;
  float *qd = call.ptr<float>(Q), *kd = n_kv_heads > 0 ? call.ptr<float>(K) : nullptr;
  const float *td = call.ptr<const float>(T);
  const bool aligned = head_dim % 4 == 0 && (((uintptr_t)qd | (uintptr_t)kd) & 15) == 0;
  if (rows == 1 && !call.staged() && n_kv_heads > 0 && aligned && quantize_fusion_enabled()) {
    // one device-resident row: recorded, so the cache stores of k and v and the decode attention that follow can
    // rotate, store and attend in one launch (any other call runs it first)
    defer_rope(PendingRope{qd, kd, td, n_heads, n_kv_heads, head_dim, 0, {}});
    return;
  }
  if (launch_rope(qd, q_stride, kd, k_stride, td, table_stride, rows, n_heads, n_kv_heads, head_dim, call.stream()))
    call.finish();
}

void strides(int n_kv_heads, int head_dim, int seq_len, bool head_major, size_t *pos_stride, size_t *head_base) {
  *pos_stride = head_major ? (size_t)head_dim : (size_t)n_kv_heads * head_dim;
  *head_base = head_major ? (size_t)seq_len * head_dim : (size_t)head_dim;
}

// The extent of one layer's cache as a layout addresses it: positions [0, last] of every KV head.
size_t cache_floats(int n_kv_heads, int head_dim, int last, size_t pos_stride, size_t head_base) {
  return (size_t)last * pos_stride + (size_t)(n_kv_heads - 1) * head_base + (size_t)head_dim;
}

// noalloc: the partials go to the per-device scratch array instead of the grown workspace, and nothing may allocate
// (no staging of host buffers, no device init).
// The attention entry points (k_attention*, the allocation-free form, and with qout the rows quantized in groups of
// qgs as k_quantize_rows would quantize them from out).
void attention(const char *name, float *out, const float *q, const float *key_cache, const float *value_cache,
               int n_heads, int n_kv_heads, int head_dim, int seq_len, int pos0, int m, size_t pos_stride,
               size_t head_base, bool noalloc = false, int8_t *qout = nullptr, float *qscale = nullptr, int qgs = 0) {
  if (m <= 0 || n_heads <= 0)
    return;
  if (!attention_shape_ok(n_heads, n_kv_heads, head_dim)) {
    raise("%s: %d heads over %d KV heads of dimension %d are not supported (n_heads a multiple of n_kv_heads, at "
          "most 16 per KV head, head_dim <= 256)",
          name, n_heads, n_kv_heads, head_dim);
    return;
  }
  if (!positions_fit(pos0, m, seq_len)) {
    raise("%s: positions %d..%lld are outside the cache of %d", name, pos0, (long long)pos0 + m - 1, seq_len);
    return;
  }
  if (pos_stride < (size_t)head_dim || pos_stride > (size_t)INT32_MAX) {
    raise("%s: position stride %zu is not in [head_dim, INT_MAX]", name, pos_stride); // src/attention.c:1369-1370
    return;
  }
  if (!out || !q || !key_cache || !value_cache) {
    raise("%s: null buffer", name);
    return;
  }
  const size_t partial_floats = attention_partial_floats(m, n_heads, head_dim, pos0 + m - 1);
  if (noalloc) {
    if (!device().ready) {
      raise("%s: the library is not initialized on this device (call llhip_init first: opening the device "
            "allocates)", name);
      return;
    }
  }
  Call call(name, true); // a recorded RoPE with its cache stores may be taken along
  const size_t f = sizeof(float), row = (size_t)n_heads * head_dim * f;
  const size_t cache = cache_floats(n_kv_heads, head_dim, pos0 + m - 1, pos_stride, head_base) * f;
  Ref Q = call.in(q, row * m), K = call.in(key_cache, cache), V = call.in(value_cache, cache);
  Ref O = call.out(out, row * m, false);
  const size_t qrow = (size_t)n_heads * head_dim;
  Ref QO{}, QS{};
  if (qout) {
    QO = call.out(qout, qrow * m, false);
    QS = call.out(qscale, qrow / qgs * m * f, false);
  }
  if (noalloc && call.staged()) { // staging would allocate the arena
    raise("%s: every buffer must be device memory or inside a registered range", name);
    return;
  }
  if (!call.ready())
    return;
  AttentionJob job{call.ptr<float>(O), call.ptr<const float>(Q), call.ptr<const float>(K), call.ptr<const float>(V),
                   n_heads, n_kv_heads, head_dim, pos0, m, pos_stride, head_base, nullptr, nullptr, nullptr};
  // the flash kernel (16 rows and more) splits a tile's positions only as far as its partials fit the scratch, so only
  // the split kernels' need is checked; a fused RoPE is taken only for one row, which never runs the flash kernel
  if (noalloc)
    job.partial_room = kAttentionScratchFloats;
  if (qout) {
    job.qout = call.ptr<int8_t>(QO);
    job.qscale = call.ptr<float>(QS);
    job.qgs = qgs;
  }
  if (noalloc && !attention_uses_flash(job) && partial_floats > kAttentionScratchFloats) {
    raise("%s: %d rows of %d heads up to position %d need %zu floats of scratch; it holds %zu", name, m, n_heads,
          pos0 + m - 1, partial_floats, kAttentionScratchFloats);
    return;
  }
  float *partial = noalloc ? attention_scratch(device().ordinal) : attention_partials(partial_floats);
  if (!partial) {
    if (noalloc)
      raise("%s: the attention scratch has no device address", name);
    return;
  }
  // the fused form reads the caches, q and the new rows as 16-byte vectors
  const bool aligned = head_dim % 4 == 0 && pos_stride % 4 == 0 && head_base % 4 == 0 &&
                       (((uintptr_t)job.q | (uintptr_t)job.key | (uintptr_t)job.value) & 15) == 0;
  PendingRope rope;
  if (m == 1 && !call.staged() && aligned &&
      take_pending_rope(job.q, job.key, job.value, pos0, pos_stride, head_base, n_heads, n_kv_heads, head_dim, &rope)) {
    job.k_new = rope.k;
    job.v_new = rope.store[1].src;
    job.table = rope.table;
  } else if (!flush_pending_quantize()) {
    return;
  }
  if (launch_attention(job, partial, call.stream()))
    call.finish();
}

int chunk_count(int position) { return position / 64 + 1; }

} // namespace

extern "C" {

// ---- RMSNorm (kernels.h:57-60, src/kernels.c:8-21) ----------------------------------------------------------------

void k_rmsnorm(float *out, const float *x, const float *weight, int size, float epsilon) {
  rmsnorm("k_rmsnorm", out, x, weight, 1, size, epsilon);
}

void k_rmsnorm_rows(float *out, const float *x, const float *weight, int rows, int size, float epsilon) {
  rmsnorm("k_rmsnorm_rows", out, x, weight, rows, size, epsilon);
}

// No counterpart in the reference: k_rmsnorm_rows then k_quantize_rows of the same rows in one launch, without the
// normalized rows in memory (the engine's batched forward, src/tp.c:546-547 and 576-577); bitwise the two calls.
void llhip_rmsnorm_quantize_rows(int8_t *q, float *s, const float *x, const float *weight, int rows, int size,
                                 float epsilon, int gs) {
  const char *name = "llhip_rmsnorm_quantize_rows";
  if (rows <= 0 || size <= 0)
    return;
  if (!q || !s || !x || !weight) {
    raise("%s: null buffer", name);
    return;
  }
  if (!rmsnorm_quantize_fits(size, gs)) {
    raise("%s: %d values per row in groups of %d: at most 8192, a whole number of groups of a power of two from 4 to "
          "256", name, size, gs);
    return;
  }
  if (((uintptr_t)x | (uintptr_t)weight) & 15 || (uintptr_t)q & 3) {
    raise("%s: x and weight must be 16-byte aligned and q 4-byte aligned", name);
    return;
  }
  Call call(name);
  Ref X = call.in(x, (size_t)rows * size * sizeof(float)), W = call.in(weight, (size_t)size * sizeof(float));
  Ref Q = call.out(q, (size_t)rows * size, false), S = call.out(s, (size_t)rows * (size / gs) * sizeof(float), false);
  if (!call.ready())
    return;
  if (launch_rmsnorm_quantize(call.ptr<int8_t>(Q), call.ptr<float>(S), call.ptr<const float>(X),
                              call.ptr<const float>(W), rows, size, epsilon, gs, call.stream()))
    call.finish();
}

// ---- RoPE (kernels.h:61-68, src/kernels_simd.c:194-225, src/kernels.c:49-61) ----------------------------------

// The table is computed on the host with the C library's powf / cosf / sinf, the reference's own expressions, so it is
// bitwise the reference's on the same C library; device memory receives it by a copy.
void k_rope_table(const Config *p, int position, float *table) {
  if (!p || !table || p->head_dim <= 0 || p->head_dim % 2) {
    raise("k_rope_table: needs a configuration with an even head_dim and a table");
    return;
  }
  const int hd = p->head_dim;
  std::vector<float> host((size_t)2 * hd);
  for (int j = 0; j < hd; j += 2) {
    float freq = 1.0f / powf(p->rope_theta, (float)j / (float)hd); // src/kernels.c:49-61
    if (p->rope_type == 1) {
      const float wavelength = 6.2831853071795864769f / freq;
      if (wavelength > p->rope_original / p->rope_low)
        freq /= p->rope_factor;
      else if (wavelength >= p->rope_original / p->rope_high) {
        const float smooth = (p->rope_original / wavelength - p->rope_low) / (p->rope_high - p->rope_low);
        freq = (1 - smooth) * freq / p->rope_factor + smooth * freq;
      }
    }
    const float angle = position * freq, c = cosf(angle), s = sinf(angle);
    host[j] = host[j + 1] = c;
    host[hd + j] = -s;
    host[hd + j + 1] = s;
  }
  const size_t bytes = host.size() * sizeof(float);
  if (plain_host_memory(table, bytes)) {
    memcpy(table, host.data(), bytes);
    return;
  }
  Call call("k_rope_table");
  Ref T = call.out(table, bytes, false);
  if (!call.ready())
    return;
  if (hipMemcpyAsync(call.ptr<float>(T), host.data(), bytes, hipMemcpyHostToDevice, call.stream()) != hipSuccess ||
      hipStreamSynchronize(call.stream()) != hipSuccess) {
    (void)hipGetLastError();
    raise("k_rope_table: copying the table to the device failed");
    return;
  }
  call.finish();
}

void k_rope_apply(float *q, float *k, const float *table, int n_heads, int n_kv_heads, int head_dim) {
  rope("k_rope_apply", q, (size_t)n_heads * head_dim, k, (size_t)n_kv_heads * head_dim, table, 2 * (size_t)head_dim, 1,
       n_heads, n_kv_heads, head_dim);
}

void k_rope_apply_rows(float *q, size_t q_stride, float *k, size_t k_stride, const float *table, size_t table_stride,
                       int rows, int n_heads, int n_kv_heads, int head_dim) {
  rope("k_rope_apply_rows", q, q_stride, k, k_stride, table, table_stride, rows, n_heads, n_kv_heads, head_dim);
}

// ---- the K/V cache (kernels.h:168-179, src/attention.c:1375-1455) ---------------------------------------------

int kernels_kv_layout_head(void) { return kv_head_major() ? 1 : 0; }
const char *kernels_kv_layout_name(void) { return kv_head_major() ? "head" : "rows"; }

int kernels_kv_layout_select(const char *name) {
  if (!name)
    return 0;
  if (!strcmp(name, "rows"))
    kv_layout_head_flag = 0;
  else if (!strcmp(name, "head"))
    kv_layout_head_flag = 1;
  else
    return 0;
  return 1;
}

void k_kv_strides(int n_kv_heads, int head_dim, int seq_len, size_t *pos_stride, size_t *head_base) {
  strides(n_kv_heads, head_dim, seq_len, kv_head_major(), pos_stride, head_base);
}

void k_kv_store(float *cache, const float *src, size_t src_ld, int pos0, int count, int n_kv_heads, int head_dim,
                int seq_len) {
  if (count <= 0 || n_kv_heads <= 0 || head_dim <= 0)
    return;
  if (!cache || !src) {
    raise("k_kv_store: null buffer");
    return;
  }
  if (!positions_fit(pos0, count, seq_len)) {
    raise("k_kv_store: positions %d..%lld are outside the cache of %d", pos0, (long long)pos0 + count - 1, seq_len);
    return;
  }
  size_t pos_stride, head_base;
  strides(n_kv_heads, head_dim, seq_len, kv_head_major(), &pos_stride, &head_base);
  const size_t kv_dim = (size_t)n_kv_heads * head_dim, f = sizeof(float);
  Call call("k_kv_store", true); // may join a recorded RoPE
  Ref S = call.in2d(src, kv_dim * f, src_ld * f, (size_t)count);
  // the whole layer's cache: every position of every KV head (read too, so a staged copy keeps the other positions)
  Ref C = call.out(cache, (size_t)seq_len * kv_dim * f, true);
  if (!call.ready())
    return;
  float *cd = call.ptr<float>(C);
  const float *sd = call.ptr<const float>(S);
  if (count == 1 && !call.staged() && attach_kv_store(PendingKvStore{cd, sd, pos0, pos_stride, head_base}, n_kv_heads,
                                                      head_dim))
    return; // recorded with the RoPE before it
  if (flush_pending_quantize() &&
      launch_kv_store(cd, sd, src_ld, pos0, count, n_kv_heads, head_dim, pos_stride, head_base, call.stream()))
    call.finish();
}

// No counterpart in the reference: k_rope_apply_rows of q and k, then k_kv_store of k and of v at pos0.. (the engine's
// batched forward, src/tp.c:550-557), in one launch and bitwise those calls; rows of q, k and v and both caches
// 16-byte aligned, and the k and v rows outside both caches (a thread's cache store must not land on a row another
// thread has still to read).
void llhip_rope_kv_store_rows(float *q, size_t q_stride, float *k, const float *v, size_t kv_stride, const float *table,
                              size_t table_stride, int rows, int n_heads, int n_kv_heads, int head_dim,
                              float *key_cache, float *value_cache, int pos0, int seq_len) {
  const char *name = "llhip_rope_kv_store_rows";
  if (rows <= 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0)
    return;
  if (!q || !k || !v || !table || !key_cache || !value_cache) {
    raise("%s: null buffer", name);
    return;
  }
  if (head_dim % 4 || n_kv_heads > n_heads || q_stride % 4 || kv_stride % 4 || table_stride % 4 ||
      table_stride < 2 * (size_t)head_dim ||
      ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)table | (uintptr_t)key_cache |
       (uintptr_t)value_cache) & 15) {
    raise("%s: needs head_dim and the row strides multiples of 4, a table row per row and 16-byte aligned rows and "
          "caches", name);
    return;
  }
  if (!positions_fit(pos0, rows, seq_len)) {
    raise("%s: positions %d..%lld are outside the cache of %d", name, pos0, (long long)pos0 + rows - 1, seq_len);
    return;
  }
  size_t pos_stride, head_base;
  strides(n_kv_heads, head_dim, seq_len, kv_head_major(), &pos_stride, &head_base);
  const size_t f = sizeof(float), kv_dim = (size_t)n_kv_heads * head_dim;
  {
    const uintptr_t rows_bytes = ((size_t)(rows - 1) * kv_stride + kv_dim) * f, cache_bytes = (size_t)seq_len * kv_dim * f;
    auto overlaps = [&](const void *a, const void *cache) {
      return (uintptr_t)a < (uintptr_t)cache + cache_bytes && (uintptr_t)cache < (uintptr_t)a + rows_bytes;
    };
    if (overlaps(k, key_cache) || overlaps(k, value_cache) || overlaps(v, key_cache) || overlaps(v, value_cache)) {
      raise("%s: the k and v rows must lie outside both caches", name);
      return;
    }
  }
  Call call(name);
  Ref Q = call.out2d(q, (size_t)n_heads * head_dim * f, q_stride * f, (size_t)rows, true);
  Ref K = call.out2d(k, kv_dim * f, kv_stride * f, (size_t)rows, true);
  Ref V = call.in2d(v, kv_dim * f, kv_stride * f, (size_t)rows);
  Ref T = call.in2d(table, 2 * (size_t)head_dim * f, table_stride * f, (size_t)rows);
  Ref KC = call.out(key_cache, (size_t)seq_len * kv_dim * f, true), VC = call.out(value_cache, (size_t)seq_len * kv_dim * f, true);
  if (!call.ready())
    return;
  if (launch_rope_kv_rows(call.ptr<float>(Q), q_stride, call.ptr<float>(K), call.ptr<const float>(V), kv_stride,
                          call.ptr<const float>(T), table_stride, rows, n_heads, n_kv_heads, head_dim,
                          call.ptr<float>(KC), call.ptr<float>(VC), pos0, pos_stride, head_base, call.stream()))
    call.finish();
}

// ---- embedding rows (src/tp.c:395-396, 444-456) -------------------------------------------------------------------

void k_embed_q8_rows(float *out, const int8_t *table, const float *scales, const int *ids, int count, int dim, int gs,
                     int vocab) {
  if (count <= 0)
    return;
  if (!out || !table || !scales || !ids) {
    raise("k_embed_q8_rows: null buffer");
    return;
  }
  if (dim <= 0 || vocab <= 0 || gs <= 0 || ((size_t)vocab * dim) % gs != 0) {
    raise("k_embed_q8_rows: a %d x %d table in groups of %d", vocab, dim, gs);
    return;
  }
  const size_t values = (size_t)vocab * dim;
  Call call("k_embed_q8_rows");
  Ref T = call.in(table, values), S = call.in(scales, values / gs * sizeof(float));
  Ref I = call.in(ids, (size_t)count * sizeof(int));
  Ref O = call.out(out, (size_t)count * dim * sizeof(float), false);
  if (!call.ready())
    return;
  if (launch_embed_rows(call.ptr<float>(O), call.ptr<const int8_t>(T), call.ptr<const float>(S),
                        call.ptr<const int>(I), count, dim, gs, vocab, call.stream()))
    call.finish();
}

void k_embed_f32_rows(float *out, const float *table, const int *ids, int count, int dim, int vocab) {
  if (count <= 0)
    return;
  if (!out || !table || !ids) {
    raise("k_embed_f32_rows: null buffer");
    return;
  }
  if (dim <= 0 || vocab <= 0) {
    raise("k_embed_f32_rows: a %d x %d table", vocab, dim);
    return;
  }
  Call call("k_embed_f32_rows");
  Ref T = call.in(table, (size_t)vocab * dim * sizeof(float));
  Ref I = call.in(ids, (size_t)count * sizeof(int));
  Ref O = call.out(out, (size_t)count * dim * sizeof(float), false);
  if (!call.ready())
    return;
  if (launch_embed_rows_f32(call.ptr<float>(O), call.ptr<const float>(T), call.ptr<const int>(I), count, dim, vocab,
                            call.stream()))
    call.finish();
}

// ---- attention (kernels.h:124-179, src/attention.c:516-596, 1357-1455) -------------------------------------------
//
// The device attention keeps its split-K partials in a library workspace, so AttentionWork is the reference's record
// of the shapes: partial stays what the caller gave (NULL from k_attention_init), max_chunks is the chunk count of
// the longest context, workers 1, and nothing here reads or writes through partial.

size_t k_attention_bytes(int n_heads, int n_kv_heads, int head_dim, int seq_len) {
  (void)n_kv_heads;
  return attention_partial_floats(1, n_heads, head_dim, seq_len > 0 ? seq_len - 1 : 0) * sizeof(float);
}

size_t k_attention_bytes_rows(int n_heads, int n_kv_heads, int head_dim, int seq_len, int rows) {
  (void)n_kv_heads;
  return attention_partial_floats(rows > 0 ? rows : 1, n_heads, head_dim, seq_len > 0 ? seq_len - 1 : 0) *
         sizeof(float);
}

static void attention_record(AttentionWork *work, int n_heads, int head_dim, int seq_len, int rows, float *memory) {
  if (!work)
    return;
  work->partial = memory;
  work->max_chunks = chunk_count(seq_len > 0 ? seq_len - 1 : 0);
  work->n_heads = n_heads;
  work->head_dim = head_dim;
  work->workers = 1;
  work->external = memory != nullptr;
  work->capacity = attention_partial_floats(rows > 0 ? rows : 1, n_heads, head_dim, seq_len > 0 ? seq_len - 1 : 0);
}

void k_attention_init(AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len) {
  (void)n_kv_heads;
  attention_record(work, n_heads, head_dim, seq_len, 1, nullptr);
}

void k_attention_init_in(AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, float *memory) {
  (void)n_kv_heads;
  attention_record(work, n_heads, head_dim, seq_len, 1, memory);
}

void k_attention_init_rows(AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int rows,
                           float *memory) {
  (void)n_kv_heads;
  attention_record(work, n_heads, head_dim, seq_len, rows, memory);
}

int k_attention_chunk_count(const AttentionWork *work, int n_kv_heads, int position) {
  (void)work, (void)n_kv_heads;
  return chunk_count(position);
}

void k_attention_free(AttentionWork *work) {
  if (work)
    work->partial = nullptr;
}

void k_attention(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                 AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int position) {
  (void)att, (void)work;
  attention("k_attention", out, q, key_cache, value_cache, n_heads, n_kv_heads, head_dim, seq_len, position, 1,
            (size_t)n_kv_heads * head_dim, (size_t)head_dim);
}

void k_attention_layout(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                        AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int position,
                        size_t pos_stride, size_t head_base) {
  (void)att, (void)work;
  attention("k_attention_layout", out, q, key_cache, value_cache, n_heads, n_kv_heads, head_dim, seq_len, position, 1,
            pos_stride, head_base);
}

void k_attention_batch(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                       AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int pos0, int m) {
  (void)att, (void)work;
  attention("k_attention_batch", out, q, key_cache, value_cache, n_heads, n_kv_heads, head_dim, seq_len, pos0, m,
            (size_t)n_kv_heads * head_dim, (size_t)head_dim);
}

void k_attention_batch_layout(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                              AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int pos0,
                              int m, size_t pos_stride, size_t head_base) {
  (void)att, (void)work;
  attention("k_attention_batch_layout", out, q, key_cache, value_cache, n_heads, n_kv_heads, head_dim, seq_len, pos0,
            m, pos_stride, head_base);
}

void k_attention_batch_layout_noalloc(float *out, const float *q, const float *key_cache, const float *value_cache,
                                      float *att, AttentionWork *work, int n_heads, int n_kv_heads, int head_dim,
                                      int seq_len, int pos0, int m, size_t pos_stride, size_t head_base) {
  (void)att, (void)work;
  attention("k_attention_batch_layout_noalloc", out, q, key_cache, value_cache, n_heads, n_kv_heads, head_dim, seq_len,
            pos0, m, pos_stride, head_base, true);
}

void k_attention_kv(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                    AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int position) {
  size_t pos_stride, head_base;
  strides(n_kv_heads, head_dim, seq_len, kv_head_major(), &pos_stride, &head_base);
  k_attention_layout(out, q, key_cache, value_cache, att, work, n_heads, n_kv_heads, head_dim, seq_len, position,
                     pos_stride, head_base);
}

void k_attention_batch_kv(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                          AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int pos0,
                          int m) {
  size_t pos_stride, head_base;
  strides(n_kv_heads, head_dim, seq_len, kv_head_major(), &pos_stride, &head_base);
  k_attention_batch_layout(out, q, key_cache, value_cache, att, work, n_heads, n_kv_heads, head_dim, seq_len, pos0, m,
                           pos_stride, head_base);
}

void llhip_attention_batch_quantize(int8_t *q, float *s, int gs, float *out, const float *query, const float *key_cache,
                                    const float *value_cache, int n_heads, int n_kv_heads, int head_dim, int seq_len,
                                    int pos0, int m) {
  const char *name = "llhip_attention_batch_quantize";
  if (!q || !s) {
    raise("%s: null buffer", name);
    return;
  }
  if ((gs != 16 && gs != 32 && gs != 64 && gs != 128) || head_dim <= 0 || head_dim % gs) {
    raise("%s: group size %d must be 16, 32, 64 or 128 and divide head_dim %d", name, gs, head_dim);
    return;
  }
  if ((uintptr_t)q & 3) {
    raise("%s: q must be 4-byte aligned", name);
    return;
  }
  size_t pos_stride, head_base;
  strides(n_kv_heads, head_dim, seq_len, kv_head_major(), &pos_stride, &head_base);
  attention(name, out, query, key_cache, value_cache, n_heads, n_kv_heads, head_dim, seq_len, pos0, m, pos_stride,
            head_base, false, q, s, gs);
}

// kernels.h:45-47 and testing.h: one device kernel serves both forms (split K over 64-position chunks).
const char *kernels_attention_name(void) { return "split"; }
const char *kernels_attention_decode_name(void) { return "split"; }
int kernels_attention_select(const char *batch, const char *decode) {
  const bool batch_ok = !batch || !strcmp(batch, "tiled") || !strcmp(batch, "split");
  const bool decode_ok = !decode || !strcmp(decode, "split") || !strcmp(decode, "group");
  return batch_ok && decode_ok ? 1 : 0;
}

} // extern "C"
