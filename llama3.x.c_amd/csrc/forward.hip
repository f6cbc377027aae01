// The forward around the matmuls on gfx950: RMSNorm, RoPE, the K/V cache store and causal attention (decode and
// batched), so activations can stay in HBM between layers. Citations are LucianCrainic/llama3.x.c file:line.
//
//   rmsnorm_rows   one 1024-thread block per row: the sum of squares reduced over the block, then out = w * (ss * x) in the
//                  reference's operation order (src/kernels.c:8-21). HBM-bound: 8 bytes read + 4 written per value.
//   rope_rows      one thread per (row, head, pair), products rounded before the sum (no fused multiply-add), so the
//                  result is bitwise the reference's (src/kernels_simd.c:203-225).
//   kv_store       a strided copy into the rows or head-major cache layout (src/attention.c:1420-1432).
//   attn_chunks    split-K attention: one block per (query row, KV head, chunk of kChunk positions) scores the
//                  chunk for every query head of the group (the K row read once serves kv_mul heads), keeps the
//                  chunk's maximum and sum of exponentials and the unnormalized value sum (src/attention.c:841-876);
//                  attn_merge rescales the chunks by exp(m_c - M) and normalizes (src/attention.c:664-682).
//                  HBM-bound on the K/V cache: 8 * kv_dim bytes per position and query row.
#include <cfloat>
#include <type_traits>

#include <cstring>

#include "common.h"
#include "lanes.h"
#include "quant.h"

typedef float v4f __attribute__((ext_vector_type(4)));

namespace llhip {
namespace {

constexpr int kWave = 64;
constexpr int kThreads = 256;
constexpr int kChunk = 64;      // positions per attention block
constexpr int kMaxHeadDim = 256;
constexpr int kMaxGroup = 16;   // query heads per KV head

bool launch_ok(const char *what) {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess || raise("launching %s failed: %s", what, hipGetErrorString(e));
}

// ---- RMSNorm -----------------------------------------------------------------------------------------------------

constexpr int kNormThreads = 1024;

// One block per row. Aligned rows (size % 4 == 0, 16-byte aligned) are read as float4, so a 4096-value row is one
// load per thread, all in flight at once.
__global__ __launch_bounds__(kNormThreads) void rmsnorm_rows(float *__restrict__ out, const float *__restrict__ x,
                                                             const float *__restrict__ weight, int size, float epsilon,
                                                             bool vec4) {
  __shared__ float part[kNormThreads / kWave];
  const float *row = x + (size_t)blockIdx.x * size;
  float *o = out + (size_t)blockIdx.x * size;
  float ss = 0.0f;
  if (vec4) {
    for (int j = 4 * threadIdx.x; j < size; j += 4 * kNormThreads) {
      const float4 v = *reinterpret_cast<const float4 *>(row + j);
      ss = fmaf(v.x, v.x, ss);
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
    }
  } else {
    for (int j = threadIdx.x; j < size; j += kNormThreads)
      ss = fmaf(row[j], row[j], ss);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & (kWave - 1)) == 0)
    part[threadIdx.x / kWave] = ss;
  __syncthreads();
  ss = 0.0f;
#pragma unroll
  for (int w = 0; w < kNormThreads / kWave; w++)
    ss += part[w];
  // src/kernels.c:15-17, the same three roundings (correctly rounded division and square root)
  ss /= size;
  ss += epsilon;
  ss = 1.0f / sqrtf(ss);
  // out may be x: each value is read by the thread that writes it, after every thread's sum is in
  if (vec4) {
    for (int j = 4 * threadIdx.x; j < size; j += 4 * kNormThreads) {
      const float4 v = *reinterpret_cast<const float4 *>(row + j), w = *reinterpret_cast<const float4 *>(weight + j);
      *reinterpret_cast<float4 *>(o + j) = float4{w.x * (ss * v.x), w.y * (ss * v.y), w.z * (ss * v.z), w.w * (ss * v.w)};
    }
  } else {
    for (int j = threadIdx.x; j < size; j += kNormThreads)
      o[j] = weight[j] * (ss * row[j]);
  }
}

// ---- RoPE ---------------------------------------------------------------------------------------------------------

__device__ __forceinline__ void rotate(float *v, float c, float s) {
#pragma clang fp contract(off) // a*c - b*s and a*s + b*c with the products rounded, as the reference computes them
  const float a = v[0], b = v[1];
  v[0] = a * c - b * s;
  v[1] = a * s + b * c;
}

// The cosines and sines of the pairs (j0, j0 + 1) and (j0 + 2, j0 + 3) of a row: c = table[j], s = table[hd + j + 1].
struct Rot4 {
  float c0, s0, c1, s1;
};
__device__ __forceinline__ Rot4 rot4_of(const float *table, int hd, int j0) {
  return Rot4{table[j0], table[hd + j0 + 1], table[j0 + 2], table[hd + j0 + 3]};
}

// Two pairs of a row rotated like rotate(), by the cosines and sines of rot4_of.
__device__ __forceinline__ float4 rotate4(float4 v, const Rot4 &r) {
  float a[2] = {v.x, v.y}, b[2] = {v.z, v.w};
  rotate(a, r.c0, r.s0);
  rotate(b, r.c1, r.s1);
  return float4{a[0], a[1], b[0], b[1]};
}
__device__ __forceinline__ float4 rotate4(float4 v, const float *table, int hd, int j0) {
  return rotate4(v, rot4_of(table, hd, j0));
}

// Thread i: row i / (n_heads * half), head and pair from the rest; k is rotated for heads below n_kv_heads.
__global__ __launch_bounds__(kThreads) void rope_rows(float *__restrict__ q, size_t q_stride, float *__restrict__ k,
                                                      size_t k_stride, const float *__restrict__ table,
                                                      size_t table_stride, int rows, int n_heads, int n_kv_heads,
                                                      int head_dim) {
  const int half = head_dim / 2;
  const long long per_row = (long long)n_heads * half;
  const long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i >= per_row * rows)
    return;
  const int row = (int)(i / per_row), rest = (int)(i % per_row);
  const int h = rest / half, j = 2 * (rest % half);
  const float *t = table + (size_t)row * table_stride;
  const float c = t[j], s = t[head_dim + j + 1];
  rotate(q + (size_t)row * q_stride + (size_t)h * head_dim + j, c, s);
  if (h < n_kv_heads)
    rotate(k + (size_t)row * k_stride + (size_t)h * head_dim + j, c, s);
}

// ---- K/V cache store ------------------------------------------------------------------------------------------------

__global__ __launch_bounds__(kThreads) void kv_store(float *__restrict__ cache, const float *__restrict__ src,
                                                     size_t src_ld, int pos0, int count, int n_kv_heads, int head_dim,
                                                     size_t pos_stride, size_t head_base) {
  const long long kv_dim = (long long)n_kv_heads * head_dim;
  const long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i >= kv_dim * count)
    return;
  const int r = (int)(i / kv_dim), rest = (int)(i % kv_dim);
  const int g = rest / head_dim, d = rest % head_dim;
  cache[(size_t)(pos0 + r) * pos_stride + (size_t)g * head_base + d] = src[(size_t)r * src_ld + rest];
}

// RoPE of a batch of rows and their K/V cache stores in one launch: thread i takes four dimensions (one float4) of row
// r's q heads, then of its k heads, then of its v heads. q and k are rotated as rope_rows rotates them (the same
// products, rounded the same way), k and v go into the cache at position pos0 + r, and k is also written back rotated:
// bitwise rope_rows then the two kv_store calls. 16-byte aligned rows, head_dim % 4 == 0.
__global__ __launch_bounds__(kThreads) void rope_kv_rows(float *__restrict__ q, size_t q_stride, float *__restrict__ k,
                                                         const float *__restrict__ v, size_t kv_stride,
                                                         const float *__restrict__ table, size_t table_stride, int rows,
                                                         int n_heads, int n_kv_heads, int head_dim,
                                                         float *__restrict__ key_cache, float *__restrict__ value_cache,
                                                         int pos0, size_t pos_stride, size_t head_base) {
  const int hd4 = head_dim / 4, qu = n_heads * hd4, ku = n_kv_heads * hd4;
  const long long per_row = qu + 2LL * ku;
  const long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i >= per_row * rows)
    return;
  const int r = (int)(i / per_row), u = (int)(i % per_row);
  const float *t = table + (size_t)r * table_stride;
  if (u < qu) {
    const int h = u / hd4, d = 4 * (u % hd4);
    float4 *p = reinterpret_cast<float4 *>(q + (size_t)r * q_stride + (size_t)h * head_dim + d);
    *p = rotate4(*p, t, head_dim, d);
    return;
  }
  const bool is_k = u < qu + ku;
  const int w = is_k ? u - qu : u - qu - ku, g = w / hd4, d = 4 * (w % hd4);
  const size_t at = (size_t)r * kv_stride + (size_t)g * head_dim + d;
  const size_t slot = (size_t)(pos0 + r) * pos_stride + (size_t)g * head_base + d;
  if (is_k) {
    float4 *p = reinterpret_cast<float4 *>(k + at);
    const float4 x = rotate4(*p, t, head_dim, d);
    *p = x;
    *reinterpret_cast<float4 *>(key_cache + slot) = x;
  } else {
    *reinterpret_cast<float4 *>(value_cache + slot) = *reinterpret_cast<const float4 *>(v + at);
  }
}

// rope_kv_rows for head_dim HD = 64 or 128: thread (row, d4) takes dimensions 4 d4 .. 4 d4 + 3 of every head of its
// row (q heads, then k, then v), so the row's table values for them are loaded once and all of its loads are in
// flight together; each element gets the same products in the same order as in rope_kv_rows, so the results are
// bitwise those of rope_kv_rows.
template <int HD>
__global__ __launch_bounds__(kThreads) void rope_kv_rows_hd(float *__restrict__ q, size_t q_stride, float *__restrict__ k,
                                                            const float *__restrict__ v, size_t kv_stride,
                                                            const float *__restrict__ table, size_t table_stride,
                                                            int rows, int n_heads, int n_kv_heads,
                                                            float *__restrict__ key_cache,
                                                            float *__restrict__ value_cache, int pos0,
                                                            size_t pos_stride, size_t head_base) {
  constexpr int hd4 = HD / 4, kRowsPerBlock = kThreads / hd4;
  const int r = blockIdx.x * kRowsPerBlock + threadIdx.x / hd4, d = 4 * (threadIdx.x % hd4);
  if (r >= rows)
    return;
  const Rot4 rot = rot4_of(table + (size_t)r * table_stride, HD, d);
  float *qr = q + (size_t)r * q_stride + d;
  for (int h = 0; h < n_heads; h++) {
    float4 *pq = reinterpret_cast<float4 *>(qr + (size_t)h * HD);
    *pq = rotate4(*pq, rot);
  }
  const size_t slot0 = (size_t)(pos0 + r) * pos_stride + d;
  for (int g = 0; g < n_kv_heads; g++) {
    const size_t at = (size_t)r * kv_stride + (size_t)g * HD + d, slot = slot0 + (size_t)g * head_base;
    float4 *pk = reinterpret_cast<float4 *>(k + at);
    const float4 x = rotate4(*pk, rot);
    *pk = x;
    *reinterpret_cast<float4 *>(key_cache + slot) = x;
    *reinterpret_cast<float4 *>(value_cache + slot) = *reinterpret_cast<const float4 *>(v + at);
  }
}

// ---- embedding rows -------------------------------------------------------------------------------------------------

// out[i][j] = table[ids[i]][j] * scales[(ids[i] * dim + j) / gs]: the int8 value converted exactly and one float
// product, bitwise the reference's lookup (src/tp.c:395-396, 444-456). An id outside [0, vocab) raises flag 2 and
// leaves its row untouched. One thread per value; the table row is read once.
__global__ __launch_bounds__(kThreads) void embed_rows(float *__restrict__ out, const int8_t *__restrict__ table,
                                                       const float *__restrict__ scales, const int *__restrict__ ids,
                                                       int count, int dim, int gs, int vocab, int *flags) {
  const long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i >= (long long)count * dim)
    return;
  const int r = (int)(i / dim), j = (int)(i % dim), id = ids[r];
  if (id < 0 || id >= vocab) {
    flags[2] = 1;
    return;
  }
  const size_t at = (size_t)id * dim + j;
  out[(size_t)r * dim + j] = (float)table[at] * scales[at / gs];
}

// The FP32 table's lookup (src/tp.c:342 for a token, 449 for a batch): a copy of row ids[i], 16 bytes per thread when
// dim is a multiple of 4 (the table's rows are then 16-byte aligned), else one value per thread. An id outside
// [0, vocab) raises flag 2 and leaves its row untouched.
template <int V>
__global__ __launch_bounds__(kThreads) void embed_rows_f32(float *__restrict__ out, const float *__restrict__ table,
                                                           const int *__restrict__ ids, int count, int dim, int vocab,
                                                           int *flags) {
  using Vec = typename std::conditional<V == 4, float4, float>::type;
  const int per_row = dim / V;
  const long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i >= (long long)count * per_row)
    return;
  const int r = (int)(i / per_row), j = (int)(i % per_row), id = ids[r];
  if (id < 0 || id >= vocab) {
    flags[2] = 1;
    return;
  }
  reinterpret_cast<Vec *>(out + (size_t)r * dim)[j] = reinterpret_cast<const Vec *>(table + (size_t)id * dim)[j];
}

// ---- attention ------------------------------------------------------------------------------------------------------

struct AttnParams {
  float *out;
  const float *q, *key, *value;
  float *partial; // [row][head][chunk][slot]: unnormalized value sum, chunk maximum, chunk sum (slot = head_dim + 2
                  // rounded up to 4 floats, so every slot starts 16-byte aligned)
  int *flags;
  int n_heads, n_kv_heads, head_dim, pos0, chunks; // chunks: per row, for the last row's position
  int rows, tile_rows;                              // query rows, and rows per attn_tile block
  int slot;                                         // floats per partial
  // fused RoPE and cache store (decode): q (written back rotated), the new k row (likewise) and v row, the table
  float *rope_q, *k_new;
  const float *v_new, *table;
  size_t pos_stride, head_base;
  float divisor; // sqrtf(head_dim)
  int splits;    // batched flash form: blocks per tile, each over a share of its chunks (0: the tile whole)
  // attn_flash3 unsplit: the output rows quantized in groups of qgs values (k_quantize) instead of stored in FP32
  int8_t *qout;
  float *qscale;
  int qgs;
};

constexpr int kTileThreads = 512;
constexpr int kTileWaves = kTileThreads / kWave;
constexpr int kMaxQv = 64; // query vectors (tile rows x the group's query heads) per attn_tile block
constexpr int kQvGroup = 4; // query vectors per pass in the batched form
constexpr int kTileLoads = 4; // K, V and query items per thread loaded together (64 positions x 128 dimensions)

// The aligned form (head_dim % 4 == 0, 16-byte aligned rows): block (chunk c, KV head g, tile of tile_rows query rows).
// The chunk's K rows and the tile's query vectors are staged in LDS (K rows padded to head_dim + 4 floats, so lane t's
// 16-byte reads of row t fall on distinct banks); wave w scores query vectors w, w + 8, ... with lane t taking position
// t0 + t (one dot per lane, no cross-lane sum), masks positions past each row's own (causal), and keeps the chunk
// maximum, the exponentials and their sum; then each work item (query vector, four dimensions) sums the
// exponential-weighted V rows staged beside K. The K and V rows of a chunk are read once, all loads in flight
// together, for all tile_rows x kv_mul query vectors.
// GROUP > 1 (batched rows, every tile's query-vector count a multiple of GROUP): a wave scores GROUP query vectors per
// pass over its lane's K row and a thread sums GROUP vectors' values per V read, so each K or V value read from LDS
// serves GROUP products; every dot and sum keeps its order of terms, so the results equal GROUP = 1's.
// HD: the head dimension when it is known at compile time (64 or 128; 0 takes p.head_dim), so the dot and the value
// sums unroll and their LDS reads are issued ahead of the products instead of one latency per step.
template <int GROUP, int HD> __global__ __launch_bounds__(kTileThreads) void attn_tile(AttnParams p) {
  extern __shared__ __align__(16) float lds[];
  const int c = blockIdx.x, g = blockIdx.y, r0 = blockIdx.z * p.tile_rows;
  const int nrows = min(p.tile_rows, p.rows - r0);
  const int last = p.pos0 + r0 + nrows - 1; // the tile's last position
  const int t0 = c * kChunk;
  if (t0 > last)
    return; // no row of the tile reaches this chunk; the merge reads only each row's own chunks
  const int n = min(kChunk, last + 1 - t0);
  const int kv_mul = p.n_heads / p.n_kv_heads, hd = HD ? HD : p.head_dim, hd4 = hd / 4, kst = hd + 4;
  const int nqv = nrows * kv_mul;
  float *ks = lds, *vs = ks + kChunk * kst, *qs = vs + kChunk * hd, *es = qs + p.tile_rows * kv_mul * hd;
  const float *kbase = p.key + (size_t)g * p.head_base, *vbase = p.value + (size_t)g * p.head_base;
  const bool fresh = p.table != nullptr; // decode with the RoPE and the new cache row folded in
  // Loads: work item i is 4 dimensions (d4) of K row t (and of V row t) and of query vector qv, i = t * hd4 + d4 =
  // qv * hd4 + d4. The first kTileLoads items of each thread are loaded together, K, the query vectors (and the RoPE
  // factors) first and V last, and nothing waits for V before the scores are computed. Row and query indices past
  // the chunk's or tile's last clamp to it, so every one of those loads reads a valid address; only items in range
  // are stored. The new row (fresh: it lies in this chunk, which no other block reads) comes from the QKV outputs.
  const int kv_items = n * hd4, q_items = nqv * hd4;
  float4 kr[kTileLoads], qr[kTileLoads];
  Rot4 rot[kTileLoads];
#pragma unroll
  for (int u = 0; u < kTileLoads; u++) {
    const int i = threadIdx.x + u * kTileThreads, d4 = i % hd4;
    const int t = min(i / hd4, n - 1), qv = min(i / hd4, nqv - 1), j = qv / kv_mul, h = qv % kv_mul;
    const bool novel = fresh && t0 + t == p.pos0;
    const size_t at = (size_t)(t0 + t) * p.pos_stride + 4 * d4, src = (size_t)g * hd + 4 * d4;
    kr[u] = *reinterpret_cast<const float4 *>(novel ? p.k_new + src : kbase + at);
    qr[u] = *reinterpret_cast<const float4 *>(p.q + ((size_t)(r0 + j) * p.n_heads + (size_t)g * kv_mul + h) * hd +
                                              4 * d4);
    if (fresh && (i < q_items || novel)) // the RoPE factors only where a query value or the new K row needs them
      rot[u] = rot4_of(p.table, hd, 4 * d4);
  }
  // V stays in four named registers through the scores (an array indexed after the score loop went to scratch)
  auto v_load = [&](int u) {
    const int i = threadIdx.x + u * kTileThreads, d4 = i % hd4, t = min(i / hd4, n - 1);
    const bool novel = fresh && t0 + t == p.pos0;
    return *reinterpret_cast<const float4 *>(novel ? p.v_new + (size_t)g * hd + 4 * d4
                                                   : vbase + (size_t)(t0 + t) * p.pos_stride + 4 * d4);
  };
  auto v_store = [&](int u, const float4 &v) {
    const int i = threadIdx.x + u * kTileThreads, t = i / hd4, d4 = i % hd4;
    if (i < kv_items) {
      if (fresh && t0 + t == p.pos0)
        *reinterpret_cast<float4 *>(const_cast<float *>(vbase) + (size_t)(t0 + t) * p.pos_stride + 4 * d4) = v;
      *reinterpret_cast<float4 *>(vs + t * hd + 4 * d4) = v;
    }
  };
  static_assert(kTileLoads == 4, "four V registers");
  const float4 vr0 = v_load(0), vr1 = v_load(1), vr2 = v_load(2), vr3 = v_load(3);
#pragma unroll
  for (int u = 0; u < kTileLoads; u++) {
    const int i = threadIdx.x + u * kTileThreads, t = i / hd4, d4 = i % hd4;
    if (i < kv_items) {
      float4 kv = kr[u];
      if (fresh && t0 + t == p.pos0) { // k rotated, stored into the cache and written back rotated
        kv = rotate4(kv, rot[u]);
        const size_t src = (size_t)g * hd + 4 * d4, at = (size_t)(t0 + t) * p.pos_stride + 4 * d4;
        *reinterpret_cast<float4 *>(p.k_new + src) = kv;
        *reinterpret_cast<float4 *>(const_cast<float *>(kbase) + at) = kv;
      }
      *reinterpret_cast<float4 *>(ks + t * kst + 4 * d4) = kv;
    }
    if (i < q_items) // every block rotates its own copy; attn_merge writes q back rotated once all blocks have read it
      *reinterpret_cast<float4 *>(qs + i / hd4 * hd + 4 * d4) = fresh ? rotate4(qr[u], rot[u]) : qr[u];
  }
  // items past the first kTileLoads per thread (head_dim above 128, or more than 2048 query values)
  for (int i = threadIdx.x + kTileLoads * kTileThreads; i < kv_items; i += kTileThreads) {
    const int t = i / hd4, d4 = i % hd4;
    const size_t at = (size_t)(t0 + t) * p.pos_stride + 4 * d4;
    float4 kv, vv;
    if (fresh && t0 + t == p.pos0) {
      const size_t src = (size_t)g * hd + 4 * d4;
      kv = rotate4(*reinterpret_cast<const float4 *>(p.k_new + src), p.table, hd, 4 * d4);
      vv = *reinterpret_cast<const float4 *>(p.v_new + src);
      *reinterpret_cast<float4 *>(p.k_new + src) = kv;
      *reinterpret_cast<float4 *>(const_cast<float *>(kbase) + at) = kv;
      *reinterpret_cast<float4 *>(const_cast<float *>(vbase) + at) = vv;
    } else {
      kv = *reinterpret_cast<const float4 *>(kbase + at);
      vv = *reinterpret_cast<const float4 *>(vbase + at);
    }
    *reinterpret_cast<float4 *>(ks + t * kst + 4 * d4) = kv;
    *reinterpret_cast<float4 *>(vs + t * hd + 4 * d4) = vv;
  }
  for (int i = threadIdx.x + kTileLoads * kTileThreads; i < q_items; i += kTileThreads) {
    const int qv = i / hd4, d4 = i % hd4, j = qv / kv_mul, h = qv % kv_mul;
    const size_t at = ((size_t)(r0 + j) * p.n_heads + (size_t)g * kv_mul + h) * hd + 4 * d4;
    float4 v = *reinterpret_cast<const float4 *>(p.q + at);
    if (fresh)
      v = rotate4(v, p.table, hd, 4 * d4);
    *reinterpret_cast<float4 *>(qs + qv * hd + 4 * d4) = v;
  }
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  bool bad = false;
  for (int q0 = wave * GROUP; q0 < nqv; q0 += kTileWaves * GROUP) {
    float dots[GROUP];
#pragma unroll
    for (int u = 0; u < GROUP; u++)
      dots[u] = 0.0f;
    if (lane < n && t0 + lane <= p.pos0 + r0 + (q0 + GROUP - 1) / kv_mul) { // live for some vector of the group
      const float *kr = ks + lane * kst, *qr = qs + q0 * hd;
      auto add4 = [&](const float4 &a, const float4 &b, float &dot) {
        dot = fmaf(a.x, b.x, dot);
        dot = fmaf(a.y, b.y, dot);
        dot = fmaf(a.z, b.z, dot);
        dot = fmaf(a.w, b.w, dot);
      };
      if constexpr (HD > 0) {
        // batches of B float4 of K (and of each query vector), the next batch's reads issued before this batch's
        // products, so one LDS latency is exposed per dot rather than one per step; same order of terms
        constexpr int B = GROUP >= 4 ? 1 : 4 / GROUP, NB = HD / (4 * B);
        static_assert(HD % (4 * B) == 0, "whole batches");
        float4 kb[2][B], qb[2][B][GROUP];
        auto load = [&](int slot, int i0) {
#pragma unroll
          for (int b = 0; b < B; b++) {
            kb[slot][b] = *reinterpret_cast<const float4 *>(kr + i0 + 4 * b);
#pragma unroll
            for (int u = 0; u < GROUP; u++)
              qb[slot][b][u] = *reinterpret_cast<const float4 *>(qr + u * HD + i0 + 4 * b);
          }
        };
        load(0, 0);
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
          if (nb + 1 < NB)
            load((nb + 1) & 1, 4 * B * (nb + 1));
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int b = 0; b < B; b++)
#pragma unroll
            for (int u = 0; u < GROUP; u++)
              add4(kb[nb & 1][b], qb[nb & 1][b][u], dots[u]);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
        for (int i = 0; i < hd; i += 4) {
          const float4 a = *reinterpret_cast<const float4 *>(kr + i);
#pragma unroll
          for (int u = 0; u < GROUP; u++)
            add4(a, *reinterpret_cast<const float4 *>(qr + u * hd + i), dots[u]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < GROUP; u++) {
    const int qv = q0 + u;
    const int j = qv / kv_mul, h = qv % kv_mul, pos = p.pos0 + r0 + j;
    const bool live = lane < n && t0 + lane <= pos;
    float s = -FLT_MAX;
    if (live) {
      s = dots[u] / p.divisor;
      bad |= !isfinite(s);
    }
    const float m = wave_max(s);
    const float e = live ? expf(s - m) : 0.0f;
    es[qv * kChunk + lane] = e;
    const float l = wave_sum(e);
    if (lane == 0 && t0 <= pos) {
      float *ph = p.partial + (((size_t)(r0 + j) * p.n_heads + (size_t)g * kv_mul + h) * p.chunks + c) * p.slot;
      ph[hd] = m;
      ph[hd + 1] = l;
    }
    }
  }
  if (bad)
    p.flags[1] = 1;
  v_store(0, vr0);
  v_store(1, vr1);
  v_store(2, vr2);
  v_store(3, vr3);
  __syncthreads();
  // value sums: work item (query vector, 4 consecutive dimensions), the exponentials of its row against the V rows
  for (int it = threadIdx.x; it < nqv / GROUP * hd4; it += kTileThreads) {
    const int q0 = it / hd4 * GROUP, d4 = it % hd4;
    if (t0 > p.pos0 + r0 + (q0 + GROUP - 1) / kv_mul)
      continue; // no row of the group reaches the chunk
    const float *er = es + q0 * kChunk, *vr = vs + 4 * d4;
    float4 acc[GROUP];
#pragma unroll
    for (int u = 0; u < GROUP; u++)
      acc[u] = float4{0.0f, 0.0f, 0.0f, 0.0f};
    auto add_row = [&](int t) {
      const float4 v = *reinterpret_cast<const float4 *>(vr + t * hd);
#pragma unroll
      for (int u = 0; u < GROUP; u++) {
        const float e = er[u * kChunk + t];
        acc[u].x = fmaf(e, v.x, acc[u].x);
        acc[u].y = fmaf(e, v.y, acc[u].y);
        acc[u].z = fmaf(e, v.z, acc[u].z);
        acc[u].w = fmaf(e, v.w, acc[u].w);
      }
    };
    if (n == kChunk) { // a whole chunk: unrolled, the reads of later rows in flight while earlier rows are summed
#pragma unroll 16
      for (int t = 0; t < kChunk; t++)
        add_row(t);
    } else {
      for (int t = 0; t < n; t++)
        add_row(t);
    }
#pragma unroll
    for (int u = 0; u < GROUP; u++) {
      const int qv = q0 + u, j = qv / kv_mul, h = qv % kv_mul;
      if (t0 <= p.pos0 + r0 + j) // rows that reach the chunk
        *reinterpret_cast<float4 *>(p.partial +
                                    (((size_t)(r0 + j) * p.n_heads + (size_t)g * kv_mul + h) * p.chunks + c) * p.slot +
                                    4 * d4) = acc[u];
    }
  }
}

// Decode (one query row; the kv_mul query vectors of KV head g share every K and V row). Block (chunk c, KV head g),
// 512 threads, HD dimensions known at compile time (64 or 128), kv_mul <= 8:
//   - K rows go from global memory straight into registers, read once for all the vectors (no LDS copy): wave w holds
//     rows 8 w .. 8 w + 7, eight lanes a row, lane ds of a row its float4 ds, ds + 8, ... (each load instruction reads
//     128 contiguous bytes of eight rows). A lane forms its partial dot with every query vector (read from LDS), and
//     the row's eight lanes add theirs by DPP, so every dot is whole in registers;
//   - wave v then masks vector v's 64 scores, takes the chunk maximum, the exponentials and their sum as attn_tile
//     does, while the other waves store the V rows (whose loads land meanwhile) into LDS;
//   - the value sums run over all 512 threads: item (vector, four dimensions) and a slice of the chunk's positions,
//     the position slices added in order in LDS.
// Each dot and value sum is attn_tile's sum in another association (within FP32 rounding). With the fused RoPE (table
// set), the new row's lanes rotate their K values and store them into the cache and back into k_new, and the V item
// threads of that row store it into the cache, as attn_tile does.
constexpr int kDecodeMaxQv = 8;
template <int HD> __global__ __launch_bounds__(kTileThreads) void attn_decode(AttnParams p) {
  extern __shared__ __align__(16) float lds[];
  constexpr int HD4 = HD / 4, KPER = HD4 / 8, VPER = kChunk * HD4 / kTileThreads;
  static_assert(KPER >= 1 && kChunk == 8 * kTileWaves && kChunk * HD4 % kTileThreads == 0, "rows and V items");
  const int c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  const int t0 = c * kChunk;
  if (t0 > p.pos0)
    return; // past the row's position; the merge reads only its own chunks
  const int n = min(kChunk, p.pos0 + 1 - t0);
  const int nqv = p.n_heads / p.n_kv_heads; // query vectors of the KV head (<= kDecodeMaxQv)
  float *vs = lds, *qs = vs + kChunk * HD, *dots = qs + nqv * HD, *es = dots + nqv * kChunk;
  float4 *po = reinterpret_cast<float4 *>(es + nqv * kChunk);
  const float *kbase = p.key + (size_t)g * p.head_base, *vbase = p.value + (size_t)g * p.head_base;
  const bool fresh = p.table != nullptr;
  const int lane = tid & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int row = 8 * wave + lane / 8, ds = lane % 8; // this lane's K row and its place in the row
  const int t = min(row, n - 1);                      // clamped: rows past the chunk's end are masked
  const bool novel_k = fresh && t0 + t == p.pos0;
  const float4 zero4 = float4{0.0f, 0.0f, 0.0f, 0.0f};
  // RoPE factors as two float4 of the table: cosines at j0 .. j0 + 3, sines at HD + j0 .. HD + j0 + 3
  auto factors = [&](const float4 &cs, const float4 &sn) { return Rot4{cs.x, sn.y, cs.z, sn.w}; };

  // Loads, all issued before the first wait: this lane's K values, one query item, the V items.
  float4 kreg[KPER], kcos[KPER], ksin[KPER];
#pragma unroll
  for (int s = 0; s < KPER; s++) {
    const int d4 = 8 * s + ds;
    kreg[s] = *reinterpret_cast<const float4 *>(novel_k ? p.k_new + (size_t)g * HD + 4 * d4
                                                        : kbase + (size_t)(t0 + t) * p.pos_stride + 4 * d4);
    kcos[s] = ksin[s] = zero4;
    if (novel_k) {
      kcos[s] = *reinterpret_cast<const float4 *>(p.table + 4 * d4);
      ksin[s] = *reinterpret_cast<const float4 *>(p.table + HD + 4 * d4);
    }
  }
  const bool has_q = tid < nqv * HD4;
  const int qv = has_q ? tid / HD4 : 0, qd4 = tid % HD4;
  float4 qreg = zero4, qcos = zero4, qsin = zero4;
  if (has_q) {
    qreg = *reinterpret_cast<const float4 *>(p.q + ((size_t)g * nqv + qv) * HD + 4 * qd4);
    if (fresh) {
      qcos = *reinterpret_cast<const float4 *>(p.table + 4 * qd4);
      qsin = *reinterpret_cast<const float4 *>(p.table + HD + 4 * qd4);
    }
  }
  // V items in named registers (an array indexed across the dot phase was placed in scratch)
  auto v_load = [&](int u) {
    const int i = tid + u * kTileThreads, tv = min(i / HD4, n - 1), d4 = i % HD4;
    const bool novel_v = fresh && t0 + tv == p.pos0;
    return *reinterpret_cast<const float4 *>(novel_v ? p.v_new + (size_t)g * HD + 4 * d4
                                                     : vbase + (size_t)(t0 + tv) * p.pos_stride + 4 * d4);
  };
  auto v_store = [&](int u, const float4 &x) {
    const int i = tid + u * kTileThreads, tv = i / HD4, d4 = i % HD4;
    *reinterpret_cast<float4 *>(vs + tv * HD + 4 * d4) = x;
    if (fresh && tv < n && t0 + tv == p.pos0)
      *reinterpret_cast<float4 *>(const_cast<float *>(vbase) + (size_t)(t0 + tv) * p.pos_stride + 4 * d4) = x;
  };
  static_assert(VPER == 2 || VPER == 4, "two or four V items per thread");
  const float4 v0 = v_load(0), v1 = v_load(1), v2 = VPER == 4 ? v_load(2) : zero4, v3 = VPER == 4 ? v_load(3) : zero4;
  if (novel_k) { // the new row's K: rotated; the lanes of the real row store it into the cache and back into k_new
#pragma unroll
    for (int s = 0; s < KPER; s++) {
      kreg[s] = rotate4(kreg[s], factors(kcos[s], ksin[s]));
      if (row == t) {
        const int d4 = 8 * s + ds;
        *reinterpret_cast<float4 *>(p.k_new + (size_t)g * HD + 4 * d4) = kreg[s];
        *reinterpret_cast<float4 *>(const_cast<float *>(kbase) + (size_t)(t0 + t) * p.pos_stride + 4 * d4) = kreg[s];
      }
    }
  }
  if (has_q) // every block rotates its own copy; attn_merge writes q back rotated once all blocks have read it
    *reinterpret_cast<float4 *>(qs + qv * HD + 4 * qd4) = fresh ? rotate4(qreg, factors(qcos, qsin)) : qreg;
  __syncthreads();
  // every vector's dot with this lane's row: the lane's values in order, then the row's eight lanes by DPP
  for (int v = 0; v < nqv; v++) {
    float dot = 0.0f;
#pragma unroll
    for (int s = 0; s < KPER; s++) {
      const float4 a = kreg[s], b = *reinterpret_cast<const float4 *>(qs + v * HD + 4 * (8 * s + ds));
      dot = fmaf(a.x, b.x, dot);
      dot = fmaf(a.y, b.y, dot);
      dot = fmaf(a.z, b.z, dot);
      dot = fmaf(a.w, b.w, dot);
    }
    dot = group_reduce_add(dot, 8);
    if (ds == 0)
      dots[v * kChunk + row] = dot;
  }
  __syncthreads();
  if (wave < nqv) { // wave v scores vector v
    const int v = wave;
    const bool live = lane < n;
    float sc = -FLT_MAX;
    bool bad = false;
    if (live) {
      sc = dots[v * kChunk + lane] / p.divisor;
      bad = !isfinite(sc);
    }
    const float m = wave_max(sc);
    const float e = live ? expf(sc - m) : 0.0f;
    es[v * kChunk + lane] = e;
    const float l = wave_sum(e);
    if (lane == 0) {
      float *ph = p.partial + (((size_t)g * nqv + v) * p.chunks + c) * p.slot;
      ph[HD] = m;
      ph[HD + 1] = l;
    }
    if (bad)
      p.flags[1] = 1;
  }
  v_store(0, v0);
  v_store(1, v1);
  if constexpr (VPER == 4) {
    v_store(2, v2);
    v_store(3, v3);
  }
  __syncthreads();
  // value sums: item (vector, four dimensions) over position slice `slice` of the chunk, sixteen positions at a time
  const int items = nqv * HD4, slices = kTileThreads / items, span = (kChunk + slices - 1) / slices;
  const int slice = tid / items, item = tid % items, v = item / HD4, d4 = item % HD4;
  if (slice < slices) {
    const int ta = slice * span, tb = min(n, ta + span);
    const float *er = es + v * kChunk, *vr = vs + 4 * d4;
    float4 acc = zero4;
    for (int t1 = ta; t1 < tb; t1 += 16) {
      // branch-free (each position's reads in flight together): a position past the slice adds 0 times a staged row
#pragma unroll
      for (int k = 0; k < 16; k++) {
        const int tt = min(t1 + k, kChunk - 1);
        const float e = t1 + k < tb ? er[tt] : 0.0f;
        const float4 x = *reinterpret_cast<const float4 *>(vr + tt * HD);
        acc.x = fmaf(e, x.x, acc.x);
        acc.y = fmaf(e, x.y, acc.y);
        acc.z = fmaf(e, x.z, acc.z);
        acc.w = fmaf(e, x.w, acc.w);
      }
    }
    po[slice * items + item] = acc;
  }
  __syncthreads();
  if (tid < items) {
    float4 total = po[item];
    for (int sl = 1; sl < slices; sl++) {
      const float4 x = po[sl * items + item];
      total.x += x.x;
      total.y += x.y;
      total.z += x.z;
      total.w += x.w;
    }
    *reinterpret_cast<float4 *>(p.partial + (((size_t)g * nqv + v) * p.chunks + c) * p.slot + 4 * d4) = total;
  }
}

size_t attention_decode_lds(int kv_mul, int head_dim) {
  return ((size_t)kChunk * head_dim + (size_t)kv_mul * head_dim + 2 * (size_t)kv_mul * kChunk) * sizeof(float) +
         (size_t)kTileThreads * 16;
}

// Batched attention on the FP32 matrix cores (flash form): query rows in tiles of 128 / kv_mul, rounded down (the tile's
// query vectors: row j, query head h of the group as vector j * kv_mul + h, in 8 waves of 16; the 128 % kv_mul vectors
// past the last row idle). Block (p, KV head g) takes tile T - 1 - p and then tile p, so every block has about the
// same number of causal chunks (one block per CU). Per tile it walks the 64-position chunks the tile's rows reach,
// the K and V rows of a chunk staged in LDS by DMA (row stride HD + 4 floats, zero past the last position), two
// buffers each, with K one chunk ahead of V: step c scores chunk c + 1 while it takes chunk c's softmax and value
// sums, and the loads of chunk c + 2's K and chunk c + 1's V are in flight meanwhile, one barrier per step. Each wave
//   - scores its 16 vectors against the 64 positions on v_mfma_f32_16x16x4_f32, as S^T = K Q^T: four 16-position
//     tiles, HD / 4 MFMAs each; the dot's terms go in a permuted order (MFMA step kk, lane group q takes dimension
//     q * HD / 4 + kk), so a lane's share of its query vector is HD / 4 consecutive floats held in registers and its
//     K reads are 16-byte runs;
//   - masks the positions past each row's own (causal), takes the chunk maximum and the running maximum, rescales
//     its running sum and value sums by exp(m_old - m_new), and forms p = exp(s - m_new); the scores are kept in base
//     2 (s * log2(e) / divisor, one multiply where the split form divides), so each exponential is the native exp2;
//   - adds P V to its value sums as O^T = V^T P^T: the score accumulators are the B operand as they stand (MFMA step
//     (tile t, element e) takes positions 16 t + 4 q + e from lane group q), and V^T is read from LDS, value tile d
//     holding dimensions 4 m + d % 4 + 64 (d / 4) (m = 0..15): a lane's values of a position are runs of four, and
//     the 16 lanes of a read take one contiguous 64-float span of the row, free of LDS bank conflicts.
// At the end each vector's value sum is divided by its running sum and stored. Every product is FP32 on the matrix
// cores; the sums run in other orders than the split form's and the scores are rounded once more, within FP32
// rounding of the same softmax.

// Staging of a 64-position chunk of K (or V) rows into LDS by DMA (buffer_load_dwordx4 ... lds): a load takes
// 1 KB, lane l's 16 bytes landing at byte 16 l from the wave-uniform base. The rows lie HD + 4 floats apart, so a
// chunk is 64 (HD / 4 + 1) pieces of 16 bytes, a whole number of loads; a lane whose piece is a row's padding loads
// a copy of that row's first piece. The buffer resource ends after the tile's last position, so the rows past it
// read as zero.
template <int HD> struct FlashDma {
  static constexpr int kWaves = kTileThreads / kWave;
  static constexpr int kPieces = HD / 4 + 1;             // per staged row, the padding included
  static constexpr int kLoads = kChunk * kPieces / kWave; // 1 KB loads per chunk
  static_assert(kChunk * kPieces % kWave == 0, "a chunk is a whole number of loads");
  __device__ __forceinline__ static void load(__amdgpu_buffer_rsrc_t r, float *dst, int t0, unsigned stride_bytes,
                                              int wave, int lane) {
#pragma unroll
    for (int u = 0; u < (kLoads + kWaves - 1) / kWaves; u++) {
      const int n = u * kWaves + wave;
      if (n < kLoads) { // wave-uniform
        const int slot = n * kWave + lane, row = slot / kPieces, piece = slot % kPieces;
        const unsigned off = (unsigned)(t0 + row) * stride_bytes + 16u * (unsigned)(piece < HD / 4 ? piece : 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)(dst + n * 4 * kWave),
                                                 16, off, 0, 0, 0);
      }
    }
  }
};

// s_waitcnt vmcnt(0): this wave's loads, LDS DMA included, are complete
__device__ __forceinline__ void wait_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }

template <int HD> __global__ __launch_bounds__(kTileThreads) void attn_flash(AttnParams p) {
  constexpr int kQ = HD / 4;       // dimensions per lane group in the score MFMAs
  constexpr int kDt = HD / 16;     // 16-dimension tiles of the value sums
  constexpr int kQv = 128;         // query vectors per tile
  // two K and two V buffers as separate arrays: the compiler then sees that a DMA into one does not alias the reads
  // of another and lets them overlap
  constexpr int kSt = HD + 4;      // LDS row stride of a staged K or V row
  __shared__ __align__(16) float K0[kChunk * kSt], K1[kChunk * kSt], V0[kChunk * kSt], V1[kChunk * kSt];
  const int kv_mul = p.n_heads / p.n_kv_heads, tile_rows = kQv / kv_mul;
  const int ntiles = (p.rows + tile_rows - 1) / tile_rows;
  const int g = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int lq = lane >> 4, lc = lane & 15;
  const int qv = wave * 16 + lc, j = qv / kv_mul, h = qv % kv_mul;
  const float *kbase = p.key + (size_t)g * p.head_base, *vbase = p.value + (size_t)g * p.head_base;
  const unsigned stride_bytes = (unsigned)p.pos_stride * 4u;
  // scores in base 2: s * log2(e) / divisor, so that exp(s / divisor - m) is the native exp2 of (s2 - m2)
  const float scale2 = 1.4426950408889634f / p.divisor;
  bool bad = false;
  const bool split = p.splits > 0; // block (tile, g, s) takes share s of the tile's chunks and stores a partial
  for (int pass = 0; pass < 2; pass++) {
    const int tile = split ? (int)blockIdx.x : pass == 0 ? ntiles - 1 - (int)blockIdx.x : (int)blockIdx.x;
    if (pass == 1 && (split || tile >= ntiles - 1 - (int)blockIdx.x))
      break; // the middle tile of an odd count is taken once
    const int r0 = tile * tile_rows, row = r0 + j;
    // vectors past tile_rows * kv_mul (when kv_mul does not divide 128) would be the next tile's: idle, like rows past
    // the batch
    const bool active = j < tile_rows && row < p.rows;
    const int live_to = active ? p.pos0 + row : -1; // this lane's query row's position (none for an idle lane)
    const int wave_last = p.pos0 + min(r0 + min((wave * 16 + 15) / kv_mul, tile_rows - 1), p.rows - 1);
    const int last = p.pos0 + min(r0 + tile_rows, p.rows) - 1; // the tile's last position
    const int range = (int)(((unsigned)last * stride_bytes) + HD * 4); // bytes of K (V) rows up to `last`
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void *)kbase, (short)0, range, 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void *)vbase, (short)0, range, 0x00020000);
    // this lane's dimensions lq * HD / 4 .. + HD / 4 of its query vector
    float qr[kQ];
    {
      const float *src = p.q + ((size_t)(active ? row : 0) * p.n_heads + (size_t)g * kv_mul + h) * HD + lq * kQ;
#pragma unroll
      for (int i = 0; i < kQ; i += 4) {
        const float4 v = active ? *reinterpret_cast<const float4 *>(src + i) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        qr[i] = v.x, qr[i + 1] = v.y, qr[i + 2] = v.z, qr[i + 3] = v.w;
      }
    }
    v4f o[kDt];
#pragma unroll
    for (int d = 0; d < kDt; d++)
      o[d] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -FLT_MAX, l_run = 0.0f;
    // S^T of the chunk staged at ks: position 16 t + 4 lq + e (t = 0..3, e = 0..3) against this lane's query vector;
    // the four position tiles' accumulators take turns, so consecutive MFMAs never wait on each other. A slice is the
    // 16 MFMAs of dimensions i .. i + 3 of each lane group's share.
    auto score_slice = [&](const float *ks, v4f (&sc)[4], int i) {
      float4 a[4];
#pragma unroll
      for (int t = 0; t < 4; t++)
        a[t] = *reinterpret_cast<const float4 *>(ks + (16 * t + lc) * kSt + lq * kQ + i);
#pragma unroll
      for (int t = 0; t < 4; t++)
        sc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t].x, qr[i], sc[t], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 4; t++)
        sc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t].y, qr[i + 1], sc[t], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 4; t++)
        sc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t].z, qr[i + 2], sc[t], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 4; t++)
        sc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t].w, qr[i + 3], sc[t], 0, 0, 0);
    };
    auto score = [&](const float *ks, v4f (&sc)[4]) {
#pragma unroll
      for (int t = 0; t < 4; t++)
        sc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < kQ; i += 4)
        score_slice(ks, sc, i);
    };
    // the softmax of the chunk at t0 (scores in, weights out) in eight phases: phase t < 4 masks and scales position
    // tile t and takes its maximum (phase 3 also the chunk's maximum over the vector's 64 positions, 16 here and the
    // rest in lanes lc + 16, 32, 48, and the rescale of the sums); phase 4 + t takes tile t's exponentials and their
    // sum (phase 7 also the running sums)
    struct Soft {
      float cmax, alpha, m_new, psum;
    };
    auto weigh_phase = [&](int ph, int t0, v4f (&sc)[4], Soft &w) {
      if (ph < 4) {
        const int t = ph;
        if (t == 0)
          w.cmax = -FLT_MAX;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int at = t0 + 16 * t + 4 * lq + e;
          const bool live = at <= live_to;
          const float raw = sc[t][e] * scale2; // selected, not branched on: one block for the scheduler
          bad |= live & !isfinite(raw);
          const float s = live ? raw : -FLT_MAX;
          sc[t][e] = s;
          w.cmax = fmaxf(w.cmax, s);
        }
        if (t == 3) {
          w.cmax = fmaxf(w.cmax, __shfl_xor(w.cmax, 16));
          w.cmax = fmaxf(w.cmax, __shfl_xor(w.cmax, 32));
          w.m_new = fmaxf(m_run, w.cmax);
          w.alpha = exp2f(m_run - w.m_new); // 0 before the first live position, 1 when the maximum stays
          w.psum = 0.0f;
        }
      } else {
        const int t = ph - 4;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float pe = sc[t][e] > -FLT_MAX ? exp2f(sc[t][e] - w.m_new) : 0.0f;
          sc[t][e] = pe;
          w.psum += pe;
        }
        if (t == 3) {
          w.psum += __shfl_xor(w.psum, 16);
          w.psum += __shfl_xor(w.psum, 32);
          l_run = l_run * w.alpha + w.psum;
          m_run = w.m_new;
#pragma unroll
          for (int d = 0; d < kDt; d++)
            o[d] *= w.alpha;
        }
      }
    };
    auto weigh = [&](int t0, v4f (&sc)[4]) {
      Soft w;
#pragma unroll
      for (int ph = 0; ph < 8; ph++)
        weigh_phase(ph, t0, sc, w);
    };
    // the next chunk's scores into sn with this chunk's softmax between their slices, a scheduling barrier after
    // each slice so that the vector work stays spread over the MFMAs
    auto score_and_weigh = [&](const float *kn, v4f (&sn)[4], int t0, v4f (&sc)[4]) {
      constexpr int kSlices = kQ / 4, kPhases = 8 / kSlices;
      static_assert(8 % kSlices == 0, "the softmax phases spread evenly over the score slices");
#pragma unroll
      for (int t = 0; t < 4; t++)
        sn[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      Soft w;
#pragma unroll
      for (int k = 0; k < kSlices; k++) {
        score_slice(kn, sn, 4 * k);
#pragma unroll
        for (int q = 0; q < kPhases; q++)
          weigh_phase(k * kPhases + q, t0, sc, w);
        __builtin_amdgcn_sched_barrier(0x100); // only LDS reads may move across: the next slice's K rows, early
      }
    };
    // O^T += V^T P^T from the chunk staged at vs; the dimension tiles' accumulators take turns
    auto accumulate = [&](const float *vs, const v4f (&sc)[4]) {
#pragma unroll
      for (int t = 0; t < 4; t++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float *vr = vs + (16 * t + 4 * lq + e) * kSt + 4 * lc;
          float va[kDt];
#pragma unroll
          for (int d = 0; d < kDt; d += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(vr + 16 * d); // dimensions 64 (d / 4) + 4 lc ..
            va[d] = v.x, va[d + 1] = v.y, va[d + 2] = v.z, va[d + 3] = v.w;
          }
#pragma unroll
          for (int d = 0; d < kDt; d++)
            o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[d], sc[t][e], o[d], 0, 0, 0);
        }
    };
    // K of chunk c + 1 is staged one step ahead of V of chunk c, so step c scores chunk c + 1 on the matrix cores
    // while the vector ALUs take chunk c's softmax, in one stretch of code the compiler interleaves. Chunk c's K lies
    // in K(c % 2) and its V in V(c % 2). At the start of step c every wave has waited for its loads of the step
    // before and passed the barrier; then K(c % 2), last read for chunk c (in step c - 1), takes chunk c + 2, and
    // V((c + 1) % 2), last read for chunk c - 1, takes chunk c + 1.
    // this block's chunks: c0 .. c0 + chunks - 1 (all of the tile's unless split)
    const int all = last / kChunk + 1, share = split ? (all + p.splits - 1) / p.splits : all;
    const int c0 = split ? min(all, (int)blockIdx.z * share) : 0, chunks = min(all, c0 + share) - c0;
    v4f sc[4];
    auto step = [&](int c, const float *kn, float *kdma, const float *vs, float *vdma) {
      const int t0 = (c0 + c) * kChunk;
      wait_loads();
      __syncthreads();
      if (c + 2 < chunks)
        FlashDma<HD>::load(krs, kdma, t0 + 2 * kChunk, stride_bytes, wave, lane);
      if (c + 1 < chunks)
        FlashDma<HD>::load(vrs, vdma, t0 + kChunk, stride_bytes, wave, lane);
      // a wave skips the chunks past its last row (wave-uniform), and so scores the next chunk only if it reaches it
      if (c + 1 < chunks && t0 + kChunk <= wave_last) {
        v4f sn[4];
        score_and_weigh(kn, sn, t0, sc);
        accumulate(vs, sc);
#pragma unroll
        for (int t = 0; t < 4; t++)
          sc[t] = sn[t];
      } else if (t0 <= wave_last) {
        weigh(t0, sc);
        accumulate(vs, sc);
      }
    };
    if (chunks > 0) {
      FlashDma<HD>::load(krs, K0, c0 * kChunk, stride_bytes, wave, lane);
      if (chunks > 1)
        FlashDma<HD>::load(krs, K1, (c0 + 1) * kChunk, stride_bytes, wave, lane);
      FlashDma<HD>::load(vrs, V0, c0 * kChunk, stride_bytes, wave, lane);
      wait_loads();
      __syncthreads();
      score(K0, sc); // unused by a wave that does not reach the chunk (the steps check)
      for (int c = 0; c < chunks; c += 2) {
        step(c, K1, K0, V0, V1);
        if (c + 1 < chunks)
          step(c + 1, K0, K1, V1, V0);
      }
    }
    __syncthreads(); // the next tile's first loads reuse K0, K1 and V0
    if (!active)
      continue;
    if (split) { // the share's value sums, maximum (in natural units, as the merge takes it) and sum, unnormalized;
      // slots [row][head][share]: rows x n_heads x splits x slot floats in all, the room flash_splits checked
      float *slot = p.partial + (((size_t)row * p.n_heads + (size_t)g * kv_mul + h) * p.splits + blockIdx.z) * p.slot;
#pragma unroll
      for (int e = 0; e < 4; e++)
#pragma unroll
        for (int d = 0; d < kDt; d += 4)
          *reinterpret_cast<float4 *>(slot + 16 * d + 4 * (4 * lq + e)) =
              float4{o[d][e], o[d + 1][e], o[d + 2][e], o[d + 3][e]};
      if (lq == 0) {
        slot[HD] = m_run > -FLT_MAX ? m_run * 0.6931471805599453f : -FLT_MAX;
        slot[HD + 1] = l_run;
      }
      continue;
    }
    // lane (lq, lc) holds dimensions 4 (4 lq + e) + d % 4 + 64 (d / 4) of vector lc: for each e, runs of four floats
    const float inv = 1.0f / l_run;
    float *dst = p.out + ((size_t)row * p.n_heads + (size_t)g * kv_mul + h) * HD;
#pragma unroll
    for (int e = 0; e < 4; e++)
#pragma unroll
      for (int d = 0; d < kDt; d += 4)
        *reinterpret_cast<float4 *>(dst + 16 * d + 4 * (4 * lq + e)) =
            float4{o[d][e] * inv, o[d + 1][e] * inv, o[d + 2][e] * inv, o[d + 3][e] * inv};
  }
  if (bad)
    p.flags[1] = 1;
}

// The flash form on the BF16 matrix cores (attn_flash3): the same tiles, pairs of tiles, position split and online
// softmax as attn_flash, with every product of the scores and the value sums formed from exact three-part BF16 splits
// of its FP32 operands. A value x is h + m + l exactly (h the top 8 significant bits of x, m the next 8 of x - h, l the
// rest, at most 8 bits), and x y is taken as hh + hm + mh + mm + hl + lh: the three dropped products are below 2^-23 of
// |x y| and every BF16 product is exact in FP32, so each score and value sum is FP32-accurate, as on the FP32 matrix
// cores, at six v_mfma_f32_16x16x32_bf16 (16 cycles) per 16 x 16 x 32 block against eight v_mfma_f32_16x16x4_f32
// (32 cycles each). Chunks are 32 positions. A chunk's K and V rows are loaded into registers one chunk ahead (buffer
// loads, zero past the tile's last position), split once per block (each thread 8 values of K and 8 of V) and
// written to LDS as parts, two buffers, one barrier per chunk:
//   - K parts [part][position][dimension], rows padded to HD + 8 values, so the score MFMA's A operand (16 positions x
//     32 dimensions: lane l reads dimensions 8 (l / 16) .. + 7 of position l % 16) is one 16-byte read per part, free
//     of bank conflicts; the query vector's parts stay in registers as the B operand;
//   - V parts transposed, [part][dimension][slot], a dimension's 32 slots padded to 40: the value sums' B operand is
//     the scores' accumulator as it stands (lane (q, c) holds positions 16 t + 4 q + e of vector c), so slot
//     8 q + 4 t + e holds position 16 t + 4 q + e, and the A operand (16 dimensions x 32 slots) is again one 16-byte
//     read per part.
// Lane (q, c) ends with dimensions 16 d + 4 q + e of its vector c; unsplit with qout set, the epilogue quantizes them
// in groups of qgs dimensions instead of storing FP32.
template <int HD> __global__ __launch_bounds__(kTileThreads) void attn_flash3(AttnParams p) {
  typedef int v4i_t __attribute__((ext_vector_type(4)));
  typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
  constexpr int kC = 32;                   // positions per chunk
  constexpr int kSs = HD / 32;             // 32-dimension steps of the scores
  constexpr int kDt = HD / 16;             // 16-dimension tiles of the value sums
  constexpr int kQv = 128;                 // query vectors per tile
  constexpr int kKRow = HD + 8, kVRow = kC + 8;
  constexpr int kKPart = kC * kKRow, kVPart = HD * kVRow;
  constexpr int kKThreads = kC * HD / 8, kVThreads = HD * 4; // threads that stage 8 values of K, of V
  static_assert(kKThreads <= kTileThreads && kVThreads <= kTileThreads, "one staging item per thread");
  __shared__ __align__(16) uint16_t Kp[2][3 * kKPart];
  __shared__ __align__(16) uint16_t Vp[2][3 * kVPart];
  const int kv_mul = p.n_heads / p.n_kv_heads, tile_rows = kQv / kv_mul;
  const int ntiles = (p.rows + tile_rows - 1) / tile_rows;
  const int g = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int lq = lane >> 4, lc = lane & 15;
  const int qv = wave * 16 + lc, j = qv / kv_mul, h = qv % kv_mul;
  const float *kbase = p.key + (size_t)g * p.head_base, *vbase = p.value + (size_t)g * p.head_base;
  const unsigned stride_bytes = (unsigned)p.pos_stride * 4u;
  const float scale2 = 1.4426950408889634f / p.divisor;
  // staging roles: K position kpos, dimensions 8 kdg ..; V dimension vdim, slots 8 va .. (positions 4 va + e and
  // 16 + 4 va + e)
  const int kpos = tid / (HD / 8), kdg = tid % (HD / 8), vdim = tid % HD, va = tid / HD;
  const bool kstage = tid < kKThreads, vstage = tid < kVThreads;
  // the high halves of x's three parts: h in the word of x, m in the word of x - h, l in the word of the rest
  auto split3 = [](float x, unsigned &uh, unsigned &um, unsigned &ul) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const float r1 = x - __builtin_bit_cast(float, u & 0xFFFF0000u);
    const unsigned u1 = __builtin_bit_cast(unsigned, r1);
    const float r2 = r1 - __builtin_bit_cast(float, u1 & 0xFFFF0000u);
    uh = u, um = u1, ul = __builtin_bit_cast(unsigned, r2);
  };
  // eight values in slot order -> three parts of eight BF16 values (value 2 w in the low half of dword w)
  auto parts8 = [&](const float (&v)[8], v4i_t &ph, v4i_t &pm, v4i_t &pl) {
#pragma unroll
    for (int w = 0; w < 4; w++) {
      unsigned ah, am, al, bh, bm, bl;
      split3(v[2 * w], ah, am, al);
      split3(v[2 * w + 1], bh, bm, bl);
      ph[w] = (int)__builtin_amdgcn_perm(bh, ah, 0x07060302u);
      pm[w] = (int)__builtin_amdgcn_perm(bm, am, 0x07060302u);
      pl[w] = (int)__builtin_amdgcn_perm(bl, al, 0x07060302u);
    }
  };
  auto mfma = [](const v4i_t &a, const v4i_t &b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0, 0,
                                                    0);
  };
  bool bad = false, qbad = false;
  const bool split = p.splits > 0;
  for (int pass = 0; pass < 2; pass++) {
    const int tile = split ? (int)blockIdx.x : pass == 0 ? ntiles - 1 - (int)blockIdx.x : (int)blockIdx.x;
    if (pass == 1 && (split || tile >= ntiles - 1 - (int)blockIdx.x))
      break;
    const int r0 = tile * tile_rows, row = r0 + j;
    const bool active = j < tile_rows && row < p.rows;
    const int live_to = active ? p.pos0 + row : -1;
    const int wave_last = p.pos0 + min(r0 + min((wave * 16 + 15) / kv_mul, tile_rows - 1), p.rows - 1);
    const int last = p.pos0 + min(r0 + tile_rows, p.rows) - 1;
    const int range = (int)(((unsigned)last * stride_bytes) + HD * 4);
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void *)kbase, (short)0, range, 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void *)vbase, (short)0, range, 0x00020000);
    // the query vector's parts: step s holds dimensions 32 s + 8 lq .. + 7
    v4i_t qh[kSs], qm[kSs], ql[kSs];
    {
      const float *src = p.q + ((size_t)(active ? row : 0) * p.n_heads + (size_t)g * kv_mul + h) * HD + 8 * lq;
#pragma unroll
      for (int st = 0; st < kSs; st++) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i += 4) {
          const float4 x = active ? *reinterpret_cast<const float4 *>(src + 32 * st + i) : float4{0.f, 0.f, 0.f, 0.f};
          v[i] = x.x, v[i + 1] = x.y, v[i + 2] = x.z, v[i + 3] = x.w;
        }
        parts8(v, qh[st], qm[st], ql[st]);
      }
    }
    v4f o[kDt];
#pragma unroll
    for (int d = 0; d < kDt; d++)
      o[d] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -FLT_MAX, l_run = 0.0f;
    const int all = last / kC + 1, share = split ? (all + p.splits - 1) / p.splits : all;
    const int c0 = split ? min(all, (int)blockIdx.z * share) : 0, chunks = min(all, c0 + share) - c0;
    float kr[8], vr[8]; // the next chunk's K and V values of this thread's staging items
    auto load = [&](int c) {
      const int t0 = (c0 + c) * kC;
      if (kstage) {
        const unsigned off = (unsigned)(t0 + kpos) * stride_bytes + 32u * (unsigned)kdg;
        const float4 a = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, 0));
        const float4 b = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(krs, off + 16u, 0, 0));
        kr[0] = a.x, kr[1] = a.y, kr[2] = a.z, kr[3] = a.w, kr[4] = b.x, kr[5] = b.y, kr[6] = b.z, kr[7] = b.w;
      }
      if (vstage) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const int at = t0 + (e < 4 ? 4 * va + e : 16 + 4 * va + e - 4);
          vr[e] = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(vrs, (unsigned)at * stride_bytes + 4u * (unsigned)vdim, 0, 0));
        }
      }
    };
    auto stage = [&](int b) {
      if (kstage) {
        v4i_t ph, pm, pl;
        parts8(kr, ph, pm, pl);
        uint16_t *dst = &Kp[b][kpos * kKRow + 8 * kdg];
        *reinterpret_cast<v4i_t *>(dst) = ph;
        *reinterpret_cast<v4i_t *>(dst + kKPart) = pm;
        *reinterpret_cast<v4i_t *>(dst + 2 * kKPart) = pl;
      }
      if (vstage) {
        v4i_t ph, pm, pl;
        parts8(vr, ph, pm, pl);
        uint16_t *dst = &Vp[b][vdim * kVRow + 8 * va];
        *reinterpret_cast<v4i_t *>(dst) = ph;
        *reinterpret_cast<v4i_t *>(dst + kVPart) = pm;
        *reinterpret_cast<v4i_t *>(dst + 2 * kVPart) = pl;
      }
    };
    // chunk at t0 from buffer b: S^T = K Q^T (leading and correction products in separate accumulators), the online
    // softmax, O^T += V^T P^T
    auto compute = [&](int b, int t0) {
      v4f sc[2], sx[2];
#pragma unroll
      for (int t = 0; t < 2; t++)
        sc[t] = sx[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int st = 0; st < kSs; st++)
#pragma unroll
        for (int t = 0; t < 2; t++) {
          const uint16_t *kb = &Kp[b][(16 * t + lc) * kKRow + 32 * st + 8 * lq];
          const v4i_t kh = *reinterpret_cast<const v4i_t *>(kb), km = *reinterpret_cast<const v4i_t *>(kb + kKPart),
                      kl = *reinterpret_cast<const v4i_t *>(kb + 2 * kKPart);
          sc[t] = mfma(kh, qh[st], sc[t]);
          sx[t] = mfma(kh, qm[st], sx[t]);
          sx[t] = mfma(km, qh[st], sx[t]);
          sx[t] = mfma(km, qm[st], sx[t]);
          sx[t] = mfma(kh, ql[st], sx[t]);
          sx[t] = mfma(kl, qh[st], sx[t]);
        }
      float cmax = -FLT_MAX;
      float pv[8]; // slot 4 t + e: position 16 t + 4 lq + e
#pragma unroll
      for (int t = 0; t < 2; t++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int at = t0 + 16 * t + 4 * lq + e;
          const bool live = at <= live_to;
          const float raw = (sc[t][e] + sx[t][e]) * scale2;
          bad |= live & !isfinite(raw);
          pv[4 * t + e] = live ? raw : -FLT_MAX;
          cmax = fmaxf(cmax, pv[4 * t + e]);
        }
      cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
      cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
      const float m_new = fmaxf(m_run, cmax);
      const float alpha = exp2f(m_run - m_new);
      float psum = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float pe = pv[i] > -FLT_MAX ? exp2f(pv[i] - m_new) : 0.0f;
        pv[i] = pe;
        psum += pe;
      }
      psum += __shfl_xor(psum, 16);
      psum += __shfl_xor(psum, 32);
      l_run = l_run * alpha + psum;
      m_run = m_new;
      v4i_t ph, pm, pl;
      parts8(pv, ph, pm, pl);
      v4f ox[kDt];
#pragma unroll
      for (int d = 0; d < kDt; d++) {
        o[d] *= alpha;
        ox[d] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int d = 0; d < kDt; d++) {
        const uint16_t *vb = &Vp[b][(16 * d + lc) * kVRow + 8 * lq];
        const v4i_t vh = *reinterpret_cast<const v4i_t *>(vb), vm = *reinterpret_cast<const v4i_t *>(vb + kVPart),
                    vl = *reinterpret_cast<const v4i_t *>(vb + 2 * kVPart);
        o[d] = mfma(vh, ph, o[d]);
        ox[d] = mfma(vh, pm, ox[d]);
        ox[d] = mfma(vm, ph, ox[d]);
        ox[d] = mfma(vm, pm, ox[d]);
        ox[d] = mfma(vh, pl, ox[d]);
        ox[d] = mfma(vl, ph, ox[d]);
      }
#pragma unroll
      for (int d = 0; d < kDt; d++)
        o[d] += ox[d];
    };
    if (chunks > 0) {
      load(0);
      wait_loads();
      stage(0);
      if (chunks > 1)
        load(1);
      __syncthreads();
      for (int c = 0; c < chunks; c++) {
        const int b = c & 1, t0 = (c0 + c) * kC;
        if (c + 1 < chunks) { // chunk c + 1 into the other buffer, last read in step c - 1
          wait_loads();
          stage(b ^ 1);
          if (c + 2 < chunks)
            load(c + 2);
        }
        if (t0 <= wave_last) // wave-uniform: a wave whose rows end before the chunk has nothing to add
          compute(b, t0);
        __syncthreads();
      }
    }
    if (!active)
      continue;
    if (split) { // the share's value sums, maximum (natural units) and sum, unnormalized, in slot [row][head][share]
      float *slot = p.partial + (((size_t)row * p.n_heads + (size_t)g * kv_mul + h) * p.splits + blockIdx.z) * p.slot;
#pragma unroll
      for (int d = 0; d < kDt; d++)
        *reinterpret_cast<float4 *>(slot + 16 * d + 4 * lq) = float4{o[d][0], o[d][1], o[d][2], o[d][3]};
      if (lq == 0) {
        slot[HD] = m_run > -FLT_MAX ? m_run * 0.6931471805599453f : -FLT_MAX;
        slot[HD + 1] = l_run;
      }
      continue;
    }
    const float inv = 1.0f / l_run;
    const size_t vec = (size_t)row * p.n_heads + (size_t)g * kv_mul + h; // this lane's query vector
    if (p.qout) { // k_quantize of the rows the FP32 store below would write: a group of qgs dimensions is qgs / 16 of
      // the lane's dimension tiles and the same tiles of the vector's other three lanes (lq), so its maximum is the
      // lanes' maximum over those tiles; each value is quantized as quantize_lanes does, the group's scale from lq 0
      const int tiles = p.qgs / 16;
      int8_t *qrow = p.qout + vec * HD;
      for (int d0 = 0; d0 < kDt; d0 += tiles) {
        float peak = 0.0f;
#pragma unroll
        for (int d = 0; d < kDt; d++)
          if (d >= d0 && d < d0 + tiles)
#pragma unroll
            for (int e = 0; e < 4; e++)
              peak = fmaxf(peak, fabsf(o[d][e] * inv)); // a NaN is skipped here and caught by quantize_fast
        peak = fmaxf(peak, __shfl_xor(peak, 16));
        peak = fmaxf(peak, __shfl_xor(peak, 32));
        const float scale = peak / 127.0f;
        bool ok;
        const float rinv = group_reciprocal(scale, ok);
#pragma unroll
        for (int d = 0; d < kDt; d++)
          if (d >= d0 && d < d0 + tiles) {
            const float x[4] = {o[d][0] * inv, o[d][1] * inv, o[d][2] * inv, o[d][3] * inv};
            int qv[4];
            quantize_fast(x, scale, rinv, ok, qv, qbad);
            *reinterpret_cast<int *>(qrow + 16 * d + 4 * lq) = pack_bytes(qv[0], qv[1], qv[2], qv[3]);
          }
        if (lq == 0)
          p.qscale[(vec * HD + 16 * d0) / p.qgs] = scale;
      }
      continue;
    }
    float *dst = p.out + vec * HD;
#pragma unroll
    for (int d = 0; d < kDt; d++)
      *reinterpret_cast<float4 *>(dst + 16 * d + 4 * lq) =
          float4{o[d][0] * inv, o[d][1] * inv, o[d][2] * inv, o[d][3] * inv};
  }
  if (bad)
    p.flags[1] = 1;
  if (qbad)
    p.flags[0] = 1;
}

// Block (chunk c, KV head g, query row r). Waves take positions t0 + w, t0 + w + 4, ...: lane l holds dimensions
// l, l + 64, ... of the K row, dots it with each query head of the group held the same way, and the wave sum over the
// lanes gives the score, (dot) / sqrtf(head_dim) like the reference. Then per head the chunk maximum, the
// exponentials and their sum; then thread i accumulates dimension i % head_dim of the value sum for every head over a
// share of the positions, the shares meeting in LDS.
__global__ __launch_bounds__(kThreads) void attn_chunks(AttnParams p) {
  static_assert(kChunk == kWave, "a chunk's scores are one per lane");
  __shared__ float score[kMaxGroup][kChunk];
  __shared__ float acc[kThreads * kMaxGroup]; // the value-sum shares: [share][head][head_dim], shares * head_dim <= 256
  const int c = blockIdx.x, g = blockIdx.y, r = blockIdx.z;
  const int position = p.pos0 + r, positions = position + 1;
  const int t0 = c * kChunk;
  if (t0 >= positions)
    return; // beyond this row's causal range: the merge reads only the row's own chunks
  const int t1 = min(positions, t0 + kChunk);
  const int kv_mul = p.n_heads / p.n_kv_heads, hd = p.head_dim;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const float *qrow = p.q + (size_t)r * p.n_heads * hd + (size_t)g * kv_mul * hd;
  const float *kbase = p.key + (size_t)g * p.head_base, *vbase = p.value + (size_t)g * p.head_base;
  constexpr int kDims = kMaxHeadDim / kWave;
  float qv[kMaxGroup][kDims];
#pragma unroll
  for (int h = 0; h < kMaxGroup; h++)
#pragma unroll
    for (int e = 0; e < kDims; e++) {
      const int d = lane + e * kWave;
      qv[h][e] = h < kv_mul && d < hd ? qrow[(size_t)h * hd + d] : 0.0f;
    }
  bool bad = false;
  for (int t = t0 + wave; t < t1; t += kThreads / kWave) {
    const float *krow = kbase + (size_t)t * p.pos_stride;
    float kd[kDims];
#pragma unroll
    for (int e = 0; e < kDims; e++) {
      const int d = lane + e * kWave;
      kd[e] = d < hd ? krow[d] : 0.0f;
    }
#pragma unroll
    for (int h = 0; h < kMaxGroup; h++) {
      if (h < kv_mul) {
        float dot = 0.0f;
#pragma unroll
        for (int e = 0; e < kDims; e++)
          dot = fmaf(qv[h][e], kd[e], dot);
        const float s = wave_sum(dot) / p.divisor;
        bad |= !isfinite(s);
        if (lane == 0)
          score[h][t - t0] = s;
      }
    }
  }
  if (bad && lane == 0)
    p.flags[1] = 1;
  __syncthreads();
  // per head (wave w takes heads w, w + 4, ...): the chunk maximum, the exponentials in place and their sum
  const int n = t1 - t0;
  float *part = p.partial + ((size_t)(r * p.n_heads + g * kv_mul) * p.chunks + c) * p.slot;
  for (int h = wave; h < kv_mul; h += kThreads / kWave) {
    const float s = lane < n ? score[h][lane] : -FLT_MAX;
    const float m = wave_max(s);
    const float e = lane < n ? expf(s - m) : 0.0f;
    score[h][lane] = e;
    const float l = wave_sum(e);
    if (lane == 0) {
      float *ph = part + (size_t)h * p.chunks * p.slot;
      ph[hd] = m;
      ph[hd + 1] = l;
    }
  }
  __syncthreads();
  // value sums: thread i owns dimension d = i % hd (hd <= 256) for every head, over positions t0 + share, + shares ...
  const int shares = kThreads / hd > 0 ? kThreads / hd : 1;
  const int d = threadIdx.x % hd, share = threadIdx.x / hd;
  float o[kMaxGroup];
#pragma unroll
  for (int h = 0; h < kMaxGroup; h++)
    o[h] = 0.0f;
  if (share < shares) {
    for (int t = t0 + share; t < t1; t += shares) {
      const float v = vbase[(size_t)t * p.pos_stride + d];
#pragma unroll
      for (int h = 0; h < kMaxGroup; h++)
        if (h < kv_mul)
          o[h] = fmaf(score[h][t - t0], v, o[h]);
    }
  }
  if (shares == 1) { // hd > 128: threads past hd own nothing
    if (share == 0) {
#pragma unroll
      for (int h = 0; h < kMaxGroup; h++)
        if (h < kv_mul)
          part[(size_t)h * p.chunks * p.slot + d] = o[h];
    }
    return;
  }
  // shares > 1 (hd <= 128): the shares' sums meet in LDS, share order
  float *sh = acc; // [share][head][hd]
  if (share < shares) {
#pragma unroll
    for (int h = 0; h < kMaxGroup; h++)
      if (h < kv_mul)
        sh[((size_t)share * kv_mul + h) * hd + d] = o[h];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kv_mul * hd; i += kThreads) {
    const int h = i / hd, dd = i % hd;
    float total = 0.0f;
    for (int s2 = 0; s2 < shares; s2++)
      total += sh[((size_t)s2 * kv_mul + h) * hd + dd];
    part[(size_t)h * p.chunks * p.slot + dd] = total;
  }
}

// Block (head h, query row r): M = max over the row's chunks of m_c, weight_c = expf(m_c - M), L = sum of
// weight_c * l_c, out = (sum of weight_c * o_c) / L. The chunks are spread over the threads: the maxima and weights
// by chunk, the value sums by (dimension, chunk group), the groups meeting in LDS. Thread c holds chunk c's m_c and
// l_c, and each (dimension, group) thread its first kMergeHeld values o_c, all loaded together before the first
// reduction, so the block waits for the partials once (twice past 256 chunks or kMergeHeld chunks per group).
constexpr int kMaxMergeChunks = 4096; // 262144 positions
constexpr int kMergeHeld = 32;

__device__ __forceinline__ float block_reduce(float v, float *scratch, bool is_max) {
  v = is_max ? wave_max(v) : wave_sum(v);
  if ((threadIdx.x & (kWave - 1)) == 0)
    scratch[threadIdx.x / kWave] = v;
  __syncthreads();
  float r = scratch[0];
  for (int w = 1; w < kThreads / kWave; w++)
    r = is_max ? fmaxf(r, scratch[w]) : r + scratch[w];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kThreads) void attn_merge(AttnParams p) {
  __shared__ float weight[kMaxMergeChunks];
  __shared__ float red[kThreads];
  const int h = blockIdx.x, r = blockIdx.y;
  const int hd = p.head_dim, chunks = (p.pos0 + r) / kChunk + 1;
  const float *part = p.partial + ((size_t)(r * p.n_heads + h) * p.chunks) * p.slot;
  const int groups = kThreads / hd > 0 ? kThreads / hd : 1;
  const int d = threadIdx.x % hd, grp = threadIdx.x / hd;
  const bool summer = grp < groups;
  float held[kMergeHeld];
#pragma unroll
  for (int k = 0; k < kMergeHeld; k++) {
    const int c = grp + k * groups;
    held[k] = summer && c < chunks ? part[(size_t)c * p.slot + d] : 0.0f;
  }
  const bool mine = (int)threadIdx.x < chunks;
  const float m0 = mine ? part[(size_t)threadIdx.x * p.slot + hd] : -FLT_MAX;
  const float l0 = mine ? part[(size_t)threadIdx.x * p.slot + hd + 1] : 0.0f;
  float m = m0;
  for (int c = threadIdx.x + kThreads; c < chunks; c += kThreads)
    m = fmaxf(m, part[(size_t)c * p.slot + hd]);
  m = block_reduce(m, red, true);
  float l = 0.0f;
  if (mine) {
    const float w = expf(m0 - m);
    weight[threadIdx.x] = w;
    l = w * l0;
  }
  for (int c = threadIdx.x + kThreads; c < chunks; c += kThreads) {
    const float w = expf(part[(size_t)c * p.slot + hd] - m);
    weight[c] = w;
    l += w * part[(size_t)c * p.slot + hd + 1];
  }
  l = block_reduce(l, red, false); // its barriers also publish `weight`
  if (p.table) { // fused RoPE (decode): q of this head back in place, rotated (every attn_tile block has read it)
    float *qh = p.rope_q + (size_t)h * hd;
    for (int d4 = threadIdx.x; d4 < hd / 4; d4 += kThreads)
      *reinterpret_cast<float4 *>(qh + 4 * d4) =
          rotate4(*reinterpret_cast<const float4 *>(qh + 4 * d4), p.table, hd, 4 * d4);
  }
  float o = 0.0f;
  if (summer) {
    // branch-free, so every weight read is in flight at once: past the last chunk the held value is zero and the
    // weight read is clamped to the last chunk's (the product adds an exact zero)
#pragma unroll
    for (int k = 0; k < kMergeHeld; k++)
      o = fmaf(weight[min(grp + k * groups, chunks - 1)], held[k], o);
#pragma unroll 8
    for (int c = grp + kMergeHeld * groups; c < chunks; c += groups)
      o = fmaf(weight[c], part[(size_t)c * p.slot + d], o);
  }
  red[threadIdx.x] = o;
  __syncthreads();
  if (grp == 0) {
    for (int g2 = 1; g2 < groups; g2++)
      o += red[g2 * hd + d];
    p.out[((size_t)r * p.n_heads + h) * hd + d] = o / l;
  }
}

// The flash form's split partials combined, a thread per (row, head, four dimensions): M the maximum of the shares'
// maxima (a share that held no chunk stores -FLT_MAX and zero sums), weights exp(m_s - M) in share order, and the
// output sum_s w_s o_s / sum_s w_s l_s. The same combination as attn_merge with the sums in share order; with at most
// 16 shares a thread needs no reduction across the block, so the grid is as small as the output.
__global__ __launch_bounds__(kThreads) void attn_merge_shares(AttnParams p) {
  const int q4 = p.head_dim / 4;
  const long long idx = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= (long long)p.rows * p.n_heads * q4)
    return;
  const int d4 = (int)(idx % q4);
  const long long rh = idx / q4; // row * n_heads + head
  const float *part = p.partial + (size_t)rh * p.splits * p.slot; // the slots of row * n_heads + head
  const int hd = p.head_dim;
  float m = -FLT_MAX;
  for (int s = 0; s < p.splits; s++)
    m = fmaxf(m, part[(size_t)s * p.slot + hd]);
  float4 o = float4{0.0f, 0.0f, 0.0f, 0.0f};
  float l = 0.0f;
  for (int s = 0; s < p.splits; s++) {
    const float *share = part + (size_t)s * p.slot;
    const float w = expf(share[hd] - m);
    l = fmaf(w, share[hd + 1], l);
    const float4 v = *reinterpret_cast<const float4 *>(share + 4 * d4);
    o = float4{fmaf(w, v.x, o.x), fmaf(w, v.y, o.y), fmaf(w, v.z, o.z), fmaf(w, v.w, o.w)};
  }
  *reinterpret_cast<float4 *>(p.out + rh * hd + 4 * d4) = float4{o.x / l, o.y / l, o.z / l, o.w / l};
}

} // namespace

bool launch_rmsnorm(float *out, const float *x, const float *weight, int rows, int size, float epsilon,
                    hipStream_t stream) {
  const bool vec4 = size % 4 == 0 && (((uintptr_t)out | (uintptr_t)x | (uintptr_t)weight) & 15) == 0;
  hipLaunchKernelGGL(rmsnorm_rows, dim3((unsigned)rows), dim3(kNormThreads), 0, stream, out, x, weight, size, epsilon,
                     vec4);
  return launch_ok("rmsnorm_rows");
}

bool launch_rope(float *q, size_t q_stride, float *k, size_t k_stride, const float *table, size_t table_stride,
                 int rows, int n_heads, int n_kv_heads, int head_dim, hipStream_t stream) {
  const long long threads = (long long)rows * n_heads * (head_dim / 2);
  hipLaunchKernelGGL(rope_rows, dim3((unsigned)((threads + kThreads - 1) / kThreads)), dim3(kThreads), 0, stream, q,
                     q_stride, k, k_stride, table, table_stride, rows, n_heads, n_kv_heads, head_dim);
  return launch_ok("rope_rows");
}

bool launch_rope_kv_rows(float *q, size_t q_stride, float *k, const float *v, size_t kv_stride, const float *table,
                         size_t table_stride, int rows, int n_heads, int n_kv_heads, int head_dim, float *key_cache,
                         float *value_cache, int pos0, size_t pos_stride, size_t head_base, hipStream_t stream) {
  const int per_row = (n_heads + 2 * n_kv_heads) * (head_dim / 4);
  if (head_dim == 128 || head_dim == 64) {
    const int rows_per_block = kThreads / (head_dim / 4);
    const dim3 grid((unsigned)((rows + rows_per_block - 1) / rows_per_block));
    if (head_dim == 128)
      hipLaunchKernelGGL(rope_kv_rows_hd<128>, grid, dim3(kThreads), 0, stream, q, q_stride, k, v, kv_stride, table,
                         table_stride, rows, n_heads, n_kv_heads, key_cache, value_cache, pos0, pos_stride, head_base);
    else
      hipLaunchKernelGGL(rope_kv_rows_hd<64>, grid, dim3(kThreads), 0, stream, q, q_stride, k, v, kv_stride, table,
                         table_stride, rows, n_heads, n_kv_heads, key_cache, value_cache, pos0, pos_stride, head_base);
    return launch_ok("rope_kv_rows_hd");
  }
  const long long threads = (long long)rows * per_row;
  hipLaunchKernelGGL(rope_kv_rows, dim3((unsigned)((threads + kThreads - 1) / kThreads)), dim3(kThreads), 0, stream, q,
                     q_stride, k, v, kv_stride, table, table_stride, rows, n_heads, n_kv_heads, head_dim, key_cache,
                     value_cache, pos0, pos_stride, head_base);
  return launch_ok("rope_kv_rows");
}

bool launch_kv_store(float *cache, const float *src, size_t src_ld, int pos0, int count, int n_kv_heads, int head_dim,
                     size_t pos_stride, size_t head_base, hipStream_t stream) {
  const long long threads = (long long)count * n_kv_heads * head_dim;
  hipLaunchKernelGGL(kv_store, dim3((unsigned)((threads + kThreads - 1) / kThreads)), dim3(kThreads), 0, stream, cache,
                     src, src_ld, pos0, count, n_kv_heads, head_dim, pos_stride, head_base);
  return launch_ok("kv_store");
}

bool launch_embed_rows(float *out, const int8_t *table, const float *scales, const int *ids, int count, int dim,
                       int gs, int vocab, hipStream_t stream) {
  const long long threads = (long long)count * dim;
  hipLaunchKernelGGL(embed_rows, dim3((unsigned)((threads + kThreads - 1) / kThreads)), dim3(kThreads), 0, stream, out,
                     table, scales, ids, count, dim, gs, vocab, device().error_flags);
  return launch_ok("embed_rows");
}

bool launch_embed_rows_f32(float *out, const float *table, const int *ids, int count, int dim, int vocab,
                           hipStream_t stream) {
  const bool vec = dim % 4 == 0 && ((uintptr_t)out | (uintptr_t)table) % 16 == 0;
  const long long threads = (long long)count * (vec ? dim / 4 : dim);
  const dim3 grid((unsigned)((threads + kThreads - 1) / kThreads));
  if (vec)
    hipLaunchKernelGGL(embed_rows_f32<4>, grid, dim3(kThreads), 0, stream, out, table, ids, count, dim, vocab,
                       device().error_flags);
  else
    hipLaunchKernelGGL(embed_rows_f32<1>, grid, dim3(kThreads), 0, stream, out, table, ids, count, dim, vocab,
                       device().error_flags);
  return launch_ok("embed_rows_f32");
}

// ---- the allocation-free attention's scratch --------------------------------------------------------------------
//
// k_attention_batch_layout_noalloc keeps its split-K partials here instead of in the grown workspace: 4 Mi floats
// (16 MiB), one copy per device, held until the process ends. In host code `scratch` names a host-side stand-in, not
// the device memory: the device address comes from hipGetSymbolAddress, once per device with that device current
// (attention_scratch_setup, called when the library opens the device), and only that address reaches kernels.
static __device__ __align__(256) float scratch[kAttentionScratchFloats];
namespace {
constexpr int kMaxOrdinals = 64;
float *scratch_address[kMaxOrdinals] = {};
} // namespace

bool attention_scratch_setup(int ordinal) {
  if (ordinal < 0 || ordinal >= kMaxOrdinals)
    return raise("device ordinal %d: the attention scratch table holds %d devices", ordinal, kMaxOrdinals);
  if (scratch_address[ordinal])
    return true;
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    (void)hipGetLastError();
    return raise("locating the attention scratch on device %d failed: %s", ordinal, hipGetErrorString(e));
  }
  scratch_address[ordinal] = (float *)p;
  return true;
}

float *attention_scratch(int ordinal) {
  return ordinal >= 0 && ordinal < kMaxOrdinals ? scratch_address[ordinal] : nullptr;
}

int slot_floats(int head_dim) { return (head_dim + 2 + 3) & ~3; }

size_t attention_partial_floats(int rows, int n_heads, int head_dim, int last_position) {
  const size_t chunks = (size_t)last_position / kChunk + 1;
  return (size_t)rows * n_heads * chunks * (size_t)slot_floats(head_dim);
}

bool attention_shape_ok(int n_heads, int n_kv_heads, int head_dim) {
  return n_kv_heads > 0 && n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= kMaxGroup && head_dim > 0 &&
         head_dim <= kMaxHeadDim;
}

// attn_tile's rows per block: as many as keep tile_rows x kv_mul within kMaxQv (16 for head_dim > 128, so LDS fits).
int attention_tile_rows(int rows, int kv_mul, int head_dim) {
  const int cap = head_dim > 128 ? kMaxQv / 4 : kMaxQv;
  const int tile = cap / kv_mul > 1 ? cap / kv_mul : 1;
  return rows < tile ? rows : tile;
}

size_t attention_tile_lds(int tile_rows, int kv_mul, int head_dim) {
  return ((size_t)kChunk * (2 * head_dim + 4) + (size_t)tile_rows * kv_mul * (head_dim + kChunk)) * sizeof(float);
}

// Batches of at least 16 rows with 64 or 128 dimensions per head, aligned, no fused RoPE: the flash kernel on the
// matrix cores, which needs no split partials. Its loads address a KV head's rows by 32-bit byte offsets, up to 64
// positions past the batch's last.
bool attention_uses_flash(const AttentionJob &job) {
  const int kv_mul = job.n_heads / job.n_kv_heads;
  const bool aligned = job.head_dim % 4 == 0 && job.pos_stride % 4 == 0 && job.head_base % 4 == 0 &&
                       ((uintptr_t)job.q & 15) == 0 && ((uintptr_t)job.key & 15) == 0;
  const bool offsets_fit =
      ((uint64_t)job.pos0 + (uint64_t)job.rows + kChunk) * job.pos_stride * 4 + (uint64_t)job.head_dim * 4 <= UINT32_MAX;
  return !job.table && aligned && job.rows >= 16 && (job.head_dim == 64 || job.head_dim == 128) && kv_mul <= 128 &&
         offsets_fit && ((uintptr_t)job.out & 15) == 0 && ((uintptr_t)job.value & 15) == 0;
}

// The batched kernel's form: attn_flash3 (products from exact BF16 parts) unless LLAMA_HIP_FLASH_FORM = fp32 picks
// attn_flash (FP32 products); read on every call.
bool attention_flash_bf3() {
  const char *form = getenv("LLAMA_HIP_FLASH_FORM");
  return !form || strcmp(form, "fp32") != 0;
}

// Blocks per tile of the batched kernel (0: one block per pair of tiles, no partials). A block walks its tiles' 64-position
// chunks at about the same time per chunk whatever the grid, so a grid of few blocks with long walks (a short batch
// late in a sequence: a prompt prefilled in batches) leaves most CUs idle for the whole walk. Split S gives each tile S
// blocks over shares of its chunks and adds attn_merge_shares. The choice is the S in {1, 2, 4, 8, 16} of least
// estimated time, with one 64-position walk taking the kernel's measured time (below): unsplit, the longest pair's
// chunks times the rounds of the CUs its grid takes; split, the longest share's chunks times the rounds, plus the
// merge; a split must save a tenth. Its partials stay within job.partial_room. LLAMA_HIP_FLASH_SPLITS = n forces n
// (1: never split), for tuning and tests.
int flash_splits(const AttentionJob &job, int chunks) {
  const int kv_mul = job.n_heads / job.n_kv_heads;
  const int tile_rows = 128 / kv_mul, tiles = (job.rows + tile_rows - 1) / tile_rows;
  const int cus = device().cu_count > 0 ? device().cu_count : 256;
  const char *env = getenv("LLAMA_HIP_FLASH_SPLITS");
  int splits = env && *env ? atoi(env) : 0;
  if (splits <= 0) {
    auto walk = [&](int t) { return (job.pos0 + min((t + 1) * tile_rows, job.rows) - 1) / kChunk + 1; };
    auto rounds = [&](long long blocks) { return (double)((blocks + cus - 1) / cus); };
    // the BF16-part kernel walks a 64-position span in about 5.7 us at head_dim 128 (3.5 at 64), and its merge grows
    // with the shares (each share's partials read and rescaled): fitted to forced splits of 128 to 512 rows at 8B, 3B
    // and 1B heads; the FP32-product kernel's figures are the first ones measured
    const bool bf3 = attention_flash_bf3();
    const double chunk_us = bf3 ? (job.head_dim == 128 ? 5.7 : 3.5) : (job.head_dim == 128 ? 10.0 : 6.0);
    auto merge = [&](int s) {
      const double per_row = job.rows * job.n_heads / 32.0;
      return bf3 ? 2.0 + 0.011 * per_row * s * job.head_dim / 128.0 : 2.0 + 0.012 * per_row;
    };
    const int pairs = (tiles + 1) / 2;
    const double unsplit = chunk_us * (walk(tiles - 1) + (tiles > 1 ? walk(0) : 0)) *
                           rounds((long long)pairs * job.n_kv_heads);
    double best = 0.9 * unsplit;
    splits = 1;
    for (int s = 2; s <= 16; s *= 2) {
      const double t = chunk_us * ((chunks + s - 1) / s) * rounds((long long)tiles * job.n_kv_heads * s) + merge(s);
      if (t < best)
        best = t, splits = s;
    }
  }
  splits = min(min(splits, 16), chunks);
  const size_t slot = slot_floats(job.head_dim);
  const size_t room = job.partial_room ? job.partial_room
                                       : attention_partial_floats(job.rows, job.n_heads, job.head_dim,
                                                                  job.pos0 + job.rows - 1);
  while (splits > 1 && (size_t)job.rows * job.n_heads * splits * slot > room)
    splits--;
  return splits > 1 ? splits : 0;
}

// The rows of a job that asks for them quantized, from its FP32 output (the paths that do not quantize in their
// epilogue): k_quantize_rows of n_heads * head_dim values per row.
bool quantize_attention_rows(const AttentionJob &job, hipStream_t stream) {
  if (!job.qout)
    return true;
  QuantizeJob qj{};
  qj.q = job.qout;
  qj.s = job.qscale;
  qj.x = job.out;
  qj.ldx = (size_t)job.n_heads * job.head_dim;
  qj.m = job.rows;
  qj.n = job.n_heads * job.head_dim;
  qj.gs = job.qgs;
  return launch_quantize(qj, stream);
}

bool launch_attention(const AttentionJob &job, float *partial, hipStream_t stream) {
  AttnParams p{};
  p.out = job.out;
  p.q = job.q;
  p.key = job.key;
  p.value = job.value;
  p.partial = partial;
  p.flags = device().error_flags;
  p.n_heads = job.n_heads;
  p.n_kv_heads = job.n_kv_heads;
  p.head_dim = job.head_dim;
  p.pos0 = job.pos0;
  p.chunks = (job.pos0 + job.rows - 1) / kChunk + 1;
  if (p.chunks > kMaxMergeChunks)
    return raise("attention over %d positions: at most %d are supported", job.pos0 + job.rows, kMaxMergeChunks * kChunk);
  p.pos_stride = job.pos_stride;
  p.head_base = job.head_base;
  p.divisor = sqrtf((float)job.head_dim);
  p.rows = job.rows;
  p.slot = slot_floats(job.head_dim);
  p.rope_q = const_cast<float *>(job.q);
  p.k_new = job.k_new;
  p.v_new = job.v_new;
  p.table = job.table;
  const int kv_mul = job.n_heads / job.n_kv_heads;
  const bool aligned = job.head_dim % 4 == 0 && job.pos_stride % 4 == 0 && job.head_base % 4 == 0 &&
                       ((uintptr_t)job.q & 15) == 0 && ((uintptr_t)job.key & 15) == 0;
  if (job.table && !aligned)
    return raise("internal: a fused RoPE attention on operands the aligned kernel does not take");
  if (attention_uses_flash(job)) {
    // two staged chunks of K and two of V rows in static LDS: 4 x 64 x HD floats (128 KB at HD = 128); a block per
    // pair of tiles, or per tile and share of its chunks (flash_splits)
    const int tile_rows = 128 / kv_mul, tiles = (job.rows + tile_rows - 1) / tile_rows;
    p.splits = flash_splits(job, p.chunks);
    const dim3 grid(p.splits ? (unsigned)tiles : (unsigned)((tiles + 1) / 2), (unsigned)job.n_kv_heads,
                    p.splits ? (unsigned)p.splits : 1u);
    const bool bf3 = attention_flash_bf3();
    const bool fused_quant = job.qout && bf3 && !p.splits;
    if (fused_quant) {
      p.qout = job.qout;
      p.qscale = job.qscale;
      p.qgs = job.qgs;
    }
    if (bf3 && job.head_dim == 128)
      hipLaunchKernelGGL(attn_flash3<128>, grid, dim3(kTileThreads), 0, stream, p);
    else if (bf3)
      hipLaunchKernelGGL(attn_flash3<64>, grid, dim3(kTileThreads), 0, stream, p);
    else if (job.head_dim == 128)
      hipLaunchKernelGGL(attn_flash<128>, grid, dim3(kTileThreads), 0, stream, p);
    else
      hipLaunchKernelGGL(attn_flash<64>, grid, dim3(kTileThreads), 0, stream, p);
    if (!launch_ok(bf3 ? "attn_flash3" : "attn_flash"))
      return false;
    if (p.splits) {
      const long long threads = (long long)job.rows * job.n_heads * (job.head_dim / 4);
      hipLaunchKernelGGL(attn_merge_shares, dim3((unsigned)((threads + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                         stream, p);
      if (!launch_ok("attn_merge_shares"))
        return false;
    }
    return fused_quant || quantize_attention_rows(job, stream);
  }
  // decode: the slice-parallel kernel for 64 or 128 dimensions and up to eight query vectors per KV head
  if (aligned && job.rows == 1 && (job.head_dim == 64 || job.head_dim == 128) && kv_mul <= kDecodeMaxQv &&
      kv_mul * job.head_dim / 4 <= kTileThreads) {
    p.tile_rows = 1;
    const dim3 grid((unsigned)p.chunks, (unsigned)job.n_kv_heads);
    const size_t lds = attention_decode_lds(kv_mul, job.head_dim);
    if (job.head_dim == 128)
      hipLaunchKernelGGL(attn_decode<128>, grid, dim3(kTileThreads), lds, stream, p);
    else
      hipLaunchKernelGGL(attn_decode<64>, grid, dim3(kTileThreads), lds, stream, p);
    if (!launch_ok("attn_decode"))
      return false;
  } else if (aligned) {
    p.tile_rows = attention_tile_rows(job.rows, kv_mul, job.head_dim);
    const size_t lds = attention_tile_lds(p.tile_rows, kv_mul, job.head_dim);
    typedef void (*TileKernel)(AttnParams);
    // [grouped][head_dim 128, 64, other]
    static const TileKernel kernels[2][3] = {{attn_tile<1, 128>, attn_tile<1, 64>, attn_tile<1, 0>},
                                             {attn_tile<kQvGroup, 128>, attn_tile<kQvGroup, 64>, attn_tile<kQvGroup, 0>}};
    static const hipError_t allowed = [] {
      for (const auto &row : kernels)
        for (TileKernel k : row) {
          const hipError_t e =
              hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
          if (e != hipSuccess)
            return e;
        }
      return hipSuccess;
    }();
    if (allowed != hipSuccess)
      return raise("allowing the attention kernel its LDS failed: %s", hipGetErrorString(allowed));
    const unsigned tiles = (unsigned)((job.rows + p.tile_rows - 1) / p.tile_rows);
    // the grouped form needs every tile's query-vector count (rows x kv_mul) to be a multiple of the group
    const bool grouped = job.rows > 1 && kv_mul % kQvGroup == 0;
    const TileKernel kernel = kernels[grouped][job.head_dim == 128 ? 0 : job.head_dim == 64 ? 1 : 2];
    hipLaunchKernelGGL(kernel, dim3((unsigned)p.chunks, (unsigned)job.n_kv_heads, tiles), dim3(kTileThreads), lds,
                       stream, p);
    if (!launch_ok("attn_tile"))
      return false;
  } else {
    hipLaunchKernelGGL(attn_chunks, dim3((unsigned)p.chunks, (unsigned)job.n_kv_heads, (unsigned)job.rows),
                       dim3(kThreads), 0, stream, p);
    if (!launch_ok("attn_chunks"))
      return false;
  }
  hipLaunchKernelGGL(attn_merge, dim3((unsigned)job.n_heads, (unsigned)job.rows), dim3(kThreads), 0, stream, p);
  return launch_ok("attn_merge") && quantize_attention_rows(job, stream);
}

} // namespace llhip
