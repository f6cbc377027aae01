/* The forward around the matmuls, served on an MI355X (gfx950): RMSNorm, RoPE, the K/V cache and causal attention, so
 * a device-resident engine keeps its activations in HBM between the matmuls. Drop-in for these declarations of the
 * reference's include/kernels.h (and the layout selectors of include/testing.h): the same names, argument meaning and
 * struct layouts, with C linkage. Each declaration cites the one it replaces (LucianCrainic/llama3.x.c file:line).
 *
 * Pointers follow llama_hip_kernels.h: device memory in place (stream-ordered, no wait), registered host ranges through
 * their device copies, other host memory copied in and out around a synchronous call. */
#ifndef LLAMA_HIP_FORWARD_H
#define LLAMA_HIP_FORWARD_H

#include <stddef.h>
#include <stdint.h>

#include "llama_hip_prefill.h" /* Config (include/runtime.h:9-16): k_rope_table reads head_dim and the rope fields */

#ifdef __cplusplus
extern "C" {
#endif

/* kernels.h:57-60: out = weight * (ss * x) with ss = 1 / sqrtf(mean(x^2) + epsilon), per row; out may equal x. The
 * products are the reference's; the sum of squares is reduced in another order (within 1e-6 relative of it). */
void k_rmsnorm(float *out, const float *x, const float *weight, int size, float epsilon);
void k_rmsnorm_rows(float *out, const float *x, const float *weight, int rows, int size, float epsilon);
/* No counterpart in the reference: k_rmsnorm_rows then k_quantize_rows of the same rows in one launch, bitwise the two
 * calls, without the normalized rows in memory (for the engine's batched forward, src/tp.c:546-547, 576-577). Rows of
 * at most 8192 values in whole groups of gs, a power of two from 4 to 256; x and weight 16-byte aligned, q 4-byte
 * aligned. A non-finite normalized value fails at the next synchronization, as k_quantize_rows does. */
void llhip_rmsnorm_quantize_rows(int8_t *q, float *s, const float *x, const float *weight, int rows, int size,
                                 float epsilon, int gs);

/* kernels.h:61-68: one position's table (2 * head_dim floats: cosines duplicated per pair, then -sin, +sin), computed
 * on the host with the C library as the reference computes it (src/kernels.c:49-61); and the rotation of q's n_heads and
 * k's n_kv_heads heads by it, bitwise the reference's (products rounded before the sum). */
void k_rope_table(const Config *p, int position, float *table);
void k_rope_apply(float *q, float *k, const float *table, int n_heads, int n_kv_heads, int head_dim);
void k_rope_apply_rows(float *q, size_t q_stride, float *k, size_t k_stride, const float *table, size_t table_stride,
                       int rows, int n_heads, int n_kv_heads, int head_dim);
/* No counterpart in the reference: k_rope_apply_rows of q and k, then k_kv_store of k and of v at positions pos0 ..
 * pos0 + rows - 1 of the caches (the selected layout), in one launch and bitwise those three calls (k is also left
 * rotated in place); for the engine's batched forward (src/tp.c:550-557). head_dim and the strides multiples of 4, one
 * table row of 2 * head_dim values per row (table_stride >= 2 * head_dim), 16-byte aligned q, k, v, table and caches,
 * and the k and v rows outside both caches; anything else fails with a message. */
void llhip_rope_kv_store_rows(float *q, size_t q_stride, float *k, const float *v, size_t kv_stride, const float *table,
                              size_t table_stride, int rows, int n_heads, int n_kv_heads, int head_dim,
                              float *key_cache, float *value_cache, int pos0, int seq_len);

/* The embedding lookup of a Q8_0 table (vocab x dim int8 values, one float scale per gs consecutive values), inline
 * in the reference's forward (src/tp.c:395-396 for a token, 444-456 for a batch): out row i = table row ids[i], each
 * value (float)q * scale, bitwise. ids is read on the device; an id outside [0, vocab) fails with "embedding row id
 * outside the table" at the next host-visible point and leaves its row unwritten. The table and scales are usually a
 * registered host range (the tied classifier's weights) or device memory; a plain host table is staged whole on every
 * call (vocab x dim bytes), so register it once. */
void k_embed_q8_rows(float *out, const signed char *table, const float *scales, const int *ids, int count, int dim,
                     int gs, int vocab);
/* The same lookup in an FP32 table (vocab x dim floats; src/tp.c:342 for a token, 449 for a batch, where run copies
 * the row): out row i = table row ids[i], a copy; the same id check and failure. */
void k_embed_f32_rows(float *out, const float *table, const int *ids, int count, int dim, int vocab);

/* kernels.h:127-132: the attention workspace record. The device attention keeps its split-K partials in a library
 * workspace; this record only carries the shapes (partial is never dereferenced). */
typedef struct {
  float *partial;
  int max_chunks, n_heads, head_dim, workers;
  int external;
  size_t capacity;
} AttentionWork;
void k_attention_init(AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len); /* kernels.h:133 */
size_t k_attention_bytes(int n_heads, int n_kv_heads, int head_dim, int seq_len);                   /* kernels.h:135 */
void k_attention_init_in(AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len,
                         float *memory);                                                             /* kernels.h:136 */
size_t k_attention_bytes_rows(int n_heads, int n_kv_heads, int head_dim, int seq_len, int rows);    /* kernels.h:139 */
void k_attention_init_rows(AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int rows,
                           float *memory);                                                           /* kernels.h:140 */
int k_attention_chunk_count(const AttentionWork *work, int n_kv_heads, int position);               /* kernels.h:150 */
void k_attention_free(AttentionWork *work);                                                          /* kernels.h:151 */

/* kernels.h:146-166: causal attention. q and out hold m rows of n_heads * head_dim floats; row i (position pos0 + i)
 * attends to positions 0..pos0 + i of its KV head (query head h uses KV head h / (n_heads / n_kv_heads)). Scores are
 * (q . k) / sqrtf(head_dim), softmax-weighted sums of the values, computed over 64-position chunks merged by their
 * maxima (the reference's split-K form, src/attention.c:664-682, 841-876). The plain forms read the rows layout
 * [position][kv_head][head_dim]; _layout takes the strides (position t of KV head g at cache + t * pos_stride +
 * g * head_base). att is the reference's score scratch and is not used. A non-finite score fails with "nonfinite value
 * in softmax" (at the next host-visible point when the buffers are device memory). */
void k_attention(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                 AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int position);
void k_attention_layout(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                        AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int position,
                        size_t pos_stride, size_t head_base);
void k_attention_batch(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                       AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int pos0, int m);
void k_attention_batch_layout(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                              AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int pos0,
                              int m, size_t pos_stride, size_t head_base);
/* No counterpart in the reference: k_attention_batch_layout for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). It allocates nothing: its split-K partials live in
 * a fixed per-device array of 4 Mi floats (16 MiB, located when llhip_init opens the device), not in the workspace the
 * other forms grow on first use. Every buffer must be device memory or inside a registered range (host buffers would
 * need the staging arena), the library must be initialized (llhip_init), and a call that runs a split kernel (fewer
 * than 16 rows, or a head_dim other than 64 and 128, or unaligned operands) must fit: m rows of n_heads heads up to
 * position pos0 + m - 1 take m * n_heads * ((pos0 + m - 1) / 64 + 1) * ((head_dim + 5) & ~3) floats, at most 4 Mi
 * (decode with 32 heads of 128 reaches position 63487); batches the flash kernel takes (16 rows and more, head_dim
 * 64 or 128, 16-byte aligned operands) have no such limit: they keep partials only when a short batch late in a
 * sequence splits its positions over blocks, and then split only as far as the array holds. Anything else fails with
 * a message. The results equal k_attention_batch_layout's bit for bit, except for a flash batch whose position split
 * had to be narrower to fit the array (then they differ in FP32 summation order only). Every call on a device shares
 * its array, which keeps the last call's
 * contents (every slot a call reads it writes first); calls ordered on the library's stream are safe, two that may
 * run concurrently on one GPU (graphs replayed on other streams) race. */
void k_attention_batch_layout_noalloc(float *out, const float *q, const float *key_cache, const float *value_cache,
                                      float *att, AttentionWork *work, int n_heads, int n_kv_heads, int head_dim,
                                      int seq_len, int pos0, int m, size_t pos_stride, size_t head_base);

/* kernels.h:52-53, 168-179: the engine-facing K/V cache of one layer in the active layout (LLAMA_KV_LAYOUT=rows|head,
 * head-major by default), and k_attention / k_attention_batch on it. */
int kernels_kv_layout_head(void);
const char *kernels_kv_layout_name(void);
void k_kv_strides(int n_kv_heads, int head_dim, int seq_len, size_t *pos_stride, size_t *head_base);
void k_kv_store(float *cache, const float *src, size_t src_ld, int pos0, int count, int n_kv_heads, int head_dim,
                int seq_len);
void k_attention_kv(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                    AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int position);
void k_attention_batch_kv(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                          AttentionWork *work, int n_heads, int n_kv_heads, int head_dim, int seq_len, int pos0, int m);
/* No counterpart in the reference: k_attention_batch_kv, then k_quantize_rows of its m rows of n_heads * head_dim
 * values in groups of gs into q and s, bitwise those two calls (for the engine's batched forward, src/tp.c:558-576,
 * where the attention rows are quantized for Wo). The batched kernel quantizes its own output where it runs a tile
 * whole (out is then not written); otherwise out receives the FP32 rows and they are quantized from there, so out must
 * hold them. gs one of 16, 32, 64, 128 dividing head_dim; q 4-byte aligned; a non-finite value fails at the next
 * synchronization, as k_quantize_rows does. */
void llhip_attention_batch_quantize(int8_t *q, float *s, int gs, float *out, const float *query, const float *key_cache,
                                    const float *value_cache, int n_heads, int n_kv_heads, int head_dim, int seq_len,
                                    int pos0, int m);

/* kernels.h:46-47 and testing.h: the attention kernels' names ("split" for both: one device kernel) and the test-time
 * selectors, which accept the reference's names (tiled / split, split / group; rows / head). */
const char *kernels_attention_name(void);
const char *kernels_attention_decode_name(void);
int kernels_attention_select(const char *batch, const char *decode);
int kernels_kv_layout_select(const char *name);

#ifdef __cplusplus
}
#endif
#endif
