/* CPU oracle for the llama3.x.c matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library links, loads or calls this code: only tests/, the smoke
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py use it, and only as the checker (or the timed CPU
 * baseline), never as the thing measured on the GPU.
 *
 * Every function restates one piece of the reference's scalar (portable) arithmetic, cited by file:line of
 * LucianCrainic/llama3.x.c. "Scalar" matters: the reference's AVX-512/AMX rungs sum FP32 in other orders, so they agree
 * with these functions within the kernel budget, while its scalar instruction set agrees bit for bit. How each function
 * is pinned (golden vectors written by the reference itself, known-answer vectors, closed forms) is listed in
 * tests/test_oracle.py; a function without such a pin would say "parity unpinned" here. All functions are pinned.
 *
 * Build: oracle/Makefile (gcc, -std=c11 -O2 -ffp-contract=off, no -march: plain SSE2 float arithmetic, every operation
 * rounded to float, as the reference's scalar path compiles). */
#ifndef LLAMA_ORACLE_H
#define LLAMA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

/* The two epilogue enumerations of the reference, which order their members differently:
 * KernelEpilogue (include/kernels.h:82) for the GEMV entry points, GemmKind (include/gemm.h:15-20) for the GEMMs. */
enum { ORC_K_STORE = 0, ORC_K_ADD = 1, ORC_K_PARTIAL = 2, ORC_K_SWIGLU = 3 };
enum { ORC_GEMM_STORE = 0, ORC_GEMM_ADD = 1, ORC_GEMM_SWIGLU = 2, ORC_GEMM_PARTIAL = 3 };

/* Activation quantization, src/gemv.c:589-624 (k_quantize): per group of gs values, scale = max|x| / 127.0f and
 * q = (int8)roundf(clamp(x / scale, -127, 127)), q = 0 where the scale is 0. Returns -1 (and stops) on a non-finite
 * input, where the reference calls fail("nonfinite activation during INT8 quantization"); 0 otherwise. */
int orc_quantize(int8_t *q, float *s, const float *x, int n, int gs);
/* src/gemm.c:819-830 (k_quantize_rows): orc_quantize per row; q has row stride n, s row stride n / gs. */
int orc_quantize_rows(int8_t *q, float *s, const float *x, size_t ldx, int m, int n, int gs);

/* SwiGLU gate, src/gemv.c:246-250 and src/gemm.c:42-45: value * (1 / (1 + expf(-value))) * gate. */
float orc_silu_gate(float value, float gate);

/* Scalar Q8 row dots, src/gemv.c:401-439 (q8_dots, scalar branch): for each of `rows` weight rows starting at wq
 * (row stride ld values, scales row stride ld / gs), out[r] = sum over whole groups of
 * ((float)(int32 dot of the group) * ws[g]) * xs[g], in group order (W8A8). With xq == NULL the W8A32 form:
 * (sum over the group of (float)w * xf) * ws[g]. */
void orc_q8_dots(float *out, const int8_t *wq, const float *ws, size_t ld, int rows, const int8_t *xq, const float *xs,
                 const float *xf, int n, int gs);

/* The Q8 GEMV entry points, src/gemv.c:455-528 and 565-587: d outputs of n inputs, weight row stride ld (0 = n),
 * epilogue `kind` as KernelEpilogue (STORE and PARTIAL store, ADD adds, SWIGLU gates w by w3). */
void orc_matmul_q8(float *out, const int8_t *xq, const float *xs, const float *xf, const int8_t *wq, const float *ws,
                   const int8_t *w3q, const float *w3s, size_t ld, int n, int d, int gs, int kind);

/* Exact int32 group dots of m activation rows (row stride ldx) against n weight rows (row stride ldw):
 * dots[(g * m + r) * n + c] = sum over the gs values of group g of xq[r] * wq[c]. This is the closed form the
 * reference's int32 probe is checked against (tests/q8.c:198-218; the probe itself is src/gemm.c:598-599). */
void orc_group_dots(int32_t *dots, const int8_t *xq, size_t ldx, int m, const int8_t *wq, size_t ldw, int n, int k,
                    int gs);

/* The portable batched Q8 GEMM, src/gemm.c:839-854 (q8_micro_portable) with the epilogue of src/gemm.c:963-989:
 * C[m][n] (op)= per-row scalar Q8 dots, so row i is bitwise the GEMV of row i. kind is a GemmKind. xq/xs are dense
 * (row strides k and k / gs); weights have row stride k. Row padding of C beyond n (up to ldc) is never written. */
void orc_gemm_q8(const int8_t *xq, const float *xs, int m, int k, int gs, float *c, int ldc, const int8_t *wq,
                 const float *ws, const int8_t *w3q, const float *w3s, int n, int kind);

/* Scalar FP32 GEMV, src/gemv.c:252-267 (f32_dots, scalar branch) with the epilogues of src/gemv.c:284-303: ascending
 * j, one float accumulator. kind is a KernelEpilogue; ld = weight row stride (0 = n). */
void orc_matmul_f32(float *out, const float *x, const float *w, const float *w3, size_t ld, int n, int d, int kind);

/* The portable FP32 GEMM with one K block, src/gemm.c:47-57 (micro_portable) and 125-169 (accumulate, gemm_chunks):
 * per output the ascending-k float sum, added to a zeroed accumulator, then the epilogue. kind is a GemmKind. */
void orc_gemm_f32(const float *a, int lda, int m, int k, float *c, int ldc, const float *w, const float *w3,
                  size_t ldw, int n, int kind);

/* BF16 conversion, src/gemm.c:332-349: round to nearest even on the dropped 16 bits, NaN quieted (sign and top payload
 * kept), no flush of denormals, values at or past the midpoint to 2^128 become infinity; and the exact widening. */
uint16_t orc_bf16_from_f32(float x);
float orc_f32_from_bf16(uint16_t v);

/* The packed weight layouts the reference's GEMM entry points take, src/gemm.c:355-398: 16-row tiles, K padded to 32
 * (BF16 pairs) or 64 (int8 quads), zero-filled. */
size_t orc_bf16_vnni_elements(int rows, int cols);
size_t orc_s8_vnni_bytes(int rows, int cols);
void orc_pack_bf16_vnni(uint16_t *dst, const float *w, int rows, int cols, size_t ld);
void orc_pack_s8_vnni(int8_t *dst, const int8_t *w, int rows, int cols, size_t ld);

/* The portable BF16 GEMM, src/gemm.c:667-738: activations rounded to BF16 (RNE), products of two BF16 values exact in
 * FP32, summed in ascending K into one float, then the FP32 epilogue. pw/pw3 are packed by orc_pack_bf16_vnni for this
 * k. kind is a GemmKind. */
void orc_gemm_bf16(const float *a, int lda, int m, int k, float *c, int ldc, const uint16_t *pw, const uint16_t *pw3,
                   int n, int kind);

/* CPU timing rung: the scalar Q8 GEMV of orc_matmul_q8 (STORE) split statically over `threads` pthreads by rows, as the
 * reference's team driver splits a GEMV (src/gemv.c:488-495). Used only as bench.py's fallback CPU baseline when the
 * reference itself is not built. */
void orc_matmul_q8_threads(float *out, const int8_t *xq, const float *xs, const int8_t *wq, const float *ws, int n,
                           int d, int gs, int threads);


/* ---- the device-resident forward around the matmuls (RMSNorm, RoPE, the K/V cache, attention) ------------------- */

/* src/kernels.c:8-21 (rmsnorm_eps): ss = sum of x[j] * x[j] in index order, ss /= size, ss += epsilon,
 * ss = 1 / sqrtf(ss); out[j] = weight[j] * (ss * x[j]). out may equal x. */
void orc_rmsnorm(float *out, const float *x, const float *weight, int size, float epsilon);
/* src/kernels_simd.c:203-225 (scalar k_rope_apply): per head and pair j, c = table[j], s = table[head_dim + j + 1],
 * (a, b) -> (a*c - b*s, a*s + b*c), products rounded before the sum (no fused multiply-add); k for the first
 * n_kv_heads heads. */
void orc_rope_apply(float *q, float *k, const float *table, int n_heads, int n_kv_heads, int head_dim);
/* src/attention.c:1420-1432: `count` rows of n_kv_heads * head_dim floats (row stride src_ld) to positions pos0..,
 * at cache + t * pos_stride + g * head_base for KV head g (rows layout: pos_stride = kv_dim, head_base = head_dim;
 * head-major: pos_stride = head_dim, head_base = seq_len * head_dim). */
void orc_kv_store(float *cache, const float *src, size_t src_ld, int pos0, int count, int n_kv_heads, int head_dim,
                  size_t pos_stride, size_t head_base);
/* src/attention.c:606-641 with softmax src/kernels.c:23-45 (the scalar decode): per head h (KV head h / kv_mul),
 * score[t] = (sum_i q[i] * k_t[i]) / sqrtf(head_dim) for t = 0..position in index order, softmax (max, expf(x - max),
 * their sum, then each divided by it), out = sum_t w_t * v_t accumulated in t order. Returns -1 (the reference's fail)
 * when a score is not finite. att holds n_heads rows of seq_len scores. */
int orc_attention(float *out, const float *q, const float *key_cache, const float *value_cache, float *att,
                  int n_heads, int n_kv_heads, int head_dim, int seq_len, int position, size_t pos_stride,
                  size_t head_base);

/* ---- seeded synthetic inputs (shared by the golden-vector script, the tests and bench.py's CPU leg) ---------------
 * The reference tests' generator, tests/q8.c:19-30: xorshift64 (shifts 13, 7, 17) from seed 88172645463325252, and
 * uniform() = (float)((double)(x >> 40) / 2^24) * 2 - 1. orc_fill_normal draws N(mean, std) by Box-Muller from pairs
 * of those uniforms mapped to (0, 1]: z0 = sqrt(-2 ln u1) cos(2 pi u2), z1 = sqrt(-2 ln u1) sin(2 pi u2), computed in
 * double and rounded to float. `state` advances in place. */
uint64_t orc_rng_next(uint64_t *state);
float orc_rng_uniform(uint64_t *state);
void orc_fill_uniform(float *dst, size_t n, uint64_t *state, float scale);
void orc_fill_normal(float *dst, size_t n, uint64_t *state, float mean, float std);
#endif
