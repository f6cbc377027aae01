/* The batched-prefill half of the llama3.x.c kernel surface, served by MFMA kernels on an MI355X (gfx950).
 *
 * Drop-in for the reference's include/gemm.h: the same names, struct layouts and error behaviour, with C linkage, so
 * the reference's batched forward (tp.c:475-622) calls these in place of src/gemm.c. Each declaration cites the
 * reference declaration it replaces (LucianCrainic/llama3.x.c file:line). Pointer residency as in llama_hip_kernels.h. */
#ifndef LLAMA_HIP_GEMM_H
#define LLAMA_HIP_GEMM_H

#include "llama_hip_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

/* gemm.h:15-20 */
typedef LLHIP_ENUM {
  GEMM_STORE,  /* c = acc */
  GEMM_ADD,    /* c += acc */
  GEMM_SWIGLU, /* c = silu(acc of w) * acc of w3 */
  GEMM_PARTIAL /* c = acc, like STORE */
} GemmKind;

/* gemm.h:22-30 */
typedef struct {
  float *c; /* m x n output, row-major, leading dimension ldc; columns n..ldc-1 are never written */
  int ldc;
  const float *w;  /* n x k weights, leading dimension ldw */
  const float *w3; /* GEMM_SWIGLU only */
  size_t ldw;
  int n;
  GemmKind kind;
} GemmSegment;

enum { GEMM_MAX_SEGMENTS = 3 }; /* gemm.h:32 */

/* gemm.h:34: C[m][n] (op)= A[m][k] . W[n][k]^T for up to three segments sharing A, on FP32 MFMA; agrees with the
 * reference within 2e-5 * sum|a w| + 1e-6. */
void k_gemm_f32(const float *a, int lda, int m, int k, const GemmSegment *segments, int count);
int k_gemm_kc(void); /* gemm.h:37: 0 (one K block, no CPU blocking here) */

/* gemm.h:46-52: CPU AMX status, for the report: always unavailable ("not requested") in this library. */
const char *gemm_amx_unavailable(void);
const char *gemm_amx_permission(void);
void gemm_amx_enable(int on);
int gemm_amx_active(void);
int gemm_amx_emulated(void);
void gemm_amx_thread_release(void);

/* gemm.h:55-56: FP32 to BF16 with round to nearest even (NaN quieted, denormals kept, overflow to infinity), and back. */
uint16_t bf16_from_f32(float x);
float f32_from_bf16(uint16_t v);

/* gemm.h:63-68: the packed weight layouts (16-row tiles, K pairs / quads, zero padding). The BF16 GEMM below reads the
 * BF16 layout directly; the int8 one is accepted and not needed (the Q8 GEMM reads the row-major values). */
size_t bf16_vnni_elements(int rows, int cols);
size_t s8_vnni_bytes(int rows, int cols);
void pack_bf16_vnni(uint16_t *dst, const float *w, int rows, int cols, size_t ld);
void pack_bf16_vnni_tiles(uint16_t *dst, const float *w, int rows, int cols, size_t ld, int first, int last);
void pack_s8_vnni(int8_t *dst, const int8_t *w, int rows, int cols, size_t ld);
void pack_s8_vnni_tiles(int8_t *dst, const int8_t *w, int rows, int cols, size_t ld, int first, int last);

/* gemm.h:74-75: the CPU tile microkernels; not compiled into this build, they fail like the reference's build
 * without AMX (gemm.c:611-627). */
void amx_bf16_tile_gemm(float *c, size_t ldc, const uint16_t *a, size_t lda, const uint16_t *bp, int m, int n, int k);
void amx_s8_tile_gemm(int32_t *c, size_t ldc, const int8_t *a, size_t lda, const int8_t *bp, int m, int n, int k);

/* gemm.h:78-83: a 64-byte-aligned host workspace (malloc'd here; the reference's accounted allocator is not part of
 * this library, so `kind` is only recorded). */
typedef LLHIP_ENUM {
  MEM_KV,
  MEM_ACTIVATION,
  MEM_EMBEDDING,
  MEM_METADATA,
  MEM_TOKENIZER,
  MEM_SAMPLER,
  MEM_PROMPT,
  MEM_WEIGHTS_OWNED,
  MEM_WEIGHTS_PACKED,
  MEM_COUNT
} MemoryKind; /* runtime.h:38-49 */
typedef struct {
  void *base, *data;
  size_t bytes;
} AlignedBuffer;
void aligned_buffer_alloc(AlignedBuffer *buffer, size_t bytes, MemoryKind kind);
void aligned_buffer_free(AlignedBuffer *buffer);

/* gemm.h:89-104: BF16 GEMM. Activations are rounded to BF16 (RNE) on the device, weights come packed by
 * pack_bf16_vnni for this k, the sums are FP32 on BF16 MFMA. `panel` is validated like the reference's (it must hold
 * k_gemm_bf16_panel_bytes(m, k)); the device keeps its own panel, so the host buffer is not written. */
typedef struct {
  float *c;
  int ldc;
  const uint16_t *w;
  const uint16_t *w3;
  int n;
  GemmKind kind;
} GemmBf16Segment;
size_t k_gemm_bf16_panel_bytes(int m, int k);
void k_gemm_bf16(const float *a, int lda, int m, int k, const GemmBf16Segment *segments, int count,
                 AlignedBuffer *panel);

/* gemm.h:107-113 */
typedef struct {
  uint16_t *dst;
  const float *w;
  int rows, cols;
  size_t ld;
} PackBf16;
void pack_bf16_vnni_many(const PackBf16 *jobs, int count);

/* gemm.h:118-126. Q8GemmBackend gains Q8_GEMM_HIP_MFMA, the int8-MFMA kernel (gs % 64 == 0); Q8_GEMM_PORTABLE names
 * the GPU's generic kernel for other group sizes. */
typedef struct {
  float *c;
  int ldc;
  K8Weight w, w3;
  const int8_t *pw, *pw3; /* AMX packed copies: accepted, not read */
  int n;
  GemmKind kind;
} GemmQ8Segment;
typedef LLHIP_ENUM { Q8_GEMM_PORTABLE, Q8_GEMM_AVX512, Q8_GEMM_AMX, Q8_GEMM_HIP_MFMA } Q8GemmBackend;

/* gemm.h:130: k_quantize per row (row r of q has stride n, of s stride n / gs), bitwise the per-token result. */
void k_quantize_rows(int8_t *q, float *s, const float *x, size_t ldx, int m, int n, int gs);
/* gemm.h:133: C[m][n] (op)= sum over groups of (float)(int32 dot) * xs[m][g] * ws[n][g] with exact int32 group dots on
 * int8 MFMA (v_mfma_i32_16x16x64_i8, one 64-wide group per instruction) and an FP32 rescale-accumulate. */
void k_gemm_q8(const int8_t *xq, const float *xs, int m, int k, int gs, const GemmQ8Segment *segments, int count);
Q8GemmBackend k_gemm_q8_pick(int gs, const GemmQ8Segment *segments, int count); /* gemm.h:135 */
/* No counterpart in the reference: hb = silu(W1 x) * (W3 x) as k_gemm_q8's GEMM_SWIGLU forms it, quantized in the
 * GEMM's epilogue (groups of 64: hq int8 [m][n], hs [m][n / 64]) instead of written out in FP32; bitwise k_gemm_q8
 * GEMM_SWIGLU then k_quantize_rows of its output (the engine's batched forward, src/tp.c:580-584). Returns 1 when it
 * ran, 0 with nothing launched when the shape does not take the wide int8 kernel unsplit (gs 64, n % 64 == 0, the
 * launcher's choice for m, n, k); a non-finite value fails at the next synchronization, as k_quantize_rows does. */
int llhip_gemm_q8_swiglu_quantize(const int8_t *xq, const float *xs, int m, int k, int gs, const K8Weight *w1,
                                  const K8Weight *w3, int n, int8_t *hq, float *hs);

/* gemm.h:138-144 */
typedef struct {
  int8_t *dst;
  const int8_t *w;
  int rows, cols;
  size_t ld;
} PackS8;
void pack_s8_vnni_many(const PackS8 *jobs, int count);

/* shards.h:10, 28-38, 66-78: the loaded weight shard the packing jobs of gemm.h:146-153 read, in the reference's
 * layout (role is a TensorRole). */
typedef LLHIP_ENUM { DT_F32, DT_Q8 } TensorDtype;
typedef LLHIP_ENUM { SHARD_ROWS, SHARD_COLS, SHARD_COPY, SHARD_GLOBAL } ShardKind;
typedef struct {
  int role;
  int layer;
  int rows, cols;
  TensorDtype dtype;
  int group_size;
  size_t offset;
  size_t scale_offset;
  size_t bytes;
  int alias_of;
} TensorDesc;
typedef struct {
  const TensorDesc *src;
  ShardKind kind;
  int socket;
  int row0, rows, col0, cols;
  int alias;
  size_t q_offset, s_offset;
  void *q;
  float *s;
  size_t ld;
} Shard;
/* gemm.h:152-153: the packing job of a bound ROWS or COLS shard of the right dtype (FP32 for BF16, Q8 for int8) at its
 * own stride; anything else fails with the reference's message. */
PackBf16 pack_bf16_job_from_shard(uint16_t *dst, const Shard *shard);
PackS8 pack_s8_job_from_shard(int8_t *dst, const Shard *shard);

/* testing.h:27, 61-69 analogues. k_gemm_f32_portable runs the device FP32 GEMM (kc is ignored: no K blocking);
 * k_gemm_f32_simd_test returns 0 (no CPU SIMD kernel here); k_gemv_force_hybrid is accepted (one device schedule).
 * k_gemm_q8_backend_test runs one named backend (Q8_GEMM_HIP_MFMA or Q8_GEMM_PORTABLE; returns 0 for the CPU ones).
 * llhip_q8_group_dots is the int32 probe: the exact group dots the MFMA kernel forms, dots[(g * m + r) * n + c], from
 * row-major xq (m x k) and wq (n x k). k_gemm_q8_amx_dots_test (testing.h:69) returns the same dots from weights in
 * the pack_s8_vnni layout, as the reference's AMX probe does: 1 when it ran, 0 for shapes the MFMA probe does not take
 * (gs % 64 != 0 or k % gs != 0), as a build without AMX returns 0. */
void k_gemm_f32_portable(const float *a, int lda, int m, int k, const GemmSegment *segments, int count, int kc);
int k_gemm_f32_simd_test(const float *a, int lda, int m, int k, const GemmSegment *segments, int count, int kc);
void k_gemv_force_hybrid(int on);
int k_gemm_q8_backend_test(Q8GemmBackend backend, const int8_t *xq, const float *xs, int m, int k, int gs,
                           const GemmQ8Segment *segments, int count);
void llhip_q8_group_dots(int32_t *dots, const int8_t *xq, int m, int k, int gs, const int8_t *wq, int n);
int k_gemm_q8_amx_dots_test(int32_t *dots, const int8_t *xq, int m, int k, int gs, const int8_t *packed, int n);

#ifdef __cplusplus
}
#endif
#endif
