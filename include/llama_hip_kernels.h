/* The GEMV half of the llama3.x.c kernel surface, served by HIP kernels on an MI355X (gfx950).
 *
 * Drop-in for the reference's include/kernels.h as far as the matmul hot path goes: the same names, argument meaning,
 * struct layouts and error behaviour, with C linkage, so the reference's engine (tp.c) calls these in place of
 * src/gemv.c. Each declaration cites the reference declaration it replaces (LucianCrainic/llama3.x.c file:line).
 *
 * Pointers may be device memory (used in place, the calls are stream-ordered on the library stream and return
 * before the GPU finishes), host memory inside a range registered with llhip_register_host (resolved to its device
 * copy), or any other host memory (copied in and out around a synchronous call). See llama_hip.h. */
#ifndef LLAMA_HIP_KERNELS_H
#define LLAMA_HIP_KERNELS_H

#include <stddef.h>
#include <stdint.h>

/* C++ (this library) sees these C enums with int as their underlying type, so every int a C caller passes is a value
 * of the enum: an invalid request reaches the library's check instead of being undefined behaviour to load. C callers
 * see plain enums, the reference's declarations. */
#ifndef LLHIP_ENUM
#ifdef __cplusplus
#define LLHIP_ENUM enum : int
#else
#define LLHIP_ENUM enum
#endif
#endif

#ifdef __cplusplus
extern "C" {
/* The callers' atomic_int: only its address crosses the boundary, and this library never dereferences it. */
typedef int llhip_atomic_int;
#else
#include <stdatomic.h>
typedef atomic_int llhip_atomic_int;
#endif

/* kernels.h:15. KERNELS_HIP is this library's one instruction set; the CPU ones are not compiled in. */
typedef LLHIP_ENUM { KERNELS_SCALAR, KERNELS_AVX512, KERNELS_AMX, KERNELS_HIP } KernelIsa;
void kernels_init(void);                 /* kernels.h:16: reads LLAMA_KERNELS (auto|hip) and opens the device */
int kernels_select(KernelIsa isa);       /* kernels.h:17: 1 for KERNELS_HIP, 0 for the CPU instruction sets */
const char *kernels_name(void);          /* kernels.h:18: "hip-gfx950" once initialized, NULL before */

struct Team;
void kernels_set_team(struct Team *team);        /* kernels.h:25: accepted and ignored: the GPU is the team */
void kernels_set_thread_team(struct Team *team); /* kernels.h:28: likewise */
void kernels_backend_init(void);                 /* kernels.h:29: opens the device and the library stream */
void kernels_backend_free(void);                 /* kernels.h:30: synchronizes and releases the device buffers */
const char *kernels_backend_name(void);          /* kernels.h:31: "hip" */
int kernels_avx512_active(void);                 /* kernels.h:37: 0 (no CPU SIMD kernels here) */
int kernels_amx_active(void);                    /* kernels.h:38: 0 */
int kernels_select_amx_auto(void);               /* kernels.h:43: 0; the batched GEMMs run on MFMA regardless */
/* kernels.h:54-55: runs fn over every segment's chunks on the calling thread (one member), in order. */
typedef void (*SegmentFn)(const void *job, int segment, int first, int last);
void kernels_parallel_segments(int count, const int *chunks, SegmentFn fn, const void *job);

/* kernels.h:70-79: FP32 GEMV, W (d rows of n) row-major. _add accumulates, _qkv runs three projections of one input
 * in one launch, _swiglu writes silu(W1 x) * (W3 x). */
void k_matmul(float *out, const float *x, const float *w, int n, int d);
void k_matmul_add(float *out, const float *x, const float *w, int n, int d);
void k_matmul_qkv(float *q, float *k, float *v, const float *x, const float *wq, const float *wk, const float *wv, int n,
                  int dq, int dkv);
void k_matmul_swiglu(float *out, const float *x, const float *w1, const float *w3, int n, int d);

/* kernels.h:82-96. Row stride ld >= n; kind is K_STORE, K_ADD or K_PARTIAL (PARTIAL stores like STORE). The _worker
 * form computes member `worker`'s static share of the rows (rows [d*worker/workers, d*(worker+1)/workers)), so the
 * union over members is the team-level result; `claim` is never used (every split here is static) and `done`, when
 * not NULL, is called once with the share after its rows are stored. */
typedef LLHIP_ENUM { K_STORE, K_ADD, K_PARTIAL, K_SWIGLU } KernelEpilogue;
typedef void (*RowsDoneFn)(void *ctx, int r0, int r1);
void k_matmul_ld(float *out, const float *x, const float *w, size_t ld, int n, int d, int kind);
void k_matmul_ld_worker(float *out, const float *x, const float *w, size_t ld, int n, int d, int kind, int worker,
                        int workers, llhip_atomic_int *claim, RowsDoneFn done, void *done_ctx);
void k_matmul_swiglu_ld(float *out, const float *x, const float *w1, const float *w3, size_t ld, int n, int d);

/* kernels.h:101-109: Q8_0 operands. q holds int8 values in [-127, 127], s one FP32 scale per group of gs values.
 * An input with q == NULL is W8A32 (dequantized weights times the FP32 activations f). */
typedef struct {
  const int8_t *q;
  const float *s;
} K8Weight;
typedef struct {
  const int8_t *q;
  const float *s;
  const float *f;
} K8Input;

/* kernels.h:110: per group, scale = max|x| / 127.0f and q = (int8)roundf(clamp(x / scale, -127, 127)), q = 0 where
 * the scale is 0; bitwise the reference's scalar and AVX-512 quantizers. A non-finite value fails with
 * "nonfinite activation during INT8 quantization" (at the next host-visible point when x is device memory). */
void k_quantize(int8_t *q, float *s, const float *x, int n, int gs);
/* kernels.h:111-115: W8A8 GEMV, out[r] (op)= sum over groups of (float)(int32 dot) * ws[r][g] * xs[g]. The int32
 * group dots are exact; the FP32 sum agrees with the reference within 2e-5 * sum|w x| + 1e-6. */
void k_matmul_q8(float *out, const K8Input *x, K8Weight w, int n, int d, int gs);
void k_matmul_q8_add(float *out, const K8Input *x, K8Weight w, int n, int d, int gs);
void k_matmul_q8_qkv(float *q, float *k, float *v, const K8Input *x, K8Weight wq, K8Weight wk, K8Weight wv, int n,
                     int dq, int dkv, int gs);
void k_matmul_q8_swiglu(float *out, const K8Input *x, K8Weight w1, K8Weight w3, int n, int d, int gs);
/* kernels.h:116-122: shard forms (ld a multiple of gs, ld >= n). */
void k_matmul_q8_ld(float *out, const K8Input *x, const K8Weight *w, size_t ld, int n, int d, int gs, int kind);
void k_matmul_q8_ld_worker(float *out, const K8Input *x, const K8Weight *w, size_t ld, int n, int d, int gs, int kind,
                           int worker, int workers, llhip_atomic_int *claim, RowsDoneFn done, void *done_ctx);
void k_matmul_q8_swiglu_ld(float *out, const K8Input *x, const K8Weight *w1, const K8Weight *w3, size_t ld, int n,
                           int d, int gs);

#ifdef __cplusplus
}
#endif
#endif
