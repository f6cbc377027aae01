/* llama3.x.c matmul hot path on an MI355X (gfx950): the C ABI of libllama3x_hip.so.
 *
 * The reference-named entry points are declared in llama_hip_kernels.h (GEMV), llama_hip_gemm.h (batched GEMM) and
 * llama_hip_prefill.h (prefill policy). This header adds what a GPU needs and the reference has no counterpart for:
 * opening the device, making weights resident in HBM once, the stream the calls are ordered on, graph capture of a
 * decode step, and the failure mode.
 *
 * Residency. Every pointer an entry point receives is resolved per call:
 *   - device memory (hipMalloc, llhip_malloc, a torch CUDA tensor) is used in place; the call is a launch on the
 *     library stream and returns before the GPU finishes (llhip_synchronize waits);
 *   - host memory inside a range given to llhip_register_host resolves to its device copy (weights: upload once);
 *   - any other host memory is copied to a device arena before the launch and back after it, and the call waits,
 *     so it behaves like the reference's synchronous CPU call.
 * The reference's calls are synchronous; with device pointers, ordering is the stream's order, and the host must call
 * llhip_synchronize before reading results or writing inputs through another route.
 *
 * Failures. Preconditions fail as in the reference (fail(): message, then exit(EXIT_FAILURE)). A non-finite
 * activation seen by a device quantizer is reported at the next host-visible point (llhip_synchronize or any staged
 * call). */
#ifndef LLAMA_HIP_H
#define LLAMA_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "llama_hip_gemm.h"
#include "llama_hip_kernels.h"
#include "llama_hip_prefill.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Opens the device (LLAMA_HIP_DEVICE, default 0) and creates the library stream; 0 on success. Every entry point
 * calls it on first use. */
int llhip_init(void);
const char *llhip_device_name(void);
int llhip_device_cu_count(void);
/* The hipStream_t every launch goes to (default priority). */
void *llhip_stream(void);
/* Waits for the stream; then fails if a device quantizer saw a non-finite activation since the last check. */
void llhip_synchronize(void);

/* Uploads [host, host + bytes) to HBM once; pointers inside the range then resolve to the copy. The host bytes must
 * not change afterwards (re-register to refresh). Returns 0, or -1 after a failure. */
int llhip_register_host(const void *host, size_t bytes);
/* LLAMA_HIP_REGISTER_MAPPINGS=1 (read when first needed) registers on its own: the first time an entry point receives
 * an input inside a read-only mapping of a regular file that no executable segment maps (a checkpoint, not a program
 * or a library), the whole mapping is registered as above, so a caller that takes its weight views from a mapped
 * checkpoint needs no call of its own to run on resident weights. Each later call that resolves into such a range
 * first checks that the same place of the same file is still mapped there (one PROCMAP_QUERY on Linux 6.11 and
 * later, a read of /proc/self/maps before); once the caller has unmapped it, the copy is dropped and the addresses
 * mean whatever is mapped there now. The file's bytes must not change while it is mapped. */
int llhip_unregister_host(const void *host);
/* The device address a host address resolves to (NULL when it is not inside a registered range). */
void *llhip_resolve(const void *host);

/* The HBM budget (loader.h:46, src/loader.c:28-56): LLAMA_HBM_BUDGET_GIB (a positive number of GiB; anything else
 * fails with the reference's message), by default the device's whole memory. Every device allocation the library
 * makes or hands out (registered weights, llhip_malloc buffers such as K/V caches, aligned buffers, its staging and
 * workspaces) is claimed against it first, and one beyond it fails with "<what> need N bytes of HBM but
 * LLAMA_HBM_BUDGET_GIB leaves L of B". llhip_hbm_claimed reports the bytes claimed now (no counterpart in the
 * reference, whose count is private to loader.c). */
size_t placement_hbm_budget(void);
size_t llhip_hbm_claimed(void);

/* Device memory owned by the caller, and stream-ordered copies (all on the library stream). */
void *llhip_malloc(size_t bytes);
void llhip_free(void *device);
void llhip_memcpy_h2d(void *device, const void *host, size_t bytes);
void llhip_memcpy_d2h(void *host, const void *device, size_t bytes);
void llhip_memcpy_d2d(void *dst, const void *src, size_t bytes);

/* Graph capture of a sequence of entry-point calls on device-resident pointers (a decode step): begin, make the
 * calls, end. A staged (host-pointer) call inside a capture fails. The returned handle replays with
 * llhip_graph_launch (stream-ordered) and is released with llhip_graph_destroy. */
int llhip_graph_begin(void);
void *llhip_graph_end(void);
int llhip_graph_launch(void *graph);
void llhip_graph_destroy(void *graph);

/* Failure behaviour. The handler (NULL = default) receives the formatted message and is expected not to return,
 * like the reference's fail(). LLHIP_FAIL_RECORD instead keeps the message, and the failing call returns without
 * doing its work (for tests of the error paths). */
typedef void (*LlhipFailFn)(const char *message);
void llhip_set_fail_handler(LlhipFailFn handler);
enum { LLHIP_FAIL_EXIT = 0, LLHIP_FAIL_RECORD = 1 };
void llhip_set_fail_mode(int mode);
const char *llhip_last_error(void); /* "" when none */
void llhip_clear_error(void);

/* Launch shape of the streaming Q8 GEMV: waves per weight row (1, 2, 4 or 8; 0 = by K), resident 8-wave block
 * equivalents per CU of its persistent grid (1..64; 0 = 2) and waves per block (8 or 16; 0 = 16; 16-wave blocks need
 * an even block count per CU, else 8 is used). Results do not depend on it beyond FP32 summation order. For tuning
 * and tests; LLAMA_HIP_GEMV_KSPLIT, LLAMA_HIP_GEMV_BLOCKS_PER_CU and LLAMA_HIP_GEMV_BLOCK_WAVES set the same at
 * start-up. */
void llhip_set_gemv_shape(int waves_per_row, int blocks_per_cu, int block_waves);

/* Blocks per output tile of the prefill GEMMs, FP32, BF16 and INT8 (split K; 0 = chosen from the grid: about one
 * block per CU when the tiles are fewer than the CUs, at least eight K steps per block, at most 512 blocks; INT8
 * splits keep whole scale groups). Partial sums are added in split order, so results depend on it only through FP32
 * summation order, never on timing; INT8 group dots are exact either way. A forced count also sends INT8 calls of at
 * most 32 rows to the tiled kernel instead of the weight-streaming one. For tuning and tests. */
void llhip_set_gemm_splits(int splits);

/* Output tile of the BF16 prefill GEMM: 1 = 256 x 128, 2 = 256 x 256, 0 = by grid (256 x 256 when the grid has at
 * least four 256 x 128 tiles per CU; LLAMA_HIP_BF16_TILE=narrow|wide sets the same at start-up). Results do not depend
 * on it beyond FP32 summation order. For tuning and tests. */
void llhip_set_bf16_tile(int tile);

/* Output tile of the INT8 prefill GEMM with gs = 64: 1 = 256 x 128, 2 = 256 x 256, 0 = by grid (256 x 256 when the
 * grid has at least four 256 x 128 tiles per CU; LLAMA_HIP_Q8_TILE=narrow|wide sets the same at start-up). Other group
 * sizes and the group-dot probe always take 256 x 128. Results do not depend on it beyond FP32 summation order; the
 * int32 group dots are exact either way. For tuning and tests. */
void llhip_set_q8_tile(int tile);

/* Where the 256 x 256 INT8 kernel forms each group's scale products xs[r] * ws[c]: 2 = on the matrix cores (one bf16
 * MFMA over exact bf16 parts of the scales per 64 x 16 outputs, then a convert and an FMA per output; the default),
 * 1 = on the vector unit ((float)dot * ws, then an FMA with xs), 0 = the default (LLAMA_HIP_Q8_SCALES=mfma|valu sets
 * the same at start-up). The two differ in FP32 rounding only; the int32 group dots are the same. For tuning and
 * tests. */
void llhip_set_q8_scales(int where);

/* The int32 probe of the decode GEMV: dots[g * d + r] = the exact int32 dot of group g of input row xq and weight
 * row r, as the streaming GEMV kernel itself forms it before the FP32 rescale (gs % 16 == 0 takes the fast kernel). */
void llhip_q8_gemv_group_dots(int32_t *dots, const int8_t *xq, const float *xs, const int8_t *wq, const float *ws,
                              size_t ld, int n, int d, int gs);

#ifdef __cplusplus
}
#endif
#endif
