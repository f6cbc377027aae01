/* The llama3.x.c engine on an MI355X (gfx950): the reference's engine entry points (include/runtime.h:98-116) over
 * the device library's kernels. The checkpoint is mapped and uploaded to HBM once; activations and the K/V cache stay
 * in device memory; the forward calls return logits in host memory owned by the model (valid until the next forward).
 * Failures follow the library's mode (exit with "error: <message>" by default, or record and return).
 *
 * One library reads both checkpoint families the reference splits over its two executables (src/engine.c:123-139,
 * src/runtime.c:179-310): Q8_0 (runq: version 3 precision 1, or version 2) and FP32 (run: version 3 precision 0, or
 * the legacy 28-byte header). The path is chosen by the file, so the reference's refusal of the other executable's
 * format does not arise; every other header check and message is the reference's. */
#ifndef LLAMA_HIP_ENGINE_H
#define LLAMA_HIP_ENGINE_H

#include "llama_hip_prefill.h" /* Config, Model (include/runtime.h:9-16, 87-97) */

#ifdef __cplusplus
extern "C" {
#endif

extern const int engine_q8; /* runtime.h:100: 1, as runq exports it (the engine itself takes FP32 files too) */
/* runtime.h:101-102 (src/engine.c:123-159, src/runtime.c:179-310 header checks, src/shards.c:60-99 tensor order):
 * map and upload the checkpoint. context 0 sizes the K/V cache and the positions to min(seq_len, 4096); 0 < context
 * <= seq_len to exactly that; anything else fails with "requested context exceeds checkpoint context". */
void engine_load(Model *model, const char *path);
void engine_load_context(Model *model, const char *path, int context);
/* runtime.h:103 (src/engine.c:170-177, src/tp.c:337-436 with one socket): one decode token at `position`, whose prefix
 * [0, position) was run before; returns vocab_size logits, or NULL when the call failed in record mode. */
float *engine_forward(Model *model, int token, int position);
/* runtime.h:104-109 (src/engine.c:65-81, src/tp.c:528-622 with one socket): count tokens at pos0 (the prefix
 * [0, pos0) run before), 1 <= count <= engine_max_batch. With the batched GEMM on, more than one row (or any row in
 * BF16 mode) runs through the GEMMs and the batched attention; otherwise (one row, W8A32, LLAMA_PREFILL_GEMM=off)
 * the rows run one token at a time, the classifier only for the rows asked for. LAST returns vocab_size logits of the
 * last row, ALL count x vocab_size in row order, NONE returns NULL; the storage belongs to the model and is
 * invalidated by the next forward. */
float *engine_forward_batch(Model *model, const int *tokens, int count, int pos0, LogitsWanted want);
void engine_free(Model *model);   /* runtime.h:114 */
int engine_group_size(void);      /* runtime.h:116: the last loaded checkpoint's group size (0 for FP32) */
/* runtime.h:115 (src/engine.c:191-195) for the last loaded checkpoint: "int8_q8_0", "int8_q8_0_w8a32" (Q8_0 with
 * LLAMA_Q8_ACTIVATIONS=fp32, read by engine_load: int8 or fp32, anything else fails), "fp32", or "bf16_from_fp32"
 * (FP32 with LLAMA_PRECISION=bf16: the batched GEMMs run on BF16 copies of the weights packed at load). */
const char *engine_precision(void);

/* runtime.h:80-86: K/V cache accounting. */
typedef struct {
  size_t reserved_bytes, active_bytes, resident_bytes;
  int node;
  int verified;
  int full;
  size_t pages_queried, pages_wrong_node, pages_missing;
} KvStats;
/* runtime.h:113 (src/tp.c:1147-1152, src/loader.c:369-373 for one socket): reserved = both caches (2 x layers x
 * context x kv_dim floats), active = the first `position` positions of both. The caches are device memory, which has
 * no host NUMA node or pages to query: node is -1 and nothing is verified, as for the reference's heap caches. */
void engine_kv_stats(Model *model, int position, int verify, KvStats *out);

#ifdef __cplusplus
}
#endif
#endif
