/* The Q8_0 engine on an MI355X (gfx950): the reference's engine entry points (include/runtime.h:98-116) for a
 * version-3 INT8 checkpoint, running the decode forward on the device through the library's kernels. The checkpoint
 * is mapped and uploaded to HBM once; activations and the K/V cache stay in device memory; engine_forward returns
 * the logits in host memory owned by the model (valid until the next forward). Failures follow the library's mode
 * (exit with "error: <message>" by default, or record and return). */
#ifndef LLAMA_HIP_ENGINE_H
#define LLAMA_HIP_ENGINE_H

#include "llama_hip_prefill.h" /* Config, Model (include/runtime.h:9-16, 87-97) */

#ifdef __cplusplus
extern "C" {
#endif

extern const int engine_q8; /* runtime.h:100: 1, this engine reads Q8_0 checkpoints */
/* runtime.h:101-102 (src/runtime.c:179-310 header checks, src/shards.c:77-99 tensor order): map and upload the
 * checkpoint; context > 0 and below the model's seq_len sizes the K/V cache (and the positions) to it. */
void engine_load(Model *model, const char *path);
void engine_load_context(Model *model, const char *path, int context);
/* runtime.h:103 (src/tp.c:387-436 with one socket): one decode token at `position`, whose prefix [0, position) was
 * run before; returns vocab_size logits, or NULL when the call failed in record mode. */
float *engine_forward(Model *model, int token, int position);
/* runtime.h:104-109 (src/tp.c:528-622 with one socket): count tokens at pos0 (the prefix [0, pos0) run before),
 * 1 <= count <= engine_max_batch (2048), through the int8 GEMMs and the batched attention. LAST returns vocab_size
 * logits of the last row, ALL count x vocab_size in row order, NONE returns NULL; the storage belongs to the model and
 * is invalidated by the next forward. */
float *engine_forward_batch(Model *model, const int *tokens, int count, int pos0, LogitsWanted want);
void engine_free(Model *model);   /* runtime.h:114 */
int engine_group_size(void);      /* runtime.h:116: the loaded checkpoint's group size */
/* runtime.h:115 (src/engine.c:191-195): "int8_q8_0", or "int8_q8_0_w8a32" when LLAMA_Q8_ACTIVATIONS=fp32 (read by
 * engine_load: int8 or fp32, anything else fails) makes every GEMV multiply the dequantized weights by the FP32
 * activations; that mode runs batches of one row, as the reference's does. */
const char *engine_precision(void);

#ifdef __cplusplus
}
#endif
#endif
