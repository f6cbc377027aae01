/* Prefill policy for the HIP build: drop-in for the reference's include/prefill.h (src/prefill.c), same knobs and the
 * same validation, with the GPU's batch and kernel names. Each declaration cites the one it replaces
 * (LucianCrainic/llama3.x.c file:line). Config and Model repeat the reference's layouts (runtime.h:9-16, 87-97) so the
 * engine's Model is read and written in place. */
#ifndef LLAMA_HIP_PREFILL_H
#define LLAMA_HIP_PREFILL_H

#include <stddef.h>

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
#endif

typedef struct { /* runtime.h:9-16 */
  int dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len;
  int format, max_seq_len, shared, head_dim;
  float norm_eps, rope_theta, rope_factor, rope_low, rope_high;
  int rope_type, rope_original;
  int bos_id, eos_id, eot_id, eom_id;
  char name[128];
} Config;

typedef LLHIP_ENUM { LOGITS_NONE, LOGITS_LAST, LOGITS_ALL } LogitsWanted; /* runtime.h:75 */

typedef struct { /* runtime.h:87-97 */
  Config config;
  void *implementation;
  size_t file_bytes;
  size_t mapped_bytes;
  int max_batch;
  LogitsWanted prefill_logits;
  int prefill_gemm;
  const char *prefill_kernel;
  int prefill_bf16;
} Model;

/* prefill.h:12 / prefill.c:9-24: LLAMA_PRECISION=fp32 (default) or bf16; bf16 on a Q8_0 checkpoint fails. Returns 1
 * for bf16. */
int prefill_precision(int quantized);
/* prefill.h:9-10 / prefill.c:26-66: LLAMA_PREFILL_BATCH (digits only, 1..INT_MAX), LLAMA_PREFILL_GEMM (auto|on|off;
 * auto is on: the MFMA GEMM always runs here) and LLAMA_PREFILL_LOGITS (last|all), validated with the reference's
 * messages. The batch is capped at the context; prefill_kernel names the MFMA kernel that runs ("hip-mfma-int8" for
 * the Q8 engine's W8A8 prefill with gs % 64 == 0, "hip-int8" for other group sizes, "hip-mfma-bf16" in the BF16 mode,
 * "hip-mfma-f32" for FP32). `quantized` tells the two engines apart (the reference's engine.c:87-118 knows it from
 * the executable). */
void prefill_configure_engine(Model *model, int recommended, int quantized);
void prefill_configure(Model *model, int recommended); /* as prefill_configure_engine(model, recommended, 0) */
/* prefill.h:15 / prefill.c:72-83: fails unless 1 <= count <= max_batch, 0 <= pos0 < seq_len, count <= seq_len - pos0,
 * want is NONE, LAST or ALL and every token lies in [0, vocab_size). */
void prefill_validate(const Model *model, const int *tokens, int count, int pos0, LogitsWanted want);
int engine_max_batch(const Model *model); /* runtime.h:110 / prefill.c:68-70 */

/* The batch the GPU takes per prefill pass: the whole prompt up to 2048 rows for W8A8 and BF16, 1024 for FP32 (the
 * reference's D2 values are 256/128 for one CPU socket). */
enum { LLHIP_PREFILL_BATCH_Q8 = 2048, LLHIP_PREFILL_BATCH_BF16 = 2048, LLHIP_PREFILL_BATCH_F32 = 1024 };

#ifdef __cplusplus
}
#endif
#endif
