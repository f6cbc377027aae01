// The prefill policy of the HIP build (the reference's src/prefill.c and engine.c:87-118): the same knobs, the same
// validation and messages; the batch and kernel names are the GPU's.
#include <cerrno>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "common.h"

using namespace llhip;

extern "C" {

int prefill_precision(int quantized) {
  const char *value = getenv("LLAMA_PRECISION");
  int bf16 = 0;
  if (value && *value) {
    if (!strcmp(value, "bf16"))
      bf16 = 1;
    else if (strcmp(value, "fp32"))
      return raise("LLAMA_PRECISION must be fp32 or bf16"), 0;
  }
  if (bf16 && quantized)
    return raise("LLAMA_PRECISION=bf16 applies to FP32 checkpoints (run); Q8_0 checkpoints keep their int8 semantics "
                 "(runq)"),
           0;
  return bf16;
}

void prefill_configure_engine(Model *model, int recommended, int quantized) {
  const char *batch = getenv("LLAMA_PREFILL_BATCH");
  const char *gemm = getenv("LLAMA_PREFILL_GEMM");
  if (gemm && *gemm && strcmp(gemm, "auto") && strcmp(gemm, "on") && strcmp(gemm, "off"))
    return (void)raise("LLAMA_PREFILL_GEMM must be auto, on or off");
  // auto is on: the batched MFMA GEMM runs on every device this library opens.
  const int gemm_on = !(gemm && !strcmp(gemm, "off"));
  long count = gemm_on ? recommended : 1;
  if (batch && *batch) {
    if (strspn(batch, "0123456789") != strlen(batch))
      return (void)raise("LLAMA_PREFILL_BATCH must be a positive integer <= INT_MAX");
    errno = 0;
    char *end;
    count = strtol(batch, &end, 10);
    if (errno || *end || count < 1 || count > INT_MAX)
      return (void)raise("LLAMA_PREFILL_BATCH must be a positive integer <= INT_MAX");
  }
  const char *logits = getenv("LLAMA_PREFILL_LOGITS");
  if (logits && *logits && strcmp(logits, "last") && strcmp(logits, "all"))
    return (void)raise("LLAMA_PREFILL_LOGITS must be last or all");
  model->max_batch = count < model->config.seq_len ? (int)count : model->config.seq_len;
  model->prefill_gemm = gemm_on && model->max_batch > 1;
  if (model->prefill_bf16) {
    if (gemm && !strcmp(gemm, "off"))
      return (void)raise("LLAMA_PRECISION=bf16 needs the batched GEMM, but LLAMA_PREFILL_GEMM=off disables it");
    if (model->max_batch < 2)
      return (void)raise("LLAMA_PRECISION=bf16 applies to batched prefill: set LLAMA_PREFILL_BATCH to 2 or more");
    model->prefill_gemm = 1;
  }
  model->prefill_logits = logits && !strcmp(logits, "all") ? LOGITS_ALL : LOGITS_LAST;
  if (!model->prefill_gemm)
    model->prefill_kernel = nullptr;
  else if (model->prefill_bf16)
    model->prefill_kernel = "hip-mfma-bf16";
  else if (quantized)
    model->prefill_kernel = "hip-mfma-int8"; // the engine's group size decides MFMA (gs % 64 == 0) or the generic one
  else
    model->prefill_kernel = "hip-mfma-f32";
}

void prefill_configure(Model *model, int recommended) { prefill_configure_engine(model, recommended, 0); }

int engine_max_batch(const Model *model) { return model->max_batch; }

void prefill_validate(const Model *model, const int *tokens, int count, int pos0, LogitsWanted want) {
  // Subtract after checking pos0, so even INT_MAX inputs cannot overflow (prefill.c:73-76).
  if (!tokens || count < 1 || count > model->max_batch || pos0 < 0 || pos0 >= model->config.seq_len ||
      count > model->config.seq_len - pos0)
    return (void)raise("batch input out of range: count=%d position=%d maximum=%d", count, pos0, model->max_batch);
  if (want != LOGITS_NONE && want != LOGITS_LAST && want != LOGITS_ALL)
    return (void)raise("invalid batch logits request: %d", (int)want);
  for (int i = 0; i < count; i++) // every token before any KV entry is written
    if (tokens[i] < 0 || tokens[i] >= model->config.vocab_size)
      return (void)raise("forward input out of range: token=%d position=%d", tokens[i], pos0 + i);
}

} // extern "C"
