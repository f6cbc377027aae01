// Host-side parts of the reference's kernel surface that need no GPU: instruction-set selection and status (for the
// engine and its report), BF16 conversion, the packed weight layouts, aligned workspaces and the CPU-only hooks this
// build answers with "not compiled in". Citations are LucianCrainic/llama3.x.c file:line.
#include <cstdlib>
#include <cstring>

#include "common.h"

using namespace llhip;

namespace {
bool initialized = false;

size_t round_up(size_t v, size_t to) { return (v + to - 1) / to * to; }
} // namespace

extern "C" {

// ---- instruction set and backend (kernels.h:15-55) ---------------------------------------------------------------

void kernels_init(void) {
  const char *request = getenv("LLAMA_KERNELS");
  if (request && *request && strcmp(request, "auto") && strcmp(request, "hip")) {
    raise("LLAMA_KERNELS must be auto or hip in this build (the CPU instruction sets scalar, avx512 and amx are not "
          "compiled in)");
    return;
  }
  if (ensure_device())
    initialized = true;
}

int kernels_select(KernelIsa isa) {
  if (isa != KERNELS_HIP || !ensure_device())
    return 0;
  initialized = true;
  return 1;
}

const char *kernels_name(void) { return initialized ? "hip-gfx950" : nullptr; }

void kernels_set_team(struct Team *team) { (void)team; }
void kernels_set_thread_team(struct Team *team) { (void)team; }
void kernels_backend_init(void) { (void)ensure_device(); }
void kernels_backend_free(void) {
  if (device().ready)
    (void)hipStreamSynchronize(device().stream);
}
const char *kernels_backend_name(void) { return "hip"; }
int kernels_avx512_active(void) { return 0; }
int kernels_amx_active(void) { return 0; }
int kernels_select_amx_auto(void) { return 0; }

void kernels_parallel_segments(int count, const int *chunks, SegmentFn fn, const void *job) {
  for (int s = 0; s < count; s++) // one member: every segment's chunks [0, chunks[s]) in order
    if (chunks[s] > 0)
      fn(job, s, 0, chunks[s]);
}

/* testing.h:27: the hybrid FP32 split is a CPU scheduling choice; the device GEMV has one schedule. */
void k_gemv_force_hybrid(int on) { (void)on; }

// ---- AMX status (gemm.h:46-52) and the tile kernels (gemm.c:611-627's non-AMX build) -----------------------------

const char *gemm_amx_unavailable(void) { return "this build runs the batched GEMMs on the GPU's MFMA units, not AMX"; }
const char *gemm_amx_permission(void) { return "not requested"; }
void gemm_amx_enable(int on) { (void)on; }
int gemm_amx_active(void) { return 0; }
int gemm_amx_emulated(void) { return 0; }
void gemm_amx_thread_release(void) {}

void amx_bf16_tile_gemm(float *c, size_t ldc, const uint16_t *a, size_t lda, const uint16_t *bp, int m, int n, int k) {
  (void)c, (void)ldc, (void)a, (void)lda, (void)bp, (void)m, (void)n, (void)k;
  raise("AMX tile kernels are not compiled into this build");
}

void amx_s8_tile_gemm(int32_t *c, size_t ldc, const int8_t *a, size_t lda, const int8_t *bp, int m, int n, int k) {
  (void)c, (void)ldc, (void)a, (void)lda, (void)bp, (void)m, (void)n, (void)k;
  raise("AMX tile kernels are not compiled into this build");
}

int k_gemm_kc(void) { return 0; } /* one K block (gemm.c:629-636's non-AVX-512 answer) */

// ---- BF16 conversion (gemm.c:332-349) ------------------------------------------------------------------------------

uint16_t bf16_from_f32(float x) {
  uint32_t u;
  memcpy(&u, &x, sizeof(u));
  if ((u & 0x7fffffffu) > 0x7f800000u) // NaN: sign and top payload bits kept, quiet bit set
    return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u); // round to nearest even on the dropped half
  return (uint16_t)(u >> 16);
}

float f32_from_bf16(uint16_t v) {
  uint32_t u = (uint32_t)v << 16;
  float x;
  memcpy(&x, &u, sizeof(x));
  return x;
}

// ---- packed layouts (gemm.c:355-398): a format the reference's callers hand over, kept as it is ---------------------

size_t bf16_vnni_elements(int rows, int cols) { return round_up((size_t)rows, 16) * round_up((size_t)cols, 32); }

size_t s8_vnni_bytes(int rows, int cols) { return round_up((size_t)rows, 16) * round_up((size_t)cols, 64); }

void pack_bf16_vnni_tiles(uint16_t *dst, const float *w, int rows, int cols, size_t ld, int first, int last) {
  const size_t kp = round_up((size_t)cols, 32), pairs = kp / 2;
  for (int t = first; t < last; t++)
    for (size_t p = 0; p < pairs; p++) {
      uint16_t *out = dst + ((size_t)t * pairs + p) * 32;
      for (size_t c = 0; c < 16; c++) {
        const size_t row = (size_t)t * 16 + c;
        for (size_t e = 0; e < 2; e++) {
          const size_t col = 2 * p + e;
          out[c * 2 + e] = row < (size_t)rows && col < (size_t)cols ? bf16_from_f32(w[row * ld + col]) : 0;
        }
      }
    }
}

void pack_bf16_vnni(uint16_t *dst, const float *w, int rows, int cols, size_t ld) {
  pack_bf16_vnni_tiles(dst, w, rows, cols, ld, 0, (rows + 15) / 16);
}

void pack_s8_vnni_tiles(int8_t *dst, const int8_t *w, int rows, int cols, size_t ld, int first, int last) {
  const size_t kp = round_up((size_t)cols, 64), quads = kp / 4;
  for (int t = first; t < last; t++)
    for (size_t q = 0; q < quads; q++) {
      int8_t *out = dst + ((size_t)t * quads + q) * 64;
      for (size_t c = 0; c < 16; c++) {
        const size_t row = (size_t)t * 16 + c;
        for (size_t e = 0; e < 4; e++) {
          const size_t col = 4 * q + e;
          out[c * 4 + e] = row < (size_t)rows && col < (size_t)cols ? w[row * ld + col] : 0;
        }
      }
    }
}

void pack_s8_vnni(int8_t *dst, const int8_t *w, int rows, int cols, size_t ld) {
  pack_s8_vnni_tiles(dst, w, rows, cols, ld, 0, (rows + 15) / 16);
}

// gemm.c:1094-1100: the tile count of a job list must fit an int.
static bool tiles_fit(long long tiles) {
  return tiles <= INT32_MAX || raise("too many weight tiles to pack: %lld", tiles);
}

void pack_bf16_vnni_many(const PackBf16 *jobs, int count) {
  long long tiles = 0;
  for (int i = 0; i < count; i++)
    tiles += (jobs[i].rows + 15) / 16;
  if (!tiles_fit(tiles))
    return;
  for (int i = 0; i < count; i++)
    pack_bf16_vnni(jobs[i].dst, jobs[i].w, jobs[i].rows, jobs[i].cols, jobs[i].ld);
}

void pack_s8_vnni_many(const PackS8 *jobs, int count) {
  long long tiles = 0;
  for (int i = 0; i < count; i++)
    tiles += (jobs[i].rows + 15) / 16;
  if (!tiles_fit(tiles))
    return;
  for (int i = 0; i < count; i++)
    pack_s8_vnni(jobs[i].dst, jobs[i].w, jobs[i].rows, jobs[i].cols, jobs[i].ld);
}

// gemm.c:1103-1115: a job packs a bound ROWS / COLS shard of the matching dtype where it lives.
static bool packable(const Shard *shard, TensorDtype dtype, const char *what) {
  if (!shard || !shard->q || !shard->src || (shard->kind != SHARD_ROWS && shard->kind != SHARD_COLS) ||
      shard->src->dtype != dtype || shard->rows <= 0 || shard->cols <= 0 || shard->ld < (size_t)shard->cols)
    return raise("%s needs a bound ROWS or COLS %s shard", what, dtype == DT_F32 ? "FP32" : "Q8_0");
  return true;
}

PackBf16 pack_bf16_job_from_shard(uint16_t *dst, const Shard *shard) {
  if (!packable(shard, DT_F32, "pack_bf16_job_from_shard"))
    return PackBf16{};
  return PackBf16{dst, (const float *)shard->q, shard->rows, shard->cols, shard->ld};
}

PackS8 pack_s8_job_from_shard(int8_t *dst, const Shard *shard) {
  if (!packable(shard, DT_Q8, "pack_s8_job_from_shard"))
    return PackS8{};
  return PackS8{dst, (const int8_t *)shard->q, shard->rows, shard->cols, shard->ld};
}

// ---- aligned workspace (gemm.c:400-411) ----------------------------------------------------------------------------

// The reference allocates these only for the BF16 GEMM's activation panel (tp.c:920, 1001), which the GPU kernel
// fills and reads: device memory here, zeroed, at least 256-byte aligned (hipMalloc).
void aligned_buffer_alloc(AlignedBuffer *buffer, size_t bytes, MemoryKind kind) {
  (void)kind;
  buffer->base = buffer->data = nullptr;
  buffer->bytes = 0;
  void *p = nullptr;
  const size_t claim = bytes ? bytes : 1;
  if (!ensure_device() || !hbm_claim(claim, "an aligned buffer"))
    return;
  if (!check_hip(hipMalloc(&p, claim), "allocating an aligned buffer") ||
      !check_hip(hipMemset(p, 0, claim), "clearing an aligned buffer")) {
    if (p)
      (void)hipFree(p);
    hbm_release(claim);
    return;
  }
  buffer->base = buffer->data = p;
  buffer->bytes = bytes;
}

void aligned_buffer_free(AlignedBuffer *buffer) {
  if (buffer->base) {
    (void)check_hip(hipFree(buffer->base), "freeing an aligned buffer");
    hbm_release(buffer->bytes ? buffer->bytes : 1);
  }
  buffer->base = buffer->data = nullptr;
  buffer->bytes = 0;
}

} // extern "C"
