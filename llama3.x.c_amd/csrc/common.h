// Internal to the HIP library: device state, pointer residency, failure handling and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "llama_hip.h"

namespace llhip {

// ---- failure ----------------------------------------------------------------------------------------------------
// The reference's fail() prints the message and exits (runtime.c:49-63). Here the default does the same; a host that
// has its own fail() installs it with llhip_set_fail_handler, and tests switch to LLHIP_FAIL_RECORD, where the
// failing entry point returns without doing its work. raise() returns false in that mode so callers can `return`.
bool raise(const char *format, ...) __attribute__((format(printf, 1, 2)));
bool check_hip(hipError_t status, const char *what);
#define LLHIP_CHECK(call) ::llhip::check_hip((call), #call)

// ---- device state -----------------------------------------------------------------------------------------------
struct Device {
  bool ready = false;
  int ordinal = 0;
  hipStream_t stream = nullptr;
  int *error_flags = nullptr; // device: [0] non-finite activation seen by a quantizer, [1] non-finite attention score,
                              // [2] an embedding row id outside the table
  int *host_flags = nullptr;  // pinned host copy of the 16 flag words, read back with the synchronization
  int cu_count = 0;
  bool capturing = false;
  void *split_partial = nullptr;  // split-K partial tiles: LLHIP_SPLIT_SLOTS x 256 x 128 floats
  unsigned *split_count = nullptr; // split-K arrivals per tile, zero between launches
};
// Partial tiles of the split-K workspace (one per block of a split launch): 512 x 128 KB = 64 MB of HBM. Launches on
// the library's stream are ordered, so one workspace per device serves them all.
#define LLHIP_SPLIT_SLOTS 512
Device &device();
bool ensure_device(); // opens the device on first use; false (after raise) when none is usable
// Claims bytes of HBM against LLAMA_HBM_BUDGET_GIB before an allocation (false after raise when it does not fit), and
// gives them back after the free.
bool hbm_claim(size_t bytes, const char *what);
void hbm_release(size_t bytes);
// Waits for the stream and turns a device-side error flag into a failure (the reference fails at once; a device
// kernel can only report at the next host-visible point).
bool synchronize_and_check();
// Host memory that is neither device memory nor inside a registered range: written in place by host-side entry points.
bool plain_host_memory(const void *p, size_t bytes);

// ---- pointer residency ------------------------------------------------------------------------------------------
// Every pointer an entry point receives is resolved once per call: device memory is used in place, host memory
// inside a registered range maps to its uploaded copy, and any other host memory is staged through a device arena
// (copied in before the launch, copied out after it, then the call synchronizes).
// A resolved pointer: device memory in place, or an index into the call's staged copies.
struct Ref {
  void *direct = nullptr;
  int staged = -1;
};

// A k_quantize on device buffers is not launched at once: it is recorded, and the next k_matmul_q8* whose input is
// exactly those buffers quantizes in its own prologue (one launch instead of two; block 0 still stores q and s). Any
// other entry point, llhip_synchronize and the end of a graph capture launch a recorded quantization first, so every
// observer sees the reference's order. LLAMA_HIP_FUSE_QUANT=0 turns the deferral off.
// A k_quantize of one device-resident row, recorded so the next GEMV reading (q, s) can quantize in its prologue.
// norm_w set: x is the input of a k_rmsnorm recorded just before (output norm_out, the quantization's own input).
struct PendingQuantize {
  int8_t *q;
  float *s;
  const float *x;
  int n, gs;
  const float *norm_w;
  float *norm_out;
  float norm_eps;
};
// A k_rmsnorm of one device-resident row, recorded so a k_quantize of its output (and the GEMV after it) can take it.
struct PendingNorm {
  float *out;
  const float *x, *w;
  int size;
  float eps;
};
void defer_norm(const PendingNorm &job);
// A single-row k_rope_apply on device memory and the k_kv_store calls of its rotated k (and of v) that follow it,
// recorded so the decode attention over the same cache can rotate, store and attend in one launch.
struct PendingKvStore {
  float *cache;
  const float *src;
  int pos;
  size_t pos_stride, head_base;
};
struct PendingRope {
  float *q, *k;
  const float *table;
  int n_heads, n_kv_heads, head_dim;
  int stores; // 0, 1 (K) or 2 (K then V)
  PendingKvStore store[2];
};
void defer_rope(const PendingRope &job);
// Attaches a single-row cache store to the recorded RoPE (K: src is its k; V: after K); false when it does not fit.
bool attach_kv_store(const PendingKvStore &store, int n_kv_heads, int head_dim);
// Takes the recorded RoPE with both stores when they are exactly this decode attention's inputs.
bool take_pending_rope(const float *q, const float *key_cache, const float *value_cache, int position,
                       size_t pos_stride, size_t head_base, int n_heads, int n_kv_heads, int head_dim, PendingRope *out);
bool quantize_fusion_enabled();
void defer_quantize(const PendingQuantize &job);
bool take_pending_quantize(const int8_t *q, const float *s, int n, int gs, PendingQuantize *out);
bool flush_pending_quantize(); // launches a recorded norm and quantization, if any
bool launch_pending_quantize(const PendingQuantize &job, hipStream_t stream); // its norm, then the quantization

class Call {
 public:
  // keep_pending: the caller may consume a recorded quantization (the Q8 GEMV entry points); every other call
  // launches it first.
  explicit Call(const char *name, bool keep_pending = false);
  ~Call();
  Ref in(const void *p, size_t bytes) { return in2d(p, bytes, bytes, 1); }
  Ref in2d(const void *p, size_t row_bytes, size_t pitch, size_t rows);
  Ref out(void *p, size_t bytes, bool read_too) { return out2d(p, bytes, bytes, 1, read_too); }
  Ref out2d(void *p, size_t row_bytes, size_t pitch, size_t rows, bool read_too);
  // Allocates the arena and performs the staging copies; false when something failed (already raised).
  bool ready();
  // The device address of a resolved pointer (valid after ready()).
  template <class T> T *ptr(const Ref &r) const { return (T *)address(r); }
  // Copies staged outputs back and, if anything was staged, synchronizes. Returns false on failure.
  bool finish();
  bool staged() const { return staged_; }
  bool failed() const { return failed_; }
  hipStream_t stream() const;

 private:
  struct Copy {
    void *host;
    size_t offset, row_bytes, pitch, rows;
    bool to_device, to_host;
  };
  void *address(const Ref &r) const;
  Ref stage(void *host, size_t row_bytes, size_t pitch, size_t rows, bool to_device, bool to_host);
  void *resolve_registered(const void *p, size_t *room = nullptr);
  const char *name_;
  uintptr_t current_mapping_ = 0; // a registered file mapping found current during this call
  Copy copies_[16];
  int ncopies_ = 0;
  size_t arena_used_ = 0;
  bool staged_ = false, failed_ = false;
  bool bounced_ = false; // the copies go through the pinned twin of the arena
};

// ---- kernel launchers (stream-ordered, no synchronization) ------------------------------------------------------
enum Epilogue { EPI_STORE = 0, EPI_ADD = 1, EPI_SWIGLU = 2 };

struct QuantizeJob {
  int8_t *q;
  float *s;
  const float *x;
  size_t ldx; // floats
  int m, n, gs;
};
bool launch_quantize(const QuantizeJob &job, hipStream_t stream);
// RMSNorm then k_quantize of rows of n values in one launch (bitwise k_rmsnorm_rows then k_quantize_rows), for the
// shapes rmsnorm_quantize_fits takes: n <= 8192, n % gs == 0, gs a power of two from 4 to 256; 16-byte aligned x and
// weight, 4-byte aligned q.
bool rmsnorm_quantize_fits(int n, int gs);
bool launch_rmsnorm_quantize(int8_t *q, float *s, const float *x, const float *weight, int rows, int n, float epsilon,
                             int gs, hipStream_t stream);

struct GemvSegment {
  float *out;
  const int8_t *wq;
  const float *ws;
  const int8_t *w3q; // SWIGLU
  const float *w3s;
  int rows;
};
struct GemvJob {
  GemvSegment seg[3];
  int nseg;
  const int8_t *xq; // W8A8 input (xq, xs) or, with xq == nullptr, the W8A32 input xf
  const float *xs;
  const float *xf;
  int n, gs;
  size_t ld; // weight row stride in values
  Epilogue epi;
  int32_t *probe; // optional: exact int32 group dots of segment 0, probe[g * rows + r]
  // Fused quantization: quantize xf in the prologue (the k_quantize rule) and store it to (xq_out, xs_out).
  bool xf_quantize;
  int8_t *xq_out;
  float *xs_out;
  // With xf_quantize and norm_w: xf is RMSNorm's input, normalized (weights norm_w, norm_eps) before the quantization
  // and stored to norm_out (the k_rmsnorm that preceded the k_quantize).
  const float *norm_w;
  float *norm_out;
  float norm_eps;
};
bool set_gemv_shape(int waves_per_row, int blocks_per_cu, int block_waves);
void set_gemm_splits(int splits); // FP32 / BF16 / INT8 GEMM blocks per tile; 0 = chosen from the grid
void set_bf16_tile(int tile);     // BF16 GEMM tile: 0 by grid, 1 256 x 128, 2 256 x 256
void set_q8_tile(int tile);       // INT8 GEMM tile (gs = 64): 0 by grid, 1 256 x 128, 2 256 x 256
void set_q8_scales(int where);    // wide INT8 GEMM scale products: 0 default, 1 VALU, 2 matrix cores
bool gemv_fast_path(const GemvJob &job);
bool launch_q8_gemv(const GemvJob &job, hipStream_t stream);

struct F32GemvSegment {
  float *out;
  const float *w, *w3;
  int rows;
};
struct F32GemvJob {
  F32GemvSegment seg[3];
  int nseg;
  const float *x;
  int n;
  size_t ld;
  Epilogue epi;
};
bool launch_f32_gemv(const F32GemvJob &job, hipStream_t stream);

// ---- the forward around the matmuls (forward.hip) ------------------------------------------------------------------
bool launch_rmsnorm(float *out, const float *x, const float *weight, int rows, int size, float epsilon,
                    hipStream_t stream);
bool launch_rope(float *q, size_t q_stride, float *k, size_t k_stride, const float *table, size_t table_stride,
                 int rows, int n_heads, int n_kv_heads, int head_dim, hipStream_t stream);
bool launch_kv_store(float *cache, const float *src, size_t src_ld, int pos0, int count, int n_kv_heads, int head_dim,
                     size_t pos_stride, size_t head_base, hipStream_t stream);
// rope_rows of q and k, then k and v stored into the caches at pos0.. (and k written back rotated), in one launch
bool launch_rope_kv_rows(float *q, size_t q_stride, float *k, const float *v, size_t kv_stride, const float *table,
                         size_t table_stride, int rows, int n_heads, int n_kv_heads, int head_dim, float *key_cache,
                         float *value_cache, int pos0, size_t pos_stride, size_t head_base, hipStream_t stream);
bool launch_embed_rows(float *out, const int8_t *table, const float *scales, const int *ids, int count, int dim,
                       int gs, int vocab, hipStream_t stream);
bool launch_embed_rows_f32(float *out, const float *table, const int *ids, int count, int dim, int vocab,
                           hipStream_t stream);
// The allocation-free attention's partials (forward.hip): a file-scope device array of kAttentionScratchFloats floats
// per device. attention_scratch_setup finds its device address on `ordinal` (current) once, at device init;
// attention_scratch returns it (nullptr before).
constexpr size_t kAttentionScratchFloats = size_t(4) << 20;
bool attention_scratch_setup(int ordinal);
float *attention_scratch(int ordinal);
// Causal attention of `rows` query rows at positions pos0 .. pos0 + rows - 1 (q and out: rows x n_heads x head_dim);
// position t of KV head g at key / value + t * pos_stride + g * head_base.
struct AttentionJob {
  float *out;
  const float *q, *key, *value;
  int n_heads, n_kv_heads, head_dim, pos0, rows;
  size_t pos_stride, head_base;
  // Decode with a recorded RoPE and cache stores (rows == 1): q and k_new are rotated by table in the kernel, q and
  // k_new written back rotated, and k_new / v_new stored at position pos0 of the caches, which key / value then are.
  float *k_new;
  const float *v_new, *table;
  // floats of `partial` the batched kernel may use when it splits a tile's positions over blocks (0: the
  // attention_partial_floats of the job, which any split fits)
  size_t partial_room = 0;
  // the rows quantized by the k_quantize rule in groups of qgs values (qout rows of n_heads * head_dim bytes, qscale
  // rows of n_heads * head_dim / qgs scales): in the flash kernel's epilogue where it runs a tile unsplit, otherwise
  // from out by a quantize launch after it (out then holds the FP32 rows; in the fused case it is not written)
  int8_t *qout = nullptr;
  float *qscale = nullptr;
  int qgs = 0;
};
bool attention_shape_ok(int n_heads, int n_kv_heads, int head_dim); // kv_mul <= 16, head_dim <= 256
size_t attention_partial_floats(int rows, int n_heads, int head_dim, int last_position);
bool launch_attention(const AttentionJob &job, float *partial, hipStream_t stream);
// The batched kernel takes the job; its partials, when it splits a tile's positions, stay within job.partial_room.
bool attention_uses_flash(const AttentionJob &job);

struct GemmSegmentDev {
  float *c;
  int ldc;
  const void *w, *w3;   // int8 row-major (Q8), fp32 row-major (F32) or packed bf16 (BF16)
  const float *ws, *w3s; // Q8 weight scales
  size_t ldw;            // F32 only: weight row stride in floats
  int n;
  Epilogue epi;
  // Q8 SWIGLU through q8_gemm_swiglu_quantized only: the output quantized by the k_quantize rule in groups of 64
  // (cq [m][n] int8, cs [m][n / 64]) instead of written to c
  int8_t *cq = nullptr;
  float *cs = nullptr;
};
struct GemmQ8Job {
  const int8_t *xq;
  const float *xs;
  int m, k, gs;
  GemmSegmentDev seg[3];
  int nseg;
};
bool q8_gemm_fast_path(const int8_t *xq, int m, int k, int gs); // the pipelined int8-MFMA kernel takes the shape
bool launch_q8_gemm(const GemmQ8Job &job, hipStream_t stream);
// One SWIGLU segment whose output goes out quantized (seg[0].cq / cs, groups of 64): launched, and true, when the
// launcher's choice for the shape is the wide int8 kernel without split K (the epilogue holds whole output groups);
// false, with nothing launched, otherwise (the caller runs the GEMM and k_quantize_rows).
bool launch_q8_gemm_swiglu_quantized(const GemmQ8Job &job, hipStream_t stream);
bool q8_gemm_skinny_path(const int8_t *xq, int m, int k, int gs); // at most 32 rows: stream the weights once
bool launch_q8_gemm_skinny(const GemmQ8Job &job, hipStream_t stream);
bool launch_q8_gemm_generic(const GemmQ8Job &job, hipStream_t stream);
bool launch_s8_vnni_unpack(int8_t *w, const int8_t *packed, int n, int k, hipStream_t stream); // k % 64 == 0
bool launch_q8_group_dots(int32_t *dots, const int8_t *xq, int m, int k, int gs, const int8_t *wq, int n,
                          hipStream_t stream);

struct GemmF32Job {
  const float *a;
  int lda, m, k;
  GemmSegmentDev seg[3];
  int nseg;
  bool bf16; // BF16 mode: seg[].w are packed bf16 (pack_bf16_vnni layout), A is rounded to bf16 on the fly
  unsigned short *panel; // BF16 mode: device panel of m x (K rounded up to 32) for the pipelined kernel, or null
};
bool launch_f32_gemm(const GemmF32Job &job, hipStream_t stream);

} // namespace llhip
