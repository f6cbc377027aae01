// The engine's host forward over the device library: engine_load maps a checkpoint, checks its header as the
// reference does, uploads it to HBM once (llhip_register_host) and allocates the activations and the K/V cache in
// device memory; engine_forward runs one decode token in the reference's order (src/tp.c:337-436 with one socket)
// through the library's entry points, so the recorded forms apply (RMSNorm and quantization inside the GEMV, RoPE and
// the cache stores inside attention) and only the logits cross PCIe; engine_forward_batch runs a prompt through the
// batched GEMMs (src/tp.c:528-622) or, where the reference does (src/engine.c:65-81), one token at a time.
//
// Formats (src/runtime.c:179-310, tensor order src/shards.c:60-99):
//   Q8_0, version 3 (256-byte header, precision 1) or version 2 (256-byte header: shared flag byte at 36, group size
//     at 37): FP32 norms first (rms_att[L], rms_ffn[L], rms_final), then each INT8 tensor as its values followed by
//     its group scales, the embedding, per role the layers back to back (wq, wk, wv, wo, w1, w2, w3), and the
//     classifier unless it is tied to the embedding;
//   FP32, version 3 (precision 0, group size 0) or the legacy 28-byte header (seven ints, a negative vocabulary size
//     meaning an untied classifier): the embedding, rms_att[L], wq, wk, wv, wo, rms_ffn[L], w1, w2, w3, rms_final,
//     the legacy file's unused RoPE table (seq_len x head_dim floats), and the classifier unless tied.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "common.h"
#include "llama_hip_engine.h"
#include "llama_hip_forward.h"
#include "llama_hip_gemm.h"

namespace llhip {
namespace {

constexpr uint32_t kMagic = 0x616b3432; // "24ka" read little-endian: the versioned checkpoint tag
constexpr size_t kVersionedHeader = 256, kLegacyHeader = 28;
constexpr int kDefaultContext = 4096;   // src/engine.c:150: the context when none is requested
constexpr int kPackRoles = 7;           // wq, wk, wv, wo, w1, w2, w3 (src/tp.c:25)

// The last checkpoint loaded: engine_group_size and engine_precision report it, as the reference's per-process GS and
// mode do (src/engine.c:17-20, 191-198). Each engine keeps its own mode for its forwards.
int last_group_size = 0;
const char *last_precision = "int8_q8_0";

struct Tensor {
  const void *w = nullptr;   // FP32 values, or the int8 values of a Q8_0 tensor
  const float *s = nullptr;  // the Q8_0 group scales (nullptr for FP32)
  const int8_t *q() const { return (const int8_t *)w; }
  const float *f() const { return (const float *)w; }
  K8Weight k8() const { return K8Weight{q(), s}; }
};

struct Engine {
  int fd = -1;
  unsigned char *map = nullptr;
  size_t bytes = 0;
  bool q8 = true;    // Q8_0 checkpoint (else FP32)
  bool a32 = false;  // Q8_0 with LLAMA_Q8_ACTIVATIONS=fp32 (W8A32)
  bool bf16 = false; // FP32 with LLAMA_PRECISION=bf16: the batched GEMMs on packed BF16 weights
  int gs = 0;        // Q8_0 group size (0 for FP32)
  size_t header = 0; // header bytes before the first tensor
  Config c{};
  // inside the registered mapping (the library resolves them to their device copies)
  const float *rms_att = nullptr, *rms_ffn = nullptr, *rms_final = nullptr;
  Tensor embed, cls;
  std::vector<Tensor> wq, wk, wv, wo, w1, w2, w3;
  // BF16 mode: the packed copies (device memory), layer-major in the roles' order; the classifier's when all-position
  // logits are first asked for (src/tp.c:35, 838-860)
  uint16_t *packed = nullptr, *cls_packed = nullptr;
  std::vector<const uint16_t *> packed_at;
  AlignedBuffer panel{};
  // device memory
  float *x = nullptr, *xb = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *hb = nullptr, *logits = nullptr;
  float *key_cache = nullptr, *value_cache = nullptr, *xs = nullptr, *hs = nullptr;
  // the RoPE table of every position (2 * head_dim floats each), computed at load with the reference's expressions
  float *rope_all = nullptr;
  int8_t *xq = nullptr, *hq = nullptr;
  int *token_dev = nullptr;
  // pinned host memory: a decode token's id on its way in and its logits on the way out, so neither copy waits
  int *token_host = nullptr;
  float *host_logits = nullptr;
  AttentionWork work{};
  // the batched forward's rows (max_batch of each, allocated on its first call)
  int batch_rows = 0;
  float *bx = nullptr, *bxb = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr, *bhb = nullptr, *bxs = nullptr;
  float *bhs = nullptr, *blogits = nullptr;
  int8_t *bxq = nullptr, *bhq = nullptr; // quantized rows of dim (xb) and of hidden_dim (hb) values
  int *btokens = nullptr;
  // a batch's logits on the host: pinned, so the copy of every row's logits (1 GB for 2048 rows of 128256) runs at
  // the link's rate instead of through the runtime's staging of pageable memory; grown on demand
  float *host_batch = nullptr;
  size_t host_batch_floats = 0;
  // every row's logits copy to the host on a stream of their own, piece by piece behind the classifier GEMM
  hipStream_t copy_stream = nullptr;
  hipEvent_t piece_done = nullptr;
};

// Room for `floats` logits in the pinned batch buffer (false after raise when the host cannot pin that much).
bool host_batch_room(Engine *e, size_t floats) {
  if (floats <= e->host_batch_floats)
    return true;
  if (e->host_batch)
    (void)hipHostFree(e->host_batch);
  e->host_batch = nullptr;
  e->host_batch_floats = 0;
  if (hipHostMalloc((void **)&e->host_batch, floats * sizeof(float), hipHostMallocDefault) != hipSuccess) {
    (void)hipGetLastError();
    e->host_batch = nullptr;
    return raise("engine_forward_batch: %zu bytes of pinned host memory for the logits are not available",
                 floats * sizeof(float));
  }
  e->host_batch_floats = floats;
  return true;
}

template <typename T> T read_at(const unsigned char *p, size_t offset) {
  T v;
  memcpy(&v, p + offset, sizeof(T));
  return v;
}

template <typename T> void drop(T *&p) {
  if (p)
    llhip_free((void *)p);
  p = nullptr;
}

void free_batch(Engine *e) {
  drop(e->bx), drop(e->bxb), drop(e->bq), drop(e->bk), drop(e->bv), drop(e->bhb), drop(e->bxs);
  drop(e->bxq), drop(e->bhq), drop(e->bhs), drop(e->btokens), drop(e->blogits);
  if (e->panel.base)
    aligned_buffer_free(&e->panel);
  e->batch_rows = 0;
}

void release(Engine *e) {
  free_batch(e);
  drop(e->x), drop(e->xb), drop(e->q), drop(e->k), drop(e->v), drop(e->hb), drop(e->logits), drop(e->rope_all);
  drop(e->key_cache), drop(e->value_cache), drop(e->xs), drop(e->hs), drop(e->xq), drop(e->hq), drop(e->token_dev);
  if (e->token_host)
    (void)hipHostFree(e->token_host);
  if (e->host_logits)
    (void)hipHostFree(e->host_logits);
  if (e->host_batch)
    (void)hipHostFree(e->host_batch);
  if (e->copy_stream) {
    (void)hipStreamSynchronize(e->copy_stream);
    (void)hipStreamDestroy(e->copy_stream);
  }
  if (e->piece_done)
    (void)hipEventDestroy(e->piece_done);
  drop(e->packed), drop(e->cls_packed);
  if (e->map) {
    (void)llhip_unregister_host(e->map);
    munmap(e->map, e->bytes);
  }
  if (e->fd >= 0)
    close(e->fd);
  delete e;
}

// src/runtime.c:147-170: the reference's checks of the hyperparameters, in its order and with its messages.
bool validate_config(const Config &p, bool quantized, int gs) {
  if (p.dim <= 0 || p.hidden_dim <= 0 || p.n_layers <= 0 || p.n_heads <= 0 || p.n_kv_heads <= 0 ||
      p.vocab_size <= 0 || p.seq_len <= 0)
    return raise("invalid checkpoint dimensions: all seven dimensions must be positive");
  if (p.dim % p.n_heads || p.n_heads % p.n_kv_heads || (p.dim / p.n_heads) % 2)
    return raise("unsupported attention dimensions: dim must be divisible by heads, heads must be divisible by KV "
                 "heads, head size must be even");
  if (!std::isfinite(p.norm_eps) || p.norm_eps <= 0 || !std::isfinite(p.rope_theta) || p.rope_theta <= 1 ||
      p.head_dim != p.dim / p.n_heads || p.max_seq_len != p.seq_len)
    return raise("invalid RMSNorm, RoPE theta, head dimension or context metadata");
  if (p.rope_type != 0 && p.rope_type != 1)
    return raise("unsupported RoPE scaling type %d", p.rope_type);
  if (!std::isfinite(p.rope_factor) || !std::isfinite(p.rope_low) || !std::isfinite(p.rope_high) ||
      p.rope_factor < 1 || p.rope_low <= 0 || p.rope_high <= p.rope_low || p.rope_original <= 0)
    return raise("invalid RoPE scaling metadata");
  if (p.format == 3 && (p.bos_id < 0 || p.bos_id >= p.vocab_size || p.eos_id < 0 || p.eos_id >= p.vocab_size ||
                        p.eot_id < -1 || p.eot_id >= p.vocab_size || p.eom_id < -1 || p.eom_id >= p.vocab_size))
    return raise("invalid special token metadata");
  if (quantized && (gs <= 0 || gs > 131071 || p.dim % gs || p.hidden_dim % gs))
    return raise("unsupported INT8 group size %d: must divide dim and hidden_dim and fit int32 accumulation", gs);
  return true;
}

// src/runtime.c:179-270: the header of any of the four formats into e->c, e->q8, e->gs and e->header.
bool parse_header(Engine *e, const char *path) {
  const unsigned char *h = e->map;
  Config &c = e->c;
  memset(&c, 0, sizeof(c));
  // the defaults of files without the metadata (src/runtime.c:198-207)
  c.norm_eps = 1e-5f;
  c.rope_theta = 500000.0f;
  c.rope_factor = 1;
  c.rope_low = 1;
  c.rope_high = 4;
  c.rope_original = 8192;
  c.bos_id = 128000;
  c.eos_id = 128001;
  c.eot_id = 128009;
  c.eom_id = -1;
  int shared = 0;
  if (read_at<uint32_t>(h, 0) == kMagic) {
    if (e->bytes < kVersionedHeader)
      return raise("truncated versioned checkpoint header");
    e->header = kVersionedHeader;
    const int version = read_at<int>(h, 4);
    if (version == 3) {
      const int precision = read_at<int>(h, 36);
      if (precision < 0 || precision > 1)
        return raise("unsupported checkpoint precision %d", precision);
      e->q8 = precision == 1;
      memcpy(&c, h + 8, 28); // dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len
      shared = read_at<int>(h, 40);
      e->gs = read_at<int>(h, 44);
      c.norm_eps = read_at<float>(h, 48);
      c.rope_theta = read_at<float>(h, 52);
      c.rope_type = read_at<int>(h, 56);
      c.rope_factor = read_at<float>(h, 60);
      c.rope_low = read_at<float>(h, 64);
      c.rope_high = read_at<float>(h, 68);
      c.rope_original = read_at<int>(h, 72);
      c.max_seq_len = read_at<int>(h, 76);
      c.head_dim = read_at<int>(h, 80);
      c.bos_id = read_at<int>(h, 84);
      c.eos_id = read_at<int>(h, 88);
      c.eot_id = read_at<int>(h, 92);
      c.eom_id = read_at<int>(h, 96);
      memcpy(c.name, h + 100, 128);
      if (!memchr(c.name, 0, 128))
        return raise("unterminated model name");
      for (size_t i = 228; i < kVersionedHeader; i++)
        if (h[i])
          return raise("unsupported nonzero reserved checkpoint metadata");
      if (!e->q8 && e->gs != 0)
        return raise("FP32 checkpoint must have group size zero");
    } else if (version == 2) { // an INT8 format only
      e->q8 = true;
      memcpy(&c, h + 8, 28);
      shared = h[36];
      e->gs = read_at<int>(h, 37);
    } else {
      return raise("unsupported checkpoint version %d for this executable", version);
    }
    c.format = version;
    if (shared < 0 || shared > 1)
      return raise("invalid classifier flag in '%s'", path);
  } else { // the legacy FP32 header: seven ints, the sign of the vocabulary size tells the classifier apart
    e->q8 = false;
    e->gs = 0;
    e->header = kLegacyHeader;
    memcpy(&c, h, 28);
    if (c.vocab_size == INT_MIN)
      return raise("invalid vocabulary size in '%s'", path);
    shared = c.vocab_size > 0;
    c.vocab_size = std::abs(c.vocab_size);
  }
  c.shared = shared;
  if (c.format != 3) {
    c.max_seq_len = c.seq_len;
    c.head_dim = c.n_heads > 0 ? c.dim / c.n_heads : 0;
  }
  return validate_config(c, e->q8, e->gs);
}

// Walks the tensors in file order (src/runtime.c:271-296 sizes them); false (after raise) when the file is not their
// size. The tensor sizes are bounded by the validated dimensions (each below 2^31), so the products fit size_t.
bool place_tensors(Engine *e, const char *path) {
  const Config &c = e->c;
  const size_t d = c.dim, hd = c.hidden_dim, kv = (size_t)c.head_dim * c.n_kv_heads, L = c.n_layers;
  const size_t vocab = c.vocab_size;
  size_t at = e->header;
  bool aligned = true;
  auto floats = [&](size_t count) {
    const float *p = (const float *)(e->map + (at <= e->bytes ? at : 0));
    at += count * sizeof(float);
    return p;
  };
  auto tensor = [&](size_t count) {
    Tensor t;
    if (!e->q8) {
      t.w = floats(count);
      return t;
    }
    if (count % (size_t)e->gs || count % sizeof(float)) // src/runtime.c:172-177
      aligned = false;
    t.w = e->map + (at <= e->bytes ? at : 0);
    at += count;
    t.s = (const float *)(e->map + (at <= e->bytes ? at : 0));
    at += count / e->gs * sizeof(float);
    return t;
  };
  auto layers = [&](std::vector<Tensor> &v, size_t count) {
    v.resize(L);
    for (size_t l = 0; l < L; l++)
      v[l] = tensor(count);
  };
  if (e->q8) {
    e->rms_att = floats(L * d);
    e->rms_ffn = floats(L * d);
    e->rms_final = floats(d);
    e->embed = tensor(vocab * d);
    layers(e->wq, d * d);
    layers(e->wk, kv * d);
    layers(e->wv, kv * d);
    layers(e->wo, d * d);
    layers(e->w1, hd * d);
    layers(e->w2, d * hd);
    layers(e->w3, hd * d);
  } else {
    e->embed = tensor(vocab * d);
    e->rms_att = floats(L * d);
    layers(e->wq, d * d);
    layers(e->wk, kv * d);
    layers(e->wv, kv * d);
    layers(e->wo, d * d);
    e->rms_ffn = floats(L * d);
    layers(e->w1, hd * d);
    layers(e->w2, d * hd);
    layers(e->w3, hd * d);
    e->rms_final = floats(d);
    if (c.format == 0)
      (void)floats((size_t)c.seq_len * c.head_dim); // the legacy RoPE table, unused
  }
  e->cls = c.shared ? e->embed : tensor(vocab * d);
  if (!aligned)
    return raise("unsupported INT8 tensor alignment/group size: the tensors of a %dx%d model in groups of %d", c.dim,
                 c.hidden_dim, e->gs);
  if (at > e->bytes)
    return raise("truncated checkpoint '%s': need %zu bytes, found %zu", path, at, e->bytes);
  if (c.format == 3 && at != e->bytes)
    return raise("version 3 checkpoint has unexpected trailing bytes");
  // an older format may carry trailing bytes (the reference logs a warning and reads on)
  return true;
}

template <typename T> bool device_array(T **p, size_t count) {
  *p = (T *)llhip_malloc(count * sizeof(T));
  return *p != nullptr;
}

template <typename T> bool pinned(T **p, size_t count) {
  if (hipHostMalloc((void **)p, count * sizeof(T), hipHostMallocDefault) == hipSuccess)
    return true;
  (void)hipGetLastError();
  *p = nullptr;
  return raise("engine: %zu bytes of pinned host memory could not be allocated", count * sizeof(T));
}

// The RoPE table rows of positions 0 .. seq_len - 1 (k_rope_table on the host: the reference's expressions and C
// library, so each row is bitwise the one it makes per token), uploaded once; a token or a batch takes its rows in
// place.
bool rope_tables(Engine *e) {
  const size_t row = 2 * (size_t)e->c.head_dim;
  std::vector<float> host(row * e->c.seq_len);
  for (int pos = 0; pos < e->c.seq_len; pos++)
    k_rope_table(&e->c, pos, host.data() + (size_t)pos * row);
  llhip_memcpy_h2d(e->rope_all, host.data(), host.size() * sizeof(float));
  return llhip_last_error()[0] == 0;
}

bool allocate(Engine *e) {
  const Config &c = e->c;
  const size_t d = c.dim, kv = (size_t)c.head_dim * c.n_kv_heads, h = c.hidden_dim;
  const size_t cache = (size_t)c.n_layers * c.seq_len * kv;
  const size_t groups = e->q8 ? (size_t)e->gs : 1;
  return device_array(&e->x, d) && device_array(&e->xb, d) && device_array(&e->q, d) && device_array(&e->k, kv) &&
         device_array(&e->v, kv) && device_array(&e->hb, h) && device_array(&e->logits, (size_t)c.vocab_size) &&
         device_array(&e->rope_all, 2 * (size_t)c.head_dim * c.seq_len) && device_array(&e->key_cache, cache) &&
         device_array(&e->value_cache, cache) && device_array(&e->xq, d) && device_array(&e->xs, d / groups) &&
         device_array(&e->hq, h) && device_array(&e->hs, h / groups) && device_array(&e->token_dev, 1) &&
         pinned(&e->token_host, 1) && pinned(&e->host_logits, (size_t)c.vocab_size) && rope_tables(e);
}

// BF16 mode (src/tp.c:805-830): every layer's seven matrices packed once into the BF16 layout the GEMM reads
// (pack_bf16_vnni, host side), uploaded to one device allocation.
bool pack_weights(Engine *e) {
  const Config &c = e->c;
  const int d = c.dim, h = c.hidden_dim, kv = c.head_dim * c.n_kv_heads;
  const int rows[kPackRoles] = {d, kv, kv, d, h, d, h}, cols[kPackRoles] = {d, d, d, d, d, h, d};
  const std::vector<Tensor> *roles[kPackRoles] = {&e->wq, &e->wk, &e->wv, &e->wo, &e->w1, &e->w2, &e->w3};
  size_t per_layer = 0;
  for (int i = 0; i < kPackRoles; i++)
    per_layer += bf16_vnni_elements(rows[i], cols[i]);
  if (!device_array(&e->packed, per_layer * c.n_layers))
    return false;
  std::vector<uint16_t> host(per_layer);
  e->packed_at.resize((size_t)c.n_layers * kPackRoles);
  for (int l = 0; l < c.n_layers; l++) {
    size_t at = 0;
    for (int i = 0; i < kPackRoles; i++) {
      pack_bf16_vnni(host.data() + at, (*roles[i])[l].f(), rows[i], cols[i], (size_t)cols[i]);
      e->packed_at[(size_t)l * kPackRoles + i] = e->packed + (size_t)l * per_layer + at;
      at += bf16_vnni_elements(rows[i], cols[i]);
    }
    llhip_memcpy_h2d(e->packed + (size_t)l * per_layer, host.data(), per_layer * sizeof(uint16_t));
  }
  return llhip_last_error()[0] == 0;
}

Engine *open_engine(Model *model, const char *path, int context, bool a32) {
  Engine *e = new Engine();
  e->fd = open(path, O_RDONLY);
  if (e->fd < 0) {
    raise("cannot open checkpoint '%s': %s", path, strerror(errno));
    return release(e), nullptr;
  }
  struct stat st;
  if (fstat(e->fd, &st) || !S_ISREG(st.st_mode) || st.st_size < (off_t)kLegacyHeader) {
    raise("invalid/truncated checkpoint '%s': expected a regular file with complete header", path);
    return release(e), nullptr;
  }
  e->bytes = (size_t)st.st_size;
  void *m = mmap(nullptr, e->bytes, PROT_READ, MAP_PRIVATE, e->fd, 0);
  if (m == MAP_FAILED) {
    raise("cannot map checkpoint '%s' (%zu bytes): %s", path, e->bytes, strerror(errno));
    return release(e), nullptr;
  }
  e->map = (unsigned char *)m;
  if (!parse_header(e, path) || !place_tensors(e, path)) {
    munmap(e->map, e->bytes);
    e->map = nullptr;
    return release(e), nullptr;
  }
  e->a32 = e->q8 && a32;
  // src/engine.c:145-150: the context requested, else the checkpoint's up to 4096 positions
  if (context < 0 || context > e->c.seq_len) {
    raise("requested context exceeds checkpoint context");
    munmap(e->map, e->bytes);
    e->map = nullptr;
    return release(e), nullptr;
  }
  e->c.seq_len = context ? context : (e->c.seq_len < kDefaultContext ? e->c.seq_len : kDefaultContext);
  model->config = e->c;
  // src/engine.c:83-118: the prefill policy of each format
  if (e->q8) {
    prefill_precision(1); // LLAMA_PRECISION=bf16 is an error for Q8_0
    if (llhip_last_error()[0])
      return munmap(e->map, e->bytes), e->map = nullptr, release(e), nullptr;
    prefill_configure_engine(model, e->a32 ? 1 : LLHIP_PREFILL_BATCH_Q8, 1);
    if (e->a32) {
      model->prefill_gemm = 0;
      model->prefill_kernel = nullptr;
    }
  } else {
    model->prefill_bf16 = prefill_precision(0);
    if (!llhip_last_error()[0])
      prefill_configure_engine(model, model->prefill_bf16 ? LLHIP_PREFILL_BATCH_BF16 : LLHIP_PREFILL_BATCH_F32, 0);
    e->bf16 = model->prefill_bf16 != 0;
  }
  if (llhip_last_error()[0]) {
    munmap(e->map, e->bytes);
    e->map = nullptr;
    return release(e), nullptr;
  }
  kernels_init(); // src/engine.c:127-128 (LLAMA_KERNELS, and the device opens), once the file has passed its checks
  if (llhip_last_error()[0] || llhip_register_host(e->map, e->bytes) != 0) {
    munmap(e->map, e->bytes);
    e->map = nullptr;
    return release(e), nullptr;
  }
  if (!allocate(e) || (e->bf16 && !pack_weights(e)))
    return release(e), nullptr;
  k_attention_init(&e->work, e->c.n_heads, e->c.n_kv_heads, e->c.head_dim, e->c.seq_len);
  return e;
}

// One decode token (src/tp.c:337-436 with one socket). Q8_0: the embedding row, per layer RMSNorm, quantize, QKV,
// RoPE, the K/V cache (head-major: staged rows then k_kv_store; rows layout: written in place), attention, quantize,
// Wo + residual, RMSNorm, quantize, W1/W3 SwiGLU, quantize, W2 + residual; then the final RMSNorm in place, quantize
// and the classifier. W8A32 hands the FP32 rows to the GEMVs instead of quantizing; FP32 runs the FP32 GEMVs. The
// classifier runs only when the logits are wanted (src/engine.c:75-77); they land in e->host_logits.
bool forward(Engine *e, int token, int pos, bool want_logits) {
  const Config &c = e->c;
  const int d = c.dim, hidden = c.hidden_dim, hd = c.head_dim, gs = e->gs, nh = c.n_heads, nkv = c.n_kv_heads;
  const size_t kvl = (size_t)hd * nkv;
  // the id goes in through pinned memory on the library's stream, behind the previous token's work (which ended
  // with a synchronization on every path, so the pinned word is free again)
  auto fail_after_wait = [](const char *message) {
    (void)hipStreamSynchronize(device().stream); // the queued copies are done with the pinned buffers
    (void)hipGetLastError();
    return raise("%s", message);
  };
  *e->token_host = token;
  if (!flush_pending_quantize() ||
      hipMemcpyAsync(e->token_dev, e->token_host, sizeof(int), hipMemcpyHostToDevice, device().stream) != hipSuccess)
    return fail_after_wait("engine_forward: copying the token id to the device failed");
  if (e->q8)
    k_embed_q8_rows(e->x, e->embed.q(), e->embed.s, e->token_dev, 1, d, gs, c.vocab_size);
  else
    k_embed_f32_rows(e->x, e->embed.f(), e->token_dev, 1, d, c.vocab_size);
  const float *rope = e->rope_all + (size_t)pos * 2 * hd;
  const bool head = kernels_kv_layout_head() != 0;
  // W8A8 quantizes each GEMV input (q8_input, src/tp.c:380-385); W8A32 hands the FP32 rows over instead
  const bool a32 = e->a32;
  const K8Input in_d = a32 ? K8Input{nullptr, nullptr, e->xb} : K8Input{e->xq, e->xs, nullptr};
  const K8Input in_h = a32 ? K8Input{nullptr, nullptr, e->hb} : K8Input{e->hq, e->hs, nullptr};
  const K8Input in_x = a32 ? K8Input{nullptr, nullptr, e->x} : in_d;
  auto quantize = [&](int8_t *q, float *s, const float *x, int n) {
    if (e->q8 && !a32)
      k_quantize(q, s, x, n, gs);
  };
  for (int l = 0; l < c.n_layers; l++) {
    const size_t layer = (size_t)l * c.seq_len * kvl;
    float *kc = e->key_cache + layer, *vc = e->value_cache + layer;
    float *k = head ? e->k : kc + (size_t)pos * kvl, *v = head ? e->v : vc + (size_t)pos * kvl;
    k_rmsnorm(e->xb, e->x, e->rms_att + (size_t)l * d, d, c.norm_eps);
    quantize(e->xq, e->xs, e->xb, d);
    if (e->q8)
      k_matmul_q8_qkv(e->q, k, v, &in_d, e->wq[l].k8(), e->wk[l].k8(), e->wv[l].k8(), d, d, (int)kvl, gs);
    else
      k_matmul_qkv(e->q, k, v, e->xb, e->wq[l].f(), e->wk[l].f(), e->wv[l].f(), d, d, (int)kvl);
    k_rope_apply(e->q, k, rope, nh, nkv, hd);
    if (head) {
      k_kv_store(kc, k, kvl, pos, 1, nkv, hd, c.seq_len);
      k_kv_store(vc, v, kvl, pos, 1, nkv, hd, c.seq_len);
    }
    k_attention_kv(e->xb, e->q, kc, vc, nullptr, &e->work, nh, nkv, hd, c.seq_len, pos);
    quantize(e->xq, e->xs, e->xb, d);
    if (e->q8)
      k_matmul_q8_add(e->x, &in_d, e->wo[l].k8(), d, d, gs);
    else
      k_matmul_add(e->x, e->xb, e->wo[l].f(), d, d);
    k_rmsnorm(e->xb, e->x, e->rms_ffn + (size_t)l * d, d, c.norm_eps);
    quantize(e->xq, e->xs, e->xb, d);
    if (e->q8)
      k_matmul_q8_swiglu(e->hb, &in_d, e->w1[l].k8(), e->w3[l].k8(), d, hidden, gs);
    else
      k_matmul_swiglu(e->hb, e->xb, e->w1[l].f(), e->w3[l].f(), d, hidden);
    quantize(e->hq, e->hs, e->hb, hidden);
    if (e->q8)
      k_matmul_q8_add(e->x, &in_h, e->w2[l].k8(), hidden, d, gs);
    else
      k_matmul_add(e->x, e->hb, e->w2[l].f(), hidden, d);
  }
  if (want_logits) {
    k_rmsnorm(e->x, e->x, e->rms_final, d, c.norm_eps);
    quantize(e->xq, e->xs, e->x, d);
    if (e->q8)
      k_matmul_q8(e->logits, &in_x, e->cls.k8(), d, c.vocab_size, gs);
    else
      k_matmul(e->logits, e->x, e->cls.f(), d, c.vocab_size);
    if (!flush_pending_quantize() ||
        hipMemcpyAsync(e->host_logits, e->logits, (size_t)c.vocab_size * sizeof(float), hipMemcpyDeviceToHost,
                       device().stream) != hipSuccess)
      return fail_after_wait("engine_forward: copying the logits to the host failed");
  }
  llhip_synchronize(); // the logits have landed; reports a non-finite activation or score of this token
  return llhip_last_error()[0] == 0;
}

// The batched forward's rows, max_batch of each, on its first call; all or nothing.
bool allocate_batch(Engine *e, int rows) {
  const Config &c = e->c;
  const size_t m = rows, d = c.dim, kv = (size_t)c.head_dim * c.n_kv_heads, h = c.hidden_dim;
  const size_t groups = e->q8 ? (size_t)e->gs : 1;
  const bool ok = device_array(&e->bx, m * d) && device_array(&e->bxb, m * d) && device_array(&e->bq, m * d) &&
                  device_array(&e->bk, m * kv) && device_array(&e->bv, m * kv) && device_array(&e->bhb, m * h) &&
                  device_array(&e->bxq, e->q8 ? m * d : 1) && device_array(&e->bxs, e->q8 ? m * d / groups : 1) &&
                  device_array(&e->bhq, e->q8 ? m * h : 1) && device_array(&e->bhs, e->q8 ? m * h / groups : 1) &&
                  device_array(&e->btokens, m);
  if (ok && e->bf16) {
    aligned_buffer_alloc(&e->panel, k_gemm_bf16_panel_bytes(rows, c.dim > c.hidden_dim ? c.dim : c.hidden_dim),
                         MEM_ACTIVATION);
    if (!e->panel.base) {
      free_batch(e);
      return false;
    }
  }
  if (!ok) {
    free_batch(e); // nothing stays claimed, and the next call tries again
    return false;
  }
  e->batch_rows = rows;
  return true;
}

// One product on FP32 activations (src/tp.c:475-490): the FP32 GEMM, or in BF16 mode the same segments on the packed
// copies of layer l's matrices `index` (and `index3` for the SwiGLU pair).
void gemm_f32_or_bf16(Engine *e, const float *a, int lda, int m, int k, const GemmSegment *seg, int count, int l,
                      const int *index, int index3) {
  if (!e->bf16) {
    k_gemm_f32(a, lda, m, k, seg, count);
    return;
  }
  GemmBf16Segment b[GEMM_MAX_SEGMENTS];
  for (int i = 0; i < count; i++)
    b[i] = GemmBf16Segment{seg[i].c, seg[i].ldc, e->packed_at[(size_t)l * kPackRoles + index[i]],
                           index3 >= 0 ? e->packed_at[(size_t)l * kPackRoles + index3] : nullptr, seg[i].n,
                           seg[i].kind};
  k_gemm_bf16(a, lda, m, k, b, count, &e->panel);
}

// Every row's logits for Q8_0 (src/tp.c:610-618 runs the classifier GEMV row by row): the classifier GEMM over pieces
// of kLogitsPiece rows, each piece's logits copied into the pinned host buffer on the engine's copy stream (a DMA
// engine, not the CUs) while the next piece computes, so the copy at the link's rate waits only for the first piece.
// Every piece has at least kLogitsPiece rows, the classifier's 128256 columns make far more tiles than CUs (no split
// K), and each row's sums do not depend on the other rows, so the logits are bit for bit those of one GEMM over all
// rows; a batch of fewer than 2 * kLogitsPiece rows is one piece. The rows' RMSNorm and quantization are in bxq / bxs.
// LLAMA_HIP_LOGITS_PIECE (read per call) sets the piece's rows (at least 64), 0 one GEMM over all rows.
constexpr int kLogitsPiece = 256;
int logits_piece() {
  const char *env = getenv("LLAMA_HIP_LOGITS_PIECE");
  if (!env || !*env)
    return kLogitsPiece;
  const int v = atoi(env);
  return v <= 0 ? INT_MAX / 2 : v < 64 ? 64 : v;
}

bool logits_all_q8(Engine *e, int count) {
  const Config &c = e->c;
  const int d = c.dim, gs = e->gs;
  const size_t vocab = c.vocab_size;
  if (!host_batch_room(e, (size_t)count * vocab))
    return false;
  if (!e->copy_stream && hipStreamCreateWithFlags(&e->copy_stream, hipStreamNonBlocking) != hipSuccess) {
    (void)hipGetLastError();
    e->copy_stream = nullptr;
    return raise("engine_forward_batch: no stream for the logits copy");
  }
  if (!e->piece_done && hipEventCreateWithFlags(&e->piece_done, hipEventDisableTiming) != hipSuccess) {
    (void)hipGetLastError();
    e->piece_done = nullptr;
    return raise("engine_forward_batch: no event for the logits copy");
  }
  bool copied = true;
  const int piece = logits_piece();
  for (int r0 = 0; r0 < count;) {
    const int n = count - r0 < 2 * piece ? count - r0 : piece;
    const GemmQ8Segment seg{e->blogits + (size_t)r0 * vocab, c.vocab_size, e->cls.k8(), K8Weight{}, nullptr, nullptr,
                            c.vocab_size, GEMM_STORE};
    k_gemm_q8(e->bxq + (size_t)r0 * d, e->bxs + (size_t)r0 * (d / gs), n, d, gs, &seg, 1);
    if (llhip_last_error()[0])
      break;
    if (hipEventRecord(e->piece_done, device().stream) != hipSuccess ||
        hipStreamWaitEvent(e->copy_stream, e->piece_done, 0) != hipSuccess ||
        hipMemcpyAsync(e->host_batch + (size_t)r0 * vocab, e->blogits + (size_t)r0 * vocab,
                       (size_t)n * vocab * sizeof(float), hipMemcpyDeviceToHost, e->copy_stream) != hipSuccess) {
      copied = false;
      break;
    }
    r0 += n;
  }
  // the copies queued so far end before the buffers are reused or the call returns, on failure too
  if (hipStreamSynchronize(e->copy_stream) != hipSuccess)
    copied = false;
  if (!copied) {
    (void)hipGetLastError();
    if (!llhip_last_error()[0])
      raise("engine_forward_batch: copying the logits to the host failed");
    return false;
  }
  return !llhip_last_error()[0];
}

// count tokens at pos0 .. pos0 + count - 1 through the GEMMs (src/tp.c:528-622 with one socket): the embedding rows
// and RoPE tables, per layer RMSNorm of the rows, (quantize,) the QKV GEMM, RoPE, the cache rows, batched causal
// attention, (quantize,) Wo + residual, RMSNorm, (quantize,) W1/W3 SwiGLU, (quantize,) W2 + residual; then the final
// RMSNorm and classifier of the last row (LAST) or of every row (ALL; in BF16 mode one BF16 GEMM on the packed
// classifier).
float *forward_rows(Model *model, Engine *e, const int *tokens, int count, int pos0, LogitsWanted want) {
  const Config &c = e->c;
  const int d = c.dim, hidden = c.hidden_dim, hd = c.head_dim, gs = e->gs, nh = c.n_heads, nkv = c.n_kv_heads;
  const int kvl = hd * nkv;
  if (!e->batch_rows && !allocate_batch(e, model->max_batch))
    return nullptr;
  const float *brope = e->rope_all + (size_t)pos0 * 2 * hd; // rows pos0 .. pos0 + count - 1
  llhip_memcpy_h2d(e->btokens, tokens, (size_t)count * sizeof(int));
  if (e->q8)
    k_embed_q8_rows(e->bx, e->embed.q(), e->embed.s, e->btokens, count, d, gs, c.vocab_size);
  else
    k_embed_f32_rows(e->bx, e->embed.f(), e->btokens, count, d, c.vocab_size);
  const bool head = kernels_kv_layout_head() != 0;
  static const int kQkv[3] = {0, 1, 2}, kWo[1] = {3}, kW1[1] = {4}, kW2[1] = {5};
  // RMSNorm of the rows into the GEMM's input: for Q8_0 the normalized rows quantized in the same launch where the
  // shape allows (bitwise k_rmsnorm_rows then k_quantize_rows), the FP32 rows otherwise
  const bool fused_norm = e->q8 && rmsnorm_quantize_fits(d, gs);
  auto norm_rows = [&](const float *w) {
    if (fused_norm) {
      llhip_rmsnorm_quantize_rows(e->bxq, e->bxs, e->bx, w, count, d, c.norm_eps, gs);
      return;
    }
    k_rmsnorm_rows(e->bxb, e->bx, w, count, d, c.norm_eps);
    if (e->q8)
      k_quantize_rows(e->bxq, e->bxs, e->bxb, d, count, d, gs);
  };
  for (int l = 0; l < c.n_layers; l++) {
    const size_t layer = (size_t)l * c.seq_len * kvl;
    float *kc = e->key_cache + layer, *vc = e->value_cache + layer;
    float *kd = head ? e->bk : kc + (size_t)pos0 * kvl, *vd = head ? e->bv : vc + (size_t)pos0 * kvl;
    norm_rows(e->rms_att + (size_t)l * d);
    if (e->q8) {
      const GemmQ8Segment qkv[3] = {
          {e->bq, d, e->wq[l].k8(), K8Weight{}, nullptr, nullptr, d, GEMM_STORE},
          {kd, kvl, e->wk[l].k8(), K8Weight{}, nullptr, nullptr, kvl, GEMM_STORE},
          {vd, kvl, e->wv[l].k8(), K8Weight{}, nullptr, nullptr, kvl, GEMM_STORE}};
      k_gemm_q8(e->bxq, e->bxs, count, d, gs, qkv, 3);
    } else {
      const GemmSegment qkv[3] = {{e->bq, d, e->wq[l].f(), nullptr, (size_t)d, d, GEMM_STORE},
                                  {kd, kvl, e->wk[l].f(), nullptr, (size_t)d, kvl, GEMM_STORE},
                                  {vd, kvl, e->wv[l].f(), nullptr, (size_t)d, kvl, GEMM_STORE}};
      gemm_f32_or_bf16(e, e->bxb, d, count, d, qkv, 3, l, kQkv, -1);
    }
    if (head && hd % 4 == 0) { // RoPE and both cache stores in one launch (bitwise the three calls below)
      llhip_rope_kv_store_rows(e->bq, d, kd, vd, kvl, brope, 2 * (size_t)hd, count, nh, nkv, hd, kc, vc, pos0,
                               c.seq_len);
    } else { // in the rows layout the QKV GEMM wrote k and v into the cache rows themselves
      k_rope_apply_rows(e->bq, d, kd, kvl, brope, 2 * (size_t)hd, count, nh, nkv, hd);
      if (head) {
        k_kv_store(kc, kd, kvl, pos0, count, nkv, hd, c.seq_len);
        k_kv_store(vc, vd, kvl, pos0, count, nkv, hd, c.seq_len);
      }
    }
    // for Q8_0 the attention rows quantized in the batched kernel's epilogue where the group size allows (bitwise
    // k_attention_batch_kv then k_quantize_rows)
    if (e->q8 && (gs == 16 || gs == 32 || gs == 64 || gs == 128) && hd % gs == 0)
      llhip_attention_batch_quantize(e->bxq, e->bxs, gs, e->bxb, e->bq, kc, vc, nh, nkv, hd, c.seq_len, pos0, count);
    else
      k_attention_batch_kv(e->bxb, e->bq, kc, vc, nullptr, &e->work, nh, nkv, hd, c.seq_len, pos0, count);
    if (e->q8) {
      if (!((gs == 16 || gs == 32 || gs == 64 || gs == 128) && hd % gs == 0))
        k_quantize_rows(e->bxq, e->bxs, e->bxb, d, count, d, gs);
      const GemmQ8Segment wo{e->bx, d, e->wo[l].k8(), K8Weight{}, nullptr, nullptr, d, GEMM_ADD};
      k_gemm_q8(e->bxq, e->bxs, count, d, gs, &wo, 1);
    } else {
      const GemmSegment wo{e->bx, d, e->wo[l].f(), nullptr, (size_t)d, d, GEMM_ADD};
      gemm_f32_or_bf16(e, e->bxb, d, count, d, &wo, 1, l, kWo, -1);
    }
    norm_rows(e->rms_ffn + (size_t)l * d);
    if (e->q8) {
      // hb quantized in the SwiGLU GEMM's epilogue where the shape allows (bitwise the GEMM then k_quantize_rows)
      const K8Weight w1 = e->w1[l].k8(), w3 = e->w3[l].k8();
      if (!llhip_gemm_q8_swiglu_quantize(e->bxq, e->bxs, count, d, gs, &w1, &w3, hidden, e->bhq, e->bhs)) {
        const GemmQ8Segment up{e->bhb, hidden, w1, w3, nullptr, nullptr, hidden, GEMM_SWIGLU};
        k_gemm_q8(e->bxq, e->bxs, count, d, gs, &up, 1);
        k_quantize_rows(e->bhq, e->bhs, e->bhb, hidden, count, hidden, gs);
      }
      if (llhip_last_error()[0])
        return nullptr;
      const GemmQ8Segment down{e->bx, d, e->w2[l].k8(), K8Weight{}, nullptr, nullptr, d, GEMM_ADD};
      k_gemm_q8(e->bhq, e->bhs, count, hidden, gs, &down, 1);
    } else {
      const GemmSegment up{e->bhb, hidden, e->w1[l].f(), e->w3[l].f(), (size_t)d, hidden, GEMM_SWIGLU};
      gemm_f32_or_bf16(e, e->bxb, d, count, d, &up, 1, l, kW1, 6);
      const GemmSegment down{e->bx, d, e->w2[l].f(), nullptr, (size_t)hidden, d, GEMM_ADD};
      gemm_f32_or_bf16(e, e->bhb, hidden, count, hidden, &down, 1, l, kW2, -1);
    }
  }
  if (want == LOGITS_NONE) {
    llhip_synchronize();
    return nullptr;
  }
  const size_t vocab = c.vocab_size;
  if (want == LOGITS_ALL && !e->blogits && !device_array(&e->blogits, (size_t)e->batch_rows * vocab))
    return nullptr;
  if (want == LOGITS_ALL && e->bf16) { // src/tp.c:601-609: a BF16 GEMM on the packed classifier
    if (!e->cls_packed) {
      std::vector<uint16_t> host(bf16_vnni_elements(c.vocab_size, d));
      pack_bf16_vnni(host.data(), e->cls.f(), c.vocab_size, d, (size_t)d);
      if (!device_array(&e->cls_packed, host.size()))
        return nullptr;
      llhip_memcpy_h2d(e->cls_packed, host.data(), host.size() * sizeof(uint16_t));
    }
    k_rmsnorm_rows(e->bx, e->bx, e->rms_final, count, d, c.norm_eps);
    const GemmBf16Segment seg{e->blogits, c.vocab_size, e->cls_packed, nullptr, c.vocab_size, GEMM_STORE};
    k_gemm_bf16(e->bx, d, count, d, &seg, 1, &e->panel);
  } else if (want == LOGITS_ALL) {
    // Every row's RMSNorm, then the classifier as a GEMM (in pieces whose logits copy meanwhile for Q8_0), where
    // src/tp.c:610-618 runs the classifier GEMV row by row: a GEMM row equals the GEMV of that row within the kernel
    // budget (tests/q8.c:158-183), and the classifier streams once per batch instead of once per row.
    if (e->q8) {
      norm_rows(e->rms_final);
      if (!logits_all_q8(e, count))
        return nullptr;
      llhip_synchronize();
      return llhip_last_error()[0] ? nullptr : e->host_batch;
    } else {
      k_rmsnorm_rows(e->bxb, e->bx, e->rms_final, count, d, c.norm_eps);
      const GemmSegment seg{e->blogits, c.vocab_size, e->cls.f(), nullptr, (size_t)d, c.vocab_size, GEMM_STORE};
      k_gemm_f32(e->bxb, d, count, d, &seg, 1);
    }
  } else {
    const K8Input in{e->xq, e->xs, nullptr}; // the last row (src/tp.c:610-618)
    float *x = e->bx + (size_t)(count - 1) * d;
    k_rmsnorm(x, x, e->rms_final, d, c.norm_eps);
    if (e->q8) {
      k_quantize(e->xq, e->xs, x, d, gs);
      k_matmul_q8(e->logits, &in, e->cls.k8(), d, c.vocab_size, gs);
    } else {
      k_matmul(e->logits, x, e->cls.f(), d, c.vocab_size);
    }
  }
  float *host;
  if (want == LOGITS_ALL) {
    if (!host_batch_room(e, (size_t)count * vocab))
      return nullptr;
    host = e->host_batch;
    llhip_memcpy_d2h(host, e->blogits, (size_t)count * vocab * sizeof(float));
  } else {
    host = e->host_logits;
    llhip_memcpy_d2h(host, e->logits, vocab * sizeof(float));
  }
  llhip_synchronize();
  return llhip_last_error()[0] ? nullptr : host;
}

// src/engine.c:65-81: with the batched GEMM on, more than one row (in BF16 mode any row) runs through the GEMMs;
// otherwise the rows run one token at a time, the classifier only for the rows whose logits are asked for.
float *forward_batch(Model *model, Engine *e, const int *tokens, int count, int pos0, LogitsWanted want) {
  prefill_validate(model, tokens, count, pos0, want);
  if (llhip_last_error()[0])
    return nullptr;
  if (model->prefill_gemm && (count > 1 || e->bf16))
    return forward_rows(model, e, tokens, count, pos0, want);
  const size_t vocab = e->c.vocab_size;
  if (want == LOGITS_ALL && !host_batch_room(e, (size_t)count * vocab))
    return nullptr;
  for (int i = 0; i < count; i++) {
    const bool wanted = want == LOGITS_ALL || (want == LOGITS_LAST && i == count - 1);
    if (!forward(e, tokens[i], pos0 + i, wanted))
      return nullptr;
    if (want == LOGITS_ALL)
      memcpy(e->host_batch + (size_t)i * vocab, e->host_logits, vocab * sizeof(float));
  }
  return want == LOGITS_NONE ? nullptr : want == LOGITS_ALL ? e->host_batch : e->host_logits;
}

} // namespace
} // namespace llhip

using namespace llhip;

extern "C" {

const int engine_q8 = 1;

void engine_load_context(Model *model, const char *path, int context) {
  if (!model) {
    raise("engine_load: null model");
    return;
  }
  memset(model, 0, sizeof(*model));
  if (!path) {
    raise("engine_load: null path");
    return;
  }
  llhip_clear_error();
  const char *activations = getenv("LLAMA_Q8_ACTIVATIONS"); // src/engine.c:132-135
  if (activations && *activations && strcmp(activations, "int8") && strcmp(activations, "fp32")) {
    raise("LLAMA_Q8_ACTIVATIONS must be int8 or fp32");
    return;
  }
  const bool a32 = activations && !strcmp(activations, "fp32");
  Engine *e = open_engine(model, path, context, a32);
  if (!e) {
    memset(model, 0, sizeof(*model));
    return;
  }
  model->config = e->c;
  model->implementation = e;
  model->file_bytes = e->bytes;
  model->mapped_bytes = e->bytes;
  last_group_size = e->gs;
  last_precision = e->q8 ? (e->a32 ? "int8_q8_0_w8a32" : "int8_q8_0") : (e->bf16 ? "bf16_from_fp32" : "fp32");
}

void engine_load(Model *model, const char *path) { engine_load_context(model, path, 0); }

float *engine_forward(Model *model, int token, int position) {
  Engine *e = model ? (Engine *)model->implementation : nullptr;
  if (!e) {
    raise("engine_forward: no model loaded");
    return nullptr;
  }
  llhip_clear_error(); // the result reports this token's failures only
  if (token < 0 || token >= model->config.vocab_size || position < 0 || position >= model->config.seq_len) {
    raise("forward input out of range: token=%d position=%d", token, position); // src/engine.c:171-172
    return nullptr;
  }
  return forward(e, token, position, true) ? e->host_logits : nullptr;
}

float *engine_forward_batch(Model *model, const int *tokens, int count, int pos0, LogitsWanted want) {
  Engine *e = model ? (Engine *)model->implementation : nullptr;
  if (!e) {
    raise("engine_forward_batch: no model loaded");
    return nullptr;
  }
  llhip_clear_error();
  return forward_batch(model, e, tokens, count, pos0, want);
}

void engine_kv_stats(Model *model, int position, int verify, KvStats *out) {
  (void)verify;
  Engine *e = model ? (Engine *)model->implementation : nullptr;
  if (!e || !out) {
    raise("engine_kv_stats: no model loaded");
    return;
  }
  const size_t row = (size_t)e->c.head_dim * e->c.n_kv_heads * sizeof(float);
  memset(out, 0, sizeof(*out));
  out->reserved_bytes = 2 * (size_t)e->c.n_layers * (size_t)e->c.seq_len * row;
  out->active_bytes = 2 * (size_t)e->c.n_layers * (size_t)(position > 0 ? position : 0) * row;
  out->node = -1;
}

void engine_free(Model *model) {
  if (!model || !model->implementation)
    return;
  Engine *e = (Engine *)model->implementation;
  k_attention_free(&e->work);
  release(e);
  model->implementation = nullptr;
}

int engine_group_size(void) { return last_group_size; }

const char *engine_precision(void) { return last_precision; }

} // extern "C"
