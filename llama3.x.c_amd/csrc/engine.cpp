// The Q8_0 engine's host forward over the device library: engine_load maps a version-3 INT8 checkpoint, uploads it
// to HBM once (llhip_register_host) and allocates the activations and the K/V cache in device memory; engine_forward
// runs one decode token in the reference's order (src/tp.c:387-436 with one socket) through the library's entry
// points, so the recorded forms apply (RMSNorm and quantization inside the GEMV, RoPE and the cache stores inside
// attention) and only the logits cross PCIe.
//
// The header (src/runtime.c:179-260) and the tensor order (src/shards.c:77-99) are the reference's: FP32 norms first
// (rms_att[L], rms_ffn[L], rms_final), then each INT8 tensor as its values followed by its group scales, the
// embedding, then per role the layers back to back (wq, wk, wv, wo, w1, w2, w3), and the classifier unless tied.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdlib>
#include <cstdint>
#include <cstring>
#include <vector>

#include "common.h"
#include "llama_hip_engine.h"
#include "llama_hip_forward.h"
#include "llama_hip_gemm.h"

namespace llhip {
namespace {

constexpr uint32_t kMagic = 0x616b3432; // "24ka" read little-endian: the versioned checkpoint tag
constexpr int kHeaderBytes = 256;
int loaded_group_size = 0; // the group size of the last checkpoint loaded
bool fp32_activations = false; // LLAMA_Q8_ACTIVATIONS=fp32: W8A32, dequantized weights times FP32 activations

struct Q8Tensor {
  const int8_t *q;
  const float *s;
};

struct Engine {
  int fd = -1;
  unsigned char *map = nullptr;
  size_t bytes = 0;
  int gs = 0;
  Config c{};
  // inside the registered mapping (the library resolves them to their device copies)
  const float *rms_att = nullptr, *rms_ffn = nullptr, *rms_final = nullptr;
  Q8Tensor embed{}, cls{};
  std::vector<Q8Tensor> wq, wk, wv, wo, w1, w2, w3;
  // device memory
  float *x = nullptr, *xb = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *hb = nullptr, *logits = nullptr;
  float *rope = nullptr, *key_cache = nullptr, *value_cache = nullptr, *xs = nullptr, *hs = nullptr;
  int8_t *xq = nullptr, *hq = nullptr;
  std::vector<float> host_logits;
  AttentionWork work{};
  // the batched forward's rows (max_batch of each, allocated on its first call)
  int batch_rows = 0;
  float *bx = nullptr, *bxb = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr, *bhb = nullptr, *bxs = nullptr;
  float *brope = nullptr, *blogits = nullptr;
  int8_t *bxq = nullptr;
  std::vector<float> host_rope, host_batch_logits;
};

template <typename T> T read_at(const unsigned char *p, int offset) {
  T v;
  memcpy(&v, p + offset, sizeof(T));
  return v;
}

void release(Engine *e) {
  for (void *p : {(void *)e->x, (void *)e->xb, (void *)e->q, (void *)e->k, (void *)e->v, (void *)e->hb,
                  (void *)e->logits, (void *)e->rope, (void *)e->key_cache, (void *)e->value_cache, (void *)e->xs,
                  (void *)e->hs, (void *)e->xq, (void *)e->hq, (void *)e->bx, (void *)e->bxb, (void *)e->bq,
                  (void *)e->bk, (void *)e->bv, (void *)e->bhb, (void *)e->bxs, (void *)e->brope, (void *)e->blogits,
                  (void *)e->bxq})
    if (p)
      llhip_free(p);
  if (e->map) {
    (void)llhip_unregister_host(e->map);
    munmap(e->map, e->bytes);
  }
  if (e->fd >= 0)
    close(e->fd);
  delete e;
}

// The reference's checks of a version-3 INT8 header (src/runtime.c:213-247, validate_config at :150-167).
bool parse_header(Engine *e, const char *path) {
  const unsigned char *h = e->map;
  if (read_at<uint32_t>(h, 0) != kMagic)
    return raise("unsupported INT8 checkpoint: expected ak42 version 2 or 3");
  const int version = read_at<int>(h, 4);
  if (version != 3)
    return raise("unsupported checkpoint version %d for this executable", version);
  const int precision = read_at<int>(h, 36);
  if (precision < 0 || precision > 1)
    return raise("unsupported checkpoint precision %d", precision);
  if (precision != 1)
    return raise("checkpoint precision requires run executable");
  Config &c = e->c;
  memset(&c, 0, sizeof(c));
  memcpy(&c, h + 8, 28); // dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len
  c.shared = read_at<int>(h, 40);
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
  for (int i = 228; i < kHeaderBytes; i++)
    if (h[i])
      return raise("unsupported nonzero reserved checkpoint metadata");
  c.format = version;
  if (c.shared < 0 || c.shared > 1)
    return raise("invalid classifier flag in '%s'", path);
  if (c.dim <= 0 || c.hidden_dim <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 ||
      c.vocab_size <= 0 || c.seq_len <= 0 || c.n_heads % c.n_kv_heads || c.head_dim <= 0 ||
      (long long)c.head_dim * c.n_heads != c.dim)
    return raise("invalid model config in '%s'", path);
  if (e->gs <= 0 || e->gs > 131071 || c.dim % e->gs || c.hidden_dim % e->gs)
    return raise("unsupported INT8 group size %d: must divide dim and hidden_dim and fit int32 accumulation", e->gs);
  return true;
}

// Walks the tensors in file order; false (after raise) when the file is not exactly their size.
bool place_tensors(Engine *e, const char *path) {
  const Config &c = e->c;
  const size_t d = c.dim, hd = c.hidden_dim, kv = (size_t)c.head_dim * c.n_kv_heads, L = c.n_layers;
  size_t at = kHeaderBytes;
  auto floats = [&](size_t count) {
    const float *p = (const float *)(e->map + (at <= e->bytes ? at : 0));
    at += count * sizeof(float);
    return p;
  };
  auto q8 = [&](size_t count) {
    Q8Tensor t{(const int8_t *)(e->map + (at <= e->bytes ? at : 0)), nullptr};
    at += count;
    t.s = (const float *)(e->map + (at <= e->bytes ? at : 0));
    at += count / e->gs * sizeof(float);
    return t;
  };
  auto layers = [&](std::vector<Q8Tensor> &v, size_t count) {
    v.resize(L);
    for (size_t l = 0; l < L; l++)
      v[l] = q8(count);
  };
  e->rms_att = floats(L * d);
  e->rms_ffn = floats(L * d);
  e->rms_final = floats(d);
  e->embed = q8((size_t)c.vocab_size * d);
  layers(e->wq, d * d);
  layers(e->wk, kv * d);
  layers(e->wv, kv * d);
  layers(e->wo, d * d);
  layers(e->w1, hd * d);
  layers(e->w2, d * hd);
  layers(e->w3, hd * d);
  e->cls = c.shared ? e->embed : q8((size_t)c.vocab_size * d);
  if (at > e->bytes)
    return raise("truncated checkpoint '%s': need %zu bytes, found %zu", path, at, e->bytes);
  if (at != e->bytes)
    return raise("version 3 checkpoint has unexpected trailing bytes");
  return true;
}

template <typename T> bool device_array(T **p, size_t count) {
  *p = (T *)llhip_malloc(count * sizeof(T));
  return *p != nullptr;
}

bool allocate(Engine *e) {
  const Config &c = e->c;
  const size_t d = c.dim, kv = (size_t)c.head_dim * c.n_kv_heads;
  const size_t cache = (size_t)c.n_layers * c.seq_len * kv;
  return device_array(&e->x, d) && device_array(&e->xb, d) && device_array(&e->q, d) && device_array(&e->k, kv) &&
         device_array(&e->v, kv) && device_array(&e->hb, (size_t)c.hidden_dim) &&
         device_array(&e->logits, (size_t)c.vocab_size) && device_array(&e->rope, 2 * (size_t)c.head_dim) &&
         device_array(&e->key_cache, cache) && device_array(&e->value_cache, cache) &&
         device_array(&e->xq, d) && device_array(&e->xs, d / e->gs) && device_array(&e->hq, (size_t)c.hidden_dim) &&
         device_array(&e->hs, (size_t)c.hidden_dim / e->gs);
}

Engine *open_engine(const char *path, int context) {
  Engine *e = new Engine();
  e->fd = open(path, O_RDONLY);
  if (e->fd < 0) {
    raise("cannot open checkpoint '%s': %s", path, strerror(errno));
    return release(e), nullptr;
  }
  struct stat st;
  if (fstat(e->fd, &st) || !S_ISREG(st.st_mode) || st.st_size < kHeaderBytes) {
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
  if (context > 0 && context < e->c.seq_len)
    e->c.seq_len = context; // the K/V cache covers the requested context only
  if (llhip_register_host(e->map, e->bytes) != 0) {
    munmap(e->map, e->bytes);
    e->map = nullptr;
    return release(e), nullptr;
  }
  if (!allocate(e))
    return release(e), nullptr;
  k_attention_init(&e->work, e->c.n_heads, e->c.n_kv_heads, e->c.head_dim, e->c.seq_len);
  e->host_logits.resize((size_t)e->c.vocab_size);
  return e;
}

// One decode token (src/tp.c:387-436, one socket, W8A8): the embedding row, per layer RMSNorm, quantize, QKV, RoPE,
// the K/V cache (head-major: staged rows then k_kv_store; rows layout: written in place), attention, quantize,
// Wo + residual, RMSNorm, quantize, W1/W3 SwiGLU, quantize, W2 + residual; then the final RMSNorm in place, quantize
// and the classifier.
bool forward(Engine *e, int token, int pos) {
  const Config &c = e->c;
  const int d = c.dim, hidden = c.hidden_dim, hd = c.head_dim, gs = e->gs, nh = c.n_heads, nkv = c.n_kv_heads;
  const size_t kvl = (size_t)hd * nkv;
  llhip_clear_error(); // the result below reports this token's failures only
  if (token < 0 || token >= c.vocab_size)
    return raise("token %d outside the vocabulary of %d", token, c.vocab_size);
  if (pos < 0 || pos >= c.seq_len)
    return raise("position %d outside the context of %d", pos, c.seq_len);
  k_embed_q8_rows(e->x, e->embed.q, e->embed.s, &token, 1, d, gs, c.vocab_size);
  k_rope_table(&c, pos, e->rope);
  const bool head = kernels_kv_layout_head() != 0;
  // W8A8 quantizes each GEMV input (q8_input, src/tp.c:380-385); W8A32 hands the FP32 rows over instead
  const bool a32 = fp32_activations;
  const K8Input in_d = a32 ? K8Input{nullptr, nullptr, e->xb} : K8Input{e->xq, e->xs, nullptr};
  const K8Input in_h = a32 ? K8Input{nullptr, nullptr, e->hb} : K8Input{e->hq, e->hs, nullptr};
  const K8Input in_x = a32 ? K8Input{nullptr, nullptr, e->x} : in_d;
  auto quantize = [&](int8_t *q, float *s, const float *x, int n) {
    if (!a32)
      k_quantize(q, s, x, n, gs);
  };
  for (int l = 0; l < c.n_layers; l++) {
    const size_t layer = (size_t)l * c.seq_len * kvl;
    float *kc = e->key_cache + layer, *vc = e->value_cache + layer;
    float *k = head ? e->k : kc + (size_t)pos * kvl, *v = head ? e->v : vc + (size_t)pos * kvl;
    k_rmsnorm(e->xb, e->x, e->rms_att + (size_t)l * d, d, c.norm_eps);
    quantize(e->xq, e->xs, e->xb, d);
    k_matmul_q8_qkv(e->q, k, v, &in_d, K8Weight{e->wq[l].q, e->wq[l].s}, K8Weight{e->wk[l].q, e->wk[l].s},
                    K8Weight{e->wv[l].q, e->wv[l].s}, d, d, (int)kvl, gs);
    k_rope_apply(e->q, k, e->rope, nh, nkv, hd);
    if (head) {
      k_kv_store(kc, k, kvl, pos, 1, nkv, hd, c.seq_len);
      k_kv_store(vc, v, kvl, pos, 1, nkv, hd, c.seq_len);
    }
    k_attention_kv(e->xb, e->q, kc, vc, nullptr, &e->work, nh, nkv, hd, c.seq_len, pos);
    quantize(e->xq, e->xs, e->xb, d);
    k_matmul_q8_add(e->x, &in_d, K8Weight{e->wo[l].q, e->wo[l].s}, d, d, gs);
    k_rmsnorm(e->xb, e->x, e->rms_ffn + (size_t)l * d, d, c.norm_eps);
    quantize(e->xq, e->xs, e->xb, d);
    k_matmul_q8_swiglu(e->hb, &in_d, K8Weight{e->w1[l].q, e->w1[l].s}, K8Weight{e->w3[l].q, e->w3[l].s}, d, hidden,
                       gs);
    quantize(e->hq, e->hs, e->hb, hidden);
    k_matmul_q8_add(e->x, &in_h, K8Weight{e->w2[l].q, e->w2[l].s}, hidden, d, gs);
  }
  k_rmsnorm(e->x, e->x, e->rms_final, d, c.norm_eps);
  quantize(e->xq, e->xs, e->x, d);
  k_matmul_q8(e->logits, &in_x, K8Weight{e->cls.q, e->cls.s}, d, c.vocab_size, gs);
  llhip_memcpy_d2h(e->host_logits.data(), e->logits, (size_t)c.vocab_size * sizeof(float));
  llhip_synchronize(); // reports a non-finite activation or score of this token
  return llhip_last_error()[0] == 0;
}

bool allocate_batch(Engine *e, int rows) {
  const Config &c = e->c;
  const size_t m = rows, d = c.dim, kv = (size_t)c.head_dim * c.n_kv_heads, h = c.hidden_dim;
  if (!(device_array(&e->bx, m * d) && device_array(&e->bxb, m * d) && device_array(&e->bq, m * d) &&
        device_array(&e->bk, m * kv) && device_array(&e->bv, m * kv) && device_array(&e->bhb, m * h) &&
        device_array(&e->bxq, m * h) && device_array(&e->bxs, m * h / e->gs) &&
        device_array(&e->brope, m * 2 * c.head_dim)))
    return false;
  e->host_rope.resize(m * 2 * c.head_dim);
  e->batch_rows = rows;
  return true;
}

// count tokens at pos0 .. pos0 + count - 1 (src/tp.c:528-622 with one socket, W8A8): the embedding rows and RoPE
// tables, per layer RMSNorm of the rows, quantize, the QKV GEMM, RoPE, the cache rows, batched causal attention,
// quantize, Wo + residual, RMSNorm, quantize, W1/W3 SwiGLU, quantize, W2 + residual; then the final RMSNorm,
// quantize and classifier GEMV of the last row (LAST) or of every row (ALL).
float *forward_batch(Model *model, Engine *e, const int *tokens, int count, int pos0, LogitsWanted want) {
  llhip_clear_error();
  prefill_validate(model, tokens, count, pos0, want);
  if (llhip_last_error()[0])
    return nullptr;
  const Config &c = e->c;
  const int d = c.dim, hidden = c.hidden_dim, hd = c.head_dim, gs = e->gs, nh = c.n_heads, nkv = c.n_kv_heads;
  const int kvl = hd * nkv;
  if (fp32_activations) { // W8A32 has no batched GEMM: the batch is one row (src/engine.c:97-104)
    if (!forward(e, tokens[0], pos0))
      return nullptr;
    return want == LOGITS_NONE ? nullptr : e->host_logits.data();
  }
  if (!e->batch_rows && !allocate_batch(e, model->max_batch))
    return nullptr;
  for (int i = 0; i < count; i++)
    k_rope_table(&c, pos0 + i, e->host_rope.data() + (size_t)i * 2 * hd);
  llhip_memcpy_h2d(e->brope, e->host_rope.data(), (size_t)count * 2 * hd * sizeof(float));
  k_embed_q8_rows(e->bx, e->embed.q, e->embed.s, tokens, count, d, gs, c.vocab_size);
  const bool head = kernels_kv_layout_head() != 0;
  for (int l = 0; l < c.n_layers; l++) {
    const size_t layer = (size_t)l * c.seq_len * kvl;
    float *kc = e->key_cache + layer, *vc = e->value_cache + layer;
    float *kd = head ? e->bk : kc + (size_t)pos0 * kvl, *vd = head ? e->bv : vc + (size_t)pos0 * kvl;
    k_rmsnorm_rows(e->bxb, e->bx, e->rms_att + (size_t)l * d, count, d, c.norm_eps);
    k_quantize_rows(e->bxq, e->bxs, e->bxb, d, count, d, gs);
    const GemmQ8Segment qkv[3] = {
        {e->bq, d, K8Weight{e->wq[l].q, e->wq[l].s}, K8Weight{}, nullptr, nullptr, d, GEMM_STORE},
        {kd, kvl, K8Weight{e->wk[l].q, e->wk[l].s}, K8Weight{}, nullptr, nullptr, kvl, GEMM_STORE},
        {vd, kvl, K8Weight{e->wv[l].q, e->wv[l].s}, K8Weight{}, nullptr, nullptr, kvl, GEMM_STORE}};
    k_gemm_q8(e->bxq, e->bxs, count, d, gs, qkv, 3);
    k_rope_apply_rows(e->bq, d, kd, kvl, e->brope, 2 * (size_t)hd, count, nh, nkv, hd);
    if (head) {
      k_kv_store(kc, kd, kvl, pos0, count, nkv, hd, c.seq_len);
      k_kv_store(vc, vd, kvl, pos0, count, nkv, hd, c.seq_len);
    }
    k_attention_batch_kv(e->bxb, e->bq, kc, vc, nullptr, &e->work, nh, nkv, hd, c.seq_len, pos0, count);
    k_quantize_rows(e->bxq, e->bxs, e->bxb, d, count, d, gs);
    const GemmQ8Segment wo{e->bx, d, K8Weight{e->wo[l].q, e->wo[l].s}, K8Weight{}, nullptr, nullptr, d, GEMM_ADD};
    k_gemm_q8(e->bxq, e->bxs, count, d, gs, &wo, 1);
    k_rmsnorm_rows(e->bxb, e->bx, e->rms_ffn + (size_t)l * d, count, d, c.norm_eps);
    k_quantize_rows(e->bxq, e->bxs, e->bxb, d, count, d, gs);
    const GemmQ8Segment up{e->bhb,  hidden,  K8Weight{e->w1[l].q, e->w1[l].s}, K8Weight{e->w3[l].q, e->w3[l].s},
                           nullptr, nullptr, hidden,                          GEMM_SWIGLU};
    k_gemm_q8(e->bxq, e->bxs, count, d, gs, &up, 1);
    k_quantize_rows(e->bxq, e->bxs, e->bhb, hidden, count, hidden, gs);
    const GemmQ8Segment down{e->bx, d, K8Weight{e->w2[l].q, e->w2[l].s}, K8Weight{}, nullptr, nullptr, d, GEMM_ADD};
    k_gemm_q8(e->bxq, e->bxs, count, hidden, gs, &down, 1);
  }
  if (want == LOGITS_NONE) {
    llhip_synchronize();
    return nullptr;
  }
  const size_t vocab = c.vocab_size;
  if (want == LOGITS_ALL && !e->blogits && !device_array(&e->blogits, (size_t)e->batch_rows * vocab))
    return nullptr;
  const K8Input in{e->xq, e->xs, nullptr};
  for (int i = want == LOGITS_ALL ? 0 : count - 1; i < count; i++) {
    float *x = e->bx + (size_t)i * d;
    k_rmsnorm(x, x, e->rms_final, d, c.norm_eps);
    k_quantize(e->xq, e->xs, x, d, gs);
    k_matmul_q8(want == LOGITS_ALL ? e->blogits + (size_t)i * vocab : e->logits, &in, K8Weight{e->cls.q, e->cls.s}, d,
                c.vocab_size, gs);
  }
  float *host;
  if (want == LOGITS_ALL) {
    e->host_batch_logits.resize((size_t)count * vocab);
    host = e->host_batch_logits.data();
    llhip_memcpy_d2h(host, e->blogits, (size_t)count * vocab * sizeof(float));
  } else {
    host = e->host_logits.data();
    llhip_memcpy_d2h(host, e->logits, vocab * sizeof(float));
  }
  llhip_synchronize();
  return llhip_last_error()[0] ? nullptr : host;
}

} // namespace
} // namespace llhip

using namespace llhip;

extern "C" {

const int engine_q8 = 1;

void engine_load_context(Model *model, const char *path, int context) {
  memset(model, 0, sizeof(*model));
  if (!path) {
    raise("engine_load: null path");
    return;
  }
  const char *activations = getenv("LLAMA_Q8_ACTIVATIONS"); // src/engine.c:132-135
  if (activations && *activations && strcmp(activations, "int8") && strcmp(activations, "fp32")) {
    raise("LLAMA_Q8_ACTIVATIONS must be int8 or fp32");
    return;
  }
  fp32_activations = activations && !strcmp(activations, "fp32");
  Engine *e = open_engine(path, context);
  if (!e)
    return;
  model->config = e->c;
  model->implementation = e;
  loaded_group_size = e->gs;
  model->file_bytes = e->bytes;
  model->mapped_bytes = e->bytes;
  prefill_configure_engine(model, fp32_activations ? 1 : LLHIP_PREFILL_BATCH_Q8, 1);
  if (fp32_activations) {
    model->prefill_gemm = 0;
    model->prefill_kernel = nullptr;
  }
}

void engine_load(Model *model, const char *path) { engine_load_context(model, path, 0); }

float *engine_forward(Model *model, int token, int position) {
  Engine *e = model ? (Engine *)model->implementation : nullptr;
  if (!e) {
    raise("engine_forward: no model loaded");
    return nullptr;
  }
  return forward(e, token, position) ? e->host_logits.data() : nullptr;
}

float *engine_forward_batch(Model *model, const int *tokens, int count, int pos0, LogitsWanted want) {
  Engine *e = model ? (Engine *)model->implementation : nullptr;
  if (!e) {
    raise("engine_forward_batch: no model loaded");
    return nullptr;
  }
  return forward_batch(model, e, tokens, count, pos0, want);
}

void engine_free(Model *model) {
  if (!model || !model->implementation)
    return;
  Engine *e = (Engine *)model->implementation;
  k_attention_free(&e->work);
  release(e);
  model->implementation = nullptr;
}

int engine_group_size(void) { return loaded_group_size; }

const char *engine_precision(void) { return fp32_activations ? "int8_q8_0_w8a32" : "int8_q8_0"; }

} // extern "C"
