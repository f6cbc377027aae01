// Decode-path kernels for gfx950: the activation quantizer, the streaming W8A8 GEMV and the FP32 GEMV.
//
// Lane layout shared by the quantizer and the GEMV: a wave covers 1024 consecutive values of a row per step, lane l
// holding values [16 l, 16 l + 16). With gs % 16 == 0 a group is gs / 16 consecutive lanes (a quad for gs = 64), so
// group maxima and int32 group dots are lane reductions inside the wave (DPP / swizzle shuffles), with no LDS.
#include <atomic>
#include <cstdlib>

#include "common.h"
#include "lanes.h"
#include "quant.h"

namespace llhip {
namespace {

constexpr int kWave = 64;
constexpr int kBlock = 256;

__device__ __forceinline__ float silu_gate(float value, float gate) {
  // src/gemv.c:246-250: value * (1 / (1 + expf(-value))) * gate, same operation order.
  value *= (1.0f / (1.0f + expf(-value)));
  return value * gate;
}

// Quantizes the 16 values a lane holds; every lane of the wave must call it (the group max is a lane reduction).
// Returns the packed int8 values and the group's scale; flags a non-finite input.
__device__ __forceinline__ int4 quantize_slice(const float4 (&v)[4], int lpg, float &scale, bool &bad) {
  const float e[16] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w,
                       v[2].x, v[2].y, v[2].z, v[2].w, v[3].x, v[3].y, v[3].z, v[3].w};
  float peak = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; j++)
    peak = fmaxf(peak, fabsf(e[j])); // a NaN is skipped here and caught by quantize_fast
  peak = group_reduce_max(peak, lpg);
  scale = peak / 127.0f;
  bool ok;
  const float inv = group_reciprocal(scale, ok);
  int q[16];
  quantize_fast(e, scale, inv, ok, q, bad);
  return int4{pack_bytes(q[0], q[1], q[2], q[3]), pack_bytes(q[4], q[5], q[6], q[7]),
              pack_bytes(q[8], q[9], q[10], q[11]), pack_bytes(q[12], q[13], q[14], q[15])};
}

// k_quantize / k_quantize_rows, fast form: gs = 16 * lpg with lpg a power of two <= 64, n % 16 == 0, 16-byte aligned
// rows. Grid (ceil(n / 4096), m): block y quantizes row y, block x a 4096-value slab of it.
__global__ __launch_bounds__(kBlock) void quantize_lanes(int8_t *__restrict__ q, float *__restrict__ s,
                                                         const float *__restrict__ x, size_t ldx, int n, int gs,
                                                         int lpg, int *__restrict__ flags) {
  const int row = blockIdx.y;
  const int off = (blockIdx.x * kBlock + threadIdx.x) * 16;
  const bool active = off < n;
  float4 v[4] = {};
  if (active) {
    const float4 *src = reinterpret_cast<const float4 *>(x + (size_t)row * ldx + off);
#pragma unroll
    for (int i = 0; i < 4; i++)
      v[i] = src[i];
  }
  float scale;
  bool bad = false;
  int4 packed = quantize_slice(v, lpg, scale, bad);
  if (!active)
    return;
  if (bad)
    flags[0] = 1;
  *reinterpret_cast<int4 *>(q + (size_t)row * n + off) = packed;
  if ((threadIdx.x & (lpg - 1)) == 0)
    s[(size_t)row * (n / gs) + off / gs] = scale;
}

// RMSNorm of each row, then k_quantize of the normalized values, without the normalized row in memory: one 256-thread
// block per row. The sum of squares runs in rmsnorm_rows' order, whose 1024 threads (16 waves) each hold values
// 4 t + 4096 p: here logical thread t = 64 (4 W + r) + l lives in register set r of lane l of wave W, so each of the
// block's four waves holds four of those logical waves in registers and takes each one's DPP sum over the same lane
// positions; each logical thread's values go by fmaf and the 16 wave sums in order, and w * (ss * x) rounds as there,
// so the values quantized are rmsnorm_rows' bit for bit. Four rows' worth of waves per 1024 threads keeps every row of
// a 2048-row batch resident at once (one 1024-thread block per row took four rounds). A group of gs values is gs / 4
// consecutive lanes of one register set (the group maximum a lane reduction) quantized by the k_quantize rule as
// quantize_lanes applies it. Bitwise k_rmsnorm_rows then k_quantize_rows. n <= PASSES * 4096 (one pass holds 32 values
// a thread, in few enough registers for eight waves per SIMD), n % gs == 0, gs a power of two from 4 to 256.
constexpr int kNormQThreads = 256, kNormQLogical = 1024, kNormQSets = kNormQLogical / kNormQThreads, kNormQPasses = 2;
template <int PASSES>
__global__ __launch_bounds__(kNormQThreads) void rmsnorm_quantize_rows(int8_t *__restrict__ q, float *__restrict__ s,
                                                                       const float *__restrict__ x,
                                                                       const float *__restrict__ weight, int n,
                                                                       float epsilon, int gs, int *__restrict__ flags) {
  __shared__ float part[kNormQLogical / kWave];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const float *row = x + (size_t)blockIdx.x * n;
  float4 v[kNormQSets][PASSES], w[kNormQSets][PASSES];
  float ss[kNormQSets];
#pragma unroll
  for (int r = 0; r < kNormQSets; r++) {
    const int t = kWave * (kNormQSets * wave + r) + lane; // the logical thread
    ss[r] = 0.0f;
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
      const int j = 4 * t + p * 4 * kNormQLogical;
      v[r][p] = w[r][p] = float4{0.0f, 0.0f, 0.0f, 0.0f};
      if (j < n) {
        v[r][p] = *reinterpret_cast<const float4 *>(row + j);
        w[r][p] = *reinterpret_cast<const float4 *>(weight + j);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kNormQSets; r++) {
    const int t = kWave * (kNormQSets * wave + r) + lane;
#pragma unroll
    for (int p = 0; p < PASSES; p++)
      if (4 * t + p * 4 * kNormQLogical < n) {
        ss[r] = fmaf(v[r][p].x, v[r][p].x, ss[r]);
        ss[r] = fmaf(v[r][p].y, v[r][p].y, ss[r]);
        ss[r] = fmaf(v[r][p].z, v[r][p].z, ss[r]);
        ss[r] = fmaf(v[r][p].w, v[r][p].w, ss[r]);
      }
    ss[r] = wave_sum(ss[r]);
  }
  if (lane == 0)
#pragma unroll
    for (int r = 0; r < kNormQSets; r++)
      part[kNormQSets * wave + r] = ss[r];
  __syncthreads();
  float inv_rms = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormQLogical / kWave; i++)
    inv_rms += part[i];
  // src/kernels.c:15-17, the same three roundings
  inv_rms /= n;
  inv_rms += epsilon;
  inv_rms = 1.0f / sqrtf(inv_rms);
  const int lpg = gs / 4, groups = n / gs;
  bool bad = false;
#pragma unroll
  for (int r = 0; r < kNormQSets; r++) {
    const int lw = kNormQSets * wave + r, t = kWave * lw + lane;
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
      const int base = p * 4 * kNormQLogical, j = 4 * t + base;
      if (base + 4 * kWave * lw >= n)
        continue; // the whole logical wave is past the row (groups never straddle it: n % gs == 0)
      const float e[4] = {w[r][p].x * (inv_rms * v[r][p].x), w[r][p].y * (inv_rms * v[r][p].y),
                          w[r][p].z * (inv_rms * v[r][p].z), w[r][p].w * (inv_rms * v[r][p].w)};
      float peak = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; i++)
        peak = fmaxf(peak, fabsf(e[i])); // a NaN is skipped here and caught by quantize_fast
      peak = group_reduce_max(peak, lpg);
      const float scale = peak / 127.0f;
      bool ok;
      const float inv = group_reciprocal(scale, ok);
      int qv[4];
      quantize_fast(e, scale, inv, ok, qv, bad);
      if (j < n) {
        *reinterpret_cast<int *>(q + (size_t)blockIdx.x * n + j) = pack_bytes(qv[0], qv[1], qv[2], qv[3]);
        if ((lane & (lpg - 1)) == 0)
          s[(size_t)blockIdx.x * groups + j / gs] = scale;
      }
    }
  }
  if (bad)
    flags[0] = 1;
}

// Any group size: one thread per group, the reference's loop order (src/gemv.c:599-623).
__global__ __launch_bounds__(kBlock) void quantize_groups(int8_t *__restrict__ q, float *__restrict__ s,
                                                          const float *__restrict__ x, size_t ldx, int n, int gs,
                                                          int *__restrict__ flags) {
  const int groups = n / gs;
  const int row = blockIdx.y;
  const int g = blockIdx.x * kBlock + threadIdx.x;
  if (g >= groups)
    return;
  const float *in = x + (size_t)row * ldx + (size_t)g * gs;
  int8_t *dst = q + (size_t)row * n + (size_t)g * gs;
  float peak = 0.0f;
  bool bad = false;
  for (int i = 0; i < gs; i++) {
    bad |= !isfinite(in[i]);
    peak = fmaxf(peak, fabsf(in[i]));
  }
  if (bad)
    flags[0] = 1;
  const float scale = peak / 127.0f;
  s[(size_t)row * groups + g] = scale;
  for (int i = 0; i < gs; i++)
    dst[i] = (int8_t)quantize_one(in[i], scale);
}

// ---- W8A8 GEMV ------------------------------------------------------------------------------------------------------

struct GemvSeg {
  float *out;
  const int8_t *wq;
  const float *ws;
  const int8_t *w3q;
  const float *w3s;
  int rows;
  int first_row; // index of the segment's first row among all segments' rows
};

struct GemvParams {
  GemvSeg seg[3];
  int nseg;
  const int8_t *xq; // the quantized input (xq, xs), or with FUSED the FP32 input xf, quantized in the prologue
  const float *xs;
  const float *xf;
  int8_t *xq_out;   // FUSED: where block 0 stores the quantization it made (the caller's k_quantize outputs)
  float *xs_out;
  const float *norm_w; // NORM: xf is RMSNorm's input; the kernel normalizes it (weights norm_w) before quantizing
  float *norm_out;     // and block 0 stores the normalized row there (the caller's k_rmsnorm output)
  float norm_eps;
  int n, gs, lpg, nchunks;
  long long ld;     // weight row stride in values
  long long sld;    // weight scale row stride (ld / gs)
  int epi;
  int total_rows;   // rows of all segments
  int32_t *probe;   // optional, segment 0 only: probe[g * seg[0].rows + r]
  int *flags;
};

// A wave-uniform segment from a kernel-argument array, by selects rather than a dynamic index (which would copy the
// arguments to scratch memory).
template <class T> __device__ __forceinline__ T pick(const T (&segs)[3], int s) {
  return s == 0 ? segs[0] : s == 1 ? segs[1] : segs[2];
}

typedef int v4i __attribute__((ext_vector_type(4)));

// Buffer resources (V#): a base address and a byte bound. A buffer load past the bound returns zero and touches no
// memory, so a row's resource bounded to its n valid bytes (0 for a row the wave does not own) needs no clamping or
// masking, and the loads take a 32-bit offset plus an immediate instead of a 64-bit address each.
constexpr int kBufferWord3 = 0x00020000; // raw buffer, 32-bit data format
constexpr int kStream = 2;               // cache policy nt: weights are read once, stream them past the caches

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer(const void *base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, kBufferWord3);
}

__device__ __forceinline__ int4 load16(__amdgpu_buffer_rsrc_t r, int offset, int policy) {
  const v4i v = policy ? __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, kStream)
                       : __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0);
  return int4{v.x, v.y, v.z, v.w};
}

// One FP32 value: the builtin returns the 32 bits as an integer, reinterpreted here (not converted).
__device__ __forceinline__ float load4(__amdgpu_buffer_rsrc_t r, int offset) {
  return __uint_as_float((unsigned)__builtin_amdgcn_raw_buffer_load_b32(r, offset, 0, 0));
}

__device__ __forceinline__ int dot16(int4 w, int4 x) {
  int d = __builtin_amdgcn_sdot4(w.x, x.x, 0, false);
  d = __builtin_amdgcn_sdot4(w.y, x.y, d, false);
  d = __builtin_amdgcn_sdot4(w.z, x.z, d, false);
  return __builtin_amdgcn_sdot4(w.w, x.w, d, false);
}

// W8A32: the FP32 dot of 16 int8 weights (byte j of the int4 is weight j) with 16 FP32 inputs, each weight widened
// exactly to FP32; two accumulators halve the FMA dependency chain.
__device__ __forceinline__ float dot16f(int4 w, const float4 (&x)[4]) {
  const int words[4] = {w.x, w.y, w.z, w.w};
  float a = 0.0f, b = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int v = words[q];
    a = fmaf((float)((v << 24) >> 24), x[q].x, a);
    b = fmaf((float)((v << 16) >> 24), x[q].y, b);
    a = fmaf((float)((v << 8) >> 24), x[q].z, a);
    b = fmaf((float)(v >> 24), x[q].w, b);
  }
  return a + b;
}

// The block's copy of the input in LDS: the int8 activations and their scales, copied from (xq, xs), or (FUSED) made
// here from the FP32 input with the k_quantize rule, block 0 also storing them for the caller. load() only issues the
// global loads into registers; the kernel issues it before the weight loads, so waiting for the input does not wait
// for the weights (loads complete in issue order for the counter the waits use).
template <bool FUSED, int BLOCK, int MAXC, bool NORM = false> struct Input {
  static constexpr int kFusedPasses = (MAXC * 1024 + BLOCK * 16 - 1) / (BLOCK * 16); // 16 values per thread and pass
  static constexpr int kCopyPasses = (MAXC * 1024 + BLOCK * 16 - 1) / (BLOCK * 16);
  static constexpr int kScalePasses = (MAXC * 64 + BLOCK - 1) / BLOCK; // gs >= 16: at most n / 16 scales
  float4 xf[FUSED ? 4 * kFusedPasses : 1];
  float4 xw[NORM ? 4 * kFusedPasses : 1]; // NORM: the RMSNorm weights of the same values
  int4 xq[FUSED ? 1 : kCopyPasses];
  float xs[FUSED ? 1 : kScalePasses];

  // Unconditional buffer loads bounded to the input (see RowSet::load): values past n read zero.
  __device__ __forceinline__ void load(const GemvParams &p) {
    const int tid = threadIdx.x;
    if (FUSED) {
      const __amdgpu_buffer_rsrc_t r = buffer(p.xf, (unsigned)p.n * 4u);
#pragma unroll
      for (int i = 0; i < kFusedPasses; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int4 v = load16(r, (i * BLOCK * 16 + tid * 16) * 4 + j * 16, 0);
          xf[4 * i + j] = float4{__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w)};
        }
      if constexpr (NORM) {
        const __amdgpu_buffer_rsrc_t rw = buffer(p.norm_w, (unsigned)p.n * 4u);
#pragma unroll
        for (int i = 0; i < kFusedPasses; i++)
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int4 v = load16(rw, (i * BLOCK * 16 + tid * 16) * 4 + j * 16, 0);
            xw[4 * i + j] = float4{__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w)};
          }
      }
    } else {
      const __amdgpu_buffer_rsrc_t rq = buffer(p.xq, (unsigned)p.n), rs = buffer(p.xs, (unsigned)(p.n / p.gs) * 4u);
#pragma unroll
      for (int i = 0; i < kCopyPasses; i++)
        xq[i] = load16(rq, i * BLOCK * 16 + tid * 16, 0);
#pragma unroll
      for (int i = 0; i < kScalePasses; i++)
        xs[i] = load4(rs, (i * BLOCK + tid) * 4);
    }
  }

  // NORM: RMSNorm of the loaded row in place, src/kernels.c:10-20: the sum of squares reduced over the block (every
  // block forms the same one), ss /= n, ss += eps, ss = 1 / sqrtf(ss), then w * (ss * x); block 0 stores the result.
  // `scratch` holds one float per wave.
  __device__ __forceinline__ void normalize(const GemvParams &p, float *scratch) {
    const int tid = threadIdx.x;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 4 * kFusedPasses; i++) { // values past n were loaded as zeros
      ss = fmaf(xf[i].x, xf[i].x, ss);
      ss = fmaf(xf[i].y, xf[i].y, ss);
      ss = fmaf(xf[i].z, xf[i].z, ss);
      ss = fmaf(xf[i].w, xf[i].w, ss);
    }
    ss = wave_sum(ss);
    if ((tid & (kWave - 1)) == 0)
      scratch[tid / kWave] = ss;
    __syncthreads();
    ss = 0.0f;
#pragma unroll
    for (int w = 0; w < BLOCK / kWave; w++)
      ss += scratch[w];
    ss /= p.n;
    ss += p.norm_eps;
    ss = 1.0f / sqrtf(ss);
    const bool keep = blockIdx.x == 0;
#pragma unroll
    for (int i = 0; i < kFusedPasses; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float4 v = xf[4 * i + j], w = xw[4 * i + j];
        xf[4 * i + j] = float4{w.x * (ss * v.x), w.y * (ss * v.y), w.z * (ss * v.z), w.w * (ss * v.w)};
        const int off = i * BLOCK * 16 + tid * 16 + 4 * j;
        if (keep && off < p.n)
          *reinterpret_cast<float4 *>(p.norm_out + off) = xf[4 * i + j];
      }
  }

  __device__ __forceinline__ void stage(const GemvParams &p, int8_t *sxq, float *sxs) const {
    const int tid = threadIdx.x;
    if (!FUSED) {
#pragma unroll
      for (int i = 0; i < kCopyPasses; i++) {
        const int off = i * BLOCK * 16 + tid * 16;
        if (off < p.n)
          *reinterpret_cast<int4 *>(sxq + off) = xq[i];
      }
#pragma unroll
      for (int i = 0; i < kScalePasses; i++) {
        const int g = i * BLOCK + tid;
        if (g < p.n / p.gs)
          sxs[g] = xs[i];
      }
      return;
    }
    const bool keep = blockIdx.x == 0;
    bool bad = false;
    // 16 values per lane, a group over lpg lanes: one group maximum, division and reciprocal per 16 values. A wave
    // whose pass lies wholly past n skips it; otherwise all its lanes take part (the group max is a lane reduction),
    // lanes past n holding zeros (n is a whole number of groups, so no group mixes them with values).
    const int wave_off = (tid & ~(kWave - 1)) * 16;
#pragma unroll
    for (int i = 0; i < kFusedPasses; i++) {
      if (i * BLOCK * 16 + wave_off >= p.n)
        continue;
      const int off = i * BLOCK * 16 + tid * 16;
      const float4 v[4] = {xf[4 * i], xf[4 * i + 1], xf[4 * i + 2], xf[4 * i + 3]};
      float scale;
      const int4 q = quantize_slice(v, p.lpg, scale, bad);
      if (off < p.n) {
        *reinterpret_cast<int4 *>(sxq + off) = q;
        const bool first = (tid & (p.lpg - 1)) == 0;
        if (first)
          sxs[off / p.gs] = scale;
        if (keep) {
          *reinterpret_cast<int4 *>(p.xq_out + off) = q;
          if (first)
            p.xs_out[off / p.gs] = scale;
        }
      }
    }
    if (bad)
      p.flags[0] = 1;
  }
};

// Streaming W8A8 GEMV on a persistent grid of 8-wave blocks, about two per CU. KS waves share a row: wave `part` of
// the KS takes the row's 1024-byte chunks part, part + KS, part + 2 KS, ... (at most CH of them), so a long row (W2's
// 14336 inputs) is streamed by several waves at once and a block works on 8 / KS rows per step. Blocks take steps
// blockIdx.x, blockIdx.x + gridDim.x, ... and stage (or, FUSED, quantize) the input into LDS once for all of them.
//
// The weight loads are software-pipelined: a wave holds two register sets and issues the loads of its next step
// before it computes the current one, so every wave keeps a step's worth of HBM reads in flight while it works. For
// the first step they are issued before the input is staged. Per 1024-value chunk a lane forms its partial int32 dot
// of 16 values with four dot4 instructions, the group's lanes add theirs into the exact int32 group dot, and the
// group's first lane adds ((float)dot * ws) * xs to its FP32 accumulator (the reference's per-group expression,
// src/gemv.c:428). A wave reduction gives the wave's part of the row; with KS > 1 the parts meet in LDS and the first
// wave of the row adds them in part order and applies the epilogue.
template <int CH, int KS, bool SWIGLU, bool SG>
struct RowPart {
  // SG (gs = 64, 16 groups per 1024-byte chunk): scale register h of lane l holds the scale of group l % 16 of the
  // wave's chunk 4 h + l / 16, one load for four chunks, and each chunk's group leaders fetch theirs from the lane that
  // holds it (ds_bpermute); otherwise every lane loads its group's scale for every chunk.
  static constexpr int kScaleRegs = SG ? (CH + 3) / 4 : CH;
  int4 w[CH], w3[CH];
  float ws[kScaleRegs], w3s[kScaleRegs];
  float prior; // ADD: the output's current value, loaded with the weights
  GemvSeg seg;
  int s, row;
  bool own;

  // Every load is issued unconditionally through per-row buffer resources: a row past total_rows has a zero bound,
  // and chunks past n fall outside the row's bound, so all of them read zero with no memory access. With no branch
  // around any load the compiler can count them and wait for each only when it is used.
  __device__ __forceinline__ void load(const GemvParams &p, int index, int part, int lane) {
    own = index < p.total_rows;
    const int gl = own ? index : p.total_rows - 1;
    s = 0;
    while (s + 1 < p.nseg && gl >= p.seg[s + 1].first_row)
      s++;
    seg = pick(p.seg, s);
    row = gl - seg.first_row;
    const unsigned wbytes = own ? (unsigned)p.n : 0u, sbytes = own ? (unsigned)(p.n / p.gs) * 4u : 0u;
    const __amdgpu_buffer_rsrc_t rw = buffer(seg.wq + (long long)row * p.ld, wbytes);
    const __amdgpu_buffer_rsrc_t rs = buffer(seg.ws + (long long)row * p.sld, sbytes);
    __amdgpu_buffer_rsrc_t rw3 = rw, rs3 = rs;
    if (SWIGLU) {
      rw3 = buffer(seg.w3q + (long long)row * p.ld, wbytes);
      rs3 = buffer(seg.w3s + (long long)row * p.sld, sbytes);
    }
#pragma unroll
    for (int c = 0; c < CH; c++) {
      const int off = ((c * KS + part) << 10) + lane * 16;
      w[c] = load16(rw, off, 1);
      if (SWIGLU)
        w3[c] = load16(rw3, off, 1);
      if (!SG) {
        const int soff = (off / p.gs) * 4;
        ws[c] = load4(rs, soff);
        if (SWIGLU)
          w3s[c] = load4(rs3, soff);
      }
    }
    if (SG) {
#pragma unroll
      for (int h = 0; h < kScaleRegs; h++) {
        const int j = 4 * h + (lane >> 4); // the wave's chunk this lane's scale belongs to
        // past the wave's chunks the offset lies beyond every row's scales: zero, no access
        const int soff = j < CH ? (((j * KS + part) << 4) + (lane & 15)) * 4 : 0x7ffffff0;
        ws[h] = load4(rs, soff);
        if (SWIGLU)
          w3s[h] = load4(rs3, soff);
      }
    }
    // The residual read of ADD is issued here, after this step's weights: loads complete in issue order for the
    // counter the waits use, so reading it when the step's weights have arrived never waits on the loads of the
    // step issued after this one (a read issued at store time would).
    if (!SWIGLU)
      prior = load4(buffer(seg.out + row, own && part == 0 && p.epi == EPI_ADD ? 4u : 0u), 0);
  }

  // The scale of this lane's group in the wave's chunk c (and of the gate row's): under SG from lane
  // (c % 4) * 16 + lane / 4, which loaded it.
  __device__ __forceinline__ float scale(int c, int lane) const {
    const int src = ((c & 3) * 16 + (lane >> 2)) * 4;
    return SG ? __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(ws[c / 4 < kScaleRegs ? c / 4 : 0])))
              : ws[c < kScaleRegs ? c : 0];
  }
  __device__ __forceinline__ float gate_scale(int c, int lane) const {
    const int src = ((c & 3) * 16 + (lane >> 2)) * 4;
    return SG ? __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(w3s[c / 4 < kScaleRegs ? c / 4 : 0])))
              : w3s[c < kScaleRegs ? c : 0];
  }

  // W8A32: this wave's part of the row against the FP32 input the wave holds in registers (x[c]: its 16 values of
  // chunk c). Per chunk a lane forms the FP32 dot of its 16 widened weights and adds it times the group scale: the
  // reference's per-group sum times ws (src/gemv.c:141-181) up to FP32 rounding order.
  __device__ __forceinline__ float2 dot_f32(const GemvParams &p, const float4 (&x)[CH][4], int part, int lane) const {
    float acc = 0.0f, gacc = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
      if (c * KS + part < p.nchunks) {
        // lanes past n read zero weights, inputs and scales
        acc = fmaf(dot16f(w[c], x[c]), scale(c, lane), acc);
        if (SWIGLU)
          gacc = fmaf(dot16f(w3[c], x[c]), gate_scale(c, lane), gacc);
      }
    }
    return float2{wave_sum(acc), SWIGLU ? wave_sum(gacc) : 0.0f};
  }

  // This wave's part of the row (and of the gate row), reduced over the wave. Fully unrolled over compile-time
  // indices with guards, not early exits, so the arrays stay in registers.
  __device__ __forceinline__ float2 dot(const GemvParams &p, const int8_t *sxq, const float *sxs, int part,
                                        int lane) const {
    const bool leader = (lane & (p.lpg - 1)) == 0;
    int32_t *probe = (s == 0 && own) ? p.probe : nullptr;
    float acc = 0.0f, gacc = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
      if (c * KS + part < p.nchunks) {
        const int off = ((c * KS + part) << 10) + lane * 16;
        const bool active = off < p.n;
        const int4 xv = active ? *reinterpret_cast<const int4 *>(sxq + off) : int4{0, 0, 0, 0};
        const int g = off / p.gs;
        const float xsg = active ? sxs[g] : 0.0f;
        // this lane's int32 dot of its 16 values (exact); the group's lanes add theirs for the probe only
        const int pd = dot16(w[c], xv);
        if (probe) {
          const int d = group_reduce_add(pd, p.lpg);
          if (active && leader)
            probe[(long long)g * seg.rows + row] = d;
        }
        // every lane scales its partial: sum over the group's lanes of (float)partial * ws * xs, which differs from
        // ((float)dot * ws) * xs only in FP32 rounding
        acc = fmaf((float)pd, scale(c, lane) * xsg, acc);
        if (SWIGLU)
          gacc = fmaf((float)dot16(w3[c], xv), gate_scale(c, lane) * xsg, gacc);
      }
    }
    return float2{wave_sum(acc), SWIGLU ? wave_sum(gacc) : 0.0f};
  }

  __device__ __forceinline__ void store(const GemvParams &p, float total, float gate) const {
    if (!own)
      return;
    float *o = seg.out + row;
    if (SWIGLU)
      *o = silu_gate(total, gate);
    else if (p.epi == EPI_ADD)
      *o = prior + total;
    else
      *o = total;
  }
};

constexpr int kMaxGemvWaves = 16;

// One row step: the wave's part r of the row (and gate row) is combined with the row's other parts and stored.
template <int WAVES, int CH, int KS, bool SWIGLU, bool SG>
__device__ __forceinline__ void gemv_step(const GemvParams &p, const RowPart<CH, KS, SWIGLU, SG> &set, float2 r,
                                          float2 *red, int wave, int part, int lane, int &parity) {
  if (KS == 1) {
    if (lane == 0)
      set.store(p, r.x, r.y);
    return;
  }
  // Partials of step t go to half t % 2 of `red`: a half is rewritten two steps later, after the barrier of the step
  // in between, by which time its readers are done.
  float2 *half = red + parity * WAVES;
  if (lane == 0)
    half[wave] = r;
  __syncthreads();
  if (part == 0 && lane == 0) {
    float total = 0.0f, gate = 0.0f;
#pragma unroll
    for (int j = 0; j < KS; j++) {
      total += half[wave + j].x;
      gate += half[wave + j].y;
    }
    set.store(p, total, gate);
  }
  parity ^= 1;
}

template <int WAVES, int CH, int KS, bool SWIGLU, bool FUSED, bool SG, bool NORM = false>
__global__ __launch_bounds__(WAVES * 64) void q8_gemv(GemvParams p) {
  constexpr int kRows = WAVES / KS; // rows per block step
  extern __shared__ __align__(16) unsigned char smem[];
  int8_t *sxq = reinterpret_cast<int8_t *>(smem);
  float *sxs = reinterpret_cast<float *>(smem + ((p.n + 15) & ~15));
  float2 *red = reinterpret_cast<float2 *>(sxs + ((p.n / p.gs + 1) & ~1));
  const int lane = threadIdx.x & (kWave - 1);
  // wave-uniform by construction; readfirstlane lets the compiler keep row indices and pointers in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slot = wave / KS, part = wave % KS;
  const int steps = (p.total_rows + kRows - 1) / kRows;
  const int stride = gridDim.x;
  int step = blockIdx.x; // block-uniform, < steps (the grid never exceeds the step count)
  int parity = 0;
  Input<FUSED, WAVES * 64, CH * KS, NORM> in;
  in.load(p);
  __builtin_amdgcn_sched_barrier(0);
  // the first two steps' weights are in flight while the block stages its input
  RowPart<CH, KS, SWIGLU, SG> a, b;
  a.load(p, step * kRows + slot, part, lane);
  b.load(p, (step + stride) * kRows + slot, part, lane);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (NORM)
    in.normalize(p, reinterpret_cast<float *>(red)); // red is free until the first step's partials
  in.stage(p, sxq, sxs);
  __syncthreads();
  while (true) {
    gemv_step<WAVES>(p, a, a.dot(p, sxq, sxs, part, lane), red, wave, part, lane, parity);
    step += stride;
    if (step >= steps)
      break;
    a.load(p, (step + stride) * kRows + slot, part, lane);
    __builtin_amdgcn_sched_barrier(0);
    gemv_step<WAVES>(p, b, b.dot(p, sxq, sxs, part, lane), red, wave, part, lane, parity);
    step += stride;
    if (step >= steps)
      break;
    b.load(p, (step + stride) * kRows + slot, part, lane);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// W8A32 (FP32 input, src/gemv.c:141-181): the same persistent, software-pipelined row stream, the input not staged
// in LDS but held in registers. A wave's chunks (part, part + KS, ...) are the same for every row it takes, so each
// wave loads its 16 inputs per chunk and lane once (L2-resident after the first blocks) and keeps them for all its
// rows; LDS only carries the partial sums of a split row.
template <int WAVES, int CH, int KS, bool SWIGLU, bool SG>
__global__ __launch_bounds__(WAVES * 64) void q8_gemv_a32(GemvParams p) {
  constexpr int kRows = WAVES / KS;
  __shared__ float2 red[2 * WAVES];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slot = wave / KS, part = wave % KS;
  const int steps = (p.total_rows + kRows - 1) / kRows;
  const int stride = gridDim.x;
  int step = blockIdx.x; // block-uniform, < steps (the grid never exceeds the step count)
  int parity = 0;
  float4 x[CH][4];
  {
    // bounded to the n inputs: chunks and lanes past n read zero
    const __amdgpu_buffer_rsrc_t r = buffer(p.xf, (unsigned)p.n * 4u);
#pragma unroll
    for (int c = 0; c < CH; c++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int4 v = load16(r, ((((c * KS + part) << 10) + lane * 16) << 2) + q * 16, 0);
        x[c][q] = float4{__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w)};
      }
  }
  RowPart<CH, KS, SWIGLU, SG> a, b;
  a.load(p, step * kRows + slot, part, lane);
  b.load(p, (step + stride) * kRows + slot, part, lane);
  __builtin_amdgcn_sched_barrier(0);
  while (true) {
    gemv_step<WAVES>(p, a, a.dot_f32(p, x, part, lane), red, wave, part, lane, parity);
    step += stride;
    if (step >= steps)
      break;
    a.load(p, (step + stride) * kRows + slot, part, lane);
    __builtin_amdgcn_sched_barrier(0);
    gemv_step<WAVES>(p, b, b.dot_f32(p, x, part, lane), red, wave, part, lane, parity);
    step += stride;
    if (step >= steps)
      break;
    b.load(p, (step + stride) * kRows + slot, part, lane);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Any group size, W8A8 or W8A32 (xq == nullptr): one wave per output row, lane j takes groups j, j + 64, ...
// (src/gemv.c:417-438 per group).
struct GemvGenericParams {
  GemvSeg seg[3];
  int nseg;
  const int8_t *xq;
  const float *xs;
  const float *xf;
  int n, gs;
  long long ld, sld;
  int epi;
  int total_rows;
  int32_t *probe;
};

__device__ float generic_row(const int8_t *w, const float *ws, const GemvGenericParams &p, int lane, int32_t *probe,
                             long long row, int rows) {
  const int groups = p.n / p.gs;
  float acc = 0.0f;
  for (int g = lane; g < groups; g += kWave) {
    const int8_t *wg = w + (long long)g * p.gs;
    if (p.xq) {
      const int8_t *xg = p.xq + (long long)g * p.gs;
      int dot = 0;
      for (int t = 0; t < p.gs; t++)
        dot += (int)xg[t] * (int)wg[t];
      if (probe)
        probe[(long long)g * rows + row] = dot;
      acc += ((float)dot * ws[g]) * p.xs[g];
    } else {
      const float *xg = p.xf + (long long)g * p.gs;
      float part = 0.0f;
      for (int t = 0; t < p.gs; t++)
        part += (float)wg[t] * xg[t];
      acc += part * ws[g];
    }
  }
  return wave_sum(acc);
}

__global__ __launch_bounds__(kBlock) void q8_gemv_generic(GemvGenericParams p) {
  const int lane = threadIdx.x & (kWave - 1);
  int row = blockIdx.x * (kBlock / kWave) + (threadIdx.x >> 6);
  if (row >= p.total_rows)
    return;
  int s = 0;
  while (s + 1 < p.nseg && row >= p.seg[s + 1].first_row)
    s++;
  const GemvSeg seg = pick(p.seg, s);
  const long long r = row - seg.first_row;
  int32_t *probe = s == 0 ? p.probe : nullptr;
  const float total = generic_row(seg.wq + r * p.ld, seg.ws + r * p.sld, p, lane, probe, r, seg.rows);
  float gate = 0.0f;
  if (p.epi == EPI_SWIGLU)
    gate = generic_row(seg.w3q + r * p.ld, seg.w3s + r * p.sld, p, lane, nullptr, r, seg.rows);
  if (lane == 0) {
    float *o = seg.out + r;
    if (p.epi == EPI_SWIGLU)
      *o = silu_gate(total, gate);
    else if (p.epi == EPI_ADD)
      *o += total;
    else
      *o = total;
  }
}

// ---- FP32 GEMV ------------------------------------------------------------------------------------------------------

struct F32Seg {
  float *out;
  const float *w, *w3;
  int rows;
  int first_wave;
};
struct F32Params {
  F32Seg seg[3];
  int nseg;
  const float *x;
  int n;
  long long ld;
  int epi;
  int total_waves;
  bool vec4; // n % 4 == 0, ld % 4 == 0 and 16-byte aligned bases
};

template <int ROWS>
__global__ __launch_bounds__(kBlock) void f32_gemv(F32Params p) {
  const int lane = threadIdx.x & (kWave - 1);
  // wave-uniform: readfirstlane keeps the row pointers, and so the buffer resources, in scalar registers
  const int gw = blockIdx.x * (kBlock / kWave) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (gw >= p.total_waves)
    return;
  int s = 0;
  while (s + 1 < p.nseg && gw >= p.seg[s + 1].first_wave)
    s++;
  const F32Seg seg = pick(p.seg, s);
  const int r0 = (gw - seg.first_wave) * ROWS;
  const int nrows = min(ROWS, seg.rows - r0);
  const bool swiglu = p.epi == EPI_SWIGLU;
  float acc[ROWS], gacc[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++)
    acc[i] = gacc[i] = 0.0f;
  if (p.vec4) {
    // U 1 KB steps of every row in flight at once, the weights streamed past the caches (nt); rows and columns past
    // the end read zero through bounded buffer resources, so no load is conditional
    constexpr int U = ROWS >= 4 ? 2 : 4;
    const unsigned rowb = (unsigned)p.n * 4u;
    for (int off = lane * 4; off < p.n; off += kWave * 4 * U) {
      float4 wv[U][ROWS], gv[U][ROWS], xv[U];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int o = off + u * kWave * 4;
        const int4 xi = load16(buffer(p.x, rowb), o * 4, 0);
        xv[u] = float4{__int_as_float(xi.x), __int_as_float(xi.y), __int_as_float(xi.z), __int_as_float(xi.w)};
#pragma unroll
        for (int i = 0; i < ROWS; i++) {
          const unsigned bytes = i < nrows ? rowb : 0u;
          const int4 a = load16(buffer(seg.w + (r0 + i) * p.ld, bytes), o * 4, 1);
          wv[u][i] = float4{__int_as_float(a.x), __int_as_float(a.y), __int_as_float(a.z), __int_as_float(a.w)};
          if (swiglu) {
            const int4 g = load16(buffer(seg.w3 + (r0 + i) * p.ld, bytes), o * 4, 1);
            gv[u][i] = float4{__int_as_float(g.x), __int_as_float(g.y), __int_as_float(g.z), __int_as_float(g.w)};
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; u++)
#pragma unroll
        for (int i = 0; i < ROWS; i++) {
          acc[i] = fmaf(wv[u][i].x, xv[u].x, fmaf(wv[u][i].y, xv[u].y, fmaf(wv[u][i].z, xv[u].z, fmaf(wv[u][i].w, xv[u].w, acc[i]))));
          if (swiglu)
            gacc[i] = fmaf(gv[u][i].x, xv[u].x, fmaf(gv[u][i].y, xv[u].y, fmaf(gv[u][i].z, xv[u].z, fmaf(gv[u][i].w, xv[u].w, gacc[i]))));
        }
    }
  } else {
    for (int off = lane; off < p.n; off += kWave) {
      const float xv = p.x[off];
#pragma unroll
      for (int i = 0; i < ROWS; i++) {
        if (i >= nrows)
          break;
        acc[i] = fmaf(seg.w[(r0 + i) * p.ld + off], xv, acc[i]);
        if (swiglu)
          gacc[i] = fmaf(seg.w3[(r0 + i) * p.ld + off], xv, gacc[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < ROWS; i++) {
    if (i >= nrows)
      break;
    const float total = wave_sum(acc[i]);
    const float gate = swiglu ? wave_sum(gacc[i]) : 0.0f;
    if (lane == 0) {
      float *o = seg.out + r0 + i;
      if (swiglu)
        *o = silu_gate(total, gate);
      else if (p.epi == EPI_ADD)
        *o += total;
      else
        *o = total;
    }
  }
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

int lanes_per_group(int gs) {
  if (gs % 16 || gs > 1024)
    return 0;
  int lpg = gs / 16;
  return (lpg & (lpg - 1)) == 0 ? lpg : 0;
}

bool launch_ok(const char *what) {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess)
    return true;
  return raise("launching %s failed: %s", what, hipGetErrorString(e));
}

} // namespace

bool rmsnorm_quantize_fits(int n, int gs) {
  return n > 0 && n <= kNormQPasses * 4 * kNormQLogical && gs >= 4 && gs <= 256 && (gs & (gs - 1)) == 0 &&
         n % gs == 0;
}

bool launch_rmsnorm_quantize(int8_t *q, float *s, const float *x, const float *weight, int rows, int n, float epsilon,
                             int gs, hipStream_t stream) {
  if (rows <= 0)
    return true;
  if (n <= 4 * kNormQLogical)
    hipLaunchKernelGGL(rmsnorm_quantize_rows<1>, dim3((unsigned)rows), dim3(kNormQThreads), 0, stream, q, s, x, weight,
                       n, epsilon, gs, device().error_flags);
  else
    hipLaunchKernelGGL(rmsnorm_quantize_rows<kNormQPasses>, dim3((unsigned)rows), dim3(kNormQThreads), 0, stream, q, s,
                       x, weight, n, epsilon, gs, device().error_flags);
  return launch_ok("rmsnorm_quantize_rows");
}

bool launch_quantize(const QuantizeJob &job, hipStream_t stream) {
  if (job.m <= 0 || job.n / job.gs <= 0)
    return true;
  const int lpg = lanes_per_group(job.gs);
  int *flags = device().error_flags;
  const bool lanes =
      lpg && job.n % job.gs == 0 && job.ldx % 4 == 0 && aligned16(job.x) && aligned16(job.q) && job.n % 16 == 0;
  const int groups = job.n / job.gs;
  // Rows go to grid.y, at most 65535 per launch.
  for (int r0 = 0; r0 < job.m; r0 += 65535) {
    const int rows = job.m - r0 < 65535 ? job.m - r0 : 65535;
    int8_t *q = job.q + (size_t)r0 * job.n;
    float *s = job.s + (size_t)r0 * groups;
    const float *x = job.x + (size_t)r0 * job.ldx;
    if (lanes) {
      dim3 grid((job.n + kBlock * 16 - 1) / (kBlock * 16), rows);
      hipLaunchKernelGGL(quantize_lanes, grid, dim3(kBlock), 0, stream, q, s, x, job.ldx, job.n, job.gs, lpg, flags);
    } else {
      dim3 grid((groups + kBlock - 1) / kBlock, rows);
      hipLaunchKernelGGL(quantize_groups, grid, dim3(kBlock), 0, stream, q, s, x, job.ldx, job.n, job.gs, flags);
    }
    if (!launch_ok(lanes ? "quantize_lanes" : "quantize_groups"))
      return false;
  }
  return true;
}

// Launch-shape overrides set by llhip_set_gemv_shape (0: the default, or the environment's).
static std::atomic<int> forced_split{0}, forced_blocks{0}, forced_waves{0};

// Launch-shape overrides from the environment, read once (0: none).
static int env_shape(const char *name, int lo, int hi) {
  const char *env = getenv(name);
  const int v = env && *env ? atoi(env) : 0;
  return v >= lo && v <= hi ? v : 0;
}

// Dynamic LDS of the fast GEMV: the int8 input (rounded to 16 bytes), its scales (rounded to an even count) and the
// two halves of the per-wave partial sums.
static size_t gemv_lds_bytes(int n, int gs) {
  return ((size_t)(n + 15) & ~(size_t)15) + (size_t)((n / gs + 1) & ~1) * sizeof(float) + 2 * kMaxGemvWaves * 8;
}

// The input a fast GEMV takes: int8 (xq, xs), FP32 quantized in the prologue, or FP32 as it is (W8A32).
// IN_NORM: FP32 input normalized (RMSNorm) and quantized in the prologue (gs = 64 only).
enum GemvInput { IN_Q8, IN_FUSED, IN_F32, IN_NORM };

template <int WAVES, int CH, int KS, bool SWIGLU>
static void launch_shape(const GemvParams &p, GemvInput in, int per_cu, hipStream_t stream) {
  const size_t lds = gemv_lds_bytes(p.n, p.gs);
  const int steps = (p.total_rows + WAVES / KS - 1) / (WAVES / KS);
  const int cap = device().cu_count * per_cu;
  const int blocks = steps < cap ? steps : cap;
  const bool sg = p.gs == 64, fused = in == IN_FUSED;
  if (in == IN_F32) {
    if constexpr (CH <= 4) {
      if (sg)
        hipLaunchKernelGGL((q8_gemv_a32<WAVES, CH, KS, SWIGLU, true>), dim3(blocks), dim3(WAVES * 64), 0, stream, p);
      else
        hipLaunchKernelGGL((q8_gemv_a32<WAVES, CH, KS, SWIGLU, false>), dim3(blocks), dim3(WAVES * 64), 0, stream, p);
    } else {
      raise("internal: a W8A32 GEMV of more than four chunks per wave");
    }
  } else if (in == IN_NORM)
    hipLaunchKernelGGL((q8_gemv<WAVES, CH, KS, SWIGLU, true, true, true>), dim3(blocks), dim3(WAVES * 64), lds, stream,
                       p);
  else if (fused && sg)
    hipLaunchKernelGGL((q8_gemv<WAVES, CH, KS, SWIGLU, true, true>), dim3(blocks), dim3(WAVES * 64), lds, stream, p);
  else if (fused)
    hipLaunchKernelGGL((q8_gemv<WAVES, CH, KS, SWIGLU, true, false>), dim3(blocks), dim3(WAVES * 64), lds, stream, p);
  else if (sg)
    hipLaunchKernelGGL((q8_gemv<WAVES, CH, KS, SWIGLU, false, true>), dim3(blocks), dim3(WAVES * 64), lds, stream, p);
  else
    hipLaunchKernelGGL((q8_gemv<WAVES, CH, KS, SWIGLU, false, false>), dim3(blocks), dim3(WAVES * 64), lds, stream, p);
}

// The launch shape of one GEMV: waves per row (split of K), resident 8-wave block equivalents per CU, waves per block.
struct GemvShape {
  int split, per_cu, waves;
};

// Measured on MI355X over the 8B shapes (the 16-wave block stages the input once for twice the waves):
//   - rows of K <= 8192 take two waves each (at most four 1024-byte chunks per wave), longer rows four (W2's 14336);
//   - the SwiGLU pair (twice the registers per row) streams best from two 8-wave blocks per CU (21.9 us against
//     22.6 with three, 14336 x 4096 twice, in the 8B decode step);
//   - a long matrix (the 128256-row classifier) from one wave per row and four block equivalents per CU;
//   - everything else from one 16-wave block per CU;
//   - W8A32 (inputs in registers) from three 8-wave blocks per CU, at most two chunks per wave (W2 14.6 us against
//     17.2 with one 16-wave block of four-chunk waves, the SwiGLU pair 22.8 against 24.3), the classifier as above.
// llhip_set_gemv_shape and LLAMA_HIP_GEMV_KSPLIT / _BLOCKS_PER_CU / _BLOCK_WAVES override each part.
static GemvShape gemv_shape(int total_rows, int nchunks, bool swiglu, bool f32_input) {
  static const int env_split = env_shape("LLAMA_HIP_GEMV_KSPLIT", 1, 8);
  static const int env_per_cu = env_shape("LLAMA_HIP_GEMV_BLOCKS_PER_CU", 1, 64);
  static const int env_waves = env_shape("LLAMA_HIP_GEMV_BLOCK_WAVES", 8, 16);
  // waves per row by row length, measured: one for k <= 2048 (Llama-3.2-1B: QKV 5.0 -> 4.35 us, W1/W3 9.9 -> 9.1 us
  // against two), two for k <= 4096 (the 8B shapes), four beyond (1B W2, k = 8192: 7.5 -> 6.6 us; 8B W2, k = 14336)
  GemvShape g{nchunks <= 2 ? 1 : nchunks <= 4 ? 2 : 4, 2, 16};
  if (swiglu) {
    g.per_cu = 2;
    g.waves = 8;
  } else if (total_rows >= 32768) {
    g.split = nchunks <= 4 ? 1 : g.split;
    g.per_cu = 4;
  }
  if (f32_input && total_rows < 32768) {
    g.per_cu = 3;
    g.waves = 8;
  }
  const int split = forced_split.load(std::memory_order_relaxed), per_cu = forced_blocks.load(std::memory_order_relaxed),
            waves = forced_waves.load(std::memory_order_relaxed);
  g.split = split ? split : (env_split == 1 || env_split == 2 || env_split == 4 || env_split == 8) ? env_split : g.split;
  g.per_cu = per_cu ? per_cu : env_per_cu ? env_per_cu : g.per_cu;
  g.waves = waves ? waves : (env_waves == 8 || env_waves == 16) ? env_waves : g.waves;
  // W8A32 holds 16 FP32 inputs per chunk and lane in registers: at most four chunks per wave, two where the gate row
  // doubles the weight registers or more than two 8-wave blocks share a CU (spill-free and resident, as compiled)
  const int max_per = swiglu || g.per_cu > 2 ? 2 : 4;
  while (f32_input && g.split < 8 && (nchunks + g.split - 1) / g.split > max_per)
    g.split *= 2;
  return g;
}

template <int CH, int KS, bool SWIGLU>
static void launch_fast(const GemvParams &p, GemvInput in, const GemvShape &g, hipStream_t stream) {
  // per_cu counts 8-wave blocks: a 16-wave block stands for two
  if (g.waves == 16 && g.per_cu % 2 == 0)
    launch_shape<16, CH, KS, SWIGLU>(p, in, g.per_cu / 2, stream);
  else
    launch_shape<8, CH, KS, SWIGLU>(p, in, g.per_cu, stream);
}

template <int KS, bool SWIGLU>
static void launch_split(const GemvParams &p, GemvInput in, const GemvShape &g, hipStream_t stream) {
  const int per = (p.nchunks + KS - 1) / KS; // chunks per wave
  if (per <= 1)
    launch_fast<1, KS, SWIGLU>(p, in, g, stream);
  else if (per <= 2)
    launch_fast<2, KS, SWIGLU>(p, in, g, stream);
  else if (per <= 4)
    launch_fast<4, KS, SWIGLU>(p, in, g, stream);
  else if (in == IN_F32) // (gemv_shape keeps W8A32 at <= 4 chunks per wave) four waves of four cover 16 chunks
    launch_fast<4, 4, SWIGLU>(p, in, g, stream);
  else // per <= 16 only with one wave per row: two waves of at most 8 chunks instead (16 would spill registers)
    launch_fast<8, 2, SWIGLU>(p, in, g, stream);
}

bool set_gemv_shape(int waves_per_row, int blocks_per_cu, int block_waves) {
  if (!(waves_per_row == 0 || waves_per_row == 1 || waves_per_row == 2 || waves_per_row == 4 || waves_per_row == 8))
    return raise("llhip_set_gemv_shape: waves per row must be 0, 1, 2, 4 or 8, got %d", waves_per_row);
  if (blocks_per_cu < 0 || blocks_per_cu > 64)
    return raise("llhip_set_gemv_shape: blocks per CU must be 0..64, got %d", blocks_per_cu);
  if (!(block_waves == 0 || block_waves == 8 || block_waves == 16))
    return raise("llhip_set_gemv_shape: waves per block must be 0, 8 or 16, got %d", block_waves);
  forced_split.store(waves_per_row, std::memory_order_relaxed);
  forced_blocks.store(blocks_per_cu, std::memory_order_relaxed);
  forced_waves.store(block_waves, std::memory_order_relaxed);
  return true;
}

bool gemv_fast_path(const GemvJob &job) {
  const int lpg = lanes_per_group(job.gs);
  // W8A32: the FP32 input as it is (the int32 probe needs int8 activations: the generic kernel records none either)
  const bool f32_input = !job.xq && !job.xf_quantize && job.xf && !job.probe;
  const size_t lds = job.gs > 0 && !f32_input ? gemv_lds_bytes(job.n, job.gs) : 0;
  bool fast = (job.xq || job.xf_quantize || f32_input) && lpg && job.n > 0 && job.n % job.gs == 0 &&
              job.ld % 16 == 0 && lds <= 65536 && (job.n + 1023) / 1024 <= 16;
  // The fused prologue quantizes the FP32 input 16 values per lane, a group within a wave (lpg <= 64).
  fast = fast && (job.xf_quantize ? aligned16(job.xf) && aligned16(job.xq_out)
                  : f32_input     ? aligned16(job.xf)
                                  : aligned16(job.xq));
  // RMSNorm in the prologue: gs = 64, aligned weights and output, and the normalized row written by block 0 may not
  // be the input the other blocks read
  const bool norm = job.xf_quantize && job.norm_w;
  if (norm) {
    const uintptr_t n0 = (uintptr_t)job.norm_out, n1 = n0 + (size_t)job.n * sizeof(float);
    const uintptr_t x0 = (uintptr_t)job.xf, x1 = x0 + (size_t)job.n * sizeof(float);
    fast = fast && job.gs == 64 && aligned16(job.norm_w) && aligned16(job.norm_out) && (n1 <= x0 || x1 <= n0);
  }
  for (int s = 0; s < job.nseg && fast; s++) {
    fast = aligned16(job.seg[s].wq) && (job.epi != EPI_SWIGLU || aligned16(job.seg[s].w3q));
    // With an FP32 input every block reads it while others already write outputs: an output inside the input would
    // change what later blocks read (fused: quantize), so that case takes the quantization's own launch first, or
    // (W8A32) the generic kernel.
    if (job.xf_quantize || f32_input) {
      const uintptr_t o0 = (uintptr_t)job.seg[s].out, o1 = o0 + (size_t)job.seg[s].rows * sizeof(float);
      const uintptr_t x0 = (uintptr_t)job.xf, x1 = x0 + (size_t)job.n * sizeof(float);
      fast = fast && (o1 <= x0 || x1 <= o0);
      if (norm) { // nor inside the normalized row block 0 writes, nor in the norm weights
        const uintptr_t n0 = (uintptr_t)job.norm_out, n1 = n0 + (size_t)job.n * sizeof(float);
        const uintptr_t w0 = (uintptr_t)job.norm_w, w1 = w0 + (size_t)job.n * sizeof(float);
        fast = fast && (o1 <= n0 || n1 <= o0) && (o1 <= w0 || w1 <= o0);
      }
    }
  }
  return fast;
}

bool launch_q8_gemv(const GemvJob &job, hipStream_t stream) {
  int total_rows = 0;
  for (int s = 0; s < job.nseg; s++)
    total_rows += job.seg[s].rows;
  if (total_rows <= 0)
    return true;
  if (gemv_fast_path(job)) {
    GemvParams p{};
    int rows = 0;
    for (int s = 0; s < job.nseg; s++) {
      const GemvSegment &g = job.seg[s];
      p.seg[s] = GemvSeg{g.out, g.wq, g.ws, g.w3q, g.w3s, g.rows, rows};
      rows += g.rows;
    }
    p.nseg = job.nseg;
    p.xq = job.xq;
    p.xs = job.xs;
    p.xf = job.xf;
    p.xq_out = job.xq_out;
    p.xs_out = job.xs_out;
    p.norm_w = job.norm_w;
    p.norm_out = job.norm_out;
    p.norm_eps = job.norm_eps;
    p.n = job.n;
    p.gs = job.gs;
    p.lpg = lanes_per_group(job.gs);
    p.nchunks = (job.n + 1023) / 1024;
    p.ld = (long long)job.ld;
    p.sld = (long long)(job.ld / job.gs);
    p.epi = job.epi;
    p.total_rows = rows;
    p.probe = job.probe;
    p.flags = device().error_flags;
    const GemvInput in = job.xf_quantize ? (job.norm_w ? IN_NORM : IN_FUSED) : job.xq ? IN_Q8 : IN_F32;
    const bool swiglu = job.epi == EPI_SWIGLU;
    const GemvShape g = gemv_shape(rows, p.nchunks, swiglu, in == IN_F32);
    switch (g.split) {
    case 1:
      swiglu ? launch_split<1, true>(p, in, g, stream) : launch_split<1, false>(p, in, g, stream);
      break;
    case 2:
      swiglu ? launch_split<2, true>(p, in, g, stream) : launch_split<2, false>(p, in, g, stream);
      break;
    case 4:
      swiglu ? launch_split<4, true>(p, in, g, stream) : launch_split<4, false>(p, in, g, stream);
      break;
    default:
      swiglu ? launch_split<8, true>(p, in, g, stream) : launch_split<8, false>(p, in, g, stream);
      break;
    }
    return launch_ok(in == IN_F32 ? "q8_gemv_a32" : "q8_gemv");
  }
  if (job.xf_quantize)
    return raise("internal: a fused quantization was routed to the generic GEMV");
  GemvGenericParams p{};
  int rows = 0;
  for (int s = 0; s < job.nseg; s++) {
    const GemvSegment &g = job.seg[s];
    p.seg[s] = GemvSeg{g.out, g.wq, g.ws, g.w3q, g.w3s, g.rows, rows};
    rows += g.rows;
  }
  p.nseg = job.nseg;
  p.xq = job.xq;
  p.xs = job.xs;
  p.xf = job.xf;
  p.n = job.n;
  p.gs = job.gs;
  p.ld = (long long)job.ld;
  p.sld = (long long)(job.ld / job.gs);
  p.epi = job.epi;
  p.total_rows = rows;
  p.probe = job.probe;
  hipLaunchKernelGGL(q8_gemv_generic, dim3((rows + 3) / 4), dim3(kBlock), 0, stream, p);
  return launch_ok("q8_gemv_generic");
}

bool launch_f32_gemv(const F32GemvJob &job, hipStream_t stream) {
  F32Params p{};
  int total_rows = 0;
  for (int s = 0; s < job.nseg; s++)
    total_rows += job.seg[s].rows;
  if (total_rows <= 0)
    return true;
  const int rows = total_rows >= 16384 ? 4 : total_rows >= 8192 ? 2 : 1;
  int waves = 0;
  bool vec4 = job.n % 4 == 0 && job.ld % 4 == 0 && aligned16(job.x);
  for (int s = 0; s < job.nseg; s++) {
    const F32GemvSegment &g = job.seg[s];
    p.seg[s] = F32Seg{g.out, g.w, g.w3, g.rows, waves};
    waves += (g.rows + rows - 1) / rows;
    vec4 = vec4 && aligned16(g.w) && (job.epi != EPI_SWIGLU || aligned16(g.w3));
  }
  p.nseg = job.nseg;
  p.x = job.x;
  p.n = job.n;
  p.ld = (long long)job.ld;
  p.epi = job.epi;
  p.total_waves = waves;
  p.vec4 = vec4;
  const int blocks = (waves + 3) / 4;
  if (rows == 4)
    hipLaunchKernelGGL(f32_gemv<4>, dim3(blocks), dim3(kBlock), 0, stream, p);
  else if (rows == 2)
    hipLaunchKernelGGL(f32_gemv<2>, dim3(blocks), dim3(kBlock), 0, stream, p);
  else
    hipLaunchKernelGGL(f32_gemv<1>, dim3(blocks), dim3(kBlock), 0, stream, p);
  return launch_ok("f32_gemv");
}

} // namespace llhip
