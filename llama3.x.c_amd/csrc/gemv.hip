// Decode-path kernels for gfx950: the activation quantizer, the streaming W8A8 GEMV and the FP32 GEMV.
//
// Lane layout shared by the quantizer and the GEMV: a wave covers 1024 consecutive values of a row per step, lane l
// holding values [16 l, 16 l + 16). With gs % 16 == 0 a group is gs / 16 consecutive lanes (a quad for gs = 64), so
// group maxima and int32 group dots are lane reductions inside the wave (DPP / swizzle shuffles), with no LDS.
#include "common.h"

namespace llhip {
namespace {

constexpr int kWave = 64;
constexpr int kBlock = 256;

__device__ __forceinline__ float silu_gate(float value, float gate) {
  // src/gemv.c:246-250: value * (1 / (1 + expf(-value))) * gate, same operation order.
  value *= (1.0f / (1.0f + expf(-value)));
  return value * gate;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1)
    v += __shfl_xor(v, m);
  return v;
}

template <class T> __device__ __forceinline__ T group_reduce_add(T v, int lpg) {
  for (int m = 1; m < lpg; m <<= 1)
    v += __shfl_xor(v, m);
  return v;
}

__device__ __forceinline__ float group_reduce_max(float v, int lpg) {
  for (int m = 1; m < lpg; m <<= 1)
    v = fmaxf(v, __shfl_xor(v, m));
  return v;
}

// One value of k_quantize (src/gemv.c:618-620): the IEEE quotient (hipcc emits a correctly rounded fp32 division by
// default), the clamp before rounding, roundf's half-away-from-zero rule.
__device__ __forceinline__ int quantize_one(float x, float scale) {
  float ratio = scale == 0.0f ? 0.0f : x / scale;
  return (int)roundf(fmaxf(-127.0f, fminf(127.0f, ratio)));
}

__device__ __forceinline__ int pack_bytes(int a, int b, int c, int d) {
  return (a & 0xff) | ((b & 0xff) << 8) | ((c & 0xff) << 16) | ((int)((unsigned)d << 24));
}

// Quantizes the 16 values a lane holds; every lane of the wave must call it (the group max is a lane reduction).
// Returns the packed int8 values and the group's scale; flags a non-finite input.
__device__ __forceinline__ int4 quantize_slice(const float4 (&v)[4], int lpg, float &scale, bool &bad) {
  float peak = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float e[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      bad |= !isfinite(e[j]);
      peak = fmaxf(peak, fabsf(e[j]));
    }
  }
  peak = group_reduce_max(peak, lpg);
  scale = peak / 127.0f;
  int4 q;
  q.x = pack_bytes(quantize_one(v[0].x, scale), quantize_one(v[0].y, scale), quantize_one(v[0].z, scale),
                   quantize_one(v[0].w, scale));
  q.y = pack_bytes(quantize_one(v[1].x, scale), quantize_one(v[1].y, scale), quantize_one(v[1].z, scale),
                   quantize_one(v[1].w, scale));
  q.z = pack_bytes(quantize_one(v[2].x, scale), quantize_one(v[2].y, scale), quantize_one(v[2].z, scale),
                   quantize_one(v[2].w, scale));
  q.w = pack_bytes(quantize_one(v[3].x, scale), quantize_one(v[3].y, scale), quantize_one(v[3].z, scale),
                   quantize_one(v[3].w, scale));
  return q;
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
  int first_wave;
};

struct GemvParams {
  GemvSeg seg[3];
  int nseg;
  const int8_t *xq;
  const float *xs;
  int n, gs, lpg;
  long long ld;     // weight row stride in values
  long long sld;    // weight scale row stride (ld / gs)
  int epi;
  int total_waves;
  int32_t *probe;   // optional, segment 0 only: probe[g * seg[0].rows + r]
};

// A wave-uniform segment from a kernel-argument array, by selects rather than a dynamic index (which would copy the
// arguments to scratch memory).
template <class T> __device__ __forceinline__ T pick(const T (&segs)[3], int s) {
  return s == 0 ? segs[0] : s == 1 ? segs[1] : segs[2];
}

__device__ __forceinline__ int dot16(int4 w, int4 x) {
  int d = __builtin_amdgcn_sdot4(w.x, x.x, 0, false);
  d = __builtin_amdgcn_sdot4(w.y, x.y, d, false);
  d = __builtin_amdgcn_sdot4(w.z, x.z, d, false);
  return __builtin_amdgcn_sdot4(w.w, x.w, d, false);
}

// Streaming W8A8 GEMV: each wave owns ROWS consecutive output rows of one segment and walks K in 1024-value steps.
// The block stages the int8 activations and their scales in LDS once; per row and step a lane reads 16 weight bytes
// (one 128-bit load), forms its partial int32 dot with four dot4 instructions, the group's lanes add their partials
// into the exact int32 group dot, and the group's first lane adds ((float)dot * ws) * xs to its FP32 accumulator (the
// reference's per-group expression, src/gemv.c:428). A wave reduction and the epilogue finish each row.
template <int ROWS, bool SWIGLU>
__global__ __launch_bounds__(kBlock) void q8_gemv(GemvParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  int8_t *sxq = reinterpret_cast<int8_t *>(smem);
  float *sxs = reinterpret_cast<float *>(smem + ((p.n + 15) & ~15));
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  for (int off = tid * 16; off < p.n; off += kBlock * 16)
    *reinterpret_cast<int4 *>(sxq + off) = *reinterpret_cast<const int4 *>(p.xq + off);
  for (int g = tid; g < p.n / p.gs; g += kBlock)
    sxs[g] = p.xs[g];
  __syncthreads();

  const int gw = blockIdx.x * (kBlock / kWave) + (tid >> 6);
  if (gw >= p.total_waves)
    return;
  int s = 0;
  while (s + 1 < p.nseg && gw >= p.seg[s + 1].first_wave)
    s++;
  const GemvSeg seg = pick(p.seg, s);
  const int r0 = (gw - seg.first_wave) * ROWS;
  const int nrows = min(ROWS, seg.rows - r0);
  const bool leader = (lane & (p.lpg - 1)) == 0;
  int32_t *probe = (s == 0) ? p.probe : nullptr;

  float acc[ROWS], gacc[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++)
    acc[i] = gacc[i] = 0.0f;

  const int steps = (p.n + 1023) >> 10;
  for (int c = 0; c < steps; c++) {
    const int off = (c << 10) + lane * 16;
    const bool active = off < p.n;
    const int4 xv = active ? *reinterpret_cast<const int4 *>(sxq + off) : int4{0, 0, 0, 0};
    const int g = off / p.gs;
    const float xsg = active ? sxs[g] : 0.0f;
    int4 wv[ROWS], w3v[ROWS];
#pragma unroll
    for (int i = 0; i < ROWS; i++) {
      wv[i] = w3v[i] = int4{0, 0, 0, 0};
      if (i < nrows && active) {
        const long long row = r0 + i;
        wv[i] = *reinterpret_cast<const int4 *>(seg.wq + row * p.ld + off);
        if (SWIGLU)
          w3v[i] = *reinterpret_cast<const int4 *>(seg.w3q + row * p.ld + off);
      }
    }
#pragma unroll
    for (int i = 0; i < ROWS; i++) {
      if (i >= nrows)
        break;
      const long long row = r0 + i;
      int d = group_reduce_add(dot16(wv[i], xv), p.lpg);
      if (probe && active && leader)
        probe[(long long)g * seg.rows + row] = d;
      if (active && leader)
        acc[i] += ((float)d * seg.ws[row * p.sld + g]) * xsg;
      if (SWIGLU) {
        int d3 = group_reduce_add(dot16(w3v[i], xv), p.lpg);
        if (active && leader)
          gacc[i] += ((float)d3 * seg.w3s[row * p.sld + g]) * xsg;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < ROWS; i++) {
    if (i >= nrows)
      break;
    const float total = wave_sum(acc[i]);
    const float gate = SWIGLU ? wave_sum(gacc[i]) : 0.0f;
    if (lane == 0) {
      float *o = seg.out + r0 + i;
      if (SWIGLU)
        *o = silu_gate(total, gate);
      else if (p.epi == EPI_ADD)
        *o += total;
      else
        *o = total;
    }
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
  while (s + 1 < p.nseg && row >= p.seg[s + 1].first_wave)
    s++;
  const GemvSeg seg = pick(p.seg, s);
  const long long r = row - seg.first_wave;
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
  const int gw = blockIdx.x * (kBlock / kWave) + (threadIdx.x >> 6);
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
    for (int off = lane * 4; off < p.n; off += kWave * 4) {
      const float4 xv = *reinterpret_cast<const float4 *>(p.x + off);
#pragma unroll
      for (int i = 0; i < ROWS; i++) {
        if (i >= nrows)
          break;
        const float4 wv = *reinterpret_cast<const float4 *>(seg.w + (r0 + i) * p.ld + off);
        acc[i] = fmaf(wv.x, xv.x, fmaf(wv.y, xv.y, fmaf(wv.z, xv.z, fmaf(wv.w, xv.w, acc[i]))));
        if (swiglu) {
          const float4 gv = *reinterpret_cast<const float4 *>(seg.w3 + (r0 + i) * p.ld + off);
          gacc[i] = fmaf(gv.x, xv.x, fmaf(gv.y, xv.y, fmaf(gv.z, xv.z, fmaf(gv.w, xv.w, gacc[i]))));
        }
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

template <int ROWS, bool SWIGLU> static void launch_fast(const GemvParams &p, hipStream_t stream) {
  const int blocks = (p.total_waves + 3) / 4;
  const size_t lds = ((size_t)(p.n + 15) & ~(size_t)15) + (size_t)(p.n / p.gs) * sizeof(float);
  hipLaunchKernelGGL((q8_gemv<ROWS, SWIGLU>), dim3(blocks), dim3(kBlock), lds, stream, p);
}

bool launch_q8_gemv(const GemvJob &job, hipStream_t stream) {
  int total_rows = 0;
  for (int s = 0; s < job.nseg; s++)
    total_rows += job.seg[s].rows;
  if (total_rows <= 0)
    return true;
  const int lpg = lanes_per_group(job.gs);
  const size_t lds = job.gs > 0 ? ((size_t)(job.n + 15) & ~(size_t)15) + (size_t)(job.n / job.gs) * sizeof(float) : 0;
  bool fast = job.xq && lpg && job.n % job.gs == 0 && job.ld % 16 == 0 && aligned16(job.xq) && lds <= 65536;
  for (int s = 0; s < job.nseg && fast; s++)
    fast = aligned16(job.seg[s].wq) && (job.epi != EPI_SWIGLU || aligned16(job.seg[s].w3q));
  if (fast) {
    GemvParams p{};
    // Rows per wave: four when there are enough rows to fill the chip with several waves per SIMD, fewer otherwise.
    const int rows = job.epi == EPI_SWIGLU ? (total_rows >= 8192 ? 2 : 1) : (total_rows >= 16384 ? 4 : total_rows >= 8192 ? 2 : 1);
    int waves = 0;
    for (int s = 0; s < job.nseg; s++) {
      const GemvSegment &g = job.seg[s];
      p.seg[s] = GemvSeg{g.out, g.wq, g.ws, g.w3q, g.w3s, g.rows, waves};
      waves += (g.rows + rows - 1) / rows;
    }
    p.nseg = job.nseg;
    p.xq = job.xq;
    p.xs = job.xs;
    p.n = job.n;
    p.gs = job.gs;
    p.lpg = lpg;
    p.ld = (long long)job.ld;
    p.sld = (long long)(job.ld / job.gs);
    p.epi = job.epi;
    p.total_waves = waves;
    p.probe = job.probe;
    if (job.epi == EPI_SWIGLU) {
      if (rows == 2)
        launch_fast<2, true>(p, stream);
      else
        launch_fast<1, true>(p, stream);
    } else if (rows == 4) {
      launch_fast<4, false>(p, stream);
    } else if (rows == 2) {
      launch_fast<2, false>(p, stream);
    } else {
      launch_fast<1, false>(p, stream);
    }
    return launch_ok("q8_gemv");
  }
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
