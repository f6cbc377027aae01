// The int8 GEMM for short batches: k_gemm_q8 with at most 32 activation rows (a prompt of a few tokens, or a batch of
// decode steps that share one pass over the weights).
//
// The tiled kernel (gemm.hip) computes 256 activation rows per tile whatever m is, so below a few dozen rows its time
// is that of m = 256, about three times the time to stream the weights. Here the weights are streamed once, as in the
// decode GEMV: a block owns 16 weight rows (16 output columns, and the same 16 of W3 under SWIGLU), or 32 as two MFMA
// tiles sharing each activation load for batches of 17-32 rows on wide grids, and its waves (four or eight) split K
// into consecutive ranges. A wave loads the weights of two 64-value K steps at once, as two loads of 1 KB that each
// take 128 contiguous bytes of eight rows (a load of one step's operand would take 64 bytes of each of 16 rows, half a
// cache line, and took up to 19% longer on the 8B shapes), and forms the B operand of v_mfma_i32_16x16x64_i8 for each
// step with one DPP row shift per register. The activations (16 rows per MFMA tile, MT = 1 or 2 tiles) load straight
// into the A operand; two pairs of steps are in flight. At a group's last step the exact int32 dots are rescaled,
// acc += ((float)dot * ws) * xs, from scales staged in LDS. The waves' partial sums of an output meet in LDS and are
// added in wave order; the epilogue (STORE, ADD, SWIGLU) follows.
#include <atomic>

#include "common.h"

namespace llhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kSkPairs = 2; // pairs of K steps in flight per wave

struct SkSeg {
  float *c;
  int ldc;
  const int8_t *w, *w3;
  const float *ws, *w3s;
  int n, epi;
  int first_tile;
};

struct SkParams {
  SkSeg seg[3];
  int nseg;
  const int8_t *xq;
  const float *xs;
  int m, k, gs, groups, steps, per; // per: K steps of each wave (a multiple of the steps per group)
};

__device__ __forceinline__ SkSeg sk_pick(const SkParams &p, int s) { return s == 0 ? p.seg[0] : s == 1 ? p.seg[1] : p.seg[2]; }

// A raw buffer resource from wave-uniform values (readfirstlane keeps it in scalar registers); loads past `bytes` read
// zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_buffer(const void *base, long long bytes) {
  const unsigned long long b = (unsigned long long)(uintptr_t)base;
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)b);
  const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(b >> 32));
  const int n = __builtin_amdgcn_readfirstlane((int)(bytes > 0 ? bytes : 0));
  return __builtin_amdgcn_make_buffer_rsrc((void *)(uintptr_t)(((unsigned long long)hi << 32) | lo), (short)0, n,
                                           0x00020000);
}

__device__ __forceinline__ float sk_silu_gate(float value, float gate) {
  value *= (1.0f / (1.0f + expf(-value)));
  return value * gate;
}

constexpr int kStream = 2; // cache policy nt for the weights, read once

// s_waitcnt vmcnt(N), the other counters left alone (gfx9 encoding: vmcnt bits 3:0 and 15:14)
template <int N> __device__ __forceinline__ void sk_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

__host__ __device__ constexpr int sk_pad64(int n) { return (n + 63) / 64 * 64; }

// G64: gs = 64, so every K step is a whole group, rescaled as soon as its MFMAs are done (no int32 sums carried
// from step to step, no group index to divide out). SW: some segment is SWIGLU; without it the kernel holds no W3
// registers at all, and with it every block loads its W3 operand registers unconditionally (from an empty buffer when
// its own segment has no W3: zeros, no memory traffic), so no load is left pending on a conditionally kept register.
template <int MT, int NT, int WAVES, bool G64, bool SW>
__global__ __launch_bounds__(64 * WAVES, 2) void q8_gemm_skinny(SkParams p) {
  constexpr int RB = 16 * NT; // weight rows of the block: NT MFMA tiles of 16 sharing each activation load
  extern __shared__ __align__(16) float sk_smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = blockIdx.x;
  int s = 0;
  while (s + 1 < p.nseg && tile >= p.seg[s + 1].first_tile)
    s++;
  const SkSeg seg = sk_pick(p, s);
  const bool swiglu = SW && seg.epi == EPI_SWIGLU;
  const int col0 = (tile - seg.first_tile) * RB;
  const int G = p.groups, spg = p.gs / 64;

  // Scales of the block's RB weight rows (and their W3 rows), all groups, as they lie in memory (row r's group g at
  // r * G + g: one contiguous range), and of the activation rows group-major (group g's at g * 16 MT + r), so a lane
  // reads the four activation rows of its elements at once. They go global -> LDS by DMA, one scale per lane and 64
  // per load (each region padded to whole loads; a padding lane reads past its buffer: zero), before the first weight
  // loads and without waiting on either: a register copy waits for each load in turn, a dozen memory latencies
  // before the block's first weight load. (Weight scales gathered group-major took 16 cache lines per load where the
  // contiguous copy takes two.)
  const int nw = sk_pad64(RB * G), nx = sk_pad64(16 * MT * G);
  float *sws = sk_smem, *sw3s = sws + nw, *sxs = sw3s + (SW ? nw : 0);
  {
    constexpr unsigned kPast = 1u << 30; // past any scale buffer here (at most 2^23 bytes on this path)
    const long long wrows = (long long)min(RB, seg.n - col0);
    const __amdgpu_buffer_rsrc_t rws = sk_buffer(seg.ws + (long long)col0 * G, wrows * G * 4);
    const __amdgpu_buffer_rsrc_t rw3s = sk_buffer(swiglu ? seg.w3s + (long long)col0 * G : seg.ws, swiglu ? wrows * G * 4 : 0);
    const __amdgpu_buffer_rsrc_t rxs = sk_buffer(p.xs, (long long)p.m * G * 4);
    for (int base = 64 * wave; base < nw; base += 64 * WAVES) { // entry base + lane, a straight copy
      const int i = base + lane;
      const unsigned off = i < RB * G ? (unsigned)i * 4u : kPast;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rws, (__attribute__((address_space(3))) void *)(sws + base), 4, off, 0,
                                               0, 0);
      if constexpr (SW)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw3s, (__attribute__((address_space(3))) void *)(sw3s + base), 4,
                                                 off, 0, 0, 0);
    }
    for (int base = 64 * wave; base < nx; base += 64 * WAVES) { // activation row r >= m: past the buffer, zero
      const int i = base + lane, g = i / (16 * MT), r = i % (16 * MT);
      const unsigned off = i < 16 * MT * G ? (unsigned)(r * G + g) * 4u : kPast;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rxs, (__attribute__((address_space(3))) void *)(sxs + base), 4, off, 0,
                                               0, 0);
    }
  }

  // this wave's K steps [s0, s1); steps past s1 load zeros
  const int s0 = wave * p.per, s1 = min(p.steps, s0 + p.per);
  const long long k = p.k;
  __amdgpu_buffer_rsrc_t rB[NT], rB3[NT]; // weight tile j: rows col0 + 16 j .. (none past n: zero bytes)
#pragma unroll
  for (int j = 0; j < NT; j++) {
    const int c = min(col0 + 16 * j, seg.n);
    const long long wrows = (long long)min(16, seg.n - c);
    rB[j] = sk_buffer(seg.w + (long long)c * k, wrows * k);
    rB3[j] = sk_buffer(swiglu ? seg.w3 + (long long)c * k : seg.w, swiglu ? wrows * k : 0);
  }
  const __amdgpu_buffer_rsrc_t rA = sk_buffer(p.xq, (long long)p.m * k);
  const __amdgpu_buffer_rsrc_t none = sk_buffer(p.xq, 0);
  const int off = (int)((lane & 15) * k) + (lane >> 4) * 16; // MFMA operand: row lane % 16, K bytes 16 (lane / 16) ..
  // Weights two K steps at a time: load X takes rows 0-7 and Y rows 8-15, each row's 128 bytes whole (lane l: row
  // l % 8, 16-byte chunk l / 16 + 4 ((l % 16) / 8), so lanes 0-7 of each 16-lane row hold the first step's chunk and
  // lanes 8-15 the second's). A pair may reach past the wave's range or the row's end: the activations of such a step
  // read zero, so whatever weight bytes it holds add nothing.
  const int chunk = (lane >> 4) + 4 * ((lane >> 3) & 1);
  const int offX = (int)((lane & 7) * k) + 16 * chunk, offY = offX + (int)(8 * k);

  v4i x[kSkPairs][NT], y[kSkPairs][NT], x3[kSkPairs][NT], y3[kSkPairs][NT], a[kSkPairs][2][MT];
  auto issue = [&](int st, int d) { // steps st and st + 1
    const bool live = st < s1;
    const int k0 = st * 64;
#pragma unroll
    for (int j = 0; j < NT; j++) {
      x[d][j] = __builtin_amdgcn_raw_buffer_load_b128(live ? rB[j] : none, offX, k0, kStream);
      y[d][j] = __builtin_amdgcn_raw_buffer_load_b128(live ? rB[j] : none, offY, k0, kStream);
      if constexpr (SW) {
        x3[d][j] = __builtin_amdgcn_raw_buffer_load_b128(live ? rB3[j] : none, offX, k0, kStream);
        y3[d][j] = __builtin_amdgcn_raw_buffer_load_b128(live ? rB3[j] : none, offY, k0, kStream);
      }
    }
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int t = 0; t < MT; t++)
        a[d][h][t] =
            __builtin_amdgcn_raw_buffer_load_b128(st + h < s1 ? rA : none, off + (int)(16 * t * k), k0 + 64 * h, 0);
  };
#pragma unroll
  for (int d = 0; d < kSkPairs; d++)
    issue(s0 + 2 * d, d);
  // this wave's scale loads are older than its operand loads: wait for them alone, then for every wave's
  constexpr int kPairLoads = 2 * NT * (SW ? 2 : 1) + 2 * MT;
  sk_wait_vmcnt<kSkPairs * kPairLoads>();
  __syncthreads(); // the scales are staged

  v4f acc[MT][NT], acc3[MT][NT];
  v4i dot[MT][NT], dot3[MT][NT];
#pragma unroll
  for (int t = 0; t < MT; t++)
#pragma unroll
    for (int j = 0; j < NT; j++) {
      acc[t][j] = acc3[t][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      dot[t][j] = dot3[t][j] = v4i{0, 0, 0, 0};
    }
  // The operand of step h of a pair (row lane % 16, chunk lane / 16): X with lanes 8-15 of each 16-lane row taken from
  // Y's lanes 0-7 (h = 0, DPP row_shr:8 into banks 2-3), or Y with lanes 0-7 taken from X's lanes 8-15 (h = 1,
  // row_shl:8 into banks 0-1).
  auto operand = [&](const v4i &lo, const v4i &hi, int h) {
    v4i r;
#pragma unroll
    for (int e = 0; e < 4; e++)
      r[e] = h == 0 ? __builtin_amdgcn_update_dpp(lo[e], hi[e], 0x118, 0xF, 0xC, false)
                    : __builtin_amdgcn_update_dpp(hi[e], lo[e], 0x108, 0xF, 0x3, false);
    return r;
  };
  const int lr = (lane >> 4) * 4, lc = lane & 15;
  // group g's scales of this lane's elements: activation rows 16 t + lr + e (one 16-byte read per tile), weight rows
  // 16 j + lc
  auto xscales = [&](int g, int t) { return *reinterpret_cast<const v4f *>(sxs + g * 16 * MT + 16 * t + lr); };
  if constexpr (G64) {
    // whole rounds of kSkPairs pairs (the ring's slots are constants); steps past s1 multiply zero activations, and
    // their (any) group's scales leave the sums as they are
    for (int step = s0; step < s1; step += 2 * kSkPairs) {
#pragma unroll
      for (int d = 0; d < kSkPairs; d++) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const int g = min(step + 2 * d + h, G - 1);
          v4f xsc[MT];
#pragma unroll
          for (int t = 0; t < MT; t++)
            xsc[t] = xscales(g, t);
#pragma unroll
          for (int j = 0; j < NT; j++) {
            const v4i b = operand(x[d][j], y[d][j], h);
            const float wsc = sws[(16 * j + lc) * G + g];
#pragma unroll
            for (int t = 0; t < MT; t++) {
              const v4i dd = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[d][h][t], b, v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
              for (int e = 0; e < 4; e++)
                acc[t][j][e] = fmaf((float)dd[e] * wsc, xsc[t][e], acc[t][j][e]);
            }
            if (swiglu) {
              const v4i b3 = operand(x3[d][j], y3[d][j], h);
              const float w3sc = sw3s[(16 * j + lc) * G + g];
#pragma unroll
              for (int t = 0; t < MT; t++) {
                const v4i dd3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[d][h][t], b3, v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; e++)
                  acc3[t][j][e] = fmaf((float)dd3[e] * w3sc, xsc[t][e], acc3[t][j][e]);
              }
            }
          }
          if (h == 1) { // the pair's registers are free: its next loads go out here, not after the round's MFMAs
            __builtin_amdgcn_sched_barrier(0);
            issue(step + 2 * d + 2 * kSkPairs, d);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    }
  } else
  // whole rounds of kSkPairs pairs (the ring's slots are constants); steps past s1 multiply zero activations
  for (int step = s0; step < s1; step += 2 * kSkPairs) {
#pragma unroll
    for (int d = 0; d < kSkPairs; d++) {
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int st = step + 2 * d + h;
        const bool first = st % spg == 0, last = st % spg == spg - 1;
#pragma unroll
        for (int j = 0; j < NT; j++) {
          const v4i b = operand(x[d][j], y[d][j], h);
          v4i b3 = b;
          if (swiglu)
            b3 = operand(x3[d][j], y3[d][j], h);
#pragma unroll
          for (int t = 0; t < MT; t++) {
            dot[t][j] =
                __builtin_amdgcn_mfma_i32_16x16x64_i8(a[d][h][t], b, first ? v4i{0, 0, 0, 0} : dot[t][j], 0, 0, 0);
            if (swiglu)
              dot3[t][j] =
                  __builtin_amdgcn_mfma_i32_16x16x64_i8(a[d][h][t], b3, first ? v4i{0, 0, 0, 0} : dot3[t][j], 0, 0, 0);
          }
        }
        if (h == 1)
          issue(step + 2 * d + 2 * kSkPairs, d);
        if (last) {
          const int g = min(st / spg, G - 1); // past the end the dots are zero; any group's scales will do
#pragma unroll
          for (int j = 0; j < NT; j++) {
            const float wsc = sws[(16 * j + lc) * G + g], w3sc = sw3s[(16 * j + lc) * G + g];
#pragma unroll
            for (int t = 0; t < MT; t++) {
              const v4f xsc = xscales(g, t);
#pragma unroll
              for (int e = 0; e < 4; e++) {
                acc[t][j][e] = fmaf((float)dot[t][j][e] * wsc, xsc[e], acc[t][j][e]);
                if (swiglu)
                  acc3[t][j][e] = fmaf((float)dot3[t][j][e] * w3sc, xsc[e], acc3[t][j][e]);
              }
            }
          }
        }
      }
    }
  }

  // the waves' partial sums, added in wave order, in the scales' place once every wave is past its last step
  constexpr int kParts = MT * NT * 4; // (activation tile, weight tile, element) of each lane
  float *red = sk_smem;               // [wave][part][lane], then the same for W3
  const int red3 = WAVES * kParts * 64;
  __syncthreads();
#pragma unroll
  for (int t = 0; t < MT; t++)
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int part = (t * NT + j) * 4 + e;
        red[(wave * kParts + part) * 64 + lane] = acc[t][j][e];
        if (swiglu)
          red[red3 + (wave * kParts + part) * 64 + lane] = acc3[t][j][e];
      }
  __syncthreads();
  // wave w finishes parts w, w + WAVES, ... of every lane
  for (int part = wave; part < kParts; part += WAVES) {
    const int t = part / (4 * NT), j = part / 4 % NT, e = part % 4;
    float total = 0.0f, gate = 0.0f;
    for (int w = 0; w < WAVES; w++) {
      total += red[(w * kParts + part) * 64 + lane];
      if (swiglu)
        gate += red[red3 + (w * kParts + part) * 64 + lane];
    }
    const int row = 16 * t + lr + e, col = col0 + 16 * j + lc;
    if (row >= p.m || col >= seg.n)
      continue;
    float *o = seg.c + (long long)row * seg.ldc + col;
    if (swiglu)
      *o = sk_silu_gate(total, gate);
    else if (seg.epi == EPI_ADD)
      *o += total;
    else
      *o = total;
  }
}

// LDS bytes: the staged scales (W3's only with a SWIGLU segment), or the waves' partial sums where they go after the
// loop, whichever is more
size_t skinny_lds(int mt, int nt, int waves, int groups, bool sw) {
  const size_t scales = (size_t)sk_pad64(16 * nt * groups) * (sw ? 2 : 1) + sk_pad64(16 * mt * groups);
  const size_t sums = (size_t)waves * mt * nt * 4 * 64 * (sw ? 2 : 1);
  return (scales > sums ? scales : sums) * sizeof(float);
}

template <int MT, int NT, int WAVES, bool G64, bool SW>
bool skinny_launch_gs(const SkParams &p, int tiles, hipStream_t stream) {
  static const hipError_t status = hipFuncSetAttribute((const void *)q8_gemm_skinny<MT, NT, WAVES, G64, SW>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (!check_hip(status, "allowing the skinny Q8 GEMM its LDS"))
    return false;
  hipLaunchKernelGGL((q8_gemm_skinny<MT, NT, WAVES, G64, SW>), dim3((unsigned)tiles), dim3(64 * WAVES),
                     skinny_lds(MT, NT, WAVES, p.groups, SW), stream, p);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess || raise("launching q8_gemm_skinny failed: %s", hipGetErrorString(e));
}

template <int MT, int NT, int WAVES> bool skinny_launch(const SkParams &p, int tiles, hipStream_t stream) {
  bool sw = false;
  for (int s = 0; s < p.nseg; s++)
    sw = sw || p.seg[s].epi == EPI_SWIGLU;
  if (sw)
    return p.gs == 64 ? skinny_launch_gs<MT, NT, WAVES, true, true>(p, tiles, stream)
                      : skinny_launch_gs<MT, NT, WAVES, false, true>(p, tiles, stream);
  return p.gs == 64 ? skinny_launch_gs<MT, NT, WAVES, true, false>(p, tiles, stream)
                    : skinny_launch_gs<MT, NT, WAVES, false, false>(p, tiles, stream);
}

} // namespace

// Shapes the skinny kernel takes: at most 32 rows, gs a multiple of 64, 16-byte aligned rows, scales that fit LDS.
bool q8_gemm_skinny_path(const int8_t *xq, int m, int k, int gs) {
  return m > 0 && m <= 32 && gs > 0 && gs % 64 == 0 && k % gs == 0 && ((uintptr_t)xq & 15) == 0 &&
         32LL * k < (1LL << 31) && skinny_lds(m > 16 ? 2 : 1, 1, 8, k / gs, true) <= 160 * 1024;
}

bool launch_q8_gemm_skinny(const GemmQ8Job &job, hipStream_t stream) {
  const int mt = job.m > 16 ? 2 : 1, groups = job.k / job.gs;
  int tiles16 = 0;
  for (int s = 0; s < job.nseg; s++)
    tiles16 += (job.seg[s].n + 15) / 16;
  // Two weight tiles per block halve the activation loads. That pays once the activations are 32 rows and the grid
  // keeps at least 192 blocks (8B, m = 32: QKV 21.1 -> 16.6 us, W1/W3 43.9 -> 36.7 us); on the 256-tile W2 and Wo it
  // leaves half the CUs idle (W2 16.4 -> 29.0 us at m = 1).
  const int nt = mt == 2 && tiles16 >= 384 && skinny_lds(mt, 2, 8, groups, true) <= 160 * 1024 ? 2 : 1;
  SkParams p{};
  int tiles = 0;
  for (int s = 0; s < job.nseg; s++) {
    const GemmSegmentDev &d = job.seg[s];
    p.seg[s] = SkSeg{d.c, d.ldc, (const int8_t *)d.w, (const int8_t *)d.w3, d.ws, d.w3s, d.n, d.epi, tiles};
    tiles += (d.n + 16 * nt - 1) / (16 * nt);
  }
  if (tiles <= 0)
    return true;
  p.nseg = job.nseg;
  p.xq = job.xq;
  p.xs = job.xs;
  p.m = job.m;
  p.k = job.k;
  p.gs = job.gs;
  p.groups = groups;
  p.steps = job.k / 64;
  // Waves per block split K: eight for grids of fewer than 512 column tiles (W2, Wo: 256), four otherwise (W1/W3: 896),
  // which measured best on the 8B shapes (W2 17.5 vs 24.0 us with four; W1/W3 29.4 vs 31.6 with eight).
  const int waves = tiles16 < 512 ? 8 : 4, spg = job.gs / 64;
  p.per = ((p.steps + waves - 1) / waves + spg - 1) / spg * spg;
  if (nt == 2)
    return waves == 8 ? skinny_launch<2, 2, 8>(p, tiles, stream) : skinny_launch<2, 2, 4>(p, tiles, stream);
  if (mt == 1)
    return waves == 8 ? skinny_launch<1, 1, 8>(p, tiles, stream) : skinny_launch<1, 1, 4>(p, tiles, stream);
  return waves == 8 ? skinny_launch<2, 1, 8>(p, tiles, stream) : skinny_launch<2, 1, 4>(p, tiles, stream);
}

} // namespace llhip
