// Batched-prefill GEMMs for gfx950 on MFMA: W8A8 Q8_0 on int8 MFMA, FP32 on FP32 MFMA, BF16 on BF16 MFMA.
//
// All compute C[m][n] (op)= A[m][k] . W[n][k]^T over up to three segments that share A, with the epilogues STORE,
// ADD and SWIGLU (a column tile then holds columns of W1 and the same columns of W3, so the gate is applied in
// registers). The kernels, each described where it is defined:
//   q8_gemm_lds     int8, 256 x 128 tiles (or 128 x 128), A/B/scales streamed into LDS five stages deep;
//   mm_gemm_lds     FP32 and BF16, 256 x 128 tiles, the same pipeline;
//   bf16_gemm_wide  BF16, 256 x 256 tiles for large grids;
//   split_reduce    the second kernel of a split-K launch of the int8 and wide kernels;
//   f32_gemm_mfma   FP32 shapes the pipeline does not take (K % 16 != 0, unaligned rows): 128 x 128 tiles staged
//                   through registers into double-buffered LDS;
//   q8_gemm_generic int8 with a group size that is not a multiple of 64.
// Each wave owns 64 x 64 (64 x 128 in the wide kernel) as a grid of 16 x 16 MFMA tiles. MFMA operand loads are
// symmetric (lane l supplies row l % 16 of A and column l % 16 of W with the same K slice), so the dot products do not
// depend on how the instruction orders K inside a lane; the 16 x 16 result holds C[4 (l / 16) + e][l % 16] in element
// e of lane l.
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <vector>

#include "common.h"
#include "lanes.h"
#include "quant.h"

namespace llhip {
namespace {

constexpr int kBlock = 256;
constexpr int kTile = 128; // block tile rows and columns of f32_gemm_mfma

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float silu_gate(float value, float gate) {
  value *= (1.0f / (1.0f + expf(-value)));
  return value * gate;
}

struct TileSeg {
  float *c;
  int ldc;
  const void *w, *w3;
  const float *ws, *w3s;
  long long ldw;
  int n;
  int epi;
  int first_tile; // first logical tile of this segment
  int ntiles;     // its column tiles
  int8_t *cq;     // SWIGLU output quantized in groups of 64 (the wide int8 kernel only), else null
  float *cs;
};

struct TileGrid {
  TileSeg seg[3];
  int nseg;
  int mtiles;
  int total;
};

// Blocks go to the eight XCDs round-robin (block b on XCD b % 8). Renumbering gives every XCD a contiguous run of
// logical tiles, and logical tiles walk M fastest, so the blocks that share a weight tile meet in one XCD's L2.
__device__ __forceinline__ int xcd_logical(int b, int total) {
  const int q = total / 8, r = total % 8, xcd = b % 8, pos = b / 8;
  return xcd < r ? xcd * (q + 1) + pos : r * (q + 1) + (xcd - r) * q + pos;
}

struct TilePos {
  int s, m0, n0;
  bool swiglu;
};

__device__ __forceinline__ TilePos tile_of(const TileGrid &g, int logical) {
  int s = 0;
  while (s + 1 < g.nseg && logical >= g.seg[s + 1].first_tile)
    s++;
  const int local = logical - g.seg[s].first_tile;
  TilePos t;
  t.s = s;
  t.swiglu = g.seg[s].epi == EPI_SWIGLU;
  t.m0 = (local % g.mtiles) * kTile;
  t.n0 = (local / g.mtiles) * (t.swiglu ? kTile / 2 : kTile);
  return t;
}

__device__ __forceinline__ TileSeg seg_of(const TileGrid &g, int s) { return s == 0 ? g.seg[0] : s == 1 ? g.seg[1] : g.seg[2]; }

// Row r (0..127) of the block's B tile: which weight matrix and which output column it feeds.
__device__ __forceinline__ int b_col(const TilePos &t, int r) { return t.swiglu ? t.n0 + (r & 63) : t.n0 + r; }

// The B-tile row a wave's column tile j reads: waves split columns 64/64, or 32/32 of W1 and W3 under SWIGLU.
__device__ __forceinline__ int b_row(bool swiglu, int wn, int j) {
  return swiglu ? (j < 2 ? 32 * wn + 16 * j : 64 + 32 * wn + 16 * (j - 2)) : 64 * wn + 16 * j;
}

__device__ __forceinline__ void store_tile(const TileSeg &seg, const TilePos &t, const v4f (&acc)[4][4], int wm, int wn,
                                           int lane, int m) {
  const int lc = lane & 15, lr = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int row = t.m0 + wm * 64 + 16 * i + lr + e;
      if (row >= m)
        continue;
      float *crow = seg.c + (long long)row * seg.ldc;
      if (t.swiglu) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
          const int col = t.n0 + 32 * wn + 16 * j + lc;
          if (col < seg.n)
            crow[col] = silu_gate(acc[i][j][e], acc[i][j + 2][e]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int col = t.n0 + 64 * wn + 16 * j + lc;
          if (col >= seg.n)
            continue;
          if (seg.epi == EPI_ADD)
            crow[col] += acc[i][j][e];
          else
            crow[col] = acc[i][j][e];
        }
      }
    }
}

// The 256 x 128 int8 tile's SWIGLU epilogue with seg.cq set: a tile's 64 outputs of a row are one quantization group,
// 32 in each of the row's two waves (wn). Each wave takes its 32 values' maximum (the row's 16 lanes by a DPP row
// reduction), the two meet in LDS (`xchg`, free once every wave has left the K loop), and each quantizes its values
// with the group's scale by the k_quantize rule, as store_tile_wide does (bitwise the FP32 output then
// k_quantize_rows); a non-finite value sets flags[0]. Every wave of the block calls it (two barriers).
__device__ __forceinline__ void store_tile_quantized(const TileSeg &seg, const TilePos &t, const v4f (&acc)[4][4],
                                                     int wm, int wn, int lane, int m, float *xchg, int *flags) {
  const int lc = lane & 15, lr = (lane >> 4) * 4;
  // two passes over the sums (the SwiGLU values formed twice) so that only the sums stay live across the barriers
  __syncthreads(); // every wave is past its K loop: the LDS is free
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      float pk = 0.0f;
#pragma unroll
      for (int j = 0; j < 2; j++)
        pk = fmaxf(pk, fabsf(silu_gate(acc[i][j][e], acc[i][j + 2][e]))); // a NaN: caught by quantize_fast
      pk = group_reduce_max(pk, 16);
      if (lc == 0)
        xchg[(wm * 64 + 16 * i + lr + e) * 2 + wn] = pk;
    }
  __syncthreads();
  const int c0 = t.n0; // the tile's group (seg.n % 64 == 0)
  const int groups = seg.ldc / 64; // row strides of cq and cs: the whole width (a tail segment has its share)
  bool bad = false;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int r = wm * 64 + 16 * i + lr + e, row = t.m0 + r;
      const float scale = fmaxf(xchg[r * 2], xchg[r * 2 + 1]) / 127.0f;
      bool ok;
      const float inv = group_reciprocal(scale, ok);
      float v[2];
#pragma unroll
      for (int j = 0; j < 2; j++)
        v[j] = silu_gate(acc[i][j][e], acc[i][j + 2][e]);
      int q[2];
      quantize_fast(v, scale, inv, ok, q, bad);
      if (row < m && c0 < seg.n) {
        int8_t *qrow = seg.cq + (long long)row * seg.ldc;
#pragma unroll
        for (int j = 0; j < 2; j++)
          qrow[c0 + 32 * wn + 16 * j + lc] = (int8_t)q[j];
        if (wn == 0 && lc == 0)
          seg.cs[(long long)row * groups + c0 / 64] = scale;
      }
    }
  if (bad && flags)
    flags[0] = 1;
}

// The wide BF16 tile's epilogue: rows 64 wm + 16 i + 4 (l / 16) + e, columns 128 wn + 16 j + l % 16, or under SWIGLU
// silu(W1 column 64 wn + 16 j + l % 16) * (the same W3 column) from tiles j and j + 4. With seg.cq set (SWIGLU, the
// int8 kernel) a wave's 64 columns of a row are one quantization group, held by the 16 lanes of the row's lane group:
// their maximum is a DPP row reduction, and the values go out by the k_quantize rule as int8 with the group's scale
// (bitwise the FP32 output then k_quantize_rows); a non-finite value sets flags[0].
__device__ __forceinline__ void store_tile_wide(const TileSeg &seg, const TilePos &t, const v4f (&acc)[4][8], int wm,
                                                int wn, int lane, int m, int *flags = nullptr) {
  const int lc = lane & 15, lr = (lane >> 4) * 4;
  if (t.swiglu && seg.cq) {
    const int c0 = t.n0 + 64 * wn; // the wave's group (seg.n % 64 == 0)
    const int groups = seg.ldc / 64; // row strides of cq and cs: the whole width (a tail segment has its share)
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int row = t.m0 + wm * 64 + 16 * i + lr + e;
        float v[4];
        float peak = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          v[j] = silu_gate(acc[i][j][e], acc[i][j + 4][e]);
          peak = fmaxf(peak, fabsf(v[j])); // a NaN is skipped here and caught by quantize_fast
        }
        peak = group_reduce_max(peak, 16);
        const float scale = peak / 127.0f;
        bool ok;
        const float inv = group_reciprocal(scale, ok);
        int q[4];
        quantize_fast(v, scale, inv, ok, q, bad);
        if (row < m && c0 < seg.n) {
          int8_t *qrow = seg.cq + (long long)row * seg.ldc;
#pragma unroll
          for (int j = 0; j < 4; j++)
            qrow[c0 + 16 * j + lc] = (int8_t)q[j];
          if (lc == 0)
            seg.cs[(long long)row * groups + c0 / 64] = scale;
        }
      }
    if (bad && flags)
      flags[0] = 1;
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int row = t.m0 + wm * 64 + 16 * i + lr + e;
      if (row >= m)
        continue;
      float *crow = seg.c + (long long)row * seg.ldc;
      if (t.swiglu) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int col = t.n0 + 64 * wn + 16 * j + lc;
          if (col < seg.n)
            crow[col] = silu_gate(acc[i][j][e], acc[i][j + 4][e]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const int col = t.n0 + 128 * wn + 16 * j + lc;
          if (col >= seg.n)
            continue;
          if (seg.epi == EPI_ADD)
            crow[col] += acc[i][j][e];
          else
            crow[col] = acc[i][j][e];
        }
      }
    }
}

// ---- W8A8 Q8_0: the pipelined int8-MFMA kernel ------------------------------------------------------------------------
//
// 512 threads own a 256 x 128 output tile (a 128-column tile holds 64 columns of W1 and the same 64 of W3 under
// SWIGLU); eight waves in 4 x 2 each own 64 x 64 as 4 x 4 v_mfma_i32_16x16x64_i8 tiles. A K step is 64 values. Its A
// and B tiles (256 x 64 and 128 x 64 int8) and their group scales travel from global memory straight into LDS with
// buffer loads (no register staging), four steps ahead: at step s the block waits for step s + 1's loads, then issues
// step s + 4's into the stage step s - 1 used.
//
// LDS holds 16-row blocks of 1 KB: A block b of stage t at (b * 5 + t) KB, B blocks after the A ones likewise, so a
// wave's operand reads of any stage are one base register plus an immediate, and the K loop, unrolled by the five
// stages, spends no vector instructions on addresses. A block row is 64 bytes whose four 16-byte chunks are
// XOR-swizzled by (row / 2) % 4, so the MFMA operand reads (16 rows, one chunk each) fall on distinct banks.
//
// One set of int32 results per wave: at a group's last step, tile by tile, the results are converted, the tile's MFMA
// of the next step overwrites them, and ((float)dot * ws) * xs is added to the FP32 accumulator from the converted
// copy, so each wave keeps the matrix pipe and the VALU busy together; inside a group (gs > 64) the next step's MFMA
// accumulates onto the results instead.
constexpr int kQ8Waves = 8, kQ8Threads = 64 * kQ8Waves;
constexpr int kQ8TileM = 256, kQ8TileN = 128, kQ8Stages = 5;
constexpr int kQ8ABlocks = kQ8TileM / 16, kQ8BBlocks = kQ8TileN / 16; // 1 KB blocks per stage
constexpr int kQ8BOff = kQ8ABlocks * kQ8Stages * 1024;               // B blocks after the A blocks
constexpr int kQ8SOff = kQ8BOff + kQ8BBlocks * kQ8Stages * 1024;     // then the scales, a group per stage
constexpr int kQ8SStride = (kQ8TileM + kQ8TileN + 64) * 4;            // xs, ws, spare (zero-length loads land there)
constexpr size_t kQ8Lds = (size_t)kQ8SOff + (size_t)kQ8Stages * kQ8SStride;

// The int8 kernel's tile shapes: WM rows of 64 x 64 wave tiles over 128 columns. WM = 4 is the layout above (one
// 129 KB block per CU); WM = 2 is a 128 x 128 tile of four waves with four stages (69 KB), two blocks per CU, so a
// block waiting at its barrier or for its loads leaves the SIMDs to the other block's waves.
template <int WM_, int STAGES_> struct Q8Cfg {
  static constexpr int WM = WM_, Waves = 2 * WM, Threads = 64 * Waves;
  static constexpr int TileM = 64 * WM, TileN = 128, Stages = STAGES_;
  static constexpr int ABlocks = TileM / 16, BBlocks = TileN / 16;
  static constexpr int BPerWave = BBlocks / Waves;         // B blocks each wave loads per step
  static constexpr int LoadsPerStep = 2 + BPerWave + 1;    // two A, the B blocks, one scale load
  static constexpr int BOff = ABlocks * Stages * 1024;
  static constexpr int SOff = BOff + BBlocks * Stages * 1024;
  static constexpr int SStride = (TileM + TileN + 64) * 4; // xs, ws, spare (zero-length loads land there)
  static constexpr size_t Lds = (size_t)SOff + (size_t)Stages * SStride;
  static_assert(BBlocks % Waves == 0 && (TileM + TileN) / 64 <= Waves, "every load has a wave");
};
using Q8Wide = Q8Cfg<4, 5>;
using Q8Pair = Q8Cfg<2, 4>;
static_assert(Q8Wide::Lds == kQ8Lds, "the 256 x 128 layout");
static_assert(2 * Q8Pair::Lds <= 160 * 1024, "two 128 x 128 blocks fit one CU's LDS");

__device__ __forceinline__ int q8_swizzle(int row) { return (row >> 1) & 3; }

struct Q8Grid {
  TileSeg seg[3];
  int nseg;
  int mtiles;
  int total;
};

constexpr int kSplitSlots = LLHIP_SPLIT_SLOTS; // partial tiles the workspace holds

struct SplitK {
  v4f *partial;    // [tile * splits + split][16][threads] partial sums, in the accumulators' register order
  unsigned *count; // [tile] blocks arrived; zero between launches
  int splits;      // blocks per tile (1: no split)
  int per;         // K steps per split
};

struct Q8Params {
  Q8Grid grid;
  const int8_t *xq;
  const float *xs;
  int m, k, gs;
  int32_t *probe; // optional (one segment, no SWIGLU): probe[(g * m + r) * n + c]
  SplitK sk;
  int *flags; // [0]: a non-finite value met by a quantizing epilogue
};

__device__ __forceinline__ TilePos q8_tile_of(const Q8Grid &g, int logical, int tile_m = kQ8TileM,
                                              int tile_n = kQ8TileN) {
  int s = 0;
  while (s + 1 < g.nseg && logical >= g.seg[s + 1].first_tile)
    s++;
  const int local = logical - g.seg[s].first_tile;
  TilePos t;
  t.s = s;
  t.swiglu = g.seg[s].epi == EPI_SWIGLU;
  t.m0 = (local % g.mtiles) * tile_m;
  t.n0 = (local / g.mtiles) * (t.swiglu ? tile_n / 2 : tile_n);
  return t;
}

__device__ __forceinline__ TileSeg q8_seg_of(const Q8Grid &g, int s) {
  return s == 0 ? g.seg[0] : s == 1 ? g.seg[1] : g.seg[2];
}

// A buffer resource from wave-uniform values, built from scalar registers (readfirstlane states the uniformity the
// compiler cannot always prove; a resource in vector registers would make every load a loop over lanes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t q8_buffer(const void *base, long long bytes) {
  const unsigned long long b = (unsigned long long)(uintptr_t)base;
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)b);
  const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(b >> 32));
  const int n = __builtin_amdgcn_readfirstlane((int)(bytes > 0 ? bytes : 0));
  return __builtin_amdgcn_make_buffer_rsrc((void *)(uintptr_t)(((unsigned long long)hi << 32) | lo), (short)0, n,
                                           0x00020000);
}

// s_waitcnt with vmcnt = n and the other counters left alone (gfx9 encoding: vmcnt bits 3:0 and 15:14).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}
// The same with lgkmcnt = 0 too (every LDS access of this thread done).
template <int N> __device__ __forceinline__ void wait_vmcnt_lgkm0() {
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | ((N >> 4) << 14));
}

// Split K: a grid with fewer tiles than CUs runs each tile as `splits` blocks over consecutive K ranges, each writing
// its partial tile to a device workspace. The partials are added in split order, so results do not depend on timing:
// by split_reduce, a second kernel (int8 and wide BF16 kernels, which have no registers to spare), or by the last of
// the tile's blocks to arrive (split_combine, the FP32 / BF16 kernel), which counts the arrivals and puts the counter
// back to zero.

// Cache policy of the partial tiles' stores and loads: device-coherent (sc1), so a store is written through past the
// XCD's L2 before its completion is counted, and a load reads from past it. No cache-wide write-back or invalidate is
// needed, which would also evict the operands of every other block on the XCD.
constexpr int kDeviceCoherent = 16;

// The last of a tile's blocks to arrive gets true with acc holding the whole sum; the others get false.
template <int THREADS>
__device__ __forceinline__ bool split_combine(const SplitK &sk, int tile, int split, v4f (&acc)[4][4]) {
  __shared__ int last;
  const int tid = threadIdx.x;
  constexpr int kSlotBytes = 16 * THREADS * 16; // one partial tile
  const __amdgpu_buffer_rsrc_t r =
      q8_buffer((const unsigned char *)sk.partial + (size_t)tile * sk.splits * kSlotBytes, (long long)sk.splits * kSlotBytes);
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, acc[i][j]), r,
                                             split * kSlotBytes + ((i * 4 + j) * THREADS + tid) * 16, 0,
                                             kDeviceCoherent);
  __builtin_amdgcn_s_waitcnt(0); // this thread's partial sums have reached the device-coherent level
  __syncthreads();               // ... and every thread's
  if (tid == 0)
    last = __hip_atomic_fetch_add(&sk.count[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           (unsigned)(sk.splits - 1);
  __syncthreads();
  if (!last)
    return false;
  v4f own[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
      own[i][j] = acc[i][j];
  for (int s = 0; s < sk.splits; s++) {
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const v4f v = s == split ? own[i][j]
                                 : __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(
                                                               r, s * kSlotBytes + ((i * 4 + j) * THREADS + tid) * 16,
                                                               0, kDeviceCoherent));
        acc[i][j] = s == 0 ? v : acc[i][j] + v;
      }
  }
  if (tid == 0)
    __hip_atomic_store(&sk.count[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// The second kernel of a split launch whose kernel wrote partial tiles (the int8 and the wide BF16 kernels): thread by
// thread over every tile's partial sums. A thread takes one accumulator pair, tiles j and j + J/2 of row tile i of
// one lane of the block layout (the SWIGLU pair, or two plain column tiles), adds the splits in order and applies the
// epilogue to its four rows. Partial tile layout: [tile][split][i * J + j][THREADS] v4f.
struct SplitOut {
  Q8Grid grid;
  const v4f *partial;
  int splits, m, tile_m, tile_n;
};

template <int J, int THREADS> __global__ __launch_bounds__(256) void split_reduce(SplitOut p) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long per_tile = 4LL * (J / 2) * THREADS;
  if (idx >= per_tile * p.grid.total)
    return;
  const int tile = (int)(idx / per_tile), rest = (int)(idx % per_tile);
  const int tid = rest % THREADS, jp = (rest / THREADS) % (J / 2), i = rest / THREADS / (J / 2);
  const TilePos t = q8_tile_of(p.grid, tile, p.tile_m, p.tile_n);
  const TileSeg seg = q8_seg_of(p.grid, t.s);
  const v4f *part = p.partial + (size_t)tile * p.splits * (4 * J * THREADS) + tid;
  // The partials are added in split order; they are loaded kBatch splits at a time, all in flight together (a loop
  // that adds each as it arrives waits for one load per split). Past the last split a load repeats the last one and
  // its sum is not taken.
  constexpr int kBatch = 8;
  const size_t lo_at = (size_t)(i * J + jp) * THREADS, hi_at = (size_t)(i * J + jp + J / 2) * THREADS;
  v4f lo{}, hi{};
  for (int s0 = 0; s0 < p.splits; s0 += kBatch) {
    v4f l[kBatch], h[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; u++) {
      const size_t at = (size_t)min(s0 + u, p.splits - 1) * (4 * J * THREADS);
      l[u] = part[at + lo_at];
      h[u] = part[at + hi_at];
    }
#pragma unroll
    for (int u = 0; u < kBatch; u++) {
      if (s0 + u == 0) {
        lo = l[u];
        hi = h[u];
      } else if (s0 + u < p.splits) {
        lo += l[u];
        hi += h[u];
      }
    }
  }
  const int lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
  const int lc = lane & 15, lr = (lane >> 4) * 4;
  constexpr int kSpan = 16 * J; // columns a wave covers
  const int rows = min(4, p.m - (t.m0 + wm * 64 + 16 * i + lr)); // this thread's rows below m
  if (t.swiglu) {
    const int col = t.n0 + (kSpan / 2) * wn + 16 * jp + lc;
#pragma unroll
    for (int e = 0; e < 4; e++)
      if (e < rows && col < seg.n)
        seg.c[(long long)(t.m0 + wm * 64 + 16 * i + lr + e) * seg.ldc + col] = silu_gate(lo[e], hi[e]);
    return;
  }
  const int c0 = t.n0 + kSpan * wn + 16 * jp + lc, c1 = c0 + 16 * (J / 2);
  const bool in0 = c0 < seg.n, in1 = c1 < seg.n;
  float *crow0 = seg.c + (long long)(t.m0 + wm * 64 + 16 * i + lr) * seg.ldc;
  if (seg.epi == EPI_ADD) { // every current value read before any sum is written back
    float prior0[4], prior1[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      prior0[e] = e < rows && in0 ? crow0[(long long)e * seg.ldc + c0] : 0.0f;
      prior1[e] = e < rows && in1 ? crow0[(long long)e * seg.ldc + c1] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
      lo[e] = prior0[e] + lo[e];
      hi[e] = prior1[e] + hi[e];
    }
  }
#pragma unroll
  for (int e = 0; e < 4; e++) {
    if (e < rows && in0)
      crow0[(long long)e * seg.ldc + c0] = lo[e];
    if (e < rows && in1)
      crow0[(long long)e * seg.ldc + c1] = hi[e];
  }
}

// The K loop unrolled by the stages (every stage index a constant), leaving after the last step.
template <int I, int N, class F> __device__ __forceinline__ bool unrolled_steps(F &f, int step, int steps) {
  if constexpr (I < N) {
    f(step + I, std::integral_constant<int, I>{});
    if (I + 1 < N && step + I + 1 >= steps)
      return false;
    return unrolled_steps<I + 1, N>(f, step, steps);
  }
  return true;
}

// The loads of steps first .. first + N - 1 into stages 0 .. N - 1.
template <int I, int N, class F> __device__ __forceinline__ void issue_first(F &f, int first) {
  if constexpr (I < N) {
    f(first + I, std::integral_constant<int, I>{});
    issue_first<I + 1, N>(f, first);
  }
}

// QUANT: SWIGLU segments with the quantized output (seg.cq) take store_tile_quantized (an instantiation of its own:
// the epilogue's registers would otherwise crowd the K loop of every other launch).
template <class C, bool PROBE, bool GS64, bool SPLIT, bool QUANT = false>
__global__ __launch_bounds__(C::Threads, 2) void q8_gemm_lds(Q8Params p) {
  extern __shared__ __align__(16) unsigned char q8_smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  // readfirstlane: the divisions run on the vector unit, and a step base the compiler cannot prove uniform would
  // turn every buffer load (the step is its scalar offset) into a loop over lanes
  // SPLIT is its own instantiation: the unsplit kernel sits at the register limit, and a K range that does not start
  // at 0 pushes it into spilling.
  const int logical = xcd_logical(blockIdx.x, p.grid.total * (SPLIT ? p.sk.splits : 1));
  const int tile = SPLIT ? __builtin_amdgcn_readfirstlane(logical / p.sk.splits) : logical;
  const int split = SPLIT ? __builtin_amdgcn_readfirstlane(logical % p.sk.splits) : 0;
  const TilePos t = q8_tile_of(p.grid, tile, C::TileM);
  const TileSeg seg = q8_seg_of(p.grid, t.s);
  const int groups = p.k / p.gs, spg = GS64 ? 1 : p.gs / 64, steps = p.k / 64;
  // this block's K steps [s0, s1): whole groups (per is a multiple of the steps per group)
  const int s0 = SPLIT ? split * p.sk.per : 0, s1 = SPLIT ? min(steps, s0 + p.sk.per) : steps;
  const long long k = p.k;

  // This wave's loads of every step, as buffer resources bounded to the rows that exist (rows past m or n read zeros)
  // and per-lane offsets that place lane l's 16 bytes at l * 16 of a 1 KB block (row l / 4, swizzled chunk l % 4).
  const int lrow4 = lane >> 2, chunk = lane & 3;
  const int ra = 32 * wave + lrow4; // A rows ra (block 2 wave) and ra + 16 (block 2 wave + 1)
  const __amdgpu_buffer_rsrc_t rA = q8_buffer(p.xq + (long long)t.m0 * k, (long long)min(C::TileM, p.m - t.m0) * k);
  const int offA0 = (int)(ra * k) + ((chunk ^ q8_swizzle(ra)) << 4);
  const int offA1 = (int)((ra + 16) * k) + ((chunk ^ q8_swizzle(ra + 16)) << 4);
  // B tile rows 16 bb .. 16 bb + 15 (block bb = BPerWave wave + b, b < 2), all of one matrix. Two named resources, not
  // an array: the host compilation silently drops a kernel that holds an array of buffer resources.
  static_assert(C::BPerWave == 1 || C::BPerWave == 2, "one or two B blocks per wave");
  auto b_resource = [&](int b, int &off) {
    const int rb0 = 16 * (C::BPerWave * wave + b);
    const int colB = t.swiglu ? t.n0 + (rb0 & 63) : t.n0 + rb0;
    const int8_t *wmat = (const int8_t *)((t.swiglu && rb0 >= 64) ? seg.w3 : seg.w);
    off = (int)(lrow4 * k) + ((chunk ^ q8_swizzle(rb0 + lrow4)) << 4);
    return q8_buffer(wmat + (long long)colB * k, (long long)min(16, seg.n - colB) * k);
  };
  int offB0, offB1 = 0;
  const __amdgpu_buffer_rsrc_t rB0 = b_resource(0, offB0);
  const __amdgpu_buffer_rsrc_t rB1 = C::BPerWave == 2 ? b_resource(1, offB1) : rB0;
  // scale loads: waves 0 .. WM - 1 the xs rows (64 each), the next two the 128 ws rows, any others nothing
  __amdgpu_buffer_rsrc_t rS;
  int scale_dst; // byte offset inside a stage's scales: xs, then ws, then spare
  if (wave < C::WM) {
    const int r0 = t.m0 + 64 * wave;
    rS = q8_buffer(p.xs + (long long)r0 * groups, (long long)min(64, p.m - r0) * groups * 4);
    scale_dst = 64 * wave * 4;
  } else if (wave < C::WM + 2) {
    const int h = wave - C::WM;
    const float *src = t.swiglu ? (h ? seg.w3s : seg.ws) : seg.ws;
    const int c0 = t.swiglu ? t.n0 : t.n0 + 64 * h;
    rS = q8_buffer(src + (long long)c0 * groups, (long long)min(64, seg.n - c0) * groups * 4);
    scale_dst = (C::TileM + 64 * h) * 4;
  } else {
    rS = q8_buffer(p.xs, 0);
    scale_dst = (C::TileM + C::TileN) * 4;
  }
  const int offS = lane * groups * 4;
  const __amdgpu_buffer_rsrc_t none = q8_buffer(p.xq, 0);

  // The loads of K step `step` into stage ST; a step past the end loads nothing (zero-length resources). The K offset
  // goes in the scalar offset operand.
  auto issue = [&](int step, auto ST) {
    constexpr int st = decltype(ST)::value;
    const bool live = step < s1;
    const int k0 = step * 64, g = step / spg;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rA : none, (void *)(q8_smem + ((2 * wave) * C::Stages + st) * 1024),
                                             16, offA0, k0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rA : none,
                                             (void *)(q8_smem + ((2 * wave + 1) * C::Stages + st) * 1024), 16, offA1,
                                             k0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        live ? rB0 : none, (void *)(q8_smem + C::BOff + (C::BPerWave * wave * C::Stages + st) * 1024), 16, offB0, k0,
        0, 0);
    if constexpr (C::BPerWave == 2)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          live ? rB1 : none, (void *)(q8_smem + C::BOff + ((2 * wave + 1) * C::Stages + st) * 1024), 16, offB1, k0,
          0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rS : none,
                                             (void *)(q8_smem + C::SOff + st * C::SStride + scale_dst), 4, offS,
                                             g * 4, 0, 0);
  };

  // Per-lane LDS read bases; the stage and the 16-row block add immediates.
  const int lrow = lane & 15, lq = lane >> 4, lr4 = (lane >> 4) * 4;
  const int lane_part = lrow * 64 + ((lq ^ q8_swizzle(lrow)) << 4);
  const unsigned char *abase = q8_smem + (4 * wm) * C::Stages * 1024 + lane_part;
  const unsigned char *bbase[4];
#pragma unroll
  for (int j = 0; j < 4; j++)
    bbase[j] = q8_smem + C::BOff + (b_row(t.swiglu, wn, j) / 16) * C::Stages * 1024 + lane_part;
  const unsigned char *xsbase = q8_smem + C::SOff + (wm * 64 + lr4) * 4;
  const unsigned char *wsbase[4];
#pragma unroll
  for (int j = 0; j < 4; j++)
    wsbase[j] = q8_smem + C::SOff + (C::TileM + b_row(t.swiglu, wn, j) + lrow) * 4;

  auto operands = [&](auto ST, v4i (&a)[4], v4i (&b)[4]) {
    constexpr int st = decltype(ST)::value;
#pragma unroll
    for (int i = 0; i < 4; i++)
      a[i] = *reinterpret_cast<const v4i *>(abase + (i * C::Stages + st) * 1024);
#pragma unroll
    for (int j = 0; j < 4; j++)
      b[j] = *reinterpret_cast<const v4i *>(bbase[j] + st * 1024);
  };

  v4f acc[4][4];
  v4i dot[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
      acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  // One step in stage ST: step + 1's loads have landed once only the two later steps' may be outstanding; the barrier
  // makes that true of every wave and means every wave is done with the stage step - 1 used, which step + 4 now
  // fills. Then the next step's MFMAs and, at a group's end, this step's rescale. After the last step the MFMAs run
  // on stale operands whose products are never used.
  auto advance = [&](int step, auto ST) {
    constexpr int st = decltype(ST)::value, nst = (st + 1) % C::Stages, fill = (st + C::Stages - 1) % C::Stages;
    wait_vmcnt<(C::Stages - 3) * C::LoadsPerStep>();
    __builtin_amdgcn_s_barrier();
    issue(step + C::Stages - 1, std::integral_constant<int, fill>{});
    v4i a[4], b[4];
    operands(std::integral_constant<int, nst>{}, a, b);
    if (GS64 || step % spg == spg - 1) {
      v4f xsv[4];
      float wsc[4];
#pragma unroll
      for (int i = 0; i < 4; i++)
        xsv[i] = *reinterpret_cast<const v4f *>(xsbase + st * C::SStride + i * 64);
#pragma unroll
      for (int j = 0; j < 4; j++)
        wsc[j] = *reinterpret_cast<const float *>(wsbase[j] + st * C::SStride);
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          if (PROBE) {
            const int g = step / spg;
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const int row = t.m0 + wm * 64 + 16 * i + lr4 + e, col = t.n0 + 64 * wn + 16 * j + lrow;
              if (row < p.m && col < seg.n)
                p.probe[((long long)g * p.m + row) * seg.n + col] = dot[i][j][e];
            }
          }
          float f[4];
#pragma unroll
          for (int e = 0; e < 4; e++)
            f[e] = (float)dot[i][j][e];
          dot[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
          for (int e = 0; e < 4; e++)
            acc[i][j][e] = fmaf(f[e] * wsc[j], xsv[i][e], acc[i][j][e]);
        }
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          dot[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], dot[i][j], 0, 0, 0);
    }
  };

  issue_first<0, C::Stages - 1>(issue, s0);
  wait_vmcnt<(C::Stages - 2) * C::LoadsPerStep>(); // step s0 has landed for this wave
  __builtin_amdgcn_s_barrier();                      // ... and for every wave
  {
    v4i a[4], b[4];
    operands(std::integral_constant<int, 0>{}, a, b);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
        dot[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], v4i{0, 0, 0, 0}, 0, 0, 0);
  }
  // the K loop unrolled by the stages, so every stage index is a constant
  for (int step = s0; step < s1; step += C::Stages)
    if (!unrolled_steps<0, C::Stages>(advance, step, s1))
      break;
  // the loads issued for steps past the end still target this block's LDS: let them land before the block exits
  __builtin_amdgcn_s_waitcnt(0);
  if (SPLIT) { // a partial tile for split_reduce (the register budget leaves no room for an in-kernel sum)
    v4f *slot = p.sk.partial + (size_t)(tile * p.sk.splits + split) * 16 * C::Threads + threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
        slot[(i * 4 + j) * C::Threads] = acc[i][j];
    return;
  }
  if constexpr (QUANT)
    store_tile_quantized(seg, t, acc, wm, wn, lane, p.m, reinterpret_cast<float *>(q8_smem), p.flags);
  else
    store_tile(seg, t, acc, wm, wn, lane, p.m);
}


// Round to nearest even on the 16 dropped bits, NaN quieted with its sign and top payload bits, denormals kept,
// overflow to infinity: the conversion of the reference's bf16_from_f32 (src/gemm.c:335-342), as an integer formula.
__device__ __forceinline__ unsigned short to_bf16(float x) {
  unsigned u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u)
    return (unsigned short)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (unsigned short)(u >> 16);
}

// ---- FP32 and BF16: the pipelined MFMA kernel, with split K for short grids ---------------------------------------------
//
// k_gemm_bf16 rounds A to BF16 once per call into the caller's panel (the reference's bf16_convert_rows,
// src/gemm.c:693-706): rows of kp = K rounded up to 32 values, zero past K. Both modes then share the structure of the
// int8 kernel above: a 256 x 128 output tile over eight waves of 64 x 64, 4 x 4 MFMA tiles of 16 x 16 per wave, and a
// K step of 64 bytes per row (32 BF16 or 16 FP32 values) whose A and B tiles go straight from global memory into LDS
// five stages deep, in 1 KB blocks of 16 rows interleaved by stage. A block row is XOR-swizzled in 16-byte chunks like
// the int8 tiles. MFMA operands take 16 contiguous bytes of a row per lane group q = lane / 16:
//   BF16: v_mfma_f32_16x16x32_bf16, K values 8 q .. 8 q + 7. B arrives in the pack_bf16_vnni layout, whose 16-row
//         tile and 32-value K step is one contiguous 1 KB block (16 K pairs of 16 rows x 2 values), copied with its
//         16-byte chunks reordered so that a lane's four K pairs are four conflict-free 4-byte reads.
//   FP32: four v_mfma_f32_16x16x4_f32 per tile and step; lane group q holds K values 4 q .. 4 q + 3 of A and W and
//         feeds value s to the s-th instruction. W rows are read like A rows (row pitch ldw).
// The FP32 sums stay in the MFMA accumulators: no per-step vector work.
//
// Short grids split K; this kernel's register budget leaves room to add the partial tiles in the last block to
// arrive (split_combine) instead of a second kernel.
__global__ __launch_bounds__(256) void bf16_panel(const float *__restrict__ a, long long lda, int m, int k, int kp,
                                                  unsigned short *__restrict__ panel) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x; // 8 values per thread
  const int per_row = kp / 8;
  if (idx >= (long long)m * per_row)
    return;
  const int row = (int)(idx / per_row), c0 = (int)(idx % per_row) * 8;
  const float *src = a + row * lda;
  unsigned packed[4];
  if (c0 + 8 <= k && ((uintptr_t)(src + c0) & 15) == 0) { // eight values in two 16-byte loads
    const float4 v0 = *reinterpret_cast<const float4 *>(src + c0), v1 = *reinterpret_cast<const float4 *>(src + c0 + 4);
    packed[0] = to_bf16(v0.x) | ((unsigned)to_bf16(v0.y) << 16);
    packed[1] = to_bf16(v0.z) | ((unsigned)to_bf16(v0.w) << 16);
    packed[2] = to_bf16(v1.x) | ((unsigned)to_bf16(v1.y) << 16);
    packed[3] = to_bf16(v1.z) | ((unsigned)to_bf16(v1.w) << 16);
  } else { // the row's tail (zeros past k) or an unaligned row
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = c0 + 2 * i;
      const unsigned lo = c < k ? to_bf16(src[c]) : 0u, hi = c + 1 < k ? to_bf16(src[c + 1]) : 0u;
      packed[i] = lo | (hi << 16);
    }
  }
  *reinterpret_cast<uint4 *>(panel + (long long)row * kp + c0) = uint4{packed[0], packed[1], packed[2], packed[3]};
}

typedef __bf16 v8bf_t __attribute__((ext_vector_type(8)));

constexpr int kMmLoadsPerStep = 3;                   // per wave: two A and one B load
constexpr size_t kMmLds = (size_t)kQ8SOff;           // A and B blocks of five stages, no scales

struct MmParams {
  Q8Grid grid;
  const unsigned char *a; // BF16 panel or FP32 rows
  long long arow;         // bytes per A row
  int m, steps;           // rows; K steps of 64 bytes per row
  SplitK sk;
};

template <bool F32> __global__ __launch_bounds__(kQ8Threads, 2) void mm_gemm_lds(MmParams p) {
  extern __shared__ __align__(16) unsigned char q8_smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int logical = xcd_logical(blockIdx.x, p.grid.total * p.sk.splits);
  const int tile = __builtin_amdgcn_readfirstlane(logical / p.sk.splits); // uniform (see q8_gemm_lds)
  const int split = __builtin_amdgcn_readfirstlane(logical % p.sk.splits);
  const TilePos t = q8_tile_of(p.grid, tile);
  const TileSeg seg = q8_seg_of(p.grid, t.s);
  const int s0 = split * p.sk.per, s1 = min(p.steps, s0 + p.sk.per);

  const int lrow4 = lane >> 2, chunk = lane & 3;
  const int ra = 32 * wave + lrow4;
  const __amdgpu_buffer_rsrc_t rA = q8_buffer(p.a + (long long)t.m0 * p.arow, (long long)min(kQ8TileM, p.m - t.m0) * p.arow);
  const int offA0 = (int)(ra * p.arow) + ((chunk ^ q8_swizzle(ra)) << 4);
  const int offA1 = (int)((ra + 16) * p.arow) + ((chunk ^ q8_swizzle(ra + 16)) << 4);
  // B: this wave's 16 rows of one matrix. BF16: one VNNI tile, step s at bytes [s * 1024, s * 1024 + 1024); FP32: 16
  // weight rows, read like the A rows.
  const int rb0 = 16 * wave;
  const int colB = t.swiglu ? t.n0 + (rb0 & 63) : t.n0 + rb0;
  const unsigned char *wmat = (const unsigned char *)((t.swiglu && rb0 >= 64) ? seg.w3 : seg.w);
  const long long brow = F32 ? seg.ldw * 4 : 0;
  const long long tile_bytes = (long long)p.steps * 1024;
  const __amdgpu_buffer_rsrc_t rB =
      F32 ? q8_buffer(wmat + (long long)colB * brow, (long long)min(16, seg.n - colB) * brow)
          : q8_buffer(wmat + (long long)(colB / 16) * tile_bytes, colB < seg.n ? tile_bytes : 0);
  // BF16: the 1 KB VNNI block holds 16-byte chunks of one K pair for four rows (chunk 4 P + rg: pair P, rows
  // 4 rg .. 4 rg + 3). Lane l copies chunk (pair 4 q + p, rows 4 rg ..) with p = l / 16, q = (l / 4) % 4, rg = l % 4
  // to LDS position l = 16 p + 4 q + rg, so the MFMA lane (row r, group q) finds its pair 4 q + p at byte
  // 256 p + 64 q + 4 r: one 4-byte read per p, on 64 distinct banks across the wave.
  const int offB = F32 ? (int)(lrow4 * brow) + ((chunk ^ q8_swizzle(lrow4)) << 4)
                       : ((4 * ((lane >> 2) & 3) + (lane >> 4)) << 6) + ((lane & 3) << 4);
  const int bstep = F32 ? 64 : 1024; // B bytes per K step
  const __amdgpu_buffer_rsrc_t none = q8_buffer(p.a, 0);

  auto issue = [&](int step, auto ST) {
    constexpr int st = decltype(ST)::value;
    const bool live = step < s1;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rA : none, (void *)(q8_smem + ((2 * wave) * kQ8Stages + st) * 1024),
                                             16, offA0, step * 64, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rA : none,
                                             (void *)(q8_smem + ((2 * wave + 1) * kQ8Stages + st) * 1024), 16, offA1,
                                             step * 64, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rB : none,
                                             (void *)(q8_smem + kQ8BOff + (wave * kQ8Stages + st) * 1024), 16, offB,
                                             step * bstep, 0, 0);
  };

  const int lrow = lane & 15, lq = lane >> 4;
  const int lane_part = lrow * 64 + ((lq ^ q8_swizzle(lrow)) << 4);
  const unsigned char *abase = q8_smem + (4 * wm) * kQ8Stages * 1024 + lane_part;
  const unsigned char *bbase[4];
#pragma unroll
  for (int j = 0; j < 4; j++)
    bbase[j] = q8_smem + kQ8BOff + (b_row(t.swiglu, wn, j) / 16) * kQ8Stages * 1024 +
               (F32 ? lane_part : lq * 64 + lrow * 4);

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
      acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  // MFMA operands of one step, read from LDS a step ahead of their use
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  struct Operands {
    v4u a[4], b[4];
  };
  auto operands = [&](auto ST, Operands &o) {
    constexpr int st = decltype(ST)::value;
#pragma unroll
    for (int i = 0; i < 4; i++)
      o.a[i] = *reinterpret_cast<const v4u *>(abase + (i * kQ8Stages + st) * 1024);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const unsigned char *bp = bbase[j] + st * 1024;
      if constexpr (F32)
        o.b[j] = *reinterpret_cast<const v4u *>(bp);
      else
        o.b[j] = v4u{*reinterpret_cast<const unsigned *>(bp), *reinterpret_cast<const unsigned *>(bp + 256),
                     *reinterpret_cast<const unsigned *>(bp + 512), *reinterpret_cast<const unsigned *>(bp + 768)};
    }
  };
  auto mfmas = [&](const Operands &o) {
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if constexpr (F32) {
          const v4f a = __builtin_bit_cast(v4f, o.a[i]), b = __builtin_bit_cast(v4f, o.b[j]);
#pragma unroll
          for (int s = 0; s < 4; s++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], acc[i][j], 0, 0, 0);
        } else {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf_t, o.a[i]),
                                                              __builtin_bit_cast(v8bf_t, o.b[j]), acc[i][j], 0, 0, 0);
        }
      }
  };

  // One step in stage ST: step + 1's loads have landed once only the two later steps' may be outstanding; the barrier
  // makes that true of every wave and means every wave is done with the stage step - 1 used, which step + 4 now
  // fills. The operands of step + 1 are read while this step's MFMAs (on operands read one step earlier) run.
  Operands cur, next;
  auto advance = [&](int step, auto ST) {
    constexpr int st = decltype(ST)::value, nst = (st + 1) % kQ8Stages, fill = (st + kQ8Stages - 1) % kQ8Stages;
    wait_vmcnt<(kQ8Stages - 3) * kMmLoadsPerStep>();
    __builtin_amdgcn_s_barrier();
    issue(step + kQ8Stages - 1, std::integral_constant<int, fill>{});
    operands(std::integral_constant<int, nst>{}, next);
    __builtin_amdgcn_sched_barrier(0); // keep the reads ahead of the MFMAs that do not need them
    mfmas(cur);
    __builtin_amdgcn_sched_barrier(0);
    cur = next;
  };

  issue(s0, std::integral_constant<int, 0>{});
  issue(s0 + 1, std::integral_constant<int, 1>{});
  issue(s0 + 2, std::integral_constant<int, 2>{});
  issue(s0 + 3, std::integral_constant<int, 3>{});
  wait_vmcnt<(kQ8Stages - 2) * kMmLoadsPerStep>(); // step s0 has landed for this wave
  __builtin_amdgcn_s_barrier();                    // ... and for every wave
  operands(std::integral_constant<int, 0>{}, cur);
  // Whole rounds of five steps, with no exit between them: steps past the end load zeros (an empty buffer) and add
  // nothing, and the accumulators stay in place across the unrolled body instead of being copied at every exit.
  for (int step = s0; step < s1; step += kQ8Stages) {
    advance(step, std::integral_constant<int, 0>{});
    advance(step + 1, std::integral_constant<int, 1>{});
    advance(step + 2, std::integral_constant<int, 2>{});
    advance(step + 3, std::integral_constant<int, 3>{});
    advance(step + 4, std::integral_constant<int, 4>{});
  }
  __builtin_amdgcn_s_waitcnt(0);
  if (p.sk.splits > 1 && !split_combine<kQ8Threads>(p.sk, tile, split, acc))
    return;
  store_tile(seg, t, acc, wm, wn, lane, p.m);
}

// ---- FP32 on the BF16 matrix cores -----------------------------------------------------------------------------
//
// mm_gemm_f32x3: the FP32 GEMM with every product formed from exact three-part BF16 splits of its FP32 operands, as
// the batched attention forms them: x = h + m + l exactly (h the top 8 significant bits of x, m the next 8 of x - h, l
// the rest, at most 8 bits) and x y is taken as hh + hm + mh + mm + hl + lh, the dropped products below 2^-23 of |x y|
// and every BF16 product exact in FP32, so each sum is FP32-accurate. Six v_mfma_f32_16x16x32_bf16 (16 cycles) replace
// eight v_mfma_f32_16x16x4_f32 (32 cycles each). The tiles, A and W staging (64 bytes of 16 rows per 1 KB block, XOR
// swizzle, buffer loads straight into LDS), split K and epilogues are mm_gemm_lds's FP32 ones, with six stages so
// that a round of steps is a whole number of pairs: the MFMAs run at every second step on the K values of the pair,
// lane group q's slots 8 q .. 8 q + 3 from the first step's values 4 q .. 4 q + 3 and slots 8 q + 4 .. from the
// second's, the same in A and in W, and each lane splits its own operands in registers.
constexpr int kX3Stages = 6;
constexpr int kX3BOff = kQ8ABlocks * kX3Stages * 1024;
constexpr size_t kX3Lds = (size_t)kX3BOff + (size_t)kQ8BBlocks * kX3Stages * 1024;

__global__ __launch_bounds__(kQ8Threads, 2) void mm_gemm_f32x3(MmParams p) {
  extern __shared__ __align__(16) unsigned char q8_smem[];
  typedef int v4i_t __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int logical = xcd_logical(blockIdx.x, p.grid.total * p.sk.splits);
  const int tile = __builtin_amdgcn_readfirstlane(logical / p.sk.splits);
  const int split = __builtin_amdgcn_readfirstlane(logical % p.sk.splits);
  const TilePos t = q8_tile_of(p.grid, tile);
  const TileSeg seg = q8_seg_of(p.grid, t.s);
  const int s0 = split * p.sk.per, s1 = min(p.steps, s0 + p.sk.per);

  const int lrow4 = lane >> 2, chunk = lane & 3;
  const int ra = 32 * wave + lrow4;
  const __amdgpu_buffer_rsrc_t rA = q8_buffer(p.a + (long long)t.m0 * p.arow, (long long)min(kQ8TileM, p.m - t.m0) * p.arow);
  const int offA0 = (int)(ra * p.arow) + ((chunk ^ q8_swizzle(ra)) << 4);
  const int offA1 = (int)((ra + 16) * p.arow) + ((chunk ^ q8_swizzle(ra + 16)) << 4);
  const int rb0 = 16 * wave;
  const int colB = t.swiglu ? t.n0 + (rb0 & 63) : t.n0 + rb0;
  const unsigned char *wmat = (const unsigned char *)((t.swiglu && rb0 >= 64) ? seg.w3 : seg.w);
  const long long brow = seg.ldw * 4;
  const __amdgpu_buffer_rsrc_t rB = q8_buffer(wmat + (long long)colB * brow, (long long)min(16, seg.n - colB) * brow);
  const int offB = (int)(lrow4 * brow) + ((chunk ^ q8_swizzle(lrow4)) << 4);
  const __amdgpu_buffer_rsrc_t none = q8_buffer(p.a, 0);

  auto issue = [&](int step, auto ST) {
    constexpr int st = decltype(ST)::value;
    const bool live = step < s1;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rA : none, (void *)(q8_smem + ((2 * wave) * kX3Stages + st) * 1024),
                                             16, offA0, step * 64, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rA : none,
                                             (void *)(q8_smem + ((2 * wave + 1) * kX3Stages + st) * 1024), 16, offA1,
                                             step * 64, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rB : none,
                                             (void *)(q8_smem + kX3BOff + (wave * kX3Stages + st) * 1024), 16, offB,
                                             step * 64, 0, 0);
  };

  const int lrow = lane & 15, lq = lane >> 4;
  const int lane_part = lrow * 64 + ((lq ^ q8_swizzle(lrow)) << 4);
  const unsigned char *abase = q8_smem + (4 * wm) * kX3Stages * 1024 + lane_part;
  const unsigned char *bbase[4];
#pragma unroll
  for (int j = 0; j < 4; j++)
    bbase[j] = q8_smem + kX3BOff + (b_row(t.swiglu, wn, j) / 16) * kX3Stages * 1024 + lane_part;

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
      acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  struct Operands {
    v4f a[4], b[4];
  };
  auto operands = [&](auto ST, Operands &o) {
    constexpr int st = decltype(ST)::value;
#pragma unroll
    for (int i = 0; i < 4; i++)
      o.a[i] = *reinterpret_cast<const v4f *>(abase + (i * kX3Stages + st) * 1024);
#pragma unroll
    for (int j = 0; j < 4; j++)
      o.b[j] = *reinterpret_cast<const v4f *>(bbase[j] + st * 1024);
  };
  // the high halves of the three parts of x and y, packed: x in the low half of each dword
  struct Parts2 {
    int h, m, l;
  };
  auto parts2 = [](float x, float y) {
    const unsigned ux = __builtin_bit_cast(unsigned, x), uy = __builtin_bit_cast(unsigned, y);
    const float rx = x - __builtin_bit_cast(float, ux & 0xFFFF0000u), ry = y - __builtin_bit_cast(float, uy & 0xFFFF0000u);
    const unsigned ux1 = __builtin_bit_cast(unsigned, rx), uy1 = __builtin_bit_cast(unsigned, ry);
    const float rx2 = rx - __builtin_bit_cast(float, ux1 & 0xFFFF0000u), ry2 = ry - __builtin_bit_cast(float, uy1 & 0xFFFF0000u);
    return Parts2{(int)__builtin_amdgcn_perm(uy, ux, 0x07060302u), (int)__builtin_amdgcn_perm(uy1, ux1, 0x07060302u),
                  (int)__builtin_amdgcn_perm(__builtin_bit_cast(unsigned, ry2), __builtin_bit_cast(unsigned, rx2),
                                             0x07060302u)};
  };
  auto mfma = [](const v4i_t &a, const v4i_t &b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf_t, a), __builtin_bit_cast(v8bf_t, b), c, 0,
                                                    0, 0);
  };
  // A pair's operands as BF16 parts: dwords 0 and 1 of each part from the first step's four values (split at the
  // first step, while the previous pair's MFMAs drain), dwords 2 and 3 from the second's
  struct PairParts {
    v4i_t ah[4], am[4], al[4], bh[4], bm[4], bl[4];
  };
  auto split_half = [&](const Operands &o, PairParts &pp, int half) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const Parts2 lo = parts2(o.a[i][0], o.a[i][1]), hi = parts2(o.a[i][2], o.a[i][3]);
      pp.ah[i][2 * half] = lo.h, pp.ah[i][2 * half + 1] = hi.h;
      pp.am[i][2 * half] = lo.m, pp.am[i][2 * half + 1] = hi.m;
      pp.al[i][2 * half] = lo.l, pp.al[i][2 * half + 1] = hi.l;
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const Parts2 lo = parts2(o.b[j][0], o.b[j][1]), hi = parts2(o.b[j][2], o.b[j][3]);
      pp.bh[j][2 * half] = lo.h, pp.bh[j][2 * half + 1] = hi.h;
      pp.bm[j][2 * half] = lo.m, pp.bm[j][2 * half + 1] = hi.m;
      pp.bl[j][2 * half] = lo.l, pp.bl[j][2 * half + 1] = hi.l;
    }
  };
  // the MFMAs of a pair: the small products first
  auto mfmas3 = [&](const PairParts &pp) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
      for (int j = 0; j < 4; j++)
        acc[i][j] = mfma(pp.al[i], pp.bh[j], acc[i][j]);
#pragma unroll
      for (int j = 0; j < 4; j++)
        acc[i][j] = mfma(pp.ah[i], pp.bl[j], acc[i][j]);
#pragma unroll
      for (int j = 0; j < 4; j++)
        acc[i][j] = mfma(pp.am[i], pp.bm[j], acc[i][j]);
#pragma unroll
      for (int j = 0; j < 4; j++)
        acc[i][j] = mfma(pp.am[i], pp.bh[j], acc[i][j]);
#pragma unroll
      for (int j = 0; j < 4; j++)
        acc[i][j] = mfma(pp.ah[i], pp.bm[j], acc[i][j]);
#pragma unroll
      for (int j = 0; j < 4; j++)
        acc[i][j] = mfma(pp.ah[i], pp.bh[j], acc[i][j]);
    }
  };

  // As mm_gemm_lds: step + 1's loads have landed once only the later steps' may be outstanding, the barrier makes that
  // true of every wave and frees the stage step - 1 used, which step + 5 now fills; the operands of step + 1 are read
  // a step ahead. An even stage splits its step's half of the pair, an odd stage the other half and runs the MFMAs.
  Operands cur, next;
  PairParts pp;
  auto advance = [&](int step, auto ST) {
    constexpr int st = decltype(ST)::value, nst = (st + 1) % kX3Stages, fill = (st + kX3Stages - 1) % kX3Stages;
    wait_vmcnt<(kX3Stages - 3) * kMmLoadsPerStep>();
    __builtin_amdgcn_s_barrier();
    issue(step + kX3Stages - 1, std::integral_constant<int, fill>{});
    operands(std::integral_constant<int, nst>{}, next);
    __builtin_amdgcn_sched_barrier(0);
    split_half(cur, pp, st % 2);
    if constexpr (st % 2 == 1) {
      mfmas3(pp);
      __builtin_amdgcn_sched_barrier(0);
    }
    cur = next;
  };

  issue(s0, std::integral_constant<int, 0>{});
  issue(s0 + 1, std::integral_constant<int, 1>{});
  issue(s0 + 2, std::integral_constant<int, 2>{});
  issue(s0 + 3, std::integral_constant<int, 3>{});
  issue(s0 + 4, std::integral_constant<int, 4>{});
  wait_vmcnt<(kX3Stages - 2) * kMmLoadsPerStep>();
  __builtin_amdgcn_s_barrier();
  operands(std::integral_constant<int, 0>{}, cur);
  for (int step = s0; step < s1; step += kX3Stages) {
    advance(step, std::integral_constant<int, 0>{});
    advance(step + 1, std::integral_constant<int, 1>{});
    advance(step + 2, std::integral_constant<int, 2>{});
    advance(step + 3, std::integral_constant<int, 3>{});
    advance(step + 4, std::integral_constant<int, 4>{});
    advance(step + 5, std::integral_constant<int, 5>{});
  }
  __builtin_amdgcn_s_waitcnt(0);
  if (p.sk.splits > 1 && !split_combine<kQ8Threads>(p.sk, tile, split, acc))
    return;
  store_tile(seg, t, acc, wm, wn, lane, p.m);
}

// ---- BF16, wide tiles ---------------------------------------------------------------------------------------------
//
// The BF16 kernel above waits on L2: its operands arrive at about 18 bytes per clock per CU, far below the L1's rate,
// because the misses a CU keeps in flight bound it (TCP_PENDING_STALL_CYCLES 62% of the time, MFMA pipe 38% busy).
// This one owns a 256 x 256 tile, which needs a third fewer operand bytes per flop: eight waves in 4 x 2, each
// 64 x 128 as 4 x 8 MFMA tiles (128 accumulators, which the compiler keeps in AGPRs), four stages of 32 KB. Under
// SWIGLU the tile holds 128 columns of W1 and the same 128 of W3, a wave's j = 0..3 and 4..7. Short grids split K;
// the partial tiles are added in split order by split_reduce.
constexpr int kWStages = 4, kWLoadsPerStep = 4; // per wave: two A and two B blocks
constexpr int kWTileM = 256, kWTileN = 256;
constexpr int kWBOff = 16 * kWStages * 1024;                      // 16 A blocks per stage, then 16 B blocks
constexpr size_t kWLds = (size_t)kWBOff + 16 * kWStages * 1024;  // 128 KB
constexpr int kWSlotV4 = 32 * kQ8Threads;                         // v4f per partial tile

// The B-tile row (0..255) that a wave's column tile j reads.
__device__ __forceinline__ int b_row_wide(bool swiglu, int wn, int j) {
  return swiglu ? (j < 4 ? 64 * wn + 16 * j : 128 + 64 * wn + 16 * (j - 4)) : 128 * wn + 16 * j;
}

template <bool SPLIT> __global__ __launch_bounds__(kQ8Threads, 2) void bf16_gemm_wide(MmParams p) {
  extern __shared__ __align__(16) unsigned char q8_smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int logical = xcd_logical(blockIdx.x, p.grid.total * (SPLIT ? p.sk.splits : 1));
  const int tile = SPLIT ? __builtin_amdgcn_readfirstlane(logical / p.sk.splits) : logical;
  const int split = SPLIT ? __builtin_amdgcn_readfirstlane(logical % p.sk.splits) : 0;
  const TilePos t = q8_tile_of(p.grid, tile, kWTileM, kWTileN);
  const TileSeg seg = q8_seg_of(p.grid, t.s);
  const int s0 = SPLIT ? split * p.sk.per : 0, s1 = SPLIT ? min(p.steps, s0 + p.sk.per) : p.steps;

  const int lrow4 = lane >> 2, chunk = lane & 3;
  const int ra = 32 * wave + lrow4;
  const __amdgpu_buffer_rsrc_t rA =
      q8_buffer(p.a + (long long)t.m0 * p.arow, (long long)min(kWTileM, p.m - t.m0) * p.arow);
  const int offA0 = (int)(ra * p.arow) + ((chunk ^ q8_swizzle(ra)) << 4);
  const int offA1 = (int)((ra + 16) * p.arow) + ((chunk ^ q8_swizzle(ra + 16)) << 4);
  // B blocks 2 wave and 2 wave + 1: one VNNI tile of one matrix each (chunks reordered as in mm_gemm_lds)
  const long long tile_bytes = (long long)p.steps * 1024;
  auto b_resource = [&](int blk) {
    const int rb = 16 * blk;
    const int colB = t.swiglu ? t.n0 + (rb & 127) : t.n0 + rb;
    const unsigned char *wmat = (const unsigned char *)((t.swiglu && rb >= 128) ? seg.w3 : seg.w);
    return q8_buffer(wmat + (long long)(colB / 16) * tile_bytes, colB < seg.n ? tile_bytes : 0);
  };
  const __amdgpu_buffer_rsrc_t rB0 = b_resource(2 * wave), rB1 = b_resource(2 * wave + 1);
  const int offB = ((4 * ((lane >> 2) & 3) + (lane >> 4)) << 6) + ((lane & 3) << 4);
  const __amdgpu_buffer_rsrc_t none = q8_buffer(p.a, 0);

  auto issue = [&](int step, auto ST) {
    constexpr int st = decltype(ST)::value;
    const bool live = step < s1;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rA : none, (void *)(q8_smem + ((2 * wave) * kWStages + st) * 1024),
                                             16, offA0, step * 64, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rA : none,
                                             (void *)(q8_smem + ((2 * wave + 1) * kWStages + st) * 1024), 16, offA1,
                                             step * 64, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rB0 : none,
                                             (void *)(q8_smem + kWBOff + ((2 * wave) * kWStages + st) * 1024), 16,
                                             offB, step * 1024, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rB1 : none,
                                             (void *)(q8_smem + kWBOff + ((2 * wave + 1) * kWStages + st) * 1024), 16,
                                             offB, step * 1024, 0, 0);
  };

  const int lrow = lane & 15, lq = lane >> 4;
  const unsigned char *abase = q8_smem + (4 * wm) * kWStages * 1024 + lrow * 64 + ((lq ^ q8_swizzle(lrow)) << 4);
  const unsigned char *bbase = q8_smem + kWBOff + lq * 64 + lrow * 4;
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  struct Operands {
    v4u a[4], b[8];
  };
  auto operands = [&](auto ST, Operands &o) {
    constexpr int st = decltype(ST)::value;
#pragma unroll
    for (int i = 0; i < 4; i++)
      o.a[i] = *reinterpret_cast<const v4u *>(abase + (i * kWStages + st) * 1024);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const unsigned char *bp = bbase + ((b_row_wide(t.swiglu, wn, j) / 16) * kWStages + st) * 1024;
      o.b[j] = v4u{*reinterpret_cast<const unsigned *>(bp), *reinterpret_cast<const unsigned *>(bp + 256),
                   *reinterpret_cast<const unsigned *>(bp + 512), *reinterpret_cast<const unsigned *>(bp + 768)};
    }
  };
  v4f acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 8; j++)
      acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  auto mfmas = [&](const Operands &o) {
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 8; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf_t, o.a[i]),
                                                            __builtin_bit_cast(v8bf_t, o.b[j]), acc[i][j], 0, 0, 0);
  };

  Operands cur, next;
  auto advance = [&](int step, auto ST) {
    constexpr int st = decltype(ST)::value, nst = (st + 1) % kWStages, fill = (st + kWStages - 1) % kWStages;
    wait_vmcnt<(kWStages - 3) * kWLoadsPerStep>(); // step + 1 has landed for this wave
    __builtin_amdgcn_s_barrier();                 // ... and every wave; the stage of step - 1 is free
    issue(step + kWStages - 1, std::integral_constant<int, fill>{});
    operands(std::integral_constant<int, nst>{}, next);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(cur);
    __builtin_amdgcn_sched_barrier(0);
    cur = next;
  };

  issue_first<0, kWStages - 1>(issue, s0);
  wait_vmcnt<(kWStages - 2) * kWLoadsPerStep>();
  __builtin_amdgcn_s_barrier();
  operands(std::integral_constant<int, 0>{}, cur);
  for (int step = s0; step < s1; step += kWStages) { // whole rounds: steps past the end load zeros
    advance(step, std::integral_constant<int, 0>{});
    advance(step + 1, std::integral_constant<int, 1>{});
    advance(step + 2, std::integral_constant<int, 2>{});
    advance(step + 3, std::integral_constant<int, 3>{});
  }
  __builtin_amdgcn_s_waitcnt(0);
  if (SPLIT) {
    v4f *slot = p.sk.partial + (size_t)(tile * p.sk.splits + split) * kWSlotV4 + threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 8; j++)
        slot[(i * 8 + j) * kQ8Threads] = acc[i][j];
    return;
  }
  store_tile_wide(seg, t, acc, wm, wn, lane, p.m);
}


// ---- W8A8 Q8_0, wide tiles ----------------------------------------------------------------------------------------
//
// q8_gemm_lds waits on its operands as much as on its rescale. On the 8B W1/W3 launch (2048 x 2 * 14336 x 4096) it
// takes 538 us. Copies of it measured: without the rescale, 450 us; without the operand loads, 402; without both,
// 202. The weight tile's loads, half the bytes, cost more than the activations': the weights come from HBM and the
// activations from L2, so what limits is the misses a CU keeps in flight, not bandwidth.
//
// This kernel owns a 256 x 256 tile (the wide BF16 kernel's shape). That is a third fewer operand bytes per output, and
// A is read half as often. Eight waves in 4 x 2 each own 64 x 128 as 4 x 8 MFMA tiles. Their FP32 sums take 128
// registers, so the int32 results cannot all wait for the next step as in q8_gemm_lds. Instead:
// - a step's MFMAs run column tile by column tile (j = 0..7, rows i = 0..3);
// - each tile's results are rescaled one column tile later, just before tile (j, i)'s MFMA overwrites those of
//   (j - 1, i): converted, then added with that step's scales;
// - only column tile 7 crosses into the next step, where its rescale keeps the VALU busy while the next operands
//   arrive behind the barrier.
// Four stages of 34 KB (the A and B tiles, and the xs / ws of the step's group) keep three steps in flight. gs = 64
// only (one group per step). Under SWIGLU the tile holds 128 columns of W1 and the same 128 of W3 (b_row_wide).
constexpr int kQWStages = 4, kQWLoadsPerStep = 5; // per wave: two A blocks, two B blocks, one scale load
constexpr int kQWBOff = 16 * kQWStages * 1024;     // 16 A blocks per stage, then 16 B blocks
constexpr int kQWSOff = kQWBOff + 16 * kQWStages * 1024;
constexpr int kQWSStride = 512 * 4; // xs of the 256 rows, then ws of the 256 B-tile rows
constexpr size_t kQWLds = (size_t)kQWSOff + (size_t)kQWStages * kQWSStride; // 136 KB
static_assert(kQWLds <= 160 * 1024, "one wide int8 block fits a CU's LDS");

template <bool SPLIT> __global__ __launch_bounds__(kQ8Threads, 2) void q8_gemm_wide(Q8Params p) {
  extern __shared__ __align__(16) unsigned char q8_smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int logical = xcd_logical(blockIdx.x, p.grid.total * (SPLIT ? p.sk.splits : 1));
  const int tile = SPLIT ? __builtin_amdgcn_readfirstlane(logical / p.sk.splits) : logical;
  const int split = SPLIT ? __builtin_amdgcn_readfirstlane(logical % p.sk.splits) : 0;
  const TilePos t = q8_tile_of(p.grid, tile, kWTileM, kWTileN);
  const TileSeg seg = q8_seg_of(p.grid, t.s);
  const int groups = p.k / 64, steps = groups;
  const int s0 = SPLIT ? split * p.sk.per : 0, s1 = SPLIT ? min(steps, s0 + p.sk.per) : steps;
  const long long k = p.k;

  // Loads: lane l places its 16 bytes at l * 16 of a 1 KB block (row l / 4, chunk l % 4 XOR-swizzled by the row).
  const int lrow4 = lane >> 2, chunk = lane & 3;
  const int ra = 32 * wave + lrow4; // A rows ra (block 2 wave) and ra + 16 (block 2 wave + 1)
  const __amdgpu_buffer_rsrc_t rA = q8_buffer(p.xq + (long long)t.m0 * k, (long long)min(kWTileM, p.m - t.m0) * k);
  const int offA0 = (int)(ra * k) + ((chunk ^ q8_swizzle(ra)) << 4);
  const int offA1 = (int)((ra + 16) * k) + ((chunk ^ q8_swizzle(ra + 16)) << 4);
  // B-tile blocks 2 wave and 2 wave + 1 (rows 16 blk ..), each of one matrix
  auto b_resource = [&](int blk) {
    const int rb = 16 * blk;
    const int colB = t.swiglu ? t.n0 + (rb & 127) : t.n0 + rb;
    const int8_t *wmat = (const int8_t *)((t.swiglu && rb >= 128) ? seg.w3 : seg.w);
    return q8_buffer(wmat + (long long)colB * k, (long long)min(16, seg.n - colB) * k);
  };
  const __amdgpu_buffer_rsrc_t rB0 = b_resource(2 * wave), rB1 = b_resource(2 * wave + 1);
  const int offB = (int)(lrow4 * k) + ((chunk ^ q8_swizzle(lrow4)) << 4);
  // scale loads: waves 0..3 the xs of rows 64 wave .., waves 4..7 the ws of B-tile rows 64 (wave - 4) ..
  __amdgpu_buffer_rsrc_t rS;
  int scale_dst;
  if (wave < 4) {
    const int r0 = t.m0 + 64 * wave;
    rS = q8_buffer(p.xs + (long long)r0 * groups, (long long)min(64, p.m - r0) * groups * 4);
    scale_dst = 64 * wave * 4;
  } else {
    const int h = wave - 4;
    const float *src = (t.swiglu && h >= 2) ? seg.w3s : seg.ws;
    const int c0 = t.swiglu ? t.n0 + 64 * (h & 1) : t.n0 + 64 * h;
    rS = q8_buffer(src + (long long)c0 * groups, (long long)min(64, seg.n - c0) * groups * 4);
    scale_dst = (kWTileM + 64 * h) * 4;
  }
  const int offS = lane * groups * 4;
  const __amdgpu_buffer_rsrc_t none = q8_buffer(p.xq, 0);

  // The loads of K step `step` into stage ST; a step past the end loads nothing (zero-length resources).
  auto issue = [&](int step, auto ST) {
    constexpr int st = decltype(ST)::value;
    const bool live = step < s1;
    const int k0 = step * 64;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rA : none,
                                             (void *)(q8_smem + ((2 * wave) * kQWStages + st) * 1024), 16, offA0, k0,
                                             0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rA : none,
                                             (void *)(q8_smem + ((2 * wave + 1) * kQWStages + st) * 1024), 16, offA1,
                                             k0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rB0 : none,
                                             (void *)(q8_smem + kQWBOff + ((2 * wave) * kQWStages + st) * 1024), 16,
                                             offB, k0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rB1 : none,
                                             (void *)(q8_smem + kQWBOff + ((2 * wave + 1) * kQWStages + st) * 1024),
                                             16, offB, k0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rS : none,
                                             (void *)(q8_smem + kQWSOff + st * kQWSStride + scale_dst), 4, offS,
                                             step * 4, 0, 0);
  };

  // Per-lane LDS read bases; the stage, the row tile and the column tile within a half add immediates.
  const int lrow = lane & 15, lr4 = (lane >> 4) * 4;
  const int lane_part = lrow * 64 + (((lane >> 4) ^ q8_swizzle(lrow)) << 4);
  const unsigned char *abase = q8_smem + (4 * wm) * kQWStages * 1024 + lane_part;
  const unsigned char *blo = q8_smem + kQWBOff + (b_row_wide(t.swiglu, wn, 0) / 16) * kQWStages * 1024 + lane_part;
  const unsigned char *bhi = q8_smem + kQWBOff + (b_row_wide(t.swiglu, wn, 4) / 16) * kQWStages * 1024 + lane_part;
  const unsigned char *xsbase = q8_smem + kQWSOff + (64 * wm + lr4) * 4;
  const unsigned char *wslo = q8_smem + kQWSOff + (kWTileM + b_row_wide(t.swiglu, wn, 0) + lrow) * 4;
  const unsigned char *wshi = q8_smem + kQWSOff + (kWTileM + b_row_wide(t.swiglu, wn, 4) + lrow) * 4;

  v4f acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 8; j++)
      acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // The int32 results of two column tiles: round j of a step writes set j % 2 while the VALU rescales the other,
  // written one round earlier (column tile j - 1, or tile 7 of the previous step), so no VALU waits on a running MFMA.
  v4i dot[2][4] = {};

  auto rescale = [&](const v4i &d, float ws, const v4f &xs, v4f &c) {
#pragma unroll
    for (int e = 0; e < 4; e++)
      c[e] = fmaf((float)d[e] * ws, xs[e], c[e]);
  };
  // One step's MFMAs from stage ST. CARRY: tile 7 of the previous step (stage ST - 1, whose scales are still in
  // place) waits in dot[1], rescaled in round 0.
  auto mma_step = [&](auto ST, auto CARRY) {
    constexpr int st = decltype(ST)::value, pst = (st + kQWStages - 1) % kQWStages;
    constexpr bool carry = decltype(CARRY)::value;
    auto b_op = [&](int j) {
      return *reinterpret_cast<const v4i *>((j < 4 ? blo : bhi) + ((j & 3) * kQWStages + st) * 1024);
    };
    auto xs_op = [&](int stage, int i) {
      return *reinterpret_cast<const v4f *>(xsbase + stage * kQWSStride + i * 64);
    };
    auto ws_op = [&](int stage, int j) {
      return *reinterpret_cast<const float *>((j < 4 ? wslo : wshi) + stage * kQWSStride + (j & 3) * 64);
    };
    v4i a[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
      a[i] = *reinterpret_cast<const v4i *>(abase + (i * kQWStages + st) * 1024);
    v4i b = b_op(0);
    v4f xs[4];
    float ws = 0.f;
    if (carry) {
#pragma unroll
      for (int i = 0; i < 4; i++)
        xs[i] = xs_op(pst, i);
      ws = ws_op(pst, 7);
    }
    __builtin_amdgcn_sched_barrier(0);
    // Round j: first the reads the next round needs (its B operand and ws, and in round 0 this step's xs), then four
    // MFMAs into set j % 2, each followed by the 12 VALU instructions of one tile of the other set. The rounds are
    // fenced from each other, so the next round's MFMAs are not hoisted over these rescales.
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const v4i bn = j < 7 ? b_op(j + 1) : b;
      const float wsn = j < 7 ? ws_op(st, j) : ws;
      v4f xsn[4];
      if (j == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++)
          xsn[i] = xs_op(st, i);
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        dot[j & 1][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b, v4i{0, 0, 0, 0}, 0, 0, 0);
        if (j > 0 || carry)
          rescale(dot[(j & 1) ^ 1][i], ws, xs[i], acc[i][j > 0 ? j - 1 : 7]);
      }
      if (j == 0) // DS reads
        __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
      else
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // one MFMA
        if (j > 0 || carry)
          __builtin_amdgcn_sched_group_barrier(0x002, 12, 0); // one tile's convert, multiply, FMA
      }
      __builtin_amdgcn_sched_barrier(0);
      b = bn;
      ws = wsn;
      if (j == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++)
          xs[i] = xsn[i];
      }
    }
  };
  // Step `step` is in stage ST: wait until step + 1 has landed for every wave (the stage of step - 1 is then free for
  // step + 3), then step + 1's MFMAs, after the rescale of step's column tile 7.
  auto advance = [&](int step, auto ST) {
    constexpr int st = decltype(ST)::value, nst = (st + 1) % kQWStages, fill = (st + kQWStages - 1) % kQWStages;
    wait_vmcnt<(kQWStages - 3) * kQWLoadsPerStep>();
    __builtin_amdgcn_s_barrier();
    issue(step + kQWStages - 1, std::integral_constant<int, fill>{});
    mma_step(std::integral_constant<int, nst>{}, std::true_type{});
  };

  issue_first<0, kQWStages - 1>(issue, s0);
  wait_vmcnt<(kQWStages - 2) * kQWLoadsPerStep>(); // step s0 has landed for this wave
  __builtin_amdgcn_s_barrier();                      // ... and for every wave
  mma_step(std::integral_constant<int, 0>{}, std::false_type{});
  // Whole rounds of four steps: the stages of steps past the end hold zeros (zero-length loads), so their MFMAs and
  // rescales add nothing, and advance(s1 - 1), which every round count reaches, rescales the last step's tile 7.
  for (int step = s0; step < s1; step += kQWStages) {
    advance(step, std::integral_constant<int, 0>{});
    advance(step + 1, std::integral_constant<int, 1>{});
    advance(step + 2, std::integral_constant<int, 2>{});
    advance(step + 3, std::integral_constant<int, 3>{});
  }
  // the loads issued for steps past the end still target this block's LDS: let them land before the block exits
  __builtin_amdgcn_s_waitcnt(0);
  if (SPLIT) {
    v4f *slot = p.sk.partial + (size_t)(tile * p.sk.splits + split) * kWSlotV4 + threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 8; j++)
        slot[(i * 8 + j) * kQ8Threads] = acc[i][j];
    return;
  }
  store_tile_wide(seg, t, acc, wm, wn, lane, p.m, p.flags);
}

// ---- W8A8 Q8_0, wide tiles, the scale products on the matrix cores ------------------------------------------------
//
// q8_gemm_wide spends three VALU instructions per output and group (convert, multiply by ws, FMA with xs): 48 cycles
// of a 16-lane SIMD per 16 x 16 tile against the 16 of its int8 MFMA. This kernel takes the product xs[r] * ws[c]
// from the matrix cores instead, so a tile's rescale is a convert and an FMA: c += (float)dot * S[r][c].
//
// S for a wave's 64 rows and one 16-column tile is one v_mfma_f32_32x32x16_bf16 (32 cycles for four tiles). Each FP32
// scale x is split exactly into three bf16 parts, x = h + m + l: h the top 8 significant bits, m the next 8 of x - h,
// l the 8 that remain (each part is the exact high half of a float). Slots 0..7 of K carry eight of the nine cross
// products of the two scales (all but l * l, below 2^-32 of the product): A holds [h h m m h l m l] of xs and B
// [h m h m l h l m] of ws, pairing hh, hm, mh, mm, hl, lh, ml, lm. In that order each dword of A and of B draws on
// the same two of the three parts, so one v_perm with a wave-uniform selector builds either. Bf16 products are exact
// in FP32, so S is xs * ws to FP32 rounding (the MFMA's sum of eight exact terms), where q8_gemm_wide rounds
// (dot * ws) and then its product with xs: the two orders differ in FP32 rounding only.
//
// The 32 x 32 result puts element v of lane l at row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32 (checked on the
// hardware), where the int8 tiles need rows 16 i + 4 (l / 16) + e at column l % 16. So row o of the bf16 tile stands
// for two rows of the wave, one per column half: K slots 0..7 of A row o hold the parts of row
// 16 (o / 8) + 8 ((o % 8) / 4) + o % 4, slots 8..15 those of the row 4 further, and B column c holds its column's
// parts in slots 0..7 when c < 16 and in slots 8..15 when c >= 16 (zeros elsewhere). Lane l then receives in element
// 4 i + e exactly S of its int8 element e of row tile i.
//
// The parts are made once per group for the whole block: each thread splits one scale (xs of a row for waves 0..3, ws
// of a B-tile row for waves 4..7) into a double-buffered parts area. A group's FP32 scales are loaded one step ahead
// of its operands, so when the block waits for step s + 1's operands, step s + 2's scales have landed; they are split
// during step s + 1's MFMAs, and the next barrier publishes them. Results differ from q8_gemm_wide's only in FP32
// rounding; the int32 group dots are the same exact MFMA sums.
constexpr int kQSStages = 4, kQSLoadsPerStep = 5; // per wave: two A blocks, two B blocks, one scale load
constexpr int kQSBOff = 16 * kQSStages * 1024;
constexpr int kQSSOff = kQSBOff + 16 * kQSStages * 1024;
constexpr int kQSSStride = 512 * 4;                              // xs of the 256 rows, then ws of the 256 B-tile rows
constexpr int kQSPOff = kQSSOff + kQSStages * kQSSStride;        // parts: [2 buffers][512 scales] x 16 bytes
constexpr int kQSPBuf = 512 * 16;
constexpr int kQSZOff = kQSPOff + 2 * kQSPBuf;                   // zeros read by the B lanes outside their half
constexpr size_t kQSLds = (size_t)kQSZOff + 1024;                // 153 KB
static_assert(kQSLds <= 160 * 1024, "one wide int8 block fits a CU's LDS");

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

// The wave row whose scale parts sit in slots 0..7 (q = 0) or 8..15 (q = 1) of row o of the bf16 A operand.
__device__ __forceinline__ int smma_row(int o, int q) { return 16 * (o >> 3) + 8 * ((o & 7) >> 2) + 4 * q + (o & 3); }

// v_perm selectors over (S0, S1) picking the high halves: low half from S1 or S0, high half from S1 or S0.
constexpr unsigned kLo1Hi1 = 0x03020302u, kLo1Hi0 = 0x07060302u, kLo0Hi0 = 0x07060706u, kLo0Hi1 = 0x03020706u;

template <bool SPLIT> __global__ __launch_bounds__(kQ8Threads, 2) void q8_gemm_wide_smma(Q8Params p) {
  extern __shared__ __align__(16) unsigned char q8_smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int logical = xcd_logical(blockIdx.x, p.grid.total * (SPLIT ? p.sk.splits : 1));
  const int tile = SPLIT ? __builtin_amdgcn_readfirstlane(logical / p.sk.splits) : logical;
  const int split = SPLIT ? __builtin_amdgcn_readfirstlane(logical % p.sk.splits) : 0;
  const TilePos t = q8_tile_of(p.grid, tile, kWTileM, kWTileN);
  const TileSeg seg = q8_seg_of(p.grid, t.s);
  const int groups = p.k / 64, steps = groups;
  const int s0 = SPLIT ? split * p.sk.per : 0, s1 = SPLIT ? min(steps, s0 + p.sk.per) : steps;
  const long long k = p.k;

  // Operand loads as in q8_gemm_wide: lane l's 16 bytes at l * 16 of a 1 KB block (row l / 4, chunk l % 4 swizzled).
  const int lrow4 = lane >> 2, chunk = lane & 3;
  const int ra = 32 * wave + lrow4;
  const __amdgpu_buffer_rsrc_t rA = q8_buffer(p.xq + (long long)t.m0 * k, (long long)min(kWTileM, p.m - t.m0) * k);
  const int offA0 = (int)(ra * k) + ((chunk ^ q8_swizzle(ra)) << 4);
  const int offA1 = (int)((ra + 16) * k) + ((chunk ^ q8_swizzle(ra + 16)) << 4);
  auto b_resource = [&](int blk) {
    const int rb = 16 * blk;
    const int colB = t.swiglu ? t.n0 + (rb & 127) : t.n0 + rb;
    const int8_t *wmat = (const int8_t *)((t.swiglu && rb >= 128) ? seg.w3 : seg.w);
    return q8_buffer(wmat + (long long)colB * k, (long long)min(16, seg.n - colB) * k);
  };
  const __amdgpu_buffer_rsrc_t rB0 = b_resource(2 * wave), rB1 = b_resource(2 * wave + 1);
  const int offB = (int)(lrow4 * k) + ((chunk ^ q8_swizzle(lrow4)) << 4);
  // Scale loads: thread (wave, lane) loads scale 64 wave + lane of the step: the xs of row 64 wave + lane (waves 0..3)
  // or the ws of B-tile row 64 (wave - 4) + lane (waves 4..7), and later splits that same scale. Rows past m or n
  // load zeros (bounded resources).
  __amdgpu_buffer_rsrc_t rS;
  if (wave < 4) {
    const int r0 = t.m0 + 64 * wave;
    rS = q8_buffer(p.xs + (long long)r0 * groups, (long long)min(64, p.m - r0) * groups * 4);
  } else {
    const int h = wave - 4;
    const float *src = (t.swiglu && h >= 2) ? seg.w3s : seg.ws;
    const int c0 = t.swiglu ? t.n0 + 64 * (h & 1) : t.n0 + 64 * h;
    rS = q8_buffer(src + (long long)c0 * groups, (long long)min(64, seg.n - c0) * groups * 4);
  }
  const int offS = lane * groups * 4;
  const __amdgpu_buffer_rsrc_t none = q8_buffer(p.xq, 0);

  // The scales of K step `step` into scale stage SST (a step past the end loads zeros).
  auto issue_scales = [&](int step, auto SST) {
    constexpr int sst = decltype(SST)::value;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(step < s1 ? rS : none,
                                             (void *)(q8_smem + kQSSOff + sst * kQSSStride + 64 * wave * 4), 4, offS,
                                             step * 4, 0, 0);
  };
  // Stage ST gets step `step`'s operands; the scales going out with them are step + 1's (scale stage ST + 1).
  auto issue = [&](int step, auto ST) {
    constexpr int st = decltype(ST)::value;
    const bool live = step < s1;
    const int k0 = step * 64;
    issue_scales(step + 1, std::integral_constant<int, (st + 1) % kQSStages>{});
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rA : none,
                                             (void *)(q8_smem + ((2 * wave) * kQSStages + st) * 1024), 16, offA0, k0,
                                             0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rA : none,
                                             (void *)(q8_smem + ((2 * wave + 1) * kQSStages + st) * 1024), 16, offA1,
                                             k0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rB0 : none,
                                             (void *)(q8_smem + kQSBOff + ((2 * wave) * kQSStages + st) * 1024), 16,
                                             offB, k0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(live ? rB1 : none,
                                             (void *)(q8_smem + kQSBOff + ((2 * wave + 1) * kQSStages + st) * 1024),
                                             16, offB, k0, 0, 0);
  };

  // Splitting this thread's scale of scale stage SST into parts buffer PAR (parts of scale i at 16 i of the buffer).
  const unsigned char *own_scale = q8_smem + kQSSOff + (64 * wave + lane) * 4;
  unsigned char *own_parts = q8_smem + kQSPOff + (64 * wave + lane) * 16;
  // xs parts (waves 0..3) go to slots h h m m h l m l, ws parts (waves 4..7) to h m h m l h l m
  const bool xs_wave = wave < 4;
  const unsigned sel0 = xs_wave ? kLo1Hi1 : kLo1Hi0, sel1 = xs_wave ? kLo0Hi0 : kLo1Hi0;
  const unsigned sel23 = xs_wave ? kLo1Hi0 : kLo0Hi1;
  auto split_scale = [&](float x, auto PAR) {
    constexpr int par = decltype(PAR)::value;
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const float r1 = x - __builtin_bit_cast(float, u & 0xFFFF0000u); // exact: the bits of x below its top 8
    const unsigned u1 = __builtin_bit_cast(unsigned, r1);
    const float r2 = r1 - __builtin_bit_cast(float, u1 & 0xFFFF0000u); // exact, and at most 8 significant bits
    const unsigned u2 = __builtin_bit_cast(unsigned, r2);
    const v4i parts{(int)__builtin_amdgcn_perm(u1, u, sel0), (int)__builtin_amdgcn_perm(u1, u, sel1),
                    (int)__builtin_amdgcn_perm(u2, u, sel23), (int)__builtin_amdgcn_perm(u2, u1, sel23)};
    *reinterpret_cast<v4i *>(own_parts + par * kQSPBuf) = parts;
  };

  // Per-lane LDS read bases.
  const int lrow = lane & 15;
  const int lane_part = lrow * 64 + (((lane >> 4) ^ q8_swizzle(lrow)) << 4);
  const unsigned char *abase = q8_smem + (4 * wm) * kQSStages * 1024 + lane_part;
  const unsigned char *blo = q8_smem + kQSBOff + (b_row_wide(t.swiglu, wn, 0) / 16) * kQSStages * 1024 + lane_part;
  const unsigned char *bhi = q8_smem + kQSBOff + (b_row_wide(t.swiglu, wn, 4) / 16) * kQSStages * 1024 + lane_part;
  // bf16 A operand: lane l holds row o = l % 32 of the 32 x 16 tile, slots 8 (l / 32) ..: the parts of one wave row
  const unsigned char *xsparts = q8_smem + kQSPOff + (64 * wm + smma_row(lane & 31, lane >> 5)) * 16;
  // bf16 B operand: lane l holds column l % 32, slots 8 (l / 32) ..: parts of column l % 16 of the column tile for
  // lanes 0..15 and 48..63, zeros for lanes 16..47 (one base per parts buffer, so the zero block only needs to cover
  // the column tiles' offsets, 256 bytes apart)
  const bool bs_live = lane < 16 || lane >= 48;
  const unsigned char *zeros = q8_smem + kQSZOff;
  const unsigned char *wslo0 = bs_live ? q8_smem + kQSPOff + (kWTileM + b_row_wide(t.swiglu, wn, 0) + lrow) * 16 : zeros;
  const unsigned char *wshi0 = bs_live ? q8_smem + kQSPOff + (kWTileM + b_row_wide(t.swiglu, wn, 4) + lrow) * 16 : zeros;
  const unsigned char *wslo1 = bs_live ? wslo0 + kQSPBuf : zeros, *wshi1 = bs_live ? wshi0 + kQSPBuf : zeros;
  if (threadIdx.x < 1024 / 16)
    *reinterpret_cast<v4i *>(q8_smem + kQSZOff + threadIdx.x * 16) = v4i{0, 0, 0, 0};

  v4f acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 8; j++)
      acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // Round j of a step writes the int32 results and the scale products of column tile j into set j % 2 while the
  // VALU folds in the other set, written one round earlier (column tile j - 1, or tile 7 of the previous step).
  v4i dot[2][4] = {};
  v16f sprod[2] = {};

  auto rescale = [&](const v4i &d, const v16f &s, int i, v4f &c) {
#pragma unroll
    for (int e = 0; e < 4; e++)
      c[e] = fmaf((float)d[e], s[4 * i + e], c[e]);
  };
  // One step's MFMAs from operand stage ST and parts buffer PAR; meanwhile this thread splits its scale of scale stage
  // SST into parts buffer SPAR (SST < 0: none). CARRY: tile 7 of the previous step waits in set 1.
  auto mma_step = [&](auto ST, auto PAR, auto CARRY, auto SST, auto SPAR) {
    constexpr int st = decltype(ST)::value, par = decltype(PAR)::value;
    constexpr bool carry = decltype(CARRY)::value;
    constexpr int sst = decltype(SST)::value, spar = decltype(SPAR)::value;
    auto b_op = [&](int j) {
      return *reinterpret_cast<const v4i *>((j < 4 ? blo : bhi) + ((j & 3) * kQSStages + st) * 1024);
    };
    auto ws_op = [&](int j) {
      const unsigned char *base = par ? (j < 4 ? wslo1 : wshi1) : (j < 4 ? wslo0 : wshi0);
      return *reinterpret_cast<const v8bf *>(base + (j & 3) * 256);
    };
    v4i a[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
      a[i] = *reinterpret_cast<const v4i *>(abase + (i * kQSStages + st) * 1024);
    const v8bf xsp = *reinterpret_cast<const v8bf *>(xsparts + par * kQSPBuf);
    v4i b = b_op(0);
    v8bf wsp = ws_op(0);
    float scale = 0.0f;
    if constexpr (sst >= 0)
      scale = *reinterpret_cast<const float *>(own_scale + sst * kQSSStride);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const v4i bn = j < 7 ? b_op(j + 1) : b;
      const v8bf wspn = j < 7 ? ws_op(j + 1) : wsp;
      sprod[j & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xsp, wsp, v16f{}, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        dot[j & 1][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b, v4i{0, 0, 0, 0}, 0, 0, 0);
        if (j > 0 || carry)
          rescale(dot[(j & 1) ^ 1][i], sprod[(j & 1) ^ 1], i, acc[i][j > 0 ? j - 1 : 7]);
      }
      if constexpr (sst >= 0) {
        if (j == 3)
          split_scale(scale, std::integral_constant<int, spar>{});
      }
      if (j < 7)
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0); // the next round's DS reads
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // the scale-product MFMA
#pragma unroll
      for (int i = 0; i < 4; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // one int8 MFMA
        if (j > 0 || carry)
          __builtin_amdgcn_sched_group_barrier(0x002, 8, 0); // one tile's convert and FMA
      }
      if (sst >= 0 && j == 3) {
        __builtin_amdgcn_sched_group_barrier(0x002, 8, 0); // splitting the scale
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0); // storing its parts
      }
      __builtin_amdgcn_sched_barrier(0);
      b = bn;
      wsp = wspn;
    }
  };
  // Step `step` is in stage ST: wait until step + 1's operands (and so step + 2's scales) have landed for every wave,
  // load step + 3 (with step + 4's scales), then step + 1's MFMAs while step + 2's scales are split.
  auto advance = [&](int step, auto ST) {
    constexpr int st = decltype(ST)::value, nst = (st + 1) % kQSStages, fill = (st + kQSStages - 1) % kQSStages;
    wait_vmcnt_lgkm0<kQSLoadsPerStep>(); // ... and this thread's parts store of the last step
    __builtin_amdgcn_s_barrier();
    issue(step + kQSStages - 1, std::integral_constant<int, fill>{});
    mma_step(std::integral_constant<int, nst>{}, std::integral_constant<int, nst % 2>{}, std::true_type{},
             std::integral_constant<int, (st + 2) % kQSStages>{}, std::integral_constant<int, st % 2>{});
  };

  issue_scales(s0, std::integral_constant<int, 0>{});
  issue_first<0, kQSStages - 1>(issue, s0);
  wait_vmcnt<(kQSStages - 1) * kQSLoadsPerStep>(); // step s0's scales have landed for this wave
  __builtin_amdgcn_s_barrier();                      // ... and for every wave (the zero block is written too)
  split_scale(*reinterpret_cast<const float *>(own_scale), std::integral_constant<int, 0>{});
  wait_vmcnt_lgkm0<(kQSStages - 2) * kQSLoadsPerStep>(); // step s0's operands, s0 + 1's scales, the parts store
  __builtin_amdgcn_s_barrier();
  mma_step(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, std::false_type{},
           std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
  for (int step = s0; step < s1; step += kQSStages) {
    advance(step, std::integral_constant<int, 0>{});
    advance(step + 1, std::integral_constant<int, 1>{});
    advance(step + 2, std::integral_constant<int, 2>{});
    advance(step + 3, std::integral_constant<int, 3>{});
  }
  __builtin_amdgcn_s_waitcnt(0);
  if (SPLIT) {
    v4f *slot = p.sk.partial + (size_t)(tile * p.sk.splits + split) * kWSlotV4 + threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 8; j++)
        slot[(i * 8 + j) * kQ8Threads] = acc[i][j];
    return;
  }
  store_tile_wide(seg, t, acc, wm, wn, lane, p.m, p.flags);
}

// Any group size (gs % 64 != 0): one thread per output, the per-group int32 dot in plain integer arithmetic.
__global__ __launch_bounds__(kBlock) void q8_gemm_generic(TileGrid g, const int8_t *xq, const float *xs, int m, int k,
                                                          int gs) {
  long long idx = (long long)blockIdx.x * kBlock + threadIdx.x;
  int s = 0;
  long long base = 0;
  for (; s < g.nseg; s++) {
    const long long count = (long long)m * g.seg[s].n;
    if (idx < base + count)
      break;
    base += count;
  }
  if (s >= g.nseg)
    return;
  const TileSeg seg = seg_of(g, s);
  const long long local = idx - base;
  const int row = (int)(local / seg.n), col = (int)(local % seg.n);
  const int groups = k / gs;
  auto dots = [&](const int8_t *w, const float *ws) {
    const int8_t *x = xq + (long long)row * k, *wr = w + (long long)col * k;
    float total = 0.0f;
    for (int grp = 0; grp < groups; grp++) {
      int d = 0;
      for (int t = 0; t < gs; t++)
        d += (int)x[grp * gs + t] * (int)wr[grp * gs + t];
      total += ((float)d * ws[(long long)col * groups + grp]) * xs[(long long)row * groups + grp];
    }
    return total;
  };
  const float sum = dots((const int8_t *)seg.w, seg.ws);
  float *o = seg.c + (long long)row * seg.ldc + col;
  if (seg.epi == EPI_SWIGLU)
    *o = silu_gate(sum, dots((const int8_t *)seg.w3, seg.w3s));
  else if (seg.epi == EPI_ADD)
    *o += sum;
  else
    *o = sum;
}

// ---- FP32 and BF16 on MFMA -----------------------------------------------------------------------------------------

constexpr int kF32Slice = 16; // K values staged per step
constexpr int kF32Pitch = 17; // floats per LDS row of a K slice, padded against bank conflicts

struct F32Params {
  TileGrid grid;
  const float *a;
  long long lda;
  int m, k;
};

// FP32: v_mfma_f32_16x16x4_f32, K staged 16 at a time; lane l supplies A[l % 16][k0 + l / 16] and the matching W value.
__global__ __launch_bounds__(kBlock) void f32_gemm_mfma(F32Params p) {
  __shared__ float sa[2][kTile * kF32Pitch];
  __shared__ float sb[2][kTile * kF32Pitch];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
  const TilePos t = tile_of(p.grid, xcd_logical(blockIdx.x, p.grid.total));
  const TileSeg seg = seg_of(p.grid, t.s);
  const float *w1 = (const float *)seg.w, *w3 = (const float *)seg.w3;
  const int steps = (p.k + kF32Slice - 1) / kF32Slice;
  float ra[8], rb[8];
  // thread t moves rows (t / 16) + 16 h (h = 0..7) at column t % 16 of each 128 x 16 slice
  auto load = [&](int step) {
    const int kk = step * kF32Slice + (tid & 15);
#pragma unroll
    for (int h = 0; h < 8; h++) {
      const int r = (tid >> 4) + 16 * h;
      const int row = t.m0 + r;
      ra[h] = (row < p.m && kk < p.k) ? p.a[(long long)row * p.lda + kk] : 0.0f;
      const int wc = b_col(t, r);
      const float *src = (t.swiglu && r >= 64) ? w3 : w1;
      rb[h] = (wc < seg.n && kk < p.k) ? src[(long long)wc * seg.ldw + kk] : 0.0f;
    }
  };
  auto store = [&](int buf) {
    const int col = tid & 15;
#pragma unroll
    for (int h = 0; h < 8; h++) {
      const int r = (tid >> 4) + 16 * h;
      sa[buf][r * kF32Pitch + col] = ra[h];
      sb[buf][r * kF32Pitch + col] = rb[h];
    }
  };
  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
      acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  load(0);
  store(0);
  __syncthreads();
  const int lrow = lane & 15, lk = lane >> 4;
  for (int step = 0; step < steps; step++) {
    const int buf = step & 1;
    if (step + 1 < steps)
      load(step + 1);
#pragma unroll
    for (int kk = 0; kk < kF32Slice; kk += 4) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; i++)
        a[i] = sa[buf][(wm * 64 + 16 * i + lrow) * kF32Pitch + kk + lk];
#pragma unroll
      for (int j = 0; j < 4; j++)
        b[j] = sb[buf][(b_row(t.swiglu, wn, j) + lrow) * kF32Pitch + kk + lk];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (step + 1 < steps)
      store(buf ^ 1);
    __syncthreads();
  }
  store_tile(seg, t, acc, wm, wn, lane, p.m);
}


bool launch_ok(const char *what) {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess)
    return true;
  return raise("launching %s failed: %s", what, hipGetErrorString(e));
}

template <int J, int THREADS> bool launch_split_reduce(const Q8Grid &grid, const SplitK &sk, int m, int tile_m,
                                                       int tile_n, hipStream_t stream) {
  SplitOut o{grid, sk.partial, sk.splits, m, tile_m, tile_n};
  const long long threads = 4LL * (J / 2) * THREADS * grid.total;
  hipLaunchKernelGGL((split_reduce<J, THREADS>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, o);
  return launch_ok("split_reduce");
}

TileGrid make_grid(const GemmSegmentDev *segs, int nseg, int m) {
  TileGrid g{};
  g.nseg = nseg;
  g.mtiles = (m + kTile - 1) / kTile;
  int tiles = 0;
  for (int s = 0; s < nseg; s++) {
    const GemmSegmentDev &d = segs[s];
    const int width = d.epi == EPI_SWIGLU ? kTile / 2 : kTile;
    g.seg[s] = TileSeg{d.c,   d.ldc, d.w,   d.w3,  d.ws, d.w3s, (long long)d.ldw, d.n, d.epi, tiles, (d.n + width - 1) / width,
                       d.cq, d.cs};
    tiles += g.seg[s].ntiles * g.mtiles;
  }
  g.total = tiles;
  return g;
}

Q8Grid make_q8_grid(const GemmSegmentDev *segs, int nseg, int m, int tile_m = kQ8TileM, int tile_n = kQ8TileN) {
  Q8Grid g{};
  g.nseg = nseg;
  g.mtiles = (m + tile_m - 1) / tile_m;
  int tiles = 0;
  for (int s = 0; s < nseg; s++) {
    const GemmSegmentDev &d = segs[s];
    const int width = d.epi == EPI_SWIGLU ? tile_n / 2 : tile_n;
    g.seg[s] = TileSeg{d.c,   d.ldc, d.w,   d.w3,  d.ws, d.w3s, (long long)d.ldw, d.n, d.epi, tiles, (d.n + width - 1) / width,
                       d.cq, d.cs};
    tiles += g.seg[s].ntiles * g.mtiles;
  }
  g.total = tiles;
  return g;
}

std::atomic<int> forced_splits{0};

// Blocks per tile: one when the tiles fill the CUs (one 256 x 128 block per CU fits in LDS), else enough to reach
// about one block per CU, keeping at least eight K steps per block and within the workspace's partial tiles. A
// block's steps are a multiple of `unit` (the int8 kernel's steps per scale group).
int choose_splits(int tiles, int steps, int *per, int unit = 1, int slots = kSplitSlots) {
  int s = forced_splits.load();
  if (s <= 0) {
    const int cus = device().cu_count > 0 ? device().cu_count : 256;
    s = tiles < cus ? cus / tiles : 1;
    s = min(s, steps / 8);
  }
  s = max(1, min(s, min(slots / max(tiles, 1), steps)));
  *per = ((steps + s - 1) / s + unit - 1) / unit * unit;
  return (steps + *per - 1) / *per; // no empty split
}

struct SegList {
  const GemmSegmentDev *seg;
  int nseg;
};

// The pipelined kernel takes more than the default 64 KB of dynamic LDS: raised once per instantiation.
template <class C, bool PROBE, bool GS64, bool SPLIT, bool QUANT = false> bool q8_ready() {
  static const hipError_t status = hipFuncSetAttribute((const void *)q8_gemm_lds<C, PROBE, GS64, SPLIT, QUANT>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::Lds);
  return check_hip(status, "allowing the Q8 GEMM its LDS");
}

template <class C, bool PROBE, bool GS64, bool QUANT = false>
bool q8_launch(Q8Params p, const SegList &segs, hipStream_t stream) {
  p.grid = make_q8_grid(segs.seg, segs.nseg, p.m, C::TileM);
  if (p.grid.total <= 0)
    return true;
  const int steps = p.k / 64;
  p.sk.splits = p.grid.total > kSplitSlots ? 1 : choose_splits(p.grid.total, steps, &p.sk.per, p.gs / 64);
  if (p.sk.splits == 1)
    p.sk.per = steps;
  p.sk.partial = (v4f *)device().split_partial;
  p.sk.count = device().split_count;
  if (p.sk.splits == 1) {
    if (!q8_ready<C, PROBE, GS64, false, QUANT>())
      return false;
    hipLaunchKernelGGL((q8_gemm_lds<C, PROBE, GS64, false, QUANT>), dim3((unsigned)p.grid.total), dim3(C::Threads), C::Lds,
                       stream, p);
    return launch_ok("q8_gemm_lds");
  }
  if (QUANT) // the quantized epilogue has no split form
    return raise("q8_gemm_lds: a quantized SwiGLU output cannot be split");
  if (!q8_ready<C, PROBE, GS64, true>())
    return false;
  hipLaunchKernelGGL((q8_gemm_lds<C, PROBE, GS64, true>), dim3((unsigned)(p.grid.total * p.sk.splits)),
                     dim3(C::Threads), C::Lds, stream, p);
  if (!launch_ok("q8_gemm_lds"))
    return false;
  return launch_split_reduce<4, C::Threads>(p.grid, p.sk, p.m, C::TileM, kQ8TileN, stream);
}

// Tile shape: 256 x 128 unless LLAMA_HIP_Q8_TILE_M = 128 (read once). On the 8B W1/W3 shape the 128-row tiles with
// two blocks per CU measured about 5% slower: the extra A traffic costs more than the second block's overlap gains.
int q8_tile_m() {
  static const int tile = [] {
    const char *env = getenv("LLAMA_HIP_Q8_TILE_M");
    return env && atoi(env) == 128 ? 128 : 256;
  }();
  return tile;
}

std::atomic<int> forced_q8_tile{0}; // llhip_set_q8_tile: 0 unset, 1 narrow, 2 wide

// The wide kernel (256 x 256 tiles) for gs = 64, when it is picked: LLAMA_HIP_Q8_TILE = wide / narrow (read once) or
// llhip_set_q8_tile force it; otherwise by grid. A wide tile takes about 1.7 times a 256 x 128 tile (measured on the
// 8B shapes at 1024 to 4096 rows: 15% less time per output), so the wide grid wins when its rounds of one tile per CU,
// weighted 1.7, are fewer than the narrow grid's. Grids of fewer narrow tiles than CUs keep the narrow kernel, whose
// split K fills the CUs. Measured (us, narrow / wide): W1/W3 of 2048 rows 507 / 492 (7 rounds against 3.5), QKV 137 /
// 120 (2 against 1); Wo and W2 87 / 101 and 243 / 252 (one round each); at 4096 rows Wo 170 / 156, W2 483 / 443.
bool q8_use_wide(const Q8Params &p, const SegList &segs) {
  if (p.gs != 64)
    return false;
  static const int env_tile = [] {
    const char *env = getenv("LLAMA_HIP_Q8_TILE");
    return env && !strcmp(env, "wide") ? 2 : env && !strcmp(env, "narrow") ? 1 : 0;
  }();
  const int forced = forced_q8_tile.load() ? forced_q8_tile.load() : env_tile;
  if (forced)
    return forced == 2;
  const int cus = device().cu_count > 0 ? device().cu_count : 256;
  const int narrow = make_q8_grid(segs.seg, segs.nseg, p.m).total;
  if (narrow < cus)
    return false;
  const int wide = make_q8_grid(segs.seg, segs.nseg, p.m, kWTileM, kWTileN).total;
  return 17LL * ((wide + cus - 1) / cus) < 10LL * ((narrow + cus - 1) / cus);
}

// The wide int8 kernel's grid and split count; its partial tiles are twice the size, so half as many fit the workspace.
void q8_wide_grid(Q8Params &p, const SegList &segs) {
  constexpr int kWideSlots = kSplitSlots / 2;
  p.grid = make_q8_grid(segs.seg, segs.nseg, p.m, kWTileM, kWTileN);
  const int steps = p.k / 64;
  p.sk.splits = p.grid.total > kWideSlots ? 1 : choose_splits(p.grid.total, steps, &p.sk.per, 1, kWideSlots);
  if (p.sk.splits == 1)
    p.sk.per = steps;
  p.sk.partial = (v4f *)device().split_partial;
  p.sk.count = device().split_count;
}

std::atomic<int> forced_q8_scales{0}; // llhip_set_q8_scales: 0 unset, 1 VALU products, 2 matrix-core products

// Which wide kernel forms the per-group scale products: q8_gemm_wide_smma (on the matrix cores) unless
// LLAMA_HIP_Q8_SCALES = valu (read once) or llhip_set_q8_scales picks q8_gemm_wide.
bool q8_scales_on_mfma() {
  static const int env = [] {
    const char *v = getenv("LLAMA_HIP_Q8_SCALES");
    return v && !strcmp(v, "valu") ? 1 : v && !strcmp(v, "mfma") ? 2 : 0;
  }();
  const int forced = forced_q8_scales.load() ? forced_q8_scales.load() : env;
  return forced != 1;
}

// One launch of a wide int8 kernel (SPLIT: the partial-tile instantiation), its LDS allowance raised once.
bool q8_wide_kernel(const Q8Params &p, bool split, unsigned blocks, hipStream_t stream) {
  static const hipError_t a[4] = {
      hipFuncSetAttribute((const void *)q8_gemm_wide<false>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kQWLds),
      hipFuncSetAttribute((const void *)q8_gemm_wide<true>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kQWLds),
      hipFuncSetAttribute((const void *)q8_gemm_wide_smma<false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)kQSLds),
      hipFuncSetAttribute((const void *)q8_gemm_wide_smma<true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)kQSLds)};
  const bool smma = q8_scales_on_mfma();
  if (!check_hip(a[2 * smma + split], "allowing the Q8 GEMM its LDS"))
    return false;
  if (smma) {
    if (split)
      hipLaunchKernelGGL(q8_gemm_wide_smma<true>, dim3(blocks), dim3(kQ8Threads), kQSLds, stream, p);
    else
      hipLaunchKernelGGL(q8_gemm_wide_smma<false>, dim3(blocks), dim3(kQ8Threads), kQSLds, stream, p);
    return launch_ok("q8_gemm_wide_smma");
  }
  if (split)
    hipLaunchKernelGGL(q8_gemm_wide<true>, dim3(blocks), dim3(kQ8Threads), kQWLds, stream, p);
  else
    hipLaunchKernelGGL(q8_gemm_wide<false>, dim3(blocks), dim3(kQ8Threads), kQWLds, stream, p);
  return launch_ok("q8_gemm_wide");
}

// A wide grid of whole rounds of one tile per CU plus a partial last round: the partial round costs a whole round's
// time (a wide block is bound by its own MFMA and VALU work, not by bandwidth the idle CUs would leave it), so when
// that round is at most half the CUs and whole column tiles across every row tile, its columns go to the 256 x 128
// kernel instead, one round of tiles that take 1 / 1.7 of a wide tile's time. One segment; with the quantized output
// (seg.cq) only where the 256 x 128 tiles are exactly one round (they then run unsplit, and their epilogue quantizes
// whole 64-column groups). Returns the first columns' segment in `head` and the rest in `tail`, or false to leave the
// grid whole.
bool q8_wide_tail(const Q8Params &p, const GemmSegmentDev &seg, GemmSegmentDev &head, GemmSegmentDev &tail) {
  if (p.grid.nseg != 1 || p.sk.splits != 1)
    return false;
  const int cus = device().cu_count > 0 ? device().cu_count : 256;
  const int rest = p.grid.total % cus, mtiles = p.grid.mtiles;
  if (p.grid.total < cus || rest == 0 || 2 * rest > cus || rest % mtiles ||
      (seg.cq && (2 * rest != cus || forced_splits.load() > 1)))
    return false;
  const int width = seg.epi == EPI_SWIGLU ? kWTileN / 2 : kWTileN;
  const int n1 = (p.grid.seg[0].ntiles - rest / mtiles) * width;
  if (n1 <= 0 || n1 >= seg.n)
    return false;
  const long long groups = p.k / p.gs;
  head = seg;
  head.n = n1;
  tail = seg;
  tail.n = seg.n - n1;
  tail.c = seg.c ? seg.c + n1 : nullptr;
  if (seg.cq) { // the same row strides (seg.n): the tail's columns of cq and their groups' scales
    tail.cq = seg.cq + n1;
    tail.cs = seg.cs + n1 / 64;
  }
  tail.w = (const int8_t *)seg.w + (long long)n1 * p.k;
  tail.ws = seg.ws + n1 * groups;
  if (seg.epi == EPI_SWIGLU) {
    tail.w3 = (const int8_t *)seg.w3 + (long long)n1 * p.k;
    tail.w3s = seg.w3s + n1 * groups;
  }
  return true;
}

bool q8_wide_launch(Q8Params p, const SegList &segs, hipStream_t stream) {
  q8_wide_grid(p, segs);
  if (p.grid.total <= 0)
    return true;
  GemmSegmentDev head, tail;
  if (q8_wide_tail(p, segs.seg[0], head, tail)) {
    q8_wide_grid(p, SegList{&head, 1});
    if (!q8_wide_kernel(p, false, (unsigned)p.grid.total, stream))
      return false;
    const SegList rest{&tail, 1};
    return q8_tile_m() == 256 ? q8_launch<Q8Wide, false, true>(p, rest, stream) : q8_launch<Q8Pair, false, true>(p, rest, stream);
  }
  if (p.sk.splits == 1)
    return q8_wide_kernel(p, false, (unsigned)p.grid.total, stream);
  if (!q8_wide_kernel(p, true, (unsigned)(p.grid.total * p.sk.splits), stream))
    return false;
  return launch_split_reduce<8, kQ8Threads>(p.grid, p.sk, p.m, kWTileM, kWTileN, stream);
}

template <bool PROBE> bool launch_q8_lds(Q8Params p, const GemmSegmentDev *segs, int nseg, hipStream_t stream) {
  const SegList list{segs, nseg};
  if (!PROBE && q8_use_wide(p, list))
    return q8_wide_launch(p, list, stream);
  if (q8_tile_m() == 256)
    return p.gs == 64 ? q8_launch<Q8Wide, PROBE, true>(p, list, stream) : q8_launch<Q8Wide, PROBE, false>(p, list, stream);
  return p.gs == 64 ? q8_launch<Q8Pair, PROBE, true>(p, list, stream) : q8_launch<Q8Pair, PROBE, false>(p, list, stream);
}

} // namespace

// Shapes the pipelined kernel takes: gs a multiple of 64, 16-byte aligned operands whose 32-bit buffer offsets fit.
bool q8_gemm_fast_path(const int8_t *xq, int m, int k, int gs) {
  return gs > 0 && gs % 64 == 0 && k % gs == 0 && ((uintptr_t)xq & 15) == 0 &&
         (long long)kQ8TileM * k < (1LL << 31) && (long long)m * (k / gs) * 4 < (1LL << 31);
}

bool launch_q8_gemm(const GemmQ8Job &job, hipStream_t stream) {
  if (job.m <= 0 || job.k <= 0)
    return true;
  if (q8_gemm_skinny_path(job.xq, job.m, job.k, job.gs) && !forced_splits.load())
    return launch_q8_gemm_skinny(job, stream);
  Q8Params p{};
  p.xq = job.xq;
  p.xs = job.xs;
  p.m = job.m;
  p.k = job.k;
  p.gs = job.gs;
  p.flags = device().error_flags;
  return launch_q8_lds<false>(p, job.seg, job.nseg, stream);
}

bool launch_q8_gemm_swiglu_quantized(const GemmQ8Job &job, hipStream_t stream) {
  const GemmSegmentDev &seg = job.seg[0];
  if (job.nseg != 1 || seg.epi != EPI_SWIGLU || !seg.cq || !seg.cs || seg.n % 64 || job.gs != 64 || job.m <= 0 ||
      !q8_gemm_fast_path(job.xq, job.m, job.k, job.gs) ||
      (q8_gemm_skinny_path(job.xq, job.m, job.k, job.gs) && !forced_splits.load()))
    return false;
  Q8Params p{};
  p.xq = job.xq;
  p.xs = job.xs;
  p.m = job.m;
  p.k = job.k;
  p.gs = job.gs;
  p.flags = device().error_flags;
  const SegList list{job.seg, 1};
  if (!q8_use_wide(p, list))
    return false;
  q8_wide_grid(p, list);
  if (p.sk.splits != 1 || p.grid.total <= 0)
    return false;
  GemmSegmentDev head, tail;
  if (q8_wide_tail(p, job.seg[0], head, tail)) { // a partial last round: its columns on the 256 x 128 kernel
    q8_wide_grid(p, SegList{&head, 1});
    if (!q8_wide_kernel(p, false, (unsigned)p.grid.total, stream))
      return false;
    const SegList rest{&tail, 1};
    return q8_tile_m() == 256 ? q8_launch<Q8Wide, false, true, true>(p, rest, stream)
                              : q8_launch<Q8Pair, false, true, true>(p, rest, stream);
  }
  return q8_wide_kernel(p, false, (unsigned)p.grid.total, stream);
}

bool launch_q8_gemm_generic(const GemmQ8Job &job, hipStream_t stream) {
  if (job.m <= 0 || job.k <= 0)
    return true;
  TileGrid g = make_grid(job.seg, job.nseg, job.m);
  long long outputs = 0;
  for (int s = 0; s < job.nseg; s++)
    outputs += (long long)job.m * job.seg[s].n;
  if (!outputs)
    return true;
  hipLaunchKernelGGL(q8_gemm_generic, dim3((unsigned)((outputs + kBlock - 1) / kBlock)), dim3(kBlock), 0, stream, g,
                     job.xq, job.xs, job.m, job.k, job.gs);
  return launch_ok("q8_gemm_generic");
}

namespace {
// The pack_s8_vnni layout (16-row tiles, K in quads: byte ((t * quads + q) * 16 + c) * 4 + e holds row 16 t + c,
// column 4 q + e) back to row-major n x k; one thread per quad of one row.
__global__ __launch_bounds__(kBlock) void s8_vnni_unpack(int8_t *__restrict__ w, const int8_t *__restrict__ packed,
                                                         int n, int k) {
  const long long idx = (long long)blockIdx.x * kBlock + threadIdx.x;
  const int quads = k / 4;
  if (idx >= (long long)n * quads)
    return;
  const int row = (int)(idx / quads), q = (int)(idx % quads);
  const int t = row / 16, c = row % 16;
  *reinterpret_cast<int *>(w + (long long)row * k + 4 * q) =
      *reinterpret_cast<const int *>(packed + (((long long)t * quads + q) * 16 + c) * 4);
}
} // namespace

bool launch_s8_vnni_unpack(int8_t *w, const int8_t *packed, int n, int k, hipStream_t stream) {
  const long long threads = (long long)n * (k / 4);
  hipLaunchKernelGGL(s8_vnni_unpack, dim3((unsigned)((threads + kBlock - 1) / kBlock)), dim3(kBlock), 0, stream, w,
                     packed, n, k);
  return launch_ok("s8_vnni_unpack");
}

bool launch_q8_group_dots(int32_t *dots, const int8_t *xq, int m, int k, int gs, const int8_t *wq, int n,
                          hipStream_t stream) {
  if (m <= 0 || n <= 0 || k <= 0)
    return true;
  // The same kernel as k_gemm_q8 with unit scales, a scratch output and the probe on.
  float *scratch = nullptr, *ones = nullptr;
  const int groups = k / gs;
  const size_t ones_count = (size_t)(m > n ? m : n) * groups;
  if (!LLHIP_CHECK(hipMallocAsync((void **)&scratch, (size_t)m * n * sizeof(float), stream)) ||
      !LLHIP_CHECK(hipMallocAsync((void **)&ones, ones_count * sizeof(float), stream)))
    return false;
  std::vector<float> host_ones(ones_count, 1.0f);
  if (!LLHIP_CHECK(hipMemcpyAsync(ones, host_ones.data(), ones_count * sizeof(float), hipMemcpyHostToDevice, stream)) ||
      !LLHIP_CHECK(hipStreamSynchronize(stream)))
    return false;
  GemmSegmentDev seg{scratch, n, wq, nullptr, ones, nullptr, (size_t)k, n, EPI_STORE};
  Q8Params p{};
  p.xq = xq;
  p.xs = ones;
  p.m = m;
  p.k = k;
  p.gs = gs;
  p.probe = dots;
  bool ok = launch_q8_lds<true>(p, &seg, 1, stream);
  (void)hipFreeAsync(scratch, stream);
  (void)hipFreeAsync(ones, stream);
  return ok;
}

namespace {

// Which kernel takes the aligned FP32 GEMM: mm_gemm_f32x3 (products from exact BF16 parts; 3B prefill GEMMs at 512
// rows 23.7 -> 17.0 ms) unless LLAMA_HIP_F32_FORM = fp32 picks mm_gemm_lds<true> (FP32 products); read on every call.
bool f32_on_bf16_parts() {
  const char *form = getenv("LLAMA_HIP_F32_FORM");
  return !form || strcmp(form, "fp32") != 0;
}

bool x3_launch(MmParams p, hipStream_t stream) {
  static const hipError_t status =
      hipFuncSetAttribute((const void *)mm_gemm_f32x3, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kX3Lds);
  if (!check_hip(status, "allowing the FP32 GEMM on BF16 parts its LDS"))
    return false;
  p.sk.splits = p.grid.total > kSplitSlots ? 1 : choose_splits(p.grid.total, p.steps, &p.sk.per);
  if (p.sk.splits == 1)
    p.sk.per = p.steps;
  p.sk.partial = (v4f *)device().split_partial;
  p.sk.count = device().split_count;
  hipLaunchKernelGGL(mm_gemm_f32x3, dim3((unsigned)(p.grid.total * p.sk.splits)), dim3(kQ8Threads), kX3Lds, stream, p);
  return launch_ok("mm_gemm_f32x3");
}

template <bool F32> bool mm_launch(MmParams p, hipStream_t stream) {
  static const hipError_t status =
      hipFuncSetAttribute((const void *)mm_gemm_lds<F32>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMmLds);
  if (!check_hip(status, "allowing the FP32 / BF16 GEMM its LDS"))
    return false;
  p.sk.splits = p.grid.total > kSplitSlots ? 1 : choose_splits(p.grid.total, p.steps, &p.sk.per);
  if (p.sk.splits == 1)
    p.sk.per = p.steps;
  p.sk.partial = (v4f *)device().split_partial;
  p.sk.count = device().split_count;
  hipLaunchKernelGGL(mm_gemm_lds<F32>, dim3((unsigned)(p.grid.total * p.sk.splits)), dim3(kQ8Threads), kMmLds, stream,
                     p);
  return launch_ok(F32 ? "mm_gemm_lds<fp32>" : "mm_gemm_lds<bf16>");
}

// The wide BF16 kernel (256 x 256 tiles); its partial tiles are twice the size, so half as many fit the workspace.
bool wide_launch(MmParams p, const GemmF32Job &job, hipStream_t stream) {
  constexpr int kWideSlots = kSplitSlots / 2;
  p.grid = make_q8_grid(job.seg, job.nseg, job.m, kWTileM, kWTileN);
  p.sk.splits = p.grid.total > kWideSlots ? 1 : choose_splits(p.grid.total, p.steps, &p.sk.per, 1, kWideSlots);
  if (p.sk.splits == 1)
    p.sk.per = p.steps;
  p.sk.partial = (v4f *)device().split_partial;
  p.sk.count = device().split_count;
  static const hipError_t s0 =
      hipFuncSetAttribute((const void *)bf16_gemm_wide<false>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kWLds);
  static const hipError_t s1 =
      hipFuncSetAttribute((const void *)bf16_gemm_wide<true>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kWLds);
  if (!check_hip(s0, "allowing the BF16 GEMM its LDS") || !check_hip(s1, "allowing the BF16 GEMM its LDS"))
    return false;
  if (p.sk.splits == 1) {
    hipLaunchKernelGGL(bf16_gemm_wide<false>, dim3((unsigned)p.grid.total), dim3(kQ8Threads), kWLds, stream, p);
    return launch_ok("bf16_gemm_wide");
  }
  hipLaunchKernelGGL(bf16_gemm_wide<true>, dim3((unsigned)(p.grid.total * p.sk.splits)), dim3(kQ8Threads), kWLds,
                     stream, p);
  if (!launch_ok("bf16_gemm_wide"))
    return false;
  return launch_split_reduce<8, kQ8Threads>(p.grid, p.sk, p.m, kWTileM, kWTileN, stream);
}

// BF16 tile: LLAMA_HIP_BF16_TILE = wide (256 x 256) or narrow (256 x 128), read once; by default wide when the grid
// has at least four 256 x 128 tiles per CU. Measured: 2048 x 28672 x 4096 SwiGLU 886 TF/s wide, 754 narrow; with fewer
// tiles the wide grid's quantization and split cost more than its operand savings (2048 x 4096 x 4096: 677 vs 757,
// the 512-token 3B shapes 10-15% slower).
std::atomic<int> forced_bf16_tile{0}; // llhip_set_bf16_tile: 0 unset, 1 narrow, 2 wide

bool bf16_wide(int narrow_tiles) {
  static const int env_tile = [] {
    const char *env = getenv("LLAMA_HIP_BF16_TILE");
    return env && !strcmp(env, "wide") ? 2 : env && !strcmp(env, "narrow") ? 1 : 0;
  }();
  const int forced = forced_bf16_tile.load() ? forced_bf16_tile.load() : env_tile;
  if (forced)
    return forced == 2;
  const int cus = device().cu_count > 0 ? device().cu_count : 256;
  return narrow_tiles >= 4 * cus;
}

bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15) == 0; }

// Shapes the pipelined FP32 kernel takes: K a multiple of 16 and 16-byte aligned rows whose 32-bit buffer offsets fit.
bool f32_fast_path(const GemmF32Job &job) {
  if (job.k % 16 || job.lda % 4 || !aligned16(job.a) || (long long)kQ8TileM * job.lda * 4 >= (1LL << 31))
    return false;
  for (int s = 0; s < job.nseg; s++) {
    const GemmSegmentDev &g = job.seg[s];
    if (g.ldw % 4 || !aligned16(g.w) || (g.w3 && !aligned16(g.w3)) || 16LL * (long long)g.ldw * 4 >= (1LL << 31))
      return false;
  }
  return true;
}

} // namespace

void set_gemm_splits(int splits) { forced_splits.store(splits > 0 ? splits : 0); }

void set_bf16_tile(int tile) { forced_bf16_tile.store(tile == 1 || tile == 2 ? tile : 0); }

void set_q8_tile(int tile) { forced_q8_tile.store(tile == 1 || tile == 2 ? tile : 0); }

void set_q8_scales(int where) { forced_q8_scales.store(where == 1 || where == 2 ? where : 0); }

bool launch_f32_gemm(const GemmF32Job &job, hipStream_t stream) {
  if (job.m <= 0 || job.k <= 0)
    return true;
  MmParams p{};
  p.grid = make_q8_grid(job.seg, job.nseg, job.m);
  p.m = job.m;
  if (p.grid.total <= 0)
    return true;
  if (job.bf16) {
    // round A into the panel, then the pipelined kernel
    const int kp = (job.k + 31) / 32 * 32;
    if (!job.panel)
      return raise("k_gemm_bf16 needs a device panel");
    if ((long long)kQ8TileM * kp * 2 >= (1LL << 31))
      return raise("k_gemm_bf16: K = %d is beyond the kernel's 32-bit offsets", job.k);
    const long long threads = (long long)job.m * (kp / 8);
    hipLaunchKernelGGL(bf16_panel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, job.a,
                       (long long)job.lda, job.m, job.k, kp, job.panel);
    if (!launch_ok("bf16_panel"))
      return false;
    p.a = (const unsigned char *)job.panel;
    p.arow = (long long)kp * 2;
    p.steps = kp / 32;
    return bf16_wide(p.grid.total) ? wide_launch(p, job, stream) : mm_launch<false>(p, stream);
  }
  if (f32_fast_path(job)) {
    p.a = (const unsigned char *)job.a;
    p.arow = (long long)job.lda * 4;
    p.steps = job.k / 16;
    return f32_on_bf16_parts() ? x3_launch(p, stream) : mm_launch<true>(p, stream);
  }
  F32Params f{};
  f.grid = make_grid(job.seg, job.nseg, job.m);
  f.a = job.a;
  f.lda = job.lda;
  f.m = job.m;
  f.k = job.k;
  hipLaunchKernelGGL(f32_gemm_mfma, dim3(f.grid.total), dim3(kBlock), 0, stream, f);
  return launch_ok("f32_gemm_mfma");
}

} // namespace llhip
