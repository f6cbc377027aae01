// Lane exchanges and reductions inside a 64-lane wave (gfx950), shared by the GEMV and forward kernels.
#pragma once

namespace llhip {
namespace {

// Lane exchanges inside a row of 16 lanes use DPP (a VALU operand modifier, no LDS round trip): quad_perm [1,0,3,2]
// and [2,3,0,1] pair lanes at distance 1 and 2, row_half_mirror pairs each lane with one in the other half of its
// 8-lane group and row_mirror with one in the other half of its row. After the quad steps every lane of a quad holds
// the same value, so the mirror steps complete the reduction over 8 and 16 lanes. Distances 16 and 32 use a swizzle.
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppRowHalfMirror = 0x141, kDppRowMirror = 0x140;

template <int CTRL> __device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
template <int CTRL> __device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

struct AddOp {
  template <class T> __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct MaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

// Reduction over aligned groups of `lanes` lanes (a power of two <= 64, wave-uniform); every lane gets its group's
// result.
template <class T, class Op> __device__ __forceinline__ T group_reduce(T v, int lanes, Op op) {
  if (lanes > 1)
    v = op(v, dpp<kDppQuadXor1>(v));
  if (lanes > 2)
    v = op(v, dpp<kDppQuadXor2>(v));
  if (lanes > 4)
    v = op(v, dpp<kDppRowHalfMirror>(v));
  if (lanes > 8)
    v = op(v, dpp<kDppRowMirror>(v));
  if (lanes > 16)
    v = op(v, __shfl_xor(v, 16));
  if (lanes > 32)
    v = op(v, __shfl_xor(v, 32));
  return v;
}

template <class T> __device__ __forceinline__ T group_reduce_add(T v, int lanes) { return group_reduce(v, lanes, AddOp{}); }

__device__ __forceinline__ float group_reduce_max(float v, int lanes) { return group_reduce(v, lanes, MaxOp{}); }

// Sum over the wave: each 16-lane row reduces with DPP, then the four row sums are read out of lanes 0, 16, 32, 48.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<kDppQuadXor1>(v);
  v += dpp<kDppQuadXor2>(v);
  v += dpp<kDppRowHalfMirror>(v);
  v += dpp<kDppRowMirror>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
}

// Maximum over the wave, in the same pattern as wave_sum (a maximum does not depend on the order).
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppQuadXor1>(v));
  v = fmaxf(v, dpp<kDppQuadXor2>(v));
  v = fmaxf(v, dpp<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp<kDppRowMirror>(v));
  return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
                     __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16))),
               fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)),
                     __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48))));
}

} // namespace
} // namespace llhip
