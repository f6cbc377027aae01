// The k_quantize rule on the device (src/gemv.c:589-624), shared by the quantizer, the GEMV prologue and the GEMM
// epilogue that quantizes its output.
#pragma once

namespace llhip {
namespace {

// One value of k_quantize (src/gemv.c:618-620): the IEEE quotient (hipcc emits a correctly rounded fp32 division by
// default), the clamp before rounding, roundf's half-away-from-zero rule.
__device__ __forceinline__ int quantize_one(float x, float scale) {
  float ratio = scale == 0.0f ? 0.0f : x / scale;
  return (int)roundf(fmaxf(-127.0f, fminf(127.0f, ratio)));
}

// Values through the reciprocal, for normal finite scales: r = x * rcp(scale) lies within 127 * 3 * 2^-24 < 2.3e-5 of
// the correctly rounded quotient fl(x / scale) (v_rcp_f32 is within 1 ulp, the product rounds once, |x / scale| <=
// 127 (1 + 2^-23)). The kernels keep FP32 denormals (the compiler's default mode), so a subnormal x or r changes this
// only by an absolute 2^-150. roundf changes value only at k + 0.5 and the clamp binds only from 127.5, which r never
// reaches, so wherever r is at least 2^-12 from every k + 0.5, i.e. |r - rint(r)| <= 0.5 - 2^-12 (an exact
// subtraction), both give rint(r). rint is r + M - M with M = 1.5 * 2^23: for |r| < 2^22 the sum rounds r to the
// nearest integer (ties to even) in the low mantissa bits, so the low byte of the sum's bits is rint(r) as int8, with
// no conversion. If any value of the call is inside the margin or not finite (r is then NaN or infinite, and the test
// fails), or the scale is 0, not normal or infinite, the exact quotient decides for all of them, and the non-finite
// values are flagged: one branch per call, rarely taken.
constexpr float kTieGuard = 0.5f - 0x1p-12f;
constexpr float kRoundMagic = 12582912.0f; // 1.5 * 2^23

// q[j]'s low byte is the int8 value of x[j].
template <int N>
__device__ __forceinline__ void quantize_fast(const float (&x)[N], float scale, float inv, bool inv_ok, int (&q)[N],
                                              bool &bad) {
#pragma clang fp contract(off) // r is the rounded product: the margin test must see the value that was rounded
  bool slow = !inv_ok;
#pragma unroll
  for (int j = 0; j < N; j++) {
    const float r = x[j] * inv;
    const float t = r + kRoundMagic;
    slow |= !(fabsf(r - (t - kRoundMagic)) <= kTieGuard);
    q[j] = __float_as_int(t);
  }
  if (slow) {
#pragma unroll
    for (int j = 0; j < N; j++) {
      bad |= !isfinite(x[j]);
      q[j] = quantize_one(x[j], scale);
    }
  }
}

__device__ __forceinline__ float group_reciprocal(float scale, bool &ok) {
  ok = scale >= 1.17549435e-38f && scale <= 3.40282347e+38f; // normal and finite
  return ok ? __builtin_amdgcn_rcpf(scale) : 0.0f;
}

__device__ __forceinline__ int pack_bytes(int a, int b, int c, int d) {
  return (a & 0xff) | ((b & 0xff) << 8) | ((c & 0xff) << 16) | ((int)((unsigned)d << 24));
}

} // namespace
} // namespace llhip
