// The E2M1 / E8M0 steps of MXFP4 quantization (nvfp4_mxfp4.py:85-174) used by the codec kernels of
// sqx_fp4.hip.
#pragma once

#include "sqx_common.h"

namespace sqx {

static constexpr float kTiny = 1e-30f;  // _TINY

// e2m1_round_to_code (:85-98): the first index of the smallest fp32 distance |a - m| over the eight
// magnitudes (torch.argmin), so exact midpoints go to the lower magnitude and inputs whose distances
// all round equal (above ~2**25, infinities) and NaN take index 0; sign bit = x < 0.
__device__ inline uint32_t e2m1_code_argmin(float x) {
  constexpr float kMag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const float a = fabsf(x);
  uint32_t idx = 0;
  float best = a;
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    const float d = fabsf(a - kMag[i]);
    if (d < best) {
      best = d;
      idx = static_cast<uint32_t>(i);
    }
  }
  return (x < 0.0f ? 8u : 0u) | idx;
}

// The same code in ~10 instructions instead of ~28. Below 2**22 every distance |a - m| is exact in
// fp32 (a and the magnitudes are multiples of a's ulp), so the first minimum is the number of
// midpoints between consecutive magnitudes (0.25 0.75 1.25 1.75 2.5 3.5 5) strictly below a, found
// by a three-level comparison; larger inputs, infinities and NaN take the argmin above. Checked
// equal to e2m1_code_argmin on all 2**32 fp32 bit patterns.
__device__ inline uint32_t e2m1_code(float x) {
  const float a = fabsf(x);
  if (!(a < 4194304.0f)) return e2m1_code_argmin(x);
  const bool hi = a > 1.75f;
  const bool b1 = a > (hi ? 3.5f : 0.75f);
  const bool b0 = a > (hi ? (b1 ? 5.0f : 2.5f) : (b1 ? 1.25f : 0.25f));
  return (x < 0.0f ? 8u : 0u) | (hi ? 4u : 0u) | (b1 ? 2u : 0u) | (b0 ? 1u : 0u);
}

// fp32 log2 correctly rounded (double log2, one rounding): what torch's CPU log2 returns for the
// reference's inputs (pinned by golden vectors at and around every power of two in range).
__device__ inline float log2_f32(float v) { return static_cast<float>(log2(static_cast<double>(v))); }

// _e8m0_no_overflow_scale (:162-174) as an exponent: clamp(ceil(log2(max(amax/6, 1e-30))), +-127).
// The 1e-30 floor makes the exponent >= -99, so the reference's later clamp_min(1e-30) of 2**e is a
// no-op. NaN amax gives a NaN scale (returned as exponent 128).
// Without the double log2 in the common case: t >= 1e-30 is a normal float 2**e * (1 + m * 2**-23),
// so log2(t) lies in [e, e + 1). For m = 0 it is e exactly. For m >= 64 it exceeds e by more than
// 64 * 2**-23 / ln 2 > 1.1e-5, above half an fp32 ulp of any |e| <= 128 (2**-18), so its fp32
// rounding is above e and its ceil is e + 1 (a rounding up to e + 1 gives the same). Only
// 1 <= m < 64 can round down to e and takes the correctly rounded log2. Infinity (e = 128, m = 0)
// clamps to 127 as before.
__device__ inline int mx_exponent(float amax) {
  float t = __fdiv_rn(amax, 6.0f);
  if (t < kTiny) t = kTiny;
  if (t != t) return 128;
  const uint32_t u = __builtin_bit_cast(uint32_t, t);
  const int e = static_cast<int>((u >> 23) & 0xffu) - 127;
  const uint32_t m = u & 0x7fffffu;
  int c;
  if (m == 0u) c = e;
  else if (m >= 64u) c = e + 1;
  else c = static_cast<int>(ceilf(log2_f32(t)));
  return min(max(c, -127), 127);
}

// NaN-propagating max of |v| (torch amax propagates NaN). For m and v that are both maxima of this
// kind, amax_step(m, v) is their joint maximum, in either order.
__device__ inline float amax_step(float m, float v) {
  const float a = fabsf(v);
  return (a > m || a != a) ? a : m;
}

// mxfp4_dequantize(mxfp4_quantize(.)) of two elements of one 32-element block whose exponent is ex
// (mx_exponent of the block's amax): code(v * 2**-ex) * 2**ex as a bf16 pair, low half v0. Every such
// value is exact in bf16 wherever it is finite in fp32 (an E2M1 value has 2 significant bits); a
// NaN block (ex = 128) gives NaN.
__device__ inline uint32_t mx_fake_pair(float v0, float v1, int ex) {
  constexpr float kMag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const float inv = ex == 128 ? __builtin_nanf("") : ldexpf(1.0f, -ex);
  const float sc = ex == 128 ? __builtin_nanf("") : ldexpf(1.0f, ex);
  const uint32_t c0 = e2m1_code(v0 * inv), c1 = e2m1_code(v1 * inv);
  const float d0 = (c0 & 8u ? -kMag[c0 & 7u] : kMag[c0 & 7u]) * sc;
  const float d1 = (c1 & 8u ? -kMag[c1 & 7u] : kMag[c1 & 7u]) * sc;
  return static_cast<uint32_t>(f32_to_bf16_bits(d0)) | (static_cast<uint32_t>(f32_to_bf16_bits(d1)) << 16);
}

}  // namespace sqx
