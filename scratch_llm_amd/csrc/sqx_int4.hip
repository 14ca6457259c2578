// INT4 group-wise weights on gfx950: bit-exact quantize / pack / unpack / dequantize
// (src/scratch_llm/quant/int4_group.py) and the fused dequant linear that streams tiled codes.
//
// Tiled layout (the HBM layout the linear reads; written by sqx_int4_tile):
//   T = ceil(rows/16) row tiles, KB = ceil(cols/128) k-blocks of 128 columns.
//   Block (t, kb) is 1024 contiguous bytes at ((t*KB + kb) * 1024). Lane L (0..63) of the wave
//   that consumes the block owns bytes [16L, 16L+16) = four dwords. Dword i (0..3) holds the codes
//   of row r = 16t + (L & 15), columns c = kb*128 + 32i + 8(L >> 4) + e (e = 0..7): element e sits in
//   nibble e/2 when e is even and nibble 4 + e/2 when e is odd, so ((d >> 4p) & 0x000F000F) yields
//   the column pair (2p, 2p+1) in the low/high 16-bit halves. Codes are stored unsigned:
//   u = q + 8 for symmetric codes q in [-8, 7], u as given for asymmetric codes.
//   Per-group parameters: Gp = KB * 128/group groups per row, stored [T][Gp][16] so one 64-byte
//   line serves the 16 rows of a tile. Padding rows / columns carry a zero scale.
//
// Linear: one wave computes a 16-row tile for up to 16*MCH activation rows with
// v_mfma_f32_16x16x32_{bf16,f16}. A = activations (rows = tokens), B = weights (columns = weight
// rows). OR-ing a code into the mantissa of MAGIC (bf16 128.0 / fp16 1024.0) gives MAGIC + u
// exactly, so B needs three VALU ops per column pair; a second set of MFMAs with the constant
// B = -(MAGIC + zero) removes the offset, and the group scale is applied to the fp32 partial.
#include "sqx_gemv.h"
#include "sqx_skinny.h"

#include <float.h>

// k-blocks per pipeline round for 1 and 2 MFMA row chunks (tuning knobs for sweeps).
#ifndef SQX_INT4_U1
#define SQX_INT4_U1 4
#endif
#ifndef SQX_INT4_U2
#define SQX_INT4_U2 2
#endif

namespace sqx {

// ----------------------------------------------------------------------------------------------
// quantize_groupwise_int4 (int4_group.py:108-129)
// ----------------------------------------------------------------------------------------------
// Fast path: group is a power of two in [8, 512]; each lane owns 8 consecutive elements, the
// group's lanes are consecutive in the wave, and the absmax is reduced with xor shuffles.
// COLMUL: the weight is first multiplied by a per-column fp32 scale (AWQ's W * s, awq.py:173, one
// fp32 rounding). FAKE: instead of codes and scales, write the AWQ effective weight
// dequant(q, s_g) / s (awq.py:115-119) in fp32.
template <int LPG, bool COLMUL, bool FAKE>
__global__ __launch_bounds__(256) void int4_quantize_sym_kernel(const void* __restrict__ w, int w_dtype,
                                                                int64_t n_elems, int64_t cols, int64_t group,
                                                                const float* __restrict__ colmul,
                                                                int8_t* __restrict__ q, float* __restrict__ scales,
                                                                float* __restrict__ weff) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t e0 = i * 8;
  const bool live = e0 < n_elems;
  const int64_t c0 = COLMUL ? e0 % cols : 0;
  float v[8];
  float amax = 0.0f;
  bool nan = false;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    v[e] = live ? load_as_f32(w, w_dtype, e0 + e) : 0.0f;
    if (COLMUL && live) v[e] = v[e] * colmul[c0 + e];
    float a = fabsf(v[e]);
    nan |= (a != a);
    amax = fmaxf(amax, a);
  }
#pragma unroll
  for (int off = 1; off < LPG; off <<= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, off));
    nan |= (__shfl_xor((int)nan, off) != 0);
  }
  if (!live) return;
  // torch: scales = (absmax / 7).clamp_min(finfo(fp32).tiny); amax propagates NaN.
  float s = nan ? __builtin_nanf("") : __fdiv_rn(amax, 7.0f);
  if (s < FLT_MIN) s = FLT_MIN;
  uint64_t packed = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float r = __builtin_rintf(__fdiv_rn(v[e], s));  // round half to even, like torch.round
    r = fminf(fmaxf(r, -8.0f), 7.0f);
    int8_t c = (r == r) ? static_cast<int8_t>(r) : 0;  // NaN codes are unspecified upstream
    if (FAKE) weff[e0 + e] = __fdiv_rn(static_cast<float>(c) * s, colmul[c0 + e]);
    packed |= static_cast<uint64_t>(static_cast<uint8_t>(c)) << (8 * e);
  }
  if (!FAKE) {
    *reinterpret_cast<uint64_t*>(q + e0) = packed;
    if ((threadIdx.x & (LPG - 1)) == 0) scales[e0 / group] = s;
  }
}

// Generic path: any group size; one thread per group (COLMUL / FAKE as above).
template <bool COLMUL, bool FAKE>
__global__ __launch_bounds__(256) void int4_quantize_sym_generic_kernel(const void* __restrict__ w, int w_dtype,
                                                                        int64_t n_groups, int64_t cols, int64_t group,
                                                                        const float* __restrict__ colmul,
                                                                        int8_t* __restrict__ q,
                                                                        float* __restrict__ scales,
                                                                        float* __restrict__ weff) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= n_groups) return;
  const int64_t base = g * group;
  const int64_t c0 = COLMUL ? base % cols : 0;
  auto val = [&](int64_t e) {
    const float v = load_as_f32(w, w_dtype, base + e);
    return COLMUL ? v * colmul[c0 + e] : v;
  };
  float amax = 0.0f;
  bool nan = false;
  for (int64_t e = 0; e < group; ++e) {
    float a = fabsf(val(e));
    nan |= (a != a);
    amax = fmaxf(amax, a);
  }
  float s = nan ? __builtin_nanf("") : __fdiv_rn(amax, 7.0f);
  if (s < FLT_MIN) s = FLT_MIN;
  for (int64_t e = 0; e < group; ++e) {
    float r = __builtin_rintf(__fdiv_rn(val(e), s));
    r = fminf(fmaxf(r, -8.0f), 7.0f);
    const int8_t c = (r == r) ? static_cast<int8_t>(r) : 0;
    if (FAKE) weff[base + e] = __fdiv_rn(static_cast<float>(c) * s, colmul[c0 + e]);
    else q[base + e] = c;
  }
  if (!FAKE) scales[g] = s;
}

// Build-defined asymmetric uint4 (no reference symbol; the 4-bit form of quantize_affine,
// int8.py:142-172, per group): lo = min(min(w), 0), hi = max(max(w), 0), s = max((hi - lo) / 15,
// 1e-12) (rounded to bf16 first when the parameters are stored as bf16), z = clamp(rint(-lo / s),
// 0, 15), q = clamp(rint(w / s + z), 0, 15). One thread per group.
template <bool PBF16>
__global__ __launch_bounds__(256) void int4_quantize_asym_kernel(const void* __restrict__ w, int w_dtype,
                                                                 int64_t n_groups, int64_t group,
                                                                 uint8_t* __restrict__ q, void* __restrict__ scales,
                                                                 void* __restrict__ zeros) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= n_groups) return;
  const int64_t base = g * group;
  float lo = 0.0f, hi = 0.0f;
  for (int64_t e = 0; e < group; ++e) {
    const float v = load_as_f32(w, w_dtype, base + e);
    lo = (v < lo || v != v) ? v : lo;
    hi = (v > hi || v != v) ? v : hi;
  }
  float s = __fdiv_rn(hi - lo, 15.0f);
  if (s < 1e-12f) s = 1e-12f;
  if (PBF16) s = bf16_bits_to_f32(f32_to_bf16_bits(s));
  const float z = fminf(fmaxf(__builtin_rintf(__fdiv_rn(-lo, s)), 0.0f), 15.0f);
  for (int64_t e = 0; e < group; ++e) {
    const float r = fminf(fmaxf(__builtin_rintf(__fdiv_rn(load_as_f32(w, w_dtype, base + e), s) + z), 0.0f), 15.0f);
    q[base + e] = static_cast<uint8_t>(r == r ? r : 0.0f);
  }
  if (PBF16) {
    static_cast<uint16_t*>(scales)[g] = f32_to_bf16_bits(s);
    static_cast<uint16_t*>(zeros)[g] = f32_to_bf16_bits(z);
  } else {
    static_cast<float*>(scales)[g] = s;
    static_cast<float*>(zeros)[g] = z;
  }
}

// awq_dequantize (awq.py:178-181): dequant(q, s_g) / s per column, fp32.
__global__ __launch_bounds__(256) void awq_dequantize_kernel(const int8_t* __restrict__ q, const float* __restrict__ gs,
                                                             const float* __restrict__ cs, int64_t n_elems,
                                                             int64_t cols, int64_t group, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_elems) return;
  out[i] = __fdiv_rn(static_cast<float>(q[i]) * gs[i / group], cs[i % cols]);
}

// act_scale (awq.py:94-101): mean over rows of |x| per column, accumulated in fp64 and rounded once.
__global__ __launch_bounds__(256) void col_absmean_kernel(const void* __restrict__ x, int dtype, int64_t rows,
                                                          int64_t cols, float* __restrict__ out) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  double acc = 0.0;
  for (int64_t r = 0; r < rows; ++r) acc += fabs(static_cast<double>(load_as_f32(x, dtype, r * cols + c)));
  out[c] = static_cast<float>(acc / static_cast<double>(rows));
}

// The AWQ channel scale for grid exponent `ratio` (awq.py:104-112, 141-142):
// s = max(a ** ratio, 1e-4); s / sqrt(max(s) * min(s)). One workgroup.
__global__ __launch_bounds__(1024) void awq_scale_kernel(const float* __restrict__ a, int64_t n, float ratio,
                                                         float* __restrict__ out) {
  __shared__ float rmax[1024], rmin[1024];
  float mx = -INFINITY, mn = INFINITY;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    float v = ratio == 0.0f ? 1.0f : (ratio == 1.0f ? a[i] : powf(a[i], ratio));
    if (v < 1e-4f) v = 1e-4f;
    out[i] = v;
    mx = fmaxf(mx, v);
    mn = fminf(mn, v);
  }
  rmax[threadIdx.x] = mx;
  rmin[threadIdx.x] = mn;
  __syncthreads();
  for (int s = 512; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      rmax[threadIdx.x] = fmaxf(rmax[threadIdx.x], rmax[threadIdx.x + s]);
      rmin[threadIdx.x] = fminf(rmin[threadIdx.x], rmin[threadIdx.x + s]);
    }
    __syncthreads();
  }
  const float norm = sqrtf(rmax[0] * rmin[0]);
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) out[i] = __fdiv_rn(out[i], norm);
}

// x / s per column, rounded back to the activation dtype (the AWQ linear folds 1/s into x).
template <class A>
__global__ __launch_bounds__(256) void scale_columns_kernel(const uint16_t* __restrict__ x, const float* __restrict__ s,
                                                            int64_t n, int64_t cols, uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = A::from_f32(__fdiv_rn(A::to_f32(x[i]), s[i % cols]));
}

// The same for rows of a multiple of 8 columns and 16-byte aligned buffers: thread (x, y) takes the
// 8 columns 8x .. 8x+7 of row y (16-byte loads and stores; the row's scales are the same for every
// row, so they stay in the caches).
template <class A>
__global__ __launch_bounds__(256) void scale_columns8_kernel(const uint16_t* __restrict__ x, const float* __restrict__ s,
                                                             int cols, uint16_t* __restrict__ out) {
  const int c = 8 * (blockIdx.x * 256 + threadIdx.x);
  if (c >= cols) return;
  const int64_t o = (int64_t)blockIdx.y * cols + c;
  const u32x4_t v = *reinterpret_cast<const u32x4_t*>(x + o);
  const f32x4_t s0 = *reinterpret_cast<const f32x4_t*>(s + c), s1 = *reinterpret_cast<const f32x4_t*>(s + c + 4);
  const float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  u32x4_t r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = __fdiv_rn(A::to_f32(static_cast<uint16_t>(v[j] & 0xffffu)), sv[2 * j]);
    const float hi = __fdiv_rn(A::to_f32(static_cast<uint16_t>(v[j] >> 16)), sv[2 * j + 1]);
    r[j] = static_cast<uint32_t>(A::from_f32(lo)) | (static_cast<uint32_t>(A::from_f32(hi)) << 16);
  }
  *reinterpret_cast<u32x4_t*>(out + o) = r;
}

// ----------------------------------------------------------------------------------------------
// pack_int4 / unpack_int4 (int4_group.py:62-102)
// ----------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void int4_pack_kernel(const int8_t* __restrict__ q, int64_t n,
                                                        uint8_t* __restrict__ packed) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nb = (n + 1) / 2;
  if (i >= nb) return;
  const uint8_t hi = static_cast<uint8_t>(q[2 * i]) & 0xF;
  const uint8_t lo = (2 * i + 1 < n) ? (static_cast<uint8_t>(q[2 * i + 1]) & 0xF) : 0;
  packed[i] = static_cast<uint8_t>((hi << 4) | lo);
}

__device__ inline int8_t sext4(uint32_t nib) { return static_cast<int8_t>(nib >= 8 ? (int)nib - 16 : (int)nib); }

__global__ __launch_bounds__(256) void int4_unpack_kernel(const uint8_t* __restrict__ packed, int64_t n,
                                                          int8_t* __restrict__ q) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (2 * i >= n) return;
  const uint32_t b = packed[i];
  q[2 * i] = sext4(b >> 4);
  if (2 * i + 1 < n) q[2 * i + 1] = sext4(b & 0xF);
}

// ----------------------------------------------------------------------------------------------
// dequantize_groupwise_int4 (int4_group.py:132-142)
// ----------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void int4_dequantize_kernel(const int8_t* __restrict__ q,
                                                              const float* __restrict__ scales,
                                                              int64_t n_elems, int64_t group,
                                                              float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_elems) return;
  out[i] = static_cast<float>(q[i]) * scales[i / group];
}

// ----------------------------------------------------------------------------------------------
// Tile re-layout
// ----------------------------------------------------------------------------------------------
// One thread per output dword. SRC_PACKED reads the reference byte stream (high nibble = even
// element), otherwise int8 codes. SIGNED stores u = q + 8.
template <bool SRC_PACKED, bool SIGNED>
__global__ __launch_bounds__(256) void int4_tile_weights_kernel(const void* __restrict__ src, int64_t rows,
                                                                int64_t cols, int64_t KB, int64_t n_dwords,
                                                                uint32_t* __restrict__ wt) {
  const int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= n_dwords) return;
  const int i = static_cast<int>(d & 3);
  const int L = static_cast<int>((d >> 2) & 63);
  const int64_t blk = d >> 8;  // t*KB + kb
  const int64_t t = blk / KB;
  const int64_t kb = blk - t * KB;
  const int64_t r = 16 * t + (L & 15);
  const int64_t c0 = kb * 128 + 32 * i + 8 * (L >> 4);
  uint32_t word = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t c = c0 + e;
    uint32_t u = SIGNED ? 8u : 0u;
    if (r < rows && c < cols) {
      if (SRC_PACKED) {
        const int64_t f = r * cols + c;
        const uint32_t b = static_cast<const uint8_t*>(src)[f >> 1];
        const uint32_t nib = (f & 1) ? (b & 0xF) : (b >> 4);
        u = nib ^ 8u;  // two's-complement nibble q -> q + 8
      } else {
        const int8_t qv = static_cast<const int8_t*>(src)[r * cols + c];
        u = SIGNED ? static_cast<uint32_t>(qv + 8) : static_cast<uint32_t>(qv);
        u &= 0xF;
      }
    }
    const int pos = (e & 1) ? (16 + 4 * (e >> 1)) : (4 * (e >> 1));
    word |= u << pos;
  }
  wt[d] = word;
}

// One thread per tiled parameter element; param elements are 4 (F32) or 2 (BF16) bytes.
template <typename P>
__global__ __launch_bounds__(256) void int4_tile_params_kernel(const P* __restrict__ src, int64_t rows,
                                                               int64_t n_groups, int64_t Gp, int64_t n_out,
                                                               P* __restrict__ dst) {
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= n_out) return;
  const int64_t nl = o & 15;
  const int64_t tg = o >> 4;
  const int64_t t = tg / Gp;
  const int64_t g = tg - t * Gp;
  const int64_t r = 16 * t + nl;
  dst[o] = (r < rows && g < n_groups) ? src[r * n_groups + g] : P(0);
}

// Asymmetric codes with bf16 parameters: the scale and zero of a (row, group) interleaved into one
// dword (scale bits | zero bits << 16), so the kernels fetch both with one load.
__global__ __launch_bounds__(256) void int4_tile_param_pairs_kernel(const uint16_t* __restrict__ sc,
                                                                    const uint16_t* __restrict__ zr, int64_t rows,
                                                                    int64_t n_groups, int64_t Gp, int64_t n_out,
                                                                    uint32_t* __restrict__ dst) {
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= n_out) return;
  const int64_t nl = o & 15;
  const int64_t tg = o >> 4;
  const int64_t t = tg / Gp;
  const int64_t g = tg - t * Gp;
  const int64_t r = 16 * t + nl;
  dst[o] = (r < rows && g < n_groups) ? (static_cast<uint32_t>(sc[r * n_groups + g]) |
                                         (static_cast<uint32_t>(zr[r * n_groups + g]) << 16))
                                      : 0u;
}

__global__ __launch_bounds__(256) void int4_untile_param_pairs_kernel(const uint32_t* __restrict__ src, int64_t rows,
                                                                      int64_t n_groups, int64_t Gp, int64_t n_in,
                                                                      uint16_t* __restrict__ sc,
                                                                      uint16_t* __restrict__ zr) {
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= n_in) return;
  const int64_t nl = o & 15;
  const int64_t tg = o >> 4;
  const int64_t t = tg / Gp;
  const int64_t g = tg - t * Gp;
  const int64_t r = 16 * t + nl;
  if (r < rows && g < n_groups) {
    const uint32_t v = src[o];
    sc[r * n_groups + g] = static_cast<uint16_t>(v & 0xffffu);
    zr[r * n_groups + g] = static_cast<uint16_t>(v >> 16);
  }
}

// The inverse re-layout (tiles -> the reference's row-major codes and [rows, groups] parameters):
// one thread per tiled dword writes its 8 codes (u - 8 for SIGNED), one per tiled parameter element
// writes it back; padding rows and columns are skipped.
template <bool SIGNED>
__global__ __launch_bounds__(256) void int4_untile_weights_kernel(const uint32_t* __restrict__ wt, int64_t rows,
                                                                  int64_t cols, int64_t KB, int64_t n_dwords,
                                                                  int8_t* __restrict__ codes) {
  const int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= n_dwords) return;
  const int i = static_cast<int>(d & 3);
  const int L = static_cast<int>((d >> 2) & 63);
  const int64_t blk = d >> 8;
  const int64_t t = blk / KB;
  const int64_t kb = blk - t * KB;
  const int64_t r = 16 * t + (L & 15);
  if (r >= rows) return;
  const int64_t c0 = kb * 128 + 32 * i + 8 * (L >> 4);
  const uint32_t word = wt[d];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t c = c0 + e;
    if (c >= cols) break;
    const int pos = (e & 1) ? 16 + 4 * (e >> 1) : 4 * (e >> 1);
    const int u = static_cast<int>((word >> pos) & 0xFu);
    codes[r * cols + c] = static_cast<int8_t>(SIGNED ? u - 8 : u);
  }
}

template <typename P>
__global__ __launch_bounds__(256) void int4_untile_params_kernel(const P* __restrict__ src, int64_t rows,
                                                                 int64_t n_groups, int64_t Gp, int64_t n_in,
                                                                 P* __restrict__ dst) {
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= n_in) return;
  const int64_t nl = o & 15;
  const int64_t tg = o >> 4;
  const int64_t t = tg / Gp;
  const int64_t g = tg - t * Gp;
  const int64_t r = 16 * t + nl;
  if (r < rows && g < n_groups) dst[r * n_groups + g] = src[o];
}

// ----------------------------------------------------------------------------------------------
// The linear: the int4 weight policy of the shared GEMV (sqx_gemv.h)
// ----------------------------------------------------------------------------------------------
// Block layout: dword i of lane L holds the codes of row 16t + (L & 15), columns
// 32i + 8(L >> 4) + e, element e in nibble e/2 (even e) or 4 + e/2 (odd e), stored unsigned.
// v_and_or_b32(d >> 4p, 0x000F000F, MAGIC pair) turns the column pair (2p, 2p+1) into the 16-bit
// pair (MAGIC + u) exactly (bf16 128 / fp16 1024 have an integer spacing of 1); a second MFMA
// against the constant -(MAGIC + zero) removes the offset, and the group scale is applied to the
// fp32 partial.
template <bool PBF16>
__device__ inline float load_param(rsrc_t r, uint32_t voff, uint32_t soff) {
  if (PBF16) return bf16_bits_to_f32(static_cast<uint16_t>(bload16(r, voff, soff)));
  return __builtin_bit_cast(float, bload32(r, voff, soff));
}

template <int GROUP, bool ASYM, bool PBF16>
struct WInt4 {
  static constexpr int KBLK = 128, STEPS = 4;
  static constexpr int NG = 128 / GROUP;  // groups per block
  static constexpr int MPG = 4 / NG;      // MFMA steps (of 32 columns) per group
  // asymmetric bf16 parameters come as (scale, zero) pairs in one dword: one load per group
  static constexpr bool PAIR = ASYM && PBF16;
  static constexpr int PB = (PBF16 && !PAIR) ? 2 : 4;  // bytes per tiled parameter element
  struct Args {
    const uint8_t* wt;
    const void* st;
    const void* zt;
  };
  struct Ctx {
    rsrc_t wr, sr, zr;
    uint32_t wvo, pvo;
  };
  struct P {
    float sc[NG];
    float zf[NG];
  };
  __device__ static Ctx ctx(const Args& a, int t, int KB, int lane) { return ctx_tiles(a, t, 1, KB, lane); }
  // tiles t .. t+nt-1: tile r's block kb is block r*KB + kb of the range
  __device__ static Ctx ctx_tiles(const Args& a, int t, int nt, int KB, int lane) {
    Ctx c;
    c.wr = make_rsrc(a.wt + (int64_t)t * KB * 1024, (uint32_t)nt * (uint32_t)KB * 1024u);
    const uint32_t pbytes = (uint32_t)KB * NG * 16u * PB;
    c.sr = make_rsrc(static_cast<const char*>(a.st) + (int64_t)t * pbytes, (uint32_t)nt * pbytes);
    c.zr = ASYM ? make_rsrc(static_cast<const char*>(a.zt) + (int64_t)t * pbytes, (uint32_t)nt * pbytes) : c.sr;
    c.wvo = (uint32_t)lane * 16u;
    c.pvo = (uint32_t)(lane & 15) * PB;
    return c;
  }
  __device__ static void load(const Ctx& c, int kb, u32x4_t& w, P& p) {
    w = bload128<2>(c.wr, c.wvo, (uint32_t)kb * 1024u);
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const uint32_t off = (uint32_t)(kb * NG + g) * 16u * PB;
      if constexpr (PAIR) {
        const uint32_t v = bload32(c.sr, c.pvo, off);
        p.sc[g] = bf16_bits_to_f32(static_cast<uint16_t>(v & 0xffffu));
        p.zf[g] = bf16_bits_to_f32(static_cast<uint16_t>(v >> 16));
      } else {
        p.sc[g] = load_param<PBF16>(c.sr, c.pvo, off);
        p.zf[g] = ASYM ? load_param<PBF16>(c.zr, c.pvo, off) : 8.0f;
      }
    }
  }
  __device__ static int xk(int i, int jg) { return 32 * i + 8 * jg; }
  template <class A, int MCH>
  __device__ static void mma(const u32x4_t& w, const P& p, const u32x4_t (&xv)[MCH][4], f32x4_t (&yacc)[MCH]) {
    const uint32_t kMask = 0x000F000Fu;
    const uint32_t magic = A::kMagicPair;
    u32x4_t b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t d = w[i];
      b[i] = u32x4_t{and_or(d, kMask, magic), and_or(d >> 4, kMask, magic), and_or(d >> 8, kMask, magic),
                     and_or(d >> 12, kMask, magic)};
    }
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const uint32_t off = A::pair_from_f32(-(A::kMagic + p.zf[g]));
      const u32x4_t boff = u32x4_t{off, off, off, off};
#pragma unroll
      for (int c = 0; c < MCH; ++c) {
        f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = g * MPG; i < (g + 1) * MPG; ++i) acc = A::mfma(xv[c][i], b[i], acc);
#pragma unroll
        for (int i = g * MPG; i < (g + 1) * MPG; ++i) acc = A::mfma(xv[c][i], boff, acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) yacc[c][r] = fmaf(p.sc[g], acc[r], yacc[c][r]);
      }
    }
  }
  // One activation row (the GEMV's ONE form): the code chains only, with the offset charged
  // through the groups' activation sums sig[g]; y0 is the row's output for this lane's weight row.
  static constexpr bool kSumOffset = true;
  template <class A>
  __device__ static void mma_one(const u32x4_t& w, const P& p, const u32x4_t (&xv)[4], const float (&sig)[NG],
                                 float& y0) {
    const uint32_t kMask = 0x000F000Fu;
    const uint32_t magic = A::kMagicPair;
    u32x4_t b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t d = w[i];
      b[i] = u32x4_t{and_or(d, kMask, magic), and_or(d >> 4, kMask, magic), and_or(d >> 8, kMask, magic),
                     and_or(d >> 12, kMask, magic)};
    }
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = g * MPG; i < (g + 1) * MPG; ++i) acc = A::mfma(xv[i], b[i], acc);
      y0 = fmaf(p.sc[g], fmaf(-(A::kMagic + p.zf[g]), sig[g], acc[0]), y0);
    }
  }
  __device__ static float out_scale(const Args&, int) { return 1.0f; }

  // The skinny linear's hooks: B fragment of step i as (magic + code) pairs, the value each
  // activation must be charged back per group (magic + zero point), and the group scale.
  template <class A>
  __device__ static u32x4_t bfrag(const u32x4_t& w, int i) {
    const uint32_t d = w[i];
    const uint32_t kMask = 0x000F000Fu;
    const uint32_t magic = A::kMagicPair;
    return u32x4_t{and_or(d, kMask, magic), and_or(d >> 4, kMask, magic), and_or(d >> 8, kMask, magic),
                   and_or(d >> 12, kMask, magic)};
  }
  static constexpr bool kConstOffset = !ASYM;
  static constexpr int kLoads = 1 + NG * (ASYM ? 2 : 1);  // buffer loads of one block (codes + parameters)
  template <class A>
  __device__ static float const_offset() { return A::kMagic + 8.0f; }
  template <class A>
  __device__ static float offset(const P& p, int g) { return A::kMagic + p.zf[g]; }
  __device__ static float scale(const P& p, int g) { return p.sc[g]; }
};

template <class A, int GROUP, bool ASYM, bool PBF16, bool YF32 = false>
static hipError_t launch_int4(const uint8_t* wt, const void* st, const void* zt, const uint16_t* x, void* y,
                              const uint16_t* bias, const float* colscale, int64_t m, int64_t rows, int64_t cols,
                              int k_slices, hipStream_t s) {
  using W = WInt4<GROUP, ASYM, PBF16>;
  const typename W::Args a{wt, st, zt};
  return gemv_launch<A, W, SQX_INT4_U1, SQX_INT4_U2, YF32>(a, x, y, bias, colscale, m, rows, cols, k_slices, s);
}

// The decode GEMV with fp32 outputs and no bias (bf16 activation rows; the fp32-activation linear
// runs its hi/lo rows through it).
hipError_t int4_gemv_f32out(const uint8_t* wt, const void* st, const void* zt, bool pbf16, const uint16_t* x,
                            float* y, int64_t m, int64_t rows, int64_t cols, int group, hipStream_t s) {
#define SQX_F32G(G_)                                                                                             \
  {                                                                                                              \
    if (zt) {                                                                                                    \
      if (pbf16) return launch_int4<ActBF16, G_, true, true, true>(wt, st, zt, x, y, nullptr, nullptr, m, rows, cols, 0, s); \
      return launch_int4<ActBF16, G_, true, false, true>(wt, st, zt, x, y, nullptr, nullptr, m, rows, cols, 0, s);  \
    }                                                                                                            \
    if (pbf16) return launch_int4<ActBF16, G_, false, true, true>(wt, st, zt, x, y, nullptr, nullptr, m, rows, cols, 0, s); \
    return launch_int4<ActBF16, G_, false, false, true>(wt, st, zt, x, y, nullptr, nullptr, m, rows, cols, 0, s);   \
  }
  if (group == 128) SQX_F32G(128)
  if (group == 64) SQX_F32G(64)
  SQX_F32G(32)
#undef SQX_F32G
}

// The decode step's fused linears (symmetric codes, fp32 scales, bf16 activations): the residual
// add + RMSNorm, or the SiLU gate, computed in the LDS copy of the activations.
// RES: the residual epilogue (one row): y is unused, pa.res_out and pa.ss_out are written.
template <int PRO, bool RES, bool SWI = false>
static hipError_t launch_int4_pro_res(int group, const uint8_t* wt, const float* st, const uint16_t* x, uint16_t* y,
                                      int64_t m, int64_t rows, int64_t cols, int k_slices, hipStream_t s,
                                      const ProArgs& pa) {
#define SQX_PRO(G_)                                                                                                 \
  {                                                                                                                 \
    using W = WInt4<G_, false, false>;                                                                              \
    const typename W::Args a{wt, st, nullptr};                                                                      \
    return gemv_launch<ActBF16, W, SQX_INT4_U1, SQX_INT4_U2, false, PRO, RES, false, SWI>(                          \
        a, x, y, nullptr, nullptr, m, rows, cols, k_slices, s, pa);                                                 \
  }
  if (group == 128) SQX_PRO(128)
  if (group == 64) SQX_PRO(64)
  SQX_PRO(32)
#undef SQX_PRO
}

template <int PRO>
static hipError_t launch_int4_pro(int group, const uint8_t* wt, const float* st, const uint16_t* x, uint16_t* y,
                                  int64_t m, int64_t rows, int64_t cols, int k_slices, hipStream_t s, const ProArgs& pa) {
  return launch_int4_pro_res<PRO, false>(group, wt, st, x, y, m, rows, cols, k_slices, s, pa);
}

template <class A, bool ASYM, bool PBF16>
static hipError_t launch_int4_skinny(int group, const uint8_t* wt, const void* st, const void* zt, const uint16_t* x,
                                     uint16_t* y, const uint16_t* bias, int64_t m, int64_t rows, int64_t cols,
                                     SkinnyShape sh, float* ws, int64_t ws_bytes, hipStream_t s,
                                     bool reduce = true) {
#define SQX_SKG(G_)                                                                                  \
  {                                                                                                  \
    using W = WInt4<G_, ASYM, PBF16>;                                                                \
    const typename W::Args a{wt, st, zt};                                                            \
    return skinny_launch<A, W>(a, x, y, bias, m, rows, cols, sh, ws, ws_bytes, s, reduce);           \
  }
  if (group == 128) SQX_SKG(128)
  if (group == 64) SQX_SKG(64)
  SQX_SKG(32)
#undef SQX_SKG
}

template <class A, bool ASYM, bool PBF16>
static hipError_t launch_int4_rows(int group, const uint8_t* wt, const void* st, const void* zt, const uint16_t* x,
                                   uint16_t* y, const uint16_t* bias, int64_t m, int64_t rows, int64_t cols, int waves,
                                   int groups, hipStream_t s) {
#define SQX_ROWG(G_)                                                                        \
  {                                                                                         \
    using W = WInt4<G_, ASYM, PBF16>;                                                       \
    const typename W::Args a{wt, st, zt};                                                   \
    return gemv_rows_launch<A, W>(a, x, y, bias, m, rows, cols, waves, s, ProArgs{}, groups); \
  }
  if (group == 128) SQX_ROWG(128)
  if (group == 64) SQX_ROWG(64)
  SQX_ROWG(32)
#undef SQX_ROWG
}

template <class A, bool ASYM, bool PBF16>
static hipError_t launch_int4_g(int group, const uint8_t* wt, const void* st, const void* zt, const uint16_t* x,
                                uint16_t* y, const uint16_t* bias, const float* colscale, int64_t m, int64_t rows,
                                int64_t cols, int k_slices, hipStream_t s) {
  if (group == 128) return launch_int4<A, 128, ASYM, PBF16>(wt, st, zt, x, y, bias, colscale, m, rows, cols, k_slices, s);
  if (group == 64) return launch_int4<A, 64, ASYM, PBF16>(wt, st, zt, x, y, bias, colscale, m, rows, cols, k_slices, s);
  return launch_int4<A, 32, ASYM, PBF16>(wt, st, zt, x, y, bias, colscale, m, rows, cols, k_slices, s);
}

}  // namespace sqx

using namespace sqx;

// ==============================================================================================
// extern "C" entry points
// ==============================================================================================
static bool is_float_dtype(int d) { return d == SQX_DTYPE_F32 || d == SQX_DTYPE_BF16 || d == SQX_DTYPE_F16; }

static int int4_quantize_impl(const void* w, int w_dtype, int64_t rows, int64_t cols, int64_t group,
                              const float* colmul, int8_t* q, float* scales, float* weff, sqx_stream_t stream,
                              const char* fn) {
  SQX_REQUIRE(w && (weff || (q && scales)), SQX_E_ARG, "%s: null pointer", fn);
  SQX_REQUIRE(is_float_dtype(w_dtype), SQX_E_ARG, "%s: unsupported w_dtype %d", fn, w_dtype);
  SQX_REQUIRE(rows >= 0 && cols >= 0 && group > 0, SQX_E_ARG, "%s: bad shape", fn);
  SQX_REQUIRE(cols % group == 0, SQX_E_ARG, "in_features=%lld not divisible by group_size=%lld", (long long)cols,
              (long long)group);
  const int64_t n = rows * cols;
  if (n == 0) return SQX_OK;
  hipStream_t s = as_stream(stream);
  const bool fast = group >= 8 && group <= 512 && (group & (group - 1)) == 0 &&
                    (weff != nullptr || reinterpret_cast<uintptr_t>(q) % 8 == 0);
  const bool cm = colmul != nullptr;
  const bool fk = weff != nullptr;
  if (fast) {
    const dim3 grid(static_cast<unsigned>(ceil_div(n / 8, 256)));
#define SQX_Q_LAUNCH(L, CM, FK) \
  hipLaunchKernelGGL((int4_quantize_sym_kernel<L, CM, FK>), grid, dim3(256), 0, s, w, w_dtype, n, cols, group, colmul, q, scales, weff)
#define SQX_Q_CASE(L) \
  case L: if (fk) SQX_Q_LAUNCH(L, true, true); else if (cm) SQX_Q_LAUNCH(L, true, false); else SQX_Q_LAUNCH(L, false, false); break;
    switch (group / 8) { SQX_Q_CASE(1) SQX_Q_CASE(2) SQX_Q_CASE(4) SQX_Q_CASE(8) SQX_Q_CASE(16) SQX_Q_CASE(32) SQX_Q_CASE(64) }
#undef SQX_Q_CASE
#undef SQX_Q_LAUNCH
  } else {
    const int64_t ng = n / group;
    const dim3 grid(static_cast<unsigned>(ceil_div(ng, 256)));
    if (fk)
      hipLaunchKernelGGL((int4_quantize_sym_generic_kernel<true, true>), grid, dim3(256), 0, s, w, w_dtype, ng, cols,
                         group, colmul, q, scales, weff);
    else if (cm)
      hipLaunchKernelGGL((int4_quantize_sym_generic_kernel<true, false>), grid, dim3(256), 0, s, w, w_dtype, ng, cols,
                         group, colmul, q, scales, weff);
    else
      hipLaunchKernelGGL((int4_quantize_sym_generic_kernel<false, false>), grid, dim3(256), 0, s, w, w_dtype, ng, cols,
                         group, colmul, q, scales, weff);
  }
  SQX_LAUNCH_CHECK(fn);
  return SQX_OK;
}

extern "C" int sqx_int4_quantize_sym(const void* w, int w_dtype, int64_t rows, int64_t cols, int64_t group,
                                     int8_t* q, float* scales, sqx_stream_t stream) {
  return int4_quantize_impl(w, w_dtype, rows, cols, group, nullptr, q, scales, nullptr, stream,
                            "sqx_int4_quantize_sym");
}

extern "C" int sqx_awq_quantize(const void* w, int w_dtype, const float* chan_scale, int64_t rows, int64_t cols,
                                int64_t group, int8_t* q, float* scales, sqx_stream_t stream) {
  SQX_REQUIRE(chan_scale, SQX_E_ARG, "sqx_awq_quantize: null chan_scale");
  return int4_quantize_impl(w, w_dtype, rows, cols, group, chan_scale, q, scales, nullptr, stream, "sqx_awq_quantize");
}

extern "C" int sqx_awq_fake_quant(const void* w, int w_dtype, const float* chan_scale, int64_t rows, int64_t cols,
                                  int64_t group, float* w_eff, sqx_stream_t stream) {
  SQX_REQUIRE(chan_scale && w_eff, SQX_E_ARG, "sqx_awq_fake_quant: null pointer");
  return int4_quantize_impl(w, w_dtype, rows, cols, group, chan_scale, nullptr, nullptr, w_eff, stream,
                            "sqx_awq_fake_quant");
}

extern "C" int sqx_awq_dequantize(const int8_t* q, const float* group_scales, const float* chan_scale, int64_t rows,
                                  int64_t cols, int64_t group, float* out, sqx_stream_t stream) {
  SQX_REQUIRE(rows >= 0 && cols > 0 && group > 0 && cols % group == 0, SQX_E_ARG, "sqx_awq_dequantize: bad shape");
  const int64_t n = rows * cols;
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(q && group_scales && chan_scale && out, SQX_E_ARG, "sqx_awq_dequantize: null pointer");
  hipLaunchKernelGGL(awq_dequantize_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0,
                     as_stream(stream), q, group_scales, chan_scale, n, cols, group, out);
  SQX_LAUNCH_CHECK("sqx_awq_dequantize");
  return SQX_OK;
}

extern "C" int sqx_col_absmean(const void* x, int dtype, int64_t rows, int64_t cols, float* out, sqx_stream_t stream) {
  SQX_REQUIRE(is_float_dtype(dtype) && rows > 0 && cols >= 0, SQX_E_ARG, "sqx_col_absmean: bad dtype or shape");
  if (cols == 0) return SQX_OK;
  SQX_REQUIRE(x && out, SQX_E_ARG, "sqx_col_absmean: null pointer");
  hipLaunchKernelGGL(col_absmean_kernel, dim3(static_cast<unsigned>(ceil_div(cols, 256))), dim3(256), 0,
                     as_stream(stream), x, dtype, rows, cols, out);
  SQX_LAUNCH_CHECK("sqx_col_absmean");
  return SQX_OK;
}

extern "C" int sqx_awq_scale(const float* act, int64_t n, float ratio, float* out, sqx_stream_t stream) {
  SQX_REQUIRE(n > 0 && act && out, SQX_E_ARG, "sqx_awq_scale: bad arguments");
  hipLaunchKernelGGL(awq_scale_kernel, dim3(1), dim3(1024), 0, as_stream(stream), act, n, ratio, out);
  SQX_LAUNCH_CHECK("sqx_awq_scale");
  return SQX_OK;
}

extern "C" int sqx_scale_columns(const void* x, int act_dtype, const float* s, int64_t rows, int64_t cols, void* out,
                                 sqx_stream_t stream) {
  SQX_REQUIRE(act_dtype == SQX_DTYPE_BF16 || act_dtype == SQX_DTYPE_F16, SQX_E_ARG,
              "sqx_scale_columns: activations must be BF16 or F16");
  const int64_t n = rows * cols;
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(x && s && out && cols > 0, SQX_E_ARG, "sqx_scale_columns: bad arguments");
  if (cols % 8 == 0 && rows < 65536 && cols < (int64_t(1) << 30) && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(s) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0) {
    const dim3 grid8(static_cast<unsigned>(ceil_div(cols / 8, 256)), static_cast<unsigned>(rows));
    if (act_dtype == SQX_DTYPE_BF16)
      hipLaunchKernelGGL(scale_columns8_kernel<ActBF16>, grid8, dim3(256), 0, as_stream(stream),
                         static_cast<const uint16_t*>(x), s, static_cast<int>(cols), static_cast<uint16_t*>(out));
    else
      hipLaunchKernelGGL(scale_columns8_kernel<ActF16>, grid8, dim3(256), 0, as_stream(stream),
                         static_cast<const uint16_t*>(x), s, static_cast<int>(cols), static_cast<uint16_t*>(out));
    SQX_LAUNCH_CHECK("sqx_scale_columns");
    return SQX_OK;
  }
  const dim3 grid(static_cast<unsigned>(ceil_div(n, 256)));
  if (act_dtype == SQX_DTYPE_BF16)
    hipLaunchKernelGGL(scale_columns_kernel<ActBF16>, grid, dim3(256), 0, as_stream(stream),
                       static_cast<const uint16_t*>(x), s, n, cols, static_cast<uint16_t*>(out));
  else
    hipLaunchKernelGGL(scale_columns_kernel<ActF16>, grid, dim3(256), 0, as_stream(stream),
                       static_cast<const uint16_t*>(x), s, n, cols, static_cast<uint16_t*>(out));
  SQX_LAUNCH_CHECK("sqx_scale_columns");
  return SQX_OK;
}

extern "C" int sqx_int4_quantize_asym(const void* w, int w_dtype, int64_t rows, int64_t cols, int64_t group,
                                      int param_dtype, uint8_t* q, void* scales, void* zeros, sqx_stream_t stream) {
  SQX_REQUIRE(is_float_dtype(w_dtype), SQX_E_ARG, "sqx_int4_quantize_asym: unsupported w_dtype %d", w_dtype);
  SQX_REQUIRE(param_dtype == SQX_DTYPE_F32 || param_dtype == SQX_DTYPE_BF16, SQX_E_ARG,
              "sqx_int4_quantize_asym: param_dtype must be F32 or BF16");
  SQX_REQUIRE(rows >= 0 && cols >= 0 && group > 0, SQX_E_ARG, "sqx_int4_quantize_asym: bad shape");
  SQX_REQUIRE(cols % group == 0, SQX_E_ARG, "in_features=%lld not divisible by group_size=%lld", (long long)cols,
              (long long)group);
  const int64_t ng = rows * cols / group;
  if (ng == 0) return SQX_OK;
  SQX_REQUIRE(w && q && scales && zeros, SQX_E_ARG, "sqx_int4_quantize_asym: null pointer");
  const dim3 grid(static_cast<unsigned>(ceil_div(ng, 256)));
  if (param_dtype == SQX_DTYPE_BF16)
    hipLaunchKernelGGL(int4_quantize_asym_kernel<true>, grid, dim3(256), 0, as_stream(stream), w, w_dtype, ng, group, q,
                       scales, zeros);
  else
    hipLaunchKernelGGL(int4_quantize_asym_kernel<false>, grid, dim3(256), 0, as_stream(stream), w, w_dtype, ng, group,
                       q, scales, zeros);
  SQX_LAUNCH_CHECK("sqx_int4_quantize_asym");
  return SQX_OK;
}

extern "C" int sqx_int4_pack(const int8_t* q, int64_t n, uint8_t* packed, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0, SQX_E_ARG, "sqx_int4_pack: negative length");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(q && packed, SQX_E_ARG, "sqx_int4_pack: null pointer");
  const int64_t nb = (n + 1) / 2;
  hipLaunchKernelGGL(int4_pack_kernel, dim3(static_cast<unsigned>(ceil_div(nb, 256))), dim3(256), 0,
                     as_stream(stream), q, n, packed);
  SQX_LAUNCH_CHECK("sqx_int4_pack");
  return SQX_OK;
}

extern "C" int sqx_int4_unpack(const uint8_t* packed, int64_t n, int8_t* q, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0, SQX_E_ARG, "sqx_int4_unpack: negative length");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(q && packed, SQX_E_ARG, "sqx_int4_unpack: null pointer");
  const int64_t nb = (n + 1) / 2;
  hipLaunchKernelGGL(int4_unpack_kernel, dim3(static_cast<unsigned>(ceil_div(nb, 256))), dim3(256), 0,
                     as_stream(stream), packed, n, q);
  SQX_LAUNCH_CHECK("sqx_int4_unpack");
  return SQX_OK;
}

extern "C" int sqx_int4_dequantize(const int8_t* q, const float* scales, int64_t rows, int64_t cols,
                                   int64_t group, float* out, sqx_stream_t stream) {
  SQX_REQUIRE(rows >= 0 && cols >= 0 && group > 0 && cols % group == 0, SQX_E_ARG,
              "sqx_int4_dequantize: bad shape [%lld, %lld] / group %lld", (long long)rows, (long long)cols,
              (long long)group);
  const int64_t n = rows * cols;
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(q && scales && out, SQX_E_ARG, "sqx_int4_dequantize: null pointer");
  hipLaunchKernelGGL(int4_dequantize_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0,
                     as_stream(stream), q, scales, n, group, out);
  SQX_LAUNCH_CHECK("sqx_int4_dequantize");
  return SQX_OK;
}

extern "C" int64_t sqx_int4_tiled_weight_bytes(int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0) return -1;
  return ceil_div(rows, 16) * ceil_div(cols, 128) * 1024;
}

extern "C" int64_t sqx_int4_tiled_param_count(int64_t rows, int64_t cols, int64_t group) {
  if (rows < 0 || cols < 0 || !(group == 32 || group == 64 || group == 128)) return -1;
  return ceil_div(rows, 16) * ceil_div(cols, 128) * (128 / group) * 16;
}

static int tile_params(const void* src, int param_dtype, int64_t rows, int64_t cols, int64_t group, void* dst,
                       hipStream_t s) {
  const int64_t Gp = ceil_div(cols, 128) * (128 / group);
  const int64_t n_out = ceil_div(rows, 16) * Gp * 16;
  const dim3 grid(static_cast<unsigned>(ceil_div(n_out, 256)));
  if (param_dtype == SQX_DTYPE_F32)
    hipLaunchKernelGGL(int4_tile_params_kernel<float>, grid, dim3(256), 0, s, static_cast<const float*>(src), rows,
                       cols / group, Gp, n_out, static_cast<float*>(dst));
  else
    hipLaunchKernelGGL(int4_tile_params_kernel<uint16_t>, grid, dim3(256), 0, s, static_cast<const uint16_t*>(src),
                       rows, cols / group, Gp, n_out, static_cast<uint16_t*>(dst));
  return SQX_OK;
}

static int check_tile_args(int64_t rows, int64_t cols, int64_t group, int param_dtype) {
  SQX_REQUIRE(rows > 0 && cols > 0, SQX_E_ARG, "sqx_int4_tile: empty weight [%lld, %lld]", (long long)rows,
              (long long)cols);
  SQX_REQUIRE(group == 32 || group == 64 || group == 128, SQX_E_ARG,
              "sqx_int4_tile: group_size %lld unsupported by the tiled kernels (32, 64 or 128)", (long long)group);
  SQX_REQUIRE(cols % group == 0, SQX_E_ARG, "in_features=%lld not divisible by group_size=%lld", (long long)cols,
              (long long)group);
  SQX_REQUIRE(param_dtype == SQX_DTYPE_F32 || param_dtype == SQX_DTYPE_BF16, SQX_E_ARG,
              "sqx_int4_tile: param_dtype must be F32 or BF16");
  SQX_REQUIRE(rows <= (int64_t)1 << 30 && cols <= (int64_t)1 << 30, SQX_E_ARG, "sqx_int4_tile: shape too large");
  return SQX_OK;
}

extern "C" int sqx_int4_tile(const int8_t* codes, int code_kind, const void* scales, const void* zeros,
                             int param_dtype, int64_t rows, int64_t cols, int64_t group, uint8_t* wt, void* st,
                             void* zt, sqx_stream_t stream) {
  int rc = check_tile_args(rows, cols, group, param_dtype);
  if (rc) return rc;
  SQX_REQUIRE(code_kind == 0 || code_kind == 1, SQX_E_ARG, "sqx_int4_tile: code_kind must be 0 or 1");
  SQX_REQUIRE(codes && scales && wt && st, SQX_E_ARG, "sqx_int4_tile: null pointer");
  SQX_REQUIRE(code_kind == 0 || (zeros && zt), SQX_E_ARG, "sqx_int4_tile: asymmetric codes need zeros and zt");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0, SQX_E_ARG, "sqx_int4_tile: wt must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  const int64_t KB = ceil_div(cols, 128);
  const int64_t n_dwords = ceil_div(rows, 16) * KB * 256;
  const dim3 grid(static_cast<unsigned>(ceil_div(n_dwords, 256)));
  if (code_kind == 0)
    hipLaunchKernelGGL((int4_tile_weights_kernel<false, true>), grid, dim3(256), 0, s, codes, rows, cols, KB,
                       n_dwords, reinterpret_cast<uint32_t*>(wt));
  else
    hipLaunchKernelGGL((int4_tile_weights_kernel<false, false>), grid, dim3(256), 0, s, codes, rows, cols, KB,
                       n_dwords, reinterpret_cast<uint32_t*>(wt));
  if (code_kind == 1 && param_dtype == SQX_DTYPE_BF16) {  // (scale, zero) pairs in st; zt unused
    const int64_t Gp = KB * (128 / group);
    const int64_t n_out = ceil_div(rows, 16) * Gp * 16;
    hipLaunchKernelGGL(int4_tile_param_pairs_kernel, dim3(static_cast<unsigned>(ceil_div(n_out, 256))), dim3(256), 0, s,
                       static_cast<const uint16_t*>(scales), static_cast<const uint16_t*>(zeros), rows, cols / group,
                       Gp, n_out, static_cast<uint32_t*>(st));
  } else {
    tile_params(scales, param_dtype, rows, cols, group, st, s);
    if (code_kind == 1) tile_params(zeros, param_dtype, rows, cols, group, zt, s);
  }
  SQX_LAUNCH_CHECK("sqx_int4_tile");
  return SQX_OK;
}

extern "C" int sqx_int4_tile_packed(const uint8_t* packed, const void* scales, int param_dtype, int64_t rows,
                                    int64_t cols, int64_t group, uint8_t* wt, void* st, sqx_stream_t stream) {
  int rc = check_tile_args(rows, cols, group, param_dtype);
  if (rc) return rc;
  SQX_REQUIRE(packed && scales && wt && st, SQX_E_ARG, "sqx_int4_tile_packed: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0, SQX_E_ARG, "sqx_int4_tile_packed: wt must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  const int64_t KB = ceil_div(cols, 128);
  const int64_t n_dwords = ceil_div(rows, 16) * KB * 256;
  hipLaunchKernelGGL((int4_tile_weights_kernel<true, true>), dim3(static_cast<unsigned>(ceil_div(n_dwords, 256))),
                     dim3(256), 0, s, packed, rows, cols, KB, n_dwords, reinterpret_cast<uint32_t*>(wt));
  tile_params(scales, param_dtype, rows, cols, group, st, s);
  SQX_LAUNCH_CHECK("sqx_int4_tile_packed");
  return SQX_OK;
}

extern "C" int sqx_int4_untile(const uint8_t* wt, const void* st, const void* zt, int param_dtype, int code_kind,
                               int64_t rows, int64_t cols, int64_t group, int8_t* codes, void* scales, void* zeros,
                               sqx_stream_t stream) {
  int rc = check_tile_args(rows, cols, group, param_dtype);
  if (rc) return rc;
  SQX_REQUIRE(code_kind == 0 || code_kind == 1, SQX_E_ARG, "sqx_int4_untile: code_kind must be 0 or 1");
  SQX_REQUIRE(wt && st && codes && scales, SQX_E_ARG, "sqx_int4_untile: null pointer");
  SQX_REQUIRE(code_kind == 0 || (zt && zeros), SQX_E_ARG, "sqx_int4_untile: asymmetric codes need zt and zeros");
  hipStream_t s = as_stream(stream);
  const int64_t KB = ceil_div(cols, 128);
  const int64_t n_dwords = ceil_div(rows, 16) * KB * 256;
  const dim3 grid(static_cast<unsigned>(ceil_div(n_dwords, 256)));
  const uint32_t* w32 = reinterpret_cast<const uint32_t*>(wt);
  if (code_kind == 0)
    hipLaunchKernelGGL(int4_untile_weights_kernel<true>, grid, dim3(256), 0, s, w32, rows, cols, KB, n_dwords, codes);
  else
    hipLaunchKernelGGL(int4_untile_weights_kernel<false>, grid, dim3(256), 0, s, w32, rows, cols, KB, n_dwords, codes);
  const int64_t n_groups = cols / group, Gp = KB * (128 / group);
  const int64_t n_in = ceil_div(rows, 16) * Gp * 16;
  const dim3 pgrid(static_cast<unsigned>(ceil_div(n_in, 256)));
  if (code_kind == 1 && param_dtype == SQX_DTYPE_BF16) {
    hipLaunchKernelGGL(int4_untile_param_pairs_kernel, pgrid, dim3(256), 0, s, static_cast<const uint32_t*>(st), rows,
                       n_groups, Gp, n_in, static_cast<uint16_t*>(scales), static_cast<uint16_t*>(zeros));
    SQX_LAUNCH_CHECK("sqx_int4_untile");
    return SQX_OK;
  }
  for (int k = 0; k < (code_kind == 1 ? 2 : 1); ++k) {
    const void* src = k == 0 ? st : zt;
    void* dst = k == 0 ? scales : zeros;
    if (param_dtype == SQX_DTYPE_F32)
      hipLaunchKernelGGL(int4_untile_params_kernel<float>, pgrid, dim3(256), 0, s, static_cast<const float*>(src), rows,
                         n_groups, Gp, n_in, static_cast<float*>(dst));
    else
      hipLaunchKernelGGL(int4_untile_params_kernel<uint16_t>, pgrid, dim3(256), 0, s,
                         static_cast<const uint16_t*>(src), rows, n_groups, Gp, n_in, static_cast<uint16_t*>(dst));
  }
  SQX_LAUNCH_CHECK("sqx_int4_untile");
  return SQX_OK;
}

extern "C" int sqx_int4_linear_default_kslices(int64_t m, int64_t rows, int64_t cols) {
  if (m <= 0 || rows <= 0 || cols <= 0) return 1;
  return gemv_default_kslices(rows, cols, 128, m);
}

static int int4_skinny_impl(const uint8_t* wt, const void* st, const void* zt, int param_dtype, const void* x,
                            int act_dtype, void* y, const void* bias, int64_t m, int64_t rows, int64_t cols,
                            int64_t group, SkinnyShape sh, void* ws, int64_t ws_bytes, sqx_stream_t stream,
                            const char* fn, bool reduce = true);

static int int4_linear_impl(const uint8_t* wt, const void* st, const void* zt, int param_dtype, const void* x,
                            int act_dtype, void* y, const void* bias, const float* colscale, int64_t m,
                            int64_t rows, int64_t cols, int64_t group, int k_slices, sqx_stream_t stream,
                            const char* fn) {
  SQX_REQUIRE(m >= 0 && rows > 0 && cols > 0, SQX_E_ARG, "%s: bad shape m=%lld rows=%lld cols=%lld", fn,
              (long long)m, (long long)rows, (long long)cols);
  SQX_REQUIRE(group == 32 || group == 64 || group == 128, SQX_E_ARG, "%s: group_size %lld unsupported (32, 64 or 128)",
              fn, (long long)group);
  SQX_REQUIRE(cols % group == 0, SQX_E_ARG, "in_features=%lld not divisible by group_size=%lld", (long long)cols,
              (long long)group);
  SQX_REQUIRE(act_dtype == SQX_DTYPE_BF16 || act_dtype == SQX_DTYPE_F16, SQX_E_ARG,
              "%s: activations must be BF16 or F16", fn);
  SQX_REQUIRE(param_dtype == SQX_DTYPE_F32 || param_dtype == SQX_DTYPE_BF16, SQX_E_ARG,
              "%s: param_dtype must be F32 or BF16", fn);
  SQX_REQUIRE(rows < ((int64_t)1 << 31) && m < ((int64_t)1 << 31) && ceil_div(cols, 128) * 1024 < ((int64_t)1 << 31) &&
                  64 * cols * 2 < ((int64_t)1 << 31),
              SQX_E_ARG, "%s: shape too large for 32-bit buffer offsets", fn);
  SQX_REQUIRE(k_slices <= 16, SQX_E_ARG, "%s: k_slices %d > 16", fn, k_slices);
  if (m == 0) return SQX_OK;
  SQX_REQUIRE(wt && st && x && y, SQX_E_ARG, "%s: null pointer", fn);
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0, SQX_E_ARG,
              "%s: wt and x must be 16-byte aligned", fn);
  if (colscale != nullptr) {
    SQX_REQUIRE(m <= 16 && gemv_xlds_bytes(m, ceil_div(cols, 128)) <= kXldsMax, SQX_E_ARG,
                "%s: per-column activation scaling needs m <= 16 and m*cols*2 <= %lld bytes", fn,
                (long long)kXldsMax);
  }
  if (k_slices <= 0 && colscale == nullptr && m >= 2 && m <= 64) {  // the decode-regime kernels (no K split)
    const SkinnyShape sh = skinny_default_shape(m, rows, cols, 128, false);
    if (!sh.gemv)
      return int4_skinny_impl(wt, st, zt, param_dtype, x, act_dtype, y, bias, m, rows, cols, group, sh, nullptr, 0,
                              stream, fn);
  }
  const bool asym = zt != nullptr;
  const bool pbf = param_dtype == SQX_DTYPE_BF16;
  hipStream_t s = as_stream(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  uint16_t* yp = static_cast<uint16_t*>(y);
  const uint16_t* b16 = static_cast<const uint16_t*>(bias);
  const int g = static_cast<int>(group);
  hipError_t e;
#define SQX_LIN(ACT, ASYM, PBF) \
  e = launch_int4_g<ACT, ASYM, PBF>(g, wt, st, zt, xp, yp, b16, colscale, m, rows, cols, k_slices, s)
  if (act_dtype == SQX_DTYPE_BF16) {
    if (asym) { if (pbf) SQX_LIN(ActBF16, true, true); else SQX_LIN(ActBF16, true, false); }
    else { if (pbf) SQX_LIN(ActBF16, false, true); else SQX_LIN(ActBF16, false, false); }
  } else {
    if (asym) { if (pbf) SQX_LIN(ActF16, true, true); else SQX_LIN(ActF16, true, false); }
    else { if (pbf) SQX_LIN(ActF16, false, true); else SQX_LIN(ActF16, false, false); }
  }
#undef SQX_LIN
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return SQX_OK;
}

extern "C" int sqx_int4_linear(const uint8_t* wt, const void* st, const void* zt, int param_dtype, const void* x,
                               int act_dtype, void* y, const void* bias, int64_t m, int64_t rows, int64_t cols,
                               int64_t group, int k_slices, sqx_stream_t stream) {
  return int4_linear_impl(wt, st, zt, param_dtype, x, act_dtype, y, bias, nullptr, m, rows, cols, group, k_slices,
                          stream, "sqx_int4_linear");
}

extern "C" int sqx_int4_linear_colscaled(const uint8_t* wt, const void* st, const void* zt, int param_dtype,
                                         const void* x, int act_dtype, const float* col_scale, void* y,
                                         const void* bias, int64_t m, int64_t rows, int64_t cols, int64_t group,
                                         int k_slices, sqx_stream_t stream) {
  SQX_REQUIRE(col_scale != nullptr, SQX_E_ARG, "sqx_int4_linear_colscaled: null col_scale");
  return int4_linear_impl(wt, st, zt, param_dtype, x, act_dtype, y, bias, col_scale, m, rows, cols, group, k_slices,
                          stream, "sqx_int4_linear_colscaled");
}

// The 1..64-row linear with an explicit launch shape: variant 0 (waves splitting K, 2 or 4 tiles
// per wave, 1..8 waves) or 1 (LDS-staged, 1, 2 or 4 tiles per wave, 4 or 8 compute waves), splits
// >= 1 workgroups along K. variant < 0 is the library's choice for the shape (the GEMV included when
// no other argument is given); tiles, waves or splits <= 0 pick the default of the variant.
static int int4_skinny_impl(const uint8_t* wt, const void* st, const void* zt, int param_dtype, const void* x,
                            int act_dtype, void* y, const void* bias, int64_t m, int64_t rows, int64_t cols,
                            int64_t group, SkinnyShape sh, void* ws, int64_t ws_bytes, sqx_stream_t stream,
                            const char* fn, bool reduce) {
  SQX_REQUIRE(m >= 0 && m <= 64 && rows > 0 && cols > 0, SQX_E_ARG,
              "%s: bad shape m=%lld rows=%lld cols=%lld (m <= 64)", fn, (long long)m, (long long)rows,
              (long long)cols);
  SQX_REQUIRE(group == 32 || group == 64 || group == 128, SQX_E_ARG, "%s: group_size %lld unsupported (32, 64 or 128)",
              fn, (long long)group);
  SQX_REQUIRE(cols % group == 0, SQX_E_ARG, "in_features=%lld not divisible by group_size=%lld", (long long)cols,
              (long long)group);
  SQX_REQUIRE(act_dtype == SQX_DTYPE_BF16 || act_dtype == SQX_DTYPE_F16, SQX_E_ARG,
              "%s: activations must be BF16 or F16", fn);
  SQX_REQUIRE(param_dtype == SQX_DTYPE_F32 || param_dtype == SQX_DTYPE_BF16, SQX_E_ARG,
              "%s: param_dtype must be F32 or BF16", fn);
  SQX_REQUIRE(rows < ((int64_t)1 << 31) && ceil_div(rows, 16) * ceil_div(cols, 128) * 1024 < ((int64_t)1 << 31) &&
                  64 * cols * 2 < ((int64_t)1 << 31),
              SQX_E_ARG, "%s: shape too large for 32-bit buffer offsets", fn);
  SQX_REQUIRE(sh.S >= 1 &&
                  ((sh.variant == 0 && (sh.R == 2 || sh.R == 4) && sh.waves >= 1 && sh.waves <= kSkinnyMaxWaves) ||
                   (sh.variant == 1 && (sh.R == 1 || sh.R == 2 || sh.R == 4) && (sh.waves == 4 || sh.waves == 8)) ||
                   (sh.variant == 2 && sh.S == 1 && sh.R >= 0 && sh.R <= 2 && sh.waves >= 0 && sh.waves <= 16)),
              SQX_E_ARG, "%s: bad launch shape (variant %d, tiles %d, waves %d, splits %d)", fn, sh.variant, sh.R,
              sh.waves, sh.S);
  SQX_REQUIRE(sh.variant != 2 || m == 0 || gemv_rows_groups(m, rows, cols, sh.waves, false, sh.R) != 0, SQX_E_ARG,
              "%s: the multi-row GEMV (variant 2) takes 2..8 rows with k-slices of at most 8 blocks (4 for 5..8 rows "
              "in one workgroup, tiles 1) (m=%lld, cols=%lld, waves %d, tiles %d)", fn, (long long)m, (long long)cols,
              sh.waves, sh.R);
  if (m == 0) return SQX_OK;
  SQX_REQUIRE(wt && st && x && (y || !reduce), SQX_E_ARG, "%s: null pointer", fn);
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0, SQX_E_ARG,
              "%s: wt and x must be 16-byte aligned", fn);
  {
    const int S = skinny_splits(ceil_div(cols, 128), sh.S);
    SQX_REQUIRE(S == 1 || (ws != nullptr && ws_bytes >= skinny_workspace_bytes(m, rows, (int)S) &&
                           reinterpret_cast<uintptr_t>(ws) % 16 == 0),
                SQX_E_ARG, "%s: %lld splits need a 16-byte aligned workspace of %lld bytes", fn, (long long)S,
                (long long)skinny_workspace_bytes(m, rows, (int)S));
  }
  const bool asym = zt != nullptr;
  const bool pbf = param_dtype == SQX_DTYPE_BF16;
  hipStream_t s = as_stream(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  uint16_t* yp = static_cast<uint16_t*>(y);
  const uint16_t* b16 = static_cast<const uint16_t*>(bias);
  float* wsp = static_cast<float*>(ws);
  const int g = static_cast<int>(group);
  hipError_t e;
  if (sh.variant == 2) {
    SQX_REQUIRE(reduce, SQX_E_ARG, "%s: the multi-row GEMV leaves no partials", fn);
#define SQX_ROWL(ACT, ASYM, PBF) \
  e = launch_int4_rows<ACT, ASYM, PBF>(g, wt, st, zt, xp, yp, b16, m, rows, cols, sh.waves, sh.R, s)
    if (act_dtype == SQX_DTYPE_BF16) {
      if (asym) { if (pbf) SQX_ROWL(ActBF16, true, true); else SQX_ROWL(ActBF16, true, false); }
      else { if (pbf) SQX_ROWL(ActBF16, false, true); else SQX_ROWL(ActBF16, false, false); }
    } else {
      if (asym) { if (pbf) SQX_ROWL(ActF16, true, true); else SQX_ROWL(ActF16, true, false); }
      else { if (pbf) SQX_ROWL(ActF16, false, true); else SQX_ROWL(ActF16, false, false); }
    }
#undef SQX_ROWL
    SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return SQX_OK;
  }
#define SQX_SKL(ACT, ASYM, PBF) \
  e = launch_int4_skinny<ACT, ASYM, PBF>(g, wt, st, zt, xp, yp, b16, m, rows, cols, sh, wsp, ws_bytes, s, reduce)
  if (act_dtype == SQX_DTYPE_BF16) {
    if (asym) { if (pbf) SQX_SKL(ActBF16, true, true); else SQX_SKL(ActBF16, true, false); }
    else { if (pbf) SQX_SKL(ActBF16, false, true); else SQX_SKL(ActBF16, false, false); }
  } else {
    if (asym) { if (pbf) SQX_SKL(ActF16, true, true); else SQX_SKL(ActF16, true, false); }
    else { if (pbf) SQX_SKL(ActF16, false, true); else SQX_SKL(ActF16, false, false); }
  }
#undef SQX_SKL
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return SQX_OK;
}

// Splits of the library's launch shape for m rows with a workspace (1 when it runs without a split,
// including the GEMV it picks for some shapes).
extern "C" int sqx_int4_skinny_default_splits(int64_t m, int64_t rows, int64_t cols) {
  if (m < 2 || m > 64 || rows <= 0 || cols <= 0) return 1;
  const SkinnyShape sh = skinny_default_shape(m, rows, cols, 128, true);
  return sh.gemv ? 1 : skinny_splits(ceil_div(cols, 128), sh.S);
}

extern "C" int sqx_int4_skinny_partials(const uint8_t* wt, const void* st, const void* zt, int param_dtype,
                                        const void* x, int act_dtype, int64_t m, int64_t rows, int64_t cols,
                                        int64_t group, void* ws, int64_t ws_bytes, sqx_stream_t stream) {
  const char* fn = "sqx_int4_skinny_partials";
  SQX_REQUIRE(m >= 2 && m <= 64 && rows > 0 && cols > 0, SQX_E_ARG, "%s: bad shape m=%lld (2..64 rows)", fn,
              (long long)m);
  const SkinnyShape sh = skinny_default_shape(m, rows, cols, 128, true);
  SQX_REQUIRE(!sh.gemv && skinny_splits(ceil_div(cols, 128), sh.S) >= 2, SQX_E_ARG,
              "%s: the library's shape for m=%lld rows=%lld cols=%lld does not split K (sqx_int4_skinny_default_splits "
              "is 1)", fn, (long long)m, (long long)rows, (long long)cols);
  return int4_skinny_impl(wt, st, zt, param_dtype, x, act_dtype, nullptr, nullptr, m, rows, cols, group, sh, ws,
                          ws_bytes, stream, fn, false);
}

extern "C" int64_t sqx_int4_skinny_workspace_bytes(int64_t m, int64_t rows, int64_t cols, int splits) {
  if (m <= 0 || m > 64 || rows <= 0 || cols <= 0) return 0;
  const int S = splits > 0 ? splits : skinny_default_shape(m, rows, cols, 128, true).S;
  return skinny_workspace_bytes(m, rows, skinny_splits(ceil_div(cols, 128), S));
}

extern "C" int sqx_int4_skinny(const uint8_t* wt, const void* st, const void* zt, int param_dtype, const void* x,
                               int act_dtype, void* y, const void* bias, int64_t m, int64_t rows, int64_t cols,
                               int64_t group, int variant, int tiles, int waves, int splits, void* ws,
                               int64_t ws_bytes, sqx_stream_t stream) {
  SkinnyShape sh = skinny_default_shape(m, rows, cols, 128, ws != nullptr);
  if (variant < 0 && tiles <= 0 && waves <= 0 && splits <= 0 && sh.gemv)  // the library's choice: the GEMV
    return int4_linear_impl(wt, st, zt, param_dtype, x, act_dtype, y, bias, nullptr, m, rows, cols, group,
                            sqx_int4_linear_default_kslices(m, rows, cols), stream, "sqx_int4_skinny");
  if (variant >= 0 && (variant != sh.variant || sh.gemv))  // the variant's own defaults
    sh = variant == 0 ? SkinnyShape{0, 2, 8, 1, false}
                      : (variant == 2 ? SkinnyShape{2, 0, 0, 1, false} : SkinnyShape{1, 2, 4, 1, false});
  if (variant > 2) sh.variant = variant;  // refused below
  if (tiles > 0) sh.R = tiles;
  if (waves > 0) sh.waves = waves;
  if (splits > 0) sh.S = splits;
  return int4_skinny_impl(wt, st, zt, param_dtype, x, act_dtype, y, bias, m, rows, cols, group, sh, ws, ws_bytes,
                          stream, "sqx_int4_skinny");
}

// The fused prologues keep a 64 KiB limit: at 8 rows of 4096 (65,664 bytes) the decode step with the
// norm fused into qkv and gate/up was slower (2.38 ms) than the one with separate norm kernels (2.35 ms).
static constexpr int64_t kProXldsMax = 64 * 1024;

extern "C" int sqx_int4_prologue_fits(int64_t m, int64_t cols) {
  return m >= 1 && m <= kProMaxRows && cols % 8 == 0 && cols > 0 &&
         gemv_xlds_bytes(m, ceil_div(cols, 128)) <= kProXldsMax;
}

static int int4_pro_check(const uint8_t* wt, const float* st, const void* x, void* y, int64_t m, int64_t rows,
                          int64_t cols, int64_t group, int k_slices, const char* fn) {
  SQX_REQUIRE(rows > 0 && cols > 0 && rows < ((int64_t)1 << 31), SQX_E_ARG, "%s: bad shape", fn);
  SQX_REQUIRE(group == 32 || group == 64 || group == 128, SQX_E_ARG, "%s: group_size %lld unsupported (32, 64 or 128)",
              fn, (long long)group);
  SQX_REQUIRE(cols % group == 0, SQX_E_ARG, "in_features=%lld not divisible by group_size=%lld", (long long)cols,
              (long long)group);
  SQX_REQUIRE(sqx_int4_prologue_fits(m, cols), SQX_E_ARG,
              "%s: m=%lld, cols=%lld: the fused prologue needs m <= %d and the rows in %lld bytes of LDS", fn,
              (long long)m, (long long)cols, kProMaxRows, (long long)kProXldsMax);
  SQX_REQUIRE(k_slices <= 16, SQX_E_ARG, "%s: k_slices %d > 16", fn, k_slices);
  SQX_REQUIRE(wt && st && x && y, SQX_E_ARG, "%s: null pointer", fn);
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0, SQX_E_ARG,
              "%s: wt and x must be 16-byte aligned", fn);
  return SQX_OK;
}

extern "C" int sqx_int4_linear_rmsnorm(const uint8_t* wt, const float* st, const void* x, const void* delta,
                                       const void* gain, float eps, void* h_out, void* y, int64_t m, int64_t rows,
                                       int64_t cols, int64_t group, int k_slices, sqx_stream_t stream) {
  const char* fn = "sqx_int4_linear_rmsnorm";
  const int rc = int4_pro_check(wt, st, x, y, m, rows, cols, group, k_slices, fn);
  if (rc != SQX_OK) return rc;
  SQX_REQUIRE(gain != nullptr && (delta == nullptr || h_out != nullptr), SQX_E_ARG, "%s: null gain or h_out", fn);
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(gain) % 16 == 0 && reinterpret_cast<uintptr_t>(delta) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(h_out) % 16 == 0,
              SQX_E_ARG, "%s: gain, delta and h_out must be 16-byte aligned", fn);
  const ProArgs pa{static_cast<const uint16_t*>(delta), static_cast<const uint16_t*>(gain), static_cast<uint16_t*>(h_out),
                   eps};
  const hipError_t e = launch_int4_pro<kProResNorm>(static_cast<int>(group), wt, st, static_cast<const uint16_t*>(x),
                                                    static_cast<uint16_t*>(y), m, rows, cols, k_slices,
                                                    as_stream(stream), pa);
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return SQX_OK;
}

// Whether the SiLU gate runs in the slices of the multi-row GEMV: where the library's plain linear of
// these rows is that kernel (so the fused and the two-call forms share one kernel and its sums).
static bool int4_silu_rows(int64_t m, int64_t rows, int64_t cols, int k_slices) {
  return k_slices <= 0 && m >= 2 && m <= 8 && rows > 0 && cols > 0 && cols % 8 == 0 &&
         skinny_default_shape(m, rows, cols, 128, true).variant == 2;
}

extern "C" int sqx_int4_linear_silu_fits(int64_t m, int64_t rows, int64_t cols) {
  return int4_silu_rows(m, rows, cols, 0) || sqx_int4_prologue_fits(m, cols);
}

extern "C" int sqx_int4_linear_silu(const uint8_t* wt, const float* st, const void* gate_up, void* y, int64_t m,
                                    int64_t rows, int64_t cols, int64_t group, int k_slices, sqx_stream_t stream) {
  const char* fn = "sqx_int4_linear_silu";
  if (int4_silu_rows(m, rows, cols, k_slices) && (group == 32 || group == 64 || group == 128) && cols % group == 0 &&
      rows < ((int64_t)1 << 31)) {
    SQX_REQUIRE(wt && st && gate_up && y, SQX_E_ARG, "%s: null pointer", fn);
    SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0 && reinterpret_cast<uintptr_t>(gate_up) % 16 == 0, SQX_E_ARG,
                "%s: wt and gate_up must be 16-byte aligned", fn);
    hipError_t e;
#define SQX_ROWSILU(G_)                                                                                          \
  {                                                                                                              \
    using W = WInt4<G_, false, false>;                                                                           \
    const typename W::Args a{wt, st, nullptr};                                                                   \
    e = gemv_rows_launch<ActBF16, W, kProSiluGate>(a, static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(y), \
                                                   nullptr, m, rows, cols, 0, as_stream(stream));                \
  }
    if (group == 128) SQX_ROWSILU(128) else if (group == 64) SQX_ROWSILU(64) else SQX_ROWSILU(32)
#undef SQX_ROWSILU
    SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return SQX_OK;
  }
  const int rc = int4_pro_check(wt, st, gate_up, y, m, rows, cols, group, k_slices, fn);
  if (rc != SQX_OK) return rc;
  const hipError_t e = launch_int4_pro<kProSiluGate>(static_cast<int>(group), wt, st,
                                                     static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(y),
                                                     m, rows, cols, k_slices, as_stream(stream),
                                                     ProArgs{nullptr, nullptr, nullptr, 0.0f});
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return SQX_OK;
}

// The decode step's fused forms at 2..8 rows: the multi-row GEMV (symmetric codes, fp32 scales, bf16).
template <int PRO, bool RES, bool RKV, bool SWI = false>
static hipError_t launch_int4_rows_fused(int group, const uint8_t* wt, const float* st, const uint16_t* x, uint16_t* y,
                                         int64_t m, int64_t rows, int64_t cols, int k_slices, hipStream_t s,
                                         const ProArgs& pa) {
#define SQX_RF(G_)                                                                                                 \
  {                                                                                                                \
    using W = WInt4<G_, false, false>;                                                                             \
    const typename W::Args a{wt, st, nullptr};                                                                     \
    return gemv_rows_launch<ActBF16, W, PRO, RES, RKV, SWI>(a, x, y, nullptr, m, rows, cols, k_slices, s, pa);     \
  }
  if (group == 128) SQX_RF(128)
  if (group == 64) SQX_RF(64)
  SQX_RF(32)
#undef SQX_RF
}

static int int4_rows_check(const uint8_t* wt, const float* st, const void* x, const void* y, int64_t m, int64_t rows,
                           int64_t cols, int64_t group, int k_slices, bool scale_sum, const char* fn) {
  SQX_REQUIRE(rows > 0 && cols > 0 && rows < ((int64_t)1 << 31) && m * rows < ((int64_t)1 << 31) &&
                  m * cols * 2 < ((int64_t)1 << 31),
              SQX_E_ARG, "%s: bad shape", fn);
  SQX_REQUIRE(group == 32 || group == 64 || group == 128, SQX_E_ARG, "%s: group_size %lld unsupported (32, 64 or 128)",
              fn, (long long)group);
  SQX_REQUIRE(cols % group == 0, SQX_E_ARG, "in_features=%lld not divisible by group_size=%lld", (long long)cols,
              (long long)group);
  SQX_REQUIRE(k_slices <= 16, SQX_E_ARG, "%s: k_slices %d > 16", fn, k_slices);
  SQX_REQUIRE(gemv_rows_fits(m, rows, cols, k_slices, scale_sum), SQX_E_ARG,
              "%s: m=%lld rows of %lld columns do not fit the multi-row form (2..8 rows; k-slices of at most 8 "
              "blocks for m <= 4, 4 for m <= 8; see sqx_int4_rows_fits)", fn, (long long)m, (long long)cols);
  SQX_REQUIRE(wt && st && x && y, SQX_E_ARG, "%s: null pointer", fn);
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0, SQX_E_ARG,
              "%s: wt and x must be 16-byte aligned", fn);
  return SQX_OK;
}

extern "C" int sqx_int4_rows_fits(int64_t m, int64_t rows, int64_t cols, int scale_sum) {
  return gemv_rows_fits(m, rows, cols, 0, scale_sum != 0) ? 1 : 0;
}

// Arguments of the residual epilogue shared by the entry points that end in it.
static int int4_res_check(const void* res, const void* res_out, const float* ss_out, const void* gain_next,
                          const void* hg_out, int64_t m, const char* fn) {
  SQX_REQUIRE(m >= 1 && m <= 8, SQX_E_ARG, "%s: the residual epilogue takes 1..8 rows, m=%lld", fn, (long long)m);
  SQX_REQUIRE(res && res_out && ss_out, SQX_E_ARG, "%s: null residual or sums", fn);
  SQX_REQUIRE((gain_next == nullptr) == (hg_out == nullptr), SQX_E_ARG, "%s: gain_next and hg_out go together", fn);
  return SQX_OK;
}

extern "C" int sqx_int4_linear_residual(const uint8_t* wt, const float* st, const void* x, const void* res,
                                        void* res_out, float* ss_out, const void* gain_next, void* hg_out, int64_t m,
                                        int64_t rows, int64_t cols, int64_t group, int k_slices, sqx_stream_t stream) {
  const char* fn = "sqx_int4_linear_residual";
  int rc = m >= 2 ? int4_rows_check(wt, st, x, res_out, m, rows, cols, group, k_slices, false, fn)
                  : int4_pro_check(wt, st, x, res_out, m, rows, cols, group, k_slices, fn);
  if (rc == SQX_OK) rc = int4_res_check(res, res_out, ss_out, gain_next, hg_out, m, fn);
  if (rc != SQX_OK) return rc;
  ProArgs pa{};
  pa.res = static_cast<const uint16_t*>(res);
  pa.res_out = static_cast<uint16_t*>(res_out);
  pa.ss_out = ss_out;
  pa.gain_next = static_cast<const uint16_t*>(gain_next);
  pa.hg_out = static_cast<uint16_t*>(hg_out);
  const hipError_t e =
      m >= 2 ? launch_int4_rows_fused<kProPlain, true, false>(static_cast<int>(group), wt, st,
                                                              static_cast<const uint16_t*>(x), nullptr, m, rows, cols,
                                                              k_slices, as_stream(stream), pa)
             : launch_int4_pro_res<kProPlain, true>(static_cast<int>(group), wt, st, static_cast<const uint16_t*>(x),
                                                    nullptr, m, rows, cols, k_slices, as_stream(stream), pa);
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return SQX_OK;
}

extern "C" int sqx_int4_linear_attn_residual(const uint8_t* wt, const float* st, const float* part, const int* lengths,
                                             int64_t tmax, const void* res, void* res_out, float* ss_out,
                                             const void* gain_next, void* hg_out, int64_t m, int64_t rows,
                                             int64_t cols, int64_t group, int k_slices, sqx_stream_t stream) {
  const char* fn = "sqx_int4_linear_attn_residual";
  SQX_REQUIRE(m == 1, SQX_E_ARG, "%s: the attention merge is the one-row (decode) form, m=%lld", fn, (long long)m);
  int rc = int4_pro_check(wt, st, part, res_out, m, rows, cols, group, k_slices, fn);
  if (rc == SQX_OK) rc = int4_res_check(res, res_out, ss_out, gain_next, hg_out, m, fn);
  if (rc != SQX_OK) return rc;
  SQX_REQUIRE(lengths != nullptr && tmax > 0 && tmax < (int64_t(1) << 30), SQX_E_ARG, "%s: null lengths or bad tmax", fn);
  SQX_REQUIRE(cols % 128 == 0, SQX_E_ARG, "%s: in_features=%lld is not a whole number of 128-dim heads", fn,
              (long long)cols);
  const int chunk = sqx_attn_partials_chunk(tmax);
  const int64_t nchunk = ceil_div(tmax, chunk);
  SQX_REQUIRE(nchunk <= kAttnFoldChunks, SQX_E_ARG, "%s: %lld key chunks (at most %d)", fn, (long long)nchunk,
              kAttnFoldChunks);
  const int64_t KB = cols / 128;
  int nw = k_slices <= 0 ? gemv_default_kslices(rows, cols, 128, 1) : k_slices;
  if (nw > KB) nw = static_cast<int>(KB);
  SQX_REQUIRE(ceil_div(KB, nw) == 2 && nw <= 16, SQX_E_ARG,
              "%s: the merge prologue runs two k-blocks per wave: %lld k-blocks over %d waves (k_slices)", fn,
              (long long)KB, nw);
  ProArgs pa{};
  pa.res = static_cast<const uint16_t*>(res);
  pa.res_out = static_cast<uint16_t*>(res_out);
  pa.ss_out = ss_out;
  pa.gain_next = static_cast<const uint16_t*>(gain_next);
  pa.hg_out = static_cast<uint16_t*>(hg_out);
  pa.lengths = lengths;
  pa.tmax = static_cast<int>(tmax);
  pa.part = part;
  pa.nchunk = static_cast<int>(nchunk);
  pa.chunk = chunk;
  const hipError_t e = launch_int4_pro_res<kProAttnCombine, true>(static_cast<int>(group), wt, st, nullptr, nullptr, m,
                                                                  rows, cols, nw, as_stream(stream), pa);
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return SQX_OK;
}

extern "C" int sqx_int4_linear_silu_residual(const uint8_t* wt, const float* st, const void* gate_up, const void* res,
                                             void* res_out, float* ss_out, const void* gain_next, void* hg_out,
                                             int64_t m, int64_t rows, int64_t cols, int64_t group, int k_slices,
                                             sqx_stream_t stream) {
  const char* fn = "sqx_int4_linear_silu_residual";
  int rc = m >= 2 ? int4_rows_check(wt, st, gate_up, res_out, m, rows, cols, group, k_slices, false, fn)
                  : int4_pro_check(wt, st, gate_up, res_out, m, rows, cols, group, k_slices, fn);
  if (rc == SQX_OK) rc = int4_res_check(res, res_out, ss_out, gain_next, hg_out, m, fn);
  if (rc != SQX_OK) return rc;
  ProArgs pa{};
  pa.res = static_cast<const uint16_t*>(res);
  pa.res_out = static_cast<uint16_t*>(res_out);
  pa.ss_out = ss_out;
  pa.gain_next = static_cast<const uint16_t*>(gain_next);
  pa.hg_out = static_cast<uint16_t*>(hg_out);
  const hipError_t e =
      m >= 2 ? launch_int4_rows_fused<kProSiluGate, true, false>(static_cast<int>(group), wt, st,
                                                                 static_cast<const uint16_t*>(gate_up), nullptr, m, rows,
                                                                 cols, k_slices, as_stream(stream), pa)
             : launch_int4_pro_res<kProSiluGate, true>(static_cast<int>(group), wt, st,
                                                       static_cast<const uint16_t*>(gate_up), nullptr, m, rows, cols,
                                                       k_slices, as_stream(stream), pa);
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return SQX_OK;
}

extern "C" int sqx_int4_linear_rmsnorm_sumsq(const uint8_t* wt, const float* st, const void* h, const float* ss,
                                            int64_t nss, const void* gain, float eps, void* y, int64_t m,
                                            int64_t rows, int64_t cols, int64_t group, int k_slices,
                                            sqx_stream_t stream) {
  const char* fn = "sqx_int4_linear_rmsnorm_sumsq";
  const int rc = int4_pro_check(wt, st, h, y, m, rows, cols, group, k_slices, fn);
  if (rc != SQX_OK) return rc;
  SQX_REQUIRE(m == 1, SQX_E_ARG, "%s: the norm from tile sums is the one-row (decode) form, m=%lld", fn, (long long)m);
  SQX_REQUIRE(nss == ceil_div(cols, 16) && nss <= kNormSumMax, SQX_E_ARG,
              "%s: %lld sums of squares for %lld columns (one per 16 columns, at most %d)", fn, (long long)nss,
              (long long)cols, kNormSumMax);
  SQX_REQUIRE(ss && gain, SQX_E_ARG, "%s: null sums or gain", fn);
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(gain) % 16 == 0 && reinterpret_cast<uintptr_t>(ss) % 4 == 0, SQX_E_ARG,
              "%s: gain must be 16-byte and the sums 4-byte aligned", fn);
  const int64_t KB = ceil_div(cols, 128);
  int nw = k_slices <= 0 ? gemv_default_kslices(rows, cols, 128, 1) : k_slices;
  if (nw > KB) nw = static_cast<int>(KB);
  SQX_REQUIRE(ceil_div(KB, nw) <= kOneMaxKbw, SQX_E_ARG,
              "%s: %lld k-blocks over %d waves: at most %d per wave (raise k_slices)", fn, (long long)KB, nw,
              kOneMaxKbw);
  ProArgs pa{};
  pa.gain = static_cast<const uint16_t*>(gain);
  pa.eps = eps;
  pa.ss_in = ss;
  pa.nss = static_cast<int>(nss);
  const hipError_t e = launch_int4_pro<kProNormSum>(static_cast<int>(group), wt, st, static_cast<const uint16_t*>(h),
                                                    static_cast<uint16_t*>(y), m, rows, cols, k_slices,
                                                    as_stream(stream), pa);
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return SQX_OK;
}

extern "C" int sqx_int4_linear_rowscale_sumsq(const uint8_t* wt, const float* st, const void* hg, const float* ss,
                                             int64_t nss, float eps, void* y, int64_t m, int64_t rows, int64_t cols,
                                             int64_t group, int k_slices, sqx_stream_t stream) {
  const char* fn = "sqx_int4_linear_rowscale_sumsq";
  SQX_REQUIRE(m >= 1 && m <= 8, SQX_E_ARG, "%s: the norm from tile sums takes 1..8 rows, m=%lld", fn, (long long)m);
  const int rc = m >= 2 ? int4_rows_check(wt, st, hg, y, m, rows, cols, group, k_slices, true, fn)
                        : int4_pro_check(wt, st, hg, y, m, rows, cols, group, k_slices, fn);
  if (rc != SQX_OK) return rc;
  SQX_REQUIRE(nss == ceil_div(cols, 16) && nss <= kNormSumMax, SQX_E_ARG,
              "%s: %lld sums of squares for %lld columns (one per 16 columns, at most %d)", fn, (long long)nss,
              (long long)cols, kNormSumMax);
  SQX_REQUIRE(ss != nullptr && reinterpret_cast<uintptr_t>(ss) % 16 == 0 && (m == 1 || nss % 4 == 0), SQX_E_ARG,
              "%s: the sums must be 16-byte aligned (and a multiple of 4 a row)", fn);
  if (m >= 2) {
    ProArgs pa{};
    pa.eps = eps;
    pa.ss_in = ss;
    pa.nss = static_cast<int>(nss);
    const hipError_t e = launch_int4_rows_fused<kProScaleSum, false, false>(
        static_cast<int>(group), wt, st, static_cast<const uint16_t*>(hg), static_cast<uint16_t*>(y), m, rows, cols,
        k_slices, as_stream(stream), pa);
    SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return SQX_OK;
  }
  const int64_t KB = ceil_div(cols, 128);
  int nw = k_slices <= 0 ? gemv_default_kslices(rows, cols, 128, 1) : k_slices;
  if (nw > KB) nw = static_cast<int>(KB);
  SQX_REQUIRE(ceil_div(KB, nw) <= kOneMaxKbw, SQX_E_ARG,
              "%s: %lld k-blocks over %d waves: at most %d per wave (raise k_slices)", fn, (long long)KB, nw,
              kOneMaxKbw);
  ProArgs pa{};
  pa.eps = eps;
  pa.ss_in = ss;
  pa.nss = static_cast<int>(nss);
  const hipError_t e = launch_int4_pro<kProScaleSum>(static_cast<int>(group), wt, st, static_cast<const uint16_t*>(hg),
                                                     static_cast<uint16_t*>(y), m, rows, cols, k_slices,
                                                     as_stream(stream), pa);
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return SQX_OK;
}

extern "C" int sqx_int4_linear_swiglu(const uint8_t* wt, const float* st, const void* x, void* y, int64_t m,
                                     int64_t rows, int64_t cols, int64_t group, sqx_stream_t stream) {
  const char* fn = "sqx_int4_linear_swiglu";
  SQX_REQUIRE(m >= 1 && m <= 64, SQX_E_ARG, "%s: 1..64 rows, m=%lld", fn, (long long)m);
  SQX_REQUIRE(rows > 0 && rows % 16 == 0 && cols > 0 && rows < ((int64_t)1 << 31) && m * rows < ((int64_t)1 << 31),
              SQX_E_ARG, "%s: rows=%lld: the gate / up pairs fill whole 16-row tiles", fn, (long long)rows);
  SQX_REQUIRE(group == 32 || group == 64 || group == 128, SQX_E_ARG, "%s: group_size %lld unsupported (32, 64 or 128)",
              fn, (long long)group);
  SQX_REQUIRE(cols % group == 0, SQX_E_ARG, "in_features=%lld not divisible by group_size=%lld", (long long)cols,
              (long long)group);
  SQX_REQUIRE(wt && st && x && y, SQX_E_ARG, "%s: null pointer", fn);
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0, SQX_E_ARG,
              "%s: the tiles and x must be 16-byte aligned", fn);
  const hipStream_t s = as_stream(stream);
  hipError_t e = hipErrorNotSupported;
  if (m == 1) {
    e = launch_int4_pro_res<kProPlain, false, true>(static_cast<int>(group), wt, st, static_cast<const uint16_t*>(x),
                                                    static_cast<uint16_t*>(y), m, rows, cols, 0, s, ProArgs{});
  } else {
    SkinnyShape sh = skinny_default_shape(m, rows, cols, 128, false);
    if (sh.variant == 2 || (sh.gemv && gemv_rows_fits(m, rows, cols))) {
      e = launch_int4_rows_fused<kProPlain, false, false, true>(static_cast<int>(group), wt, st,
                                                               static_cast<const uint16_t*>(x),
                                                               static_cast<uint16_t*>(y), m, rows, cols, 0, s, ProArgs{});
    } else {
      if (sh.gemv || sh.variant == 2) sh = SkinnyShape{0, 2, 8, 1, false};
      sh.S = 1;
#define SQX_SWG(G_)                                                                                          \
  {                                                                                                          \
    using W = WInt4<G_, false, false>;                                                                       \
    const typename W::Args a{wt, st, nullptr};                                                               \
    e = skinny_launch<ActBF16, W>(a, static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), nullptr, m, \
                                  rows, cols, sh, nullptr, 0, s, true, true);                                \
  }
      if (group == 128) SQX_SWG(128)
      else if (group == 64) SQX_SWG(64)
      else SQX_SWG(32)
#undef SQX_SWG
    }
  }
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: m=%lld rows of %lld columns: launch failed: %s", fn, (long long)m,
              (long long)cols, hipGetErrorString(e));
  return SQX_OK;
}

extern "C" int sqx_int4_linear_rowscale_swiglu(const uint8_t* wt, const float* st, const void* hg, const float* ss,
                                             int64_t nss, float eps, void* y, int64_t m, int64_t rows, int64_t cols,
                                             int64_t group, int k_slices, sqx_stream_t stream) {
  const char* fn = "sqx_int4_linear_rowscale_swiglu";
  SQX_REQUIRE(m >= 1 && m <= 8, SQX_E_ARG, "%s: the norm from tile sums takes 1..8 rows, m=%lld", fn, (long long)m);
  const int rc = m >= 2 ? int4_rows_check(wt, st, hg, y, m, rows, cols, group, k_slices, true, fn)
                        : int4_pro_check(wt, st, hg, y, m, rows, cols, group, k_slices, fn);
  if (rc != SQX_OK) return rc;
  SQX_REQUIRE(rows % 16 == 0, SQX_E_ARG, "%s: rows=%lld: the gate / up pairs fill whole 16-row tiles", fn, (long long)rows);
  SQX_REQUIRE(nss == ceil_div(cols, 16) && nss <= kNormSumMax, SQX_E_ARG,
              "%s: %lld sums of squares for %lld columns (one per 16 columns, at most %d)", fn, (long long)nss,
              (long long)cols, kNormSumMax);
  SQX_REQUIRE(ss != nullptr && reinterpret_cast<uintptr_t>(ss) % 16 == 0 && (m == 1 || nss % 4 == 0), SQX_E_ARG,
              "%s: the sums must be 16-byte aligned (and a multiple of 4 a row)", fn);
  if (m >= 2) {
    ProArgs pa{};
    pa.eps = eps;
    pa.ss_in = ss;
    pa.nss = static_cast<int>(nss);
    const hipError_t e = launch_int4_rows_fused<kProScaleSum, false, false, true>(
        static_cast<int>(group), wt, st, static_cast<const uint16_t*>(hg), static_cast<uint16_t*>(y), m, rows, cols,
        k_slices, as_stream(stream), pa);
    SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return SQX_OK;
  }
  const int64_t KB = ceil_div(cols, 128);
  int nw = k_slices <= 0 ? gemv_default_kslices(rows, cols, 128, 1) : k_slices;
  if (nw > KB) nw = static_cast<int>(KB);
  SQX_REQUIRE(ceil_div(KB, nw) <= kOneMaxKbw, SQX_E_ARG,
              "%s: %lld k-blocks over %d waves: at most %d per wave (raise k_slices)", fn, (long long)KB, nw,
              kOneMaxKbw);
  ProArgs pa{};
  pa.eps = eps;
  pa.ss_in = ss;
  pa.nss = static_cast<int>(nss);
  const hipError_t e = launch_int4_pro_res<kProScaleSum, false, true>(static_cast<int>(group), wt, st,
                                                                     static_cast<const uint16_t*>(hg),
                                                                     static_cast<uint16_t*>(y), m, rows, cols, k_slices,
                                                                     as_stream(stream), pa);
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return SQX_OK;
}

extern "C" int sqx_int4_linear_rope_kv(const uint8_t* wt, const float* st, const void* x, const float* ss, int64_t nss,
                                      float eps, const int* lengths, const float* cos_t, const float* sin_t,
                                      int64_t rope_rows, int64_t n_heads, int64_t n_kv_heads, int64_t tmax,
                                      void* q_out, void* k_cache, void* v_cache, int64_t m, int64_t rows, int64_t cols,
                                      int64_t group, int k_slices, sqx_stream_t stream) {
  const char* fn = "sqx_int4_linear_rope_kv";
  SQX_REQUIRE(m >= 1 && m <= 8, SQX_E_ARG, "%s: the RoPE epilogue takes 1..8 rows, m=%lld", fn, (long long)m);
  const int rc = m >= 2 ? int4_rows_check(wt, st, x, q_out, m, rows, cols, group, k_slices, ss != nullptr, fn)
                        : int4_pro_check(wt, st, x, q_out, 1, rows, cols, group, k_slices, fn);
  if (rc != SQX_OK) return rc;
  SQX_REQUIRE(n_heads > 0 && n_kv_heads > 0 && rows == (n_heads + 2 * n_kv_heads) * 128, SQX_E_ARG,
              "%s: rows=%lld is not (%lld + 2 * %lld) heads of 128", fn, (long long)rows, (long long)n_heads,
              (long long)n_kv_heads);
  SQX_REQUIRE(m >= 2 || ceil_div(rows, 16) < 1024, SQX_E_ARG,
              "%s: %lld rows: the one-row RoPE epilogue needs fewer than 1024 tiles", fn, (long long)rows);
  SQX_REQUIRE(lengths && cos_t && sin_t && k_cache && v_cache, SQX_E_ARG, "%s: null pointer", fn);
  SQX_REQUIRE(rope_rows > 0 && rope_rows < (int64_t(1) << 24) && tmax > 0 && tmax < (int64_t(1) << 30), SQX_E_ARG,
              "%s: bad rope_rows or tmax", fn);
  SQX_REQUIRE(ss == nullptr || (nss == ceil_div(cols, 16) && nss <= kNormSumMax &&
                                reinterpret_cast<uintptr_t>(ss) % 16 == 0 && (m == 1 || nss % 4 == 0)),
              SQX_E_ARG, "%s: %lld sums of squares for %lld columns (one per 16 columns, at most %d, 16-byte aligned)",
              fn, (long long)nss, (long long)cols, kNormSumMax);
  const int64_t KB = ceil_div(cols, 128);
  int nw = k_slices <= 0 ? gemv_default_kslices(rows, cols, 128, 1) : k_slices;
  if (nw > KB) nw = static_cast<int>(KB);
  SQX_REQUIRE(m >= 2 || ceil_div(KB, nw) <= kOneMaxKbw, SQX_E_ARG,
              "%s: %lld k-blocks over %d waves: at most %d per wave (raise k_slices)", fn, (long long)KB, nw,
              kOneMaxKbw);
  ProArgs pa{};
  pa.eps = eps;
  pa.ss_in = ss;
  pa.nss = static_cast<int>(nss);
  pa.lengths = lengths;
  pa.cos_t = cos_t;
  pa.sin_t = sin_t;
  pa.rope_rows = static_cast<int>(rope_rows);
  pa.qn = static_cast<int>(n_heads * 128);
  pa.kn = static_cast<int>(n_kv_heads * 128);
  pa.tmax = static_cast<int>(tmax);
  pa.q_out = static_cast<uint16_t*>(q_out);
  pa.k_cache = static_cast<uint16_t*>(k_cache);
  pa.v_cache = static_cast<uint16_t*>(v_cache);
  hipError_t e;
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  hipStream_t s = as_stream(stream);
  if (m >= 2) {
    e = ss != nullptr ? launch_int4_rows_fused<kProScaleSum, false, true>(static_cast<int>(group), wt, st, xp, nullptr, m,
                                                                         rows, cols, k_slices, s, pa)
                      : launch_int4_rows_fused<kProPlain, false, true>(static_cast<int>(group), wt, st, xp, nullptr, m,
                                                                      rows, cols, k_slices, s, pa);
    SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return SQX_OK;
  }
#define SQX_RKV(G_)                                                                                               \
  {                                                                                                               \
    using W = WInt4<G_, false, false>;                                                                            \
    const typename W::Args a{wt, st, nullptr};                                                                    \
    if (ss != nullptr)                                                                                            \
      e = gemv_launch<ActBF16, W, SQX_INT4_U1, SQX_INT4_U2, false, kProScaleSum, false, true>(a, xp, nullptr, nullptr, \
                                                                                     nullptr, 1, rows, cols,     \
                                                                                     k_slices, s, pa);           \
    else                                                                                                          \
      e = gemv_launch<ActBF16, W, SQX_INT4_U1, SQX_INT4_U2, false, kProPlain, false, true>(a, xp, nullptr, nullptr, \
                                                                                  nullptr, 1, rows, cols,        \
                                                                                  k_slices, s, pa);              \
  }
  if (group == 128) SQX_RKV(128)
  else if (group == 64) SQX_RKV(64)
  else SQX_RKV(32)
#undef SQX_RKV
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return SQX_OK;
}
